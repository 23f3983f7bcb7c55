"""CPU restatement of the reference's INT8 decode step and prefill -- TEST
INFRASTRUCTURE ONLY.

``decode_int8_step`` follows ``decoder.rs:848-965`` op by op with the oracle's
kernel restatements (oracle/qasr_oracle.c): input RMSNorm, the three
``linear_nobias_int8`` projections, per-head RMSNorm + NeoX RoPE at ``pos``,
the K/V row copies into the cache, ``causal_attention`` over rows 0..pos, the
o projection and residual add, post-attention RMSNorm, the fused gate/up
projection with the loop's libm SwiGLU (decoder.rs:916-921), the down
projection and residual add; then the final RMSNorm, the lm_head logits and
the greedy argmax (decoder.rs:929-963). ``prefill_int8`` follows
``decoder.rs:751-847``: the same layer for seq_len rows at positions
start_pos.., with the prefill's fast_exp SwiGLU (kernels::swiglu_multiply)
and no final norm or lm_head. ``decode_w8a8_step`` is ``decode_int8_step``
with the activation rounded to int8 per row (quantize.rs:633-662, out_dim 1)
at the four projection inputs and the projections taken as exact int32 dots
with the ``((f32)dot * x_scale) * w_scale`` dequantization (the W8A8 gate/up
arithmetic, a10-a11 of the hot-path table, extended to q/k/v, o and down);
the gate/up keeps its libm SwiGLU epilogue and the lm_head stays W8A32.
Only tests/ and bench.py's cpu_baseline leg use it.

Pinned by its parts: every primitive it calls is pinned in tests/test_oracle.py;
the compositions are checked against float64 numpy evaluations of the same
formulas in tests/test_oracle.py::test_decode_step_composition and
::test_prefill_composition.
"""
from __future__ import annotations

import math

import numpy as np

from . import (add_inplace, apply_rope_neox, argmax_rows, causal_attention, gate_up_swiglu_w8a8,
               linear_nobias_int8, linear_w8a8, quantize_f32_to_int8, rms_norm, rms_norm_per_head,
               rope_table, swiglu_multiply, swiglu_split)


def decode_int8_step(w: dict, k_cache: np.ndarray, v_cache: np.ndarray, pos: int,
                     embed: np.ndarray, n_heads: int, n_kv_heads: int, head_dim: int,
                     eps: float = 1e-6, theta: float = 1e6, threads: int = 1):
    """One token. ``w``: {"layers": [{"wq": (int8 [out,in], scales), ..., "gate_up": fused
    interleaved (w, s), "down", "q_norm", "k_norm", "input_norm", "post_attn_norm"}], "norm",
    "lm_head": (w, s)}. ``k_cache``/``v_cache``: [layers, max_seq, kv_dim] float32, row ``pos``
    is written. Returns (token, final normed hidden, logits)."""
    H = embed.size
    q_dim, kv_dim = n_heads * head_dim, n_kv_heads * head_dim
    cos, sin = rope_table(pos + 1, head_dim, theta)
    c, s = cos[pos * head_dim:(pos + 1) * head_dim], sin[pos * head_dim:(pos + 1) * head_dim]
    scale = 1.0 / math.sqrt(head_dim)
    x = np.array(embed, np.float32)
    for l, lw in enumerate(w["layers"]):
        xn = rms_norm(x, lw["input_norm"], 1, H, eps)
        q = linear_nobias_int8(xn, *lw["wq"], 1, H, q_dim, threads)
        k = linear_nobias_int8(xn, *lw["wk"], 1, H, kv_dim, threads)
        v = linear_nobias_int8(xn, *lw["wv"], 1, H, kv_dim, threads)
        q = rms_norm_per_head(q, lw["q_norm"], 1, n_heads, head_dim, eps)
        k = rms_norm_per_head(k, lw["k_norm"], 1, n_kv_heads, head_dim, eps)
        q = apply_rope_neox(q, c, s, 1, n_heads, head_dim)
        k = apply_rope_neox(k, c, s, 1, n_kv_heads, head_dim)
        k_cache[l, pos] = k
        v_cache[l, pos] = v
        attn = causal_attention(q, k_cache[l, :pos + 1].ravel(), v_cache[l, :pos + 1].ravel(), 1, pos + 1,
                                n_heads, n_kv_heads, head_dim, scale, pos)
        proj = linear_nobias_int8(attn, *lw["wo"], 1, q_dim, H, threads)
        add_inplace(x, proj)
        xn = rms_norm(x, lw["post_attn_norm"], 1, H, eps)
        inter = lw["gate_up"][1].size // 2
        gu = linear_nobias_int8(xn, *lw["gate_up"], 1, H, 2 * inter, threads)
        ffn = swiglu_split(gu[0::2].copy(), gu[1::2].copy())
        down = linear_nobias_int8(ffn, *lw["down"], 1, inter, H, threads)
        add_inplace(x, down)
    xn = rms_norm(x, w["norm"], 1, H, eps)
    vocab = w["lm_head"][1].size
    logits = linear_nobias_int8(xn, *w["lm_head"], 1, H, vocab, threads)
    return int(argmax_rows(logits, 1, vocab)[0]), xn, logits


def decode_w8a8_step(w: dict, k_cache: np.ndarray, v_cache: np.ndarray, pos: int,
                     embed: np.ndarray, n_heads: int, n_kv_heads: int, head_dim: int,
                     eps: float = 1e-6, theta: float = 1e6, threads: int = 1, quant=None,
                     lm_head_w8a8: bool = False):
    """``decode_int8_step`` (same arguments and results) with W8A8 projections:
    each projection input is quantized per row and multiplied as int8 x int8
    with int32 sums; the gate/up is the fused SwiGLU W8A8 product. With
    ``lm_head_w8a8`` the lm_head is one too (the final normed row quantized,
    logits = ((f32)dot * x_scale) * row_scale); otherwise it stays W8A32.
    ``quant(x, n) -> (q, scale)`` replaces the per-row quantizer at the four
    points, in order per layer: input norm, attention rows, post-attention
    norm, SwiGLU rows, then (``lm_head_w8a8``) the final norm (tests use it to
    see and steer the rounding)."""
    if quant is None:
        quant = lambda v, n: quantize_f32_to_int8(v, 1, n)  # noqa: E731
    H = embed.size
    q_dim, kv_dim = n_heads * head_dim, n_kv_heads * head_dim
    cos, sin = rope_table(pos + 1, head_dim, theta)
    c, s = cos[pos * head_dim:(pos + 1) * head_dim], sin[pos * head_dim:(pos + 1) * head_dim]
    scale = 1.0 / math.sqrt(head_dim)
    x = np.array(embed, np.float32)
    for l, lw in enumerate(w["layers"]):
        xn = rms_norm(x, lw["input_norm"], 1, H, eps)
        xq, xs = quant(xn, H)
        q = linear_w8a8(*lw["wq"], xq, xs, 1, H, q_dim)[0]
        k = linear_w8a8(*lw["wk"], xq, xs, 1, H, kv_dim)[0]
        v = linear_w8a8(*lw["wv"], xq, xs, 1, H, kv_dim)[0]
        q = rms_norm_per_head(q, lw["q_norm"], 1, n_heads, head_dim, eps)
        k = rms_norm_per_head(k, lw["k_norm"], 1, n_kv_heads, head_dim, eps)
        q = apply_rope_neox(q, c, s, 1, n_heads, head_dim)
        k = apply_rope_neox(k, c, s, 1, n_kv_heads, head_dim)
        k_cache[l, pos] = k
        v_cache[l, pos] = v
        attn = causal_attention(q, k_cache[l, :pos + 1].ravel(), v_cache[l, :pos + 1].ravel(), 1, pos + 1,
                                n_heads, n_kv_heads, head_dim, scale, pos)
        aq, as_ = quant(attn, q_dim)
        add_inplace(x, linear_w8a8(*lw["wo"], aq, as_, 1, q_dim, H)[0])
        xn = rms_norm(x, lw["post_attn_norm"], 1, H, eps)
        inter = lw["gate_up"][1].size // 2
        xq, xs = quant(xn, H)
        ffn = gate_up_swiglu_w8a8(*lw["gate_up"], xq, xs, 1, H, inter)[0]
        fq, fs = quant(ffn, inter)
        add_inplace(x, linear_w8a8(*lw["down"], fq, fs, 1, inter, H)[0])
    xn = rms_norm(x, w["norm"], 1, H, eps)
    vocab = w["lm_head"][1].size
    if lm_head_w8a8:
        xq, xs = quant(xn, H)
        logits = linear_w8a8(*w["lm_head"], xq, xs, 1, H, vocab)[0]
    else:
        logits = linear_nobias_int8(xn, *w["lm_head"], 1, H, vocab, threads)
    return int(argmax_rows(logits, 1, vocab)[0]), xn, logits


def prefill_int8(w: dict, k_cache: np.ndarray, v_cache: np.ndarray, start_pos: int,
                 embeds: np.ndarray, seq_len: int, n_heads: int, n_kv_heads: int, head_dim: int,
                 eps: float = 1e-6, theta: float = 1e6, threads: int = 1, layers=None) -> np.ndarray:
    """``seq_len`` tokens at positions start_pos.. (decoder.rs:751-847). Cache rows
    start_pos..start_pos+seq_len-1 of every layer are written; returns the
    residual stream x [seq_len * hidden] after the last layer. ``layers`` (an
    iterable of layer dicts) replaces w["layers"] when given."""
    T = seq_len
    H = embeds.size // T
    q_dim, kv_dim = n_heads * head_dim, n_kv_heads * head_dim
    cos, sin = rope_table(start_pos + T, head_dim, theta)
    c = cos[start_pos * head_dim:(start_pos + T) * head_dim]
    s = sin[start_pos * head_dim:(start_pos + T) * head_dim]
    scale = 1.0 / math.sqrt(head_dim)
    total = start_pos + T
    x = np.array(embeds, np.float32).ravel()
    for l, lw in enumerate(w["layers"] if layers is None else layers):
        xn = rms_norm(x, lw["input_norm"], T, H, eps)
        q = linear_nobias_int8(xn, *lw["wq"], T, H, q_dim, threads)
        k = linear_nobias_int8(xn, *lw["wk"], T, H, kv_dim, threads)
        v = linear_nobias_int8(xn, *lw["wv"], T, H, kv_dim, threads)
        q = rms_norm_per_head(q, lw["q_norm"], T, n_heads, head_dim, eps)
        k = rms_norm_per_head(k, lw["k_norm"], T, n_kv_heads, head_dim, eps)
        q = apply_rope_neox(q, c, s, T, n_heads, head_dim)
        k = apply_rope_neox(k, c, s, T, n_kv_heads, head_dim)
        k_cache[l, start_pos:total] = k.reshape(T, kv_dim)
        v_cache[l, start_pos:total] = v.reshape(T, kv_dim)
        attn = causal_attention(q, k_cache[l, :total].ravel(), v_cache[l, :total].ravel(), T, total,
                                n_heads, n_kv_heads, head_dim, scale, start_pos)
        proj = linear_nobias_int8(attn, *lw["wo"], T, q_dim, H, threads)
        add_inplace(x, proj)
        xn = rms_norm(x, lw["post_attn_norm"], T, H, eps)
        inter = lw["gate_up"][1].size // 2
        gu = linear_nobias_int8(xn, *lw["gate_up"], T, H, 2 * inter, threads)
        gate = swiglu_multiply(gu, T, inter)
        ffn = linear_nobias_int8(gate, *lw["down"], T, inter, H, threads)
        add_inplace(x, ffn)
    return x
