"""Host mirror of ``qwen_asr::kernels`` over device memory.

Every function keeps the reference's name, argument order and meaning
(crates/qwen-asr/src/kernels/mod.rs and decoder.rs), with Rust slices replaced
by device-resident ``torch`` tensors (torch supplies device memory and the
current HIP stream; all arithmetic runs in the gfx950 kernels of
``libqasr_hip.so`` through the C-ABI of include/qasr.h).

Error behaviour mirrors the reference: where the Rust code would panic on a
slice that is too short, these raise ``IndexError`` before anything is
launched; a wrong dtype/device raises ``TypeError``; a status returned by the
C-ABI raises ``QasrError``.

Calls only enqueue work on the current stream; nothing here synchronises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import QasrError  # noqa: F401  (re-export)

__all__ = [
    "add_inplace", "rms_norm", "add_rms_norm", "add_rms_norm_quant", "rms_norm_per_head", "apply_rope_neox",
    "head_rms_norm_rope", "swiglu_multiply", "swiglu_multiply_inplace", "swiglu_split", "silu",
    "gelu", "gelu_erf", "layer_norm", "sinusoidal_pe", "pe_add", "tok_embed_f32_to_f32",
    "tok_embed_bf16_to_f32", "tok_embed_int8_to_f32", "embed_gather_f32", "embed_gather_bf16",
    "embed_gather_i8", "quantize_f32_to_int8", "quantize_rows_i8", "linear_nobias_int8",
    "linear_int8", "interleave_gate_up", "gate_up_swiglu_w8a8", "gate_up_swiglu_w8a8_f32in",
    "pack_w8a8_tiles", "gate_up_swiglu_w8a8_packed", "RopeCache", "QuantWeight",
]


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need(t: torch.Tensor, dtype: torch.dtype, n: int, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise TypeError(f"{name}: must be a device tensor (got {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.numel() < n:
        raise IndexError(f"{name}: range end index {n} out of range for slice of length {t.numel()}")


F32, I8, I32, U16 = torch.float32, torch.int8, torch.int32, torch.int16


# ---------------------------------------------------------------------------
# Basic / normalisation (kernels/mod.rs)
# ---------------------------------------------------------------------------
def add_inplace(a: torch.Tensor, b: torch.Tensor, n: int) -> None:
    """``a[i] += b[i]`` for i < n (kernels/mod.rs:486-488)."""
    _need(a, F32, n, "a")
    _need(b, F32, n, "b")
    _lib.call("qasr_add_inplace_f32", _ptr(a), _ptr(b), n, _stream())


def rms_norm(out, x, weight, seq_len: int, hidden: int, eps: float) -> None:
    """Row RMSNorm (kernels/mod.rs:897-918)."""
    _need(out, F32, seq_len * hidden, "out")
    _need(x, F32, seq_len * hidden, "x")
    _need(weight, F32, hidden, "weight")
    _lib.call("qasr_rms_norm_f32", _ptr(out), _ptr(x), _ptr(weight), seq_len, hidden, eps, _stream())


def add_rms_norm(x, delta, weight, out, seq_len: int, hidden: int, eps: float) -> None:
    """Fused ``add_inplace(x, delta)`` + ``rms_norm(out, x)`` (decoder.rs:908+910)."""
    n = seq_len * hidden
    _need(x, F32, n, "x")
    _need(delta, F32, n, "delta")
    _need(weight, F32, hidden, "weight")
    _need(out, F32, n, "out")
    _lib.call("qasr_add_rms_norm_f32", _ptr(x), _ptr(delta), _ptr(weight), _ptr(out), seq_len,
              hidden, eps, _stream())


def add_rms_norm_quant(x, delta, weight, out, q, q_scales, seq_len: int, hidden: int,
                       eps: float) -> None:
    """Fused ``x += delta`` (skipped if delta is None), ``y = rms_norm(x)`` and
    per-row int8 quantization of y into ``q``/``q_scales``; ``out`` (may be None)
    receives y."""
    n = seq_len * hidden
    _need(x, F32, n, "x")
    if delta is not None:
        _need(delta, F32, n, "delta")
    _need(weight, F32, hidden, "weight")
    if out is not None:
        _need(out, F32, n, "out")
    _need(q, I8, n, "q")
    _need(q_scales, F32, seq_len, "q_scales")
    _lib.call("qasr_add_rms_norm_quant_f32", _ptr(x), _ptr(delta), _ptr(weight), _ptr(out),
              _ptr(q), _ptr(q_scales), seq_len, hidden, eps, _stream())


def layer_norm(out, x, weight, bias, seq_len: int, hidden: int, eps: float) -> None:
    """Row LayerNorm (kernels/mod.rs:866-895)."""
    _need(out, F32, seq_len * hidden, "out")
    _need(x, F32, seq_len * hidden, "x")
    _need(weight, F32, hidden, "weight")
    _need(bias, F32, hidden, "bias")
    _lib.call("qasr_layer_norm_f32", _ptr(out), _ptr(x), _ptr(weight), _ptr(bias), seq_len,
              hidden, eps, _stream())



def add_layer_norm(x, delta, weight, bias, out, seq_len: int, hidden: int, eps: float) -> None:
    """``x += delta`` then ``out = layer_norm(x)`` in one pass: an encoder
    residual add (encoder.rs:386, 397) and the LayerNorm that reads its rows
    next (encoder.rs:389-390, 370-371, 401-402); equal to ``add_inplace`` +
    ``layer_norm`` bit for bit."""
    n = seq_len * hidden
    _need(x, F32, n, "x")
    _need(delta, F32, n, "delta")
    _need(weight, F32, hidden, "weight")
    _need(bias, F32, hidden, "bias")
    _need(out, F32, n, "out")
    _lib.call("qasr_add_layer_norm_f32", _ptr(x), _ptr(delta), _ptr(weight), _ptr(bias), _ptr(out),
              seq_len, hidden, eps, _stream())


def rms_norm_per_head(x, weight, seq_len: int, n_heads: int, head_dim: int, eps: float) -> None:
    """In-place per-head RMSNorm (kernels/mod.rs:920-935)."""
    _need(x, F32, seq_len * n_heads * head_dim, "x")
    _need(weight, F32, head_dim, "weight")
    _lib.call("qasr_rms_norm_per_head_f32", _ptr(x), _ptr(weight), seq_len, n_heads, head_dim,
              eps, _stream())


def apply_rope_neox(x, cos_vals, sin_vals, seq: int, n_heads: int, head_dim: int) -> None:
    """In-place NeoX RoPE, row s uses cos/sin row s (kernels/mod.rs:1247-1267)."""
    _need(x, F32, seq * n_heads * head_dim, "x")
    _need(cos_vals, F32, seq * head_dim, "cos_vals")
    _need(sin_vals, F32, seq * head_dim, "sin_vals")
    _lib.call("qasr_apply_rope_neox_f32", _ptr(x), _ptr(cos_vals), _ptr(sin_vals), seq, n_heads,
              head_dim, _stream())


def head_rms_norm_rope(q, k, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, seq: int,
                       n_heads: int, n_kv_heads: int, head_dim: int, eps: float) -> None:
    """Fused q/k head RMSNorm + RoPE at per-row positions (decoder.rs:888-892).

    ``positions`` is an int32 device tensor of ``seq`` entries or None (row s at
    position s). ``cos_tab``/``sin_tab`` are RopeCache tables; a position outside
    the table poisons that row with NaN.
    """
    if n_heads:
        _need(q, F32, seq * n_heads * head_dim, "q")
        _need(q_norm_w, F32, head_dim, "q_norm_w")
    if n_kv_heads:
        _need(k, F32, seq * n_kv_heads * head_dim, "k")
        _need(k_norm_w, F32, head_dim, "k_norm_w")
    _need(cos_tab, F32, head_dim, "cos_tab")
    _need(sin_tab, F32, cos_tab.numel(), "sin_tab")
    if positions is not None:
        _need(positions, I32, seq, "positions")
    rows = cos_tab.numel() // head_dim
    _lib.call("qasr_head_rms_norm_rope_f32", _ptr(q if n_heads else None),
              _ptr(k if n_kv_heads else None), _ptr(q_norm_w if n_heads else None),
              _ptr(k_norm_w if n_kv_heads else None), _ptr(cos_tab), _ptr(sin_tab),
              _ptr(positions), seq, n_heads, n_kv_heads, head_dim, rows, eps, _stream())


def head_rms_norm_rope_kv(q, k, v, q_norm_w, k_norm_w, rope: "RopeCache", positions, start_pos: int,
                          seq: int, n_heads: int, n_kv_heads: int, head_dim: int, eps: float,
                          k_cache, v_cache, cache_rows: int) -> None:
    """q/k head RMSNorm + RoPE with the KV-cache store fused in
    (decoder.rs:888-895: norm, rope, then ``k_at``/``v_at`` copies).

    Without ``positions`` row s is position ``start_pos + s`` of one sequence
    and ``k_cache``/``v_cache`` are that layer's ``[cache_rows, kv_dim]`` block
    (``KvCache.k_layer_block``). With ``positions`` (int32, ``seq`` entries) row s
    is its own decode stream and the caches are ``[seq, cache_rows, kv_dim]``.
    k and v are read only; q is rotated in place.
    """
    kv_dim = n_kv_heads * head_dim
    if n_heads:
        _need(q, F32, seq * n_heads * head_dim, "q")
        _need(q_norm_w, F32, head_dim, "q_norm_w")
    if n_kv_heads:
        _need(k, F32, seq * kv_dim, "k")
        _need(v, F32, seq * kv_dim, "v")
        _need(k_norm_w, F32, head_dim, "k_norm_w")
        streams = seq if positions is not None else 1
        _need(k_cache, F32, streams * cache_rows * kv_dim, "k_cache")
        _need(v_cache, F32, streams * cache_rows * kv_dim, "v_cache")
    if positions is not None:
        _need(positions, I32, seq, "positions")
    if rope.head_dim != head_dim:
        raise ValueError("RopeCache head_dim does not match")
    _lib.call("qasr_head_rms_norm_rope_kv_f32", _ptr(q if n_heads else None), _ptr(k), _ptr(v),
              _ptr(q_norm_w if n_heads else None), _ptr(k_norm_w), _ptr(rope.cos), _ptr(rope.sin),
              _ptr(positions), start_pos, seq, n_heads, n_kv_heads, head_dim, rope.cap, eps,
              _ptr(k_cache), _ptr(v_cache), cache_rows, _stream())


def causal_attention(out, q, k, v, seq_q: int, seq_k: int, n_heads: int, n_kv_heads: int,
                     head_dim: int, scale: float, q_offset: int) -> None:
    """Causal GQA attention over a KV block (kernels/mod.rs:1124-1207)."""
    _need(out, F32, seq_q * n_heads * head_dim, "out")
    _need(q, F32, seq_q * n_heads * head_dim, "q")
    if seq_k:
        _need(k, F32, seq_k * n_kv_heads * head_dim, "k")
        _need(v, F32, seq_k * n_kv_heads * head_dim, "v")
    _lib.call("qasr_causal_attention_f32", _ptr(out), _ptr(q), _ptr(k if seq_k else None),
              _ptr(v if seq_k else None), seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale,
              q_offset, _stream())


def batched_decode_workspace(batch: int, n_heads: int, head_dim: int, cache_rows: int,
                             device="cuda") -> torch.Tensor | None:
    """Workspace for batched_decode_attention's chunked form (None if the cache
    is a single chunk): allocate once, reuse per call on one stream."""
    n = _lib.lib().qasr_batched_decode_attention_workspace_floats(batch, n_heads, head_dim, cache_rows)
    return torch.empty(n, dtype=F32, device=device) if n else None


def batched_decode_order(order, positions, batch: int, cache_rows: int) -> None:
    """order (int32 [2 * batch]) = (stream, position) pairs, the streams with the
    most keys first, for batched_decode_attention's ``order``."""
    _need(order, I32, 2 * batch, "order")
    _need(positions, I32, batch, "positions")
    _lib.call("qasr_batched_decode_order_i32", _ptr(order), _ptr(positions), batch, cache_rows, _stream())


def batched_decode_attention(out, q, k_cache, v_cache, cache_rows: int, positions, batch: int, n_heads: int,
                             n_kv_heads: int, head_dim: int, scale: float, workspace=None, out_q=None,
                             out_scales=None, order=None) -> None:
    """Decode attention of ``batch`` streams, each over rows 0..positions[m] of its
    own cache block ``[batch, cache_rows, n_kv_heads * head_dim]`` (decoder.rs:900-903
    per stream). With ``workspace`` (batched_decode_workspace) every stream's
    keys are cut into chunks of 512 and the chunk partials merged; without it
    one workgroup per (stream, kv head) walks all of its keys. ``out_q`` /
    ``out_scales`` (int8 [batch * n_heads * head_dim], f32 [batch]) also get each
    stream's row quantized per row, as quantize_rows_i8 would on ``out``."""
    if workspace is not None:
        _need(workspace, F32, 1, "workspace")
    if (out_q is None) != (out_scales is None):
        raise ValueError("out_q and out_scales go together")
    if out_q is not None:
        _need(out_q, I8, batch * n_heads * head_dim, "out_q")
        _need(out_scales, F32, batch, "out_scales")
    if order is not None:
        _need(order, I32, 2 * batch, "order")
    kv = n_kv_heads * head_dim
    _need(out, F32, batch * n_heads * head_dim, "out")
    _need(q, F32, batch * n_heads * head_dim, "q")
    _need(k_cache, F32, batch * cache_rows * kv, "k_cache")
    _need(v_cache, F32, batch * cache_rows * kv, "v_cache")
    _need(positions, I32, batch, "positions")
    _lib.call("qasr_batched_decode_attention_f32", _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), cache_rows,
              _ptr(positions), batch, n_heads, n_kv_heads, head_dim, scale, _ptr(workspace),
              0 if workspace is None else workspace.numel(), _ptr(out_q), _ptr(out_scales), _ptr(order),
              _stream())


def attention_workspace(seq_q: int, n_heads: int, head_dim: int, device="cuda") -> torch.Tensor:
    """Workspace for causal_attention_split: allocate once, reuse per call on
    one stream."""
    n = _lib.lib().qasr_causal_attention_workspace_floats(seq_q, n_heads, head_dim)
    return torch.empty(n, dtype=F32, device=device)


def causal_attention_split(out, q, k, v, seq_q: int, seq_k: int, n_heads: int, n_kv_heads: int,
                           head_dim: int, scale: float, q_offset: int, workspace) -> None:
    """causal_attention with the keys split over workgroups (decode shape);
    partials go to ``workspace`` (see attention_workspace)."""
    _need(out, F32, seq_q * n_heads * head_dim, "out")
    _need(q, F32, seq_q * n_heads * head_dim, "q")
    if seq_k:
        _need(k, F32, seq_k * n_kv_heads * head_dim, "k")
        _need(v, F32, seq_k * n_kv_heads * head_dim, "v")
    _need(workspace, F32, 0, "workspace")
    _lib.call("qasr_causal_attention_split_f32", _ptr(out), _ptr(q), _ptr(k if seq_k else None),
              _ptr(v if seq_k else None), seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale,
              q_offset, _ptr(workspace), workspace.numel(), _stream())


def decode_attention(out, q, k, v, q_norm_w, k_norm_w, rope: "RopeCache", pos: int, n_heads: int,
                     n_kv_heads: int, head_dim: int, eps: float, scale: float, k_cache, v_cache,
                     cache_rows: int, workspace) -> None:
    """One decode token: q/k head RMSNorm + RoPE at ``pos``, the K/V rows into the
    layer's cache block and causal attention over rows 0..pos, equal bit for bit
    to head_rms_norm_rope_kv + causal_attention_split (decoder.rs:888-903). With
    the keys split over workgroups it is one attention launch; ``q`` is scratch
    (it may come back normalised and rotated)."""
    kv_dim = n_kv_heads * head_dim
    _need(out, F32, n_heads * head_dim, "out")
    _need(q, F32, n_heads * head_dim, "q")
    _need(k, F32, kv_dim, "k")
    _need(v, F32, kv_dim, "v")
    _need(q_norm_w, F32, head_dim, "q_norm_w")
    _need(k_norm_w, F32, head_dim, "k_norm_w")
    _need(k_cache, F32, cache_rows * kv_dim, "k_cache")
    _need(v_cache, F32, cache_rows * kv_dim, "v_cache")
    _need(workspace, F32, 0, "workspace")
    if rope.head_dim != head_dim:
        raise ValueError("RopeCache head_dim does not match")
    _lib.call("qasr_decode_attention_f32", _ptr(out), _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w),
              _ptr(k_norm_w), _ptr(rope.cos), _ptr(rope.sin), rope.cap, pos, n_heads, n_kv_heads,
              head_dim, eps, scale, _ptr(k_cache), _ptr(v_cache), cache_rows, _ptr(workspace),
              workspace.numel(), _stream())


def argmax_rows(idx, x, rows: int, cols: int) -> None:
    """Per-row argmax with the lm_head loop's semantics (decoder.rs:941-949)."""
    _need(idx, I32, rows, "idx")
    _need(x, F32, rows * cols, "x")
    _lib.call("qasr_argmax_rows_f32", _ptr(idx), _ptr(x), rows, cols, _stream())


def lm_head_workspace(vocab: int, device="cuda") -> torch.Tensor:
    """Workspace for the one-token lm_head argmax (bytes as a uint8 tensor)."""
    n = _lib.lib().qasr_lm_head_argmax_workspace_bytes(vocab)
    return torch.empty(max(n, 8), dtype=torch.uint8, device=device)


def lm_head_int8_argmax(idx, logits, x, w: QuantWeight, rows: int, in_dim: int, vocab: int,
                        workspace: torch.Tensor | None = None) -> None:
    """INT8 lm_head logits + greedy argmax (decoder.rs:935-963). With a
    ``lm_head_workspace`` and one row the argmax is reduced inside the matvec."""
    _need(idx, I32, rows, "idx")
    _need(logits, F32, rows * vocab, "logits")
    _need(x, F32, rows * in_dim, "x")
    _need(w.data, I8, vocab * in_dim, "w")
    _need(w.scales, F32, vocab, "scales")
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _lib.call("qasr_lm_head_int8_argmax_f32", _ptr(idx), _ptr(logits), _ptr(x), _ptr(w.data),
              _ptr(w.scales), rows, in_dim, vocab, _ptr(workspace), ws_bytes, _stream())


class KvCache:
    """Device KV cache with the reference's layout and growth rule
    (decoder.rs:129-228): ``k``/``v`` are ``[n_layers, max_seq, kv_dim]`` fp32,
    ``grow`` doubles ``max_seq`` until it covers the request and copies the first
    ``len`` rows of every layer."""

    def __init__(self, n_layers: int, max_seq: int, kv_dim: int, device="cuda"):
        self.n_layers, self.max_seq, self.kv_dim, self.len = n_layers, max_seq, kv_dim, 0
        self.k = torch.zeros(n_layers * max_seq * kv_dim, dtype=F32, device=device)
        self.v = torch.zeros_like(self.k)

    def grow(self, required: int) -> None:
        if required <= self.max_seq:
            return
        new_max = self.max_seq
        while new_max < required:
            new_max *= 2
        k = torch.zeros(self.n_layers * new_max * self.kv_dim, dtype=F32, device=self.k.device)
        v = torch.zeros_like(k)
        n = self.len * self.kv_dim
        for layer in range(self.n_layers):
            src, dst = layer * self.max_seq * self.kv_dim, layer * new_max * self.kv_dim
            k[dst:dst + n].copy_(self.k[src:src + n])
            v[dst:dst + n].copy_(self.v[src:src + n])
        self.k, self.v, self.max_seq = k, v, new_max

    def k_layer_block(self, layer: int) -> torch.Tensor:
        off = layer * self.max_seq * self.kv_dim
        return self.k[off:off + self.max_seq * self.kv_dim]

    def v_layer_block(self, layer: int) -> torch.Tensor:
        off = layer * self.max_seq * self.kv_dim
        return self.v[off:off + self.max_seq * self.kv_dim]

    def k_layer(self, layer: int) -> torch.Tensor:
        return self.k_layer_block(layer)[: self.len * self.kv_dim]

    def v_layer(self, layer: int) -> torch.Tensor:
        return self.v_layer_block(layer)[: self.len * self.kv_dim]


class RopeCache:
    """Device RoPE table with the reference's growth rule (decoder.rs:234-306).

    ``ensure(required_pos, head_dim, theta)`` grows capacity by doubling from
    1024; new rows are filled on the GPU from the f32 inverse frequencies
    ``1/theta^(2d/head_dim)`` (computed on the host by the library, as the
    reference does). A change of head_dim rebuilds the table from row 0.
    """

    def __init__(self, device: str | torch.device = "cuda"):
        self.device = torch.device(device)
        self.cos = torch.empty(0, dtype=F32, device=self.device)
        self.sin = torch.empty(0, dtype=F32, device=self.device)
        self.cap = 0
        self.head_dim = 0
        self.theta = None

    def ensure(self, required_pos: int, head_dim: int, theta: float) -> None:
        if self.head_dim != head_dim or self.theta != theta:
            self.cap = 0
            self.head_dim = head_dim
            self.theta = theta
            self.cos = torch.empty(0, dtype=F32, device=self.device)
            self.sin = torch.empty(0, dtype=F32, device=self.device)
        if required_pos <= self.cap:
            return
        new_cap = self.cap if self.cap > 0 else 1024
        while new_cap < required_pos:
            new_cap *= 2
        cos = torch.empty(new_cap * head_dim, dtype=F32, device=self.device)
        sin = torch.empty(new_cap * head_dim, dtype=F32, device=self.device)
        if self.cap:
            cos[: self.cap * head_dim].copy_(self.cos)
            sin[: self.cap * head_dim].copy_(self.sin)
        _lib.call("qasr_rope_table_fill_f32", _ptr(cos), _ptr(sin), self.cap, new_cap, head_dim,
                  theta, _stream())
        self.cos, self.sin, self.cap = cos, sin, new_cap

    def cos_at(self, pos: int) -> torch.Tensor:
        return self.cos[pos * self.head_dim:(pos + 1) * self.head_dim]

    def sin_at(self, pos: int) -> torch.Tensor:
        return self.sin[pos * self.head_dim:(pos + 1) * self.head_dim]

    def cos_range(self, start: int, length: int) -> torch.Tensor:
        return self.cos[start * self.head_dim:(start + length) * self.head_dim]

    def sin_range(self, start: int, length: int) -> torch.Tensor:
        return self.sin[start * self.head_dim:(start + length) * self.head_dim]


# ---------------------------------------------------------------------------
# Activations
# ---------------------------------------------------------------------------
def swiglu_multiply(out, gate_up, seq_len: int, intermediate: int) -> None:
    """SwiGLU on the row-interleaved gate/up buffer (kernels/mod.rs:965-985)."""
    _need(out, F32, seq_len * intermediate, "out")
    _need(gate_up, F32, seq_len * 2 * intermediate, "gate_up")
    _lib.call("qasr_swiglu_multiply_f32", _ptr(out), _ptr(gate_up), seq_len, intermediate,
              _stream())


def swiglu_multiply_inplace(gate, up) -> None:
    """``gate = silu(gate) * up`` (kernels/mod.rs:988-994)."""
    n = gate.numel()
    _need(gate, F32, n, "gate")
    _need(up, F32, n, "up")
    _lib.call("qasr_swiglu_split_f32", _ptr(gate), _ptr(gate), _ptr(up), n, _stream())


def swiglu_split(out, gate, up, n: int) -> None:
    """``out = silu(gate) * up`` on split buffers (decode SwiGLU, decoder.rs:916-921)."""
    _need(out, F32, n, "out")
    _need(gate, F32, n, "gate")
    _need(up, F32, n, "up")
    _lib.call("qasr_swiglu_split_f32", _ptr(out), _ptr(gate), _ptr(up), n, _stream())


def silu(x, n: int) -> None:
    """In-place SiLU (kernels/mod.rs:941-946)."""
    _need(x, F32, n, "x")
    _lib.call("qasr_silu_f32", _ptr(x), n, _stream())


def gelu(x, n: int) -> None:
    """In-place tanh-approximation GELU, reference arithmetic (kernels/mod.rs:948-963)."""
    _need(x, F32, n, "x")
    _lib.call("qasr_gelu_tanh_f32", _ptr(x), n, _stream())


def gelu_erf(x, n: int) -> None:
    """In-place exact GELU 0.5*x*(1+erf(x/sqrt(2)))."""
    _need(x, F32, n, "x")
    _lib.call("qasr_gelu_erf_f32", _ptr(x), n, _stream())


# ---------------------------------------------------------------------------
# Position embeddings (encoder)
# ---------------------------------------------------------------------------
def sinusoidal_pe(pe, n_pos: int, d_model: int) -> None:
    """Sinusoidal PE table [n_pos, d_model] (kernels/mod.rs:1213-1226)."""
    _need(pe, F32, n_pos * d_model, "pe")
    _lib.call("qasr_sinusoidal_pe_f32", _ptr(pe), n_pos, d_model, _stream())


def pe_add(x, pe, rows: int, d_model: int, n_pos: int) -> None:
    """``x[r] += pe[r % n_pos]`` (encoder.rs:340-343 with the table reused)."""
    _need(x, F32, rows * d_model, "x")
    _need(pe, F32, n_pos * d_model, "pe")
    _lib.call("qasr_pe_add_f32", _ptr(x), _ptr(pe), rows, d_model, n_pos, _stream())


def pe_add_layer_norm(x, pe, out, weight, bias, rows: int, d_model: int, n_pos: int,
                      eps: float) -> None:
    """``x[r] += pe[r % n_pos]`` then ``out = layer_norm(x)`` in one pass: the
    encoder's PE add (encoder.rs:341-343) and layer 0's LayerNorm of the same
    rows (encoder.rs:370-371); equal to ``pe_add`` + ``layer_norm`` bit for bit."""
    _need(x, F32, rows * d_model, "x")
    _need(pe, F32, n_pos * d_model, "pe")
    _need(out, F32, rows * d_model, "out")
    _need(weight, F32, d_model, "weight")
    _need(bias, F32, d_model, "bias")
    _lib.call("qasr_pe_add_layer_norm_f32", _ptr(x), _ptr(pe), _ptr(out), _ptr(weight), _ptr(bias),
              rows, d_model, n_pos, eps, _stream())


# ---------------------------------------------------------------------------
# Token embeddings (decoder.rs:631-646)
# ---------------------------------------------------------------------------
@dataclass
class QuantWeight:
    """Device view of a .qint8 weight (quantize.rs:77-84): int8 [out_dim, in_dim] + f32 scales."""

    data: torch.Tensor
    scales: torch.Tensor
    out_dim: int
    in_dim: int


def embed_gather_f32(out, table, ids, n: int, dim: int) -> None:
    _need(out, F32, n * dim, "out")
    _need(table, F32, dim, "table")
    _need(ids, I32, n, "ids")
    _lib.call("qasr_embed_gather_f32", _ptr(out), _ptr(table), _ptr(ids), n, dim,
              table.numel() // dim, _stream())


def embed_gather_bf16(out, table, ids, n: int, dim: int) -> None:
    """Batched tok_embed_bf16_to_f32; ``table`` holds bf16 bits as int16 or bfloat16."""
    _need(out, F32, n * dim, "out")
    if table.dtype == torch.bfloat16:
        table = table.view(U16)
    _need(table, U16, dim, "table")
    _need(ids, I32, n, "ids")
    _lib.call("qasr_embed_gather_bf16", _ptr(out), _ptr(table), _ptr(ids), n, dim,
              table.numel() // dim, _stream())


def embed_gather_i8(out, w: QuantWeight, ids, n: int, dim: int) -> None:
    """Batched tok_embed_int8_to_f32."""
    _need(out, F32, n * dim, "out")
    _need(w.data, I8, w.out_dim * dim, "w.data")
    _need(w.scales, F32, w.out_dim, "w.scales")
    _need(ids, I32, n, "ids")
    _lib.call("qasr_embed_gather_i8", _ptr(out), _ptr(w.data), _ptr(w.scales), _ptr(ids), n, dim,
              w.out_dim, _stream())


def _one_id(token_id: int, device) -> torch.Tensor:
    return torch.tensor([token_id], dtype=I32, device=device)


def tok_embed_f32_to_f32(dst, table, token_id: int, dim: int) -> None:
    embed_gather_f32(dst, table, _one_id(token_id, dst.device), 1, dim)


def tok_embed_bf16_to_f32(dst, tok_emb_bf16, token_id: int, dim: int) -> None:
    """One token (decoder.rs:631-636)."""
    embed_gather_bf16(dst, tok_emb_bf16, _one_id(token_id, dst.device), 1, dim)


def tok_embed_int8_to_f32(dst, w: QuantWeight, token_id: int, dim: int) -> None:
    """One token (decoder.rs:639-646)."""
    embed_gather_i8(dst, w, _one_id(token_id, dst.device), 1, dim)


# ---------------------------------------------------------------------------
# INT8
# ---------------------------------------------------------------------------
def quantize_rows_i8(q, scales, x, rows: int, cols: int) -> None:
    """Per-row int8 quantization into caller buffers (quantize.rs:633-662)."""
    _need(q, I8, rows * cols, "q")
    _need(scales, F32, rows, "scales")
    _need(x, F32, rows * cols, "x")
    _lib.call("qasr_quantize_rows_i8", _ptr(q), _ptr(scales), _ptr(x), rows, cols, _stream())


def quantize_f32_to_int8(f32_data, out_dim: int, in_dim: int):
    """Returns ``(int8 data, f32 scales)`` like quantize.rs:633-662 (device tensors)."""
    q = torch.empty(out_dim * in_dim, dtype=I8, device=f32_data.device)
    s = torch.empty(out_dim, dtype=F32, device=f32_data.device)
    quantize_rows_i8(q, s, f32_data, out_dim, in_dim)
    return q, s


def linear_nobias_int8(y, x, w_int8, scales, seq_len: int, in_dim: int, out_dim: int) -> None:
    """W8A32 ``y = scale * (W_int8 @ x)`` (kernels/mod.rs:650-661)."""
    _need(y, F32, seq_len * out_dim, "y")
    _need(x, F32, seq_len * in_dim, "x")
    _need(w_int8, I8, out_dim * in_dim, "w_int8")
    _need(scales, F32, out_dim, "scales")
    _lib.call("qasr_linear_nobias_int8_f32", _ptr(y), _ptr(x), _ptr(w_int8), _ptr(scales),
              seq_len, in_dim, out_dim, _stream())


def linear_nobias_int8_multi(ys, ws: list, x, seq_len: int, in_dim: int) -> None:
    """Several W8A32 projections of the same x in one launch (q/k/v, decoder.rs:881-886);
    ``ws`` are QuantWeights, ``ys[m]`` gets ``seq_len * ws[m].out_dim`` floats."""
    if len(ys) != len(ws):
        raise ValueError("one output per weight")
    for y, w in zip(ys, ws):
        _need(y, F32, seq_len * w.out_dim, "y")
        _need(w.data, I8, w.out_dim * in_dim, "w")
        _need(w.scales, F32, w.out_dim, "scales")
    _need(x, F32, seq_len * in_dim, "x")
    n = len(ws)
    arr = ctypes.c_void_p * max(n, 1)
    _lib.call("qasr_linear_nobias_int8_multi_f32", n, arr(*[y.data_ptr() for y in ys]),
              arr(*[w.data.data_ptr() for w in ws]), arr(*[w.scales.data_ptr() for w in ws]),
              (ctypes.c_size_t * max(n, 1))(*[w.out_dim for w in ws]), _ptr(x), seq_len, in_dim,
              _stream())


def qkv_heads_int8(q, k_cache, v_cache, cache_rows: int, wq: QuantWeight, wk: QuantWeight, wv: QuantWeight,
                   x, seq_len: int, in_dim: int, n_heads: int, n_kv_heads: int, head_dim: int, q_norm_w,
                   k_norm_w, rope: "RopeCache", start_pos: int, eps: float) -> None:
    """A prefill chunk's q/k/v projections + q/k head norms + RoPE + the K/V
    cache rows in one launch (decoder.rs:795-810). Same results, bit for bit, as
    ``linear_nobias_int8_multi`` followed by ``head_rms_norm_rope_kv`` (positions
    None); ``k_cache``/``v_cache`` are the layer's ``[cache_rows, kv_dim]`` blocks.
    head_dim 128, seq_len >= 8 and in_dim % 64 == 0 (else the library raises)."""
    kv = n_kv_heads * head_dim
    _need(q, F32, seq_len * n_heads * head_dim, "q")
    _need(k_cache, F32, cache_rows * kv, "k_cache")
    _need(v_cache, F32, cache_rows * kv, "v_cache")
    for w, rows, name in ((wq, n_heads * head_dim, "wq"), (wk, kv, "wk"), (wv, kv, "wv")):
        _need(w.data, I8, rows * in_dim, name)
        _need(w.scales, F32, rows, name + ".scales")
    _need(x, F32, seq_len * in_dim, "x")
    _need(q_norm_w, F32, head_dim, "q_norm_w")
    _need(k_norm_w, F32, head_dim, "k_norm_w")
    if rope.head_dim != head_dim:
        raise ValueError("RopeCache head_dim does not match")
    _lib.call("qasr_qkv_heads_int8_f32", _ptr(q), _ptr(k_cache), _ptr(v_cache), cache_rows, _ptr(wq.data),
              _ptr(wq.scales), _ptr(wk.data), _ptr(wk.scales), _ptr(wv.data), _ptr(wv.scales), _ptr(x), seq_len,
              in_dim, n_heads, n_kv_heads, head_dim, _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope.cos),
              _ptr(rope.sin), rope.cap, start_pos, eps, _stream())


def norm_slices(hidden: int) -> int:
    """Partial sums of squares per token that ``linear_int8_residual`` writes
    (one per 64 columns of the residual stream)."""
    return (hidden + 63) // 64


def linear_int8_residual(h, ss, x, w: QuantWeight, seq_len: int, in_dim: int, out_dim: int, hg=None,
                         gain=None) -> None:
    """The prefill residual add folded into the o / down projection
    (decoder.rs:821-822, 837-838): ``h += linear_nobias_int8(x, w)`` bit for bit;
    ``ss[t, s]`` = the sum of squares of the updated ``h[t, 64s:64s+64]``, and
    with ``hg``/``gain`` also ``hg = h * gain`` -- what the next folded RMSNorm
    reads. seq_len >= 8 and in_dim % 64 == 0 (else the library raises)."""
    _need(h, F32, seq_len * out_dim, "h")
    _need(ss, F32, seq_len * norm_slices(out_dim), "ss")
    _need(x, F32, seq_len * in_dim, "x")
    _need(w.data, I8, out_dim * in_dim, "w")
    _need(w.scales, F32, out_dim, "scales")
    if (hg is None) != (gain is None):
        raise ValueError("linear_int8_residual: hg and gain go together")
    if hg is not None:
        _need(hg, F32, seq_len * out_dim, "hg")
        _need(gain, F32, out_dim, "gain")
    _lib.call("qasr_linear_int8_residual_f32", _ptr(h), _ptr(ss), _ptr(hg) if hg is not None else None,
              _ptr(gain) if gain is not None else None, _ptr(x), _ptr(w.data), _ptr(w.scales), seq_len, in_dim,
              out_dim, _stream())


def rms_norm_gate_up_swiglu_multiply_int8(out, hg, ss, eps: float, x_norm, w: QuantWeight, seq_len: int,
                                          in_dim: int, intermediate: int) -> None:
    """The prefill post-attention RMSNorm folded into the gate/up GEMM + SwiGLU
    (decoder.rs:826-833): ``hg`` = h * norm gain and ``ss`` from
    ``linear_int8_residual``; each token's outputs are multiplied by its 1 / rms.
    ``x_norm`` ([seq_len, in_dim], may be ``hg``) receives the normalised rows
    only on shapes the folded kernel does not take."""
    _need(out, F32, seq_len * intermediate, "out")
    _need(hg, F32, seq_len * in_dim, "hg")
    _need(ss, F32, seq_len * norm_slices(in_dim), "ss")
    _need(x_norm, F32, seq_len * in_dim, "x_norm")
    _need(w.data, I8, 2 * intermediate * in_dim, "w")
    _need(w.scales, F32, 2 * intermediate, "scales")
    _lib.call("qasr_rms_norm_gate_up_swiglu_multiply_int8_f32", _ptr(out), _ptr(hg), _ptr(ss),
              norm_slices(in_dim), eps, _ptr(x_norm), _ptr(w.data), _ptr(w.scales), seq_len, in_dim,
              intermediate, _stream())


def rms_norm_qkv_heads_int8(q, k_cache, v_cache, cache_rows: int, wq: QuantWeight, wk: QuantWeight,
                            wv: QuantWeight, hg, ss, norm_eps: float, x_norm, seq_len: int, in_dim: int,
                            n_heads: int, n_kv_heads: int, head_dim: int, q_norm_w, k_norm_w, rope: "RopeCache",
                            start_pos: int, eps: float) -> None:
    """``qkv_heads_int8`` on the layer-input RMSNorm folded in: ``hg`` = h *
    input_norm and ``ss`` from ``linear_int8_residual`` (decoder.rs:789-810);
    ``x_norm`` as in ``rms_norm_gate_up_swiglu_multiply_int8``."""
    kv = n_kv_heads * head_dim
    _need(q, F32, seq_len * n_heads * head_dim, "q")
    _need(k_cache, F32, cache_rows * kv, "k_cache")
    _need(v_cache, F32, cache_rows * kv, "v_cache")
    for w, rows, name in ((wq, n_heads * head_dim, "wq"), (wk, kv, "wk"), (wv, kv, "wv")):
        _need(w.data, I8, rows * in_dim, name)
        _need(w.scales, F32, rows, name + ".scales")
    _need(hg, F32, seq_len * in_dim, "hg")
    _need(ss, F32, seq_len * norm_slices(in_dim), "ss")
    _need(x_norm, F32, seq_len * in_dim, "x_norm")
    _need(q_norm_w, F32, head_dim, "q_norm_w")
    _need(k_norm_w, F32, head_dim, "k_norm_w")
    if rope.head_dim != head_dim:
        raise ValueError("RopeCache head_dim does not match")
    _lib.call("qasr_rms_norm_qkv_heads_int8_f32", _ptr(q), _ptr(k_cache), _ptr(v_cache), cache_rows,
              _ptr(wq.data), _ptr(wq.scales), _ptr(wk.data), _ptr(wk.scales), _ptr(wv.data), _ptr(wv.scales),
              _ptr(hg), _ptr(ss), norm_slices(in_dim), norm_eps, _ptr(x_norm), seq_len, in_dim, n_heads,
              n_kv_heads, head_dim, _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope.cos), _ptr(rope.sin), rope.cap,
              start_pos, eps, _stream())


def gate_up_swiglu_int8(out, x, w: QuantWeight, seq_len: int, in_dim: int, intermediate: int) -> None:
    """W8A32 gate/up projection on the interleaved weight + the decode loop's
    SwiGLU (decoder.rs:912-921), one launch; gate/up values are not stored."""
    _need(out, F32, seq_len * intermediate, "out")
    _need(x, F32, seq_len * in_dim, "x")
    _need(w.data, I8, 2 * intermediate * in_dim, "w")
    _need(w.scales, F32, 2 * intermediate, "scales")
    _lib.call("qasr_gate_up_swiglu_int8_f32", _ptr(out), _ptr(x), _ptr(w.data), _ptr(w.scales),
              seq_len, in_dim, intermediate, _stream())


def add_rms_norm_linear_nobias_int8_multi(ys, ws: list, h_out, x, delta, norm_w, in_dim: int,
                                          eps: float) -> None:
    """One decode token: h = x + delta (``delta`` None: h = x), the RMSNorm of h,
    and the projections of the normalised row in one launch (decoder.rs:924->878
    then 881-886). ``h_out`` (None: not written) gets h and must be a different
    buffer from x and delta; ``ys[m]`` equals add_rms_norm + linear_nobias_int8_multi
    bit for bit."""
    if len(ys) != len(ws):
        raise ValueError("one output per weight")
    for y, w in zip(ys, ws):
        _need(y, F32, w.out_dim, "y")
        _need(w.data, I8, w.out_dim * in_dim, "w")
        _need(w.scales, F32, w.out_dim, "scales")
    _need(x, F32, in_dim, "x")
    _need(norm_w, F32, in_dim, "norm_w")
    if delta is not None:
        _need(delta, F32, in_dim, "delta")
    if h_out is not None:
        _need(h_out, F32, in_dim, "h_out")
    n = len(ws)
    arr = ctypes.c_void_p * max(n, 1)
    _lib.call("qasr_add_rms_norm_linear_nobias_int8_multi_f32", n, arr(*[y.data_ptr() for y in ys]),
              arr(*[w.data.data_ptr() for w in ws]), arr(*[w.scales.data_ptr() for w in ws]),
              (ctypes.c_size_t * max(n, 1))(*[w.out_dim for w in ws]), _ptr(h_out), _ptr(x),
              _ptr(delta), _ptr(norm_w), in_dim, eps, _stream())


def add_rms_norm_gate_up_swiglu_int8(out, h_out, x, delta, norm_w, w: QuantWeight, in_dim: int,
                                     intermediate: int, eps: float) -> None:
    """One decode token: the post-attention add + RMSNorm, the gate/up projection
    and the decode SwiGLU in one launch (decoder.rs:908-921); equals add_rms_norm
    followed by gate_up_swiglu_int8 bit for bit."""
    _need(out, F32, intermediate, "out")
    _need(x, F32, in_dim, "x")
    _need(norm_w, F32, in_dim, "norm_w")
    if delta is not None:
        _need(delta, F32, in_dim, "delta")
    if h_out is not None:
        _need(h_out, F32, in_dim, "h_out")
    _need(w.data, I8, 2 * intermediate * in_dim, "w")
    _need(w.scales, F32, 2 * intermediate, "scales")
    _lib.call("qasr_add_rms_norm_gate_up_swiglu_int8_f32", _ptr(out), _ptr(h_out), _ptr(x), _ptr(delta),
              _ptr(norm_w), _ptr(w.data), _ptr(w.scales), in_dim, intermediate, eps, _stream())


def gate_up_swiglu_multiply_int8(out, x, w: QuantWeight, seq_len: int, in_dim: int, intermediate: int) -> None:
    """The prefill's W8A32 gate/up projection on the interleaved weight + swiglu_multiply
    (decoder.rs:831-834; the fast_exp SwiGLU), one launch; gate/up values are not stored."""
    _need(out, F32, seq_len * intermediate, "out")
    _need(x, F32, seq_len * in_dim, "x")
    _need(w.data, I8, 2 * intermediate * in_dim, "w")
    _need(w.scales, F32, 2 * intermediate, "scales")
    _lib.call("qasr_gate_up_swiglu_multiply_int8_f32", _ptr(out), _ptr(x), _ptr(w.data), _ptr(w.scales),
              seq_len, in_dim, intermediate, _stream())


def linear_int8(y, x, w_int8, scales, bias, seq_len: int, in_dim: int, out_dim: int) -> None:
    """W8A32 linear with optional bias (kernels/mod.rs:664-673)."""
    _need(y, F32, seq_len * out_dim, "y")
    _need(x, F32, seq_len * in_dim, "x")
    _need(w_int8, I8, out_dim * in_dim, "w_int8")
    _need(scales, F32, out_dim, "scales")
    if bias is not None:
        _need(bias, F32, out_dim, "bias")
    _lib.call("qasr_linear_int8_f32", _ptr(y), _ptr(x), _ptr(w_int8), _ptr(scales), _ptr(bias),
              seq_len, in_dim, out_dim, _stream())


def interleave_gate_up(gate: QuantWeight, up: QuantWeight) -> QuantWeight:
    """Fused row-interleaved gate/up weight (decoder.rs:701-719), built on the device."""
    inter, hidden = gate.out_dim, gate.in_dim
    if (up.out_dim, up.in_dim) != (inter, hidden):
        raise ValueError("gate and up must have the same shape")
    _need(gate.data, I8, inter * hidden, "gate.data")
    _need(up.data, I8, inter * hidden, "up.data")
    _need(gate.scales, F32, inter, "gate.scales")
    _need(up.scales, F32, inter, "up.scales")
    data = torch.empty(2 * inter * hidden, dtype=I8, device=gate.data.device)
    scales = torch.empty(2 * inter, dtype=F32, device=gate.data.device)
    _lib.call("qasr_interleave_gate_up_i8", _ptr(data), _ptr(scales), _ptr(gate.data),
              _ptr(gate.scales), _ptr(up.data), _ptr(up.scales), inter, hidden, _stream())
    return QuantWeight(data, scales, 2 * inter, hidden)


def gate_up_swiglu_w8a8(out, w: QuantWeight, xq, x_scales, batch: int, in_dim: int,
                        intermediate: int) -> None:
    """W8A8 gate/up projection + SwiGLU on the interleaved weight (int32-exact dots)."""
    _need(out, F32, batch * intermediate, "out")
    _need(w.data, I8, 2 * intermediate * in_dim, "w.data")
    _need(w.scales, F32, 2 * intermediate, "w.scales")
    _need(xq, I8, batch * in_dim, "xq")
    _need(x_scales, F32, batch, "x_scales")
    _lib.call("qasr_gate_up_swiglu_w8a8", _ptr(out), _ptr(w.data), _ptr(w.scales), _ptr(xq),
              _ptr(x_scales), batch, in_dim, intermediate, _stream())


def gate_up_swiglu_w8a8_f32in(out, w: QuantWeight, x, in_dim: int, intermediate: int) -> None:
    """Batch-1 W8A8 gate/up + SwiGLU quantizing the fp32 input vector in-kernel."""
    _need(out, F32, intermediate, "out")
    _need(w.data, I8, 2 * intermediate * in_dim, "w.data")
    _need(w.scales, F32, 2 * intermediate, "w.scales")
    _need(x, F32, in_dim, "x")
    _lib.call("qasr_gate_up_swiglu_w8a8_f32in", _ptr(out), _ptr(w.data), _ptr(w.scales), _ptr(x),
              in_dim, intermediate, _stream())


def pack_w8a8_tiles(w: QuantWeight) -> QuantWeight:
    """MFMA tile layout of an int8 weight (see include/qasr.h); scales are shared."""
    _need(w.data, I8, w.out_dim * w.in_dim, "w.data")
    packed = torch.empty(w.out_dim * w.in_dim, dtype=I8, device=w.data.device)
    _lib.call("qasr_pack_w8a8_tiles", _ptr(packed), _ptr(w.data), w.out_dim, w.in_dim, _stream())
    return QuantWeight(packed, w.scales, w.out_dim, w.in_dim)


def linear_w8a8_packed(y, w_packed: QuantWeight, xq, x_scales, batch: int, in_dim: int, out_dim: int) -> None:
    """Batched W8A8 projection: y[m, n] = ((f32)dot * x_scales[m]) * scales[n]."""
    _need(y, F32, batch * out_dim, "y")
    _need(w_packed.data, I8, out_dim * in_dim, "w.data")
    _need(w_packed.scales, F32, out_dim, "w.scales")
    _need(xq, I8, batch * in_dim, "xq")
    _need(x_scales, F32, batch, "x_scales")
    _lib.call("qasr_linear_w8a8_packed", _ptr(y), _ptr(w_packed.data), _ptr(w_packed.scales), _ptr(xq),
              _ptr(x_scales), batch, in_dim, out_dim, _stream())


def qkv_heads_w8a8_packed(q_out, k_cache, v_cache, cache_rows: int, w_packed: QuantWeight, xq, x_scales,
                          q_norm_w, k_norm_w, rope: "RopeCache", positions, batch: int, in_dim: int,
                          n_heads: int, n_kv_heads: int, head_dim: int, eps: float) -> None:
    """q/k/v projections of ``batch`` streams + q/k head norms + RoPE at each
    stream's position + the K/V cache rows, one launch (decoder.rs:881-895 per
    stream). ``k_cache``/``v_cache``: [batch, cache_rows, n_kv_heads * head_dim]."""
    n = (n_heads + 2 * n_kv_heads) * head_dim
    kv = n_kv_heads * head_dim
    _need(q_out, F32, batch * n_heads * head_dim, "q_out")
    _need(k_cache, F32, batch * cache_rows * kv, "k_cache")
    _need(v_cache, F32, batch * cache_rows * kv, "v_cache")
    _need(w_packed.data, I8, n * in_dim, "w.data")
    _need(w_packed.scales, F32, n, "w.scales")
    _need(xq, I8, batch * in_dim, "xq")
    _need(x_scales, F32, batch, "x_scales")
    _need(q_norm_w, F32, head_dim, "q_norm_w")
    _need(k_norm_w, F32, head_dim, "k_norm_w")
    _need(positions, I32, batch, "positions")
    _lib.call("qasr_qkv_heads_w8a8_packed", _ptr(q_out), _ptr(k_cache), _ptr(v_cache), cache_rows,
              _ptr(w_packed.data), _ptr(w_packed.scales), _ptr(xq), _ptr(x_scales), _ptr(q_norm_w),
              _ptr(k_norm_w), _ptr(rope.cos), _ptr(rope.sin), rope.cap, _ptr(positions), batch, in_dim,
              n_heads, n_kv_heads, head_dim, eps, _stream())


def gate_up_swiglu_w8a8_packed(out, w_packed: QuantWeight, xq, x_scales, batch: int, in_dim: int,
                               intermediate: int) -> None:
    """gate_up_swiglu_w8a8 on a pack_w8a8_tiles weight (same results)."""
    _need(out, F32, batch * intermediate, "out")
    _need(w_packed.data, I8, 2 * intermediate * in_dim, "w.data")
    _need(w_packed.scales, F32, 2 * intermediate, "w.scales")
    _need(xq, I8, batch * in_dim, "xq")
    _need(x_scales, F32, batch, "x_scales")
    _lib.call("qasr_gate_up_swiglu_w8a8_packed", _ptr(out), _ptr(w_packed.data),
              _ptr(w_packed.scales), _ptr(xq), _ptr(x_scales), batch, in_dim, intermediate,
              _stream())
