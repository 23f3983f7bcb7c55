"""Device-resident INT8 decoder step: the reference's ``DecoderInt8`` decode
(crates/qwen-asr/src/decoder.rs:848-965) over the C-ABI kernels.

Per layer, in the reference's order:
  the previous layer's residual add + input RMSNorm + q/k/v projections (one
  launch), q/k head RMSNorm + RoPE, the K/V rows written into the cache and
  causal attention over the layer's cache block (one launch with the keys
  split over workgroups, then the merge), o projection, residual add +
  post-attention RMSNorm + gate/up projection + SwiGLU (one launch), down
  projection: 6 launches (7 below 256 cached keys, where attention does not
  split and the head norm runs as its own launch).
The fused add + RMSNorm + projection launches normalise the row inside every
workgroup, in the element order of the standalone add_rms_norm kernel, so the
results equal the unfused sequence (``fuse_norms=False``: add_rms_norm, then
the projection; the head norm kernel, then attention) bit for bit. The residual stream alternates between two
buffers, since no workgroup may write the row the others still read.
Then the last residual add + final RMSNorm and the INT8 lm_head with the greedy
argmax (decoder.rs:929-963). Everything stays on the device: the token id is
written to a device int32, and the hidden state, KV cache and RoPE tables
never leave HBM.

``DecoderInt8.prefill`` runs the reference's INT8 prefill
(decoder.rs:751-847) for a chunk of tokens: per layer RMSNorm (fused with the
previous layer's residual add), q/k/v (one matrix-core GEMM launch), q/k head
RMSNorm + RoPE with the chunk's K/V rows written into the cache (in the q/k/v
GEMM's epilogue where that launch fills the chip, else a launch of its own),
causal attention over the cache (matrix cores), o, residual add +
post-attention RMSNorm, gate/up with the prefill SwiGLU (fast_exp form) in its
epilogue, down: 7 or 8 launches per layer, then the last residual add.

Weights come from ``qint8.load_decoder_int8`` (or any dict of the same
layout); ``DecoderInt8.decode`` runs one token and can be captured in a HIP
graph (no host synchronisation, no allocation after construction for a fixed
position).
"""
from __future__ import annotations

import math

import torch

from . import kernels as K


class DecoderInt8:
    def __init__(self, weights: dict, hidden: int, intermediate: int, n_layers: int, n_heads: int = 16,
                 n_kv_heads: int = 8, head_dim: int = 128, eps: float = 1e-6, theta: float = 1e6,
                 vocab: int | None = None, max_seq: int = 256, device="cuda",
                 fuse_norms: bool | None = None, fuse_prefill_heads: bool | None = None,
                 fuse_prefill_norms: bool | None = None):
        self.w = weights
        self.H, self.I, self.L = hidden, intermediate, n_layers
        self.nq, self.nk, self.hd = n_heads, n_kv_heads, head_dim
        self.eps, self.theta = eps, theta
        lm = weights.get("lm_head") or weights["tok_embeddings"]  # tied weights: decoder.rs:951-954
        self.lm = lm
        self.vocab = vocab if vocab is not None else lm.out_dim
        dev = device
        f32 = dict(dtype=torch.float32, device=dev)
        # the fused launches take rows of 1024..8192 floats in steps of 1024
        ok = hidden % 1024 == 0 and 1024 <= hidden <= 8192
        self.fuse_norms = ok if fuse_norms is None else (fuse_norms and ok)
        # prefill q/k/v with the head norms, RoPE and cache rows in the GEMM's
        # epilogue (one workgroup per 128-row head x 64 tokens): None takes it
        # where that launch fills the chip (>= 256 workgroups); below, the
        # unfused split-K GEMM + head kernel is faster
        self.fuse_prefill_heads = fuse_prefill_heads
        # prefill residual adds folded into the o / down GEMMs and the RMSNorms
        # into the q/k/v and gate/up GEMMs' staging (None: wherever the GEMMs run)
        self.fuse_prefill_norms = fuse_prefill_norms
        self.x = torch.zeros(hidden, **f32)
        self.x2 = torch.zeros(hidden, **f32)  # the residual's other buffer (fused path)
        self.x_norm = torch.empty(hidden, **f32)
        self.q = torch.empty(n_heads * head_dim, **f32)
        self.k = torch.empty(n_kv_heads * head_dim, **f32)
        self.v = torch.empty(n_kv_heads * head_dim, **f32)
        self.attn = torch.empty(n_heads * head_dim, **f32)
        self.proj = torch.empty(hidden, **f32)
        self.ffn = torch.empty(intermediate, **f32)
        self.down = torch.empty(hidden, **f32)
        self.logits = torch.empty(self.vocab, **f32)
        self.token = torch.empty(1, dtype=torch.int32, device=dev)
        self.kv = K.KvCache(n_layers, max_seq, n_kv_heads * head_dim, dev)
        self.rope = K.RopeCache(dev)
        self.attn_ws = K.attention_workspace(1, n_heads, head_dim, dev)
        self.lm_ws = K.lm_head_workspace(self.vocab, dev)
        self.scale = 1.0 / math.sqrt(head_dim)

    def _ensure_prefill(self, T: int) -> None:
        if getattr(self, "_pcap", 0) >= T:
            return
        f32 = dict(dtype=torch.float32, device=self.x.device)
        H, I, q_dim, kv_dim = self.H, self.I, self.nq * self.hd, self.nk * self.hd
        self.px = torch.empty(T * H, **f32)
        self.pxn = torch.empty(T * H, **f32)
        self.pq = torch.empty(T * q_dim, **f32)
        self.pk = torch.empty(T * kv_dim, **f32)
        self.pv = torch.empty(T * kv_dim, **f32)
        self.pattn = torch.empty(T * q_dim, **f32)
        self.pproj = torch.empty(T * H, **f32)
        self.pgate = torch.empty(T * I, **f32)
        self.pffn = torch.empty(T * H, **f32)
        self.pss = torch.empty(T * K.norm_slices(H), **f32)  # per-token partial sums of squares
        self._pcap = T

    def _check_pos(self, pos: int | None, what: str) -> int:
        """The reference takes the position from the cache length
        (decoder.rs:771, 866): a position other than ``kv.len`` would leave rows
        the cache does not count (a later growth copies ``kv.len`` rows only)."""
        if pos is None:
            return self.kv.len
        if pos != self.kv.len:
            raise ValueError(f"{what}: position {pos} != cache length {self.kv.len} "
                             "(set kv.len for an externally filled cache)")
        return pos

    def prepare_prefill(self, start_pos: int | None, T: int) -> None:
        """Host-side growth before a prefill of T tokens at start_pos
        (decoder.rs:770-781): cache capacity, RoPE rows, the chunk's buffers.
        ``start_pos`` must equal the cache length (None: take it from there)."""
        start_pos = self._check_pos(start_pos, "prepare_prefill")
        if start_pos + T > self.kv.max_seq:
            self.kv.grow(start_pos + T + 1024)
        self.rope.ensure(start_pos + T, self.hd, self.theta)
        self._ensure_prefill(T)

    def prefill_heads_fused(self, T: int) -> bool:
        """Whether a prefill of T tokens runs q/k/v with the heads in one launch."""
        fits = self.hd == 128 and self.H % 64 == 0 and T >= 8
        if self.fuse_prefill_heads is None:
            return fits and (self.nq + 2 * self.nk) * ((T + 63) // 64) >= 256
        return self.fuse_prefill_heads and fits

    def prefill_norms_folded(self, T: int) -> bool:
        """Whether a prefill of T tokens folds the residual adds into the o / down
        GEMMs and the RMSNorms into the following GEMMs (the GEMM path: T >= 8,
        every in_dim a multiple of 64)."""
        fits = T >= 8 and self.H % 64 == 0 and (self.nq * self.hd) % 64 == 0 and self.I % 64 == 0
        return fits and self.fuse_prefill_norms is not False

    def prefill(self, embeds: torch.Tensor, T: int, start_pos: int | None = None) -> None:
        """T tokens at positions start_pos.. (decoder.rs:751-847): writes cache rows
        start_pos..start_pos+T-1 of every layer; ``self.px[:T*H]`` receives the
        residual stream after the last layer. Call ``prepare_prefill`` first."""
        start_pos = self._check_pos(start_pos, "prefill")
        H, I, nq, nk, hd, eps = self.H, self.I, self.nq, self.nk, self.hd, self.eps
        q_dim = nq * hd
        total = start_pos + T
        fused_heads = self.prefill_heads_fused(T)
        fold = self.prefill_norms_folded(T)
        x = self.px
        x[:T * H].copy_(embeds[:T * H])
        layers = self.w["layers"]
        for l, lw in enumerate(layers):
            kb, vb = self.kv.k_layer_block(l), self.kv.v_layer_block(l)
            if fold and l > 0 and fused_heads:  # input norm: h * gain and the sums of squares from down
                K.rms_norm_qkv_heads_int8(self.pq, kb, vb, self.kv.max_seq, lw["wq"], lw["wk"], lw["wv"], self.pxn,
                                          self.pss, eps, self.pxn, T, H, nq, nk, hd, lw["q_norm"], lw["k_norm"],
                                          self.rope, start_pos, eps)
            else:
                if l == 0 or fold:  # fold: the residual add happened in the down GEMM
                    K.rms_norm(self.pxn, x, lw["input_norm"], T, H, eps)
                else:  # previous layer's residual add (decoder.rs:837-838) + this layer's input norm
                    K.add_rms_norm(x, self.pffn, lw["input_norm"], self.pxn, T, H, eps)
                self._prefill_qkv(l, lw, T, start_pos, fused_heads)
            K.causal_attention(self.pattn, self.pq, kb, vb, T, total, nq, nk, hd, self.scale, start_pos)
            wo, dn = lw["wo"], lw["down"]
            if fold:
                K.linear_int8_residual(x, self.pss, self.pattn, wo, T, q_dim, H, self.pxn, lw["post_attn_norm"])
                K.rms_norm_gate_up_swiglu_multiply_int8(self.pgate, self.pxn, self.pss, eps, self.pxn,
                                                        lw["gate_up"], T, H, I)
                nxt = layers[l + 1]["input_norm"] if l + 1 < len(layers) and fused_heads else None
                K.linear_int8_residual(x, self.pss, self.pgate, dn, T, I, H, self.pxn if nxt is not None else None,
                                       nxt)
            else:
                K.linear_nobias_int8(self.pproj, self.pattn, wo.data, wo.scales, T, q_dim, H)
                K.add_rms_norm(x, self.pproj, lw["post_attn_norm"], self.pxn, T, H, eps)
                K.gate_up_swiglu_multiply_int8(self.pgate, self.pxn, lw["gate_up"], T, H, I)
                K.linear_nobias_int8(self.pffn, self.pgate, dn.data, dn.scales, T, I, H)
        if not fold:
            K.add_inplace(x, self.pffn, T * H)
        self.kv.len = total

    def _prefill_qkv(self, l: int, lw: dict, T: int, start_pos: int, fused_heads: bool) -> None:
        """q/k/v of the normalised rows in ``self.pxn`` with the head norms, RoPE
        and the layer's cache rows (decoder.rs:795-810)."""
        nq, nk, hd, eps, H = self.nq, self.nk, self.hd, self.eps, self.H
        kb, vb = self.kv.k_layer_block(l), self.kv.v_layer_block(l)
        if fused_heads:
            K.qkv_heads_int8(self.pq, kb, vb, self.kv.max_seq, lw["wq"], lw["wk"], lw["wv"], self.pxn, T, H,
                             nq, nk, hd, lw["q_norm"], lw["k_norm"], self.rope, start_pos, eps)
        else:
            K.linear_nobias_int8_multi([self.pq, self.pk, self.pv], [lw["wq"], lw["wk"], lw["wv"]],
                                       self.pxn, T, H)
            K.head_rms_norm_rope_kv(self.pq, self.pk, self.pv, lw["q_norm"], lw["k_norm"], self.rope, None,
                                    start_pos, T, nq, nk, hd, eps, kb, vb, self.kv.max_seq)

    def prepare(self, pos: int | None = None) -> None:
        """Host-side growth before a decode at ``pos`` (decoder.rs:866-872):
        cache capacity and RoPE rows. Nothing here runs in the timed step.
        ``pos`` must equal the cache length (None: take it from there)."""
        pos = self._check_pos(pos, "prepare")
        if pos >= self.kv.max_seq:
            self.kv.grow(pos + 1024)
        self.rope.ensure(pos + 1, self.hd, self.theta)

    def decode(self, embed: torch.Tensor, pos: int | None = None) -> None:
        """One token at position ``pos`` (the cache holds rows 0..pos-1):
        ``self.token`` receives the greedy next token, ``self.x_norm`` the final
        normed hidden state. Call ``prepare(pos)`` first."""
        pos = self._check_pos(pos, "decode")
        if self.fuse_norms:
            self._decode_fused(embed, pos)
            return
        H, I, nq, nk, hd, eps = self.H, self.I, self.nq, self.nk, self.hd, self.eps
        self.x.copy_(embed)
        for l, lw in enumerate(self.w["layers"]):
            if l == 0:
                K.rms_norm(self.x_norm, self.x, lw["input_norm"], 1, H, eps)
            else:  # previous layer's residual add fused with this layer's input norm
                K.add_rms_norm(self.x, self.down, lw["input_norm"], self.x_norm, 1, H, eps)
            K.linear_nobias_int8_multi([self.q, self.k, self.v], [lw["wq"], lw["wk"], lw["wv"]],
                                       self.x_norm, 1, H)
            K.head_rms_norm_rope_kv(self.q, self.k, self.v, lw["q_norm"], lw["k_norm"], self.rope, None,
                                    pos, 1, nq, nk, hd, eps, self.kv.k_layer_block(l),
                                    self.kv.v_layer_block(l), self.kv.max_seq)
            K.causal_attention_split(self.attn, self.q, self.kv.k_layer_block(l), self.kv.v_layer_block(l),
                                     1, pos + 1, nq, nk, hd, self.scale, pos, self.attn_ws)
            wo = lw["wo"]
            K.linear_nobias_int8(self.proj, self.attn, wo.data, wo.scales, 1, nq * hd, H)
            K.add_rms_norm(self.x, self.proj, lw["post_attn_norm"], self.x_norm, 1, H, eps)
            K.gate_up_swiglu_int8(self.ffn, self.x_norm, lw["gate_up"], 1, H, I)
            dn = lw["down"]
            K.linear_nobias_int8(self.down, self.ffn, dn.data, dn.scales, 1, I, H)
        K.add_rms_norm(self.x, self.down, self.w["norm"], self.x_norm, 1, H, eps)
        K.lm_head_int8_argmax(self.token, self.logits, self.x_norm, self.lm, 1, H, self.vocab, self.lm_ws)

    def _decode_fused(self, embed: torch.Tensor, pos: int) -> None:
        H, I, nq, nk, hd, eps = self.H, self.I, self.nq, self.nk, self.hd, self.eps
        h, h2 = self.x, self.x2
        h.copy_(embed)
        for l, lw in enumerate(self.w["layers"]):
            qkv_w = [lw["wq"], lw["wk"], lw["wv"]]
            if l == 0:
                K.add_rms_norm_linear_nobias_int8_multi([self.q, self.k, self.v], qkv_w, None, h, None,
                                                        lw["input_norm"], H, eps)
            else:  # previous layer's residual add + this layer's input norm + q/k/v
                K.add_rms_norm_linear_nobias_int8_multi([self.q, self.k, self.v], qkv_w, h2, h, self.down,
                                                        lw["input_norm"], H, eps)
                h, h2 = h2, h
            K.decode_attention(self.attn, self.q, self.k, self.v, lw["q_norm"], lw["k_norm"], self.rope, pos,
                               nq, nk, hd, eps, self.scale, self.kv.k_layer_block(l), self.kv.v_layer_block(l),
                               self.kv.max_seq, self.attn_ws)
            wo = lw["wo"]
            K.linear_nobias_int8(self.proj, self.attn, wo.data, wo.scales, 1, nq * hd, H)
            K.add_rms_norm_gate_up_swiglu_int8(self.ffn, h2, h, self.proj, lw["post_attn_norm"], lw["gate_up"],
                                               H, I, eps)
            h, h2 = h2, h
            dn = lw["down"]
            K.linear_nobias_int8(self.down, self.ffn, dn.data, dn.scales, 1, I, H)
        K.add_rms_norm(h, self.down, self.w["norm"], self.x_norm, 1, H, eps)
        K.lm_head_int8_argmax(self.token, self.logits, self.x_norm, self.lm, 1, H, self.vocab, self.lm_ws)

    def finish(self, pos: int | None = None) -> None:
        """The cache now holds rows 0..pos (decoder.rs:926)."""
        pos = self._check_pos(pos, "finish")
        self.kv.len = pos + 1


class DecoderInt8Batched:
    """B independent decode streams through the INT8 decoder in one pass per
    layer: the reference's decode step (decoder.rs:848-965) for every stream,
    each at its own position (its own cache length), batched on the device.

    Each stream has its own KV cache with the reference's layout; layer l's
    blocks of all streams are ``k[l]``/``v[l]`` = ``[batch, cache_rows, kv_dim]``
    (stream m's block is what the reference's attention reads for it). Per
    layer, in the reference's order, over all streams at once:
      residual add + input RMSNorm; the q/k/v projections (one matrix-core
      launch for the three, the reference's W8A32 arithmetic); q/k head
      RMSNorm + RoPE at each stream's position with its K/V rows stored into
      its cache; attention of each stream over its own rows 0..pos (the
      streams walked longest first, ``attn_chunked`` below); o;
      residual add + post-attention RMSNorm; gate/up with the decode loop's
      SwiGLU in the GEMM epilogue; down.
    Then the last residual add + final RMSNorm and the lm_head with each
    stream's greedy argmax. ``positions`` (device int32) holds each stream's
    position; ``finish`` advances them all by one (decoder.rs:926).

    ``w8a8=True`` runs the four projections on int8 matrix cores with each
    stream's activation row quantized per row (quantize.rs:633-662 arithmetic),
    the c5 way: add + RMSNorm + quantization in one launch; q/k/v with the head
    norms, RoPE and the K/V cache rows in the GEMM epilogue; attention, its
    rows quantized in the launch after it (which also merges key chunks); o;
    add + RMSNorm + quantization; gate/up with
    SwiGLU in the epilogue; the SwiGLU rows quantized, down. The int8 weights
    are the same; the activations are rounded to int8 at those four points,
    so the results follow the reference's within that rounding, not 1e-5.
    ``lm_head_w8a8`` (default: with ``w8a8``, when the vocabulary is a
    multiple of 128 and hidden one of 1024..6144 in the W8A8 projection's
    steps) makes the lm_head one too: the final add + RMSNorm quantizes the
    rows in the same launch, the logits are ((f32)dot * x_scale) * row_scale,
    each stream's argmax follows; otherwise the lm_head stays W8A32.

    ``attn_chunked`` (default: when batch * n_kv_heads < 1024) also cuts each
    stream's keys into chunks for the attention, to give a small batch enough
    workgroups; the results are the same either way within 1e-6.
    """

    def __init__(self, weights: dict, hidden: int, intermediate: int, n_layers: int, batch: int,
                 cache_rows: int, n_heads: int = 16, n_kv_heads: int = 8, head_dim: int = 128,
                 eps: float = 1e-6, theta: float = 1e6, vocab: int | None = None, device="cuda",
                 w8a8: bool = False, attn_chunked: bool | None = None, lm_head_w8a8: bool | None = None):
        self.w = weights
        self.H, self.I, self.L, self.B = hidden, intermediate, n_layers, batch
        self.nq, self.nk, self.hd = n_heads, n_kv_heads, head_dim
        self.eps, self.theta = eps, theta
        self.lm = weights.get("lm_head") or weights["tok_embeddings"]  # tied weights: decoder.rs:951-954
        self.vocab = vocab if vocab is not None else self.lm.out_dim
        self.rows = cache_rows
        kv = n_kv_heads * head_dim
        f32 = dict(dtype=torch.float32, device=device)
        B = batch
        self.k = torch.zeros(n_layers, B * cache_rows * kv, **f32)
        self.v = torch.zeros(n_layers, B * cache_rows * kv, **f32)
        self.positions = torch.zeros(B, dtype=torch.int32, device=device)
        self.x = torch.zeros(B * hidden, **f32)
        self.x_norm = torch.empty(B * hidden, **f32)
        self.q = torch.empty(B * n_heads * head_dim, **f32)
        self.kk = torch.empty(B * kv, **f32)
        self.vv = torch.empty(B * kv, **f32)
        self.attn = torch.empty(B * n_heads * head_dim, **f32)
        self.proj = torch.empty(B * hidden, **f32)
        self.ffn = torch.empty(B * intermediate, **f32)
        self.down = torch.empty(B * hidden, **f32)
        self.logits = torch.empty(B * self.vocab, **f32)
        self.tokens = torch.empty(B, dtype=torch.int32, device=device)
        self.rope = K.RopeCache(device)
        self.rope.ensure(cache_rows, head_dim, theta)
        self.scale = 1.0 / math.sqrt(head_dim)
        # Attention walks the streams longest first (one order per step). With
        # B * n_kv_heads >= 1024 workgroups that alone balances the GPU and
        # each (stream, kv head) walks all its keys; below it the keys are also
        # cut into chunks (merged in a second launch) to give the GPU work.
        if attn_chunked is None:
            attn_chunked = B * n_kv_heads < 1024
        self.attn_ws = K.batched_decode_workspace(B, n_heads, head_dim, cache_rows, device) if attn_chunked else None
        self.order = torch.empty(2 * B, dtype=torch.int32, device=device)
        self.w8a8 = w8a8
        if w8a8:
            i8 = dict(dtype=torch.int8, device=device)
            self.xq, self.xs = torch.empty(B * hidden, **i8), torch.empty(B, **f32)
            self.aq, self.as_ = torch.empty(B * n_heads * head_dim, **i8), torch.empty(B, **f32)
            self.fq, self.fs = torch.empty(B * intermediate, **i8), torch.empty(B, **f32)
            self.packed = []
            for lw in weights["layers"]:  # the same int8 weights, re-laid into MFMA tiles once
                ws = [lw["wq"], lw["wk"], lw["wv"]]
                qkv = K.QuantWeight(torch.cat([w.data.reshape(-1) for w in ws]),
                                    torch.cat([w.scales for w in ws]), sum(w.out_dim for w in ws), hidden)
                self.packed.append({k: K.pack_w8a8_tiles(w) for k, w in
                                    (("qkv", qkv), ("wo", lw["wo"]), ("gate_up", lw["gate_up"]),
                                     ("down", lw["down"]))})
        fits = self.vocab % 128 == 0 and self.vocab == self.lm.out_dim and hidden in (1024, 2048, 3072, 4096, 6144)
        if lm_head_w8a8 is None:
            lm_head_w8a8 = w8a8 and fits
        if lm_head_w8a8 and not (w8a8 and fits):
            raise ValueError("lm_head_w8a8 needs w8a8=True, a vocabulary that is a multiple of 128 "
                             "and hidden in 1024..6144 (steps of 1024, or 6144)")
        self.lm_head_w8a8 = lm_head_w8a8
        if lm_head_w8a8:
            self.lm_packed = K.pack_w8a8_tiles(self.lm)

    def _layer_w8a8(self, l: int, lw: dict) -> None:
        H, I, B, nq, nk, hd, eps = self.H, self.I, self.B, self.nq, self.nk, self.hd, self.eps
        pk = self.packed[l]
        kb, vb = self.k[l], self.v[l]
        K.add_rms_norm_quant(self.x, None if l == 0 else self.down, lw["input_norm"], None, self.xq, self.xs,
                             B, H, eps)
        K.qkv_heads_w8a8_packed(self.q, kb, vb, self.rows, pk["qkv"], self.xq, self.xs, lw["q_norm"],
                                lw["k_norm"], self.rope, self.positions, B, H, nq, nk, hd, eps)
        K.batched_decode_attention(self.attn, self.q, kb, vb, self.rows, self.positions, B, nq, nk, hd,
                                   self.scale, self.attn_ws, self.aq, self.as_, self.order)  # + rows quantized
        K.linear_w8a8_packed(self.proj, pk["wo"], self.aq, self.as_, B, nq * hd, H)
        K.add_rms_norm_quant(self.x, self.proj, lw["post_attn_norm"], None, self.xq, self.xs, B, H, eps)
        K.gate_up_swiglu_w8a8_packed(self.ffn, pk["gate_up"], self.xq, self.xs, B, H, I)
        K.quantize_rows_i8(self.fq, self.fs, self.ffn, B, I)
        K.linear_w8a8_packed(self.down, pk["down"], self.fq, self.fs, B, I, H)

    def decode(self, embeds: torch.Tensor) -> None:
        """One token for every stream (``embeds``: [batch, hidden]) at its
        position: ``tokens`` receives each stream's greedy next token,
        ``x_norm`` the final normed hidden states. Positions outside the cache
        give NaN rows and write no cache row."""
        H, I, B, nq, nk, hd, eps = self.H, self.I, self.B, self.nq, self.nk, self.hd, self.eps
        self.x.copy_(embeds[:B * H])
        K.batched_decode_order(self.order, self.positions, B, self.rows)
        for l, lw in enumerate(self.w["layers"]):
            if self.w8a8:
                self._layer_w8a8(l, lw)
                continue
            if l == 0:
                K.rms_norm(self.x_norm, self.x, lw["input_norm"], B, H, eps)
            else:  # previous layer's residual add + this layer's input norm
                K.add_rms_norm(self.x, self.down, lw["input_norm"], self.x_norm, B, H, eps)
            K.linear_nobias_int8_multi([self.q, self.kk, self.vv], [lw["wq"], lw["wk"], lw["wv"]],
                                       self.x_norm, B, H)
            kb, vb = self.k[l], self.v[l]
            K.head_rms_norm_rope_kv(self.q, self.kk, self.vv, lw["q_norm"], lw["k_norm"], self.rope,
                                    self.positions, 0, B, nq, nk, hd, eps, kb, vb, self.rows)
            K.batched_decode_attention(self.attn, self.q, kb, vb, self.rows, self.positions, B, nq, nk, hd,
                                       self.scale, self.attn_ws, order=self.order)
            wo = lw["wo"]
            K.linear_nobias_int8(self.proj, self.attn, wo.data, wo.scales, B, nq * hd, H)
            K.add_rms_norm(self.x, self.proj, lw["post_attn_norm"], self.x_norm, B, H, eps)
            K.gate_up_swiglu_int8(self.ffn, self.x_norm, lw["gate_up"], B, H, I)
            dn = lw["down"]
            K.linear_nobias_int8(self.down, self.ffn, dn.data, dn.scales, B, I, H)
        if self.lm_head_w8a8:
            K.add_rms_norm_quant(self.x, self.down, self.w["norm"], self.x_norm, self.xq, self.xs, B, H, eps)
            K.linear_w8a8_packed(self.logits, self.lm_packed, self.xq, self.xs, B, H, self.vocab)
            K.argmax_rows(self.tokens, self.logits, B, self.vocab)
            return
        K.add_rms_norm(self.x, self.down, self.w["norm"], self.x_norm, B, H, eps)
        K.lm_head_int8_argmax(self.tokens, self.logits, self.x_norm, self.lm, B, H, self.vocab)

    def finish(self) -> None:
        """Every stream's cache now holds one more row (decoder.rs:926)."""
        self.positions.add_(1)
