#!/usr/bin/env python3
"""Benchmark of the fused-layer kernel path on one MI355X.

    python bench.py [--workload c5] [--configs c1,c1_cold,...] [--steps K] [--warmup W] [--gpus 1]

Workloads (shapes of the Qwen3-ASR decoder/encoder; synthetic seeded data,
random-init weights -- no checkpoints):
  c1       0.6B decode-token chain, B=1: add+RMSNorm[1,1024] + q/k head-norm+RoPE + SwiGLU[3072] (LLC-hot)
  c1_cold  c1 with every step's inputs read from HBM (caches flushed between timed replays)
  c2       0.6B prefill chain, T=512: embed gather + add+RMSNorm + q/k norm+RoPE + SwiGLU
  c3       audio-encoder ops: PE add + LayerNorm on [3000,896], erf-GELU on [3000,3584]
  c3_fused c3 with the PE add folded into the LayerNorm that reads its rows
  c4       1.7B INT8 decode gate/up matvec + SwiGLU, B=1, 28 distinct layers per step
  c5       1.7B batched decode, B=256: add+RMSNorm+quantize, q/k norm+RoPE, INT8 MFMA gate/up GEMM+SwiGLU
           (the default, headline workload)
  c5_b32   c5 at B=32 (one GPU's data-parallel share of 256 streams over 8)
  w8a32_decode  1.7B INT8 decode projections via the W8A32 drop-in (q/k/v/o, gate/up, down), 28 layers
  attn_decode   1.7B decode attention at position 2047 (keys split over workgroups), 28 layers
  attn_prefill  0.6B causal prefill attention, T=512
  lm_head       0.6B INT8 lm_head [151936,1024] logits + greedy argmax, B=1
  decode_step   1.7B INT8 decode of one token, all 28 layers + lm_head argmax on the device (tokens/s)
  prefill_step  0.6B INT8 prefill of 512 tokens through all 28 layers (tokens/s)

A step is one pass of the workload's kernel chain over one buffer set; sets
rotate so the working set exceeds the 256 MB last-level cache. Steps are
captured once into a HIP graph; the graph of K steps is replayed at least 5
times (and for at least 100 steps), each replay bracketed by synchronisation
and HIP events on the launch stream, and the median per step is reported with
p10/p90/min. Each kernel's duration is measured the same way (its launches
alone, K of them), and its algorithmic bytes per launch give
roofline.achieved.

Prints ONE JSON line: the headline workload's value, roofline and CPU
baseline, and under "configs" the other workloads measured in the same run,
each with its per-kernel figures and its own CPU baseline. The CPU baseline is
the oracle (a C restatement of the reference Rust kernels, compiled here with
-march=native) timed on this host for a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fused-layer-kernel GB/s (% MI355X HBM peak) + decode tokens/s, 0.6B/1.7B shapes"
HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
LLC_BYTES = 256 << 20
ROTATE_BYTES = 2 * LLC_BYTES  # each kernel's rotating footprint must exceed 2x the LLC
FLUSH_BYTES = 4 * LLC_BYTES   # written before every timed replay of a cold workload

DEC_0_6B = dict(hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, inter=3072, eps=1e-6, theta=1e6)
DEC_1_7B = dict(hidden=2048, n_heads=16, n_kv_heads=8, head_dim=128, inter=6144, eps=1e-6, theta=1e6)
ENC_0_6B = dict(d_model=896, ffn=3584, eps=1e-5, pe_rows=13)
VOCAB = 151936
F = 4  # bytes per fp32


def sets_for(bytes_per_set: int, minimum: int = 2) -> int:
    return max(minimum, math.ceil(ROTATE_BYTES / max(1, bytes_per_set)))


# ---------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------
class Workload:
    name = ""
    description = ""
    unit_tokens = 1  # tokens per step (for tokens/s)
    tokens_per_step = 1.0  # tokens a step advances (28 layers make one decode token)
    step_bytes = 0   # algorithmic bytes per step
    dtype = "f32"    # arithmetic type of the path
    steps_hint = 200  # K of the timed region (a cold workload rotates at least K buffer sets)
    hot = False       # True: the workload is meant to run from the caches (no flush before replays)
    min_steps = 1     # the timed region holds at least this many steps
    rotation = None   # distinct buffer sets a kernel's launches rotate over (None: at least K)

    def __init__(self, dev, torch):
        self.dev = dev
        self.torch = torch
        self.gen = torch.Generator(device=dev).manual_seed(1234)
        self.kernels = {}  # name -> (launch(i), algorithmic bytes per launch)

    def randn(self, n, scale=1.0, mean=0.0):
        t = self.torch.randn(n, generator=self.gen, device=self.dev)
        if scale != 1.0:
            t.mul_(scale)
        if mean != 0.0:
            t.add_(mean)
        return t

    def step(self, i: int) -> None:
        for spec in self.kernels.values():
            spec[0](i)

    def config(self) -> dict:
        return {}


class C1DecodeChain(Workload):
    name = "c1"
    description = ("qwen3-asr-0.6b decode-token chain B=1: add+RMSNorm[1,1024] + q/k head-RMSNorm"
                   "+RoPE(theta 1e6, pos~U[0,511]) + SwiGLU[3072]")
    unit_tokens = 1
    hot = True
    min_steps = 1000  # the configuration's 1000 repetitions per timed region

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = DEC_0_6B
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        self.S = self.n_sets()
        self.rotation = self.S
        self.x = [self.randn(H) for _ in range(self.S)]
        self.d = [self.randn(H) for _ in range(self.S)]
        self.y = [torch.empty(H, device=dev) for _ in range(self.S)]
        self.q = [self.randn(nq * hd) for _ in range(self.S)]
        self.k = [self.randn(nk * hd) for _ in range(self.S)]
        self.g = [self.randn(I) for _ in range(self.S)]
        self.u = [self.randn(I) for _ in range(self.S)]
        self.o = [torch.empty(I, device=dev) for _ in range(self.S)]
        self.w = self.randn(H, 0.1, 1.0)
        self.qw, self.kw = self.randn(hd, 0.1, 1.0), self.randn(hd, 0.1, 1.0)
        self.rope = K.RopeCache(dev)
        self.rope.ensure(512, hd, c["theta"])
        self.pos = [torch.randint(0, 512, (1,), generator=self.gen, device=dev, dtype=torch.int32)
                    for _ in range(self.S)]
        S = self.S
        self.kernels = {
            "add_rms_norm": (lambda i: K.add_rms_norm(self.x[i % S], self.d[i % S], self.w, self.y[i % S], 1, H, c["eps"]),
                             5 * H * F),
            "head_rms_norm_rope": (lambda i: K.head_rms_norm_rope(
                self.q[i % S], self.k[i % S], self.qw, self.kw, self.rope.cos, self.rope.sin,
                self.pos[i % S], 1, nq, nk, hd, c["eps"]),
                2 * (nq + nk) * hd * F + 2 * hd * F + 2 * hd * F + 4),
            "swiglu": (lambda i: K.swiglu_split(self.o[i % S], self.g[i % S], self.u[i % S], I), 3 * I * F),
        }
        self.step_bytes = sum(b for _, b in self.kernels.values())
        self.tokens_per_step = 1.0 / 28  # one layer's chain; 28 layers make a token

    def n_sets(self) -> int:
        return 64  # 5.4 MB of inputs: the rotation stays in the last-level cache (hot)

    def config(self):
        return {"batch": 1, "hidden": 1024, "heads": "16q/8kv x 128", "intermediate": 3072,
                "buffer_sets": self.S, "cache": "hot (64 sets, 5.4 MB, resident in the last-level cache)"}


class C1Cold(C1DecodeChain):
    """c1 with every step on input buffers not touched since the caches were
    flushed: at least K sets rotate, and 1 GiB is written between timed
    replays (the last-level cache is 256 MB), so each step reads its
    activations from HBM. The gains and the RoPE table are shared by the
    steps (as one layer's are across decode tokens)."""
    name = "c1_cold"
    description = C1DecodeChain.description + " -- cold: inputs read from HBM"
    hot = False

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        self.flush_buf = torch.empty(1 << 28, device=dev)  # 1 GiB

    def n_sets(self) -> int:
        return max(64, self.steps_hint, self.min_steps)

    def between(self) -> None:
        self.flush_buf.fill_(1.0)

    def config(self):
        return {**super().config(), "cache": f"cold ({self.S} sets, 1 GiB written between timed replays)"}


class C2PrefillChain(Workload):
    name = "c2"
    description = ("qwen3-asr-0.6b prefill chain T=512: fp32 embed gather from [151936,1024] + "
                   "add+RMSNorm[512,1024] + q/k head-RMSNorm+RoPE(pos 0..511) + SwiGLU[512,3072]")
    unit_tokens = 512

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = DEC_0_6B
        T = 512
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        smallest = 5 * T * H * F  # add+RMSNorm bytes: the smallest kernel footprint
        self.S = sets_for(smallest)
        self.rotation = self.S
        self.table = self.randn(VOCAB * H, 0.02)
        S = self.S
        self.ids = [torch.randint(0, VOCAB, (T,), generator=self.gen, device=dev, dtype=torch.int32)
                    for _ in range(S)]
        self.x = [torch.empty(T * H, device=dev) for _ in range(S)]
        self.d = [self.randn(T * H) for _ in range(S)]
        self.y = [torch.empty(T * H, device=dev) for _ in range(S)]
        self.q = [self.randn(T * nq * hd) for _ in range(S)]
        self.k = [self.randn(T * nk * hd) for _ in range(S)]
        self.gu = [self.randn(T * 2 * I) for _ in range(S)]
        self.o = [torch.empty(T * I, device=dev) for _ in range(S)]
        self.w = self.randn(H, 0.1, 1.0)
        self.qw, self.kw = self.randn(hd, 0.1, 1.0), self.randn(hd, 0.1, 1.0)
        self.rope = K.RopeCache(dev)
        self.rope.ensure(T, hd, c["theta"])
        self.pos = torch.arange(T, device=dev, dtype=torch.int32)
        self.kernels = {
            "embed_gather": (lambda i: K.embed_gather_f32(self.x[i % S], self.table, self.ids[i % S], T, H),
                             T * 4 + 2 * T * H * F),
            "add_rms_norm": (lambda i: K.add_rms_norm(self.x[i % S], self.d[i % S], self.w, self.y[i % S], T, H, c["eps"]),
                             4 * T * H * F + H * F),
            "head_rms_norm_rope": (lambda i: K.head_rms_norm_rope(
                self.q[i % S], self.k[i % S], self.qw, self.kw, self.rope.cos, self.rope.sin, self.pos,
                T, nq, nk, hd, c["eps"]),
                2 * T * (nq + nk) * hd * F + 2 * hd * F + 2 * T * hd * F + T * 4),
            "swiglu_multiply": (lambda i: K.swiglu_multiply(self.o[i % S], self.gu[i % S], T, I),
                                3 * T * I * F),
        }
        self.step_bytes = sum(b for _, b in self.kernels.values())
        self.tokens_per_step = 512.0

    def config(self):
        return {"seq_len": 512, "hidden": 1024, "heads": "16q/8kv x 128", "intermediate": 3072,
                "vocab": VOCAB, "buffer_sets": self.S}


class C3EncoderOps(Workload):
    name = "c3"
    description = ("qwen3-asr-0.6b audio-encoder ops: sinusoidal PE add (13-row per-chunk table) + "
                   "LayerNorm(eps 1e-5) on [3000,896], exact erf-GELU on [3000,3584]")
    unit_tokens = 3000

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = ENC_0_6B
        T, D, FF, P = 3000, c["d_model"], c["ffn"], c["pe_rows"]
        self.S = sets_for(2 * T * D * F)
        self.rotation = self.S
        S = self.S
        self.x = [self.randn(T * D) for _ in range(S)]
        self.y = [torch.empty(T * D, device=dev) for _ in range(S)]
        self.h = [self.randn(T * FF) for _ in range(S)]
        self.w, self.b = self.randn(D, 0.1, 1.0), self.randn(D, 0.02)
        self.pe = torch.empty(P * D, device=dev)
        K.sinusoidal_pe(self.pe, P, D)
        self.kernels = {
            "pe_add": (lambda i: K.pe_add(self.x[i % S], self.pe, T, D, P), 2 * T * D * F + P * D * F),
            "layer_norm": (lambda i: K.layer_norm(self.y[i % S], self.x[i % S], self.w, self.b, T, D, c["eps"]),
                           2 * T * D * F + 2 * D * F),
            "gelu_erf": (lambda i: K.gelu_erf(self.h[i % S], T * FF), 2 * T * FF * F),
        }
        self.step_bytes = sum(b for _, b in self.kernels.values())
        self.tokens_per_step = 3000.0

    def config(self):
        return {"rows": 3000, "d_model": 896, "ffn": 3584, "pe_period": 13, "buffer_sets": self.S}


class C3Fused(C3EncoderOps):
    """c3 with the PE add and the LayerNorm that reads its rows (layer 0's
    attention norm, encoder.rs:341-343 then 370-371) in one pass."""
    name = "c3_fused"
    description = ("qwen3-asr-0.6b audio-encoder ops with the PE add fused into layer 0's LayerNorm: "
                   "x[3000,896] += pe (13-row table), LayerNorm(eps 1e-5) of it, one pass; exact erf-GELU "
                   "on [3000,3584]")

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = ENC_0_6B
        T, D, FF, P, S = 3000, c["d_model"], c["ffn"], c["pe_rows"], self.S
        gelu = self.kernels["gelu_erf"]
        self.kernels = {
            "pe_add_layer_norm": (lambda i: K.pe_add_layer_norm(
                self.x[i % S], self.pe, self.y[i % S], self.w, self.b, T, D, P, c["eps"]),
                3 * T * D * F + P * D * F + 2 * D * F),
            "gelu_erf": gelu,
        }
        self.step_bytes = sum(b for _, b in self.kernels.values())


class EncAddLayerNorm(C3EncoderOps):
    """An encoder residual add and the LayerNorm that reads its rows next
    (encoder.rs:386 + 389-390) at the c3 shape, one pass."""
    name = "enc_add_ln"
    description = ("qwen3-asr-0.6b encoder residual add + LayerNorm(eps 1e-5) in one pass on [3000,896] "
                   "(x += delta; out = LayerNorm(x))")

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = ENC_0_6B
        T, D, S = 3000, c["d_model"], self.S
        self.d = [self.randn(T * D) for _ in range(S)]
        self.kernels = {
            "add_layer_norm": (lambda i: K.add_layer_norm(
                self.x[i % S], self.d[i % S], self.w, self.b, self.y[i % S], T, D, c["eps"]),
                4 * T * D * F + 2 * D * F),
        }
        self.step_bytes = sum(b for _, b in self.kernels.values())


class C4Int8Matvec(Workload):
    name = "c4"
    description = ("qwen3-asr-1.7b INT8 W8A8 gate/up matvec [12288,2048] + SwiGLU, B=1, 28 distinct "
                   "layers per step (fp32 x quantized per-vector in-kernel)")
    unit_tokens = 1

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = DEC_1_7B
        H, I, L = c["hidden"], c["inter"], 28
        self.layers = []
        for _ in range(L):
            w = self.randn(2 * I * H, 0.02)
            q, s = K.quantize_f32_to_int8(w, 2 * I, H)
            del w
            self.layers.append(K.QuantWeight(q, s, 2 * I, H))
        self.xs = [self.randn(H) for _ in range(L)]
        self.outs = [torch.empty(I, device=dev) for _ in range(L)]
        self.L = L
        self.rotation = L
        self.H, self.I = H, I
        layer_bytes = 2 * I * H + 2 * I * F + H * F + I * F

        def all_layers(i):
            for l in range(L):
                K.gate_up_swiglu_w8a8_f32in(self.outs[l], self.layers[l], self.xs[l], H, I)

        self.kernels = {"gate_up_swiglu_w8a8_matvec": (lambda i: K.gate_up_swiglu_w8a8_f32in(
            self.outs[i % L], self.layers[i % L], self.xs[i % L], H, I), layer_bytes)}
        self.all_layers = all_layers
        self.layer_bytes = layer_bytes
        self.step_bytes = L * layer_bytes
        self.tokens_per_step = 1.0  # a step is 28 layers: one token
        self.dtype = "int8/int32->f32"

    def step(self, i):
        self.all_layers(i)

    def config(self):
        return {"batch": 1, "in_dim": 2048, "gate_up_rows": 12288, "layers": 28}


class C5BatchedDecode(Workload):
    name = "c5"
    B = 256
    description = ("qwen3-asr-1.7b batched decode B=256 (positions U[0,2047]): add+RMSNorm[256,2048] "
                   "fused with per-row int8 quantization + q/k head-RMSNorm+RoPE + W8A8 MFMA gate/up "
                   "GEMM [256,2048]x[2048,12288] + SwiGLU; 28 distinct layers rotate")
    unit_tokens = 256

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = DEC_1_7B
        B, L = self.B, 28
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        self.layers = []
        for _ in range(L):
            w = self.randn(2 * I * H, 0.02)
            q, s = K.quantize_f32_to_int8(w, 2 * I, H)
            del w
            # weights are re-laid into MFMA tiles once, at load
            self.layers.append(K.pack_w8a8_tiles(K.QuantWeight(q, s, 2 * I, H)))
            del q
        S = L
        self.rotation = S
        self.x = [self.randn(B * H) for _ in range(S)]
        self.d = [self.randn(B * H) for _ in range(S)]
        self.q = [self.randn(B * nq * hd) for _ in range(S)]
        self.k = [self.randn(B * nk * hd) for _ in range(S)]
        self.xq = [torch.empty(B * H, dtype=torch.int8, device=dev) for _ in range(S)]
        self.xsc = [torch.empty(B, device=dev) for _ in range(S)]
        self.o = [torch.empty(B * I, device=dev) for _ in range(S)]
        self.w = self.randn(H, 0.1, 1.0)
        self.qw, self.kw = self.randn(hd, 0.1, 1.0), self.randn(hd, 0.1, 1.0)
        self.rope = K.RopeCache(dev)
        self.rope.ensure(2048, hd, c["theta"])
        self.pos = [torch.randint(0, 2048, (B,), generator=self.gen, device=dev, dtype=torch.int32)
                    for _ in range(S)]
        self.kernels = {
            "add_rms_norm_quant": (lambda i: K.add_rms_norm_quant(
                self.x[i % S], self.d[i % S], self.w, None, self.xq[i % S], self.xsc[i % S], B, H, c["eps"]),
                3 * B * H * F + H * F + B * H + B * F),
            "head_rms_norm_rope": (lambda i: K.head_rms_norm_rope(
                self.q[i % S], self.k[i % S], self.qw, self.kw, self.rope.cos, self.rope.sin,
                self.pos[i % S], B, nq, nk, hd, c["eps"]),
                2 * B * (nq + nk) * hd * F + 2 * hd * F + 2 * B * hd * F + B * 4),
            "gate_up_swiglu_w8a8_gemm": (lambda i: K.gate_up_swiglu_w8a8_packed(
                self.o[i % S], self.layers[i % L], self.xq[i % S], self.xsc[i % S], B, H, I),
                2 * I * H + 2 * I * F + B * H + B * F + B * I * F),
        }
        self.step_bytes = sum(b for _, b in self.kernels.values())
        self.tokens_per_step = B / 28.0  # one layer for B streams
        self.dtype = "int8/int32->f32"
        self.gemm_ops = 2 * B * 2 * I * H

    def config(self):
        return {"batch": self.B, "hidden": 2048, "heads": "16q/8kv x 128", "intermediate": 6144,
                "layers_rotated": 28}


class C5Share(C5BatchedDecode):
    """c5 at one GPU's data-parallel share of a 256-stream batch over 8 GPUs."""
    name = "c5_b32"
    B = 32
    description = ("qwen3-asr-1.7b batched decode B=32 (one GPU's share of 256 streams over 8): "
                   "add+RMSNorm[32,2048]+int8 quant, q/k head-RMSNorm+RoPE, W8A8 gate/up + SwiGLU "
                   "[32,2048]x[2048,12288]; 28 distinct layers rotate")
    unit_tokens = 32


class C5Layer(Workload):
    """The batched decode layer's projections at B=256 with their fused
    neighbours (decoder.rs:878-895, 908-921 per stream, W8A8): residual add +
    input RMSNorm + int8 quantization; the q/k/v projection with the q/k head
    norms, RoPE at each stream's position and the K/V cache rows in its
    epilogue; residual add + post-attention RMSNorm + quantization; gate/up +
    SwiGLU. Attention, o and down are not in this chain."""
    name = "c5_layer"
    B = 256
    description = ("qwen3-asr-1.7b batched decode layer projections, B=256 streams at positions U[0,2047]: "
                   "add+RMSNorm+int8 quant [256,2048]; W8A8 q/k/v [256,2048]x[2048,4096] with q/k head "
                   "RMSNorm + RoPE + K/V cache store in the epilogue; add+RMSNorm+quant; W8A8 gate/up "
                   "[256,2048]x[2048,12288] + SwiGLU; 28 distinct layers of weights rotate")
    unit_tokens = 256

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        c = DEC_1_7B
        B, L = self.B, 28
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        N = (nq + 2 * nk) * hd
        self.qkv, self.gu = [], []
        for _ in range(L):
            for rows, dst in ((N, self.qkv), (2 * I, self.gu)):
                w = self.randn(rows * H, 0.02)
                q, s = K.quantize_f32_to_int8(w, rows, H)
                del w
                dst.append(K.pack_w8a8_tiles(K.QuantWeight(q, s, rows, H)))
                del q
        S = L
        self.rotation = S
        self.x = [self.randn(B * H) for _ in range(S)]
        self.d = [self.randn(B * H) for _ in range(S)]
        self.d2 = [self.randn(B * H) for _ in range(S)]
        self.xq = [torch.empty(B * H, dtype=torch.int8, device=dev) for _ in range(S)]
        self.xsc = [torch.empty(B, device=dev) for _ in range(S)]
        self.xq2 = [torch.empty(B * H, dtype=torch.int8, device=dev) for _ in range(S)]
        self.xsc2 = [torch.empty(B, device=dev) for _ in range(S)]
        self.q = [torch.empty(B * nq * hd, device=dev) for _ in range(S)]
        self.o = [torch.empty(B * I, device=dev) for _ in range(S)]
        self.rows = 2048
        kv = nk * hd
        # one layer's per-stream cache blocks [B, 2048, kv] (4 GiB for K and V)
        self.kc = torch.zeros(B * self.rows * kv, device=dev)
        self.vc = torch.zeros(B * self.rows * kv, device=dev)
        self.w1, self.w2 = self.randn(H, 0.1, 1.0), self.randn(H, 0.1, 1.0)
        self.qw, self.kw = self.randn(hd, 0.1, 1.0), self.randn(hd, 0.1, 1.0)
        self.rope = K.RopeCache(dev)
        self.rope.ensure(self.rows, hd, c["theta"])
        self.pos = [torch.randint(0, self.rows, (B,), generator=self.gen, device=dev, dtype=torch.int32)
                    for _ in range(S)]
        eps = c["eps"]
        norm_bytes = 3 * B * H * F + H * F + B * H + B * F
        qkv_bytes = (N * H + N * F + B * H + B * F + B * nq * hd * F + 2 * B * kv * F + 2 * hd * F
                     + 2 * B * hd * F + B * 4)
        gu_bytes = 2 * I * H + 2 * I * F + B * H + B * F + B * I * F
        self.kernels = {
            "add_rms_norm_quant": (lambda i: K.add_rms_norm_quant(
                self.x[i % S], self.d[i % S], self.w1, None, self.xq[i % S], self.xsc[i % S], B, H, eps),
                norm_bytes),
            "qkv_heads_w8a8_gemm": (lambda i: K.qkv_heads_w8a8_packed(
                self.q[i % S], self.kc, self.vc, self.rows, self.qkv[i % L], self.xq[i % S], self.xsc[i % S],
                self.qw, self.kw, self.rope, self.pos[i % S], B, H, nq, nk, hd, eps),
                qkv_bytes, 2 * B * N * H),
            "add_rms_norm_quant_post": (lambda i: K.add_rms_norm_quant(
                self.x[i % S], self.d2[i % S], self.w2, None, self.xq2[i % S], self.xsc2[i % S], B, H, eps),
                norm_bytes),
            "gate_up_swiglu_w8a8_gemm": (lambda i: K.gate_up_swiglu_w8a8_packed(
                self.o[i % S], self.gu[i % L], self.xq2[i % S], self.xsc2[i % S], B, H, I),
                gu_bytes, 2 * B * 2 * I * H),
        }
        self.step_bytes = sum(spec[1] for spec in self.kernels.values())
        self.tokens_per_step = B / 28.0
        self.dtype = "int8/int32->f32"
        self.gemm_ops = 2 * B * 2 * I * H
        # the int8 MFMA ceiling; both GEMMs sit below its ridge (HBM-bound)
        self.mfma_peak_tflops = 5000.0
        self.mfma_peak_basis = "int8 MFMA 5.0 POP/s dense"

    def config(self):
        return {"batch": self.B, "hidden": 2048, "heads": "16q/8kv x 128", "intermediate": 6144,
                "cache_rows_per_stream": self.rows, "layers_rotated": 28}


class W8A32Decode(Workload):
    name = "w8a32_decode"
    description = ("qwen3-asr-1.7b INT8 decode projections as the reference runs them (W8A32 "
                   "linear_nobias_int8, B=1): q/k/v in one launch, o, fused gate/up and down per layer, "
                   "28 distinct layers")
    unit_tokens = 1
    dtype = "int8/f32"

    SHAPES = {"wq": (2048, 2048), "wk": (1024, 2048), "wv": (1024, 2048), "wo": (2048, 2048),
              "gate_up": (12288, 2048), "down": (2048, 6144)}

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        L = 28
        self.L = L
        self.rotation = L
        self.w = {n: [] for n in self.SHAPES}
        for n, (o, i) in self.SHAPES.items():
            for _ in range(L):
                # int8 weights and per-row scales with the quantizer's value range
                q = torch.randint(-127, 128, (o * i,), generator=self.gen, device=dev, dtype=torch.int8)
                self.w[n].append((q, self.randn(o, 1e-4, 1e-3).abs_()))
        self.x = {n: [self.randn(i) for _ in range(L)] for n, (o, i) in self.SHAPES.items()}
        self.y = {n: [torch.empty(o, device=dev) for _ in range(L)] for n, (o, i) in self.SHAPES.items()}

        def mk(n):
            o, i = self.SHAPES[n]
            return (lambda j: K.linear_nobias_int8(self.y[n][j % L], self.x[n][j % L], self.w[n][j % L][0],
                                                   self.w[n][j % L][1], 1, i, o),
                    o * i + o * F + i * F + o * F)

        def qkv(j):
            names = ("wq", "wk", "wv")
            ws = [K.QuantWeight(self.w[n][j % L][0], self.w[n][j % L][1], self.SHAPES[n][0], 2048)
                  for n in names]
            K.linear_nobias_int8_multi([self.y[n][j % L] for n in names], ws, self.x["wq"][j % L], 1, 2048)

        qkv_rows = sum(self.SHAPES[n][0] for n in ("wq", "wk", "wv"))
        # q/k/v read one x: weights, scales and outputs of the three, x once
        self.kernels = {"qkv": (qkv, qkv_rows * 2048 + 2 * qkv_rows * F + 2048 * F)}
        self.kernels.update({n: mk(n) for n in ("wo", "gate_up", "down")})
        self.step_bytes = L * sum(spec[1] for spec in self.kernels.values())
        self.tokens_per_step = 1.0

    def step(self, i):
        for l in range(self.L):
            for spec in self.kernels.values():
                spec[0](l)

    def config(self):
        return {"batch": 1, "hidden": 2048, "intermediate": 6144, "layers": 28,
                "projections": {n: f"[{o},{i}]" for n, (o, i) in self.SHAPES.items()}}


class W8A32Prefill(Workload):
    name = "w8a32_prefill"
    description = ("qwen3-asr-0.6b INT8 prefill projections, T=512 (W8A32 linear_nobias_int8 with "
                   "seq_len 512, as the reference runs them): q/k/v in one call, o, fused gate/up, down; "
                   "28 distinct layers rotate")
    unit_tokens = 512
    dtype = "int8/f32"
    T = 512
    # each fp32 multiply-add is three exact bf16 products on the bf16 matrix
    # cores (x split into hi/mid/lo bf16 terms, int8 weights exact in bf16)
    mfma_peak_tflops = BF16_PEAK_TFLOPS / 3
    mfma_peak_basis = "bf16 MFMA 2500 TFLOP/s dense / 3 bf16 products per fp32 multiply-add"
    SHAPES = {"wq": (2048, 1024), "wk": (1024, 1024), "wv": (1024, 1024), "wo": (1024, 2048),
              "gate_up": (6144, 1024), "down": (1024, 3072)}

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        L, T = 28, self.T
        self.L = L
        self.rotation = L
        self.w = {n: [K.QuantWeight(torch.randint(-127, 128, (o * i,), generator=self.gen, device=dev,
                                                  dtype=torch.int8), self.randn(o, 1e-4, 1e-3).abs_(), o, i)
                      for _ in range(L)] for n, (o, i) in self.SHAPES.items()}
        self.x = {i: [self.randn(T * i) for _ in range(2)] for i in (1024, 2048, 3072)}
        self.y = {n: torch.empty(T * o, device=dev) for n, (o, i) in self.SHAPES.items()}

        def mk(n):
            o, i = self.SHAPES[n]
            return (lambda j: K.linear_nobias_int8(self.y[n], self.x[i][j % 2], self.w[n][j % L].data,
                                                   self.w[n][j % L].scales, T, i, o),
                    o * i + o * F + T * i * F + T * o * F, 2 * T * o * i)

        def qkv(j):
            K.linear_nobias_int8_multi([self.y[n] for n in ("wq", "wk", "wv")],
                                       [self.w[n][j % L] for n in ("wq", "wk", "wv")], self.x[1024][j % 2], T, 1024)

        rows = 2048 + 1024 + 1024
        self.kernels = {"qkv": (qkv, rows * 1024 + rows * F + T * 1024 * F + T * rows * F, 2 * T * rows * 1024)}
        self.kernels.update({n: mk(n) for n in ("wo", "gate_up", "down")})
        self.step_bytes = sum(spec[1] for spec in self.kernels.values())
        self.tokens_per_step = T / 28.0  # one layer of a 512-token prefill

    def config(self):
        return {"seq_len": self.T, "hidden": 1024, "intermediate": 3072, "layers_rotated": 28,
                "projections": {n: f"[{o},{i}]" for n, (o, i) in self.SHAPES.items()}}


class DecodeStep(Workload):
    name = "decode_step"
    description = ("qwen3-asr-1.7b INT8 decode of one token at position 1023, B=1, fully on the device: "
                   "28 layers of residual add+input RMSNorm+q/k/v (one launch), q/k norm+RoPE+KV store+"
                   "split attention over 1024 cached rows (one launch) + merge, o, add+RMSNorm+gate/up+"
                   "SwiGLU (one launch), down; final norm and INT8 lm_head [151936,2048] greedy argmax")
    unit_tokens = 1
    dtype = "int8/f32"
    POS = 1023

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K
        from qwenasr_amd.decoder import DecoderInt8

        c = DEC_1_7B
        H, I, nq, nk, hd, L = c["hidden"], c["inter"], c["n_heads"], c["n_kv_heads"], c["head_dim"], 28

        def qw(o, i):  # int8 weights and per-row scales with the quantizer's value range
            q = torch.randint(-127, 128, (o * i,), generator=self.gen, device=dev, dtype=torch.int8)
            return K.QuantWeight(q, self.randn(o, 1e-4, 1e-3).abs_(), o, i)

        def gain(n):
            return self.randn(n, 0.1, 1.0)

        layers = [{"wq": qw(nq * hd, H), "wk": qw(nk * hd, H), "wv": qw(nk * hd, H), "wo": qw(H, nq * hd),
                   "gate_up": qw(2 * I, H), "down": qw(H, I), "q_norm": gain(hd), "k_norm": gain(hd),
                   "input_norm": gain(H), "post_attn_norm": gain(H)} for _ in range(L)]
        weights = {"layers": layers, "norm": gain(H), "lm_head": qw(VOCAB, H)}
        self.dec = DecoderInt8(weights, H, I, L, nq, nk, hd, c["eps"], c["theta"], max_seq=2048, device=dev)
        self.dec.kv.k.normal_(generator=self.gen)  # rows 0..1022: an earlier context
        self.dec.kv.v.normal_(generator=self.gen)
        self.dec.kv.len = self.POS
        self.dec.prepare(self.POS)
        self.embed = [self.randn(H) for _ in range(4)]
        kv = nk * hd
        layer_bytes = (sum(w.out_dim * w.in_dim + w.out_dim * F for k, w in layers[0].items()
                           if isinstance(w, K.QuantWeight))
                       + (2 * hd + 2 * H) * F                      # norm gains
                       + 2 * (self.POS + 1) * kv * F              # k/v rows read by attention
                       + 2 * kv * F)                              # the new k/v rows
        head_bytes = VOCAB * H + 2 * VOCAB * F + H * F + 4       # lm_head weights, scales, logits, token
        step_bytes = L * layer_bytes + head_bytes
        self.kernels = {"decode_token": (lambda i: self.dec.decode(self.embed[i % 4], self.POS), step_bytes)}
        self.step_bytes = step_bytes
        self.tokens_per_step = 1.0

    def config(self):
        return {"batch": 1, "position": self.POS, "hidden": 2048, "intermediate": 6144,
                "heads": "16q/8kv x 128", "layers": 28, "vocab": VOCAB}


class DecodeStepBatched(Workload):
    """B=256 decode streams, each at its own position U[0,2047] over its own
    KV cache, one token each through all 28 layers and the lm_head."""
    name = "decode_step_b256"
    B = 256
    description = ("qwen3-asr-1.7b INT8 batched decode: 256 streams, each at its own position U[0,2047] over "
                   "its own KV cache (28 layers x 2048 rows), one token each through all 28 layers (W8A32 "
                   "matrix-core projections, per-stream head norm+RoPE+KV store, per-stream attention, "
                   "gate/up with the decode SwiGLU) and the lm_head [151936,2048] with each stream's argmax")
    unit_tokens = 256
    dtype = "int8/f32"
    max_steps = 10  # ~15 ms per step: 10 steps per replay keep the run short

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K
        from qwenasr_amd.decoder import DecoderInt8Batched

        c = DEC_1_7B
        H, I, nq, nk, hd, L, B = c["hidden"], c["inter"], c["n_heads"], c["n_kv_heads"], c["head_dim"], 28, self.B
        rows = 2048

        def qw(o, i):
            q = torch.randint(-127, 128, (o * i,), generator=self.gen, device=dev, dtype=torch.int8)
            return K.QuantWeight(q, self.randn(o, 1e-4, 1e-3).abs_(), o, i)

        def gain(n):
            return self.randn(n, 0.1, 1.0)

        layers = [{"wq": qw(nq * hd, H), "wk": qw(nk * hd, H), "wv": qw(nk * hd, H), "wo": qw(H, nq * hd),
                   "gate_up": qw(2 * I, H), "down": qw(H, I), "q_norm": gain(hd), "k_norm": gain(hd),
                   "input_norm": gain(H), "post_attn_norm": gain(H)} for _ in range(L)]
        weights = {"layers": layers, "norm": gain(H), "lm_head": qw(VOCAB, H)}
        self.dec = DecoderInt8Batched(weights, H, I, L, B, rows, nq, nk, hd, c["eps"], c["theta"], device=dev,
                                      w8a8=getattr(self, "w8a8", False))
        # each stream's earlier context: its cache rows (all 28 layers, 120 GB in all)
        for l in range(L):
            self.dec.k[l].normal_(generator=self.gen)
            self.dec.v[l].normal_(generator=self.gen)
        pos = torch.randint(0, rows, (B,), generator=self.gen, device=dev, dtype=torch.int32)
        self.dec.positions.copy_(pos)
        self.embeds = [self.randn(B * H) for _ in range(2)]
        kv, q_dim = nk * hd, nq * hd
        keys = int(pos.to(torch.int64).sum().item()) + B  # keys 0..pos of every stream
        w_bytes = sum(w.out_dim * w.in_dim + w.out_dim * F for k, w in layers[0].items()
                      if isinstance(w, K.QuantWeight)) + (2 * hd + 2 * H) * F  # + norm gains
        act = F * B * (4 * H + H + (q_dim + 2 * kv) + 2 * (q_dim + 2 * kv) + q_dim + q_dim + q_dim + H
                       + 4 * H + H + I + I + H)
        layer_bytes = w_bytes + act + 2 * keys * kv * F + 2 * B * kv * F
        head_bytes = VOCAB * H + VOCAB * F + 4 * B * H * F + B * H * F + 2 * B * VOCAB * F + B * 4
        step_bytes = L * layer_bytes + head_bytes
        self.kernels = {"decode_step": (lambda i: self.dec.decode(self.embeds[i % 2]), step_bytes)}
        self.step_bytes = step_bytes
        self.tokens_per_step = float(B)
        self.mean_position = keys / B - 1

    def config(self):
        return {"batch": self.B, "positions": "U[0,2047] per stream", "mean_position": round(self.mean_position, 1),
                "cache_rows_per_stream": 2048, "hidden": 2048, "intermediate": 6144, "heads": "16q/8kv x 128",
                "layers": 28, "vocab": VOCAB}


class DecodeStepBatchedW8A8(DecodeStepBatched):
    """decode_step_b256 with the projections on int8 matrix cores (each
    stream's activation rows quantized per row at the four projection inputs,
    as the c5 gate/up does) and the lm_head W8A8 as well: a fifth rounding
    point before the greedy argmax, which the reference (W8A32 lm_head,
    decoder.rs:929-963) does not have."""
    name = "decode_step_b256_w8a8"
    description = (DecodeStepBatched.description.replace("W8A32 matrix-core projections",
                                                         "W8A8 int8-MFMA projections")
                   + "; the lm_head is W8A8 too (final norm rows quantized per row), so its greedy "
                     "tokens are not the reference's W8A32 ones")
    dtype = "int8/int32->f32"
    w8a8 = True


class PrefillStep(Workload):
    name = "prefill_step"
    description = ("qwen3-asr-0.6b INT8 prefill of a 512-token chunk at position 0, fully on the device "
                   "(decoder.rs:751-847): 28 layers of q/k/v (one bf16x3 matrix-core GEMM with the input "
                   "RMSNorm folded in) with q/k norm+RoPE+KV store of 512 rows in its epilogue, causal "
                   "attention (fp32 matrix cores), o with the residual add in its epilogue, gate/up with the "
                   "post-attention RMSNorm folded in + prefill SwiGLU, down with the residual add; layer 0's "
                   "input RMSNorm as its own launch")
    unit_tokens = 512
    dtype = "int8/f32"
    T = 512
    max_steps = 20  # ~3.9 ms per step

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K
        from qwenasr_amd.decoder import DecoderInt8

        c = DEC_0_6B
        H, I, nq, nk, hd, L, T = c["hidden"], c["inter"], c["n_heads"], c["n_kv_heads"], c["head_dim"], 28, self.T

        def qw(o, i):
            q = torch.randint(-127, 128, (o * i,), generator=self.gen, device=dev, dtype=torch.int8)
            return K.QuantWeight(q, self.randn(o, 1e-4, 1e-3).abs_(), o, i)

        def gain(n):
            return self.randn(n, 0.1, 1.0)

        layers = [{"wq": qw(nq * hd, H), "wk": qw(nk * hd, H), "wv": qw(nk * hd, H), "wo": qw(H, nq * hd),
                   "gate_up": qw(2 * I, H), "down": qw(H, I), "q_norm": gain(hd), "k_norm": gain(hd),
                   "input_norm": gain(H), "post_attn_norm": gain(H)} for _ in range(L)]
        weights = {"layers": layers, "norm": gain(H), "lm_head": qw(1000, H)}
        self.dec = DecoderInt8(weights, H, I, L, nq, nk, hd, c["eps"], c["theta"], max_seq=T, device=dev)
        self.dec.prepare_prefill(0, T)
        self.embeds = [self.randn(T * H) for _ in range(2)]
        kv, q_dim = nk * hd, nq * hd
        proj = sum(w.out_dim * w.in_dim for k, w in layers[0].items() if isinstance(w, K.QuantWeight))
        # algorithmic bytes of the 9 kernels of a layer: each one's inputs read and
        # outputs written once (the reference's op sequence moves every activation
        # between its ops through memory)
        row = T * F
        qkv_out = q_dim + 2 * kv
        layer_bytes = (
            4 * row * H + H * F                                          # add + RMSNorm: x, delta in; x, norm out
            + qkv_out * H + qkv_out * F + row * H + row * qkv_out        # q/k/v GEMM
            + 2 * row * q_dim + 4 * row * kv + 2 * hd * F + 2 * T * hd * F  # head norm+RoPE+KV store (+ gains, tables)
            + 2 * row * q_dim + 2 * row * kv                             # attention: q, k, v rows in, out
            + H * q_dim + H * F + row * q_dim + row * H                  # o GEMM
            + 4 * row * H + H * F                                        # add + post-attention RMSNorm
            + 2 * I * H + 2 * I * F + row * H + row * 2 * I              # gate/up GEMM
            + row * 2 * I + row * I                                      # SwiGLU
            + H * I + H * F + row * I + row * H)                         # down GEMM
        step_bytes = L * layer_bytes + 3 * row * H                       # + the last residual add
        gemm_flops = 2 * T * proj
        attn_flops = 2 * 2 * hd * nq * (T * (T + 1) // 2)         # QK and PV over the causal triangle
        self.step_flops = L * (gemm_flops + attn_flops)
        # ceiling: GEMM flops at the bf16x3 rate (three bf16 products per fp32
        # multiply-add), attention flops at the fp32 matrix-core rate
        floor_s = L * (gemm_flops / (BF16_PEAK_TFLOPS / 3 * 1e12) + attn_flops / (FP32_PEAK_TFLOPS * 1e12))
        self.mfma_peak_tflops = self.step_flops / floor_s / 1e12
        self.mfma_peak_basis = ("projections at bf16 MFMA 2500/3 TFLOP/s (bf16x3), attention at fp32 MFMA "
                                "157.3 TFLOP/s, weighted by their flops")
        def prefill_at_0(i):
            self.dec.kv.len = 0  # every step prefills a chunk at position 0
            self.dec.prefill(self.embeds[i % 2], T, 0)

        self.kernels = {"prefill": (prefill_at_0, step_bytes, self.step_flops)}
        self.step_bytes = step_bytes
        self.tokens_per_step = float(T)

    def config(self):
        return {"seq_len": self.T, "start_pos": 0, "hidden": 1024, "intermediate": 3072,
                "heads": "16q/8kv x 128", "layers": 28}


class AttnDecode(Workload):
    name = "attn_decode"
    description = ("qwen3-asr-1.7b decode attention at position 2047: q[16,128] against a 2048-row "
                   "KV block [2048, 8x128] per layer, keys split over workgroups; 28 distinct layers per step")
    unit_tokens = 1
    dtype = "f32"

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        nq, nk, hd, L, seq_k = 16, 8, 128, 28, 2048
        self.k = [self.randn(seq_k * nk * hd) for _ in range(L)]
        self.v = [self.randn(seq_k * nk * hd) for _ in range(L)]
        self.q = [self.randn(nq * hd) for _ in range(L)]
        self.o = [torch.empty(nq * hd, device=dev) for _ in range(L)]
        self.ws = K.attention_workspace(1, nq, hd, dev)
        scale = hd ** -0.5

        def one(i):
            l = i % L
            K.causal_attention_split(self.o[l], self.q[l], self.k[l], self.v[l], 1, seq_k, nq, nk, hd,
                                     scale, seq_k - 1, self.ws)

        self.one, self.L = one, L
        layer_bytes = 2 * seq_k * nk * hd * F + 2 * nq * hd * F
        self.kernels = {"causal_attention_split": (one, layer_bytes)}
        self.step_bytes = L * layer_bytes
        self.tokens_per_step = 1.0

    def step(self, i):
        for l in range(self.L):
            self.one(l)

    def config(self):
        return {"batch": 1, "position": 2047, "heads": "16q/8kv x 128", "layers": 28}


class AttnPrefill(Workload):
    name = "attn_prefill"
    description = ("qwen3-asr-0.6b causal prefill attention T=512: q[512,16x128] over k/v[512,8x128], "
                   "fp32 (VALU)")
    unit_tokens = 512
    dtype = "f32"

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        T, nq, nk, hd = 512, 16, 8, 128
        per_set = (2 * T * nq * hd + 2 * T * nk * hd) * F
        self.S = sets_for(per_set)
        self.rotation = self.S
        S = self.S
        self.q = [self.randn(T * nq * hd) for _ in range(S)]
        self.k = [self.randn(T * nk * hd) for _ in range(S)]
        self.v = [self.randn(T * nk * hd) for _ in range(S)]
        self.o = [torch.empty(T * nq * hd, device=dev) for _ in range(S)]
        scale = hd ** -0.5
        flops = 2 * 2 * nq * hd * (T * (T + 1) // 2)
        self.kernels = {"causal_attention": (
            lambda i: K.causal_attention(self.o[i % S], self.q[i % S], self.k[i % S], self.v[i % S],
                                         T, T, nq, nk, hd, scale, 0), per_set, flops)}
        self.step_bytes = per_set
        self.tokens_per_step = float(T)

    def config(self):
        return {"seq_len": 512, "heads": "16q/8kv x 128", "buffer_sets": self.S}


class LmHead(Workload):
    name = "lm_head"
    description = ("qwen3-asr-0.6b INT8 lm_head [151936,1024] logits + greedy argmax, B=1 "
                   "(W8A32 as the reference), 4 weight copies rotate")
    unit_tokens = 1
    dtype = "int8/f32"

    def __init__(self, dev, torch):
        super().__init__(dev, torch)
        from qwenasr_amd import kernels as K

        V, H, C = VOCAB, 1024, 4
        self.w = []
        for _ in range(C):
            w = self.randn(V * H, 0.02)
            q, sc = K.quantize_f32_to_int8(w, V, H)
            del w
            self.w.append(K.QuantWeight(q, sc, V, H))
        self.x = [self.randn(H) for _ in range(C)]
        self.logits = [torch.empty(V, device=dev) for _ in range(C)]
        self.idx = [torch.empty(1, dtype=torch.int32, device=dev) for _ in range(C)]
        # weights, scales, x, the logits written once, the token index
        nbytes = V * H + V * F + H * F + V * F + 4
        self.ws = K.lm_head_workspace(V, dev)
        self.kernels = {"lm_head_int8_argmax": (
            lambda i: K.lm_head_int8_argmax(self.idx[i % C], self.logits[i % C], self.x[i % C],
                                            self.w[i % C], 1, H, V, self.ws), nbytes)}
        self.step_bytes = nbytes
        self.tokens_per_step = 1.0

    def config(self):
        return {"batch": 1, "hidden": 1024, "vocab": VOCAB, "weight_copies": 4}


WORKLOADS = {"c1": C1DecodeChain, "c1_cold": C1Cold, "c2": C2PrefillChain, "c3": C3EncoderOps,
             "c3_fused": C3Fused,
             "enc_add_ln": EncAddLayerNorm,
             "c4": C4Int8Matvec,
             "c5": C5BatchedDecode, "c5_b32": C5Share, "c5_layer": C5Layer, "w8a32_decode": W8A32Decode, "attn_decode": AttnDecode, "attn_prefill": AttnPrefill,
             "lm_head": LmHead, "decode_step": DecodeStep, "decode_step_b256": DecodeStepBatched,
             "decode_step_b256_w8a8": DecodeStepBatchedW8A8,
             "w8a32_prefill": W8A32Prefill, "prefill_step": PrefillStep}


# ---------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------
def replays_for(steps: int) -> int:
    """Timed replays of the K-step region: at least 5, and at least 100 steps."""
    return max(5, math.ceil(100 / max(1, steps)))


def time_stats(torch, fn, n: int, use_graph: bool, reps: int, between=None) -> dict:
    """ms per call of fn(i), i = 0..n-1: the n calls are captured once into a HIP
    graph (or launched eagerly) and timed ``reps`` times with HIP events on the
    launch stream, each replay bracketed by device synchronisation; ``between``
    runs untimed before each replay (the cache flush of a cold workload).
    Returns the median, p10, p90 and minimum over the replays."""
    import numpy as np

    stream = torch.cuda.current_stream()
    g = None
    if use_graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        g.replay()  # warm the graph once
        torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        if between is not None:
            between()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        if g is not None:
            g.replay()
        else:
            for i in range(n):
                fn(i)
        e.record(stream)
        torch.cuda.synchronize()
        per.append(s.elapsed_time(e) / n)
    del g
    a = np.asarray(per)
    return {"median": float(np.median(a)), "p10": float(np.percentile(a, 10)),
            "p90": float(np.percentile(a, 90)), "min": float(a.min()), "replays": reps}


# ---------------------------------------------------------------------------
# CPU baseline (oracle, reference thread model)
# ---------------------------------------------------------------------------
def host_info(threads: int, build: str) -> dict:
    try:
        nproc = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        nproc = os.cpu_count() or 1
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": nproc, "cpu_count": os.cpu_count(), "cpu_model": model, "threads": threads,
            "oracle_build": build}


def cpu_threads() -> int:
    """The reference pool: min(available cores, MAX_THREADS = 16) (kernels/mod.rs:177, 288-302)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _run_until(fn, budget):
    fn()  # untimed: first touch of the outputs, thread and frequency ramp
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget:
            return n, dt


def cpu_baseline(name: str, seconds: float, step_bytes: int) -> dict:
    """The oracle (a C restatement of the reference's kernels, compiled here
    with -march=native) timed on this host over a bounded sample of the same
    workload, with the reference's thread model: norms, RoPE, SwiGLU,
    LayerNorm, GELU, PE and attention on one thread; the INT8 matvec on
    min(cores, 16) threads in contiguous row chunks, one matvec per token.
    The C functions are called directly on preallocated buffers (no wrapper
    allocation or copy per call). Reported in the GPU step's unit."""
    from ctypes import c_void_p

    import numpy as np

    import oracle

    build = oracle.use_native()
    L = oracle.lib()
    P = lambda a: c_void_p(a.ctypes.data)  # noqa: E731
    r = np.random.default_rng(99)
    nt = cpu_threads()

    def f32(*shape, sc=1.0, m=0.0):
        return (m + sc * r.standard_normal(shape, dtype=np.float32)).astype(np.float32)

    def qweights(o, i, n=1):
        """n distinct int8 weight matrices [o, i] with row scales of the quantizer's range."""
        return [(np.frombuffer(r.bytes(o * i), np.int8).reshape(o, i),
                 (1e-3 + 1e-4 * r.random(o)).astype(np.float32)) for _ in range(n)]

    def qk_gains(hd):
        # q/k head norms run in place, and a step repeats them on the same
        # buffers: a non-unit gain applied hundreds of times drives the smaller
        # components into denormals (slow on x86). Unit gains keep the values
        # bounded; the arithmetic is the same for any gain.
        return np.ones(hd, np.float32), np.ones(hd, np.float32)

    def result(per, threads, sample, tokens_per_step=None):
        out = {"value": step_bytes / per / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
               "ms_per_step": per * 1e3, "sample": sample, "host": host_info(threads, build)}
        if tokens_per_step is not None:
            out["tokens_per_s"] = tokens_per_step / per
        return out

    if name in ("c1", "c1_cold"):
        c = DEC_0_6B
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        S = 64 if name == "c1" else 8192  # 8192 x 84 KB = 688 MB rotates through the host caches
        x, d, y = f32(S, H), f32(S, H), np.empty((S, H), np.float32)
        q, k = f32(S, nq * hd), f32(S, nk * hd)
        g, u, o = f32(S, I), f32(S, I), np.empty((S, I), np.float32)
        (w, (qw, kw)) = f32(H, sc=0.1, m=1.0), qk_gains(hd)
        cos, sin = oracle.rope_table(512, hd, c["theta"])
        pos = r.integers(0, 512, S).astype(np.int32)
        iters = 20000
        args = (P(x), P(d), P(w), P(y), P(q), P(k), P(qw), P(kw), P(cos), P(sin), P(pos), P(o), P(g), P(u),
                H, nq, nk, hd, I, c["eps"])
        n, dt = _run_until(lambda: L.ref_decode_chain_repeat(iters, S, *args), seconds)
        per = dt / (n * iters)
        return result(per, 1, f"{n * iters} decode chains (one layer: add+RMSNorm, q/k head norm+RoPE, "
                              f"SwiGLU) over {S} rotating input sets, one thread, repeated in C",
                      1.0 / 28)
    if name in ("c2",):
        c = DEC_0_6B
        T = 512
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        table = f32(VOCAB, H, sc=0.02)
        ids = r.integers(0, VOCAB, T).astype(np.int32)
        x, d, y = np.empty((T, H), np.float32), f32(T, H), np.empty((T, H), np.float32)
        q, k = f32(T, nq * hd), f32(T, nk * hd)
        gu, o = f32(T, 2 * I), np.empty((T, I), np.float32)
        (w, (qw, kw)) = f32(H, sc=0.1, m=1.0), qk_gains(hd)
        cos, sin = oracle.rope_table(T, hd, c["theta"])
        pos = np.arange(T, dtype=np.int32)

        def step():
            L.ref_embed_gather_f32(P(x), P(table), P(ids), T, H)
            L.ref_add_rms_norm(P(x), P(d), P(w), P(y), T, H, c["eps"])
            L.ref_head_rms_norm_rope(P(q), P(k), P(qw), P(kw), P(cos), P(sin), P(pos), T, nq, nk, hd, c["eps"])
            L.ref_swiglu_multiply(P(o), P(gu), T, I)

        n, dt = _run_until(step, seconds)
        return result(dt / n, 1, f"{n} full c2 steps (T=512) on the oracle, one thread", float(T))
    if name in ("c3", "c3_fused"):
        T, D, FF = 3000, 896, 3584
        x, h, y = f32(T, D), f32(T, FF), np.empty((T, D), np.float32)
        w, bb = f32(D, sc=0.1, m=1.0), f32(D, sc=0.02)
        pe = oracle.sinusoidal_pe(13, D)

        def step():
            L.ref_pe_add(P(x), P(pe), T, D, 13)
            L.ref_layer_norm(P(y), P(x), P(w), P(bb), T, D, 1e-5)
            L.ref_gelu_tanh(P(h), T * FF)  # the reference CPU path's GELU (tanh form)

        n, dt = _run_until(step, seconds)
        return result(dt / n, 1, f"{n} c3 steps on the oracle (PE add, then LayerNorm: the reference has no "
                                 "fused pass), one thread; GELU is the reference's tanh form")
    if name == "c4":
        H, I, NL = 2048, 6144, 28
        ws = qweights(2 * I, H, NL)
        x = f32(H)
        gu, o = np.empty(2 * I, np.float32), np.empty(I, np.float32)
        it = [0]

        def layer():
            wq, sc = ws[it[0] % NL]
            it[0] += 1
            L.ref_linear_nobias_int8(P(gu), P(x), P(wq), P(sc), 1, H, 2 * I, nt)
            L.ref_swiglu_multiply(P(o), P(gu), 1, I)

        n, dt = _run_until(layer, seconds)
        per = dt / n * 28
        return result(per, nt, f"{n} layer matvecs over 28 distinct [12288,2048] int8 weights (W8A32, the "
                               f"reference's INT8 path) + SwiGLU, {nt} threads; a step is 28 layers", 1.0)
    if name in ("c5", "c5_b32"):
        c = DEC_1_7B
        B, NL = (256 if name == "c5" else 32), 28
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        ws = qweights(2 * I, H, NL)
        x, d, y = f32(B, H), f32(B, H), np.empty((B, H), np.float32)
        q, k = f32(B, nq * hd), f32(B, nk * hd)
        (w, (qw, kw)) = f32(H, sc=0.1, m=1.0), qk_gains(hd)
        cos, sin = oracle.rope_table(2048, hd, c["theta"])
        pos = r.integers(0, 2048, B).astype(np.int32)
        gu, o = np.empty((B, 2 * I), np.float32), np.empty((B, I), np.float32)
        it = [0]

        def layer():
            wq, sc = ws[it[0] % NL]
            it[0] += 1
            L.ref_add_rms_norm(P(x), P(d), P(w), P(y), B, H, c["eps"])
            L.ref_head_rms_norm_rope(P(q), P(k), P(qw), P(kw), P(cos), P(sin), P(pos), B, nq, nk, hd, c["eps"])
            # the reference's INT8 path: one W8A32 matvec per stream, then swiglu_multiply
            L.ref_linear_nobias_int8(P(gu), P(y), P(wq), P(sc), B, H, 2 * I, nt)
            L.ref_swiglu_multiply(P(o), P(gu), B, I)

        n, dt = _run_until(layer, seconds)
        return result(dt / n, nt, f"{n} layers of the c{name[1:]} chain (B={B}) on the oracle over 28 distinct "
                                  f"gate/up weights: norms/RoPE/SwiGLU on one thread, the INT8 W8A32 matvec "
                                  f"(one per stream) on {nt} threads", B / 28.0)
    if name == "c5_layer":
        c = DEC_1_7B
        B, NL = 256, 28
        H, nq, nk, hd, I = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["inter"]
        N, kv = (nq + 2 * nk) * hd, nk * hd
        qkv_w, gu_w = qweights(N, H, NL), qweights(2 * I, H, NL)
        x, d, d2, y = f32(B, H), f32(B, H), f32(B, H), np.empty((B, H), np.float32)
        w1, w2, (qw, kw) = f32(H, sc=0.1, m=1.0), f32(H, sc=0.1, m=1.0), qk_gains(hd)
        cos, sin = oracle.rope_table(2048, hd, c["theta"])
        pos = r.integers(0, 2048, B).astype(np.int32)
        qkv, gu, o = np.empty((B, N), np.float32), np.empty((B, 2 * I), np.float32), np.empty((B, I), np.float32)
        q, k = np.empty((B, nq * hd), np.float32), np.empty((B, kv), np.float32)
        kc = np.zeros((B, 64, kv), np.float32)  # the rows written: one per stream (a 64-row block each)
        vc = np.zeros_like(kc)
        it = [0]

        def layer():
            (wq, sq), (wg, sg) = qkv_w[it[0] % NL], gu_w[it[0] % NL]
            it[0] += 1
            L.ref_add_rms_norm(P(x), P(d), P(w1), P(y), B, H, c["eps"])
            # the reference's q/k/v calls: one W8A32 matvec per stream (decoder.rs:881-886)
            L.ref_linear_nobias_int8(P(qkv), P(y), P(wq), P(sq), B, H, N, nt)
            q[:] = qkv[:, :nq * hd]
            k[:] = qkv[:, nq * hd:nq * hd + kv]
            L.ref_head_rms_norm_rope(P(q), P(k), P(qw), P(kw), P(cos), P(sin), P(pos), B, nq, nk, hd, c["eps"])
            kc[np.arange(B), pos % 64] = k        # the k_at / v_at row copies (decoder.rs:894-895)
            vc[np.arange(B), pos % 64] = qkv[:, nq * hd + kv:]
            L.ref_add_rms_norm(P(x), P(d2), P(w2), P(y), B, H, c["eps"])
            L.ref_linear_nobias_int8(P(gu), P(y), P(wg), P(sg), B, H, 2 * I, nt)
            L.ref_swiglu_multiply(P(o), P(gu), B, I)

        n, dt = _run_until(layer, seconds)
        return result(dt / n, nt, f"{n} layers of the c5_layer chain (B=256) on the oracle over 28 distinct "
                                  f"q/k/v and gate/up weights: the reference's W8A32 matvec per stream on {nt} "
                                  "threads, norms/RoPE/SwiGLU and the cache row copies on one", B / 28.0)
    if name in ("decode_step", "decode_step_b256", "decode_step_b256_w8a8"):
        from oracle.decoder import decode_int8_step

        c = DEC_1_7B
        H, I, nq, nk, hd = c["hidden"], c["inter"], c["n_heads"], c["n_kv_heads"], c["head_dim"]
        pos = DecodeStep.POS

        def gain(n):
            return f32(n, sc=0.1, m=1.0)

        layers = []
        for _ in range(28):
            (wq,), (wk,), (wv,), (wo,) = (qweights(nq * hd, H), qweights(nk * hd, H), qweights(nk * hd, H),
                                          qweights(H, nq * hd))
            (gu,), (dn,) = qweights(2 * I, H), qweights(H, I)
            layers.append({"wq": wq, "wk": wk, "wv": wv, "wo": wo, "gate_up": gu, "down": dn,
                           "q_norm": gain(hd), "k_norm": gain(hd), "input_norm": gain(H),
                           "post_attn_norm": gain(H)})
        w = {"layers": layers, "norm": gain(H), "lm_head": qweights(VOCAB, H)[0]}
        kc = f32(28, pos + 1, nk * hd)
        vc = f32(28, pos + 1, nk * hd)
        x = f32(H)
        n, dt = _run_until(lambda: decode_int8_step(w, kc, vc, pos, x, nq, nk, hd, c["eps"], c["theta"], nt),
                           seconds)
        if name.startswith("decode_step_b256"):  # the reference decodes one stream at a time: 256 in turn
            return result(dt / n * 256, nt, f"{n} decode tokens of one stream at position {pos} (the middle of "
                                            "U[0,2047]) on the oracle's restated decode step (decoder.rs:848-965) "
                                            "over 28 distinct layers, scaled to 256 streams decoded in turn (the "
                                            f"reference is single-stream): INT8 matvecs on {nt} threads", 256.0)
        return result(dt / n, nt, f"{n} decode tokens at position {pos} on the oracle's restated decode step "
                                  f"(decoder.rs:848-965) over 28 distinct layers of weights: INT8 matvecs on "
                                  f"{nt} threads, attention and norms on one", 1.0)
    if name == "prefill_step":
        from oracle.decoder import prefill_int8

        c = DEC_0_6B
        H, I, nq, nk, hd, T = c["hidden"], c["inter"], c["n_heads"], c["n_kv_heads"], c["head_dim"], PrefillStep.T

        def gain(n):
            return f32(n, sc=0.1, m=1.0)

        (wq,), (wk,), (wv,), (wo,) = (qweights(nq * hd, H), qweights(nk * hd, H), qweights(nk * hd, H),
                                      qweights(H, nq * hd))
        (gu,), (dn,) = qweights(2 * I, H), qweights(H, I)
        layer = {"wq": wq, "wk": wk, "wv": wv, "wo": wo, "gate_up": gu, "down": dn, "q_norm": gain(hd),
                 "k_norm": gain(hd), "input_norm": gain(H), "post_attn_norm": gain(H)}
        kc = np.zeros((1, T, nk * hd), np.float32)
        vc = np.zeros_like(kc)
        x = f32(T * H)
        n, dt = _run_until(lambda: prefill_int8({"layers": [layer]}, kc, vc, 0, x, T, nq, nk, hd, c["eps"],
                                                c["theta"], nt), seconds)
        per = dt / n * 28
        return result(per, nt, f"{n} layers of a {T}-token prefill on the oracle's restated prefill "
                               f"(decoder.rs:751-847; INT8 linears on {nt} threads, attention and norms on "
                               "one), timed per layer and scaled to the 28 layers", float(T))
    if name == "w8a32_decode":
        shapes = W8A32Decode.SHAPES
        ws = {nm: qweights(o, i)[0] for nm, (o, i) in shapes.items()}
        xs = {nm: f32(i) for nm, (o, i) in shapes.items()}
        ys = {nm: np.empty(o, np.float32) for nm, (o, i) in shapes.items()}

        def layer():
            for nm, (o, i) in shapes.items():
                L.ref_linear_nobias_int8(P(ys[nm]), P(xs[nm]), P(ws[nm][0]), P(ws[nm][1]), 1, i, o, nt)

        n, dt = _run_until(layer, seconds)
        return result(dt / n * 28, nt, f"{n} layers of the six W8A32 projections on the oracle, {nt} threads "
                                       "(one layer's weights reused: LLC-warm)", 1.0)
    if name in ("attn_decode", "attn_prefill"):
        nq, nk, hd = 16, 8, 128
        seq_q, seq_k, off = (1, 2048, 2047) if name == "attn_decode" else (512, 512, 0)
        q, kk, v = f32(seq_q * nq * hd), f32(seq_k * nk * hd), f32(seq_k * nk * hd)
        o = np.empty(seq_q * nq * hd, np.float32)
        n, dt = _run_until(lambda: L.ref_causal_attention(P(o), P(q), P(kk), P(v), seq_q, seq_k, nq, nk, hd,
                                                          hd ** -0.5, off), seconds)
        per = dt / n * (28 if name == "attn_decode" else 1)
        return result(per, 1, f"{n} {name} calls on the oracle, one thread (the reference threads over heads)",
                      1.0 if name == "attn_decode" else 512.0)
    if name == "lm_head":
        V, H = VOCAB, 1024
        (wq, sc), = qweights(V, H)
        x, lg, idx = f32(H), np.empty(V, np.float32), np.empty(1, np.int32)

        def step():
            L.ref_linear_nobias_int8(P(lg), P(x), P(wq), P(sc), 1, H, V, nt)
            L.ref_argmax_rows(P(idx), P(lg), 1, V)

        n, dt = _run_until(step, seconds)
        return result(dt / n, nt, f"{n} INT8 lm_head matvecs + argmax on the oracle, {nt} threads", 1.0)
    raise ValueError(name)


# ---------------------------------------------------------------------------
# Counter runs (rocprofv3 --pmc): one kernel at a time
# ---------------------------------------------------------------------------
COPY_BYTES = 64 << 20


def profile_copy(torch, dev, n: int) -> int:
    """A plain copy of known size: COPY_BYTES read + COPY_BYTES written per
    launch. Its FETCH_SIZE / WRITE_SIZE readings calibrate those counters."""
    src = [torch.ones(COPY_BYTES // 4, device=dev) for _ in range(8)]
    dst = [torch.empty(COPY_BYTES // 4, device=dev) for _ in range(8)]
    torch.cuda.synchronize()
    for i in range(n):
        dst[i % 8].copy_(src[i % 8])
    torch.cuda.synchronize()
    print(json.dumps({"profile_kernel": "copy", "launches": n, "read_bytes": COPY_BYTES,
                      "write_bytes": COPY_BYTES}), flush=True)
    return 0


def profile_kernel(torch, wl, name: str, n: int) -> int:
    """Launches one kernel of the workload n times (rotating buffers), or with
    NAME "all" every kernel in turn, n times each. In "all" mode a marker
    dispatch (argmax_rows_kernel<false> over 3 values) precedes each kernel's
    launches and follows the last, so a per-dispatch counter trace splits into
    the kernels' groups by position."""
    from qwenasr_amd import kernels as K

    names = list(wl.kernels) if name == "all" else [name]
    for nm in names:
        if nm not in wl.kernels:
            print(f"bench.py: workload {wl.name} has no kernel {nm!r} (has {sorted(wl.kernels)})",
                  file=sys.stderr)
            return 2
    idx = torch.zeros(1, dtype=torch.int32, device=wl.dev)
    mx = torch.zeros(3, device=wl.dev)
    for nm in names:
        if name == "all":
            K.argmax_rows(idx, mx, 1, 3)
        launch, nbytes = wl.kernels[nm][0], wl.kernels[nm][1]
        for i in range(n):
            launch(i)
        torch.cuda.synchronize()
        print(json.dumps({"profile_kernel": nm, "workload": wl.name, "launches": n,
                          "algorithmic_bytes": nbytes}), flush=True)
    if name == "all":
        K.argmax_rows(idx, mx, 1, 3)
        torch.cuda.synchronize()
    return 0


PROBE_MODES = {0: "one region per XCD, all its workgroups in the same order",
               1: "one region per XCD, each workgroup from its own rotation",
               2: "private 64 KiB per workgroup, L2-resident",
               3: "private region per workgroup read once (HBM stream)",
               4: "as 2, wave pairs w, w+4 on the same addresses",
               5: "as 3, wave pairs w, w+4 on the same addresses"}
PROBE_BUF = 1 << 30
PROBE_PRIV = 64 << 10


def _probe_launch(torch, buf, out, mode, depth, grid, per_wg, i):
    from qwenasr_amd import _lib

    shift = i % 4 if mode in (3, 5) else 0
    _lib.call("qasr_probe_read", mode, depth, grid, buf.data_ptr(), buf.numel(), out.data_ptr(), out.numel(),
              per_wg, PROBE_PRIV, shift, torch.cuda.current_stream().cuda_stream)


def probe_fill(torch, dev, one=None) -> int:
    """The read-rate probe (qasr_probe_read): per mode, workgroups of 512
    threads read 256 KiB, 512 KiB and 1 MiB per CU (256 or 512 workgroups);
    the marginal per-CU rate between 512 KiB and 1 MiB removes the launch and
    ramp. With ``one`` = (mode, depth, grid, KiB per workgroup): 20 eager
    launches of that case alone, for counter passes."""
    import numpy as np

    buf = torch.randint(-128, 127, (PROBE_BUF,), dtype=torch.int8, device=dev)
    out = torch.empty(4096 * 512, dtype=torch.int32, device=dev)
    if one is not None:
        mode, depth, grid, kib = one
        for i in range(20):
            _probe_launch(torch, buf, out, mode, depth, grid, kib << 10, i)
        torch.cuda.synchronize()
        print(json.dumps({"probe": one, "launches": 20}), flush=True)
        return 0
    rows = []
    for grid in (256, 512):
        for mode in PROBE_MODES:
            for depth in (4, 16):
                us = []
                per_cu = (256 << 10, 512 << 10, 1 << 20)
                for pc in per_cu:
                    per_wg = pc * 256 // grid
                    g = torch.cuda.CUDAGraph()
                    _probe_launch(torch, buf, out, mode, depth, grid, per_wg, 0)
                    with torch.cuda.graph(g):
                        for i in range(20):
                            _probe_launch(torch, buf, out, mode, depth, grid, per_wg, i)
                    g.replay()
                    torch.cuda.synchronize()
                    t = []
                    for _ in range(7):
                        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        s0.record()
                        g.replay()
                        e0.record()
                        torch.cuda.synchronize()
                        t.append(s0.elapsed_time(e0) * 1e3 / 20)
                    us.append(float(np.median(t)))
                    del g
                marginal = (per_cu[2] - per_cu[1]) / ((us[2] - us[1]) * 1e-6) / 1e9
                row = {"grid": grid, "mode": mode, "what": PROBE_MODES[mode], "depth": depth,
                       "per_cu_KiB": [x >> 10 for x in per_cu], "us": [round(x, 2) for x in us],
                       "TB/s": [round(256 * pc / (u * 1e-6) / 1e12, 2) for pc, u in zip(per_cu, us)],
                       "marginal_per_cu_GB/s": round(marginal, 1)}
                rows.append(row)
                print(f"[probe] grid {grid} mode {mode} depth {depth}: us {row['us']} marginal per CU "
                      f"{row['marginal_per_cu_GB/s']} GB/s", file=sys.stderr, flush=True)
    print(json.dumps({"probe": "qasr_probe_read", "rows": rows}), flush=True)
    return 0


# ---------------------------------------------------------------------------
DEFAULT_CONFIGS = "c1,c1_cold,c2,c3_fused,c4,c5_b32,c5_layer,decode_step,decode_step_b256,decode_step_b256_w8a8,prefill_step"


def _round(v):
    if isinstance(v, float):
        return round(v, 4)
    if isinstance(v, dict):
        return {k: _round(x) for k, x in v.items()}
    return v


_FLUSH = {}


def cache_flush(torch, dev):
    """Writes 1 GiB (4x the 256 MB last-level cache) so that nothing a timed
    replay reads afterwards is still cached."""
    if "buf" not in _FLUSH:
        _FLUSH["buf"] = torch.empty(FLUSH_BYTES // 4, device=dev)
    _FLUSH["buf"].fill_(1.0)


def measure(torch, dev, wl, K: int, W: int, use_graph: bool) -> dict:
    """Warmup, then the step and each kernel timed (median over replays of
    K launches), the roofline of the kernel moving the most bytes. A workload
    with a max_steps (a step of many milliseconds) times min(K, max_steps)
    steps per replay; one with a min_steps at least that many.

    Unless the workload is hot by design, a replay that touches less than
    2x the last-level cache (its launches x their algorithmic bytes) is
    preceded by writing 1 GiB, and a kernel's own graph holds at most as many
    launches as it has distinct buffer sets (its rotation): every launch in a
    replay then reads inputs that no cache holds."""
    K = max(K, getattr(wl, "min_steps", 1))
    K = min(K, getattr(wl, "max_steps", K))
    W = min(W, getattr(wl, "max_steps", W))
    reps = replays_for(K)
    n_kernel = min(K, wl.rotation or K)

    def flush_for(footprint):
        if getattr(wl, "between", None) is not None:
            return wl.between
        if wl.hot or footprint >= ROTATE_BYTES:
            return None
        return lambda: cache_flush(torch, dev)

    def cache_note(footprint):
        if wl.hot:
            return "hot by design (no flush)"
        if getattr(wl, "between", None) is not None:
            return "cold: the workload's own flush before each replay"
        if footprint >= ROTATE_BYTES:
            return f"replay streams {footprint / 1e6:.0f} MB (>= 2x the last-level cache)"
        return f"replay touches {footprint / 1e6:.0f} MB; 1 GiB written before each replay"

    between = flush_for(K * wl.step_bytes)
    for i in range(W):
        wl.step(i)
    torch.cuda.synchronize()
    try:
        step = time_stats(torch, wl.step, K, use_graph, reps, between)
    except RuntimeError as ex:  # capture unsupported: time eagerly
        print(f"[bench] {wl.name}: graph capture failed ({ex}); timing eagerly", file=sys.stderr)
        use_graph = False
        step = time_stats(torch, wl.step, K, False, reps, between)
    ms = step["median"]
    print(f"[bench] {wl.name}: step {ms * 1e3:.2f} us (p10 {step['p10'] * 1e3:.2f}, p90 {step['p90'] * 1e3:.2f})",
          file=sys.stderr, flush=True)
    per_kernel = {}
    for kname, spec in wl.kernels.items():
        launch, nbytes = spec[0], spec[1]
        st = time_stats(torch, launch, n_kernel, use_graph, replays_for(n_kernel), flush_for(n_kernel * nbytes))
        us = st["median"] * 1e3
        d = {"us": us, "us_p10": st["p10"] * 1e3, "us_p90": st["p90"] * 1e3, "bytes": nbytes,
             "GB/s": nbytes / (us * 1e-6) / 1e9, "frac_hbm": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
             "launches_per_replay": n_kernel, "replays": st["replays"],
             "footprint_per_replay_MB": round(n_kernel * nbytes / 1e6, 1),
             "cache": cache_note(n_kernel * nbytes)}
        if len(spec) > 2:
            d["flops"] = spec[2]
            d["TFLOP/s"] = spec[2] / (us * 1e-6) / 1e12
        per_kernel[kname] = d
        print(f"[bench] {wl.name}/{kname}: {us:.2f} us, {d['GB/s']:.0f} GB/s", file=sys.stderr, flush=True)
    value = wl.step_bytes / (ms * 1e-3) / 1e9
    return {"step": step, "use_graph": use_graph, "per_kernel": per_kernel, "value": value,
            "tokens_per_s": wl.tokens_per_step / (ms * 1e-3), "steps": K,
            "cache": cache_note(K * wl.step_bytes)}


def roofline_of(torch, dev, wl, m: dict, K: int) -> dict:
    per_kernel = m["per_kernel"]
    # dominant kernel = the one moving the most algorithmic bytes per step
    dom_name = max(per_kernel, key=lambda k: per_kernel[k]["bytes"])
    dom = per_kernel[dom_name]
    traffic = traffic_entry = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        try:
            data = json.loads(tfile.read_text())
            # a derived workload (c3_fused) runs its parent's kernels at the same shapes
            for name in [getattr(c, "name", "") for c in type(wl).__mro__]:
                entry = data.get(name, {}).get(dom_name)
                if entry:
                    traffic, traffic_entry = entry["hbm_bytes_per_launch"], entry
                    break
        except (ValueError, OSError, KeyError, TypeError):
            traffic = None
    mfma_peak = getattr(wl, "mfma_peak_tflops", FP32_PEAK_TFLOPS)
    if "flops" in dom and dom["flops"] / dom["bytes"] > mfma_peak * 1e12 / (HBM_PEAK_GBS * 1e9):
        roofline = {"bound": "mfma", "kernel": dom_name, "achieved": round(dom["TFLOP/s"], 2),
                    "peak": round(mfma_peak, 1), "unit": "TFLOP/s",
                    "frac": round(dom["TFLOP/s"] / mfma_peak, 4), "traffic": traffic,
                    "avg_us": round(dom["us"], 3), "algorithmic_flops": dom["flops"],
                    "algorithmic_bytes": dom["bytes"],
                    "peak_basis": getattr(wl, "mfma_peak_basis", "fp32 MFMA, 157.3 TFLOP/s dense")}
    else:
        roofline = {"bound": "hbm", "kernel": dom_name, "achieved": round(dom["GB/s"], 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(dom["frac_hbm"], 4),
                    "traffic": traffic, "avg_us": round(dom["us"], 3), "algorithmic_bytes": dom["bytes"]}
    roofline["timing"] = "median over replays of K graph-replayed launches, HIP events on the launch stream"
    if traffic_entry is not None:
        roofline["traffic_source"] = (f"profiles/traffic.json: rocprofv3 FETCH_SIZE/WRITE_SIZE of "
                                      f"{traffic_entry.get('kernel')}, scaled by a 64 MiB copy's readings")
    if roofline["bound"] == "hbm" and m["use_graph"]:
        # context for frac: a device copy moving the same bytes (half read, half
        # written) over rotating buffers, timed the same way
        n_f = max(1, dom["bytes"] // 8)
        n_sets = sets_for(dom["bytes"])
        src = [torch.randn(n_f, device=dev) for _ in range(n_sets)]
        dst = [torch.empty(n_f, device=dev) for _ in range(n_sets)]
        c = time_stats(torch, lambda i: dst[i % n_sets].copy_(src[i % n_sets]), K, True, replays_for(K))
        c_us = c["median"] * 1e3
        roofline["copy_same_bytes"] = {"us": round(c_us, 3), "GB/s": round(8 * n_f / (c_us * 1e-6) / 1e9, 1),
                                       "frac": round(8 * n_f / (c_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del src, dst
    if hasattr(wl, "gemm_ops") and "gate_up_swiglu_w8a8_gemm" in per_kernel:
        g = per_kernel["gate_up_swiglu_w8a8_gemm"]
        roofline["gemm_mfma_int8_TOPS"] = round(wl.gemm_ops / (g["us"] * 1e-6) / 1e12, 1)
        roofline["gemm_mfma_frac_of_5000_TOPS"] = round(wl.gemm_ops / (g["us"] * 1e-6) / 5.0e15, 4)
    return roofline


def summary(wl, m: dict, cpu) -> dict:
    st = m["step"]
    out = {"workload": wl.description, **wl.config(),
           "us_per_step": round(st["median"] * 1e3, 3), "us_p10": round(st["p10"] * 1e3, 3),
           "us_p90": round(st["p90"] * 1e3, 3), "us_min": round(st["min"] * 1e3, 3), "replays": st["replays"],
           "steps_per_replay": m["steps"], "cache": m["cache"],
           "algorithmic_bytes_per_step": wl.step_bytes, "GB/s": round(m["value"], 1),
           "frac_hbm": round(m["value"] / HBM_PEAK_GBS, 4), "tokens_per_s": round(m["tokens_per_s"], 1),
           "dtype": wl.dtype,
           "per_kernel": {k: _round(v) for k, v in m["per_kernel"].items()}}
    if cpu is not None:
        out["cpu_baseline"] = _round(cpu)
    return out


def free(torch, wl) -> None:
    import gc

    del wl
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c5", choices=sorted(WORKLOADS),
                    help="the headline workload (value, roofline, cpu_baseline)")
    ap.add_argument("--configs", default=DEFAULT_CONFIGS,
                    help="comma-separated workloads also measured in this run, each reported under "
                         "'configs' with its own CPU baseline ('none' for none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU sample of the headline workload")
    ap.add_argument("--config-cpu-seconds", type=float, default=4.0, help="CPU sample of each other config")
    ap.add_argument("--eager", action="store_true", help="launch from the host instead of graph replay")
    ap.add_argument("--profile-kernel", metavar="NAME",
                    help="for counter runs under rocprofv3: launch only this kernel of the workload "
                         "--steps times (rotating buffers), eagerly, and print what ran; NAME 'copy' "
                         "launches a plain 64 MiB device-to-device copy instead (the counter calibration)")
    ap.add_argument("--probe", action="store_true",
                    help="run the per-CU read-rate probe (qasr_probe_read) and print its table")
    ap.add_argument("--probe-one", metavar="MODE,DEPTH,GRID,KIB",
                    help="for counter runs: 20 launches of one probe case (KiB read per workgroup)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: measures one GPU; --gpus {args.gpus} is not supported "
              "(the path shards as pure data parallelism with no exchange between GPUs)",
              file=sys.stderr)
        return 2

    import torch

    from qwenasr_amd import _lib

    _lib.lib()  # fail loudly if the HIP library is missing
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    K, W = args.steps, args.warmup
    Workload.steps_hint = K

    if args.profile_kernel == "copy":
        return profile_copy(torch, dev, K)
    if args.probe or args.probe_one:
        one = tuple(int(v) for v in args.probe_one.split(",")) if args.probe_one else None
        return probe_fill(torch, dev, one)
    wl = WORKLOADS[args.workload](dev, torch)
    torch.cuda.synchronize()
    if args.profile_kernel:
        return profile_kernel(torch, wl, args.profile_kernel, K)
    use_graph = not args.eager
    print(f"[bench] workload {wl.name}: {len(wl.kernels)} kernels, warmup {W}, steps {K}, "
          f"{replays_for(K)} replays, {'graph replay' if use_graph else 'eager'}", file=sys.stderr, flush=True)

    m = measure(torch, dev, wl, K, W, use_graph)
    roofline = roofline_of(torch, dev, wl, m, K)
    cpu = None
    if not args.no_cpu_baseline:
        print(f"[bench] cpu baseline {wl.name} ({args.cpu_seconds:.0f} s sample)...", file=sys.stderr, flush=True)
        cpu = _round(cpu_baseline(wl.name, args.cpu_seconds, wl.step_bytes))
    head = summary(wl, m, None)
    st = m["step"]
    out = {
        "metric": METRIC,
        "value": round(m["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(st["median"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.dtype,
        "data": "synthetic (seeded torch.randn inputs, random-init weights; no checkpoints)",
        "config": {"workload": wl.description, **wl.config(),
                   "timing": (f"median over {st['replays']} replays of a hipGraph of K steps, HIP events"
                              if m["use_graph"] else f"median over {st['replays']} eager runs of K steps"),
                   "cache": m["cache"]},
        "ms_per_step_p10": round(st["p10"], 6),
        "ms_per_step_p90": round(st["p90"], 6),
        "ms_per_step_min": round(st["min"], 6),
        "pct_hbm_peak": round(100 * m["value"] / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(m["tokens_per_s"], 1),
        "per_kernel": head["per_kernel"],
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    free(torch, wl)

    configs = {}
    names = [c for c in args.configs.split(",") if c and c != "none" and c != args.workload]
    for name in names:
        if name not in WORKLOADS:
            print(f"bench.py: unknown config {name!r}", file=sys.stderr)
            return 2
        cw = WORKLOADS[name](dev, torch)
        torch.cuda.synchronize()
        cm = measure(torch, dev, cw, K, W, use_graph)
        ccpu = None
        if not args.no_cpu_baseline:
            # the W8A8 and W8A32 batched steps share one reference baseline (the reference is W8A32)
            same = "decode_step_b256" if name == "decode_step_b256_w8a8" else None
            if same in configs and configs[same].get("cpu_baseline"):
                ccpu = configs[same]["cpu_baseline"]
            else:
                print(f"[bench] cpu baseline {name} ({args.config_cpu_seconds:.0f} s sample)...", file=sys.stderr,
                      flush=True)
                ccpu = cpu_baseline(name, args.config_cpu_seconds, cw.step_bytes)
        configs[name] = summary(cw, cm, ccpu)
        free(torch, cw)
    if configs:
        out["configs"] = configs
    if "decode_step" in configs:
        out["decode_tokens_per_s"] = configs["decode_step"]["tokens_per_s"]
    if "decode_step_b256" in configs:
        out["batched_decode_tokens_per_s"] = configs["decode_step_b256"]["tokens_per_s"]
    if "decode_step_b256_w8a8" in configs:
        out["batched_decode_w8a8_tokens_per_s"] = configs["decode_step_b256_w8a8"]["tokens_per_s"]
    if "prefill_step" in configs:
        out["prefill_tokens_per_s"] = configs["prefill_step"]["tokens_per_s"]
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
