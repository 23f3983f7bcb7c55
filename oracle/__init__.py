"""CPU oracle for the QwenASR fused-layer path -- TEST INFRASTRUCTURE ONLY.

Thin numpy wrappers over ``oracle/_build/libqasr_oracle.so`` (built from
``oracle/qasr_oracle.c`` by ``oracle/build.py``), a C restatement of the
reference Rust kernels. Only tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this package; the product library
never does.

All wrappers take and return numpy arrays (C-contiguous, the dtype named in
each function) and follow the reference argument order.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_size_t, c_void_p
from pathlib import Path

import numpy as np

SO = Path(__file__).resolve().parent / "_build" / "libqasr_oracle.so"

_P, _Z, _F, _I = c_void_p, c_size_t, c_float, c_int

_SIGS = {
    "ref_add_inplace": [_P, _P, _Z],
    "ref_rms_norm": [_P, _P, _P, _Z, _Z, _F],
    "ref_add_rms_norm": [_P, _P, _P, _P, _Z, _Z, _F],
    "ref_layer_norm": [_P, _P, _P, _P, _Z, _Z, _F],
    "ref_rms_norm_per_head": [_P, _P, _Z, _Z, _Z, _F],
    "ref_rope_inv_freq": [_P, _Z, _F],
    "ref_rope_table": [_P, _P, _Z, _Z, _F],
    "ref_apply_rope_neox": [_P, _P, _P, _Z, _Z, _Z],
    "ref_head_rms_norm_rope": [_P, _P, _P, _P, _P, _P, _P, _Z, _Z, _Z, _Z, _F],
    "ref_swiglu_multiply": [_P, _P, _Z, _Z],
    "ref_swiglu_split": [_P, _P, _P, _Z],
    "ref_silu": [_P, _Z],
    "ref_gelu_tanh": [_P, _Z],
    "ref_gelu_erf": [_P, _Z],
    "ref_sinusoidal_pe": [_P, _Z, _Z],
    "ref_pe_add": [_P, _P, _Z, _Z, _Z],
    "ref_embed_gather_f32": [_P, _P, _P, _Z, _Z],
    "ref_embed_gather_bf16": [_P, _P, _P, _Z, _Z],
    "ref_embed_gather_i8": [_P, _P, _P, _P, _Z, _Z],
    "ref_quantize_f32_to_int8": [_P, _P, _P, _Z, _Z],
    "ref_quantize_bf16_to_int8": [_P, _P, _P, _Z, _Z],
    "ref_linear_nobias_int8": [_P, _P, _P, _P, _Z, _Z, _Z, _I],
    "ref_linear_int8": [_P, _P, _P, _P, _P, _Z, _Z, _Z, _I],
    "ref_interleave_gate_up": [_P, _P, _P, _P, _P, _P, _Z, _Z],
    "ref_gate_up_swiglu_w8a8": [_P, _P, _P, _P, _P, _P, _Z, _Z, _Z],
    "ref_argmax_rows": [_P, _P, _Z, _Z],
    "ref_linear_w8a8": [_P, _P, _P, _P, _P, _P, _Z, _Z, _Z],
    "ref_causal_attention": [_P, _P, _P, _P, _Z, _Z, _Z, _Z, _Z, _F, _Z],
    "ref_decode_chain_repeat": [_Z, _Z, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                _Z, _Z, _Z, _Z, _Z, _F],
}

_LIB = None
_LIB_KIND = "x86-64-v3"


def _load(path: Path) -> ctypes.CDLL:
    so = ctypes.CDLL(str(path))
    for name, args in _SIGS.items():
        fn = getattr(so, name)
        fn.argtypes = args
        fn.restype = None
    so.ref_fast_exp.argtypes = [_F]
    so.ref_fast_exp.restype = _F
    return so


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not SO.exists():
            from . import build as _build

            _build.build()
        _LIB = _load(SO)
    return _LIB


def use_native() -> str:
    """For the timed CPU baseline only: compile the oracle with -march=native
    on this host and route every wrapper through that copy. Returns the build
    used ("native", or "x86-64-v3" with the reason the native build failed)."""
    global _LIB, _LIB_KIND
    from . import build as _build

    try:
        _LIB = _load(_build.build(native=True))
        _LIB_KIND = "native"
    except (RuntimeError, OSError) as ex:
        _LIB_KIND = f"x86-64-v3 (native build failed: {ex})"
        lib()
    return _LIB_KIND


def _p(a: np.ndarray | None) -> c_void_p:
    if a is None:
        return c_void_p(0)
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return c_void_p(a.ctypes.data)


def _f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


# --- norms -----------------------------------------------------------------
def add_inplace(a: np.ndarray, b: np.ndarray) -> None:
    lib().ref_add_inplace(_p(a), _p(b), a.size)


def rms_norm(x, w, seq_len, hidden, eps) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    out = np.empty(seq_len * hidden, np.float32)
    lib().ref_rms_norm(_p(out), _p(x), _p(w), seq_len, hidden, eps)
    return out


def add_rms_norm(x, delta, w, seq_len, hidden, eps):
    """Returns (updated x, out)."""
    x = _f32(x).copy()
    delta, w = _f32(delta), _f32(w)
    out = np.empty(seq_len * hidden, np.float32)
    lib().ref_add_rms_norm(_p(x), _p(delta), _p(w), _p(out), seq_len, hidden, eps)
    return x, out


def layer_norm(x, w, b, seq_len, hidden, eps) -> np.ndarray:
    x, w, b = _f32(x), _f32(w), _f32(b)
    out = np.empty(seq_len * hidden, np.float32)
    lib().ref_layer_norm(_p(out), _p(x), _p(w), _p(b), seq_len, hidden, eps)
    return out


def rms_norm_per_head(x, w, seq_len, n_heads, head_dim, eps) -> np.ndarray:
    x = _f32(x).copy()
    w = _f32(w)
    lib().ref_rms_norm_per_head(_p(x), _p(w), seq_len, n_heads, head_dim, eps)
    return x


# --- RoPE ----------------------------------------------------------------------
def rope_inv_freq(head_dim, theta) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    lib().ref_rope_inv_freq(_p(out), head_dim, theta)
    return out


def rope_table(n_pos, head_dim, theta):
    cos = np.empty(n_pos * head_dim, np.float32)
    sin = np.empty(n_pos * head_dim, np.float32)
    lib().ref_rope_table(_p(cos), _p(sin), n_pos, head_dim, theta)
    return cos, sin


def apply_rope_neox(x, cos_vals, sin_vals, seq, n_heads, head_dim) -> np.ndarray:
    x = _f32(x).copy()
    lib().ref_apply_rope_neox(_p(x), _p(_f32(cos_vals)), _p(_f32(sin_vals)), seq, n_heads,
                              head_dim)
    return x


def head_rms_norm_rope(q, k, qw, kw, cos_tab, sin_tab, positions, seq, n_heads, n_kv_heads,
                       head_dim, eps):
    q = _f32(q).copy()
    k = _f32(k).copy()
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    lib().ref_head_rms_norm_rope(_p(q), _p(k), _p(_f32(qw)), _p(_f32(kw)), _p(_f32(cos_tab)),
                                 _p(_f32(sin_tab)), _p(pos), seq, n_heads, n_kv_heads, head_dim,
                                 eps)
    return q, k


# --- activations -----------------------------------------------------------
def fast_exp(x: float) -> float:
    return lib().ref_fast_exp(x)


def swiglu_multiply(gate_up, seq_len, inter) -> np.ndarray:
    out = np.empty(seq_len * inter, np.float32)
    lib().ref_swiglu_multiply(_p(out), _p(_f32(gate_up)), seq_len, inter)
    return out


def swiglu_split(gate, up) -> np.ndarray:
    gate, up = _f32(gate), _f32(up)
    out = np.empty(gate.size, np.float32)
    lib().ref_swiglu_split(_p(out), _p(gate), _p(up), gate.size)
    return out


def silu(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().ref_silu(_p(x), x.size)
    return x


def gelu_tanh(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().ref_gelu_tanh(_p(x), x.size)
    return x


def gelu_erf(x) -> np.ndarray:
    x = _f32(x).copy()
    lib().ref_gelu_erf(_p(x), x.size)
    return x


def sinusoidal_pe(n_pos, d_model) -> np.ndarray:
    pe = np.empty(n_pos * d_model, np.float32)
    lib().ref_sinusoidal_pe(_p(pe), n_pos, d_model)
    return pe


def pe_add(x, pe, rows, d_model, n_pos) -> np.ndarray:
    x = _f32(x).copy()
    lib().ref_pe_add(_p(x), _p(_f32(pe)), rows, d_model, n_pos)
    return x


# --- gathers -------------------------------------------------------------------
def embed_gather_f32(table, ids, dim) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.empty(ids.size * dim, np.float32)
    lib().ref_embed_gather_f32(_p(out), _p(_f32(table)), _p(ids), ids.size, dim)
    return out


def embed_gather_bf16(table_u16, ids, dim) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.int32)
    t = np.ascontiguousarray(table_u16, np.uint16)
    out = np.empty(ids.size * dim, np.float32)
    lib().ref_embed_gather_bf16(_p(out), _p(t), _p(ids), ids.size, dim)
    return out


def embed_gather_i8(table_i8, scales, ids, dim) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.int32)
    t = np.ascontiguousarray(table_i8, np.int8)
    out = np.empty(ids.size * dim, np.float32)
    lib().ref_embed_gather_i8(_p(out), _p(t), _p(_f32(scales)), _p(ids), ids.size, dim)
    return out


# --- INT8 ----------------------------------------------------------------------
def quantize_f32_to_int8(x, out_dim, in_dim):
    x = _f32(x)
    q = np.empty(out_dim * in_dim, np.int8)
    s = np.empty(out_dim, np.float32)
    lib().ref_quantize_f32_to_int8(_p(q), _p(s), _p(x), out_dim, in_dim)
    return q, s


def quantize_bf16_to_int8(x_u16, out_dim, in_dim):
    x = np.ascontiguousarray(x_u16, np.uint16)
    q = np.empty(out_dim * in_dim, np.int8)
    s = np.empty(out_dim, np.float32)
    lib().ref_quantize_bf16_to_int8(_p(q), _p(s), _p(x), out_dim, in_dim)
    return q, s


def linear_nobias_int8(x, w, scales, seq_len, in_dim, out_dim, n_threads=1) -> np.ndarray:
    y = np.empty(seq_len * out_dim, np.float32)
    lib().ref_linear_nobias_int8(_p(y), _p(_f32(x)), _p(np.ascontiguousarray(w, np.int8)),
                                 _p(_f32(scales)), seq_len, in_dim, out_dim, n_threads)
    return y


def linear_int8(x, w, scales, bias, seq_len, in_dim, out_dim, n_threads=1) -> np.ndarray:
    y = np.empty(seq_len * out_dim, np.float32)
    lib().ref_linear_int8(_p(y), _p(_f32(x)), _p(np.ascontiguousarray(w, np.int8)),
                          _p(_f32(scales)), _p(None if bias is None else _f32(bias)), seq_len,
                          in_dim, out_dim, n_threads)
    return y


def interleave_gate_up(wg, sg, wu, su, inter, hidden):
    wgu = np.empty(2 * inter * hidden, np.int8)
    sgu = np.empty(2 * inter, np.float32)
    lib().ref_interleave_gate_up(_p(wgu), _p(sgu), _p(np.ascontiguousarray(wg, np.int8)),
                                 _p(_f32(sg)), _p(np.ascontiguousarray(wu, np.int8)), _p(_f32(su)),
                                 inter, hidden)
    return wgu, sgu


def gate_up_swiglu_w8a8(w, scales, xq, x_scales, batch, in_dim, inter):
    """Returns (out [batch*inter] f32, dots [batch*2*inter] int32)."""
    out = np.empty(batch * inter, np.float32)
    dots = np.empty(batch * 2 * inter, np.int32)
    lib().ref_gate_up_swiglu_w8a8(_p(out), _p(dots), _p(np.ascontiguousarray(w, np.int8)),
                                  _p(_f32(scales)), _p(np.ascontiguousarray(xq, np.int8)),
                                  _p(_f32(x_scales)), batch, in_dim, inter)
    return out, dots


def linear_w8a8(w, scales, xq, x_scales, batch, in_dim, out_dim):
    """Returns (y [batch*out_dim] f32, dots [batch*out_dim] int32)."""
    y = np.empty(batch * out_dim, np.float32)
    dots = np.empty(batch * out_dim, np.int32)
    lib().ref_linear_w8a8(_p(y), _p(dots), _p(np.ascontiguousarray(w, np.int8)), _p(_f32(scales)),
                          _p(np.ascontiguousarray(xq, np.int8)), _p(_f32(x_scales)), batch, in_dim, out_dim)
    return y, dots


def argmax_rows(x, rows, cols) -> np.ndarray:
    """The lm_head argmax loop of decoder.rs:941-949 per row (first maximum
    wins; a NaN never wins unless it is element 0)."""
    x = _f32(x)
    idx = np.empty(rows, np.int32)
    lib().ref_argmax_rows(_p(idx), _p(x), rows, cols)
    return idx


def causal_attention(q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset):
    """kernels/mod.rs:1124-1168 with the x86_64 vector helpers."""
    out = np.empty(seq_q * n_heads * head_dim, np.float32)
    lib().ref_causal_attention(_p(out), _p(_f32(q)), _p(_f32(k)), _p(_f32(v)), seq_q, seq_k,
                               n_heads, n_kv_heads, head_dim, scale, q_offset)
    return out
