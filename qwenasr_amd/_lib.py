"""ctypes binding of the C-ABI in include/qasr.h.

The shared library ``qwenasr_amd/libqasr_hip.so`` is the only implementation of
the kernels: there is no CPU fallback. If it is missing, ``lib()`` raises
``QasrLibraryMissing`` -- build it with ``python -m qwenasr_amd.build``.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_size_t, c_void_p, c_char_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqasr_hip.so"

QASR_OK = 0
QASR_ERR_INVALID_ARG = 1
QASR_ERR_UNSUPPORTED = 2
QASR_ERR_HIP = 3


class QasrLibraryMissing(ImportError):
    pass


class QasrError(RuntimeError):
    """A C-ABI call returned a non-zero qasr_status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with status {code}: {msg}")
        self.fn = fn
        self.code = code
        self.msg = msg


P = c_void_p
Z = c_size_t
F = c_float

# name -> argument types (every pointer is a device pointer passed as void*;
# the trailing void* is the hipStream_t).
SIGNATURES: dict[str, list] = {
    "qasr_add_inplace_f32": [P, P, Z, P],
    "qasr_rms_norm_f32": [P, P, P, Z, Z, F, P],
    "qasr_add_rms_norm_f32": [P, P, P, P, Z, Z, F, P],
    "qasr_add_rms_norm_quant_f32": [P, P, P, P, P, P, Z, Z, F, P],
    "qasr_layer_norm_f32": [P, P, P, P, Z, Z, F, P],
    "qasr_add_layer_norm_f32": [P, P, P, P, P, Z, Z, F, P],
    "qasr_rms_norm_per_head_f32": [P, P, Z, Z, Z, F, P],
    "qasr_apply_rope_neox_f32": [P, P, P, Z, Z, Z, P],
    "qasr_head_rms_norm_rope_f32": [P, P, P, P, P, P, P, Z, Z, Z, Z, Z, F, P],
    "qasr_argmax_rows_f32": [P, P, Z, Z, P],
    "qasr_causal_attention_f32": [P, P, P, P, Z, Z, Z, Z, Z, F, Z, P],
    "qasr_causal_attention_split_f32": [P, P, P, P, Z, Z, Z, Z, Z, F, Z, P, Z, P],
    "qasr_decode_attention_f32": [P, P, P, P, P, P, P, P, Z, Z, Z, Z, Z, F, F, P, P, Z, P, Z, P],
    "qasr_lm_head_int8_argmax_f32": [P, P, P, P, P, Z, Z, Z, P, Z, P],
    "qasr_lm_head_int8_argmax_noalloc_f32": [P, P, P, P, P, Z, Z, Z, P],
    "qasr_probe_read": [c_int, c_int, ctypes.c_uint, P, Z, P, Z, Z, Z, Z, P],
    "qasr_head_rms_norm_rope_kv_f32": [P, P, P, P, P, P, P, P, Z, Z, Z, Z, Z, Z, F, P, P, Z, P],
    "qasr_rope_table_fill_f32": [P, P, Z, Z, Z, F, P],
    "qasr_swiglu_multiply_f32": [P, P, Z, Z, P],
    "qasr_swiglu_split_f32": [P, P, P, Z, P],
    "qasr_silu_f32": [P, Z, P],
    "qasr_gelu_tanh_f32": [P, Z, P],
    "qasr_gelu_erf_f32": [P, Z, P],
    "qasr_sinusoidal_pe_f32": [P, Z, Z, P],
    "qasr_pe_add_f32": [P, P, Z, Z, Z, P],
    "qasr_pe_add_layer_norm_f32": [P, P, P, P, P, Z, Z, Z, F, P],
    "qasr_embed_gather_f32": [P, P, P, Z, Z, Z, P],
    "qasr_embed_gather_bf16": [P, P, P, Z, Z, Z, P],
    "qasr_embed_gather_i8": [P, P, P, P, Z, Z, Z, P],
    "qasr_quantize_rows_i8": [P, P, P, Z, Z, P],
    "qasr_linear_nobias_int8_f32": [P, P, P, P, Z, Z, Z, P],
    "qasr_linear_int8_f32": [P, P, P, P, P, Z, Z, Z, P],
    "qasr_linear_nobias_int8_multi_f32": [Z, P, P, P, P, P, Z, Z, P],
    "qasr_qkv_heads_int8_f32": [P, P, P, Z, P, P, P, P, P, P, P, Z, Z, Z, Z, Z, P, P, P, P, Z, Z, F, P],
    "qasr_rms_norm_qkv_heads_int8_f32": [P, P, P, Z, P, P, P, P, P, P, P, P, Z, F, P, Z, Z, Z, Z, Z, P, P, P, P,
                                         Z, Z, F, P],
    "qasr_linear_int8_residual_f32": [P, P, P, P, P, P, P, Z, Z, Z, P],
    "qasr_rms_norm_gate_up_swiglu_multiply_int8_f32": [P, P, P, Z, F, P, P, P, Z, Z, Z, P],
    "qasr_gate_up_swiglu_int8_f32": [P, P, P, P, Z, Z, Z, P],
    "qasr_gate_up_swiglu_multiply_int8_f32": [P, P, P, P, Z, Z, Z, P],
    "qasr_add_rms_norm_linear_nobias_int8_multi_f32": [Z, P, P, P, P, P, P, P, P, Z, F, P],
    "qasr_add_rms_norm_gate_up_swiglu_int8_f32": [P, P, P, P, P, P, P, Z, Z, F, P],
    "qasr_interleave_gate_up_i8": [P, P, P, P, P, P, Z, Z, P],
    "qasr_gate_up_swiglu_w8a8": [P, P, P, P, P, Z, Z, Z, P],
    "qasr_gate_up_swiglu_w8a8_f32in": [P, P, P, P, Z, Z, P],
    "qasr_pack_w8a8_tiles": [P, P, Z, Z, P],
    "qasr_gate_up_swiglu_w8a8_packed": [P, P, P, P, P, Z, Z, Z, P],
    "qasr_linear_w8a8_packed": [P, P, P, P, P, Z, Z, Z, P],
    "qasr_batched_decode_attention_f32": [P, P, P, P, Z, P, Z, Z, Z, Z, F, P, Z, P, P, P, P],
    "qasr_batched_decode_order_i32": [P, P, Z, Z, P],
    "qasr_qkv_heads_w8a8_packed": [P, P, P, Z, P, P, P, P, P, P, P, P, Z, P, Z, Z, Z, Z, Z, F, P],
    # .qint8 files: host-side handle calls (out-parameters are host pointers)
    "qasr_qint8_open": [c_char_p, P],
    "qasr_qint8_close": [P],
    "qasr_qint8_info": [P, P, P],
    "qasr_qint8_find": [P, c_char_p, P],
    "qasr_qint8_tensor": [P, Z, P, P, P, P, P, Z, P, P],
    "qasr_qint8_upload": [P, Z, P, P, P],
    "qasr_qint8_upload_gate_up": [P, c_char_p, c_char_p, Z, Z, P, P, P],
}

# entry points that return a size instead of a status
SIZE_QUERIES = {
    "qasr_causal_attention_workspace_floats": [ctypes.c_size_t] * 3,
    "qasr_batched_decode_attention_workspace_floats": [ctypes.c_size_t] * 4,
    "qasr_lm_head_argmax_workspace_bytes": [ctypes.c_size_t],
}

_LIB = None


def lib() -> ctypes.CDLL:
    """Load the kernel library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise QasrLibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m qwenasr_amd.build` "
                "(there is no CPU fallback for the kernels)")
        so = ctypes.CDLL(str(LIB_PATH))
        so.qasr_version.restype = c_int
        so.qasr_version.argtypes = []
        so.qasr_last_error.restype = c_char_p
        so.qasr_last_error.argtypes = []
        for name in SIZE_QUERIES:
            getattr(so, name).restype = ctypes.c_size_t
            getattr(so, name).argtypes = SIZE_QUERIES[name]
        for name, args in SIGNATURES.items():
            fn = getattr(so, name)
            fn.argtypes = args
            fn.restype = c_int
        _LIB = so
    return _LIB


def call(name: str, *args) -> None:
    """Call entry point ``name``; raise QasrError on a non-zero status."""
    so = lib()
    rc = getattr(so, name)(*args)
    if rc != QASR_OK:
        msg = so.qasr_last_error().decode(errors="replace")
        raise QasrError(name, rc, msg)


def version() -> tuple[int, int, int]:
    v = lib().qasr_version()
    return (v >> 16) & 0xFF, (v >> 8) & 0xFF, v & 0xFF
