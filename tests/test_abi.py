"""C-ABI checks that need no GPU.

* libqasr_hip.so loads and exports every function include/qasr.h declares, and
  the ctypes table in qwenasr_amd/_lib.py covers exactly that set;
* argument validation happens on the host, before any HIP call, and returns
  the documented status codes (the reference panics on bad dimensions; here
  nothing is launched and a message is set);
* zero-sized calls are no-ops that succeed without touching the device.

No call here reaches a kernel launch: every argument set is rejected (or is
empty) before the library talks to the HIP runtime.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from qwenasr_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qasr.h"

FAKE = ctypes.c_void_p(0x10000)  # 64 KiB: aligned, never dereferenced (calls are rejected first)
NULL = ctypes.c_void_p(0)


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(qasr_[a-z0-9_]+)\s*\(", text)) - {"qasr_status"}


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert "qasr_add_rms_norm_f32" in names and "qasr_gate_up_swiglu_w8a8" in names
    assert len(names) >= 25


def test_library_exports_every_declared_symbol():
    so = _lib.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(so, n)]
    assert not missing, f"not exported: {missing}"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r" T (qasr_[a-z0-9_]+)", nm))
    assert declared_functions() <= exported
    # every exported qasr_ symbol is declared (no undocumented entry points)
    assert exported <= declared_functions(), exported - declared_functions()


def test_ctypes_table_matches_header():
    declared = declared_functions() - {"qasr_version", "qasr_last_error"} - set(_lib.SIZE_QUERIES)
    assert set(_lib.SIGNATURES) == declared


def test_static_archive_has_the_same_symbols():
    a = ROOT / "qwenasr_amd" / "libqasr_hip.a"
    assert a.exists(), "static archive not built"
    nm = subprocess.run(["nm", "--defined-only", str(a)], capture_output=True, text=True,
                        check=True).stdout
    assert declared_functions() <= set(re.findall(r" T (qasr_[a-z0-9_]+)", nm))


def test_version():
    assert _lib.version() >= (0, 1, 0)


def rc(name, *args):
    return getattr(_lib.lib(), name)(*args)


def last_error() -> str:
    return _lib.lib().qasr_last_error().decode()


def test_null_pointers_are_invalid_arg():
    assert rc("qasr_rms_norm_f32", NULL, FAKE, FAKE, 4, 64, 1e-6, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "null" in last_error()
    assert rc("qasr_add_rms_norm_f32", FAKE, NULL, FAKE, FAKE, 4, 64, 1e-6, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_layer_norm_f32", FAKE, FAKE, FAKE, NULL, 1, 8, 1e-5, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_pe_add_layer_norm_f32", FAKE, NULL, ctypes.c_void_p(0x100000), FAKE, FAKE, 1, 8, 1,
              1e-5, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_embed_gather_i8", FAKE, FAKE, NULL, FAKE, 1, 16, 10, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_gate_up_swiglu_w8a8", FAKE, FAKE, FAKE, NULL, FAKE, 1, 64, 32, NULL) == _lib.QASR_ERR_INVALID_ARG


def test_zero_sizes_are_noops():
    # no pointers needed, nothing launched
    assert rc("qasr_rms_norm_f32", NULL, NULL, NULL, 0, 1024, 1e-6, NULL) == _lib.QASR_OK
    assert rc("qasr_add_inplace_f32", NULL, NULL, 0, NULL) == _lib.QASR_OK
    assert rc("qasr_swiglu_multiply_f32", NULL, NULL, 0, 3072, NULL) == _lib.QASR_OK
    assert rc("qasr_gelu_erf_f32", NULL, 0, NULL) == _lib.QASR_OK
    assert rc("qasr_embed_gather_f32", NULL, NULL, NULL, 0, 1024, 10, NULL) == _lib.QASR_OK
    assert rc("qasr_gate_up_swiglu_w8a8", NULL, NULL, NULL, NULL, NULL, 0, 2048, 6144, NULL) == _lib.QASR_OK


def test_shape_contracts():
    # RoPE needs an even head_dim
    assert rc("qasr_apply_rope_neox_f32", FAKE, FAKE, FAKE, 2, 4, 127, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "even" in last_error()
    # W8A8 in_dim must be a multiple of 16
    assert rc("qasr_gate_up_swiglu_w8a8", FAKE, FAKE, FAKE, FAKE, FAKE, 1, 100, 32, NULL) == _lib.QASR_ERR_INVALID_ARG
    # the fp32-input matvec supports in_dim 1024..4096 in steps of 1024
    assert rc("qasr_gate_up_swiglu_w8a8_f32in", FAKE, FAKE, FAKE, FAKE, 512, 32, NULL) == _lib.QASR_ERR_UNSUPPORTED
    # misaligned weight pointer
    assert rc("qasr_gate_up_swiglu_w8a8", FAKE, ctypes.c_void_p(0x10001), FAKE, FAKE, FAKE, 1, 64, 32,
              NULL) == _lib.QASR_ERR_INVALID_ARG
    # RoPE table fill: head_dim limit
    assert rc("qasr_rope_table_fill_f32", FAKE, FAKE, 0, 10, 1024, 1e6, NULL) == _lib.QASR_ERR_INVALID_ARG
    # add_rms_norm: out must not alias the residual
    assert rc("qasr_add_rms_norm_f32", FAKE, FAKE, FAKE, FAKE, 1, 64, 1e-6, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "alias" in last_error()
    # overflowing products
    big = (1 << 62)
    assert rc("qasr_rms_norm_f32", FAKE, FAKE, FAKE, big, big, 1e-6, NULL) == _lib.QASR_ERR_INVALID_ARG
    # a RoPE table needs at least one row (out-of-table positions read row 0, then become NaN)
    assert rc("qasr_head_rms_norm_rope_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 1, 16, 8, 128, 0,
              1e-6, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "no rows" in last_error()
    # KV store: rows start_pos..start_pos+seq must fit the cache
    assert rc("qasr_head_rms_norm_rope_kv_f32", FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 60, 8,
              16, 8, 128, 2048, 1e-6, FAKE, FAKE, 64, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "exceed" in last_error()
    # attention: head groups must divide; unsupported head_dim
    assert rc("qasr_causal_attention_f32", FAKE, FAKE, FAKE, FAKE, 1, 4, 6, 4, 128, 0.1, 3,
              NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_causal_attention_f32", FAKE, FAKE, FAKE, FAKE, 1, 4, 16, 8, 96, 0.1, 3,
              NULL) == _lib.QASR_ERR_UNSUPPORTED
    # vocab must be positive
    assert rc("qasr_embed_gather_f32", FAKE, FAKE, FAKE, 1, 16, 0, NULL) == _lib.QASR_ERR_INVALID_ARG


def test_python_mirror_raises_like_a_slice_panic():
    import torch
    from qwenasr_amd import kernels

    # CPU tensors are refused before any C call
    with pytest.raises(TypeError):
        kernels.rms_norm(torch.empty(8), torch.empty(8), torch.empty(8), 1, 8, 1e-6)


def test_qasr_error_carries_status_and_message():
    with pytest.raises(_lib.QasrError) as ei:
        _lib.call("qasr_apply_rope_neox_f32", FAKE, FAKE, FAKE, 2, 4, 127, NULL)
    assert ei.value.code == _lib.QASR_ERR_INVALID_ARG
    assert "even" in ei.value.msg


def test_cpp_mirror_binary_links_the_static_archive():
    from qwenasr_amd import build

    assert build.CPP_TEST_BIN.exists(), "C++ test not built"
    ldd = subprocess.run(["ldd", str(build.CPP_TEST_BIN)], capture_output=True, text=True).stdout
    assert "libqasr_hip.so" not in ldd  # kernels come from libqasr_hip.a
    nm = subprocess.run(["nm", str(build.CPP_TEST_BIN)], capture_output=True, text=True).stdout
    assert " T qasr_rms_norm_f32" in nm


def test_attention_workspace_size_query():
    # seq_q * n_heads * 64 splits * (head_dim + 2)
    assert _lib.lib().qasr_causal_attention_workspace_floats(1, 16, 128) == 16 * 64 * 130
    assert _lib.lib().qasr_causal_attention_workspace_floats(3, 2, 64) == 6 * 64 * 66


def test_batched_attention_workspace_size_query():
    # chunks of 512 keys: 2048 rows -> 4 partials of head_dim + 2 floats per (stream, q head)
    q = _lib.lib().qasr_batched_decode_attention_workspace_floats
    assert q(256, 16, 128, 2048) == 256 * 16 * 4 * 130
    assert q(3, 4, 64, 513) == 3 * 4 * 2 * 66
    assert q(256, 16, 128, 512) == 0  # one chunk: no workspace
    assert q(256, 16, 128, 0) == 0
    assert q(1 << 62, 16, 128, 2048) == 0  # would overflow


def test_lm_head_workspace_size_query():
    # one (value, index) pair of 8 bytes per 4 logits at most
    assert _lib.lib().qasr_lm_head_argmax_workspace_bytes(151936) == 8 * 37984
    assert _lib.lib().qasr_lm_head_argmax_workspace_bytes(5) == 16
    assert _lib.lib().qasr_lm_head_argmax_workspace_bytes(0) == 0


def test_linear_multi_validation():
    so = _lib.lib()
    arr = ctypes.c_void_p * 5
    sz = ctypes.c_size_t * 5
    ptrs = arr(*([FAKE.value] * 5))
    dims = sz(*([16] * 5))
    assert so.qasr_linear_nobias_int8_multi_f32(5, ptrs, ptrs, ptrs, dims, FAKE, 1, 1024, NULL) == \
        _lib.QASR_ERR_INVALID_ARG
    assert "at most 4" in last_error()
    nul = arr(FAKE.value, 0, FAKE.value, FAKE.value, FAKE.value)
    assert so.qasr_linear_nobias_int8_multi_f32(2, nul, ptrs, ptrs, dims, FAKE, 1, 1024, NULL) == \
        _lib.QASR_ERR_INVALID_ARG
    assert so.qasr_linear_nobias_int8_multi_f32(0, None, None, None, None, None, 1, 1024, NULL) == 0


def test_qkv_heads_int8_validation():
    """The prefill q/k/v + heads entry point rejects bad calls before any launch:
    null pointers and rows past the cache or the RoPE table (INVALID_ARG, as the
    unfused head kernel), head_dim other than 128, fewer than 8 tokens and
    in_dim % 64 != 0 (UNSUPPORTED); zero tokens is a no-op."""
    inv, uns = _lib.QASR_ERR_INVALID_ARG, _lib.QASR_ERR_UNSUPPORTED
    F = FAKE
    # (q, k_cache, v_cache, cache_rows, wq, sq, wk, sk, wv, sv, x, seq_len, in_dim, n_heads, n_kv_heads,
    #  head_dim, q_norm_w, k_norm_w, cos, sin, table_rows, start_pos, eps, stream)
    def call(*, q=F, cache_rows=1024, seq=64, in_dim=1024, hd=128, table=1024, start=0, qw=F):
        return rc("qasr_qkv_heads_int8_f32", q, F, F, cache_rows, F, F, F, F, F, F, F, seq, in_dim, 16, 8, hd,
                  qw, F, F, F, table, start, 1e-6, NULL)
    assert call(q=NULL) == inv
    assert call(qw=NULL) == inv
    assert call(start=1000) == inv and "exceed the cache" in last_error()
    assert call(table=1000, start=960) == inv
    assert call(hd=64) == uns
    assert call(seq=7) == uns
    assert call(in_dim=1000) == uns
    assert call(seq=0, q=NULL) == _lib.QASR_OK


def test_prefill_norm_fold_validation():
    """The prefill folds reject bad calls before any launch: null pointers, hg
    without gain, and an ss slice count other than ceil(in_dim / 64)
    (INVALID_ARG); the residual GEMM's shape limits (fewer than 8 tokens,
    in_dim % 64 != 0: UNSUPPORTED); zero tokens is a no-op."""
    inv, uns = _lib.QASR_ERR_INVALID_ARG, _lib.QASR_ERR_UNSUPPORTED
    F = FAKE

    def residual(*, h=F, ss=F, hg=NULL, gain=NULL, seq=64, in_dim=2048, out_dim=1024):
        return rc("qasr_linear_int8_residual_f32", h, ss, hg, gain, F, F, F, seq, in_dim, out_dim, NULL)
    assert residual(h=NULL) == inv
    assert residual(ss=NULL) == inv
    assert residual(hg=F) == inv and "go together" in last_error()
    assert residual(gain=F) == inv
    assert residual(seq=7) == uns and "seq_len >= 8" in last_error()
    assert residual(in_dim=1000) == uns
    assert residual(seq=0, h=NULL) == _lib.QASR_OK

    def gate_up(*, hg=F, ss=F, slices=16, xn=F, seq=64, in_dim=1024):
        return rc("qasr_rms_norm_gate_up_swiglu_multiply_int8_f32", F, hg, ss, slices, 1e-6, xn, F, F, seq,
                  in_dim, 3072, NULL)
    assert gate_up(hg=NULL) == inv
    assert gate_up(ss=NULL) == inv
    assert gate_up(xn=NULL) == inv
    assert gate_up(slices=17) == inv and "ceil(in_dim / 64)" in last_error()
    assert gate_up(seq=0, ss=NULL) == _lib.QASR_OK

    # (q, k_cache, v_cache, cache_rows, wq, sq, wk, sk, wv, sv, hg, ss, ss_slices, norm_eps, x_norm, seq_len,
    #  in_dim, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, cos, sin, table_rows, start_pos, eps, stream)
    def qkv(*, ss=F, slices=16, xn=F, seq=64, hd=128, start=0):
        return rc("qasr_rms_norm_qkv_heads_int8_f32", F, F, F, 1024, F, F, F, F, F, F, F, ss, slices, 1e-6, xn,
                  seq, 1024, 16, 8, hd, F, F, F, F, 1024, start, 1e-6, NULL)
    assert qkv(ss=NULL) == inv
    assert qkv(xn=NULL) == inv
    assert qkv(slices=8) == inv
    assert qkv(start=1000) == inv and "exceed the cache" in last_error()
    assert qkv(hd=64) == uns
    assert qkv(seq=7) == uns
    assert qkv(seq=0, ss=NULL) == _lib.QASR_OK


def test_fused_norm_projection_validation():
    """The fused add + RMSNorm + projection entry points reject, before any
    launch: an h_out that overlaps x or delta (other workgroups still read the
    row), outputs that overlap the row, rows off the one-token vector path,
    misaligned rows, more than 4 matrices and null pointers."""
    so = _lib.lib()
    X, D, G, H, Y, W, S = (ctypes.c_void_p(a) for a in
                           (0x100000, 0x200000, 0x300000, 0x400000, 0x500000, 0x600000, 0x700000))
    arr = ctypes.c_void_p * 3
    sz = ctypes.c_size_t * 3
    ys, ws, ss, dims = arr(Y.value, Y.value + 0x10000, Y.value + 0x20000), arr(W.value, W.value, W.value), \
        arr(S.value, S.value, S.value), sz(2048, 1024, 1024)
    multi = so.qasr_add_rms_norm_linear_nobias_int8_multi_f32
    gu = so.qasr_add_rms_norm_gate_up_swiglu_int8_f32
    inv, uns = _lib.QASR_ERR_INVALID_ARG, _lib.QASR_ERR_UNSUPPORTED
    # h_out aliasing x, or overlapping delta's 8 KiB row
    assert multi(3, ys, ws, ss, dims, X, X, D, G, 2048, 1e-6, NULL) == inv
    assert "overlap" in last_error()
    assert multi(3, ys, ws, ss, dims, ctypes.c_void_p(D.value + 4096), X, D, G, 2048, 1e-6, NULL) == inv
    assert gu(Y, ctypes.c_void_p(X.value + 16), X, D, G, W, S, 2048, 6144, 1e-6, NULL) == inv
    # an output over the row
    assert multi(3, arr(X.value, Y.value, Y.value + 0x10000), ws, ss, dims, H, X, D, G, 2048, 1e-6, NULL) == inv
    assert gu(ctypes.c_void_p(D.value - 64), H, X, D, G, W, S, 2048, 6144, 1e-6, NULL) == inv
    # off the vector path / misaligned
    assert multi(3, ys, ws, ss, dims, H, X, D, G, 1000, 1e-6, NULL) == uns
    assert gu(Y, H, ctypes.c_void_p(X.value + 4), D, G, W, S, 2048, 6144, 1e-6, NULL) == uns
    assert gu(Y, H, X, D, G, W, S, 9216, 6144, 1e-6, NULL) == uns
    # counts and nulls
    arr5 = ctypes.c_void_p * 5
    p5 = arr5(*([Y.value] * 5))
    assert multi(5, p5, p5, p5, (ctypes.c_size_t * 5)(*([16] * 5)), H, X, D, G, 2048, 1e-6, NULL) == inv
    assert multi(3, ys, ws, ss, dims, H, NULL, D, G, 2048, 1e-6, NULL) == inv
    assert gu(NULL, H, X, D, G, W, S, 2048, 6144, 1e-6, NULL) == inv
    assert multi(3, ys, ws, ss, dims, H, X, D, G, 2048, -1.0, NULL) == inv
    # empty calls succeed without touching the device
    assert multi(0, None, None, None, None, NULL, NULL, NULL, NULL, 2048, 1e-6, NULL) == _lib.QASR_OK
    assert gu(Y, H, X, D, G, W, S, 2048, 0, 1e-6, NULL) == _lib.QASR_OK


def test_decode_attention_validation():
    """pos outside the RoPE table or the cache, null pointers and a head count
    that is not a multiple of the kv heads are rejected before any launch."""
    so = _lib.lib()
    f = so.qasr_decode_attention_f32
    P = [ctypes.c_void_p(0x100000 * (i + 1)) for i in range(10)]
    out, q, k, v, qw, kw, cs, sn, kc, vc = P
    inv = _lib.QASR_ERR_INVALID_ARG
    # (..., table_rows, pos, n_heads, n_kv_heads, head_dim, eps, scale, k_cache, v_cache, cache_rows, ws, n, stream)
    assert f(out, q, k, v, qw, kw, cs, sn, 1024, 1024, 16, 8, 128, 1e-6, 0.088, kc, vc, 2048, NULL, 0, NULL) == inv
    assert "inside the RoPE table" in last_error()
    assert f(out, q, k, v, qw, kw, cs, sn, 4096, 2048, 16, 8, 128, 1e-6, 0.088, kc, vc, 2048, NULL, 0, NULL) == inv
    assert f(out, q, k, v, qw, kw, cs, sn, 4096, 10, 16, 5, 128, 1e-6, 0.088, kc, vc, 2048, NULL, 0, NULL) == inv
    assert f(out, NULL, k, v, qw, kw, cs, sn, 4096, 10, 16, 8, 128, 1e-6, 0.088, kc, vc, 2048, NULL, 0, NULL) == inv
    assert f(out, q, k, v, qw, kw, cs, sn, 4096, 10, 0, 8, 128, 1e-6, 0.088, kc, vc, 2048, NULL, 0, NULL) == \
        _lib.QASR_OK


def test_batched_entry_points_validation():
    """The batched decode entry points reject bad shapes, null pointers and a
    too-small workspace before any launch."""
    so = _lib.lib()
    P = [ctypes.c_void_p(0x100000 * (i + 1)) for i in range(12)]
    inv, uns = _lib.QASR_ERR_INVALID_ARG, _lib.QASR_ERR_UNSUPPORTED
    att = so.qasr_batched_decode_attention_f32
    out, q, kc, vc, pos, ws = P[:6]
    # (out, q, k_cache, v_cache, cache_rows, positions, batch, n_heads, n_kv_heads, head_dim, scale, ws, n,
    #  out_q, out_scales, order, stream)
    assert att(out, q, kc, vc, 2048, pos, 4, 16, 5, 128, 0.088, NULL, 0, NULL, NULL, NULL, NULL) == inv  # 16 % 5 != 0
    assert att(out, NULL, kc, vc, 2048, pos, 4, 16, 8, 128, 0.088, NULL, 0, NULL, NULL, NULL, NULL) == inv
    assert att(out, q, kc, vc, 2048, pos, 4, 32, 8, 128, 0.088, NULL, 0, NULL, NULL, NULL, NULL) == uns  # G = 4 at head_dim 128
    assert att(out, q, kc, vc, 2048, pos, 4, 16, 8, 96, 0.088, NULL, 0, NULL, NULL, NULL, NULL) == uns
    need = so.qasr_batched_decode_attention_workspace_floats(4, 16, 128, 2048)
    assert att(out, q, kc, vc, 2048, pos, 4, 16, 8, 128, 0.088, ws, need - 1, NULL, NULL, NULL, NULL) == inv
    assert "workspace" in last_error()
    assert att(out, q, kc, vc, 2048, pos, 0, 16, 8, 128, 0.088, NULL, 0, NULL, NULL, NULL, NULL) == _lib.QASR_OK
    assert att(out, q, kc, vc, 2048, pos, 4, 16, 8, 128, 0.088, NULL, 0, P[6], NULL, NULL, NULL) == inv  # q without scales
    order = so.qasr_batched_decode_order_i32
    assert order(NULL, pos, 4, 2048, NULL) == inv
    assert order(P[6], pos, 65537, 2048, NULL) == inv
    assert order(P[6], pos, 0, 2048, NULL) == _lib.QASR_OK
    lin = so.qasr_linear_w8a8_packed
    y, w, sc, xq, xs = P[6:11]
    # (y, w_packed, scales, xq, x_scales, batch, in_dim, out_dim, stream)
    assert lin(y, w, sc, xq, xs, 4, 1536, 128, NULL) == uns  # in_dim
    assert lin(y, w, sc, xq, xs, 4, 2048, 100, NULL) == uns  # out_dim % 128
    assert lin(y, NULL, sc, xq, xs, 4, 2048, 128, NULL) == inv
    qkv = so.qasr_qkv_heads_w8a8_packed
    cs, sn, qw, kw = P[8:12]
    # (q_out, k_cache, v_cache, cache_rows, w, scales, xq, xs, q_norm_w, k_norm_w, cos, sin, table_rows,
    #  positions, batch, in_dim, n_heads, n_kv_heads, head_dim, eps, stream)
    assert qkv(q, kc, vc, 2048, w, sc, xq, xs, qw, kw, cs, sn, 2048, pos, 4, 2048, 16, 8, 64, 1e-6, NULL) == uns
    assert qkv(q, kc, vc, 2048, w, sc, xq, xs, NULL, kw, cs, sn, 2048, pos, 4, 2048, 16, 8, 128, 1e-6, NULL) == inv


def test_pe_add_layer_norm_validation():
    """out or pe overlapping x, and n_pos = 0, are rejected before any launch."""
    x, other = FAKE, ctypes.c_void_p(0x100000)
    assert rc("qasr_pe_add_layer_norm_f32", x, other, ctypes.c_void_p(0x10000 + 16), other, other, 4, 8,
              1, 1e-5, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "overlap" in last_error()
    assert rc("qasr_pe_add_layer_norm_f32", x, ctypes.c_void_p(0x10000 + 64), other, other, other, 4, 8,
              1, 1e-5, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_pe_add_layer_norm_f32", x, other, ctypes.c_void_p(0x200000), other, other, 4, 8, 0,
              1e-5, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "n_pos" in last_error()


def test_add_layer_norm_validation():
    """Overlapping x, delta and out, and null pointers, are rejected before any launch."""
    x, other = FAKE, ctypes.c_void_p(0x100000)
    assert rc("qasr_add_layer_norm_f32", x, other, other, other, ctypes.c_void_p(0x10000 + 16), 4, 8, 1e-5,
              NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "overlap" in last_error()
    assert rc("qasr_add_layer_norm_f32", x, ctypes.c_void_p(0x10000 + 64), other, other,
              ctypes.c_void_p(0x200000), 4, 8, 1e-5, NULL) == _lib.QASR_ERR_INVALID_ARG
    assert rc("qasr_add_layer_norm_f32", x, NULL, other, other, ctypes.c_void_p(0x200000), 4, 8, 1e-5,
              NULL) == _lib.QASR_ERR_INVALID_ARG
    assert "null" in last_error()


def _kernel_names_in_library() -> set[str]:
    """The device kernels the built library launches, as ``name<args>`` (their
    host-side launch stubs, demangled; namespaces dropped)."""
    nm = subprocess.run(["nm", "-C", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    names = set()
    for line in nm.splitlines():
        m = re.search(r"(?:^|::)([A-Za-z_][A-Za-z0-9_]*_kernel(?:<[^()]*>)?)\(", line.split(" ", 2)[-1])
        if m:
            names.add(re.sub(r"\(qasr::[A-Za-z_:]+\)", "", m.group(1)).replace(" ", ""))
    return names


def test_traffic_profile_names_current_kernels():
    """bench.py's roofline.traffic comes from profiles/traffic.json (measured
    rocprofv3 HBM bytes per launch). Every kernel that file names must still
    exist in the built library with the same template arguments, so a renamed
    or re-parameterised kernel cannot silently inherit a stale measurement."""
    import json

    _lib.lib()
    have = _kernel_names_in_library()
    assert any(n.startswith("rms_norm_vec_kernel<") for n in have), sorted(have)[:10]
    data = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    stale = []
    for workload, entries in data.items():
        if not isinstance(entries, dict):
            continue
        for label, entry in entries.items():
            if not isinstance(entry, dict) or "kernel" not in entry:
                continue
            for kname in entry["kernel"].split(" + "):
                if "whole step" in kname:
                    continue
                if kname.replace(" ", "") not in have:
                    stale.append(f"{workload}/{label}: {kname}")
    assert not stale, f"kernels in profiles/traffic.json not in the library: {stale}"


def test_probe_read_validation():
    """The read-rate probe checks every region it would read against buf_bytes
    (and its other arguments) on the host, before any launch."""
    so = _lib.lib()
    inv = _lib.QASR_ERR_INVALID_ARG
    kb = 1024
    args = dict(mode=2, depth=16, grid=256, buf=FAKE, buf_bytes=256 * 64 * kb, out=FAKE, out_ints=256 * 512,
                per_wg=512 * kb, priv=64 * kb, shift=0)

    def call(**over):
        a = {**args, **over}
        return so.qasr_probe_read(a["mode"], a["depth"], a["grid"], a["buf"], a["buf_bytes"], a["out"],
                                  a["out_ints"], a["per_wg"], a["priv"], a["shift"], NULL)

    assert call(buf=NULL) == inv
    assert call(mode=6) == inv
    assert call(depth=3) == inv
    assert call(grid=0) == inv and call(grid=5000) == inv
    assert call(per_wg=512 * kb + 8192) == inv          # not a multiple of 8192 * depth
    assert call(out_ints=256 * 512 - 1) == inv
    assert call(buf_bytes=256 * 64 * kb - 16) == inv    # the private regions do not fit
    assert call(mode=3, buf_bytes=256 * 512 * kb * 2, shift=2) == inv  # (shift + 1) * grid * per_wg
    assert call(mode=0, buf_bytes=8 * 512 * kb - 1) == inv
    assert call(priv=4096) == inv
    assert b"probe_read" in so.qasr_last_error()
