"""GPU parity: every C-ABI entry point against the CPU oracle on identical seeded
inputs, at the benchmark shapes and at ragged/edge shapes.

Tolerances (the parity contract):
  fp32 outputs          |gpu - oracle| <= 1e-5 + 1e-5 * |oracle|
  erf-GELU              |gpu - float64 closed form| <= 1e-6
  int8 / int32 / copies bit-exact
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.conftest import assert_close

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

RTOL = 1e-5
ATOL = 1e-5
ERF_ATOL = 1e-6


def rng(*tag):
    return np.random.default_rng([20261201, *tag])


def normal(r, shape, scale=1.0, mean=0.0):
    return (mean + scale * r.standard_normal(shape)).astype(np.float32)


def dev_t(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ---------------------------------------------------------------------------
# residual add + RMSNorm / RMSNorm / LayerNorm
# ---------------------------------------------------------------------------
ROW_SHAPES = [(1, 1024), (512, 1024), (256, 2048), (3, 1000), (5, 37), (2, 8192), (2, 9000)]


@pytest.mark.parametrize("seq,hidden", ROW_SHAPES)
def test_add_rms_norm(dev, seq, hidden):
    from qwenasr_amd import kernels as K

    r = rng(1, seq, hidden)
    x = normal(r, seq * hidden)
    d = normal(r, seq * hidden)
    w = normal(r, hidden, 0.1, 1.0)
    xt, dt, wt = dev_t(x, dev), dev_t(d, dev), dev_t(w, dev)
    out = torch.empty_like(xt)
    K.add_rms_norm(xt, dt, wt, out, seq, hidden, 1e-6)
    x_ref, y_ref = oracle.add_rms_norm(x, d, w, seq, hidden, 1e-6)
    np.testing.assert_array_equal(host(xt), x_ref)  # the residual is an f32 add: exact
    assert_close(host(out), y_ref, RTOL, ATOL, f"add_rms_norm {seq}x{hidden}")


@pytest.mark.parametrize("seq,hidden", ROW_SHAPES)
def test_rms_norm(dev, seq, hidden):
    from qwenasr_amd import kernels as K

    r = rng(2, seq, hidden)
    x = normal(r, seq * hidden)
    w = normal(r, hidden, 0.1, 1.0)
    xt, wt = dev_t(x, dev), dev_t(w, dev)
    out = torch.empty_like(xt)
    K.rms_norm(out, xt, wt, seq, hidden, 1e-6)
    assert_close(host(out), oracle.rms_norm(x, w, seq, hidden, 1e-6), RTOL, ATOL, "rms_norm")
    # in place (out aliases x)
    K.rms_norm(xt, xt, wt, seq, hidden, 1e-6)
    assert_close(host(xt), oracle.rms_norm(x, w, seq, hidden, 1e-6), RTOL, ATOL, "rms_norm inplace")


@pytest.mark.parametrize("seq,hidden", [(256, 2048), (1, 1024), (3, 1000), (5, 37)])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rms_norm_quant(dev, seq, hidden, with_delta):
    """x updated exactly; y within tolerance of the oracle; q/scales bit-exact to
    quantize_rows_i8 applied to the kernel's own y (and within 1 of the oracle's)."""
    from qwenasr_amd import kernels as K

    r = rng(24, seq, hidden)
    x = normal(r, seq * hidden)
    d = normal(r, seq * hidden)
    w = normal(r, hidden, 0.1, 1.0)
    xt, dt, wt = dev_t(x, dev), dev_t(d, dev), dev_t(w, dev)
    out = torch.empty_like(xt)
    q = torch.empty(seq * hidden, dtype=torch.int8, device=dev)
    qs = torch.empty(seq, dtype=torch.float32, device=dev)
    K.add_rms_norm_quant(xt, dt if with_delta else None, wt, out, q, qs, seq, hidden, 1e-6)
    if with_delta:
        x_ref, y_ref = oracle.add_rms_norm(x, d, w, seq, hidden, 1e-6)
    else:
        x_ref, y_ref = x, oracle.rms_norm(x, w, seq, hidden, 1e-6)
    np.testing.assert_array_equal(host(xt), x_ref)
    y = host(out)
    assert_close(y, y_ref, RTOL, ATOL, "add_rms_norm_quant y")
    q_self, s_self = oracle.quantize_f32_to_int8(y, seq, hidden)
    np.testing.assert_array_equal(host(q), q_self)
    np.testing.assert_array_equal(host(qs), s_self)
    q_ref, _ = oracle.quantize_f32_to_int8(y_ref, seq, hidden)
    assert np.abs(host(q).astype(np.int32) - q_ref.astype(np.int32)).max() <= 1
    # without the fp32 output the int8 result is the same
    xt2 = dev_t(x, dev)
    q2 = torch.empty_like(q)
    qs2 = torch.empty_like(qs)
    K.add_rms_norm_quant(xt2, dt if with_delta else None, wt, None, q2, qs2, seq, hidden, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(q2, q) and torch.equal(qs2, qs)


def test_rms_norm_misaligned_rows_take_scalar_path(dev):
    from qwenasr_amd import kernels as K

    r = rng(3)
    seq, hidden = 4, 64
    x = normal(r, seq * hidden + 1)
    w = normal(r, hidden, 0.1, 1.0)
    xt = dev_t(x, dev)[1:]  # 4-byte offset: not 16-byte aligned
    out = torch.empty(seq * hidden + 1, dtype=torch.float32, device=dev)[1:]
    K.rms_norm(out, xt, dev_t(w, dev), seq, hidden, 1e-6)
    assert_close(host(out), oracle.rms_norm(x[1:], w, seq, hidden, 1e-6), RTOL, ATOL, "misaligned")


def test_rms_norm_reference_kat(dev, golden):
    # tests/kernels.rs:60-72 on the GPU: unit gain -> RMS ~ 1
    from qwenasr_amd import kernels as K

    x = dev_t(golden["rms_kat_x"], dev)
    out = torch.empty_like(x)
    K.rms_norm(out, x, torch.ones(128, device=dev), 1, 128, 1e-6)
    y = host(out)
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 0.01
    assert_close(y, golden["rms_kat_y64"], RTOL, ATOL, "kat")


@pytest.mark.parametrize("seq,hidden", [(3000, 896), (7, 1024), (4, 45), (2, 8)])
def test_layer_norm(dev, seq, hidden):
    from qwenasr_amd import kernels as K

    r = rng(4, seq, hidden)
    x = normal(r, seq * hidden)
    w = normal(r, hidden, 0.1, 1.0)
    b = normal(r, hidden, 0.02)
    xt = dev_t(x, dev)
    out = torch.empty_like(xt)
    K.layer_norm(out, xt, dev_t(w, dev), dev_t(b, dev), seq, hidden, 1e-5)
    assert_close(host(out), oracle.layer_norm(x, w, b, seq, hidden, 1e-5), RTOL, ATOL, "layer_norm")


def test_layer_norm_reference_kat(dev, golden):
    from qwenasr_amd import kernels as K

    x = dev_t(golden["ln_kat_x"], dev)
    out = torch.empty_like(x)
    K.layer_norm(out, x, torch.ones(128, device=dev), torch.zeros(128, device=dev), 1, 128, 1e-5)
    y = host(out)
    assert abs(float(np.mean(y))) < 0.01 and abs(float(np.var(y.astype(np.float64))) - 1) < 0.02


# ---------------------------------------------------------------------------
# q/k head RMSNorm + RoPE
# ---------------------------------------------------------------------------
def test_rope_table_matches_oracle(dev):
    from qwenasr_amd import kernels as K

    rc = K.RopeCache(dev)
    rc.ensure(1500, 128, 1e6)  # grows 1024 -> 2048
    assert rc.cap == 2048
    cos, sin = oracle.rope_table(2048, 128, 1e6)
    assert_close(host(rc.cos), cos, 0, 2.4e-7, "cos table")
    assert_close(host(rc.sin), sin, 0, 2.4e-7, "sin table")
    rc.ensure(3000, 128, 1e6)  # second growth keeps the first rows and fills the rest
    assert rc.cap == 4096
    cos4, _ = oracle.rope_table(4096, 128, 1e6)
    assert_close(host(rc.cos), cos4, 0, 2.4e-7, "cos table grown")


HEAD_CASES = [
    # name, seq, n_heads, n_kv_heads, head_dim, position range
    ("c1_decode", 1, 16, 8, 128, 512),
    ("c2_prefill", 512, 16, 8, 128, None),
    ("c5_streams", 256, 16, 8, 128, 2048),
    ("hd64", 9, 4, 2, 64, 100),
    ("hd96_scalar", 5, 3, 1, 96, 50),
]


@pytest.mark.parametrize("name,seq,nq,nk,hd,prange", HEAD_CASES)
def test_head_rms_norm_rope(dev, name, seq, nq, nk, hd, prange):
    from qwenasr_amd import kernels as K

    r = rng(5, seq, nq, hd)
    q = normal(r, seq * nq * hd)
    k = normal(r, seq * nk * hd)
    qw = normal(r, hd, 0.1, 1.0)
    kw = normal(r, hd, 0.1, 1.0)
    pos = None if prange is None else r.integers(0, prange, seq).astype(np.int32)
    n_rows = 2048
    rc = K.RopeCache(dev)
    rc.ensure(n_rows, hd, 1e6)
    cos, sin = oracle.rope_table(rc.cap, hd, 1e6)
    qt, kt = dev_t(q, dev), dev_t(k, dev)
    K.head_rms_norm_rope(qt, kt, dev_t(qw, dev), dev_t(kw, dev), rc.cos, rc.sin,
                         None if pos is None else dev_t(pos, dev), seq, nq, nk, hd, 1e-6)
    q_ref, k_ref = oracle.head_rms_norm_rope(q, k, qw, kw, cos, sin, pos, seq, nq, nk, hd, 1e-6)
    assert_close(host(qt), q_ref, RTOL, ATOL, f"{name} q")
    assert_close(host(kt), k_ref, RTOL, ATOL, f"{name} k")


def test_head_rope_out_of_table_position_is_nan_row(dev):
    from qwenasr_amd import kernels as K

    r = rng(6)
    seq, nq, nk, hd = 3, 2, 1, 128
    q = normal(r, seq * nq * hd)
    k = normal(r, seq * nk * hd)
    rc = K.RopeCache(dev)
    rc.ensure(16, hd, 1e6)
    pos = np.array([3, 5000, 0], np.int32)  # row 1 is past the 1024-row table
    qt, kt = dev_t(q, dev), dev_t(k, dev)
    ones = torch.ones(hd, device=dev)
    K.head_rms_norm_rope(qt, kt, ones, ones, rc.cos, rc.sin, dev_t(pos, dev), seq, nq, nk, hd, 1e-6)
    qh, kh = host(qt).reshape(seq, -1), host(kt).reshape(seq, -1)
    assert np.isnan(qh[1]).all() and np.isnan(kh[1]).all()
    assert np.isfinite(qh[[0, 2]]).all() and np.isfinite(kh[[0, 2]]).all()


def kv_reference(q, k, v, qw, kw, cos, sin, pos, seq, nq, nk, hd, eps):
    """The reference's layer step (decoder.rs:543-550 / 888-895): per-head
    RMSNorm of q and k, NeoX RoPE with the table rows of each row's position,
    then the k/v rows copied into the cache. Returns q and the k/v rows."""
    qn = oracle.rms_norm_per_head(q, qw, seq, nq, hd, eps)
    kn = oracle.rms_norm_per_head(k, kw, seq, nk, hd, eps)
    c = cos.reshape(-1, hd)[pos].ravel()
    s = sin.reshape(-1, hd)[pos].ravel()
    qr = oracle.apply_rope_neox(qn, c, s, seq, nq, hd)
    kr = oracle.apply_rope_neox(kn, c, s, seq, nk, hd)
    return qr, kr.reshape(seq, nk * hd), v.reshape(seq, nk * hd)


@pytest.mark.parametrize("seq,start,nq,nk,hd,cache_rows", [
    (7, 5, 16, 8, 128, 64),       # decode-ish: rows appended after 5 cached
    (512, 0, 16, 8, 128, 1024),   # 0.6B prefill into a fresh layer block
    (3, 61, 14, 2, 64, 64),       # last rows of the cache, head_dim 64
])
def test_head_rms_norm_rope_kv_single_sequence(dev, seq, start, nq, nk, hd, cache_rows):
    from qwenasr_amd import kernels as K

    r = rng(8, seq, start, hd)
    q, k, v = normal(r, seq * nq * hd), normal(r, seq * nk * hd), normal(r, seq * nk * hd)
    qw, kw = normal(r, hd, 0.1, 1.0), normal(r, hd, 0.1, 1.0)
    rope = K.RopeCache(dev)
    rope.ensure(start + seq, hd, 1e6)
    cos, sin = oracle.rope_table(rope.cap, hd, 1e6)
    kv_dim = nk * hd
    kc = torch.full((cache_rows * kv_dim,), 7.0, device=dev)
    vc = torch.full((cache_rows * kv_dim,), 7.0, device=dev)
    qt = dev_t(q, dev)
    kt, vt = dev_t(k, dev), dev_t(v, dev)
    K.head_rms_norm_rope_kv(qt, kt, vt, dev_t(qw, dev), dev_t(kw, dev), rope, None, start, seq,
                            nq, nk, hd, 1e-6, kc, vc, cache_rows)
    pos = np.arange(start, start + seq)
    q_ref, k_rows, v_rows = kv_reference(q, k, v, qw, kw, cos, sin, pos, seq, nq, nk, hd, 1e-6)
    assert_close(host(qt), q_ref, RTOL, ATOL, "q")
    kh, vh = host(kc).reshape(cache_rows, kv_dim), host(vc).reshape(cache_rows, kv_dim)
    assert_close(kh[start:start + seq], k_rows, RTOL, ATOL, "k cache rows")
    np.testing.assert_array_equal(vh[start:start + seq], v_rows)       # v is a copy
    others = np.r_[0:start, start + seq:cache_rows]
    assert (kh[others] == 7.0).all() and (vh[others] == 7.0).all()     # nothing else written
    np.testing.assert_array_equal(host(kt), k)                          # k, v are read only
    # same arithmetic as the fused norm+rope entry point, bit for bit
    q2, k2 = dev_t(q, dev), dev_t(k, dev)
    pos_t = dev_t(pos.astype(np.int32), dev)
    K.head_rms_norm_rope(q2, k2, dev_t(qw, dev), dev_t(kw, dev), rope.cos, rope.sin, pos_t, seq,
                         nq, nk, hd, 1e-6)
    np.testing.assert_array_equal(host(qt), host(q2))
    np.testing.assert_array_equal(kh[start:start + seq], host(k2).reshape(seq, kv_dim))


@pytest.mark.parametrize("seq,H,start,cache_rows,exact,nq,nk", [
    (512, 1024, 0, 1024, True, 16, 8),    # 0.6B prefill chunk: the producer/consumer tile, 256 workgroups
    (500, 1024, 3, 1024, True, 16, 8),    # ragged last token tile, the same kernel
    (512, 1152, 0, 1024, True, 16, 8),    # K not a multiple of 4 chunks: the double-buffered kernel
    (1000, 1024, 24, 1536, True, 16, 8),  # 512 workgroups: the single-buffered tile
    (100, 2048, 37, 512, False, 16, 8),   # ragged token tile (the plain launch takes the split-K tile)
    (64, 1088, 5, 128, False, 16, 8),     # in_dim % 128 = 64: single-buffered
    (40, 1024, 88, 128, False, 16, 8),    # the chunk ends at the last cache row
    (200, 2048, 11, 256, False, 32, 4),   # 8 q heads per kv head
    (72, 1024, 0, 96, False, 8, 8),       # one q head per kv head
])
def test_qkv_heads_int8_equals_unfused(dev, seq, H, start, cache_rows, exact, nq, nk):
    """The prefill q/k/v GEMM with the heads in its epilogue equals
    linear_nobias_int8_multi + head_rms_norm_rope_kv (decoder.rs:795-810):
    bit for bit where the plain launch uses the same LDS-staged 128-row tile
    (the dequantized products and head_norm_rope are shared), else within the
    fp32 tolerance (another k order in the plain GEMM); the oracle composition
    checks the small cases. Cache rows outside the chunk keep their contents;
    a chunk past the cache or the RoPE table is rejected before any launch."""
    from qwenasr_amd import kernels as K

    hd, eps = 128, 1e-6
    kv = nk * hd
    r = rng(41, seq, H, start, nq)
    x = normal(r, seq * H)
    mats = [make_qweight(r, n, H) for n in (nq * hd, kv, kv)]
    ws = [K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), n, H) for (wq, sc), n in zip(mats, (nq * hd, kv, kv))]
    qw, kw = normal(r, hd, 0.1, 1.0), normal(r, hd, 0.1, 1.0)
    rope = K.RopeCache(dev)
    rope.ensure(start + seq, hd, 1e6)
    xt, qwt, kwt = dev_t(x, dev), dev_t(qw, dev), dev_t(kw, dev)

    q1 = torch.full((seq * nq * hd,), 7.0, device=dev)
    kc1 = torch.full((cache_rows * kv,), 7.0, device=dev)
    vc1 = torch.full((cache_rows * kv,), 7.0, device=dev)
    K.qkv_heads_int8(q1, kc1, vc1, cache_rows, *ws, xt, seq, H, nq, nk, hd, qwt, kwt, rope, start, eps)

    q2 = torch.empty(seq * nq * hd, device=dev)
    k2, v2 = torch.empty(seq * kv, device=dev), torch.empty(seq * kv, device=dev)
    kc2 = torch.full((cache_rows * kv,), 7.0, device=dev)
    vc2 = torch.full((cache_rows * kv,), 7.0, device=dev)
    K.linear_nobias_int8_multi([q2, k2, v2], ws, xt, seq, H)
    K.head_rms_norm_rope_kv(q2, k2, v2, qwt, kwt, rope, None, start, seq, nq, nk, hd, eps, kc2, vc2, cache_rows)
    got = [host(t) for t in (q1, kc1, vc1)]
    ref = [host(t) for t in (q2, kc2, vc2)]
    for g, f, what in zip(got, ref, ("q", "k cache", "v cache")):
        if exact:
            np.testing.assert_array_equal(g, f, err_msg=what)
        else:
            assert_close(g, f, RTOL, ATOL, what)
    live = seq
    kh = got[1].reshape(cache_rows, kv)
    others = np.r_[0:start, start + live:cache_rows]
    assert (kh[others] == 7.0).all() and (got[2].reshape(cache_rows, kv)[others] == 7.0).all()
    assert not np.isnan(got[0]).any()
    with pytest.raises(K.QasrError, match="exceed the cache"):
        K.qkv_heads_int8(q1, kc1, vc1, cache_rows, *ws, xt, seq, H, nq, nk, hd, qwt, kwt, rope,
                         cache_rows - seq + 1, eps)
    if seq <= 128:
        pq, pk, pv = (oracle.linear_nobias_int8(x, wq, sc, seq, H, n)
                      for (wq, sc), n in zip(mats, (nq * hd, kv, kv)))
        cos, sin = oracle.rope_table(rope.cap, hd, 1e6)
        pos = np.minimum(np.arange(start, start + seq), rope.cap - 1)
        q_ref, k_rows, v_rows = kv_reference(pq, pk, pv, qw, kw, cos, sin, pos, seq, nq, nk, hd, eps)
        assert_close(got[0].reshape(seq, -1)[:live], q_ref.reshape(seq, -1)[:live], RTOL, ATOL, "q vs oracle")
        assert_close(kh[start:start + live], k_rows[:live], RTOL, ATOL, "k rows vs oracle")
        assert_close(got[2].reshape(cache_rows, kv)[start:start + live], v_rows[:live], RTOL, ATOL,
                     "v rows vs oracle")


def slice_sums_of_squares(h, seq, hidden):
    """Per token, the float64 sum of squares of each 64-column slice of h."""
    a = h.reshape(seq, hidden).astype(np.float64) ** 2
    n = (hidden + 63) // 64
    return np.stack([a[:, 64 * s:64 * s + 64].sum(axis=1) for s in range(n)], axis=1)


@pytest.mark.parametrize("seq,in_dim,out_dim,exact", [
    (512, 2048, 1024, True),   # 0.6B o at 512 tokens: the split-K 64 x 32 tile, as the plain launch
    (512, 3072, 1024, True),   # 0.6B down
    (100, 2048, 2048, False),  # ragged token tile (the plain launch takes 32 x 32 tiles)
    (37, 1088, 1000, False),   # in_dim % 128 = 64; the last 64-row slice holds 40 rows
])
def test_linear_int8_residual(dev, seq, in_dim, out_dim, exact):
    """The prefill's o / down projection with its residual add folded in
    (decoder.rs:821-822, 837-838): h equals h + linear_nobias_int8 (fp32 add,
    the reference's add_inplace) bit for bit where the plain launch takes the
    same split-K tile, else within the fp32 tolerance; the sums of squares of
    the updated 64-row slices match float64 sums to 2e-5 (fp32 sums of 64
    terms); hg is the updated h times the gain, bit for bit."""
    from qwenasr_amd import kernels as K

    r = rng(43, seq, in_dim, out_dim)
    x = normal(r, seq * in_dim)
    wq, sc = make_qweight(r, out_dim, in_dim)
    h0 = normal(r, seq * out_dim)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), out_dim, in_dim)
    xt, ht = dev_t(x, dev), dev_t(h0, dev)
    ns = K.norm_slices(out_dim)
    ss = torch.full((seq * ns,), 7.0, device=dev)
    gain = normal(r, out_dim, 0.1, 1.0)
    hg = torch.full((seq * out_dim,), 7.0, device=dev)
    K.linear_int8_residual(ht, ss, xt, w, seq, in_dim, out_dim, hg, dev_t(gain, dev))
    y = torch.empty(seq * out_dim, device=dev)
    K.linear_nobias_int8(y, xt, w.data, w.scales, seq, in_dim, out_dim)
    got, ref = host(ht), h0 + host(y)
    if exact:
        np.testing.assert_array_equal(got, ref)
    else:
        assert_close(got, ref, RTOL, ATOL, "h")
    np.testing.assert_allclose(host(ss).reshape(seq, ns), slice_sums_of_squares(got, seq, out_dim), rtol=2e-5)
    np.testing.assert_array_equal(host(hg).reshape(seq, out_dim), got.reshape(seq, out_dim) * gain)
    h2 = dev_t(h0, dev)
    K.linear_int8_residual(h2, ss, xt, w, seq, in_dim, out_dim)  # without hg
    np.testing.assert_array_equal(host(h2), got)
    if seq <= 128:
        y_ref = oracle.linear_nobias_int8(x, wq, sc, seq, in_dim, out_dim)
        assert_close(got, h0 + y_ref, RTOL, ATOL, "h vs oracle")
    with pytest.raises(K.QasrError, match="seq_len >= 8"):
        K.linear_int8_residual(ht, ss, xt, w, 7, in_dim, out_dim)


@pytest.mark.parametrize("seq,H,I,folded", [
    (512, 1024, 3072, True),    # 0.6B at 512 tokens: the producer/consumer 192-row tile
    (500, 1024, 3072, True),    # ragged last token tile, the same kernel
    (1024, 1024, 3072, True),   # the single-buffered 128-row tile
    (1024, 2048, 6144, True),   # the 256-row tile
    (37, 1024, 3072, False),    # too few tiles for the LDS-staged kernels: x_norm = hg * rinv + the plain launch
    (512, 2112, 3072, False),   # 33 slices (not a multiple of 4): the same fallback
])
def test_rms_norm_gate_up_swiglu_multiply_int8(dev, seq, H, I, folded):
    """The prefill post-attention RMSNorm folded into the gate/up GEMM + SwiGLU
    (decoder.rs:826-833): the GEMM reads hg = h * gain and multiplies each
    token's outputs by its 1 / rms from per-slice sums of squares; within the
    fp32 tolerance of rms_norm + gate_up_swiglu_multiply_int8 (1 / rms is
    factored out of the dot products and its sum added in another order), on
    the folded kernels and on the fallback (x_norm = hg * rinv, then the plain
    launch)."""
    from qwenasr_amd import kernels as K

    eps = 1e-6
    r = rng(47, seq, H, I)
    h = normal(r, seq * H)
    g = normal(r, H, 0.1, 1.0)
    wq, sc = make_qweight(r, 2 * I, H)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), 2 * I, H)
    ss = slice_sums_of_squares(h, seq, H).astype(np.float32)
    ht, gt = dev_t(h, dev), dev_t(g, dev)
    hg = dev_t((h.reshape(seq, H) * g).ravel(), dev)
    out = torch.full((seq * I,), 7.0, device=dev)
    xn = torch.full((seq * H,), 7.0, device=dev)
    K.rms_norm_gate_up_swiglu_multiply_int8(out, hg, dev_t(ss.ravel(), dev), eps, xn, w, seq, H, I)
    xn2 = torch.empty(seq * H, device=dev)
    ref = torch.empty(seq * I, device=dev)
    K.rms_norm(xn2, ht, gt, seq, H, eps)
    K.gate_up_swiglu_multiply_int8(ref, xn2, w, seq, H, I)
    assert_close(host(out), host(ref), RTOL, ATOL, "gate/up + SwiGLU")
    if folded:
        assert (host(xn) == 7.0).all()  # not used
    else:
        assert_close(host(xn), host(xn2), RTOL, ATOL, "x_norm")


@pytest.mark.parametrize("seq,H,start,cache_rows", [
    (512, 1024, 0, 1024),    # 0.6B prefill chunk: the producer/consumer tile
    (500, 1024, 7, 1024),    # ragged last token tile, the same kernel
    (1000, 1024, 24, 1536),  # the single-buffered tile
    (100, 2048, 37, 512),    # ragged token tile
    (200, 2112, 5, 256),     # 33 slices: x_norm = hg * rinv, then the plain launch
])
def test_rms_norm_qkv_heads_int8(dev, seq, H, start, cache_rows):
    """The prefill layer-input RMSNorm folded into the q/k/v + heads GEMM
    (decoder.rs:789-810), reading hg = h * gain with each token's 1 / rms from
    per-slice sums of squares: within the fp32 tolerance of rms_norm followed
    by qkv_heads_int8 (q, and the chunk's k/v cache rows); other cache rows
    keep their contents."""
    from qwenasr_amd import kernels as K

    nq, nk, hd, eps = 16, 8, 128, 1e-6
    kv = nk * hd
    r = rng(53, seq, H, start)
    h = normal(r, seq * H)
    g = normal(r, H, 0.1, 1.0)
    mats = [make_qweight(r, n, H) for n in (nq * hd, kv, kv)]
    ws = [K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), n, H) for (wq, sc), n in zip(mats, (nq * hd, kv, kv))]
    qw, kw = normal(r, hd, 0.1, 1.0), normal(r, hd, 0.1, 1.0)
    rope = K.RopeCache(dev)
    rope.ensure(start + seq, hd, 1e6)
    ht, gt, qwt, kwt = dev_t(h, dev), dev_t(g, dev), dev_t(qw, dev), dev_t(kw, dev)
    ss = dev_t(slice_sums_of_squares(h, seq, H).astype(np.float32).ravel(), dev)
    hg = dev_t((h.reshape(seq, H) * g).ravel(), dev)
    scratch = torch.full((seq * H,), 7.0, device=dev)

    q1 = torch.full((seq * nq * hd,), 7.0, device=dev)
    kc1 = torch.full((cache_rows * kv,), 7.0, device=dev)
    vc1 = torch.full((cache_rows * kv,), 7.0, device=dev)
    K.rms_norm_qkv_heads_int8(q1, kc1, vc1, cache_rows, *ws, hg, ss, eps, scratch, seq, H, nq, nk, hd, qwt, kwt,
                              rope, start, eps)
    xn = torch.empty(seq * H, device=dev)
    K.rms_norm(xn, ht, gt, seq, H, eps)
    q2 = torch.full((seq * nq * hd,), 7.0, device=dev)
    kc2 = torch.full((cache_rows * kv,), 7.0, device=dev)
    vc2 = torch.full((cache_rows * kv,), 7.0, device=dev)
    K.qkv_heads_int8(q2, kc2, vc2, cache_rows, *ws, xn, seq, H, nq, nk, hd, qwt, kwt, rope, start, eps)
    for a, b, what in ((q1, q2, "q"), (kc1, kc2, "k cache"), (vc1, vc2, "v cache")):
        assert_close(host(a), host(b), RTOL, ATOL, what)
    others = np.r_[0:start, start + seq:cache_rows]
    assert (host(kc1).reshape(cache_rows, kv)[others] == 7.0).all()
    if H // 64 <= 32 and (H // 64) % 4 == 0:
        assert (host(scratch) == 7.0).all()  # the folded kernels do not need x_norm
    else:
        assert_close(host(scratch), host(xn), RTOL, ATOL, "x_norm (fallback)")


def test_head_rms_norm_rope_kv_per_stream(dev):
    """Batched decode: row s is stream s at its own position, each stream with
    its own [cache_rows, kv_dim] block; a position past the cache leaves that
    stream's cache untouched and its q row NaN."""
    from qwenasr_amd import kernels as K

    B, nq, nk, hd, cache_rows = 6, 16, 8, 128, 48
    r = rng(9)
    q, k, v = normal(r, B * nq * hd), normal(r, B * nk * hd), normal(r, B * nk * hd)
    qw, kw = normal(r, hd, 0.1, 1.0), normal(r, hd, 0.1, 1.0)
    pos = r.integers(0, cache_rows, B).astype(np.int32)
    pos[4] = cache_rows  # past the end of stream 4's cache
    rope = K.RopeCache(dev)
    rope.ensure(cache_rows + 1, hd, 1e6)
    cos, sin = oracle.rope_table(rope.cap, hd, 1e6)
    kv_dim = nk * hd
    kc = torch.full((B * cache_rows * kv_dim,), -3.0, device=dev)
    vc = torch.full((B * cache_rows * kv_dim,), -3.0, device=dev)
    qt = dev_t(q, dev)
    K.head_rms_norm_rope_kv(qt, dev_t(k, dev), dev_t(v, dev), dev_t(qw, dev), dev_t(kw, dev), rope,
                            dev_t(pos, dev), 0, B, nq, nk, hd, 1e-6, kc, vc, cache_rows)
    ok = pos < cache_rows
    q_ref, k_rows, v_rows = kv_reference(q, k, v, qw, kw, cos, sin, np.minimum(pos, cache_rows - 1),
                                         B, nq, nk, hd, 1e-6)
    qh = host(qt).reshape(B, nq * hd)
    assert_close(qh[ok], q_ref.reshape(B, -1)[ok], RTOL, ATOL, "q")
    assert np.isnan(qh[~ok]).all()
    kh = host(kc).reshape(B, cache_rows, kv_dim)
    vh = host(vc).reshape(B, cache_rows, kv_dim)
    for b in range(B):
        written = np.zeros(cache_rows, bool)
        if ok[b]:
            written[pos[b]] = True
            assert_close(kh[b, pos[b]], k_rows[b], RTOL, ATOL, f"k stream {b}")
            np.testing.assert_array_equal(vh[b, pos[b]], v_rows[b])
        assert (kh[b][~written] == -3.0).all() and (vh[b][~written] == -3.0).all()


def test_kv_cache_grow_keeps_rows(dev):
    """KvCache.grow doubles max_seq and keeps each layer's first len rows
    (decoder.rs:151-176)."""
    from qwenasr_amd import kernels as K

    cache = K.KvCache(3, 4, 16, dev)
    cache.k.copy_(torch.arange(cache.k.numel(), dtype=torch.float32, device=dev))
    before = [host(cache.k_layer_block(l))[:2 * 16].copy() for l in range(3)]
    cache.len = 2
    cache.grow(9)
    assert cache.max_seq == 16
    for l in range(3):
        np.testing.assert_array_equal(host(cache.k_layer(l)), before[l])
        assert (host(cache.k_layer_block(l))[2 * 16:] == 0).all()


@pytest.mark.parametrize("seq,nh,hd", [(512, 16, 128), (3, 5, 64), (2, 3, 30)])
def test_rms_norm_per_head_and_apply_rope(dev, seq, nh, hd):
    from qwenasr_amd import kernels as K

    r = rng(7, seq, nh, hd)
    x = normal(r, seq * nh * hd)
    w = normal(r, hd, 0.1, 1.0)
    xt = dev_t(x, dev)
    K.rms_norm_per_head(xt, dev_t(w, dev), seq, nh, hd, 1e-6)
    xn = oracle.rms_norm_per_head(x, w, seq, nh, hd, 1e-6)
    assert_close(host(xt), xn, RTOL, ATOL, "rms_norm_per_head")
    cos, sin = oracle.rope_table(seq + 7, hd, 1e6)
    c = cos[7 * hd:]
    s = sin[7 * hd:]  # rows 7..: a cos_range(start=7, len=seq) slice
    xt2 = dev_t(xn, dev)
    K.apply_rope_neox(xt2, dev_t(c, dev), dev_t(s, dev), seq, nh, hd)
    assert_close(host(xt2), oracle.apply_rope_neox(xn, c, s, seq, nh, hd), RTOL, ATOL, "rope")


# ---------------------------------------------------------------------------
# SwiGLU / SiLU / GELU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("seq,inter", [(512, 3072), (1, 3072), (3, 21), (2, 3076), (4, 6144)])
def test_swiglu_multiply(dev, seq, inter):
    from qwenasr_amd import kernels as K

    r = rng(8, seq, inter)
    gu = normal(r, seq * 2 * inter)
    out = torch.empty(seq * inter, dtype=torch.float32, device=dev)
    K.swiglu_multiply(out, dev_t(gu, dev), seq, inter)
    assert_close(host(out), oracle.swiglu_multiply(gu, seq, inter), RTOL, ATOL, "swiglu_multiply")


@pytest.mark.parametrize("n", [3072, 6144, 1, 1027])
def test_swiglu_split_and_silu(dev, n):
    from qwenasr_amd import kernels as K

    r = rng(9, n)
    g, u = normal(r, n), normal(r, n)
    out = torch.empty(n, dtype=torch.float32, device=dev)
    K.swiglu_split(out, dev_t(g, dev), dev_t(u, dev), n)
    assert_close(host(out), oracle.swiglu_split(g, u), RTOL, ATOL, "swiglu_split")
    gt = dev_t(g, dev)
    K.swiglu_multiply_inplace(gt, dev_t(u, dev))
    assert_close(host(gt), oracle.swiglu_split(g, u), RTOL, ATOL, "swiglu inplace")
    xt = dev_t(g, dev)
    K.silu(xt, n)
    assert_close(host(xt), oracle.silu(g), RTOL, ATOL, "silu")


def test_silu_reference_kat(dev):
    # tests/kernels.rs:115-124
    from qwenasr_amd import kernels as K

    x = np.array([0.0, 1.0, -1.0, 5.0], np.float32)
    xt = dev_t(x, dev)
    K.silu(xt, 4)
    exp = x.astype(np.float64) / (1 + np.exp(-x.astype(np.float64)))
    assert np.abs(host(xt) - exp).max() < 1e-5


@pytest.mark.parametrize("n", [3000 * 3584, 1003, 8, 5])
def test_gelu_erf_within_1e6_of_closed_form(dev, n):
    from qwenasr_amd import kernels as K

    r = rng(10, n)
    x = normal(r, n)
    xt = dev_t(x, dev)
    K.gelu_erf(xt, n)
    assert_close(host(xt), oracle.gelu_erf(x), 0, ERF_ATOL, "gelu_erf")


def test_gelu_erf_tails_and_kat(dev, golden):
    from qwenasr_amd import kernels as K

    x = golden["act_x"]
    xt = dev_t(x, dev)
    K.gelu_erf(xt, x.size)
    y = host(xt)
    assert_close(y, golden["gelu_erf_y64"], 0, ERF_ATOL, "gelu_erf grid")
    assert abs(y[0]) < 1e-5 and y[1] > 0.5 and y[2] < 0  # tests/kernels.rs:105-113


@pytest.mark.parametrize("n", [3000 * 3584, 10, 1003])
def test_gelu_tanh_matches_reference_arithmetic(dev, n):
    from qwenasr_amd import kernels as K

    r = rng(11, n)
    x = normal(r, n, 2.0)
    xt = dev_t(x, dev)
    K.gelu(xt, n)
    assert_close(host(xt), oracle.gelu_tanh(x), RTOL, ATOL, "gelu_tanh")


# ---------------------------------------------------------------------------
# Sinusoidal PE
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n_pos,dm", [(13, 896), (3000, 64), (13, 1024)])
def test_sinusoidal_pe(dev, n_pos, dm):
    from qwenasr_amd import kernels as K

    pe = torch.empty(n_pos * dm, dtype=torch.float32, device=dev)
    K.sinusoidal_pe(pe, n_pos, dm)
    assert_close(host(pe), oracle.sinusoidal_pe(n_pos, dm), RTOL, ATOL, "sinusoidal_pe")


@pytest.mark.parametrize("rows,dm,n_pos", [(3000, 896, 13), (3000, 896, 3000), (7, 30, 3)])
def test_pe_add(dev, rows, dm, n_pos):
    from qwenasr_amd import kernels as K

    r = rng(12, rows, dm)
    x = normal(r, rows * dm)
    pe = oracle.sinusoidal_pe(n_pos, dm)
    xt = dev_t(x, dev)
    K.pe_add(xt, dev_t(pe, dev), rows, dm, n_pos)
    np.testing.assert_array_equal(host(xt), oracle.pe_add(x, pe, rows, dm, n_pos))


@pytest.mark.parametrize("rows,dm,n_pos", [(3000, 896, 13), (64, 1024, 13), (50, 256, 7), (10, 2048, 13),
                                          (7, 30, 3), (5, 4096, 13)])
def test_pe_add_layer_norm_equals_the_two_passes(dev, rows, dm, n_pos):
    """The fused PE add + layer 0 LayerNorm equals pe_add followed by
    layer_norm bit for bit (x and out), on the one-wave-per-row path (hidden
    256..2048) and on the two-pass fallbacks (hidden 30, 4096); out against the
    oracle's LayerNorm of the oracle's x + pe at the LayerNorm tolerance."""
    from qwenasr_amd import kernels as K

    r = rng(14, rows, dm)
    x = normal(r, rows * dm)
    w = normal(r, dm, 0.1, 1.0)
    b = normal(r, dm, 0.02)
    pe = dev_t(oracle.sinusoidal_pe(n_pos, dm), dev)
    wt, bt = dev_t(w, dev), dev_t(b, dev)
    xa, xb = dev_t(x, dev), dev_t(x, dev)
    oa, ob = torch.empty_like(xa), torch.empty_like(xb)
    K.pe_add_layer_norm(xa, pe, oa, wt, bt, rows, dm, n_pos, 1e-5)
    K.pe_add(xb, pe, rows, dm, n_pos)
    K.layer_norm(ob, xb, wt, bt, rows, dm, 1e-5)
    np.testing.assert_array_equal(host(xa), host(xb))
    np.testing.assert_array_equal(host(oa), host(ob))
    xs = oracle.pe_add(x, host(pe), rows, dm, n_pos)
    np.testing.assert_array_equal(host(xa), xs)
    assert_close(host(oa), oracle.layer_norm(xs, w, b, rows, dm, 1e-5), RTOL, ATOL, "pe_add_layer_norm")


@pytest.mark.parametrize("rows,dm", [(3000, 896), (64, 1024), (50, 256), (10, 2048), (7, 30), (5, 4096)])
def test_add_layer_norm_equals_the_two_passes(dev, rows, dm):
    """The fused residual add + LayerNorm equals add_inplace followed by
    layer_norm bit for bit (x and out) on the one-wave-per-row path and on the
    two-pass fallbacks; out against the oracle's LayerNorm of x + delta."""
    from qwenasr_amd import kernels as K

    r = rng(15, rows, dm)
    x, d = normal(r, rows * dm), normal(r, rows * dm)
    w, b = normal(r, dm, 0.1, 1.0), normal(r, dm, 0.02)
    wt, bt, dt = dev_t(w, dev), dev_t(b, dev), dev_t(d, dev)
    xa, xb = dev_t(x, dev), dev_t(x, dev)
    oa, ob = torch.empty_like(xa), torch.empty_like(xb)
    K.add_layer_norm(xa, dt, wt, bt, oa, rows, dm, 1e-5)
    K.add_inplace(xb, dt, rows * dm)
    K.layer_norm(ob, xb, wt, bt, rows, dm, 1e-5)
    np.testing.assert_array_equal(host(xa), host(xb))
    np.testing.assert_array_equal(host(oa), host(ob))
    xs = (x + d).astype(np.float32)
    np.testing.assert_array_equal(host(xa), xs)
    assert_close(host(oa), oracle.layer_norm(xs, w, b, rows, dm, 1e-5), RTOL, ATOL, "add_layer_norm")


# ---------------------------------------------------------------------------
# Embedding gathers
# ---------------------------------------------------------------------------
def test_embed_gather_f32_bf16_i8(dev):
    from qwenasr_amd import kernels as K

    r = rng(13)
    vocab, dim, n = 4096, 1024, 512
    tab = normal(r, (vocab, dim), 0.02)
    ids = r.integers(0, vocab, n).astype(np.int32)
    out = torch.empty(n * dim, dtype=torch.float32, device=dev)
    K.embed_gather_f32(out, dev_t(tab, dev), dev_t(ids, dev), n, dim)
    np.testing.assert_array_equal(host(out), oracle.embed_gather_f32(tab, ids, dim))

    bits = r.integers(0, 1 << 16, (vocab, dim), dtype=np.uint16)
    K.embed_gather_bf16(out, dev_t(bits.view(np.int16), dev), dev_t(ids, dev), n, dim)
    np.testing.assert_array_equal(host(out).view(np.uint32), oracle.embed_gather_bf16(bits, ids, dim).view(np.uint32))

    t8 = r.integers(-128, 128, (vocab, dim), dtype=np.int8)
    s8 = r.uniform(1e-4, 1e-2, vocab).astype(np.float32)
    w = K.QuantWeight(dev_t(t8, dev), dev_t(s8, dev), vocab, dim)
    K.embed_gather_i8(out, w, dev_t(ids, dev), n, dim)
    np.testing.assert_array_equal(host(out), oracle.embed_gather_i8(t8, s8, ids, dim))


def test_embed_gather_ragged_dim_and_bad_ids(dev):
    from qwenasr_amd import kernels as K

    r = rng(14)
    vocab, dim = 50, 30  # dim not a multiple of 4: scalar path
    tab = normal(r, (vocab, dim))
    ids = np.array([0, 49, -1, 50, 7], np.int32)
    out = torch.empty(5 * dim, dtype=torch.float32, device=dev)
    K.embed_gather_f32(out, dev_t(tab, dev), dev_t(ids, dev), 5, dim)
    y = host(out).reshape(5, dim)
    np.testing.assert_array_equal(y[[0, 1, 4]], tab[[0, 49, 7]])
    assert np.isnan(y[2]).all() and np.isnan(y[3]).all()


def test_embed_gather_full_vocab_table(dev):
    # the benchmark table [151936, 1024], checked by exact row equality
    from qwenasr_amd import kernels as K

    vocab, dim, n = 151936, 1024, 512
    g = torch.Generator(device=dev).manual_seed(15)
    tab = torch.randn(vocab * dim, generator=g, device=dev) * 0.02
    ids = torch.randint(0, vocab, (n,), generator=g, device=dev, dtype=torch.int32)
    ids[0], ids[1] = 0, vocab - 1
    out = torch.empty(n * dim, dtype=torch.float32, device=dev)
    K.embed_gather_f32(out, tab, ids, n, dim)
    ref = tab.view(vocab, dim).index_select(0, ids.long()).reshape(-1)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_tok_embed_single_token(dev):
    from qwenasr_amd import kernels as K

    r = rng(16)
    bits = r.integers(0, 1 << 16, (10, 64), dtype=np.uint16)
    dst = torch.empty(64, dtype=torch.float32, device=dev)
    K.tok_embed_bf16_to_f32(dst, dev_t(bits.view(np.int16), dev), 7, 64)
    np.testing.assert_array_equal(host(dst).view(np.uint32), bits[7].astype(np.uint32) << 16)


# ---------------------------------------------------------------------------
# INT8: quantizer, W8A32, interleave, W8A8 + SwiGLU
# ---------------------------------------------------------------------------
def test_quantizer_fixture_bit_exact(dev, golden):
    from qwenasr_amd import kernels as K

    x = golden["quant_x"]
    q = torch.empty(x.size, dtype=torch.int8, device=dev)
    s = torch.empty(x.shape[0], dtype=torch.float32, device=dev)
    K.quantize_rows_i8(q, s, dev_t(x.ravel(), dev), x.shape[0], x.shape[1])
    np.testing.assert_array_equal(host(q).reshape(x.shape), golden["quant_q"])
    np.testing.assert_array_equal(host(s), golden["quant_s"])


@pytest.mark.parametrize("rows,cols", [(256, 2048), (1, 2048), (12288, 2048), (3, 77)])
def test_quantizer_matches_oracle(dev, rows, cols):
    from qwenasr_amd import kernels as K

    r = rng(17, rows, cols)
    x = normal(r, rows * cols, 0.02)
    q, s = K.quantize_f32_to_int8(dev_t(x, dev), rows, cols)
    q_ref, s_ref = oracle.quantize_f32_to_int8(x, rows, cols)
    np.testing.assert_array_equal(host(q), q_ref)
    np.testing.assert_array_equal(host(s), s_ref)


def make_qweight(r, rows, cols):
    w = normal(r, rows * cols, 0.02)
    return oracle.quantize_f32_to_int8(w, rows, cols)


@pytest.mark.parametrize("seq,in_dim,outs", [
    (1, 2048, (2048, 1024, 1024)),       # 1.7B q/k/v
    (1, 1024, (2048, 1024, 1024)),       # 0.6B q/k/v
    (1, 2048, (1, 5, 4096, 7)),          # four matrices, ragged row tails
    (1, 6144, (2048, 3)),
    (3, 2048, (2048, 1024)),             # several tokens: one launch per matrix
    (1, 1000, (17, 33)),                 # in_dim off the vector path
    (512, 1024, (2048, 1024, 1024)),     # prefill q/k/v: one matrix-core GEMM launch
    (17, 2048, (1, 5, 300, 7)),
])
def test_linear_nobias_int8_multi(dev, seq, in_dim, outs):
    """One launch over several matrices of the same x matches the separate
    linear_nobias_int8 calls and the oracle. Up to 7 tokens every row's dot is
    computed the same way whichever wave owns it, so the results are equal bit
    for bit; from 8 tokens (the matrix-core GEMM) the tile follows the total
    width, and a wider launch may use a tile that sums k in another order, so
    there both agree within the fp32 tolerance."""
    from qwenasr_amd import kernels as K

    r = rng(29, seq, in_dim, len(outs))
    x = normal(r, seq * in_dim)
    xt = dev_t(x, dev)
    ws, refs = [], []
    for o in outs:
        wq, sc = make_qweight(r, o, in_dim)
        ws.append(K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), o, in_dim))
        refs.append(oracle.linear_nobias_int8(x, wq, sc, seq, in_dim, o))
    ys = [torch.full((seq * o,), 7.0, device=dev) for o in outs]
    K.linear_nobias_int8_multi(ys, ws, xt, seq, in_dim)
    for o, y, w, ref in zip(outs, ys, ws, refs):
        z = torch.empty(seq * o, device=dev)
        K.linear_nobias_int8(z, xt, w.data, w.scales, seq, in_dim, o)
        if seq < 8:
            np.testing.assert_array_equal(host(y), host(z))
        else:
            assert_close(host(y), host(z).astype(np.float64), RTOL, ATOL, f"multi vs single out={o}")
        assert_close(host(y), ref, RTOL, ATOL, f"multi out={o}")


def _norm_inputs(r, H, dev):
    x, d, g = normal(r, H), normal(r, H), normal(r, H, 0.1, 1.0)
    return x, d, g, dev_t(x, dev), dev_t(d, dev), dev_t(g, dev)


def _unfused_norm(K, xt, dt, gt, H, eps, dev):
    """add_rms_norm (or rms_norm without delta) on copies: (residual, normalised row)."""
    xa, xn = xt.clone(), torch.empty(H, device=dev)
    if dt is not None:
        K.add_rms_norm(xa, dt, gt, xn, 1, H, eps)
    else:
        K.rms_norm(xn, xa, gt, 1, H, eps)
    return xa, xn


@pytest.mark.parametrize("H,outs,with_delta", [
    (2048, (2048, 1024, 1024), True),    # 1.7B q/k/v after the previous layer's down projection
    (2048, (2048, 1024, 1024), False),   # layer 0: plain RMSNorm of the embedding
    (1024, (2048, 1024, 1024), True),    # 0.6B
    (3072, (100, 7), True),              # three float4 per thread, ragged row tails
    (6144, (4096,), True),               # six float4 per thread
    (4096, (5, 33, 1000, 64), True),     # four matrices
])
def test_add_rms_norm_linear_multi_equals_unfused(dev, H, outs, with_delta):
    """The fused add + RMSNorm + projections launch equals add_rms_norm followed
    by linear_nobias_int8_multi bit for bit (every workgroup normalises the row
    in the standalone kernel's element order), writes h to h_out, leaves x and
    delta untouched, and matches the oracle's add + RMSNorm + matvecs."""
    from qwenasr_amd import kernels as K

    r = rng(41, H, len(outs), int(with_delta))
    eps = 1e-6
    x, d, g, xt, dt, gt = _norm_inputs(r, H, dev)
    dt = dt if with_delta else None
    qws, ws = [], []
    for o in outs:
        wq, sc = make_qweight(r, o, H)
        qws.append((wq, sc))
        ws.append(K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), o, H))
    xa, xn = _unfused_norm(K, xt, dt, gt, H, eps, dev)
    ref_ys = [torch.empty(o, device=dev) for o in outs]
    K.linear_nobias_int8_multi(ref_ys, ws, xn, 1, H)
    ys = [torch.full((o,), 7.0, device=dev) for o in outs]
    h_out = torch.full((H,), 5.0, device=dev)
    K.add_rms_norm_linear_nobias_int8_multi(ys, ws, h_out, xt, dt, gt, H, eps)
    for y, z in zip(ys, ref_ys):
        np.testing.assert_array_equal(host(y), host(z))
    np.testing.assert_array_equal(host(h_out), host(xa))
    np.testing.assert_array_equal(host(xt), x)
    if with_delta:
        np.testing.assert_array_equal(host(dt), d)
        xn_ref = oracle.add_rms_norm(x, d, g, 1, H, eps)[1]
    else:
        xn_ref = oracle.rms_norm(x, g, 1, H, eps)
    for y, (wq, sc), o in zip(ys, qws, outs):
        assert_close(host(y), oracle.linear_nobias_int8(xn_ref, wq, sc, 1, H, o), RTOL, ATOL, f"out={o}")


@pytest.mark.parametrize("H,I,with_delta", [(2048, 6144, True), (1024, 3072, True), (1024, 3072, False),
                                            (3072, 100, True), (6144, 2048, True)])
def test_add_rms_norm_gate_up_swiglu_equals_unfused(dev, H, I, with_delta):
    """The fused post-attention add + RMSNorm + gate/up + SwiGLU launch equals
    add_rms_norm followed by gate_up_swiglu_int8 bit for bit, and the oracle's
    add + RMSNorm + matvec + decode SwiGLU within the fp32 tolerance."""
    from qwenasr_amd import kernels as K

    r = rng(42, H, I, int(with_delta))
    eps = 1e-6
    x, d, g, xt, dt, gt = _norm_inputs(r, H, dev)
    dt = dt if with_delta else None
    wq, sc = make_qweight(r, 2 * I, H)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(sc, dev), 2 * I, H)
    xa, xn = _unfused_norm(K, xt, dt, gt, H, eps, dev)
    ref = torch.empty(I, device=dev)
    K.gate_up_swiglu_int8(ref, xn, w, 1, H, I)
    out = torch.full((I,), 7.0, device=dev)
    h_out = torch.full((H,), 5.0, device=dev)
    K.add_rms_norm_gate_up_swiglu_int8(out, h_out, xt, dt, gt, w, H, I, eps)
    np.testing.assert_array_equal(host(out), host(ref))
    np.testing.assert_array_equal(host(h_out), host(xa))
    np.testing.assert_array_equal(host(xt), x)
    xn_ref = oracle.add_rms_norm(x, d, g, 1, H, eps)[1] if with_delta else oracle.rms_norm(x, g, 1, H, eps)
    gu = oracle.linear_nobias_int8(xn_ref, wq, sc, 1, H, 2 * I)
    assert_close(host(out), oracle.swiglu_split(gu[0::2].copy(), gu[1::2].copy()), RTOL, ATOL, "swiglu")


@pytest.mark.parametrize("seq,in_dim,out_dim", [(1, 2048, 12288), (4, 1024, 3072), (3, 2048, 2048),
                                                (2, 100, 33),
                                                # one token: R rows per wave, ragged row tails
                                                (1, 1024, 1001), (1, 3072, 2047), (1, 4096, 33),
                                                (1, 6144, 2048), (1, 2048, 1),
                                                # rows per wave 1, 2 and 8 by output rows
                                                (1, 2048, 1024), (1, 2048, 4096), (1, 8192, 64),
                                                (1, 1024, 40000),
                                                # 8+ tokens: the bf16x3 matrix-core GEMM
                                                (8, 1024, 33), (64, 2048, 2048), (512, 1024, 6144),
                                                (100, 3072, 1000), (17, 1024, 130), (70, 6144, 257),
                                                (9, 1088, 200),
                                                # 192-row producer/consumer tiles, ragged rows and tokens
                                                (500, 1024, 5000),
                                                # split-K 64x64, 64x32 tiles (32x32 above), ragged
                                                (512, 1024, 2048), (512, 1088, 2048), (520, 1024, 2000),
                                                (512, 2048, 1024), (500, 1024, 1000),
                                                # split-K with 1-2 k steps (waves without a step)
                                                (16, 64, 64), (40, 128, 100),
                                                # 128 x 64 tiles, one workgroup per CU: the
                                                # producer/consumer kernel (ragged), and a K
                                                # (17 chunks) that it and the double-buffered
                                                # kernel refuse: the single-buffered one
                                                (512, 1024, 4096), (500, 2048, 4000), (512, 1088, 4096)])
def test_linear_nobias_int8_w8a32(dev, seq, in_dim, out_dim):
    from qwenasr_amd import kernels as K

    r = rng(18, seq, in_dim, out_dim)
    wq, ws = make_qweight(r, out_dim, in_dim)
    x = normal(r, seq * in_dim)
    y = torch.empty(seq * out_dim, dtype=torch.float32, device=dev)
    K.linear_nobias_int8(y, dev_t(x, dev), dev_t(wq, dev), dev_t(ws, dev), seq, in_dim, out_dim)
    ref = oracle.linear_nobias_int8(x, wq, ws, seq, in_dim, out_dim)
    assert_close(host(y), ref, RTOL, ATOL, "w8a32")
    b = normal(r, out_dim, 0.02)
    K.linear_int8(y, dev_t(x, dev), dev_t(wq, dev), dev_t(ws, dev), dev_t(b, dev), seq, in_dim, out_dim)
    assert_close(host(y), oracle.linear_int8(x, wq, ws, b, seq, in_dim, out_dim), RTOL, ATOL, "w8a32+bias")


def test_linear_nobias_int8_wide_tile(dev):
    """The 256 x 64 tile of the many-token GEMM (taken when it gives 512+
    workgroups, e.g. a 256-stream lm_head), ragged in tokens and rows: equal
    bit for bit to the same product computed in column blocks that take the
    128 x 64 tile (every tile adds each output's terms in the same order), and
    within 1e-5 of the oracle on a slice of the rows."""
    from qwenasr_amd import kernels as K

    r = rng(22)
    seq, in_dim, out_dim = 200, 1024, 33000  # 129 x 4 workgroups of 256 x 64
    wq, ws = make_qweight(r, out_dim, in_dim)
    x = normal(r, seq * in_dim)
    x_t, w_t, s_t = dev_t(x, dev), dev_t(wq, dev), dev_t(ws, dev)
    y = torch.empty(seq * out_dim, dtype=torch.float32, device=dev)
    K.linear_nobias_int8(y, x_t, w_t, s_t, seq, in_dim, out_dim)
    got = host(y).reshape(seq, out_dim)
    # blocks of >= 8192 rows: 64+ column blocks of 128 x 4 token blocks, < 512 of 256
    for r0, r1 in ((0, 8192), (8192, 16384), (16384, 24576), (24576, out_dim)):
        yb = torch.empty(seq * (r1 - r0), dtype=torch.float32, device=dev)
        K.linear_nobias_int8(yb, x_t, w_t[r0 * in_dim:r1 * in_dim], s_t[r0:r1], seq, in_dim, r1 - r0)
        np.testing.assert_array_equal(got[:, r0:r1], host(yb).reshape(seq, r1 - r0), err_msg=f"rows {r0}..{r1}")
    n = 300
    ref = oracle.linear_nobias_int8(x, wq.reshape(out_dim, in_dim)[out_dim - n:], ws[out_dim - n:], seq, in_dim, n)
    assert_close(got[:, out_dim - n:].ravel(), ref, RTOL, ATOL, "w8a32 256x64 tile, last rows")


def test_linear_nobias_int8_double_buffered_tile(dev):
    """The double-buffered 128 x 64 kernel (grids of at most one workgroup per
    CU) adds each output's terms in the single-buffered kernel's order: a
    product whose first 4096 rows are computed alone (256 workgroups, double
    buffered) equals, bit for bit, the same rows of the 6144-row product
    (384 workgroups, single buffered), ragged in tokens."""
    from qwenasr_amd import kernels as K

    r = rng(23)
    seq, in_dim, out_dim, part = 500, 1024, 6144, 4096
    wq, ws = make_qweight(r, out_dim, in_dim)
    x = normal(r, seq * in_dim)
    x_t, w_t, s_t = dev_t(x, dev), dev_t(wq, dev), dev_t(ws, dev)
    y = torch.empty(seq * out_dim, dtype=torch.float32, device=dev)
    K.linear_nobias_int8(y, x_t, w_t, s_t, seq, in_dim, out_dim)
    yp = torch.empty(seq * part, dtype=torch.float32, device=dev)
    K.linear_nobias_int8(yp, x_t, w_t[:part * in_dim], s_t[:part], seq, in_dim, part)
    got = host(y).reshape(seq, out_dim)
    np.testing.assert_array_equal(got[:, :part], host(yp).reshape(seq, part))
    n = 200
    ref = oracle.linear_nobias_int8(x, wq.reshape(out_dim, in_dim)[:n], ws[:n], seq, in_dim, n)
    assert_close(host(yp).reshape(seq, part)[:, :n].ravel(), ref, RTOL, ATOL, "w8a32 double-buffered")


def test_linear_int8_integer_inputs_exact(dev):
    # integer x, unit scales: the f32 accumulation is exact, so y is the int dot
    from qwenasr_amd import kernels as K

    r = rng(19)
    in_dim, out_dim = 2048, 512
    wq = r.integers(-128, 128, (out_dim, in_dim), dtype=np.int8)
    x = r.integers(-20, 21, in_dim).astype(np.float32)
    y = torch.empty(out_dim, dtype=torch.float32, device=dev)
    K.linear_nobias_int8(y, dev_t(x, dev), dev_t(wq, dev), torch.ones(out_dim, device=dev), 1,
                         in_dim, out_dim)
    exact = wq.astype(np.int64) @ x.astype(np.int64)
    np.testing.assert_array_equal(host(y).astype(np.int64), exact)


@pytest.mark.parametrize("seq,in_dim,out_dim", [
    (1, 2048, 300),      # the one-token rows kernel
    (64, 2048, 300),     # the split-K GEMM
    (500, 1024, 4096),   # the producer/consumer 128-row tile, ragged last token tile
    (512, 1024, 6144),   # its 192-row tile
])
def test_linear_int8_integer_inputs_exact_many_tokens(dev, seq, in_dim, out_dim):
    """Integer activations with unit scales: every path (one-token rows kernel,
    matrix-core GEMMs) returns the exact integer dots -- the three-term bf16
    split of an integer is exact and the fp32 sums stay below 2^24."""
    from qwenasr_amd import kernels as K

    r = rng(21, seq, in_dim, out_dim)
    wq = r.integers(-128, 128, (out_dim, in_dim), dtype=np.int8)
    x = r.integers(-20, 21, (seq, in_dim)).astype(np.float32)
    # row 0 non-integer throughout (compared to float64 below); small entries
    # beside the five specials keep its partial sums near its result, so fp32
    # accumulation stays inside the tolerance (integers up to 20 in the row
    # would cancel down to outputs far below the partial sums)
    x[0] = normal(r, in_dim, 1e-3)
    x[0, :5] = [1e-3, -2.5e-2, 3.75, 1 / 3, 65.0]
    y = torch.empty(seq * out_dim, dtype=torch.float32, device=dev)
    K.linear_nobias_int8(y, dev_t(x.ravel(), dev), dev_t(wq, dev), torch.ones(out_dim, device=dev), seq,
                         in_dim, out_dim)
    got = host(y).reshape(seq, out_dim)
    exact = x[1:].astype(np.int64) @ wq.astype(np.int64).T
    np.testing.assert_array_equal(got[1:].astype(np.int64), exact)
    ref0 = wq.astype(np.float64) @ x[0].astype(np.float64)
    assert_close(got[0], ref0, RTOL, ATOL, "non-integer row")


def test_interleave_gate_up(dev):
    from qwenasr_amd import kernels as K

    r = rng(20)
    inter, hid = 96, 256
    gq, gs = make_qweight(r, inter, hid)
    uq, us = make_qweight(r, inter, hid)
    fused = K.interleave_gate_up(K.QuantWeight(dev_t(gq, dev), dev_t(gs, dev), inter, hid),
                                 K.QuantWeight(dev_t(uq, dev), dev_t(us, dev), inter, hid))
    wgu, sgu = oracle.interleave_gate_up(gq, gs, uq, us, inter, hid)
    np.testing.assert_array_equal(host(fused.data), wgu)
    np.testing.assert_array_equal(host(fused.scales), sgu)


def gateup_inputs(r, batch, in_dim, inter):
    wq, ws = make_qweight(r, 2 * inter, in_dim)
    x = normal(r, batch * in_dim)
    xq, xs = oracle.quantize_f32_to_int8(x, batch, in_dim)
    return wq, ws, x, xq, xs


W8A8_CASES = [
    ("c4_matvec", 1, 2048, 6144),
    ("c4_0.6B", 1, 1024, 3072),
    ("c5_mfma", 256, 2048, 6144),
    ("mfma_lds_k1024_ragged", 100, 1024, 3072),
    ("mfma_lds_k512", 130, 512, 96),
    ("mfma_ragged_batch", 37, 2048, 96),
    ("mfma_small_k", 64, 512, 256),
    ("generic_path", 3, 400, 50),
    ("matvec_k3072", 1, 3072, 100),
]


@pytest.mark.parametrize("name,batch,in_dim,inter", W8A8_CASES)
def test_gate_up_swiglu_w8a8(dev, name, batch, in_dim, inter):
    from qwenasr_amd import kernels as K

    r = rng(21, batch, in_dim, inter)
    wq, ws, _, xq, xs = gateup_inputs(r, batch, in_dim, inter)
    out = torch.empty(batch * inter, dtype=torch.float32, device=dev)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(ws, dev), 2 * inter, in_dim)
    K.gate_up_swiglu_w8a8(out, w, dev_t(xq, dev), dev_t(xs, dev), batch, in_dim, inter)
    if batch * inter * in_dim <= 64 * 1024 * 1024:
        ref, _ = oracle.gate_up_swiglu_w8a8(wq, ws, xq, xs, batch, in_dim, inter)
    else:  # exact integer dots through float64 BLAS (exact below 2^53), f32 epilogue
        ref = w8a8_reference_blas(wq, ws, xq, xs, batch, in_dim, inter)
    assert_close(host(out), ref, RTOL, ATOL, name)


def w8a8_reference_blas(wq, ws, xq, xs, batch, in_dim, inter):
    dots = xq.reshape(batch, in_dim).astype(np.float64) @ wq.reshape(2 * inter, in_dim).astype(np.float64).T
    g = ((dots[:, 0::2].astype(np.float32) * xs[:, None]) * ws[None, 0::2]).astype(np.float64)
    u = ((dots[:, 1::2].astype(np.float32) * xs[:, None]) * ws[None, 1::2]).astype(np.float64)
    return (g / (1 + np.exp(-g)) * u).ravel()


@pytest.mark.parametrize("batch,in_dim,inter", [(1, 2048, 6144), (256, 2048, 6144), (5, 1024, 64)])
def test_w8a8_int32_dots_bit_exact(dev, batch, in_dim, inter):
    """Makes the epilogue the identity on the dots: positive gate rows and
    activations give dg >> 104 so expf(-g) == 0 and silu(g) == g exactly; with
    unit scales out == f32(dg) * f32(du). Any dot error shows as a bit change."""
    from qwenasr_amd import kernels as K

    r = rng(22, batch, in_dim, inter)
    w = np.empty((2 * inter, in_dim), np.int8)
    w[0::2] = r.integers(1, 128, (inter, in_dim), dtype=np.int8)      # gate rows > 0
    w[1::2] = r.integers(-128, 128, (inter, in_dim), dtype=np.int8)   # up rows: any sign
    xq = r.integers(1, 128, (batch, in_dim), dtype=np.int8)
    ones_w = np.ones(2 * inter, np.float32)
    ones_x = np.ones(batch, np.float32)
    out = torch.empty(batch * inter, dtype=torch.float32, device=dev)
    qw = K.QuantWeight(dev_t(w, dev), dev_t(ones_w, dev), 2 * inter, in_dim)
    K.gate_up_swiglu_w8a8(out, qw, dev_t(xq, dev), dev_t(ones_x, dev), batch, in_dim, inter)
    dots = xq.astype(np.float64) @ w.astype(np.float64).T   # exact integers
    assert dots[:, 0::2].min() > 200
    exp = (dots[:, 0::2].astype(np.float32) * dots[:, 1::2].astype(np.float32)).ravel()
    np.testing.assert_array_equal(host(out), exp)


@pytest.mark.parametrize("in_dim,inter", [(2048, 6144), (1024, 3072), (4096, 64)])
def test_gate_up_swiglu_w8a8_f32_input(dev, in_dim, inter):
    from qwenasr_amd import kernels as K

    r = rng(23, in_dim, inter)
    wq, ws, x, xq, xs = gateup_inputs(r, 1, in_dim, inter)
    out = torch.empty(inter, dtype=torch.float32, device=dev)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(ws, dev), 2 * inter, in_dim)
    K.gate_up_swiglu_w8a8_f32in(out, w, dev_t(x, dev), in_dim, inter)
    ref, _ = oracle.gate_up_swiglu_w8a8(wq, ws, xq, xs, 1, in_dim, inter)
    assert_close(host(out), ref, RTOL, ATOL, "f32in")
    # same result as quantize_rows_i8 + the int8-input entry point, bit for bit
    q2 = torch.empty(in_dim, dtype=torch.int8, device=dev)
    s2 = torch.empty(1, dtype=torch.float32, device=dev)
    K.quantize_rows_i8(q2, s2, dev_t(x, dev), 1, in_dim)
    out2 = torch.empty_like(out)
    K.gate_up_swiglu_w8a8(out2, w, q2, s2, 1, in_dim, inter)
    np.testing.assert_array_equal(host(out), host(out2))


def pack_tiles_reference(w: np.ndarray) -> np.ndarray:
    """The documented tile layout, built with numpy reshapes."""
    rows, cols = w.shape
    t = w.reshape(rows // 16, 16, cols // 64, 4, 16)      # [rb, r, s, g, b]
    t = t.transpose(0, 2, 3, 1, 4)                        # [rb, s, g, r, b] -> lane = 16 g + r
    return np.ascontiguousarray(t).reshape(-1)


@pytest.mark.parametrize("rows,cols", [(192, 2048), (12288, 2048), (16, 64), (48, 192)])
def test_pack_w8a8_tiles_layout(dev, rows, cols):
    from qwenasr_amd import kernels as K

    r = rng(25, rows, cols)
    w = r.integers(-128, 128, (rows, cols), dtype=np.int8)
    qw = K.QuantWeight(dev_t(w, dev), torch.ones(rows, device=dev), rows, cols)
    p = K.pack_w8a8_tiles(qw)
    np.testing.assert_array_equal(host(p.data), pack_tiles_reference(w))


# batch > 128 takes the 96-row x 128-token tile (c5, t96_*), 64 < batch <= 128
# the 192-row x 64-token tile, batch <= 64 the 48-row small kernel.
PACKED_CASES = [("c5", 256, 2048, 6144), ("ragged", 37, 2048, 96), ("k1024", 100, 1024, 3072),
                ("b1", 1, 2048, 96), ("t96_ragged", 200, 2048, 6144), ("t96_k1024", 300, 1024, 3072),
                ("t96_10tiles", 129, 2048, 480), ("b128", 128, 2048, 6144)]


@pytest.mark.parametrize("name,batch,in_dim,inter", PACKED_CASES)
def test_gate_up_swiglu_w8a8_packed(dev, name, batch, in_dim, inter):
    from qwenasr_amd import kernels as K

    r = rng(26, batch, in_dim, inter)
    wq, ws, _, xq, xs = gateup_inputs(r, batch, in_dim, inter)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(ws, dev), 2 * inter, in_dim)
    wp = K.pack_w8a8_tiles(w)
    out = torch.empty(batch * inter, dtype=torch.float32, device=dev)
    K.gate_up_swiglu_w8a8_packed(out, wp, dev_t(xq, dev), dev_t(xs, dev), batch, in_dim, inter)
    if batch * inter * in_dim <= 64 * 1024 * 1024:
        ref, _ = oracle.gate_up_swiglu_w8a8(wq, ws, xq, xs, batch, in_dim, inter)
    else:
        ref = w8a8_reference_blas(wq, ws, xq, xs, batch, in_dim, inter)
    assert_close(host(out), ref, RTOL, ATOL, name)
    # identical to the row-major entry point, bit for bit
    out2 = torch.empty_like(out)
    K.gate_up_swiglu_w8a8(out2, w, dev_t(xq, dev), dev_t(xs, dev), batch, in_dim, inter)
    np.testing.assert_array_equal(host(out), host(out2))


def test_w8a8_packed_int32_dots_bit_exact(dev):
    from qwenasr_amd import kernels as K

    batch, in_dim, inter = 256, 2048, 6144
    r = rng(27)
    w = np.empty((2 * inter, in_dim), np.int8)
    w[0::2] = r.integers(1, 128, (inter, in_dim), dtype=np.int8)
    w[1::2] = r.integers(-128, 128, (inter, in_dim), dtype=np.int8)
    xq = r.integers(1, 128, (batch, in_dim), dtype=np.int8)
    qw = K.QuantWeight(dev_t(w, dev), torch.ones(2 * inter, device=dev), 2 * inter, in_dim)
    out = torch.empty(batch * inter, dtype=torch.float32, device=dev)
    K.gate_up_swiglu_w8a8_packed(out, K.pack_w8a8_tiles(qw), dev_t(xq, dev),
                                 torch.ones(batch, device=dev), batch, in_dim, inter)
    dots = xq.astype(np.float64) @ w.astype(np.float64).T
    exp = (dots[:, 0::2].astype(np.float32) * dots[:, 1::2].astype(np.float32)).ravel()
    np.testing.assert_array_equal(host(out), exp)


# ---------------------------------------------------------------------------
# lm_head: INT8 logits + greedy argmax (decoder.rs:929-963)
# ---------------------------------------------------------------------------
def test_argmax_rows_matches_the_reference_loop(dev):
    """Index work: bit-exact against the sequential loop, including ties (first
    wins), NaN anywhere (never wins), NaN at element 0 (result 0), rows of -inf,
    all-NaN rows and +inf ties; vectorised and scalar paths."""
    from qwenasr_amd import kernels as K

    r = rng(40)
    for cols in (151936, 1003, 4, 1):
        rows = 12
        x = normal(r, rows * cols).reshape(rows, cols)
        x[1, :] = 2.5                                  # all equal: index 0
        if cols > 3:
            x[2, cols // 2] = x[2, cols - 1] = 9.0      # tie: first wins
            x[3, 0] = np.nan                            # NaN at 0: index 0
            x[4, ::7] = np.nan                          # scattered NaN
            x[4, cols - 2] = 50.0
            x[6, 1:3] = np.inf                          # +inf tie
        x[5, :] = -np.inf                               # all -inf: index 0
        x[7, :] = np.nan                                # all NaN: index 0
        ref = oracle.argmax_rows(x.ravel(), rows, cols)
        idx = torch.empty(rows, dtype=torch.int32, device=dev)
        K.argmax_rows(idx, dev_t(x.ravel(), dev), rows, cols)
        np.testing.assert_array_equal(host(idx), ref)
        # misaligned start (scalar path)
        xs = np.concatenate([[0.0], x.ravel()]).astype(np.float32)
        xt = dev_t(xs, dev)[1:]
        K.argmax_rows(idx, xt, rows, cols)
        np.testing.assert_array_equal(host(idx), ref)


@pytest.mark.parametrize("rows,in_dim,vocab,use_ws", [
    (1, 1024, 151936, True), (1, 1024, 151936, False), (3, 2048, 5000, True),
    (1, 2048, 5001, True), (1, 3072, 4099, True), (1, 6144, 997, True), (1, 1000, 300, True)])
def test_lm_head_int8_argmax(dev, rows, in_dim, vocab, use_ws):
    """Logits within the W8A32 tolerance of the oracle; the token index equals
    the reference loop's on the oracle logits whenever the top two logits are
    further apart than twice the tolerance (checked), and always equals the
    argmax of the returned logits. ``use_ws``: with the workspace (one row: argmax
    reduced inside the matvec) or without (logits scanned afterwards)."""
    from qwenasr_amd import kernels as K

    r = rng(41, rows, vocab)
    wq, ws = make_qweight(r, vocab, in_dim)
    x = normal(r, rows * in_dim)
    ref_logits = oracle.linear_nobias_int8(x, wq, ws, rows, in_dim, vocab, n_threads=8)
    ref_idx = oracle.argmax_rows(ref_logits, rows, vocab)
    idx = torch.empty(rows, dtype=torch.int32, device=dev)
    logits = torch.empty(rows * vocab, device=dev)
    w = K.QuantWeight(dev_t(wq, dev), dev_t(ws, dev), vocab, in_dim)
    wsp = K.lm_head_workspace(vocab, dev) if use_ws else None
    K.lm_head_int8_argmax(idx, logits, dev_t(x, dev), w, rows, in_dim, vocab, wsp)
    lg = host(logits)
    assert_close(lg, ref_logits, RTOL, ATOL, "logits")
    np.testing.assert_array_equal(host(idx), oracle.argmax_rows(lg, rows, vocab))
    top2 = np.sort(ref_logits.reshape(rows, vocab), axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * (ATOL + RTOL * np.abs(top2[:, 1]))
    assert clear.any()
    np.testing.assert_array_equal(host(idx)[clear], ref_idx[clear])


@pytest.mark.parametrize("in_dim,vocab", [(1024, 151936), (2048, 5003), (5120, 999)])
def test_lm_head_fused_argmax_ties_nan_and_tails(dev, in_dim, vocab):
    """The in-matvec reduction keeps the reference loop's order across
    workgroups: equal maxima in rows far apart go to the lower index, a NaN
    logit never wins, a NaN logit at index 0 gives 0, a -inf-only candidate set
    still has an index; the last partial workgroup counts."""
    from qwenasr_amd import kernels as K

    r = rng(42, in_dim, vocab)
    wq = r.integers(-3, 4, size=(vocab, in_dim), dtype=np.int8)
    ws = np.full(vocab, 1e-3, np.float32)
    x = np.ones(in_dim, np.float32)
    idx = torch.empty(1, dtype=torch.int32, device=dev)
    logits = torch.empty(vocab, device=dev)
    wsp = K.lm_head_workspace(vocab, dev)

    def run(wq, ws):
        w = K.QuantWeight(dev_t(wq, dev), dev_t(ws, dev), vocab, in_dim)
        K.lm_head_int8_argmax(idx, logits, dev_t(x, dev), w, 1, in_dim, vocab, wsp)
        lg = host(logits)
        return int(host(idx)[0]), lg

    top = [vocab // 2 + 1, 7, vocab - 1]
    w2 = wq.copy()
    for t in top:
        w2[t, :] = 127                                    # identical maxima
    w2s = ws.copy()
    w2s[top] = 1.0
    got, lg = run(w2, w2s)
    assert got == 7 == int(oracle.argmax_rows(lg, 1, vocab)[0])
    w2s[7] = np.nan                                       # NaN never wins
    got, lg = run(w2, w2s)
    assert np.isnan(lg[7]) and got == min(top[0], top[2]) == int(oracle.argmax_rows(lg, 1, vocab)[0])
    w3s = ws.copy()
    w3s[vocab - 1] = 1.0                                  # the max in the last (partial) workgroup
    w3 = wq.copy()
    w3[vocab - 1, :] = 127
    got, lg = run(w3, w3s)
    assert got == vocab - 1
    w3s[0] = np.nan                                       # NaN at index 0: result 0
    got, lg = run(w3, w3s)
    assert got == 0 == int(oracle.argmax_rows(lg, 1, vocab)[0])
    w4s = np.full(vocab, -np.inf, np.float32)             # -inf and NaN, one finite logit
    w4 = np.ones_like(wq)
    w4s[1: vocab // 3] = np.nan
    w4s[vocab - 2] = -1.0
    got, lg = run(w4, w4s)
    assert np.isneginf(lg[0]) and got == vocab - 2 == int(oracle.argmax_rows(lg, 1, vocab)[0])
    w4s[vocab - 2] = -np.inf                              # all -inf or NaN: the first -inf
    got, lg = run(w4, w4s)
    assert got == 0 == int(oracle.argmax_rows(lg, 1, vocab)[0])


# ---------------------------------------------------------------------------
# Causal GQA attention over a KV block (kernels/mod.rs:1124-1207)
# ---------------------------------------------------------------------------
ATTN_CASES = [
    ("decode_pos0", 1, 1, 16, 8, 128, 0),           # first token: a single key
    ("decode_pos300", 1, 301, 16, 8, 128, 300),     # 1.7B/0.6B decode step
    ("decode_pos2047", 1, 2048, 16, 8, 128, 2047),
    ("prefill_512", 512, 512, 16, 8, 128, 0),       # 0.6B prefill, causal triangle
    ("chunked_prefill", 37, 137, 16, 8, 128, 100),  # 37 new rows after 100 cached
    ("keys_before_limit", 6, 3, 4, 4, 64, 10),      # seq_k below the causal limit, head_dim 64
    ("gqa4_hd64", 9, 70, 8, 2, 64, 61),
    ("mha_g1", 3, 65, 4, 4, 128, 62),
    ("gqa8", 2, 129, 8, 1, 128, 127),
    ("no_keys", 2, 0, 16, 8, 128, 0),
    # prefill on the matrix cores (16 rows per workgroup, tiles alternate between 2 wave groups)
    ("mfma_16_rows", 16, 16, 16, 8, 128, 0),
    ("mfma_ragged_17", 17, 17, 16, 8, 128, 0),
    ("mfma_mha_g1", 40, 90, 8, 8, 128, 50),
    ("mfma_keys_below_limit", 33, 20, 16, 8, 128, 40),
    ("mfma_one_key", 16, 1, 16, 8, 128, 0),
    ("mfma_chunk_700", 700, 1000, 16, 8, 128, 300),
    ("mfma_no_keys", 20, 0, 16, 8, 128, 0),
    ("mfma_g4", 25, 60, 16, 4, 128, 35),
    ("mfma_g8", 9, 40, 8, 1, 128, 31),
    ("mfma_g2_8_rows", 8, 8, 16, 8, 128, 0),
]


@pytest.mark.parametrize("name,seq_q,seq_k,nq,nk,hd,q_offset", ATTN_CASES)
def test_causal_attention(dev, name, seq_q, seq_k, nq, nk, hd, q_offset):
    from qwenasr_amd import kernels as K

    r = rng(50, seq_q, seq_k, nq, hd)
    q = normal(r, seq_q * nq * hd)
    k = normal(r, max(seq_k, 1) * nk * hd)
    v = normal(r, max(seq_k, 1) * nk * hd)
    scale = hd ** -0.5
    ref = oracle.causal_attention(q, k, v, seq_q, seq_k, nq, nk, hd, scale, q_offset)
    out = torch.full((seq_q * nq * hd,), 5.0, device=dev)
    K.causal_attention(out, dev_t(q, dev), dev_t(k, dev), dev_t(v, dev), seq_q, seq_k, nq, nk, hd,
                       scale, q_offset)
    assert_close(host(out), ref, RTOL, ATOL, name)


def test_causal_attention_reads_a_cache_block(dev):
    """k/v are the first seq_k rows of a larger KvCache layer block (the
    reference passes k_layer_full): rows past seq_k are never read."""
    from qwenasr_amd import kernels as K

    nq, nk, hd, max_seq, seq_k = 16, 8, 128, 64, 20
    r = rng(51)
    q = normal(r, nq * hd)
    kc = normal(r, max_seq * nk * hd)
    vc = normal(r, max_seq * nk * hd)
    kc[seq_k * nk * hd:] = np.nan
    vc[seq_k * nk * hd:] = np.nan
    ref = oracle.causal_attention(q, kc[: seq_k * nk * hd], vc[: seq_k * nk * hd], 1, seq_k, nq, nk,
                                  hd, hd ** -0.5, seq_k - 1)
    out = torch.empty(nq * hd, device=dev)
    K.causal_attention(out, dev_t(q, dev), dev_t(kc, dev), dev_t(vc, dev), 1, seq_k, nq, nk, hd,
                       hd ** -0.5, seq_k - 1)
    assert_close(host(out), ref, RTOL, ATOL, "cache block")


@pytest.mark.parametrize("name,seq_q,seq_k,nq,nk,hd,q_offset", [
    ("decode_1.7b_pos2047", 1, 2048, 16, 8, 128, 2047),
    ("decode_pos700", 1, 701, 16, 8, 128, 700),
    ("decode_3rows", 3, 4000, 16, 8, 128, 3997),
    ("decode_hd64_g4", 1, 1500, 8, 2, 64, 1499),
    ("short_no_split", 1, 200, 16, 8, 128, 199),
    ("rows_end_early", 2, 3000, 16, 8, 128, 700),   # causal limit far below seq_k: empty splits
    # prefill shapes with a workspace: many rows (the matrix-core kernel) and
    # few rows over long key ranges (the split)
    ("prefill_0.6b_t512", 512, 512, 16, 8, 128, 0),
    ("prefill_chunk_at_200", 100, 300, 16, 8, 128, 200),
    ("prefill_g1", 130, 900, 8, 8, 128, 770),
    ("prefill_g4_long", 40, 4000, 16, 4, 128, 3960),
    ("prefill_g8", 24, 100, 16, 2, 128, 76),
    ("prefill_seq_k_short", 64, 200, 16, 8, 128, 300),  # every row limited by seq_k
])
def test_causal_attention_split(dev, name, seq_q, seq_k, nq, nk, hd, q_offset):
    from qwenasr_amd import kernels as K

    r = rng(52, seq_q, seq_k, hd)
    q = normal(r, seq_q * nq * hd)
    k = normal(r, seq_k * nk * hd)
    v = normal(r, seq_k * nk * hd)
    ref = oracle.causal_attention(q, k, v, seq_q, seq_k, nq, nk, hd, hd ** -0.5, q_offset)
    out = torch.empty(seq_q * nq * hd, device=dev)
    ws = K.attention_workspace(seq_q, nq, hd, dev)
    K.causal_attention_split(out, dev_t(q, dev), dev_t(k, dev), dev_t(v, dev), seq_q, seq_k, nq, nk,
                             hd, hd ** -0.5, q_offset, ws)
    assert_close(host(out), ref, RTOL, ATOL, name)
    # a too-small workspace falls back to fewer or no splits, same results
    out2 = torch.empty_like(out)
    K.causal_attention_split(out2, dev_t(q, dev), dev_t(k, dev), dev_t(v, dev), seq_q, seq_k, nq, nk,
                             hd, hd ** -0.5, q_offset, ws[:100])
    assert_close(host(out2), ref, RTOL, ATOL, name + " fallback")


@pytest.mark.parametrize("pos,nq,nk,hd,cache_rows", [
    (1023, 16, 8, 128, 2048),   # 1.7B / 0.6B decode: one attention launch
    (2047, 16, 8, 128, 2048),   # last cache row
    (300, 16, 16, 128, 512),    # one q head per kv head
    (1499, 8, 2, 64, 1600),     # head_dim 64, 4 q heads per kv head
    (700, 4, 2, 64, 701),
    (200, 16, 8, 128, 256),     # too few keys to split: the two-call form
    (0, 16, 8, 128, 8),         # first token
])
def test_decode_attention_equals_unfused(dev, pos, nq, nk, hd, cache_rows):
    """The one-token attention block in one call equals head_rms_norm_rope_kv
    followed by causal_attention_split bit for bit: the output and every cache
    row (the workgroup holding key pos writes the cache rows itself)."""
    from qwenasr_amd import kernels as K

    r = rng(54, pos, nq, hd)
    kv_dim = nk * hd
    q, k, v = normal(r, nq * hd), normal(r, kv_dim), normal(r, kv_dim)
    qw, kw = normal(r, hd, 0.1, 1.0), normal(r, hd, 0.1, 1.0)
    cache_k, cache_v = normal(r, cache_rows * kv_dim), normal(r, cache_rows * kv_dim)
    rope = K.RopeCache(dev)
    rope.ensure(pos + 1, hd, 1e6)
    scale = hd ** -0.5
    outs, caches = [], []
    for fused in (True, False):
        kc, vc = dev_t(cache_k, dev), dev_t(cache_v, dev)
        qt, kt, vt = dev_t(q, dev), dev_t(k, dev), dev_t(v, dev)
        out = torch.full((nq * hd,), 9.0, device=dev)
        ws = K.attention_workspace(1, nq, hd, dev)
        if fused:
            K.decode_attention(out, qt, kt, vt, dev_t(qw, dev), dev_t(kw, dev), rope, pos, nq, nk, hd, 1e-6,
                               scale, kc, vc, cache_rows, ws)
        else:
            K.head_rms_norm_rope_kv(qt, kt, vt, dev_t(qw, dev), dev_t(kw, dev), rope, None, pos, 1, nq, nk,
                                    hd, 1e-6, kc, vc, cache_rows)
            K.causal_attention_split(out, qt, kc, vc, 1, pos + 1, nq, nk, hd, scale, pos, ws)
        outs.append(host(out))
        caches.append((host(kc), host(vc)))
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(caches[0][0], caches[1][0])
    np.testing.assert_array_equal(caches[0][1], caches[1][1])
    # rows other than pos are untouched
    others = np.r_[0:pos * kv_dim, (pos + 1) * kv_dim:cache_rows * kv_dim]
    np.testing.assert_array_equal(caches[0][0][others], cache_k[others])
    # and the oracle: norm + RoPE + cache store, then attention over rows 0..pos
    cos, sin = oracle.rope_table(rope.cap, hd, 1e6)
    q_ref, k_rows, v_rows = kv_reference(q, k, v, qw, kw, cos, sin, np.array([pos]), 1, nq, nk, hd, 1e-6)
    kref = cache_k.reshape(cache_rows, kv_dim)[:pos + 1].copy()
    vref = cache_v.reshape(cache_rows, kv_dim)[:pos + 1].copy()
    kref[pos], vref[pos] = k_rows[0], v_rows[0]
    ref = oracle.causal_attention(q_ref.astype(np.float32), kref.ravel(), vref.ravel(), 1, pos + 1, nq, nk,
                                  hd, scale, pos)
    assert_close(outs[0], ref, RTOL, ATOL, "decode attention")


def test_causal_attention_split_repeated_calls_share_the_workspace(dev):
    """64 calls in a row on one workspace, with alternating inputs, each equal
    to the oracle."""
    from qwenasr_amd import kernels as K

    nq, nk, hd, seq_k = 16, 8, 128, 2048
    r = rng(53)
    cases = []
    for c in range(2):
        q = normal(r, nq * hd)
        k = normal(r, seq_k * nk * hd)
        v = normal(r, seq_k * nk * hd)
        pos = seq_k - 1 - 517 * c
        ref = oracle.causal_attention(q, k, v, 1, seq_k, nq, nk, hd, hd ** -0.5, pos)
        cases.append((dev_t(q, dev), dev_t(k, dev), dev_t(v, dev), pos, ref))
    ws = K.attention_workspace(1, nq, hd, dev)
    outs = [torch.empty(nq * hd, device=dev) for _ in range(64)]
    for it in range(64):
        q, k, v, pos, _ = cases[it % 2]
        K.causal_attention_split(outs[it], q, k, v, 1, seq_k, nq, nk, hd, hd ** -0.5, pos, ws)
    for it in range(64):
        assert_close(host(outs[it]), cases[it % 2][4], RTOL, ATOL, f"call {it}")


def test_config_chains_replay_in_graphs(dev):
    """bench.py times the c2-c5 chains (and c3 with the fused PE add + LayerNorm)
    as captured HIP graphs. For each chain,
    three replays -- inputs restored and outputs overwritten by eager work,
    the device synchronised in between -- give the eager call's results bit
    for bit (the W8A8 GEMM at B=256, the packed kernel, and at B=32, the
    small-batch kernel)."""
    from qwenasr_amd import kernels as K

    gen = torch.Generator(device=dev).manual_seed(41)

    def rnd(*n):
        return torch.randn(*n, device=dev, generator=gen)

    def run_chain(name, inputs, outputs, fn):
        pristine = {k: v.clone() for k, v in inputs.items()}

        def restore():
            for k, v in inputs.items():
                v.copy_(pristine[k])
            for t in outputs.values():
                t.fill_(-1) if t.dtype in (torch.int8, torch.int32) else t.fill_(float("nan"))

        restore()
        fn()
        torch.cuda.synchronize()
        ref = {k: v.clone() for k, v in {**inputs, **outputs}.items()}
        restore()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        for rep in range(3):
            restore()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for k, v in {**inputs, **outputs}.items():
                assert torch.equal(v, ref[k]), f"{name}: replay {rep} differs in {k}"

    rope = K.RopeCache(dev)
    rope.ensure(2048, 128, 1e6)

    # c2 at 64 tokens: gather, add+RMSNorm, q/k norm+RoPE, SwiGLU
    T, H, I, V = 64, 1024, 3072, 4096
    table = rnd(V * H)
    ids = torch.randint(0, V, (T,), device=dev, generator=gen, dtype=torch.int32)
    gin = {"x": rnd(T * H), "q": rnd(T * 16 * 128), "k": rnd(T * 8 * 128)}
    gout = {"emb": torch.empty(T * H, device=dev), "y": torch.empty(T * H, device=dev),
            "o": torch.empty(T * I, device=dev)}
    d, gu, w = rnd(T * H), rnd(T * 2 * I), rnd(H)
    qw, kw = rnd(128), rnd(128)

    def c2():
        K.embed_gather_f32(gout["emb"], table, ids, T, H)
        K.add_rms_norm(gin["x"], d, w, gout["y"], T, H, 1e-6)
        K.head_rms_norm_rope(gin["q"], gin["k"], qw, kw, rope.cos, rope.sin, None, T, 16, 8, 128, 1e-6)
        K.swiglu_multiply(gout["o"], gu, T, I)

    run_chain("c2", gin, gout, c2)

    # c3 at 300 rows: PE add, LayerNorm, erf-GELU
    R, D, F_ = 300, 896, 3584
    pe = torch.empty(13 * D, device=dev)
    K.sinusoidal_pe(pe, 13, D)
    ein = {"x": rnd(R * D), "h": rnd(R * F_)}
    eout = {"ln": torch.empty(R * D, device=dev)}
    lw, lb = rnd(D), rnd(D)

    def c3():
        K.pe_add(ein["x"], pe, R, D, 13)
        K.layer_norm(eout["ln"], ein["x"], lw, lb, R, D, 1e-5)
        K.gelu_erf(ein["h"], R * F_)

    run_chain("c3", ein, eout, c3)

    def c3_fused():
        K.pe_add_layer_norm(ein["x"], pe, eout["ln"], lw, lb, R, D, 13, 1e-5)
        K.gelu_erf(ein["h"], R * F_)

    run_chain("c3 fused", ein, eout, c3_fused)
    dres = rnd(R * D)
    run_chain("add + LayerNorm", ein, eout, lambda: K.add_layer_norm(ein["x"], dres, lw, lb, eout["ln"], R, D, 1e-5))

    # c4: W8A8 matvec + SwiGLU with the activation quantized in the kernel
    Hc, Ic = 2048, 6144
    wq, ws = K.quantize_f32_to_int8(rnd(2 * Ic * Hc) * 0.02, 2 * Ic, Hc)
    wgu = K.QuantWeight(wq, ws, 2 * Ic, Hc)
    xin = rnd(Hc)
    c4out = {"o": torch.empty(Ic, device=dev)}
    run_chain("c4", {}, c4out, lambda: K.gate_up_swiglu_w8a8_f32in(c4out["o"], wgu, xin, Hc, Ic))

    # c5 at B=256 and B=32: add+RMSNorm+quant, q/k norm+RoPE at per-row positions, GEMM
    wpk = K.pack_w8a8_tiles(wgu)
    for B in (256, 32):
        bin_ = {"x": rnd(B * Hc), "q": rnd(B * 16 * 128), "k": rnd(B * 8 * 128)}
        bout = {"xq": torch.empty(B * Hc, dtype=torch.int8, device=dev), "xs": torch.empty(B, device=dev),
                "o": torch.empty(B * Ic, device=dev)}
        bd, bw = rnd(B * Hc), rnd(Hc)
        pos = torch.randint(0, 2048, (B,), device=dev, generator=gen, dtype=torch.int32)

        def c5():
            K.add_rms_norm_quant(bin_["x"], bd, bw, None, bout["xq"], bout["xs"], B, Hc, 1e-6)
            K.head_rms_norm_rope(bin_["q"], bin_["k"], qw, kw, rope.cos, rope.sin, pos, B, 16, 8, 128, 1e-6)
            K.gate_up_swiglu_w8a8_packed(bout["o"], wpk, bout["xq"], bout["xs"], B, Hc, Ic)

        run_chain(f"c5 B={B}", bin_, bout, c5)
