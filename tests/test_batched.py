"""Batched multi-stream W8A8 projections on the GPU against the oracle.

qasr_linear_w8a8_packed is the reference's linear_nobias_int8
(kernels/mod.rs:650-661) with each stream's activation row quantized per row:
its int32 dots are exact and its dequantization is one fixed sequence of f32
multiplies, so the output equals oracle.linear_w8a8 bit for bit.

qasr_qkv_heads_w8a8_packed is the q/k/v projections of B streams plus the
steps after them (decoder.rs:881-895 per stream: q/k head RMSNorm, RoPE at
the stream's own position, the K/V rows stored in the stream's cache block).
It must equal the plain projection followed by the standalone head kernel
bit for bit, and the oracle's composition (linear_w8a8, then
head_rms_norm_rope looped over streams) within rel/abs 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.conftest import assert_close

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

NQ, NK, HD = 16, 8, 128


def _quant_rows(r, rows, cols, scale=1.0):
    x = (scale * r.standard_normal((rows, cols))).astype(np.float32)
    q, s = oracle.quantize_f32_to_int8(x.ravel(), rows, cols)
    return q.reshape(rows, cols), s


def _packed(dev, wq, ws):
    from qwenasr_amd import kernels as K

    o, i = wq.shape
    w = K.QuantWeight(torch.from_numpy(wq.ravel().copy()).to(dev), torch.from_numpy(ws).to(dev), o, i)
    return K.pack_w8a8_tiles(w)


@pytest.mark.parametrize("batch,out_dim,in_dim", [(1, 128, 1024), (5, 384, 2048), (31, 256, 1024),
                                                  (32, 2048, 2048), (33, 128, 2048), (256, 4096, 2048),
                                                  (256, 2048, 2048), (256, 2048, 6144), (17, 256, 3072),
                                                  (3, 128, 4096), (256, 1024, 4096), (37, 384, 6144)])
def test_linear_w8a8_packed_bit_exact(dev, batch, out_dim, in_dim):
    from qwenasr_amd import kernels as K

    r = np.random.default_rng([51, batch, out_dim, in_dim])
    wq, ws = _quant_rows(r, out_dim, in_dim, 0.02)
    xq, xs = _quant_rows(r, batch, in_dim)
    w = _packed(dev, wq, ws)
    y = torch.full((batch * out_dim,), float("nan"), device=dev)
    print(f"[batched] linear_w8a8 B={batch} N={out_dim} K={in_dim}", flush=True)
    K.linear_w8a8_packed(y, w, torch.from_numpy(xq.ravel().copy()).to(dev), torch.from_numpy(xs).to(dev),
                         batch, in_dim, out_dim)
    torch.cuda.synchronize()
    ref, _ = oracle.linear_w8a8(wq, ws, xq, xs, batch, in_dim, out_dim)
    np.testing.assert_array_equal(y.cpu().numpy(), ref)


@pytest.mark.parametrize("batch,out_dim,in_dim", [(8, 131072, 1024), (40, 65536, 1024), (4, 131072, 3072),
                                                  (256, 32768, 2048)])
def test_linear_w8a8_packed_persistent(dev, batch, out_dim, in_dim):
    """Outputs wide enough for 4+ tiles per CU take the persistent projection
    (each workgroup walks a range of column tiles): equal bit for bit to the
    same product computed in 8192-row column blocks (one-tile workgroups, each
    tile adds the same dots in the same order), and to the oracle on the first
    and last 256 rows; ragged batches, one-, two- and eight-tile stream
    splits, 16- and 32-stream tiles."""
    from qwenasr_amd import kernels as K

    r = np.random.default_rng([52, batch, out_dim, in_dim])
    wq = r.integers(-127, 128, (out_dim, in_dim), dtype=np.int8)
    ws = (r.random(out_dim) * 0.01 + 1e-3).astype(np.float32)
    xq, xs = _quant_rows(r, batch, in_dim)
    w = _packed(dev, wq, ws)
    xq_t, xs_t = torch.from_numpy(xq.ravel().copy()).to(dev), torch.from_numpy(xs).to(dev)
    y = torch.full((batch * out_dim,), float("nan"), device=dev)
    print(f"[batched] linear_w8a8 persistent B={batch} N={out_dim} K={in_dim}", flush=True)
    K.linear_w8a8_packed(y, w, xq_t, xs_t, batch, in_dim, out_dim)
    got = y.view(batch, out_dim).cpu().numpy()
    blk = 8192
    for r0 in range(0, out_dim, blk):
        wb = K.QuantWeight(w.data[r0 * in_dim:(r0 + blk) * in_dim], w.scales[r0:r0 + blk], blk, in_dim)
        yb = torch.empty(batch * blk, device=dev)
        K.linear_w8a8_packed(yb, wb, xq_t, xs_t, batch, in_dim, blk)
        np.testing.assert_array_equal(got[:, r0:r0 + blk], yb.view(batch, blk).cpu().numpy(),
                                      err_msg=f"rows {r0}..{r0 + blk}")
    for r0 in (0, out_dim - 256):
        ref, _ = oracle.linear_w8a8(wq[r0:r0 + 256], ws[r0:r0 + 256], xq, xs, batch, in_dim, 256)
        np.testing.assert_array_equal(got[:, r0:r0 + 256], ref.reshape(batch, 256))


def _qkv_case(dev, batch, in_dim, cache_rows, seed, bad_rows=()):
    """Inputs of one q/k/v call: packed weights, quantized rows, gains,
    positions (with the given rows set out of range), the RoPE table."""
    from qwenasr_amd import kernels as K

    r = np.random.default_rng(seed)
    N = (NQ + 2 * NK) * HD
    wq, ws = _quant_rows(r, N, in_dim, 0.02)
    xq, xs = _quant_rows(r, batch, in_dim)
    qw = (1 + 0.1 * r.standard_normal(HD)).astype(np.float32)
    kw = (1 + 0.1 * r.standard_normal(HD)).astype(np.float32)
    pos = r.integers(0, cache_rows, batch).astype(np.int32)
    for i, v in bad_rows:
        pos[i] = v
    rope = K.RopeCache(dev)
    rope.ensure(cache_rows, HD, 1e6)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return dict(wq=wq, ws=ws, xq=xq, xs=xs, qw=qw, kw=kw, pos=pos, w=_packed(dev, wq, ws), rope=rope,
                xq_t=t(xq.ravel()), xs_t=t(xs), qw_t=t(qw), kw_t=t(kw), pos_t=t(pos))


def _run_fused(dev, c, batch, in_dim, cache_rows, fill=7.0):
    from qwenasr_amd import kernels as K

    kv = NK * HD
    q = torch.full((batch * NQ * HD,), float("nan"), device=dev)
    kc = torch.full((batch * cache_rows * kv,), fill, device=dev)
    vc = torch.full((batch * cache_rows * kv,), fill, device=dev)
    K.qkv_heads_w8a8_packed(q, kc, vc, cache_rows, c["w"], c["xq_t"], c["xs_t"], c["qw_t"], c["kw_t"], c["rope"],
                            c["pos_t"], batch, in_dim, NQ, NK, HD, 1e-6)
    return q, kc, vc


@pytest.mark.parametrize("B,Kd", [(37, 2048), (250, 2048), (250, 1024)])
def test_qkv_heads_fused_equals_projection_then_head_kernel(dev, B, Kd):
    """Ragged batches (37 streams in 16-stream tiles; 250 in 32-stream tiles,
    the streamed kernel, the last tile partial), one position outside the
    RoPE table and one below 0: the fused launch equals
    qasr_linear_w8a8_packed + qasr_head_rms_norm_rope_kv_f32 bit for bit --
    q rows (NaN for the bad positions), the cache rows at each stream's
    position, and no other cache row touched."""
    from qwenasr_amd import kernels as K

    rows = 1024 if B < 64 else 256
    c = _qkv_case(dev, B, Kd, rows, [52, B, Kd], bad_rows=((3, -1), (20, 5000)))
    print(f"[batched] qkv heads fused B={B} K={Kd}", flush=True)
    q, kc, vc = _run_fused(dev, c, B, Kd, rows)
    # unfused: the projection, then the head kernel on its q/k/v slices
    N, kv = (NQ + 2 * NK) * HD, NK * HD
    y = torch.empty(B * N, device=dev)
    K.linear_w8a8_packed(y, c["w"], c["xq_t"], c["xs_t"], B, Kd, N)
    y = y.view(B, N)
    q2 = y[:, :NQ * HD].contiguous().view(-1)
    k2 = y[:, NQ * HD:(NQ + NK) * HD].contiguous().view(-1)
    v2 = y[:, (NQ + NK) * HD:].contiguous().view(-1)
    kc2 = torch.full((B * rows * kv,), 7.0, device=dev)
    vc2 = torch.full((B * rows * kv,), 7.0, device=dev)
    print("[batched] qkv heads unfused", flush=True)
    K.head_rms_norm_rope_kv(q2, k2, v2, c["qw_t"], c["kw_t"], c["rope"], c["pos_t"], 0, B, NQ, NK, HD, 1e-6,
                            kc2, vc2, rows)
    torch.cuda.synchronize()
    assert torch.equal(q.isnan(), q2.isnan())
    assert torch.equal(torch.nan_to_num(q, 0.0), torch.nan_to_num(q2, 0.0))
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    qn = q.view(B, NQ * HD).cpu().numpy()
    assert np.isnan(qn[3]).all() and np.isnan(qn[20]).all() and not np.isnan(np.delete(qn, [3, 20], 0)).any()
    # exactly the valid streams' rows were written
    written = (kc.view(B, rows, kv) != 7.0).any(dim=2).cpu().numpy()
    want = np.zeros((B, rows), bool)
    for b, p in enumerate(c["pos"]):
        if 0 <= p < rows:
            want[b, p] = True
    np.testing.assert_array_equal(written, want)


@pytest.mark.parametrize("in_dim", [2048, 1024])
def test_qkv_heads_matches_oracle_at_c5_shape(dev, in_dim):
    """256 streams at positions U[0, 2047] (the batched-decode config) against
    the oracle: linear_w8a8, then head_rms_norm_rope with per-stream positions;
    q rows and the K/V cache rows at each position, rel/abs 1e-5."""
    B, rows = 256, 2048
    c = _qkv_case(dev, B, in_dim, rows, [53, in_dim])
    print(f"[batched] qkv heads B={B} K={in_dim}", flush=True)
    q, kc, vc = _run_fused(dev, c, B, in_dim, rows)
    torch.cuda.synchronize()
    N, kv = (NQ + 2 * NK) * HD, NK * HD
    y, _ = oracle.linear_w8a8(c["wq"], c["ws"], c["xq"], c["xs"], B, in_dim, N)
    y = y.reshape(B, N)
    cos, sin = oracle.rope_table(c["rope"].cap, HD, 1e6)
    qr, kr = oracle.head_rms_norm_rope(y[:, :NQ * HD].ravel(), y[:, NQ * HD:(NQ + NK) * HD].ravel(), c["qw"],
                                       c["kw"], cos, sin, c["pos"], B, NQ, NK, HD, 1e-6)
    assert_close(q.cpu().numpy(), qr, 1e-5, 1e-5, "q")
    idx = torch.from_numpy(np.arange(B) * rows + c["pos"].astype(np.int64)).to(dev)
    k_rows = kc.view(B * rows, kv)[idx].cpu().numpy()
    v_rows = vc.view(B * rows, kv)[idx].cpu().numpy()
    assert_close(k_rows, kr.reshape(B, kv), 1e-5, 1e-5, "k rows")
    np.testing.assert_array_equal(v_rows, y[:, (NQ + NK) * HD:])  # v: the dequantized rows, no rounding step


def test_batched_projection_rejects_unsupported_shapes(dev):
    from qwenasr_amd import _lib
    from qwenasr_amd import kernels as K

    r = np.random.default_rng(54)
    wq, ws = _quant_rows(r, 128, 1024, 0.02)
    w = _packed(dev, wq, ws)
    xq = torch.zeros(1024 * 4, dtype=torch.int8, device=dev)
    xs = torch.ones(4, device=dev)
    y = torch.empty(4 * 128, device=dev)
    with pytest.raises(_lib.QasrError) as e:  # in_dim 1536: no kernel (rejected before any launch)
        w1536 = K.QuantWeight(torch.zeros(128 * 1536, dtype=torch.int8, device=dev), w.scales, 128, 1536)
        K.linear_w8a8_packed(y, w1536, torch.zeros(1536 * 4, dtype=torch.int8, device=dev), xs, 4, 1536, 128)
    assert e.value.code == _lib.QASR_ERR_UNSUPPORTED
    with pytest.raises(_lib.QasrError) as e:  # out_dim not a multiple of 128
        K.linear_w8a8_packed(y, K.QuantWeight(w.data, w.scales, 64, 1024), xq, xs, 4, 1024, 64)
    assert e.value.code == _lib.QASR_ERR_UNSUPPORTED
    torch.cuda.synchronize()


@pytest.mark.parametrize("H,I,B,chunked", [(2048, 6144, 9, None), (1024, 3072, 3, None), (1024, 3072, 9, False)])
def test_batched_decode_step_matches_the_oracle_per_stream(tmp_path, dev, H, I, B, chunked):
    """DecoderInt8Batched (B streams, each at its own position over its own
    cache) against the oracle's decode step (decoder.rs:848-965) run stream
    by stream: final hidden state, logits, the new K/V rows of every layer and
    the token, over two consecutive steps. B = 9 takes the matrix-core paths
    (8+ rows), B = 3 the per-row ones; the attention with its keys cut into
    chunks (the small-batch default) and walked whole (the large-batch one),
    both in longest-first order. Tolerance as for the single-stream decode
    step (chained kernels, rel/abs 1e-4)."""
    from oracle.decoder import decode_int8_step
    from qwenasr_amd.decoder import DecoderInt8Batched
    from tests.test_decoder_step import _load
    from tests.test_oracle import small_decoder

    L, vocab, rows, TOL = 2, 1000, 2100, 1e-4
    r = np.random.default_rng([55, H, B])
    w = small_decoder(r, H, I, L, NQ, NK, HD, vocab)
    dec = DecoderInt8Batched(_load(tmp_path, w, L, dev), H, I, L, B, rows, device=dev, attn_chunked=chunked)
    kv = NK * HD
    pos = np.array([0, 1500, 7, 64, 2100 - 3, 1, 510, 255, 1023][:B], np.int32)  # 1-5 key chunks
    kc = r.standard_normal((B, L, rows, kv)).astype(np.float32)  # earlier contexts, one per stream
    vc = r.standard_normal((B, L, rows, kv)).astype(np.float32)
    for l in range(L):
        dec.k[l].view(B, rows, kv).copy_(torch.from_numpy(kc[:, l].copy()))
        dec.v[l].view(B, rows, kv).copy_(torch.from_numpy(vc[:, l].copy()))
    dec.positions.copy_(torch.from_numpy(pos))
    for step in range(2):
        x = r.standard_normal((B, H)).astype(np.float32)
        print(f"[batched] decode step {step} H={H} B={B}", flush=True)
        dec.decode(torch.from_numpy(x.ravel().copy()).to(dev))
        torch.cuda.synchronize()
        xn = dec.x_norm.view(B, H).cpu().numpy()
        lg = dec.logits.view(B, vocab).cpu().numpy()
        tok = dec.tokens.cpu().numpy()
        for m in range(B):
            p = int(pos[m]) + step
            t_ref, xn_ref, lg_ref = decode_int8_step(w, kc[m], vc[m], p, x[m], NQ, NK, HD, threads=8)
            np.testing.assert_allclose(xn[m], xn_ref, rtol=TOL, atol=TOL, err_msg=f"stream {m} step {step}")
            np.testing.assert_allclose(lg[m], lg_ref, rtol=TOL, atol=TOL, err_msg=f"stream {m} step {step}")
            for l in range(L):
                kg = dec.k[l].view(B, rows, kv)[m, p].cpu().numpy()
                vg = dec.v[l].view(B, rows, kv)[m, p].cpu().numpy()
                np.testing.assert_allclose(kg, kc[m, l, p], rtol=TOL, atol=TOL, err_msg=f"k stream {m} layer {l}")
                np.testing.assert_allclose(vg, vc[m, l, p], rtol=TOL, atol=TOL, err_msg=f"v stream {m} layer {l}")
            top2 = np.sort(lg_ref)[-2:]
            if top2[1] - top2[0] > 2 * TOL * (1 + abs(top2[1])):
                assert int(tok[m]) == t_ref, (m, step)
        dec.finish()
    assert torch.equal(dec.positions.cpu(), torch.from_numpy(pos + 2))


@pytest.mark.parametrize("w8a8", [False, True])
def test_batched_decode_step_at_the_benchmarked_size_matches_the_oracle(dev, monkeypatch, w8a8):
    """The 256-stream steps that bench.py times (1.7B shapes: hidden 2048, 28
    layers, vocabulary 151936; the reference's W8A32 arithmetic, and the W8A8
    form with its W8A8 lm_head) against the oracle's decode step
    (decoder.rs:848-965; W8A8: oracle.decoder.decode_w8a8_step with the
    device's rounding adopted at near-ties as in the small-batch W8A8 test, at
    most one element per rounding point on average) for four of its streams, at
    positions 0, 511, 512 and 639 (one key; one whole 512-key chunk; one key
    into a second chunk; the last cache row), the other 252 streams at random
    positions: the final hidden state at rel/abs 1e-4 as in the small-batch
    test, the token, and all 151936 logits and the new K/V rows of all 28
    layers at rel 1e-4 + abs 1e-4 x the RMS of their row (the logits, one
    layer's K or V row): each is a dot product whose error is bounded by its
    weight row's norm times the error of the normed state it reads (which 28
    chained layers bring to ~1e-5 relative), not by its own value, which
    cancels to near 0 for some elements. Each stream's cache holds 640 rows here (2048, as in the
    benchmark, would take 120 GB of device memory for the same kernels and
    launch shapes)."""
    from oracle.decoder import decode_int8_step, decode_w8a8_step
    from qwenasr_amd import kernels as K
    from qwenasr_amd.decoder import DecoderInt8Batched

    H, I, L, B, rows, vocab, TOL = 2048, 6144, 28, 256, 640, 151936, 1e-4
    kv = NK * HD
    gen = torch.Generator(device=dev).manual_seed(71)

    def randn(n, scale=1.0, mean=0.0):
        return torch.randn(n, generator=gen, device=dev) * scale + mean

    def qw(o, i):
        q = torch.randint(-127, 128, (o * i,), generator=gen, device=dev, dtype=torch.int8)
        return K.QuantWeight(q, randn(o, 1e-4, 1e-3).abs_(), o, i)

    print("[batched full size] weights", flush=True)
    layers = [{"wq": qw(NQ * HD, H), "wk": qw(kv, H), "wv": qw(kv, H), "wo": qw(H, NQ * HD),
               "gate_up": qw(2 * I, H), "down": qw(H, I), "q_norm": randn(HD, 0.1, 1.0), "k_norm": randn(HD, 0.1, 1.0),
               "input_norm": randn(H, 0.1, 1.0), "post_attn_norm": randn(H, 0.1, 1.0)} for _ in range(L)]
    weights = {"layers": layers, "norm": randn(H, 0.1, 1.0), "lm_head": qw(vocab, H)}
    dec = DecoderInt8Batched(weights, H, I, L, B, rows, device=dev, w8a8=w8a8)
    assert dec.lm_head_w8a8 == w8a8
    for l in range(L):
        dec.k[l].normal_(generator=gen)
        dec.v[l].normal_(generator=gen)
    pos = torch.randint(0, rows, (B,), generator=gen, dtype=torch.int32, device=dev).cpu().numpy()
    sampled = {0: 0, 97: 511, 180: 512, 255: rows - 1}
    for m, p in sampled.items():
        pos[m] = p
    dec.positions.copy_(torch.from_numpy(pos))
    x = randn(B * H)
    if w8a8:
        rec = _RoundingRecorder(monkeypatch, K)
    print(f"[batched full size] device step w8a8={w8a8}", flush=True)
    dec.decode(x)
    torch.cuda.synchronize()
    if w8a8:
        points = 4 * L + 1
        assert len(rec.seen) == points
        gq, gs = [q for q, _ in rec.seen], [sc for _, sc in rec.seen]
    xn = dec.x_norm.view(B, H).cpu().numpy()
    lg = dec.logits.view(B, vocab).cpu().numpy()
    tok = dec.tokens.cpu().numpy()
    xh = x.view(B, H).cpu().numpy()

    def host(w):
        return (w.data.view(w.out_dim, w.in_dim).cpu().numpy(), w.scales.cpu().numpy())

    w_np = {"layers": [{k: host(v) if isinstance(v, K.QuantWeight) else v.cpu().numpy() for k, v in lw.items()}
                       for lw in layers],
            "norm": weights["norm"].cpu().numpy(), "lm_head": host(weights["lm_head"])}
    for m, p in sampled.items():
        print(f"[batched full size] oracle stream {m} at position {p}", flush=True)
        kc = np.stack([dec.k[l].view(B, rows, kv)[m].cpu().numpy() for l in range(L)])
        vc = np.stack([dec.v[l].view(B, rows, kv)[m].cpu().numpy() for l in range(L)])
        k_dev, v_dev = kc[:, p].copy(), vc[:, p].copy()  # the step's new rows; the oracle rewrites them
        if w8a8:
            log = []
            kc32, vc32 = kc.copy(), vc.copy()
            t_ref, xn_ref, lg_ref = decode_w8a8_step(w_np, kc, vc, p, xh[m], NQ, NK, HD, threads=16,
                                                     quant=_steered_quant(gq, gs, m, log), lm_head_w8a8=True)
            print(f"[batched full size] stream {m}: {sum(log)} roundings adopted over {points} points", flush=True)
            assert sum(log) <= points, log
            _, xn32, _ = decode_int8_step(w_np, kc32, vc32, p, xh[m], NQ, NK, HD, threads=16)
            assert np.abs(xn32 - xn[m]).max() > 10 * TOL * (1 + np.abs(xn32).max())  # really rounded
        else:
            t_ref, xn_ref, lg_ref = decode_int8_step(w_np, kc, vc, p, xh[m], NQ, NK, HD, threads=16)
        np.testing.assert_allclose(xn[m], xn_ref, rtol=TOL, atol=TOL, err_msg=f"stream {m}")
        for got, ref, what in ((lg[m][None], lg_ref[None], "logits"), (k_dev, kc[:, p], "k rows"),
                               (v_dev, vc[:, p], "v rows")):
            rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=1, keepdims=True))
            err = np.abs(got.astype(np.float64) - ref)
            print(f"[batched full size] stream {m} {what}: max |diff| / row RMS {(err / rms).max():.3g}", flush=True)
            assert (err <= TOL * np.abs(ref) + TOL * rms).all(), f"{what} stream {m}"
        top2 = np.sort(lg_ref)[-2:]
        if top2[1] - top2[0] > 2 * TOL * (1 + abs(top2[1])):
            assert int(tok[m]) == t_ref, m


class _RoundingRecorder:
    """Keeps a copy of every per-row int8 activation (values and scales) that
    the device computes through K.add_rms_norm_quant, K.quantize_rows_i8 and
    the quantized form of K.batched_decode_attention."""

    # entry point -> positions of (q, scales, rows) among its arguments
    WHERE = {"add_rms_norm_quant": (4, 5, 6), "quantize_rows_i8": (0, 1, 3), "batched_decode_attention": (12, 13, 6)}

    def __init__(self, monkeypatch, K):
        self.seen = []
        for name, (iq, isc, irows) in self.WHERE.items():
            orig = getattr(K, name)

            def wrap(*a, _orig=orig, _iq=iq, _isc=isc, _irows=irows):
                _orig(*a)
                if len(a) > _isc and a[_iq] is not None:
                    q, sc, rows = a[_iq], a[_isc], a[_irows]
                    self.seen.append((q.view(rows, -1).cpu().numpy().copy(), sc[:rows].cpu().numpy().copy()))

            monkeypatch.setattr(K, name, wrap)


def _steered_quant(gpu_q, gpu_s, stream, log):
    """The oracle's per-row quantizer, except that where its value lies within
    1e-3 of a rounding boundary (|x*127/absmax| ~ n + 0.5) and the device
    rounded the other way it takes the device's choice (and its scale, if the
    scales differ by no more than 1e-6 relative). Anything else that differs is
    left as the oracle computes it, so a real error still shows."""
    it = iter(range(len(gpu_q)))

    def quant(x, n):
        i = next(it)
        q, s = oracle.quantize_f32_to_int8(x, 1, n)
        gq, gs = gpu_q[i][stream], gpu_s[i][stream]
        a = float(np.abs(x).max())
        v = np.asarray(x, np.float64) * (127.0 / a) if a > 0 else np.zeros(n)
        near = np.abs(np.abs(v) - np.floor(np.abs(v)) - 0.5) < 1e-3
        take = near & (np.abs(q.astype(np.int32) - gq.astype(np.int32)) == 1)
        q = np.where(take, gq, q).astype(np.int8)
        log.append(int(take.sum()))
        if abs(float(gs) - float(s[0])) <= 1e-6 * abs(float(s[0])):
            s = np.array([gs], np.float32)
        return q, s

    return quant


@pytest.mark.parametrize("H,I,B,vocab", [(2048, 6144, 9, 1000), (1024, 3072, 3, 1024)])
def test_batched_w8a8_decode_step_matches_the_oracle_per_stream(tmp_path, dev, monkeypatch, H, I, B, vocab):
    """DecoderInt8Batched(w8a8=True) against the oracle's W8A8 decode step run
    stream by stream, over two steps. The integer dots are exact, but the
    device's RMSNorm and attention rows differ from the oracle's in the last
    bits, so an activation that lies within ~1e-6 of a rounding boundary can
    round to the neighbouring int8 value; with these weights one such flip
    moves the final hidden state by up to ~2%. So the device's int8
    activations are recorded, the oracle adopts the device's rounding only at
    elements within 1e-3 of a boundary (at most 4 per stream and step), and
    then the final hidden state, logits, new K/V rows and token must match at
    rel/abs 1e-4 as in the W8A32 step. The final hidden state must also differ
    from the W8A32 step's (the rounding is really done at the four points).
    With a vocabulary of 1024 the lm_head is W8A8 as well (a fifth rounding
    point, the final norm), with 1000 it stays W8A32."""
    from oracle.decoder import decode_int8_step, decode_w8a8_step
    from qwenasr_amd import kernels as K
    from qwenasr_amd.decoder import DecoderInt8Batched
    from tests.test_decoder_step import _load
    from tests.test_oracle import small_decoder

    L, rows, TOL = 2, 2100, 1e-4
    r = np.random.default_rng([57, H, B])
    w = small_decoder(r, H, I, L, NQ, NK, HD, vocab)
    dec = DecoderInt8Batched(_load(tmp_path, w, L, dev), H, I, L, B, rows, device=dev, w8a8=True)
    kv = NK * HD
    pos = np.array([0, 1500, 7, 64, 2100 - 3, 1, 510, 255, 1023][:B], np.int32)  # 1-5 key chunks
    kc = r.standard_normal((B, L, rows, kv)).astype(np.float32)
    vc = r.standard_normal((B, L, rows, kv)).astype(np.float32)
    kc32, vc32 = kc.copy(), vc.copy()
    for l in range(L):
        dec.k[l].view(B, rows, kv).copy_(torch.from_numpy(kc[:, l].copy()))
        dec.v[l].view(B, rows, kv).copy_(torch.from_numpy(vc[:, l].copy()))
    dec.positions.copy_(torch.from_numpy(pos))
    rec = _RoundingRecorder(monkeypatch, K)
    adopted = []
    for step in range(2):
        x = r.standard_normal((B, H)).astype(np.float32)
        print(f"[batched w8a8] decode step {step} H={H} B={B}", flush=True)
        rec.seen.clear()
        dec.decode(torch.from_numpy(x.ravel().copy()).to(dev))
        torch.cuda.synchronize()
        assert dec.lm_head_w8a8 == (vocab % 128 == 0)
        assert len(rec.seen) == 4 * L + int(dec.lm_head_w8a8)
        gq, gs = [q for q, _ in rec.seen], [s for _, s in rec.seen]
        xn = dec.x_norm.view(B, H).cpu().numpy()
        lg = dec.logits.view(B, vocab).cpu().numpy()
        tok = dec.tokens.cpu().numpy()
        for m in range(B):
            p = int(pos[m]) + step
            log = []
            t_ref, xn_ref, lg_ref = decode_w8a8_step(w, kc[m], vc[m], p, x[m], NQ, NK, HD, threads=8,
                                                     quant=_steered_quant(gq, gs, m, log),
                                                     lm_head_w8a8=dec.lm_head_w8a8)
            adopted.append(sum(log))
            assert sum(log) <= 4, (m, step, log)
            msg = f"stream {m} step {step} adopted {log}"
            np.testing.assert_allclose(xn[m], xn_ref, rtol=TOL, atol=TOL, err_msg=msg)
            np.testing.assert_allclose(lg[m], lg_ref, rtol=TOL, atol=TOL, err_msg=msg)
            for l in range(L):
                kg = dec.k[l].view(B, rows, kv)[m, p].cpu().numpy()
                vg = dec.v[l].view(B, rows, kv)[m, p].cpu().numpy()
                np.testing.assert_allclose(kg, kc[m, l, p], rtol=TOL, atol=TOL, err_msg=msg)
                np.testing.assert_allclose(vg, vc[m, l, p], rtol=TOL, atol=TOL, err_msg=msg)
            _, xn32, _ = decode_int8_step(w, kc32[m], vc32[m], p, x[m], NQ, NK, HD, threads=8)
            assert np.abs(xn32 - xn[m]).max() > 10 * TOL * (1 + np.abs(xn32).max()), msg
            top2 = np.sort(lg_ref)[-2:]
            if top2[1] - top2[0] > 2 * TOL * (1 + abs(top2[1])):
                assert int(tok[m]) == t_ref, (m, step)
        dec.finish()
    print(f"[batched w8a8] roundings adopted from the device per stream and step: {adopted}", flush=True)
    assert torch.equal(dec.positions.cpu(), torch.from_numpy(pos + 2))


@pytest.mark.parametrize("w8a8,chunked", [(False, True), (True, True), (False, False), (True, False)])
def test_batched_decode_step_graph_replay_equals_eager(tmp_path, dev, w8a8, chunked):
    """One batched decode step (both forms) captured in a HIP graph: every
    replay gives the eager step's hidden state, logits, tokens and new K/V
    rows bit for bit, with eager work and synchronisations between replays
    (the step rewrites the same cache rows while positions stay put)."""
    from qwenasr_amd.decoder import DecoderInt8Batched
    from tests.test_decoder_step import _load
    from tests.test_oracle import small_decoder

    H, I, L, B, rows = 1024, 3072, 2, 12, 1300
    vocab = 1024 if w8a8 else 1000  # the W8A8 form then has the W8A8 lm_head too
    r = np.random.default_rng([58, int(w8a8)])
    w = small_decoder(r, H, I, L, NQ, NK, HD, vocab)
    dec = DecoderInt8Batched(_load(tmp_path, w, L, dev), H, I, L, B, rows, device=dev, w8a8=w8a8,
                             attn_chunked=chunked)
    assert dec.lm_head_w8a8 == w8a8
    for l in range(L):
        dec.k[l].normal_()
        dec.v[l].normal_()
    dec.positions.copy_(torch.from_numpy(r.integers(0, rows, B).astype(np.int32)))
    emb = torch.from_numpy(r.standard_normal(B * H).astype(np.float32)).to(dev)
    kv = NK * HD
    pos = dec.positions.long().cpu()

    def outputs():
        kr = [dec.k[l].view(B, rows, kv)[torch.arange(B), pos].clone() for l in range(L)]
        vr = [dec.v[l].view(B, rows, kv)[torch.arange(B), pos].clone() for l in range(L)]
        return [dec.x_norm.clone(), dec.logits.clone(), dec.tokens.clone()] + kr + vr

    print(f"[batched] graph replay w8a8={w8a8}", flush=True)
    dec.decode(emb)
    torch.cuda.synchronize()
    ref = outputs()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dec.decode(emb)
    for rep in range(3):
        dec.x_norm.fill_(0.0)
        dec.logits.fill_(0.0)
        dec.tokens.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outputs(), ref)):
            assert torch.equal(a, b), (rep, i)


@pytest.mark.parametrize("B", [7, 300, 1500])
def test_batched_decode_order_and_ordered_attention(dev, B):
    """The longest-first order: a permutation of the streams sorted by number
    of keys (position + 1, 0 outside the cache) descending, ties by stream,
    against numpy; attention walked in that order equals the stream-order
    call bit for bit (each stream's work is the same, only its workgroup
    differs), chunked and not, with the quantized rows too."""
    from qwenasr_amd import kernels as K

    rows = 700
    r = np.random.default_rng([61, B])
    pos = r.integers(0, rows, B).astype(np.int32)
    pos[: min(B, 4)] = [5, 5, rows, -3][: min(B, 4)]  # a tie and two positions outside the cache
    keys = np.where((pos >= 0) & (pos < rows), pos + 1, 0)
    want = sorted(range(B), key=lambda i: (-int(keys[i]), i))
    order = torch.empty(2 * B, dtype=torch.int32, device=dev)
    pos_t = torch.from_numpy(pos).to(dev)
    print(f"[batched] order B={B}", flush=True)
    K.batched_decode_order(order, pos_t, B, rows)
    torch.cuda.synchronize()
    o = order.view(B, 2).cpu().numpy()
    np.testing.assert_array_equal(o[:, 0], want)
    np.testing.assert_array_equal(o[:, 1], pos[want])
    if B > 300:
        return  # the ranking at a larger batch; the attention below at two sizes
    nq, nk, hd = 16, 8, 128
    kv = nk * hd
    q = torch.from_numpy(r.standard_normal(B * nq * hd).astype(np.float32)).to(dev)
    kc = torch.from_numpy(r.standard_normal(B * rows * kv).astype(np.float32)).to(dev)
    vc = torch.from_numpy(r.standard_normal(B * rows * kv).astype(np.float32)).to(dev)
    for ws in (None, K.batched_decode_workspace(B, nq, hd, rows, dev)):
        outs = []
        for od in (None, order):
            out = torch.empty(B * nq * hd, device=dev)
            oq = torch.empty(B * nq * hd, dtype=torch.int8, device=dev)
            osc = torch.empty(B, device=dev)
            K.batched_decode_attention(out, q, kc, vc, rows, pos_t, B, nq, nk, hd, hd ** -0.5, ws, oq, osc, od)
            outs.append((out, oq, osc))
        torch.cuda.synchronize()
        (a, aq, asc), (b, bq, bsc) = outs
        assert torch.equal(a.isnan(), b.isnan()) and torch.equal(a.nan_to_num(), b.nan_to_num())
        assert torch.equal(aq, bq) and torch.equal(asc, bsc)


def test_stale_order_gives_nan_rows(dev):
    """An order computed for other positions than the call's (the positions
    advanced after it was made): the streams whose position changed get NaN
    rows, whether their chunk count grew, shrank or stayed; the other streams
    equal the stream-order call bit for bit. Chunked and not, with the
    quantized rows too."""
    from qwenasr_amd import kernels as K

    B, rows, nq, nk, hd = 7, 700, 16, 8, 128
    kv = nk * hd
    r = np.random.default_rng(62)
    old = np.array([5, 100, 650, 300, 20, 511, 512], np.int32)
    new = old.copy()
    new[1], new[2], new[4] = 650, 50, 21  # 1 -> 2 chunks, 2 -> 1 chunk, same chunk but one more key
    changed = new != old
    d = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    q = d(r.standard_normal(B * nq * hd).astype(np.float32))
    kc = d(r.standard_normal(B * rows * kv).astype(np.float32))
    vc = d(r.standard_normal(B * rows * kv).astype(np.float32))
    order = torch.empty(2 * B, dtype=torch.int32, device=dev)
    K.batched_decode_order(order, d(old), B, rows)
    pos_new = d(new)
    for ws in (None, K.batched_decode_workspace(B, nq, hd, rows, dev)):
        print(f"[batched] stale order, chunked={ws is not None}", flush=True)
        ref = torch.empty(B * nq * hd, device=dev)
        K.batched_decode_attention(ref, q, kc, vc, rows, pos_new, B, nq, nk, hd, hd ** -0.5, ws)
        for quant in (False, True):
            out = torch.zeros(B * nq * hd, device=dev)
            oq = torch.empty(B * nq * hd, dtype=torch.int8, device=dev) if quant else None
            osc = torch.empty(B, device=dev) if quant else None
            K.batched_decode_attention(out, q, kc, vc, rows, pos_new, B, nq, nk, hd, hd ** -0.5, ws, oq, osc,
                                       order)
            torch.cuda.synchronize()
            got, want = out.view(B, -1).cpu().numpy(), ref.view(B, -1).cpu().numpy()
            for m in range(B):
                if changed[m]:
                    assert np.isnan(got[m]).all(), (m, ws is not None, quant)
                else:
                    np.testing.assert_array_equal(got[m], want[m])


@pytest.mark.parametrize("nq,nk,hd,rows", [(16, 8, 128, 1300), (16, 8, 128, 400), (8, 8, 128, 1300),
                                           (4, 4, 64, 700)])
def test_batched_decode_attention_quantized_rows(dev, nq, nk, hd, rows):
    """The quantized form: out as without it, and out_q / out_scales equal to
    quantize_rows_i8 on out bit for bit -- rows merged from several chunks,
    rows of one chunk, a NaN row for a position outside the cache, fewer than
    16 heads (fewer waves in the merge workgroup), chunked and not."""
    from qwenasr_amd import kernels as K

    B, kv = 6, nk * hd
    r = np.random.default_rng([60, nq, rows])
    d = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    q = d(r.standard_normal(B * nq * hd).astype(np.float32))
    kc = d(r.standard_normal(B * rows * kv).astype(np.float32))
    vc = d(r.standard_normal(B * rows * kv).astype(np.float32))
    pos = d(np.array([0, rows - 1, rows, rows // 2, 511, 512], np.int32))
    for ws in (None, K.batched_decode_workspace(B, nq, hd, rows, dev)):
        plain = torch.empty(B * nq * hd, device=dev)
        K.batched_decode_attention(plain, q, kc, vc, rows, pos, B, nq, nk, hd, hd ** -0.5, ws)
        out = torch.empty(B * nq * hd, device=dev)
        oq = torch.full((B * nq * hd,), 99, dtype=torch.int8, device=dev)
        osc = torch.full((B,), -1.0, device=dev)
        print(f"[batched] attention quantized nq={nq} rows={rows} chunked={ws is not None}", flush=True)
        K.batched_decode_attention(out, q, kc, vc, rows, pos, B, nq, nk, hd, hd ** -0.5, ws, oq, osc)
        rq = torch.empty_like(oq)
        rs = torch.empty_like(osc)
        K.quantize_rows_i8(rq, rs, out, B, nq * hd)
        torch.cuda.synchronize()
        assert torch.equal(out.isnan(), plain.isnan()) and torch.equal(out.nan_to_num(), plain.nan_to_num())
        assert out.view(B, -1)[2].isnan().all()
        assert torch.equal(oq, rq) and torch.equal(osc, rs)


@pytest.mark.parametrize("nq,nk,hd", [(8, 8, 128), (4, 4, 64), (8, 4, 64), (16, 4, 64)])
def test_batched_decode_attention_other_head_shapes(dev, nq, nk, hd):
    """The other head shapes the batched attention takes (G = 1 at head_dim
    128; G = 1, 2, 4 at head_dim 64), chunked (1100 rows, workspace) and not,
    against the oracle at 1e-5."""
    from qwenasr_amd import kernels as K

    B, rows, kv = 5, 1100, nk * hd
    r = np.random.default_rng([59, nq, nk, hd])
    q = r.standard_normal(B * nq * hd).astype(np.float32)
    kc = r.standard_normal(B * rows * kv).astype(np.float32)
    vc = r.standard_normal(B * rows * kv).astype(np.float32)
    pos = np.array([0, 1099, 511, 512, 777], np.int32)
    d = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    kn, vn = kc.reshape(B, rows, kv), vc.reshape(B, rows, kv)
    for ws in (None, K.batched_decode_workspace(B, nq, hd, rows, dev)):
        out = torch.empty(B * nq * hd, device=dev)
        print(f"[batched] attention nq={nq} nk={nk} hd={hd} chunked={ws is not None}", flush=True)
        K.batched_decode_attention(out, d(q), d(kc), d(vc), rows, d(pos), B, nq, nk, hd, hd ** -0.5, ws)
        torch.cuda.synchronize()
        o = out.view(B, -1).cpu().numpy()
        for m in range(B):
            p = int(pos[m])
            ref = oracle.causal_attention(q.reshape(B, -1)[m], kn[m, :p + 1].ravel(), vn[m, :p + 1].ravel(), 1,
                                          p + 1, nq, nk, hd, hd ** -0.5, p)
            assert_close(o[m], ref, 1e-5, 1e-5, f"stream {m} at {p}, chunked {ws is not None}")


@pytest.mark.parametrize("rows", [300, 2300])
def test_batched_decode_attention_bad_position_and_graph_replay(dev, rows):
    """Streams at positions across 1-5 key chunks (chunks of 512; 300 rows:
    one chunk, no workspace needed) against the oracle, with and without the
    workspace (chunked and one-workgroup-per-stream forms); a stream at a
    position outside its cache gets a NaN row (the others are unaffected);
    the call captured in a HIP graph gives the eager result on every replay."""
    from qwenasr_amd import _lib
    from qwenasr_amd import kernels as K

    B, kv = 8, NK * HD
    r = np.random.default_rng([56, rows])
    q = torch.from_numpy(r.standard_normal(B * NQ * HD).astype(np.float32)).to(dev)
    kc = torch.from_numpy(r.standard_normal(B * rows * kv).astype(np.float32)).to(dev)
    vc = torch.from_numpy(r.standard_normal(B * rows * kv).astype(np.float32)).to(dev)
    good = [0, rows - 1, rows // 2, 64] + ([1023, 1024, 2048] if rows > 2048 else [5, 100, 200])
    pos_l = good[:2] + [rows, -1] + good[2:6]
    pos = torch.tensor(pos_l, dtype=torch.int32, device=dev)
    ws = K.batched_decode_workspace(B, NQ, HD, rows, dev)
    assert (ws is None) == (rows <= 512)
    if ws is not None:
        with pytest.raises(_lib.QasrError):  # too small a workspace is an error, not a silent fallback
            K.batched_decode_attention(torch.empty(B * NQ * HD, device=dev), q, kc, vc, rows, pos, B, NQ, NK, HD,
                                       HD ** -0.5, ws[:ws.numel() - 1])
    qn, kn, vn = q.cpu().numpy(), kc.cpu().numpy().reshape(B, rows, kv), vc.cpu().numpy().reshape(B, rows, kv)
    outs = []
    for w in (None, ws):
        out = torch.empty(B * NQ * HD, device=dev)
        K.batched_decode_attention(out, q, kc, vc, rows, pos, B, NQ, NK, HD, HD ** -0.5, w)
        torch.cuda.synchronize()
        o = out.view(B, NQ * HD).cpu().numpy()
        assert np.isnan(o[2]).all() and np.isnan(o[3]).all()
        for m in (0, 1, 4, 5, 6, 7):
            p = pos_l[m]
            ref = oracle.causal_attention(qn.reshape(B, -1)[m], kn[m, :p + 1].ravel(), vn[m, :p + 1].ravel(), 1,
                                          p + 1, NQ, NK, HD, HD ** -0.5, p)
            assert_close(o[m], ref, 1e-5, 1e-5, f"stream {m} at {p}, workspace {w is not None}")
        outs.append(out)
    out, eager = outs[-1], outs[-1].clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.batched_decode_attention(out, q, kc, vc, rows, pos, B, NQ, NK, HD, HD ** -0.5, ws)
    for rep in range(3):
        out.fill_(0.0)
        if ws is not None:
            ws.fill_(7.0)  # the chunk partials are rewritten by every call
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.isnan(), eager.isnan()) and torch.equal(out.nan_to_num(), eager.nan_to_num()), rep
