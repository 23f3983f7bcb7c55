"""The whole INT8 decode step on the device (qwenasr_amd/decoder.py) against
the oracle's restatement of decoder.rs:848-965, with the weights going through
a .qint8 V2 file, the C-ABI reader, the device upload and the gate/up
interleave on the way.

Tolerance: each kernel holds rel/abs 1e-5; the step chains ~10 of them per
layer, each feeding the next, so the final hidden state, the logits and the
cache rows are compared at rel/abs 1e-4 (measured error is printed on
failure). The token must equal the oracle's whenever the oracle's top two
logits are further apart than the logit tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import qint8_format as fmt
from oracle.decoder import decode_int8_step, prefill_int8
from tests.test_oracle import small_decoder

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-4


def write_model(path, w, L):
    quant, f32 = [], []
    for i, lw in enumerate(w["layers"]):
        lp = f"thinker.model.layers.{i}"
        for n, key in (("self_attn.q_proj", "wq"), ("self_attn.k_proj", "wk"), ("self_attn.v_proj", "wv"),
                       ("self_attn.o_proj", "wo"), ("mlp.gate_proj", "gate"), ("mlp.up_proj", "up"),
                       ("mlp.down_proj", "down")):
            q, s = lw[key]
            quant.append((f"{lp}.{n}.weight", list(q.shape), q, s))
        for n, key in (("self_attn.q_norm", "q_norm"), ("self_attn.k_norm", "k_norm"),
                       ("input_layernorm", "input_norm"), ("post_attention_layernorm", "post_attn_norm")):
            f32.append((f"{lp}.{n}.weight", [lw[key].size], lw[key]))
    q, s = w["lm_head"]
    quant.append(("thinker.lm_head.weight", list(q.shape), q, s))
    quant.append(("thinker.model.embed_tokens.weight", list(q.shape), q, s))
    f32.append(("thinker.model.norm.weight", [w["norm"].size], w["norm"]))
    path.write_bytes(fmt.write_v2(quant, f32, []))


@pytest.mark.parametrize("H,I,vocab", [(1024, 3072, 3000), (2048, 6144, 1000)])
def test_decode_steps_match_the_oracle(tmp_path, dev, H, I, vocab):
    from qwenasr_amd import qint8
    from qwenasr_amd.decoder import DecoderInt8

    L, nq, nk, hd, n_pos = 2, 16, 8, 128, 5
    r = np.random.default_rng([31, H])
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    p = tmp_path / "model.qint8"
    write_model(p, w, L)
    with qint8.QuantFile.open(str(p)) as qf:
        dims = qint8.detect_decoder_dims(qf)
        assert (dims.hidden, dims.intermediate, dims.lm_head_dim) == (H, I, vocab)
        dims.n_layers = L
        weights = qint8.load_decoder_int8(qf, dims, dev)
    dec = DecoderInt8(weights, H, I, L, nq, nk, hd, max_seq=4, device=dev)
    kc = np.zeros((L, 16, nk * hd), np.float32)
    vc = np.zeros_like(kc)
    for pos in range(n_pos):  # the cache grows past its first 4 rows at pos 4
        x = r.standard_normal(H).astype(np.float32)
        tok, xn, logits = decode_int8_step(w, kc, vc, pos, x, nq, nk, hd, threads=8)
        dec.prepare(pos)
        dec.decode(torch.from_numpy(x).to(dev), pos)
        dec.finish(pos)
        torch.cuda.synchronize()
        np.testing.assert_allclose(dec.x_norm.cpu().numpy(), xn, rtol=TOL, atol=TOL)
        np.testing.assert_allclose(dec.logits.cpu().numpy(), logits, rtol=TOL, atol=TOL)
        kv = nk * hd
        for l in range(L):
            kg = dec.kv.k_layer(l).cpu().numpy().reshape(pos + 1, kv)
            vg = dec.kv.v_layer(l).cpu().numpy().reshape(pos + 1, kv)
            np.testing.assert_allclose(kg, kc[l, :pos + 1], rtol=TOL, atol=TOL)
            np.testing.assert_allclose(vg, vc[l, :pos + 1], rtol=TOL, atol=TOL)
        top2 = np.sort(logits)[-2:]
        got = int(dec.token.cpu().numpy()[0])
        assert got == int(oracle.argmax_rows(dec.logits.cpu().numpy(), 1, vocab)[0])
        if top2[1] - top2[0] > 2 * TOL * (1 + abs(top2[1])):
            assert got == tok, (pos, got, tok)


def test_fused_decode_at_split_positions_matches_the_oracle(tmp_path, dev):
    """The timed decode path (fuse_norms=True: norms folded into the
    projections, q/k norm + RoPE + cache store folded into split attention)
    against the oracle at positions 300-302, where the keys are split over
    workgroups: the final hidden state, the logits, the new K/V rows of every
    layer and the token, over a cache whose rows 0..299 are the same random
    earlier context on both sides."""
    from qwenasr_amd.decoder import DecoderInt8

    H, I, L, nq, nk, hd, vocab = 2048, 6144, 2, 16, 8, 128, 1000
    r = np.random.default_rng([38, H])
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    dec = DecoderInt8(_load(tmp_path, w, L, dev), H, I, L, nq, nk, hd, max_seq=512, device=dev)
    assert dec.fuse_norms
    kv, start = nk * hd, 300
    kc = np.zeros((L, 512, kv), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :start] = r.standard_normal((L, start, kv)).astype(np.float32)
    vc[:, :start] = r.standard_normal((L, start, kv)).astype(np.float32)
    for l in range(L):
        dec.kv.k_layer_block(l).view(dec.kv.max_seq, kv)[:start] = torch.from_numpy(kc[l, :start]).to(dev)
        dec.kv.v_layer_block(l).view(dec.kv.max_seq, kv)[:start] = torch.from_numpy(vc[l, :start]).to(dev)
    dec.kv.len = start
    for pos in (start, start + 1, start + 2):
        x = r.standard_normal(H).astype(np.float32)
        tok, xn, logits = decode_int8_step(w, kc, vc, pos, x, nq, nk, hd, threads=8)
        dec.prepare()
        dec.decode(torch.from_numpy(x).to(dev))
        dec.finish()
        torch.cuda.synchronize()
        np.testing.assert_allclose(dec.x_norm.cpu().numpy(), xn, rtol=TOL, atol=TOL, err_msg=f"pos {pos}")
        np.testing.assert_allclose(dec.logits.cpu().numpy(), logits, rtol=TOL, atol=TOL, err_msg=f"pos {pos}")
        for l in range(L):
            np.testing.assert_allclose(dec.kv.k_layer(l).cpu().numpy().reshape(pos + 1, kv)[pos], kc[l, pos],
                                       rtol=TOL, atol=TOL, err_msg=f"k row {pos} layer {l}")
            np.testing.assert_allclose(dec.kv.v_layer(l).cpu().numpy().reshape(pos + 1, kv)[pos], vc[l, pos],
                                       rtol=TOL, atol=TOL, err_msg=f"v row {pos} layer {l}")
        top2 = np.sort(logits)[-2:]
        if top2[1] - top2[0] > 2 * TOL * (1 + abs(top2[1])):
            assert int(dec.token.cpu()[0]) == tok, pos


def test_decoder_position_must_be_the_cache_length(tmp_path, dev):
    """decoder.rs:771, 866 take the position from the cache length; the device
    decoder refuses any other (a later growth would drop the rows between)."""
    from qwenasr_amd.decoder import DecoderInt8

    H, I, L, nq, nk, hd, vocab = 1024, 3072, 1, 16, 8, 128, 100
    w = small_decoder(np.random.default_rng(39), H, I, L, nq, nk, hd, vocab)
    dec = DecoderInt8(_load(tmp_path, w, L, dev), H, I, L, nq, nk, hd, max_seq=8, device=dev)
    with pytest.raises(ValueError):
        dec.prepare(3)
    with pytest.raises(ValueError):
        dec.prepare_prefill(2, 4)
    with pytest.raises(ValueError):
        dec.finish(1)
    dec.prepare()  # position 0, from the cache length
    assert dec.kv.len == 0


def test_gate_up_swiglu_int8_matches_linear_plus_loop(dev):
    """The fused gate/up + SwiGLU entry against linear_nobias_int8 + the
    decode loop's SwiGLU on the oracle, one token (fused epilogue) and several
    tokens / off-vector shapes (pair kernel)."""
    from qwenasr_amd import kernels as K

    r = np.random.default_rng(32)
    for seq, H, I in ((1, 2048, 6144), (1, 1024, 3072), (1, 3072, 100), (3, 1024, 64), (1, 1000, 77)):
        wf = (0.02 * r.standard_normal((2 * I, H))).astype(np.float32)
        q, s = oracle.quantize_f32_to_int8(wf, 2 * I, H)
        x = r.standard_normal(seq * H).astype(np.float32)
        gu = oracle.linear_nobias_int8(x, q, s, seq, H, 2 * I).reshape(seq, 2 * I)
        ref = oracle.swiglu_split(gu[:, 0::2].ravel().copy(), gu[:, 1::2].ravel().copy())
        out = torch.full((seq * I,), 9.0, device=dev)
        w = K.QuantWeight(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), 2 * I, H)
        K.gate_up_swiglu_int8(out, torch.from_numpy(x).to(dev), w, seq, H, I)
        torch.cuda.synchronize()
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5, err_msg=f"{seq},{H},{I}")


def test_fused_norm_decode_equals_unfused(tmp_path, dev):
    """The decode step with the add + RMSNorm folded into the projections and
    the head norm + cache store folded into attention (fuse_norms=True)
    equals the unfused sequence bit for bit: hidden state, logits, token and
    cache rows, at positions where attention runs unsplit (0, 1) and split
    (300-302)."""
    from qwenasr_amd import qint8
    from qwenasr_amd.decoder import DecoderInt8

    H, I, L, nq, nk, hd, vocab = 2048, 6144, 2, 16, 8, 128, 1000
    r = np.random.default_rng([33, H])
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    p = tmp_path / "model.qint8"
    write_model(p, w, L)
    with qint8.QuantFile.open(str(p)) as qf:
        dims = qint8.detect_decoder_dims(qf)
        dims.n_layers = L
        weights = qint8.load_decoder_int8(qf, dims, dev)
    decs = [DecoderInt8(weights, H, I, L, nq, nk, hd, max_seq=512, device=dev, fuse_norms=f)
            for f in (True, False)]
    assert decs[0].fuse_norms and not decs[1].fuse_norms
    # an earlier context of 300 rows, so attention splits its keys (one fused launch)
    decs[0].kv.k.normal_()
    decs[0].kv.v.normal_()
    decs[1].kv.k.copy_(decs[0].kv.k)
    decs[1].kv.v.copy_(decs[0].kv.v)
    for pos in (0, 1, 300, 301, 302):
        x = torch.from_numpy(r.standard_normal(H).astype(np.float32)).to(dev)
        for d in decs:
            d.kv.len = pos  # rows 2..299 stand for an earlier context
            d.prepare(pos)
            d.decode(x, pos)
            d.finish(pos)
        torch.cuda.synchronize()
        for name in ("x_norm", "logits", "token"):
            np.testing.assert_array_equal(getattr(decs[0], name).cpu().numpy(),
                                          getattr(decs[1], name).cpu().numpy(), err_msg=f"{name} pos {pos}")
        for l in range(L):
            np.testing.assert_array_equal(decs[0].kv.k_layer(l).cpu().numpy(), decs[1].kv.k_layer(l).cpu().numpy())
            np.testing.assert_array_equal(decs[0].kv.v_layer(l).cpu().numpy(), decs[1].kv.v_layer(l).cpu().numpy())


@pytest.mark.parametrize("seq,H,I", [(512, 1024, 3072), (37, 1024, 3072), (100, 2048, 1000), (8, 1024, 100),
                                     (3, 1024, 64), (1, 1000, 77)])
def test_gate_up_swiglu_multiply_int8(dev, seq, H, I):
    """The prefill gate/up projection with the SwiGLU in its epilogue: from 8
    tokens (matrix-core GEMM; the 128x64 tile, a split-K tile, a row tail of
    the fast_exp columns) equal bit for bit to linear_nobias_int8 followed by
    swiglu_multiply; at every size within the fp32 tolerance of the oracle's
    linear + swiglu_multiply (kernels/mod.rs:965-985)."""
    from qwenasr_amd import kernels as K

    r = np.random.default_rng([36, seq, H, I])
    wf = (0.02 * r.standard_normal((2 * I, H))).astype(np.float32)
    q, s = oracle.quantize_f32_to_int8(wf, 2 * I, H)
    x = r.standard_normal(seq * H).astype(np.float32)
    w = K.QuantWeight(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), 2 * I, H)
    xt = torch.from_numpy(x).to(dev)
    gu = torch.empty(seq * 2 * I, device=dev)
    ref = torch.empty(seq * I, device=dev)
    K.linear_nobias_int8(gu, xt, w.data, w.scales, seq, H, 2 * I)
    K.swiglu_multiply(ref, gu, seq, I)
    out = torch.full((seq * I,), 9.0, device=dev)
    K.gate_up_swiglu_multiply_int8(out, xt, w, seq, H, I)
    torch.cuda.synchronize()
    if seq >= 8 and H % 64 == 0:
        np.testing.assert_array_equal(out.cpu().numpy(), ref.cpu().numpy())
    gu_ref = oracle.linear_nobias_int8(x, q, s, seq, H, 2 * I, n_threads=8)
    np.testing.assert_allclose(out.cpu().numpy(), oracle.swiglu_multiply(gu_ref, seq, I), rtol=1e-5, atol=1e-5)


def _load(tmp_path, w, L, dev):
    from qwenasr_amd import qint8

    p = tmp_path / "model.qint8"
    write_model(p, w, L)
    with qint8.QuantFile.open(str(p)) as qf:
        dims = qint8.detect_decoder_dims(qf)
        dims.n_layers = L
        return qint8.load_decoder_int8(qf, dims, dev)


@pytest.mark.parametrize("fuse_heads,fuse_norms", [(True, True), (False, True), (True, False), (False, False)])
@pytest.mark.parametrize("H,I", [(1024, 3072), (2048, 6144)])
def test_prefill_then_decode_matches_the_oracle(tmp_path, dev, H, I, fuse_heads, fuse_norms):
    """The device prefill (decoder.rs:751-847) of two chunks -- 37 rows at
    position 0 (ragged matrix-core GEMM tiles), then 20 rows at 37 -- against
    the oracle's restatement: the residual stream after the last layer and
    every cache row, then a decode step over the prefilled cache (token,
    logits), with q/k/v and the heads in one launch or two, and the residual
    adds and RMSNorms folded into the GEMMs or run as the reference's separate
    ops. Tolerance as for the decode step (chained kernels, 1e-4)."""
    from qwenasr_amd.decoder import DecoderInt8

    L, nq, nk, hd, vocab = 2, 16, 8, 128, 1000
    r = np.random.default_rng([35, H])
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    dec = DecoderInt8(_load(tmp_path, w, L, dev), H, I, L, nq, nk, hd, max_seq=64, device=dev,
                      fuse_prefill_heads=fuse_heads, fuse_prefill_norms=fuse_norms)
    assert dec.prefill_heads_fused(37) == fuse_heads
    assert dec.prefill_norms_folded(37) == fuse_norms
    kv = nk * hd
    kc = np.zeros((L, 128, kv), np.float32)
    vc = np.zeros_like(kc)
    start = 0
    for T in (37, 20):
        X = r.standard_normal((T, H)).astype(np.float32)
        x_ref = prefill_int8(w, kc, vc, start, X.ravel(), T, nq, nk, hd, threads=8)
        dec.prepare_prefill(start, T)
        dec.prefill(torch.from_numpy(X.ravel()).to(dev), T, start)
        torch.cuda.synchronize()
        np.testing.assert_allclose(dec.px[:T * H].cpu().numpy(), x_ref, rtol=TOL, atol=TOL,
                                   err_msg=f"residual after chunk at {start}")
        start += T
        assert dec.kv.len == start
        for l in range(L):
            np.testing.assert_allclose(dec.kv.k_layer(l).cpu().numpy().reshape(start, kv), kc[l, :start],
                                       rtol=TOL, atol=TOL, err_msg=f"k rows layer {l}")
            np.testing.assert_allclose(dec.kv.v_layer(l).cpu().numpy().reshape(start, kv), vc[l, :start],
                                       rtol=TOL, atol=TOL, err_msg=f"v rows layer {l}")
    e = r.standard_normal(H).astype(np.float32)
    tok, xn, logits = decode_int8_step(w, kc, vc, start, e, nq, nk, hd, threads=8)
    dec.prepare(start)
    dec.decode(torch.from_numpy(e).to(dev), start)
    dec.finish(start)
    torch.cuda.synchronize()
    np.testing.assert_allclose(dec.x_norm.cpu().numpy(), xn, rtol=TOL, atol=TOL)
    np.testing.assert_allclose(dec.logits.cpu().numpy(), logits, rtol=TOL, atol=TOL)
    top2 = np.sort(logits)[-2:]
    if top2[1] - top2[0] > 10 * TOL * max(1.0, abs(top2[1])):
        assert int(dec.token.cpu()[0]) == tok


def test_graph_replays_equal_the_eager_calls(tmp_path, dev):
    """bench.py times the decode step and the prefill as captured HIP graphs.
    Each of three replays, with the outputs overwritten by eager fills and the
    device synchronised in between, must give the eager call's results bit for
    bit: decode (fused and unfused, key splits at position 300) and a 64-token
    prefill (matrix-core GEMMs, cache rows of every layer; the residual adds
    and RMSNorms folded into the GEMMs or not)."""
    from qwenasr_amd.decoder import DecoderInt8

    H, I, L, nq, nk, hd, vocab = 2048, 6144, 2, 16, 8, 128, 1000
    r = np.random.default_rng([37, H])
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    weights = _load(tmp_path, w, L, dev)
    gen = torch.Generator(device=dev).manual_seed(37)

    def snapshot(d, names, rows):
        got = {n: getattr(d, n).clone() for n in names}
        for l in range(L):
            got[f"k{l}"] = d.kv.k_layer_block(l).view(d.kv.max_seq, -1)[rows].clone()
            got[f"v{l}"] = d.kv.v_layer_block(l).view(d.kv.max_seq, -1)[rows].clone()
        return got

    def scribble(d, names, rows):
        for n in names:
            t = getattr(d, n)
            t.fill_(-1) if t.dtype == torch.int32 else t.fill_(float("nan"))
        for l in range(L):
            d.kv.k_layer_block(l).view(d.kv.max_seq, -1)[rows] = float("nan")
            d.kv.v_layer_block(l).view(d.kv.max_seq, -1)[rows] = float("nan")

    def check(d, fn, names, rows, what):
        fn()
        torch.cuda.synchronize()
        ref = snapshot(d, names, rows)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        for rep in range(3):
            scribble(d, names, rows)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = snapshot(d, names, rows)
            for n, t in ref.items():
                assert torch.equal(got[n], t), f"{what}: replay {rep} differs in {n}"

    pos = 300
    for fuse in (True, False):
        d = DecoderInt8(weights, H, I, L, nq, nk, hd, max_seq=512, device=dev, fuse_norms=fuse)
        d.kv.k.normal_(generator=gen)
        d.kv.v.normal_(generator=gen)
        d.kv.len = pos
        d.prepare(pos)
        x = torch.randn(H, device=dev, generator=gen)
        check(d, lambda: d.decode(x, pos), ("x_norm", "logits", "token"), pos,
              f"decode fuse_norms={fuse}")

    T = 64
    e = torch.randn(T * H, device=dev, generator=gen)
    for fuse_heads, fuse_norms in ((False, False), (True, False), (True, True)):
        d = DecoderInt8(weights, H, I, L, nq, nk, hd, max_seq=512, device=dev, fuse_prefill_heads=fuse_heads,
                        fuse_prefill_norms=fuse_norms)
        d.prepare_prefill(0, T)

        def prefill_at_0():
            d.kv.len = 0  # every call (and replay) prefills the same chunk at position 0
            d.prefill(e, T, 0)

        check(d, prefill_at_0, ("px",), slice(0, T),
              f"prefill fuse_prefill_heads={fuse_heads} fuse_prefill_norms={fuse_norms}")
