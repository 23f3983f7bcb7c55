"""Pins the CPU oracle (oracle/qasr_oracle.c) before the GPU tests compare against it.

Each check compares the oracle with something it does not share code with:
the known-answer properties of the reference's own tests
(crates/qwen-asr/tests/kernels.rs), float64 closed forms and exact integer
results from tests/golden/golden.npz, and mathematical invariants. The inputs
are chosen so that a plausible mistake (a dropped eps, a swapped sin/cos, a
sign, banker's rounding, the libm exp in place of the reference's polynomial)
fails at least one check.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.conftest import assert_close


# --- RMSNorm ----------------------------------------------------------------
def test_rms_norm_reference_kat(golden):
    # tests/kernels.rs:60-72: unit gain -> output RMS ~ 1 (+-0.01)
    x = golden["rms_kat_x"]
    y = oracle.rms_norm(x, np.ones(128, np.float32), 1, 128, 1e-6)
    rms = float(np.sqrt(np.mean(y.astype(np.float64) ** 2)))
    assert abs(rms - 1.0) < 0.01
    assert_close(y, golden["rms_kat_y64"], 2e-6, 1e-7, "rms kat")


@pytest.mark.parametrize("h", [64, 48, 37])
def test_rms_norm_eps_sensitive_rows(golden, h):
    x, w = golden[f"rms_small_x_{h}"], golden[f"rms_small_w_{h}"]
    y = oracle.rms_norm(x.ravel(), w, x.shape[0], h, 1e-6).reshape(x.shape)
    assert_close(y, golden[f"rms_small_y64_{h}"], 2e-6, 1e-7, f"rms h={h}")


def test_rms_norm_zero_row_is_zero():
    y = oracle.rms_norm(np.zeros(64, np.float32), np.ones(64, np.float32), 1, 64, 1e-6)
    assert np.all(y == 0)


def test_add_rms_norm_is_add_then_norm(golden):
    r = np.random.default_rng(1)
    x = r.standard_normal(3 * 40).astype(np.float32)
    d = r.standard_normal(3 * 40).astype(np.float32)
    w = (1 + 0.1 * r.standard_normal(40)).astype(np.float32)
    x2, y = oracle.add_rms_norm(x, d, w, 3, 40, 1e-6)
    np.testing.assert_array_equal(x2, x + d)  # f32 add is exact-rounded either way
    s = (x + d).astype(np.float64).reshape(3, 40)
    ref = s / np.sqrt(np.mean(s * s, axis=1, keepdims=True) + 1e-6) * w
    assert_close(y.reshape(3, 40), ref, 2e-6, 1e-7, "add+rms")


# --- LayerNorm ----------------------------------------------------------------
def test_layer_norm_reference_kat(golden):
    # tests/kernels.rs:74-89: mean ~ 0 (+-0.01), var ~ 1 (+-0.02)
    x = golden["ln_kat_x"]
    y = oracle.layer_norm(x, np.ones(128, np.float32), np.zeros(128, np.float32), 1, 128, 1e-5)
    assert abs(float(np.mean(y))) < 0.01
    assert abs(float(np.var(y.astype(np.float64))) - 1.0) < 0.02
    assert_close(y, golden["ln_kat_y64"], 2e-6, 1e-6, "ln kat")


@pytest.mark.parametrize("h", [64, 45])
def test_layer_norm_offset_small_variance(golden, h):
    x, w, b = golden[f"ln_x_{h}"], golden[f"ln_w_{h}"], golden[f"ln_b_{h}"]
    y = oracle.layer_norm(x.ravel(), w, b, x.shape[0], h, 1e-5).reshape(x.shape)
    # x has mean 5 and std 3e-3: f32 mean subtraction leaves ~5e-7/3e-3 relative noise
    assert_close(y, golden[f"ln_y64_{h}"], 1e-4, 1e-4, f"ln h={h}")


# --- head RMSNorm / RoPE ---------------------------------------------------------
def test_rms_norm_per_head_closed_form(golden):
    x, w = golden["head_x"], golden["head_w"]
    y = oracle.rms_norm_per_head(x.ravel(), w, x.shape[0], x.shape[1], x.shape[2], 1e-6)
    assert_close(y.reshape(x.shape), golden["head_y64"], 2e-6, 1e-7, "head norm")


def test_rope_inv_freq_within_one_ulp(golden):
    inv = oracle.rope_inv_freq(128, 1e6)
    ref = golden["rope_inv_freq"]
    assert inv[0] == 1.0  # theta^0
    ulp = np.spacing(np.abs(ref))
    assert np.all(np.abs(inv - ref) <= ulp), "inv_freq differs from 1/theta^(2d/D) by > 1 ulp"


def test_rope_table_matches_f32_angle_closed_form(golden):
    pos = golden["rope_pos"]
    cos, sin = oracle.rope_table(int(pos.max()) + 1, 128, 1e6)
    cos, sin = cos.reshape(-1, 128)[pos], sin.reshape(-1, 128)[pos]
    inv = oracle.rope_inv_freq(128, 1e6)
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    c64 = np.concatenate([np.cos(ang), np.cos(ang)], 1)
    s64 = np.concatenate([np.sin(ang), np.sin(ang)], 1)
    assert_close(cos, c64, 0, 1.2e-7, "cos table")
    assert_close(sin, s64, 0, 1.2e-7, "sin table")
    # position 0 is the identity rotation, exactly
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # column 0 has inv_freq 1: angle = p exactly
    assert_close(cos[:, 0], np.cos(pos.astype(np.float64)), 0, 1.2e-7, "cos(p)")


def test_rope_rotation_closed_form(golden):
    x, c, s = golden["rope_x"], golden["rope_cos32"], golden["rope_sin32"]
    y = oracle.apply_rope_neox(x.ravel(), c.ravel(), s.ravel(), x.shape[0], x.shape[1], 128)
    y = y.reshape(x.shape)
    assert_close(y, golden["rope_y64"], 1e-6, 1e-6, "rope")
    # position 0 row: exact identity
    np.testing.assert_array_equal(y[0], x[0])
    # each (d, d+64) pair keeps its length
    n_in = np.hypot(x[..., :64].astype(np.float64), x[..., 64:].astype(np.float64))
    n_out = np.hypot(y[..., :64].astype(np.float64), y[..., 64:].astype(np.float64))
    assert_close(n_out, n_in, 1e-6, 1e-7, "pair norm")


def test_head_norm_rope_composition(golden):
    r = np.random.default_rng(7)
    seq, nq, nk, hd = 4, 3, 2, 128
    q = r.standard_normal(seq * nq * hd).astype(np.float32)
    k = r.standard_normal(seq * nk * hd).astype(np.float32)
    qw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * r.standard_normal(hd)).astype(np.float32)
    cos, sin = oracle.rope_table(64, hd, 1e6)
    pos = np.array([5, 0, 63, 17], np.int32)
    q2, k2 = oracle.head_rms_norm_rope(q, k, qw, kw, cos, sin, pos, seq, nq, nk, hd, 1e-6)
    # same as norm-per-head then rope with gathered table rows
    qn = oracle.rms_norm_per_head(q, qw, seq, nq, hd, 1e-6)
    cr = cos.reshape(64, hd)[pos].ravel()
    sr = sin.reshape(64, hd)[pos].ravel()
    np.testing.assert_array_equal(q2, oracle.apply_rope_neox(qn, cr, sr, seq, nq, hd))
    kn = oracle.rms_norm_per_head(k, kw, seq, nk, hd, 1e-6)
    np.testing.assert_array_equal(k2, oracle.apply_rope_neox(kn, cr, sr, seq, nk, hd))


# --- activations --------------------------------------------------------------------
def test_fast_exp_is_the_reference_polynomial(golden):
    x, ref = golden["exp_x"], golden["exp_y64"]
    got = np.array([oracle.fast_exp(float(v)) for v in x], np.float64)
    rel = np.abs(got - ref) / ref
    assert rel.max() < 1e-5            # a degree-5 polynomial on [-ln2/2, ln2/2]
    assert rel.max() > 1e-6            # ... and not libm expf (which is < 1 ulp)
    assert oracle.fast_exp(0.0) == 1.0
    assert oracle.fast_exp(-1000.0) == np.float32(2.0 ** -126)  # clamp at -126


def test_silu_reference_kat(golden):
    # tests/kernels.rs:115-124: max abs err < 1e-5 against v/(1+exp(-v))
    x = golden["act_x"]
    assert_close(oracle.silu(x), golden["silu_y64"], 1e-6, 1e-7, "silu")


def test_gelu_tanh_reference_kat(golden):
    x = golden["act_x"]
    y = oracle.gelu_tanh(x)
    # tests/kernels.rs:105-113 on the first five inputs [0, 1, -1, 2, -0.5]
    assert abs(y[0]) < 1e-5 and y[1] > 0.5 and y[2] < 0.0
    assert_close(y, golden["gelu_tanh_y64"], 1e-5, 2e-5, "gelu tanh")


def test_gelu_erf_closed_form(golden):
    x = golden["act_x"]
    assert_close(oracle.gelu_erf(x), golden["gelu_erf_y64"], 0, 1e-6, "gelu erf")
    # tanh vs erf GELU differ by up to ~4.7e-4 (the gap the exact form closes)
    gap = np.abs(golden["gelu_tanh_y64"] - golden["gelu_erf_y64"]).max()
    assert 4e-4 < gap < 5e-4


def test_swiglu_multiply_fast_blocks_and_tail():
    r = np.random.default_rng(3)
    seq, inter = 3, 21  # two 8-blocks via fast_exp + a 5-column libm tail per row
    gu = r.standard_normal(seq * 2 * inter).astype(np.float32) * 3
    y = oracle.swiglu_multiply(gu, seq, inter).reshape(seq, inter)
    g = gu.reshape(seq, inter, 2)[..., 0].astype(np.float64)
    u = gu.reshape(seq, inter, 2)[..., 1].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert_close(y, ref, 1e-5, 1e-6, "swiglu")
    # the tail columns use libm expf: within a few ulp of exact
    assert_close(y[:, 16:], ref[:, 16:], 1e-6, 1e-7, "swiglu tail")
    # split form == interleaved form on the libm columns
    ys = oracle.swiglu_split(gu.reshape(seq, inter, 2)[..., 0].copy(),
                             gu.reshape(seq, inter, 2)[..., 1].copy()).reshape(seq, inter)
    np.testing.assert_array_equal(ys[:, 16:], y[:, 16:])


# --- sinusoidal PE ----------------------------------------------------------------
@pytest.mark.parametrize("dm", [896, 64])
def test_sinusoidal_pe_closed_form(golden, dm):
    rows = golden[f"pe_rows_{dm}"]
    pe = oracle.sinusoidal_pe(int(rows.max()) + 1, dm).reshape(-1, dm)[rows]
    assert_close(pe, golden[f"pe64_{dm}"], 0, 2.4e-7, f"pe d={dm}")
    if rows[0] == 0:
        half = dm // 2
        assert np.all(pe[0, :half] == 0.0) and np.all(pe[0, half:] == 1.0)


# --- gathers ---------------------------------------------------------------------
def test_gathers_bit_exact(golden):
    ids = golden["gather_ids"]
    np.testing.assert_array_equal(oracle.embed_gather_f32(golden["gather_tab32"], ids, 24),
                                  golden["gather_tab32"][ids].ravel())
    np.testing.assert_array_equal(oracle.embed_gather_bf16(golden["gather_bits"], ids, 24),
                                  golden["gather_bf16_exp"].ravel())
    np.testing.assert_array_equal(
        oracle.embed_gather_i8(golden["gather_tab8"], golden["gather_sc8"], ids, 24),
        golden["gather_i8_exp"].ravel())


# --- quantizer ---------------------------------------------------------------------
def test_quantizer_bit_exact_with_ties_and_specials(golden):
    x = golden["quant_x"]
    q, s = oracle.quantize_f32_to_int8(x.ravel(), x.shape[0], x.shape[1])
    np.testing.assert_array_equal(q.reshape(x.shape), golden["quant_q"])
    np.testing.assert_array_equal(s, golden["quant_s"])
    row = q.reshape(x.shape)[1]
    assert list(row[2:10]) == [3, -3, 1, -1, 2, -2, 127, -127]  # half away from zero
    assert np.all(q.reshape(x.shape)[2] == 0) and s[2] == 0.0    # all-zero row


def test_quantizer_bf16_matches_f32_path():
    r = np.random.default_rng(11)
    x = (0.02 * r.standard_normal(4 * 96)).astype(np.float32)
    bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    xb = (bits.astype(np.uint32) << 16).view(np.float32)
    q1, s1 = oracle.quantize_bf16_to_int8(bits, 4, 96)
    q2, s2 = oracle.quantize_f32_to_int8(xb, 4, 96)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2)


# --- INT8 matvec / W8A8 -------------------------------------------------------------
def test_w8a8_dots_bit_exact_and_epilogue(golden):
    w, s, xq, xs = golden["w8a8_w"], golden["w8a8_s"], golden["w8a8_xq"], golden["w8a8_xs"]
    B, K = xq.shape
    inter = w.shape[0] // 2
    out, dots = oracle.gate_up_swiglu_w8a8(w, s, xq, xs, B, K, inter)
    np.testing.assert_array_equal(dots.reshape(B, 2 * inter), golden["w8a8_dots"])
    assert_close(out.reshape(B, inter), golden["w8a8_y64"], 2e-6, 1e-9, "w8a8 out")


def test_linear_w8a8_dots_exact_and_dequant():
    # the batched W8A8 projection: int32 dots against int64 numpy, the fp32
    # output against float64 (two f32 roundings: <= 2.4e-7 relative), and the
    # same dequantization the gate/up epilogue applies: on the interleaved
    # matrix its (g, u) pairs give the gate/up oracle's SwiGLU bit for bit
    r = np.random.default_rng(41)
    B, K, inter = 7, 192, 24
    w = r.integers(-127, 128, (2 * inter, K), dtype=np.int8)
    s = (1e-3 + 1e-2 * r.random(2 * inter)).astype(np.float32)
    xq = r.integers(-127, 128, (B, K), dtype=np.int8)
    xs = (1e-2 + r.random(B)).astype(np.float32)
    y, dots = oracle.linear_w8a8(w, s, xq, xs, B, K, 2 * inter)
    exact = xq.astype(np.int64) @ w.astype(np.int64).T
    np.testing.assert_array_equal(dots.reshape(B, -1), exact)
    ref = exact * xs.astype(np.float64)[:, None] * s.astype(np.float64)[None, :]
    assert_close(y.reshape(B, -1), ref, 2.4e-7, 0, "w8a8 dequant")
    gu = y.reshape(B, inter, 2).astype(np.float32)
    g, u = gu[..., 0], gu[..., 1]
    out, _ = oracle.gate_up_swiglu_w8a8(w, s, xq, xs, B, K, inter)
    np.testing.assert_array_equal(out, oracle.swiglu_split(g.ravel().copy(), u.ravel().copy()))
    # the reference kernel on the integer activations with unit scales gives the dots
    ref32 = oracle.linear_nobias_int8(xq.astype(np.float32), w, np.ones(2 * inter, np.float32), B, K, 2 * inter)
    np.testing.assert_array_equal(ref32.astype(np.int64), dots.astype(np.int64))


def test_w8a32_closed_form(golden):
    w, s, x = golden["w8a8_w"], golden["w8a8_s"], golden["w8a32_x"]
    y = oracle.linear_nobias_int8(x, w, s, 2, w.shape[1], w.shape[0]).reshape(2, -1)
    ref = golden["w8a32_y64"]
    assert_close(y, ref, 1e-5, 1e-6 * np.abs(ref).max(), "w8a32")
    # threaded row chunking gives identical rows
    y4 = oracle.linear_nobias_int8(x, w, s, 2, w.shape[1], w.shape[0], n_threads=4)
    np.testing.assert_array_equal(y4, y.ravel())


def test_w8a32_is_exact_on_integer_inputs(golden):
    # With integer-valued x and unit scales the reference's f32 sum is exact
    # (partial sums < 2^24), so linear_nobias_int8 reproduces the int32 W8A8 dot.
    w, xq = golden["w8a8_w"], golden["w8a8_xq"]
    B, K = xq.shape
    y = oracle.linear_nobias_int8(xq.astype(np.float32), w, np.ones(w.shape[0], np.float32), B, K,
                                  w.shape[0]).reshape(B, -1)
    np.testing.assert_array_equal(y.astype(np.int64), golden["w8a8_dots"].astype(np.int64))


def test_linear_int8_bias_after_row_scale():
    # kernels/mod.rs:664-673: y = scale[o] * (W_int8 @ x)[o], then += bias[o]
    # for every token. Checked against float64; scales far from 1 and a bias of
    # the outputs' size make "bias before the scale", a dropped bias and a bias
    # indexed by token instead of output row each fail.
    r = np.random.default_rng(23)
    T, K, O = 3, 96, 40
    w = r.integers(-127, 128, (O, K), dtype=np.int8)
    s = (2e-3 + 2e-2 * r.random(O)).astype(np.float32)
    b = r.standard_normal(O).astype(np.float32)
    x = r.standard_normal((T, K)).astype(np.float32)
    y = oracle.linear_int8(x, w, s, b, T, K, O).reshape(T, O)
    ref = (x.astype(np.float64) @ w.astype(np.float64).T) * s.astype(np.float64) + b.astype(np.float64)
    assert_close(y, ref, 1e-5, 1e-6, "linear_int8")
    wrong = ((x.astype(np.float64) @ w.astype(np.float64).T) + b) * s
    assert np.abs(y - wrong).max() > 1e-2  # the check separates the two orders
    # no bias: identical to linear_nobias_int8
    np.testing.assert_array_equal(oracle.linear_int8(x, w, s, None, T, K, O),
                                  oracle.linear_nobias_int8(x, w, s, T, K, O))


def test_linear_int8_bias_exact_on_integer_inputs():
    # integer x, power-of-two scales and integer biases: every step is exact in
    # f32 (dots < 2^24), so the result is the exact integer expression
    r = np.random.default_rng(24)
    T, K, O = 4, 64, 24
    w = r.integers(-127, 128, (O, K), dtype=np.int8)
    x = r.integers(-50, 51, (T, K)).astype(np.float32)
    s = np.array([2.0 ** -int(e) for e in r.integers(0, 4, O)], np.float32)
    b = r.integers(-1000, 1001, O).astype(np.float32)
    y = oracle.linear_int8(x, w, s, b, T, K, O, n_threads=3).reshape(T, O)
    dots = x.astype(np.int64) @ w.astype(np.int64).T
    np.testing.assert_array_equal(y.astype(np.float64), dots * s.astype(np.float64) + b)


def _encoder_chunk_rows(mel_frames, chunk_size=100):
    """Rows each mel chunk contributes after the conv stem (encoder.rs:252-274):
    three 3-wide, stride-2, pad-1 convolutions over the chunk's frames."""
    conv = lambda w: (w + 2 - 3) // 2 + 1  # noqa: E731
    return [conv(conv(conv(min(chunk_size, mel_frames - s)))) for s in range(0, mel_frames, chunk_size)]


@pytest.mark.parametrize("mel_frames,d", [(537, 64), (1000, 896), (100, 32), (41, 16)])
def test_pe_add_restarts_per_chunk(mel_frames, d):
    # encoder.rs:340-343 builds a fresh sinusoidal_pe(w3, d) for each chunk's w3
    # rows and adds it, so the position restarts at 0 for every chunk; a full
    # 100-frame chunk gives 13 rows and the last chunk may be shorter. The
    # expected sum is built chunk by chunk from that rule (f32 + f32 in float64,
    # rounded once: the f32 sum), independent of the oracle's r mod n_pos.
    rows = _encoder_chunk_rows(mel_frames)
    assert all(n == 13 for n in rows[:-1]) and 1 <= rows[-1] <= 13
    T = sum(rows)
    r = np.random.default_rng(mel_frames)
    x = r.standard_normal((T, d)).astype(np.float32)
    table = r.standard_normal((13, d)).astype(np.float32)  # any 13-row table
    exp = np.empty_like(x)
    off = 0
    for n in rows:
        exp[off:off + n] = (x[off:off + n].astype(np.float64) + table[:n]).astype(np.float32)
        off += n
    got = oracle.pe_add(x.ravel(), table.ravel(), T, d, 13).reshape(T, d)
    np.testing.assert_array_equal(got, exp)
    # and with the sinusoidal table itself, each row is x + PE(row within its
    # chunk) to float64 closed-form accuracy; positions that continue across
    # chunks (PE(13), PE(14), ...) would fail here
    pe = oracle.sinusoidal_pe(13, d).reshape(13, d)
    half = d // 2
    lts = np.log(10000.0) / (half - 1)
    inv = np.exp(-np.arange(half) * lts)
    p = np.concatenate([np.arange(n) for n in rows]).astype(np.float64)[:, None]
    pe64 = np.concatenate([np.sin(p * inv), np.cos(p * inv)], axis=1)
    got = oracle.pe_add(x.ravel(), pe.ravel(), T, d, 13).reshape(T, d)
    assert_close(got, x.astype(np.float64) + pe64, 2e-7, 1e-6, "pe_add closed form")


def test_interleave_layout():
    r = np.random.default_rng(5)
    inter, hid = 6, 32
    wg = r.integers(-128, 128, (inter, hid), dtype=np.int8)
    wu = r.integers(-128, 128, (inter, hid), dtype=np.int8)
    sg = r.random(inter).astype(np.float32)
    su = r.random(inter).astype(np.float32)
    wgu, sgu = oracle.interleave_gate_up(wg, sg, wu, su, inter, hid)
    wgu = wgu.reshape(2 * inter, hid)
    np.testing.assert_array_equal(wgu[0::2], wg)
    np.testing.assert_array_equal(wgu[1::2], wu)
    np.testing.assert_array_equal(sgu[0::2], sg)
    np.testing.assert_array_equal(sgu[1::2], su)


# --- causal attention (kernels/mod.rs:1124-1168) ---------------------------
def attention_f64(q, k, v, seq_q, seq_k, nq, nk, hd, scale, q_offset):
    """float64 softmax(q k^T * scale) v over keys 0..min(q_offset+i+1, seq_k)."""
    Q = q.reshape(seq_q, nq, hd).astype(np.float64)
    K = k[:seq_k * nk * hd].reshape(seq_k, nk, hd).astype(np.float64)
    V = v[:seq_k * nk * hd].reshape(seq_k, nk, hd).astype(np.float64)
    out = np.zeros((seq_q, nq, hd))
    for i in range(seq_q):
        ke = min(q_offset + i + 1, seq_k)
        for h in range(nq):
            if ke == 0:
                continue
            s = K[:ke, h // (nq // nk)] @ Q[i, h] * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ V[:ke, h // (nq // nk)]
    return out.ravel()


@pytest.mark.parametrize("seq_q,seq_k,nq,nk,hd,q_offset", [
    (1, 300, 16, 8, 128, 299),    # decode step at position 299
    (7, 7, 4, 2, 128, 0),         # prefill, causal triangle
    (5, 12, 14, 2, 64, 7),        # chunked prefill after 7 cached rows, head_dim 64
    (3, 2, 2, 2, 36, 5),          # keys end before the causal limit; head_dim tail
    (2, 0, 2, 1, 128, 0),         # no keys: zero output
])
def test_causal_attention_closed_form(seq_q, seq_k, nq, nk, hd, q_offset):
    r = np.random.default_rng(seq_q * 1000 + seq_k)
    q = r.standard_normal(seq_q * nq * hd).astype(np.float32)
    k = r.standard_normal(max(seq_k, 1) * nk * hd).astype(np.float32)
    v = r.standard_normal(max(seq_k, 1) * nk * hd).astype(np.float32)
    o = oracle.causal_attention(q, k, v, seq_q, seq_k, nq, nk, hd, hd ** -0.5, q_offset)
    ref = attention_f64(q, k, v, seq_q, seq_k, nq, nk, hd, hd ** -0.5, q_offset)
    assert_close(o, ref, 2e-6, 1e-6, "attention")


def test_causal_attention_single_key_is_v_and_gqa_sharing():
    # one key: softmax weight 1, output = that v row exactly (x * (1/1))
    hd = 128
    r = np.random.default_rng(3)
    q = r.standard_normal(4 * hd).astype(np.float32)
    k = r.standard_normal(2 * hd).astype(np.float32)
    v = r.standard_normal(2 * hd).astype(np.float32)
    o = oracle.causal_attention(q, k, v, 1, 1, 4, 2, hd, 0.1, 0).reshape(4, hd)
    np.testing.assert_array_equal(o[0], v[:hd])
    np.testing.assert_array_equal(o[1], v[:hd])   # q heads 0,1 share kv head 0
    np.testing.assert_array_equal(o[2], v[hd:])


# --- lm_head argmax (decoder.rs:941-949) ------------------------------------
def test_argmax_rows_semantics():
    x = np.array([[1, np.nan, 5, 5],          # first maximum wins
                  [np.nan, 3, 4, 1],          # NaN at 0 is never replaced
                  [-np.inf] * 4,              # nothing beats element 0
                  [2, 2, 1, np.inf],
                  [0, -1, np.nan, 0.5]], np.float32)
    np.testing.assert_array_equal(oracle.argmax_rows(x, 5, 4), [2, 0, 0, 3, 3])
    r = np.random.default_rng(4)
    y = r.standard_normal((6, 1000)).astype(np.float32)
    np.testing.assert_array_equal(oracle.argmax_rows(y, 6, 1000), y.argmax(axis=1))


# --- the INT8 decode step composition (decoder.rs:848-965) -------------------------
def _f64_quant(v):
    """Per-vector int8 rounding in float64: absmax/127 steps, half away from zero."""
    a = np.abs(v).max()
    if a == 0:
        return v * 0
    q = np.clip(np.sign(v) * np.floor(np.abs(v) * (127.0 / a) + 0.5), -128, 127)
    return q * (a / 127.0)


def _f64_decode(w, kc, vc, pos, x, nq, nk, hd, eps=1e-6, theta=1e6, w8a8=False):
    """float64 numpy evaluation of the decode step's formulas (no oracle
    kernels); ``w8a8`` rounds the four projection inputs to int8 per vector."""
    fq = _f64_quant if w8a8 else (lambda v: v)
    H = x.size
    half = hd // 2
    inv = theta ** (-(2.0 * np.arange(half)) / hd)
    ang = pos * inv
    cos, sin = np.cos(ang), np.sin(ang)

    def rms(v, g):
        return v / np.sqrt(np.mean(v * v) + eps) * g

    def lin(v, ws):
        return (ws[0].astype(np.float64) @ v) * ws[1]

    def heads(v, n, g):
        v = v.reshape(n, hd)
        v = v / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps) * g
        a, b = v[:, :half], v[:, half:]
        return np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=1)

    x = x.astype(np.float64)
    for l, lw in enumerate(w["layers"]):
        xn = fq(rms(x, lw["input_norm"]))
        q = heads(lin(xn, lw["wq"]), nq, lw["q_norm"])
        k = heads(lin(xn, lw["wk"]), nk, lw["k_norm"])
        kc[l, pos] = k.ravel()
        vc[l, pos] = lin(xn, lw["wv"])
        K = kc[l, :pos + 1].reshape(pos + 1, nk, hd)
        V = vc[l, :pos + 1].reshape(pos + 1, nk, hd)
        att = np.empty((nq, hd))
        for h in range(nq):
            s = K[:, h // (nq // nk)] @ q[h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            att[h] = (p / p.sum()) @ V[:, h // (nq // nk)]
        x = x + lin(fq(att.ravel()), lw["wo"])
        xn = fq(rms(x, lw["post_attn_norm"]))
        gu = lin(xn, lw["gate_up"])
        g, u = gu[0::2], gu[1::2]
        x = x + lin(fq(g / (1 + np.exp(-g)) * u), lw["down"])
    xn = rms(x, w["norm"])
    logits = lin(xn, w["lm_head"])
    return int(np.argmax(logits)), xn, logits


def small_decoder(r, H, I, L, nq, nk, hd, vocab):
    def qw(o, i):
        wf = (0.02 * r.standard_normal((o, i))).astype(np.float32)
        q, s = oracle.quantize_f32_to_int8(wf, o, i)
        return q.reshape(o, i), s

    def gain(n):
        return (1 + 0.1 * r.standard_normal(n)).astype(np.float32)

    layers = []
    for _ in range(L):
        gq, gs = qw(I, H)
        uq, us = qw(I, H)
        wgu, sgu = oracle.interleave_gate_up(gq, gs, uq, us, I, H)
        layers.append({"wq": qw(nq * hd, H), "wk": qw(nk * hd, H), "wv": qw(nk * hd, H),
                       "wo": qw(H, nq * hd), "gate_up": (wgu.reshape(2 * I, H), sgu),
                       "down": qw(H, I), "q_norm": gain(hd), "k_norm": gain(hd),
                       "input_norm": gain(H), "post_attn_norm": gain(H),
                       "gate": (gq, gs), "up": (uq, us)})
    return {"layers": layers, "norm": gain(H), "lm_head": qw(vocab, H)}


def test_decode_step_composition():
    """The restated decode step equals a float64 evaluation of decoder.rs's
    formulas (a dropped residual, a swapped gate/up, a wrong norm gain or RoPE
    position would not) over three positions, cache rows included."""
    from oracle.decoder import decode_int8_step

    r = np.random.default_rng(77)
    H, I, L, nq, nk, hd, vocab = 64, 96, 2, 4, 2, 16, 50
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    kc = np.zeros((L, 8, nk * hd), np.float32)
    vc = np.zeros_like(kc)
    kc64, vc64 = np.zeros(kc.shape), np.zeros(vc.shape)
    for pos in range(3):
        x = r.standard_normal(H).astype(np.float32)
        tok, xn, logits = decode_int8_step(w, kc, vc, pos, x, nq, nk, hd)
        tok64, xn64, logits64 = _f64_decode(w, kc64, vc64, pos, x, nq, nk, hd)
        np.testing.assert_allclose(xn, xn64, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(logits, logits64, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(kc[:, :pos + 1], kc64[:, :pos + 1], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(vc[:, :pos + 1], vc64[:, :pos + 1], rtol=1e-4, atol=1e-5)
        top2 = np.sort(logits64)[-2:]
        if top2[1] - top2[0] > 1e-3:
            assert tok == tok64


def test_decode_w8a8_step_composition():
    """The W8A8 decode step equals a float64 evaluation of the same formulas
    with the four projection inputs rounded to int8 per vector, and differs
    from the W8A32 step by several times the tolerance. Leaving out the
    rounding at any one of the four points moves the result 6-30x the
    tolerance away from the float64 evaluation (checked by planting it)."""
    from oracle.decoder import decode_int8_step, decode_w8a8_step

    r = np.random.default_rng(78)
    H, I, L, nq, nk, hd, vocab = 64, 96, 2, 4, 2, 16, 50
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    shape = (L, 8, nk * hd)
    kc, vc, kc32, vc32 = (np.zeros(shape, np.float32) for _ in range(4))
    kc64, vc64 = np.zeros(shape), np.zeros(shape)
    for pos in range(3):
        x = r.standard_normal(H).astype(np.float32)
        tok, xn, logits = decode_w8a8_step(w, kc, vc, pos, x, nq, nk, hd)
        _, xn32, _ = decode_int8_step(w, kc32, vc32, pos, x, nq, nk, hd)
        tok64, xn64, logits64 = _f64_decode(w, kc64, vc64, pos, x, nq, nk, hd, w8a8=True)
        np.testing.assert_allclose(xn, xn64, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(logits, logits64, rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(kc[:, :pos + 1], kc64[:, :pos + 1], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(vc[:, :pos + 1], vc64[:, :pos + 1], rtol=1e-4, atol=1e-5)
        assert (np.abs(xn - xn32) / (1e-5 + 1e-4 * np.abs(xn32))).max() > 3.0
        top2 = np.sort(logits64)[-2:]
        if top2[1] - top2[0] > 1e-3:
            assert tok == tok64


def _f64_prefill(w, kc, vc, start, X, nq, nk, hd, eps=1e-6, theta=1e6):
    """float64 numpy evaluation of the prefill's formulas (no oracle kernels)."""
    T, H = X.shape
    half = hd // 2
    inv = theta ** (-(2.0 * np.arange(half)) / hd)
    ang = (start + np.arange(T))[:, None] * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rms(v, g):
        return v / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps) * g

    def lin(v, ws):
        return (v @ ws[0].astype(np.float64).T) * ws[1]

    def heads(v, n, g):
        v = v.reshape(T, n, hd)
        v = v / np.sqrt(np.mean(v * v, axis=2, keepdims=True) + eps) * g
        a, b = v[..., :half], v[..., half:]
        c, s = cos[:, None, :], sin[:, None, :]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=2).reshape(T, n * hd)

    x = X.astype(np.float64)
    total = start + T
    for l, lw in enumerate(w["layers"]):
        xn = rms(x, lw["input_norm"])
        q = heads(lin(xn, lw["wq"]), nq, lw["q_norm"])
        kc[l, start:total] = heads(lin(xn, lw["wk"]), nk, lw["k_norm"])
        vc[l, start:total] = lin(xn, lw["wv"])
        K = kc[l, :total].reshape(total, nk, hd)
        V = vc[l, :total].reshape(total, nk, hd)
        att = np.empty((T, nq, hd))
        for i in range(T):
            for h in range(nq):
                sc = K[:start + i + 1, h // (nq // nk)] @ q[i].reshape(nq, hd)[h] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                att[i, h] = (p / p.sum()) @ V[:start + i + 1, h // (nq // nk)]
        x = x + lin(att.reshape(T, nq * hd), lw["wo"])
        xn = rms(x, lw["post_attn_norm"])
        gu = lin(xn, lw["gate_up"])
        g, u = gu[:, 0::2], gu[:, 1::2]
        x = x + lin(g / (1 + np.exp(-g)) * u, lw["down"])
    return x


def test_prefill_composition():
    """The restated prefill equals a float64 evaluation of decoder.rs:751-847's
    formulas (a missing residual, a row using another row's RoPE position, a
    causal mask off by one or a cache row written at the wrong offset would
    not) over two chunks: 5 rows at position 0, then 3 more at position 5; a
    decode step after them sees the same cache."""
    from oracle.decoder import decode_int8_step, prefill_int8

    r = np.random.default_rng(78)
    H, I, L, nq, nk, hd, vocab = 64, 96, 2, 4, 2, 16, 50
    w = small_decoder(r, H, I, L, nq, nk, hd, vocab)
    kc = np.zeros((L, 16, nk * hd), np.float32)
    vc = np.zeros_like(kc)
    kc64, vc64 = np.zeros(kc.shape), np.zeros(vc.shape)
    start = 0
    for T in (5, 3):
        X = r.standard_normal((T, H)).astype(np.float32)
        x = prefill_int8(w, kc, vc, start, X.ravel(), T, nq, nk, hd)
        x64 = _f64_prefill(w, kc64, vc64, start, X, nq, nk, hd)
        np.testing.assert_allclose(x.reshape(T, H), x64, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(kc[:, :start + T], kc64[:, :start + T], rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(vc[:, :start + T], vc64[:, :start + T], rtol=1e-4, atol=1e-5)
        start += T
    e = r.standard_normal(H).astype(np.float32)
    _, xn, _ = decode_int8_step(w, kc, vc, start, e, nq, nk, hd)
    _, xn64, _ = _f64_decode(w, kc64, vc64, start, e, nq, nk, hd)
    np.testing.assert_allclose(xn, xn64, rtol=1e-4, atol=1e-4)
