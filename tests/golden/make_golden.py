"""Writes the golden fixtures in tests/golden/*.npz.

The expected values here are computed independently of the oracle's C code:
float64 closed forms (numpy/scipy), exact integer arithmetic, and the known-
answer inputs of the reference's own tests (crates/qwen-asr/tests/kernels.rs).
The reference is Rust and cannot be run in this image, so nothing here is
produced by the reference itself; each fixture names the reference property or
definition it encodes.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
from scipy import special

HERE = Path(__file__).resolve().parent
SEED = 20261201


def f32(a):
    return np.asarray(a, dtype=np.float32)


def rng(tag: int) -> np.random.Generator:
    return np.random.default_rng([SEED, tag])


def rms_norm_f64(x, w, eps):
    x = x.astype(np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * w.astype(np.float64)


def layer_norm_f64(x, w, b, eps):
    x = x.astype(np.float64)
    mu = np.mean(x, axis=-1, keepdims=True)
    var = np.mean((x - mu) ** 2, axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w.astype(np.float64) + b.astype(np.float64)


def main() -> None:
    out = {}

    # --- RMSNorm ------------------------------------------------------------
    # tests/kernels.rs:60-72 input: x = i*0.02 - 1.28 (128), unit gain, eps 1e-6.
    x_kat = f32(np.arange(128) * np.float32(0.02) - np.float32(1.28))
    out["rms_kat_x"] = x_kat
    out["rms_kat_y64"] = rms_norm_f64(x_kat[None], np.ones(128, np.float32), 1e-6)[0]
    # rows whose mean square is ~eps, so dropping eps changes the result by ~40%;
    # hidden 37 exercises the scalar tail, 64/48 the 8- and 16-lane loops.
    for h in (64, 48, 37):
        r = rng(100 + h)
        x = f32(r.standard_normal((3, h)) * 1e-3)
        w = f32(1.0 + 0.1 * r.standard_normal(h))
        out[f"rms_small_x_{h}"] = x
        out[f"rms_small_w_{h}"] = w
        out[f"rms_small_y64_{h}"] = rms_norm_f64(x, w, 1e-6)

    # --- LayerNorm ------------------------------------------------------------
    # tests/kernels.rs:74-89 input: x = i*0.05 - 3.2 (128), w=1, b=0, eps 1e-5.
    xl = f32(np.arange(128) * np.float32(0.05) - np.float32(3.2))
    out["ln_kat_x"] = xl
    out["ln_kat_y64"] = layer_norm_f64(xl[None], np.ones(128, np.float32),
                                       np.zeros(128, np.float32), 1e-5)[0]
    for h in (64, 45):
        r = rng(200 + h)
        # offset mean (cancellation check) and variance ~eps (eps check)
        x = f32(5.0 + 3e-3 * r.standard_normal((3, h)))
        w = f32(1.0 + 0.1 * r.standard_normal(h))
        b = f32(0.02 * r.standard_normal(h))
        out[f"ln_x_{h}"] = x
        out[f"ln_w_{h}"] = w
        out[f"ln_b_{h}"] = b
        out[f"ln_y64_{h}"] = layer_norm_f64(x, w, b, 1e-5)

    # --- Activations -------------------------------------------------------------
    # tests/kernels.rs:105-124 inputs plus a grid and the tails.
    g = np.concatenate([[0.0, 1.0, -1.0, 2.0, -0.5, 5.0],
                        np.linspace(-10, 10, 401), [-30.0, -15.0, 15.0, 30.0, 1e-6, -1e-6]])
    g = f32(g)
    gd = g.astype(np.float64)
    out["act_x"] = g
    out["gelu_erf_y64"] = 0.5 * gd * (1.0 + special.erf(gd / np.sqrt(2.0)))
    out["gelu_tanh_y64"] = 0.5 * gd * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (gd + 0.044715 * gd ** 3)))
    out["silu_y64"] = gd / (1.0 + np.exp(-gd))
    # exp over the fast_exp domain, for its relative-error bound
    e = f32(np.linspace(-80, 80, 3201))
    out["exp_x"] = e
    out["exp_y64"] = np.exp(e.astype(np.float64))

    # --- RoPE ------------------------------------------------------------------
    # inv_freq = 1/theta^(2d/D) rounded to f32; angle = f32(p * inv) (f32 product);
    # table = cos/sin of that f32 angle, each row [c(0..63) | c(0..63)].
    D, theta = 128, 1e6
    d = np.arange(D // 2)
    inv64 = 1.0 / theta ** (2.0 * d / D)
    inv32 = f32(inv64)
    out["rope_inv_freq"] = inv32
    pos = np.array([0, 1, 2, 7, 100, 511, 1023, 1024, 2047], dtype=np.int32)
    ang32 = f32(pos[:, None].astype(np.float32) * inv32[None, :])
    cos64 = np.cos(ang32.astype(np.float64))
    sin64 = np.sin(ang32.astype(np.float64))
    out["rope_pos"] = pos
    out["rope_cos64"] = np.concatenate([cos64, cos64], axis=1)
    out["rope_sin64"] = np.concatenate([sin64, sin64], axis=1)
    # rotation closed form on given table rows: v[d] = x1 c - x2 s, v[d+h] = x2 c + x1 s
    r = rng(300)
    xq = f32(r.standard_normal((len(pos), 3, D)))
    c32 = f32(out["rope_cos64"])
    s32 = f32(out["rope_sin64"])
    x1 = xq[:, :, : D // 2].astype(np.float64)
    x2 = xq[:, :, D // 2:].astype(np.float64)
    c = c32[:, None, : D // 2].astype(np.float64)
    s = s32[:, None, : D // 2].astype(np.float64)
    out["rope_x"] = xq
    out["rope_cos32"] = c32
    out["rope_sin32"] = s32
    out["rope_y64"] = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=2)

    # head RMSNorm closed form: per 128-vector, shared weight
    hx = f32(r.standard_normal((5, 4, D)))
    hw = f32(1.0 + 0.1 * r.standard_normal(D))
    out["head_x"] = hx
    out["head_w"] = hw
    out["head_y64"] = rms_norm_f64(hx, hw, 1e-6)

    # --- Sinusoidal PE ------------------------------------------------------------
    # log_ts = ln(10000)/(half-1) in f32, inv = exp(-d*log_ts) rounded to f32,
    # angle = f32(p * inv); row = [sin | cos] of that angle.
    # rows 0..12 of the per-chunk table at d_model 896, and sampled rows of a
    # 3000-row table at d_model 64 (positions 0..2999 when not restarted per chunk)
    for dm, prow in ((896, np.arange(13)), (64, np.array([0, 1, 12, 13, 100, 999, 2047, 2999]))):
        half = dm // 2
        log_ts = np.float32(np.float32(np.log(10000.0)) / np.float32(half - 1))
        arg = f32(-np.arange(half, dtype=np.float32) * log_ts)
        inv = f32(np.exp(arg.astype(np.float64)))
        ang = f32(prow.astype(np.float32)[:, None] * inv[None, :])
        pe = np.concatenate([np.sin(ang.astype(np.float64)), np.cos(ang.astype(np.float64))], 1)
        out[f"pe_rows_{dm}"] = prow.astype(np.int32)
        out[f"pe64_{dm}"] = pe

    # --- Quantizer --------------------------------------------------------------
    # rows: random; absmax 127 with .5 ties (inv = 1 exactly); zero row; NaN; inf.
    qr = rng(400)
    rows = [f32(0.02 * qr.standard_normal(64)),
            f32(np.concatenate([[127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5],
                                np.linspace(-100, 100, 54)])),
            np.zeros(64, np.float32),
            f32(np.concatenate([[np.nan, 3.0, -6.0], np.linspace(-1, 1, 61)])),
            f32(np.concatenate([[np.inf, 1.0, -2.0], np.linspace(-1, 1, 61)]))]
    qx = np.stack(rows)
    q_exp = np.zeros(qx.shape, np.int8)
    s_exp = np.zeros(qx.shape[0], np.float32)
    for i, row in enumerate(qx):
        finite_abs = np.abs(row[~np.isnan(row)])
        am = np.float32(finite_abs.max()) if finite_abs.size else np.float32(0)
        s_exp[i] = np.float32(am / np.float32(127.0))
        inv = np.float32(np.float32(127.0) / am) if am > 0 else np.float32(0.0)
        with np.errstate(invalid="ignore"):
            t = (row * inv).astype(np.float32).astype(np.float64)
            rt = np.sign(t) * np.floor(np.abs(t) + 0.5)  # half away from zero
            rt = np.clip(rt, -128, 127)
            rt = np.where(np.isnan(rt), 0, rt)
        q_exp[i] = rt.astype(np.int8)
    out["quant_x"] = qx
    out["quant_q"] = q_exp
    out["quant_s"] = s_exp

    # --- W8A8 / W8A32 ----------------------------------------------------------------
    wr = rng(500)
    K, inter, B = 256, 24, 3
    wq = wr.integers(-128, 128, size=(2 * inter, K), dtype=np.int8)
    ws = f32(wr.uniform(1e-4, 1e-3, size=2 * inter))
    xq8 = wr.integers(-127, 128, size=(B, K), dtype=np.int8)
    xs = f32(wr.uniform(0.005, 0.05, size=B))
    dots = xq8.astype(np.int64) @ wq.astype(np.int64).T  # [B, 2*inter]
    out["w8a8_w"] = wq
    out["w8a8_s"] = ws
    out["w8a8_xq"] = xq8
    out["w8a8_xs"] = xs
    out["w8a8_dots"] = dots.astype(np.int32)
    gg = dots[:, 0::2].astype(np.float64) * xs[:, None] * ws[None, 0::2]
    uu = dots[:, 1::2].astype(np.float64) * xs[:, None] * ws[None, 1::2]
    out["w8a8_y64"] = gg / (1.0 + np.exp(-gg)) * uu
    # W8A32 closed form
    x32 = f32(wr.standard_normal((2, K)))
    out["w8a32_x"] = x32
    out["w8a32_y64"] = (x32.astype(np.float64) @ wq.astype(np.float64).T) * ws[None, :]

    # --- gathers -------------------------------------------------------------------
    gr = rng(600)
    tab32 = f32(gr.standard_normal((50, 24)))
    ids = np.array([0, 49, 7, 7, 13], dtype=np.int32)
    bits = gr.integers(0, 1 << 16, size=(50, 24), dtype=np.uint16)
    out["gather_tab32"] = tab32
    out["gather_ids"] = ids
    out["gather_bits"] = bits
    out["gather_bf16_exp"] = (bits[ids].astype(np.uint32) << 16).view(np.float32)
    tab8 = gr.integers(-128, 128, size=(50, 24), dtype=np.int8)
    sc8 = f32(gr.uniform(1e-3, 1e-1, size=50))
    out["gather_tab8"] = tab8
    out["gather_sc8"] = sc8
    out["gather_i8_exp"] = f32(tab8[ids].astype(np.float32) * sc8[ids][:, None])

    np.savez_compressed(HERE / "golden.npz", **out)
    print(f"wrote {HERE / 'golden.npz'} with {len(out)} arrays")


if __name__ == "__main__":
    main()
