// The reference's kernel unit tests (crates/qwen-asr/tests/kernels.rs) restated
// on the GPU through the C++ host mirror qwen_asr::kernels, plus drop-in
// checks the reference cannot express (device tables, panics on short slices).
//
// Built by qwenasr_amd/build.py against the static archive libqasr_hip.a;
// run by tests/test_gpu_cpp.py. Prints one line per test, exits non-zero on
// any failure.
#include <hip/hip_runtime.h>

#include <unistd.h>

#include <cmath>
#include <cstring>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

#include "qwen_asr/kernels.hpp"

namespace K = qwen_asr::kernels;

static int g_failed = 0;

#define EXPECT(cond, ...)                                \
  do {                                                   \
    if (!(cond)) {                                       \
      std::fprintf(stderr, "  expectation failed: " #cond " -- " __VA_ARGS__); \
      std::fprintf(stderr, "\n");                        \
      throw std::runtime_error("expectation failed");    \
    }                                                    \
  } while (0)

template <class T>
static K::DeviceBuffer<T> upload(const std::vector<T>& h) {
  K::DeviceBuffer<T> d(h.size());
  if (hipMemcpy(d.data(), h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
    throw std::runtime_error("hipMemcpy H2D failed");
  return d;
}

template <class T>
static std::vector<T> download(const K::DeviceBuffer<T>& d) {
  std::vector<T> h(d.size());
  if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("device sync failed");
  if (hipMemcpy(h.data(), d.data(), h.size() * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
    throw std::runtime_error("hipMemcpy D2H failed");
  return h;
}

static void copy_row(std::vector<float>& h, const float* d) {
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(h.data(), d, h.size() * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess)
    throw std::runtime_error("hipMemcpy D2H failed");
}

static float max_abs_err(const std::vector<float>& a, const std::vector<float>& b) {
  float m = 0.0f;
  for (size_t i = 0; i < a.size(); ++i) m = std::fmax(m, std::fabs(a[i] - b[i]));
  return m;
}

static void run(const char* name, const std::function<void()>& fn) {
  try {
    fn();
    std::printf("test %s ... ok\n", name);
  } catch (const std::exception& e) {
    ++g_failed;
    std::printf("test %s ... FAILED (%s)\n", name, e.what());
  }
}

// tests/kernels.rs:60-72
static void test_rms_norm() {
  const size_t dim = 128;
  std::vector<float> x(dim), w(dim, 1.0f);
  for (size_t i = 0; i < dim; ++i) x[i] = (float)i * 0.02f - 1.28f;
  auto dx = upload(x), dw = upload(w);
  K::DeviceBuffer<float> out(dim);
  K::rms_norm(out, dx, dw, 1, dim, 1e-6f);
  auto o = download(out);
  double ss = 0;
  for (float v : o) ss += (double)v * v;
  const double rms = std::sqrt(ss / dim);
  EXPECT(std::fabs(rms - 1.0) < 0.01, "RMS norm output should have RMS ~1.0, got %f", rms);
}

// tests/kernels.rs:74-89
static void test_layer_norm() {
  const size_t dim = 128;
  std::vector<float> x(dim), w(dim, 1.0f), b(dim, 0.0f);
  for (size_t i = 0; i < dim; ++i) x[i] = (float)i * 0.05f - 3.2f;
  auto dx = upload(x), dw = upload(w), db = upload(b);
  K::DeviceBuffer<float> out(dim);
  K::layer_norm(out, dx, dw, db, 1, dim, 1e-5f);
  auto o = download(out);
  double mean = 0, var = 0;
  for (float v : o) mean += v;
  mean /= dim;
  for (float v : o) var += (v - mean) * (v - mean);
  var /= dim;
  EXPECT(std::fabs(mean) < 0.01, "LayerNorm mean should be ~0, got %f", mean);
  EXPECT(std::fabs(var - 1.0) < 0.02, "LayerNorm variance should be ~1, got %f", var);
}

// The encoder's PE add fused into layer 0's LayerNorm equals the two passes
// (encoder.rs:341-343, 370-371), x and the normalised rows alike, bit for bit.
static void test_pe_add_layer_norm() {
  const size_t rows = 40, dim = 896, n_pos = 13;
  std::vector<float> x(rows * dim), w(dim), b(dim);
  for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.37f * (float)i) * 2.0f;
  for (size_t i = 0; i < dim; ++i) {
    w[i] = 1.0f + 0.1f * std::cos((float)i);
    b[i] = 0.02f * std::sin(3.0f * (float)i);
  }
  K::DeviceBuffer<float> pe(n_pos * dim);
  K::sinusoidal_pe(pe, n_pos, dim);
  auto xa = upload(x), xb = upload(x), dw = upload(w), db = upload(b);
  K::DeviceBuffer<float> oa(rows * dim), ob(rows * dim);
  K::pe_add_layer_norm(xa, pe, oa, dw, db, rows, dim, n_pos, 1e-5f);
  K::pe_add(xb, pe, rows, dim, n_pos);
  K::layer_norm(ob, xb, dw, db, rows, dim, 1e-5f);
  const auto hxa = download(xa), hxb = download(xb), hoa = download(oa), hob = download(ob);
  EXPECT(std::memcmp(hxa.data(), hxb.data(), hxa.size() * 4) == 0, "x differs from pe_add");
  EXPECT(std::memcmp(hoa.data(), hob.data(), hoa.size() * 4) == 0, "out differs from layer_norm");
}

// An encoder residual add fused into the LayerNorm that reads its rows equals
// add_inplace + layer_norm bit for bit (encoder.rs:386 + 389-390).
static void test_add_layer_norm() {
  const size_t rows = 40, dim = 1024;
  std::vector<float> x(rows * dim), d(rows * dim), w(dim), b(dim);
  for (size_t i = 0; i < x.size(); ++i) {
    x[i] = std::sin(0.37f * (float)i) * 2.0f;
    d[i] = std::cos(0.11f * (float)i);
  }
  for (size_t i = 0; i < dim; ++i) {
    w[i] = 1.0f + 0.1f * std::cos((float)i);
    b[i] = 0.02f * std::sin(3.0f * (float)i);
  }
  auto xa = upload(x), xb = upload(x), dd = upload(d), dw = upload(w), db = upload(b);
  K::DeviceBuffer<float> oa(rows * dim), ob(rows * dim);
  K::add_layer_norm(xa, dd, dw, db, oa, rows, dim, 1e-5f);
  K::add_inplace(xb, dd, rows * dim);
  K::layer_norm(ob, xb, dw, db, rows, dim, 1e-5f);
  const auto hxa = download(xa), hxb = download(xb), hoa = download(oa), hob = download(ob);
  EXPECT(std::memcmp(hxa.data(), hxb.data(), hxa.size() * 4) == 0, "x differs from add_inplace");
  EXPECT(std::memcmp(hoa.data(), hob.data(), hoa.size() * 4) == 0, "out differs from layer_norm");
}

// tests/kernels.rs:105-113, for both GELU forms
static void test_gelu() {
  for (int erf_form = 0; erf_form < 2; ++erf_form) {
    std::vector<float> x = {0.0f, 1.0f, -1.0f, 2.0f, -0.5f};
    auto d = upload(x);
    if (erf_form) K::gelu_erf(d, x.size()); else K::gelu(d, x.size());
    auto o = download(d);
    EXPECT(std::fabs(o[0]) < 1e-5f, "GELU(0) should be ~0");
    EXPECT(o[1] > 0.5f, "GELU(1) should be > 0.5");
    EXPECT(o[2] < 0.0f, "GELU(-1) should be negative");
  }
}

// tests/kernels.rs:115-124
static void test_silu() {
  std::vector<float> orig = {0.0f, 1.0f, -1.0f, 5.0f}, expected(4);
  for (int i = 0; i < 4; ++i) expected[i] = orig[i] / (1.0f + std::exp(-orig[i]));
  auto d = upload(orig);
  K::silu(d, 4);
  const float err = max_abs_err(download(d), expected);
  EXPECT(err < 1e-5f, "SiLU mismatch, max_err=%g", err);
}

// tests/kernels.rs:126-152 (the vector ops on the path: add_inplace)
static void test_vec_ops() {
  const size_t n = 256;
  std::vector<float> a(n), b(n);
  for (size_t i = 0; i < n; ++i) {
    a[i] = (float)i * 0.1f;
    b[i] = (float)(n - i) * 0.1f;
  }
  auto da = upload(a), db = upload(b);
  K::add_inplace(da, db, n);
  auto o = download(da);
  for (size_t i = 0; i < n; ++i) EXPECT(std::fabs(o[i] - (a[i] + b[i])) < 1e-5f, "add at %zu", i);
}

// RopeCache + apply_rope_neox: position 0 is the identity; the table grows by
// doubling from 1024 and keeps its rows.
static void test_rope_cache() {
  K::RopeCache rope;
  rope.ensure(10, 128, 1e6f);
  EXPECT(rope.cap() == 1024, "initial capacity 1024, got %zu", rope.cap());
  std::vector<float> x(2 * 128);
  for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin((float)i);
  auto dx = upload(x);
  K::apply_rope_neox(dx, rope.cos_range(0, 1), rope.sin_range(0, 1), 1, 2, 128);
  auto o = download(dx);
  for (size_t i = 0; i < x.size(); ++i) EXPECT(o[i] == x[i], "pos 0 must be identity at %zu", i);
  std::vector<float> row(128);
  copy_row(row, rope.cos_at(700).ptr);
  rope.ensure(3000, 128, 1e6f);
  EXPECT(rope.cap() == 4096, "grown capacity 4096, got %zu", rope.cap());
  std::vector<float> row2(128);
  copy_row(row2, rope.cos_at(700).ptr);
  EXPECT(row == row2, "growth must keep existing rows");
  EXPECT(std::fabs(row2[0] - std::cos(700.0f)) < 1e-6f, "cos(700) column 0");
}

// Decoder layer step with the KV store fused in: the cache rows equal the k/v
// rows the separate norm + rope + copy produce, the rest of the cache stays 0,
// and growing the cache keeps them.
static void test_kv_store() {
  const size_t seq = 3, nq = 2, nk = 1, hd = 128, start = 4, kv = nk * hd;
  K::KvCache cache(2, 8, kv);
  K::RopeCache rope;
  rope.ensure(start + seq, hd, 1e6f);
  std::vector<float> q(seq * nq * hd), k(seq * kv), v(seq * kv), w(hd, 1.0f);
  for (size_t i = 0; i < q.size(); ++i) q[i] = std::sin(0.1f * (float)i);
  for (size_t i = 0; i < k.size(); ++i) { k[i] = std::cos(0.07f * (float)i); v[i] = (float)i; }
  auto dq = upload(q), dk = upload(k), dv = upload(v), dw = upload(w);
  K::head_rms_norm_rope_kv(dq, dk, dv, dw, dw, rope, start, seq, nq, nk, hd, 1e-6f,
                           cache.k_block(1), cache.v_block(1), cache.max_seq());
  // reference path: per-head norm, rope on rows start.., copy
  auto dk2 = upload(k);
  K::rms_norm_per_head(dk2, dw, seq, nk, hd, 1e-6f);
  K::apply_rope_neox(dk2, rope.cos_range(start, seq), rope.sin_range(start, seq), seq, nk, hd);
  auto kref = download(dk2);
  std::vector<float> kc(8 * kv), vc(8 * kv);
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(kc.data(), cache.k_block(1).ptr, kc.size() * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(vc.data(), cache.v_block(1).ptr, vc.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
    throw std::runtime_error("copy back failed");
  for (size_t s = 0; s < 8; ++s)
    for (size_t d = 0; d < kv; ++d) {
      const bool row = s >= start && s < start + seq;
      const float ke = row ? kref[(s - start) * kv + d] : 0.0f, ve = row ? v[(s - start) * kv + d] : 0.0f;
      EXPECT(kc[s * kv + d] == ke && vc[s * kv + d] == ve, "cache row %zu col %zu", s, d);
    }
  cache.len = start + seq;
  cache.grow(20);
  EXPECT(cache.max_seq() == 32, "grown to 32, got %zu", cache.max_seq());
  std::vector<float> kc2(cache.len * kv);
  if (hipDeviceSynchronize() != hipSuccess ||
      hipMemcpy(kc2.data(), cache.k_layer(1).ptr, kc2.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
    throw std::runtime_error("copy back failed");
  for (size_t i = 0; i < kc2.size(); ++i) EXPECT(kc2[i] == kc[i], "grow kept element %zu", i);
}

// linear_nobias_int8 with integer inputs and unit scales is exact.
static void test_linear_int8_exact() {
  const size_t in = 2048, out_dim = 64;
  std::vector<int8_t> w(in * out_dim);
  std::vector<float> x(in), s(out_dim, 1.0f);
  for (size_t i = 0; i < w.size(); ++i) w[i] = (int8_t)((int)(i * 2654435761u >> 7) % 255 - 127);
  for (size_t k = 0; k < in; ++k) x[k] = (float)((int)(k % 41) - 20);
  auto dw = upload(w);
  auto dx = upload(x), ds = upload(s);
  K::DeviceBuffer<float> y(out_dim);
  K::linear_nobias_int8(y, dx, dw, ds, 1, in, out_dim);
  auto o = download(y);
  for (size_t r = 0; r < out_dim; ++r) {
    long long dot = 0;
    for (size_t k = 0; k < in; ++k) dot += (long long)w[r * in + k] * (long long)x[k];
    EXPECT((long long)o[r] == dot, "row %zu: %f vs %lld", r, o[r], dot);
  }
}

// The decode-step folds through the C++ mirror equal the unfused calls bit for bit:
// add + RMSNorm + q/k/v, add + RMSNorm + gate/up + SwiGLU, the prefill gate/up + SwiGLU.
static void test_decode_folds() {
  const size_t H = 2048, I = 512, qo = 2048, kvo = 1024, T = 24;
  auto pseudo = [](size_t i, int span) { return (int)((i * 2654435761u) >> 9) % span - span / 2; };
  std::vector<float> x(H), d(H), g(H), xt(T * H);
  for (size_t k = 0; k < H; ++k) {
    x[k] = pseudo(k, 2001) / 1000.0f;
    d[k] = pseudo(k + 7, 2001) / 1000.0f;
    g[k] = 1.0f + pseudo(k + 13, 201) / 1000.0f;
  }
  for (size_t k = 0; k < T * H; ++k) xt[k] = pseudo(k + 29, 2001) / 1000.0f;
  auto mk_w = [&](size_t rows, size_t salt) {
    std::vector<int8_t> w(rows * H);
    for (size_t i = 0; i < w.size(); ++i) w[i] = (int8_t)pseudo(i + salt, 255);
    return w;
  };
  auto mk_s = [&](size_t rows) { return std::vector<float>(rows, 1.0f / 4096.0f); };
  auto wq = upload(mk_w(qo, 1)), wk = upload(mk_w(kvo, 2)), wv = upload(mk_w(kvo, 3)), wgu = upload(mk_w(2 * I, 4));
  auto sq = upload(mk_s(qo)), sk = upload(mk_s(kvo)), sv = upload(mk_s(kvo)), sgu = upload(mk_s(2 * I));
  auto dx = upload(x), dd = upload(d), dg = upload(g), dxt = upload(xt);
  const float eps = 1e-6f;
  // unfused: add_rms_norm on a copy, then the projections
  auto xa = upload(x);
  K::DeviceBuffer<float> xn(H), q0(qo), k0(kvo), v0(kvo), q1(qo), k1(kvo), v1(kvo), h(H);
  K::add_rms_norm(xa, dd, dg, xn, 1, H, eps);
  K::linear_nobias_int8_multi({q0, k0, v0}, {wq, wk, wv}, {sq, sk, sv}, {qo, kvo, kvo}, xn, 1, H);
  K::add_rms_norm_linear_nobias_int8_multi({q1, k1, v1}, {wq, wk, wv}, {sq, sk, sv}, {qo, kvo, kvo}, h, dx, dd,
                                           dg, H, eps);
  EXPECT(download(q0) == download(q1) && download(k0) == download(k1) && download(v0) == download(v1),
         "q/k/v differ");
  EXPECT(download(h) == download(xa), "residual differs");
  K::DeviceBuffer<float> o0(I), o1(I);
  K::gate_up_swiglu_int8(o0, xn, wgu, sgu, 1, H, I);
  K::add_rms_norm_gate_up_swiglu_int8(o1, h, dx, dd, dg, wgu, sgu, H, I, eps);
  EXPECT(download(o0) == download(o1), "gate/up SwiGLU differs");
  // prefill: GEMM + swiglu_multiply vs the fused epilogue (24 tokens: the matrix-core path)
  K::DeviceBuffer<float> gu(T * 2 * I), p0(T * I), p1(T * I);
  K::linear_nobias_int8(gu, dxt, wgu, sgu, T, H, 2 * I);
  K::swiglu_multiply(p0, gu, T, I);
  K::gate_up_swiglu_multiply_int8(p1, dxt, wgu, sgu, T, H, I);
  EXPECT(download(p0) == download(p1), "prefill gate/up SwiGLU differs");
}

// Attention over one key returns that key's value row exactly (softmax weight
// exp(0)/1); two identical keys average their values; the key-split form
// agrees with the single-pass form.
static void test_causal_attention() {
  const size_t nh = 16, nk = 8, hd = 128;
  std::vector<float> q(nh * hd), k(300 * nk * hd), v(300 * nk * hd);
  for (size_t i = 0; i < q.size(); ++i) q[i] = std::sin(0.37f * (float)i);
  for (size_t i = 0; i < k.size(); ++i) k[i] = std::cos(0.11f * (float)i) * 0.5f;
  for (size_t i = 0; i < v.size(); ++i) v[i] = std::sin(0.05f * (float)i + 1.0f);
  auto dq = upload(q), dk = upload(k), dv = upload(v);
  K::DeviceBuffer<float> out(nh * hd), out2(nh * hd);
  const float scale = 1.0f / std::sqrt((float)hd);
  K::causal_attention(out, dq, dk, dv, 1, 1, nh, nk, hd, scale, 0);
  auto o = download(out);
  for (size_t h = 0; h < nh; ++h)
    for (size_t d = 0; d < hd; ++d)
      EXPECT(o[h * hd + d] == v[(h / (nh / nk)) * hd + d], "head %zu dim %zu", h, d);
  std::vector<float> k2(k.begin(), k.begin() + 2 * nk * hd);
  for (size_t i = 0; i < nk * hd; ++i) k2[nk * hd + i] = k2[i];  // key 1 == key 0
  auto dk2 = upload(k2);
  K::causal_attention(out, dq, dk2, dv, 1, 2, nh, nk, hd, scale, 1);
  o = download(out);
  for (size_t h = 0; h < nh; ++h)
    for (size_t d = 0; d < hd; ++d) {
      const size_t c = (h / (nh / nk)) * hd + d;
      const float want = 0.5f * (v[c] + v[nk * hd + c]);
      EXPECT(std::fabs(o[h * hd + d] - want) <= 1e-6f, "head %zu dim %zu", h, d);
    }
  K::DeviceBuffer<float> ws(K::attention_workspace_floats(1, nh, hd));
  K::causal_attention(out, dq, dk, dv, 1, 300, nh, nk, hd, scale, 299);
  K::causal_attention(out2, dq, dk, dv, 1, 300, nh, nk, hd, scale, 299, ws);
  const auto a = download(out), b = download(out2);
  for (size_t i = 0; i < a.size(); ++i)
    EXPECT(std::fabs(a[i] - b[i]) <= 1e-5f + 1e-5f * std::fabs(a[i]), "elem %zu: %f vs %f", i, a[i], b[i]);
}

// lm_head: equal maxima go to the lower index, with and without the workspace.
static void test_lm_head_argmax() {
  const size_t in = 1024, vocab = 5000;
  std::vector<int8_t> w(vocab * in);
  for (size_t i = 0; i < w.size(); ++i) w[i] = (int8_t)((int)(i * 2654435761u >> 9) % 7 - 3);
  for (size_t r : {4321u, 3u, 777u})
    for (size_t c = 0; c < in; ++c) w[r * in + c] = 127;
  std::vector<float> x(in, 1.0f), sc(vocab, 1e-3f);
  sc[4321] = sc[3] = sc[777] = 1.0f;
  auto dw = upload(w);
  auto dx = upload(x), ds = upload(sc);
  K::DeviceBuffer<float> logits(vocab);
  K::DeviceBuffer<int32_t> idx(1);
  K::DeviceBuffer<uint8_t> ws(K::lm_head_workspace_bytes(vocab));
  K::lm_head_int8_argmax(idx, logits, dx, dw, ds, 1, in, vocab, ws);
  EXPECT(download(idx)[0] == 3, "fused: %d", download(idx)[0]);
  K::lm_head_int8_argmax(idx, logits, dx, dw, ds, 1, in, vocab);
  EXPECT(download(idx)[0] == 3, "unfused: %d", download(idx)[0]);
}

// .qint8: a V2 file written byte by byte (quantize.rs:1-34) reads back, uploads
// bit-exactly, and the gate/up pair lands row-interleaved.
static void test_qint8_file() {
  std::string bytes = std::string("QINT8\x02\x00\x00", 8);
  auto u16 = [&](uint16_t v) { bytes.append(reinterpret_cast<const char*>(&v), 2); };
  auto u32 = [&](uint32_t v) { bytes.append(reinterpret_cast<const char*>(&v), 4); };
  auto u64 = [&](uint64_t v) { bytes.append(reinterpret_cast<const char*>(&v), 8); };
  auto entry = [&](const std::string& n, uint8_t dt, std::vector<uint32_t> shape, uint64_t d, uint64_t s) {
    u16((uint16_t)n.size());
    bytes += n;
    bytes.push_back((char)dt);
    bytes.push_back((char)shape.size());
    for (uint32_t x : shape) u32(x);
    u64(d);
    u64(s);
  };
  u32(3);
  u32(0);
  entry("g", 0, {2, 4}, 0, 8);
  entry("u", 0, {2, 4}, 16, 24);
  entry("n", 1, {3}, 32, 0);
  const int8_t g[8] = {1, 2, 3, 4, -1, -2, -3, -4}, u[8] = {5, 6, 7, 8, -5, -6, -7, -8};
  const float gs[2] = {0.5f, 0.25f}, us[2] = {2.0f, 4.0f}, n[3] = {1.5f, -2.5f, 3.25f};
  bytes.append(reinterpret_cast<const char*>(g), 8);
  bytes.append(reinterpret_cast<const char*>(gs), 8);
  bytes.append(reinterpret_cast<const char*>(u), 8);
  bytes.append(reinterpret_cast<const char*>(us), 8);
  bytes.append(reinterpret_cast<const char*>(n), 12);
  const char* tmp = std::getenv("TMPDIR");
  const std::string path = std::string(tmp ? tmp : "/tmp") + "/qasr_cpp_test_" +
                           std::to_string((long)getpid()) + ".qint8";
  FILE* f = std::fopen(path.c_str(), "wb");
  EXPECT(f, "cannot write %s", path.c_str());
  std::fwrite(bytes.data(), 1, bytes.size(), f);
  std::fclose(f);
  {
    auto qf = K::QuantFile::open(path);
    EXPECT(qf.has_value(), "open failed");
    EXPECT(qf->version() == 2 && qf->tensors().size() == 3, "table");
    const auto* m = qf->find("n");
    EXPECT(m && m->dtype == QASR_QINT8_F32 && m->numel() == 3, "n meta");
    EXPECT(qf->find("missing") == nullptr, "find missing");
    K::DeviceBuffer<float> dn(3), dsc(4);
    qf->upload("n", dn.data(), 12);
    const auto hn = download(dn);
    EXPECT(hn[0] == n[0] && hn[1] == n[1] && hn[2] == n[2], "f32 upload");
    K::DeviceBuffer<int8_t> dw(16);
    qf->upload_gate_up("g", "u", 2, 4, dw, dsc);
    const auto hw = download(dw);
    const auto hs = download(dsc);
    const int8_t want[16] = {1, 2, 3, 4, 5, 6, 7, 8, -1, -2, -3, -4, -5, -6, -7, -8};
    for (int i = 0; i < 16; ++i) EXPECT(hw[i] == want[i], "fused byte %d", i);
    EXPECT(hs[0] == 0.5f && hs[1] == 2.0f && hs[2] == 0.25f && hs[3] == 4.0f, "fused scales");
  }
  std::remove(path.c_str());
  EXPECT(!K::QuantFile::open(path).has_value(), "a missing file opens as nothing");
}

// A short slice panics before anything is launched (the reference's slice
// index panic).
static void test_short_slice_panics() {
  K::DeviceBuffer<float> out(100), x(128), w(128);
  bool threw = false;
  try {
    K::rms_norm(out, x, w, 1, 128, 1e-6f);
  } catch (const K::Panic&) {
    threw = true;
  }
  EXPECT(threw, "rms_norm with a 100-element out slice must panic");
  threw = false;
  try {
    K::DevSlice<float>(out.data(), 100).sub(90, 20);
  } catch (const K::Panic&) {
    threw = true;
  }
  EXPECT(threw, "sub-slice past the end must panic");
}

// A C-ABI contract breach surfaces as QasrError with the status code.
static void test_status_errors() {
  K::DeviceBuffer<float> x(2 * 4 * 127), c(2 * 127), s(2 * 127);
  bool threw = false;
  try {
    K::apply_rope_neox(x, c, s, 2, 4, 127);  // odd head_dim
  } catch (const K::QasrError& e) {
    threw = e.code == QASR_ERR_INVALID_ARG;
  }
  EXPECT(threw, "odd head_dim must return QASR_ERR_INVALID_ARG");
}

int main() {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
    std::printf("no GPU visible\n");
    return 2;
  }
  run("test_rms_norm", test_rms_norm);
  run("test_layer_norm", test_layer_norm);
  run("test_pe_add_layer_norm", test_pe_add_layer_norm);
  run("test_add_layer_norm", test_add_layer_norm);
  run("test_gelu", test_gelu);
  run("test_silu", test_silu);
  run("test_vec_ops", test_vec_ops);
  run("test_rope_cache", test_rope_cache);
  run("test_kv_store", test_kv_store);
  run("test_linear_int8_exact", test_linear_int8_exact);
  run("test_decode_folds", test_decode_folds);
  run("test_causal_attention", test_causal_attention);
  run("test_lm_head_argmax", test_lm_head_argmax);
  run("test_qint8_file", test_qint8_file);
  run("test_short_slice_panics", test_short_slice_panics);
  run("test_status_errors", test_status_errors);
  std::printf("%s: %d failed\n", g_failed ? "FAILED" : "ok", g_failed);
  return g_failed ? 1 : 0;
}
