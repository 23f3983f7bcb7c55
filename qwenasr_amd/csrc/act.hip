// Activations and position embeddings: SwiGLU (interleaved and split), SiLU,
// GELU (tanh reference form and exact erf form), sinusoidal PE and PE add.
//
// All are streaming kernels: grid-stride loops over float4, each element read
// and written once. The vector path needs 16-byte aligned pointers and a
// multiple-of-4 length (per row where rows matter); anything else takes the
// scalar kernels with identical arithmetic.
#include "common.hpp"

namespace qasr {
namespace {


// ---------------------------------------------------------------------------
// SwiGLU on the interleaved gate/up buffer, x86_64 reference arithmetic
// (avx.rs:565-599): columns j < (inter & ~7) use g / (1 + fast_exp(0 - g)),
// the row tail uses g / (1 + expf(-g)); out = silu * u.
// ---------------------------------------------------------------------------


// One output float4 per thread over an exact grid. Without a row tail
// (inter % 8 == 0) every column takes the fast_exp path and no row index is
// needed; with one, the column comes from a 32-bit division.
template <bool HAS_TAIL>
__global__ __launch_bounds__(256) void swiglu_interleaved_vec_kernel(
    float* out, const float* gu, size_t n4, unsigned i4, unsigned fast_end) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const float4 a = ld4_nt(gu, 2 * i);      // g_j, u_j, g_j+1, u_j+1
  const float4 b = ld4_nt(gu, 2 * i + 1);  // g_j+2, u_j+2, g_j+3, u_j+3
  bool fast = true;
  if constexpr (HAS_TAIL) {
    const unsigned j = (unsigned)(i % i4) * 4;
    fast = j < fast_end;  // a 4-block never straddles an 8-block edge
  }
  float4 o;
  o.x = swiglu_ref(a.x, a.y, fast);
  o.y = swiglu_ref(a.z, a.w, fast);
  o.z = swiglu_ref(b.x, b.y, fast);
  o.w = swiglu_ref(b.z, b.w, fast);
  st4_nt(out, i, o);
}

__global__ __launch_bounds__(256) void swiglu_interleaved_scalar_kernel(
    float* out, const float* gu, size_t rows, int inter) {
  const int fast_end = inter & ~7;
  const size_t n = rows * (size_t)inter;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const size_t r = i / inter;
    const int j = (int)(i - r * inter);
    const float* src = gu + r * 2 * (size_t)inter + 2 * j;
    out[i] = swiglu_ref(src[0], src[1], j < fast_end);
  }
}

// ---------------------------------------------------------------------------
// Split-layout SwiGLU and SiLU, libm arithmetic (decoder.rs:916-921,
// kernels/mod.rs:941-946, 988-994).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void swiglu_split_vec_kernel(float* out, const float* g,
                                                               const float* u, size_t n4) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const float4 a = ld4_nt(g, i);
  const float4 b = ld4_nt(u, i);
  float4 o;
  o.x = silu_expf(a.x) * b.x;
  o.y = silu_expf(a.y) * b.y;
  o.z = silu_expf(a.z) * b.z;
  o.w = silu_expf(a.w) * b.w;
  st4_nt(out, i, o);
}

__global__ __launch_bounds__(256) void swiglu_split_scalar_kernel(float* out, const float* g,
                                                                  const float* u, size_t begin,
                                                                  size_t n) {
  for (size_t i = begin + (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (size_t)gridDim.x * 256) {
    out[i] = silu_expf(g[i]) * u[i];
  }
}

__global__ __launch_bounds__(256) void silu_kernel(float* x, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    x[i] = silu_expf(x[i]);
  }
}

// ---------------------------------------------------------------------------
// GELU
// ---------------------------------------------------------------------------
// tanh form, x86_64 reference arithmetic: elements i < (n & ~7) follow
// avx.rs:543-554, the tail follows the scalar loop avx.rs:556-562.
QASR_DEV float gelu_tanh_ref(float v, bool fast) {
  if (fast) {
    const float v2 = v * v;
    const float v3 = v2 * v;
    const float inner = 0.7978845608028654f * __builtin_fmaf(0.044715f, v3, v);
    const float e = ref_fast_exp(2.0f * inner);
    const float th = 1.0f - 2.0f / (e + 1.0f);
    return 0.5f * (v * (1.0f + th));
  }
  const float x3 = (v * v) * v;
  const float inner = 0.7978845608028654f * (v + 0.044715f * x3);
  return (0.5f * v) * (1.0f + tanhf(inner));
}

// Exact GELU, 0.5*x*(1+erf(x/sqrt2)) = x*sigmoid(Q(x)) with
// Q(x) = 2*artanh(erf(x/sqrt2)) approximated on |x| <= 6 by the odd polynomial
// x*P(x^2) below (weighted minimax fit; gelu_erf_fit.py derives the
// coefficients and bounds the float32 error of exactly this evaluation by
// 3.1e-7 absolute against float64, including 1-ulp error in exp2 and rcp).
//   e = exp(-|q|) <= 1, t = x*e/(1+e) = x*sigmoid(-|q|)
//   gelu = x - t (x >= 0), t (x < 0), 0 (x < -6)
// Neither branch cancels and nothing overflows. ~20 VALU per element.
QASR_DEV float gelu_erf(float x) {
  constexpr float c0 = 1.5957684516906738f, c1 = 0.07266856729984283f;
  constexpr float c2 = -6.625994137721136e-05f, c3 = -0.00011048033047700301f;
  constexpr float c4 = 7.938220733194612e-06f, c5 = -2.668929255378316e-07f;
  constexpr float c6 = 3.6112353107853323e-09f;
  const float xc = fminf(fmaxf(x, -6.0f), 6.0f);
  const float x2 = xc * xc;
  float p = __builtin_fmaf(c6, x2, c5);
  p = __builtin_fmaf(p, x2, c4);
  p = __builtin_fmaf(p, x2, c3);
  p = __builtin_fmaf(p, x2, c2);
  p = __builtin_fmaf(p, x2, c1);
  p = __builtin_fmaf(p, x2, c0);
  const float q = xc * p;
  const float e = __builtin_amdgcn_exp2f(fabsf(q) * -1.4426950408889634f);
  const float t = (x * e) * __builtin_amdgcn_rcpf(1.0f + e);
  const float g = x >= 0.0f ? x - t : t;
  // beyond the clamp: exact tails (x * Phi(x) rounds to x above 6 and its
  // magnitude is below 6e-9 under -6); this also keeps +inf -> +inf
  return x > 6.0f ? x : (x < -6.0f ? 0.0f : g);
}

template <bool ERF>
__global__ __launch_bounds__(256) void gelu_vec_kernel(float* x, size_t n4, size_t fast_end) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  float4 v = ld4_nt(x, i);
  if constexpr (ERF) {
    v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
  } else {
    const bool f = 4 * i < fast_end;
    v.x = gelu_tanh_ref(v.x, f); v.y = gelu_tanh_ref(v.y, f);
    v.z = gelu_tanh_ref(v.z, f); v.w = gelu_tanh_ref(v.w, f);
  }
  st4_nt(x, i, v);
}

template <bool ERF>
__global__ __launch_bounds__(256) void gelu_scalar_kernel(float* x, size_t begin, size_t n,
                                                          size_t fast_end) {
  for (size_t i = begin + (size_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (size_t)gridDim.x * 256) {
    if constexpr (ERF) {
      x[i] = gelu_erf(x[i]);
    } else {
      x[i] = gelu_tanh_ref(x[i], i < fast_end);
    }
  }
}

// ---------------------------------------------------------------------------
// Sinusoidal PE (kernels/mod.rs:1213-1226):
//   inv[d] = exp(-(d as f32) * log_ts), angle = (p as f32) * inv[d] (f32),
//   row[d] = sin(angle), row[half+d] = cos(angle).
// exp/sin/cos are evaluated in double and rounded once to f32.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void sinusoidal_pe_kernel(float* pe, long long n_items, int d_model,
                                                            float log_ts) {
  const int half = d_model / 2;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n_items;
       i += (long long)gridDim.x * 256) {
    const long long p = i / half;
    const int d = (int)(i % half);
    const float arg = -(float)d * log_ts;
    const float inv = (float)exp((double)arg);
    const float angle = (float)p * inv;
    pe[p * d_model + d] = (float)sin((double)angle);
    pe[p * d_model + half + d] = (float)cos((double)angle);
    // an odd d_model leaves the last column unwritten; the reference's table
    // is zero-initialised there
    if ((d_model & 1) && d == 0) pe[p * d_model + d_model - 1] = 0.0f;
  }
}

// x[r,:] += pe[r % n_pos, :]: one workgroup per row, so the PE row index is
// computed once per row (the 13-row table stays in L2).
__global__ __launch_bounds__(256) void pe_add_vec_kernel(float* x, const float* pe, int d4,
                                                         int n_pos) {
  const size_t r = blockIdx.x;
  const float* pr = pe + (size_t)(r % (size_t)n_pos) * d4 * 4;
  float* xr = x + r * (size_t)d4 * 4;
  for (int c = threadIdx.x; c < d4; c += 256) {
    float4 v = ld4_nt(xr, c);
    const float4 p = ld4(pr, c);
    v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
    st4_nt(xr, c, v);
  }
}

__global__ __launch_bounds__(256) void pe_add_scalar_kernel(float* x, const float* pe, size_t rows,
                                                            int d_model, int n_pos) {
  const size_t n = rows * (size_t)d_model;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const size_t r = i / d_model;
    const int c = (int)(i - r * d_model);
    x[i] += pe[(size_t)(r % n_pos) * d_model + c];
  }
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_swiglu_multiply_f32(float* out, const float* gate_up, size_t seq_len,
                                        size_t intermediate, void* stream) {
  if (seq_len == 0 || intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && gate_up, "swiglu_multiply: null pointer");
  size_t n;
  QASR_REQUIRE(mul_ok(seq_len, 2 * intermediate, &n) && intermediate < 0x3fffffffu,
               "swiglu_multiply: size overflows");
  hipStream_t st = as_stream(stream);
  const int inter = (int)intermediate;
  if (intermediate % 4 == 0 && aligned16(out) && aligned16(gate_up) &&
      exact_grid_ok(seq_len * (intermediate / 4))) {
    const size_t n4 = seq_len * (intermediate / 4);
    const unsigned grid = (unsigned)((n4 + 255) / 256);
    if (intermediate % 8 == 0) {
      swiglu_interleaved_vec_kernel<false><<<grid, 256, 0, st>>>(out, gate_up, n4, 0, 0);
    } else {
      swiglu_interleaved_vec_kernel<true><<<grid, 256, 0, st>>>(
          out, gate_up, n4, (unsigned)(intermediate / 4), (unsigned)(intermediate & ~(size_t)7));
    }
  } else {
    swiglu_interleaved_scalar_kernel<<<grid_for(seq_len * intermediate, 256), 256, 0, st>>>(
        out, gate_up, seq_len, inter);
  }
  return launch_status("swiglu_multiply");
}

extern "C" int qasr_swiglu_split_f32(float* out, const float* gate, const float* up, size_t n,
                                     void* stream) {
  if (n == 0) return QASR_OK;
  QASR_REQUIRE(out && gate && up, "swiglu_split: null pointer");
  QASR_REQUIRE(n <= kMaxElems, "swiglu_split: n too large");
  hipStream_t st = as_stream(stream);
  size_t done = 0;
  if (aligned16(out) && aligned16(gate) && aligned16(up) && exact_grid_ok(n / 4)) {
    const size_t n4 = n / 4;
    if (n4) swiglu_split_vec_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, st>>>(out, gate, up, n4);
    done = n4 * 4;
  }
  if (done < n) {
    swiglu_split_scalar_kernel<<<grid_for(n - done, 256), 256, 0, st>>>(out, gate, up, done, n);
  }
  return launch_status("swiglu_split");
}

extern "C" int qasr_silu_f32(float* x, size_t n, void* stream) {
  if (n == 0) return QASR_OK;
  QASR_REQUIRE(x, "silu: null pointer");
  QASR_REQUIRE(n <= kMaxElems, "silu: n too large");
  silu_kernel<<<grid_for(n, 256), 256, 0, as_stream(stream)>>>(x, n);
  return launch_status("silu");
}

template <bool ERF>
static int launch_gelu(float* x, size_t n, void* stream) {
  if (n == 0) return QASR_OK;
  QASR_REQUIRE(x, "gelu: null pointer");
  QASR_REQUIRE(n <= kMaxElems, "gelu: n too large");
  hipStream_t st = as_stream(stream);
  const size_t fast_end = n & ~(size_t)7;
  size_t done = 0;
  if (aligned16(x) && exact_grid_ok(n / 4)) {
    const size_t n4 = n / 4;
    if (n4) gelu_vec_kernel<ERF><<<(unsigned)((n4 + 255) / 256), 256, 0, st>>>(x, n4, fast_end);
    done = n4 * 4;
  }
  if (done < n) {
    gelu_scalar_kernel<ERF><<<grid_for(n - done, 256), 256, 0, st>>>(x, done, n, fast_end);
  }
  return launch_status(ERF ? "gelu_erf" : "gelu_tanh");
}

extern "C" int qasr_gelu_tanh_f32(float* x, size_t n, void* stream) {
  return launch_gelu<false>(x, n, stream);
}

extern "C" int qasr_gelu_erf_f32(float* x, size_t n, void* stream) {
  return launch_gelu<true>(x, n, stream);
}

extern "C" int qasr_sinusoidal_pe_f32(float* pe, size_t n_pos, size_t d_model, void* stream) {
  if (n_pos == 0 || d_model < 2) return QASR_OK;
  QASR_REQUIRE(pe, "sinusoidal_pe: null pointer");
  QASR_REQUIRE(n_pos <= ((size_t)1 << 24) && d_model <= ((size_t)1 << 20),
               "sinusoidal_pe: size too large");
  const int half = (int)(d_model / 2);
  // kernels/mod.rs:1215: log_timescale = ln(10000) / (half - 1), in f32.
  const float log_ts = logf(10000.0f) / (float)(half - 1);
  const long long items = (long long)n_pos * half;
  sinusoidal_pe_kernel<<<grid_for((size_t)items, 256), 256, 0, as_stream(stream)>>>(
      pe, items, (int)d_model, log_ts);
  return launch_status("sinusoidal_pe");
}

extern "C" int qasr_pe_add_f32(float* x, const float* pe, size_t rows, size_t d_model,
                               size_t n_pos, void* stream) {
  if (rows == 0 || d_model == 0) return QASR_OK;
  QASR_REQUIRE(x && pe, "pe_add: null pointer");
  QASR_REQUIRE(n_pos > 0, "pe_add: n_pos must be positive");
  size_t n;
  QASR_REQUIRE(mul_ok(rows, d_model, &n) && d_model < 0x7fffffffu && n_pos < 0x7fffffffu,
               "pe_add: size overflows");
  hipStream_t st = as_stream(stream);
  if (d_model % 4 == 0 && aligned16(x) && aligned16(pe) && rows <= kMaxRows) {
    pe_add_vec_kernel<<<(unsigned)rows, 256, 0, st>>>(x, pe, (int)(d_model / 4), (int)n_pos);
  } else {
    pe_add_scalar_kernel<<<grid_for(n, 256), 256, 0, st>>>(x, pe, rows, (int)d_model, (int)n_pos);
  }
  return launch_status("pe_add");
}
