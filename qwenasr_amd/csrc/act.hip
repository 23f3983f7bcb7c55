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

QASR_DEV float4 ld4(const float* p, size_t i) { return reinterpret_cast<const float4*>(p)[i]; }
QASR_DEV void st4(float* p, size_t i, float4 v) { reinterpret_cast<float4*>(p)[i] = v; }

// ---------------------------------------------------------------------------
// SwiGLU on the interleaved gate/up buffer, x86_64 reference arithmetic
// (avx.rs:565-599): columns j < (inter & ~7) use g / (1 + fast_exp(0 - g)),
// the row tail uses g / (1 + expf(-g)); out = silu * u.
// ---------------------------------------------------------------------------
QASR_DEV float swiglu_ref(float g, float u, bool fast) {
  const float s = fast ? g / (1.0f + ref_fast_exp(0.0f - g)) : g / (1.0f + expf(-g));
  return s * u;
}

__global__ __launch_bounds__(256) void swiglu_interleaved_vec_kernel(
    float* out, const float* gu, size_t rows, int inter) {
  const int i4 = inter >> 2;
  const int fast_end = inter & ~7;
  const size_t n4 = rows * (size_t)i4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const size_t r = i / i4;
    const int j = (int)(i - r * i4) * 4;
    const float* src = gu + r * 2 * (size_t)inter + 2 * j;
    const float4 a = ld4(src, 0);  // g_j, u_j, g_j+1, u_j+1
    const float4 b = ld4(src, 1);  // g_j+2, u_j+2, g_j+3, u_j+3
    const bool fast = j < fast_end;  // a 4-block never straddles an 8-block edge
    float4 o;
    o.x = swiglu_ref(a.x, a.y, fast);
    o.y = swiglu_ref(a.z, a.w, fast);
    o.z = swiglu_ref(b.x, b.y, fast);
    o.w = swiglu_ref(b.z, b.w, fast);
    st4(out, i, o);
  }
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
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const float4 a = ld4(g, i);
    const float4 b = ld4(u, i);
    float4 o;
    o.x = silu_expf(a.x) * b.x;
    o.y = silu_expf(a.y) * b.y;
    o.z = silu_expf(a.z) * b.z;
    o.w = silu_expf(a.w) * b.w;
    st4(out, i, o);
  }
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

// Exact GELU, 0.5*x*(1+erf(x/sqrt2)) written as 0.5*x*erfc(-x/sqrt2) so the
// negative tail keeps its relative accuracy (no 1 + erf cancellation).
QASR_DEV float gelu_erf(float v) { return 0.5f * v * erfcf(-v * 0.70710678118654752f); }

template <bool ERF>
__global__ __launch_bounds__(256) void gelu_vec_kernel(float* x, size_t n4, size_t fast_end) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    float4 v = ld4(x, i);
    if constexpr (ERF) {
      v.x = gelu_erf(v.x); v.y = gelu_erf(v.y); v.z = gelu_erf(v.z); v.w = gelu_erf(v.w);
    } else {
      const bool f = 4 * i < fast_end;
      v.x = gelu_tanh_ref(v.x, f); v.y = gelu_tanh_ref(v.y, f);
      v.z = gelu_tanh_ref(v.z, f); v.w = gelu_tanh_ref(v.w, f);
    }
    st4(x, i, v);
  }
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

// x[r,:] += pe[r % n_pos, :]
__global__ __launch_bounds__(256) void pe_add_vec_kernel(float* x, const float* pe, size_t rows,
                                                         int d4, int n_pos) {
  const size_t n4 = rows * (size_t)d4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const size_t r = i / d4;
    const int c = (int)(i - r * d4);
    float4 v = ld4(x, i);
    const float4 p = ld4(pe, (size_t)(r % n_pos) * d4 + c);
    v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
    st4(x, i, v);
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
  if (intermediate % 4 == 0 && aligned16(out) && aligned16(gate_up)) {
    const size_t n4 = seq_len * (intermediate / 4);
    swiglu_interleaved_vec_kernel<<<grid_for(n4, 256), 256, 0, st>>>(out, gate_up, seq_len, inter);
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
  if (aligned16(out) && aligned16(gate) && aligned16(up)) {
    const size_t n4 = n / 4;
    if (n4) swiglu_split_vec_kernel<<<grid_for(n4, 256), 256, 0, st>>>(out, gate, up, n4);
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
  if (aligned16(x)) {
    const size_t n4 = n / 4;
    if (n4) gelu_vec_kernel<ERF><<<grid_for(n4, 256), 256, 0, st>>>(x, n4, fast_end);
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
  if (d_model % 4 == 0 && aligned16(x) && aligned16(pe)) {
    const size_t n4 = n / 4;
    pe_add_vec_kernel<<<grid_for(n4, 256), 256, 0, st>>>(x, pe, rows, (int)(d_model / 4),
                                                          (int)n_pos);
  } else {
    pe_add_scalar_kernel<<<grid_for(n, 256), 256, 0, st>>>(x, pe, rows, (int)d_model, (int)n_pos);
  }
  return launch_status("pe_add");
}
