// Row normalisations: residual add + RMSNorm, RMSNorm, LayerNorm, add_inplace.
//
// Layout: row-major [seq_len, hidden] fp32. One workgroup owns one row; each
// thread keeps NV float4 of the row in registers, so a row crosses HBM exactly
// once in each direction (read x [+ delta], write [x and] out). The sum of
// squares (or mean/variance) is reduced with wave shuffles and one LDS step.
#include "common.hpp"

namespace qasr {
namespace {

QASR_DEV float4 ld4(const float* p, size_t i) { return reinterpret_cast<const float4*>(p)[i]; }
QASR_DEV void st4(float* p, size_t i, float4 v) { reinterpret_cast<float4*>(p)[i] = v; }

// ---------------------------------------------------------------------------
// RMSNorm (optionally fused with the residual add), vectorised row kernel.
// Arithmetic per row, as kernels/mod.rs:897-918 + avx.rs:374-415:
//   rinv = 1 / sqrt(sum(x^2) / hidden + eps);  out = (x * rinv) * w
// ---------------------------------------------------------------------------
template <int BLOCK, int NV, bool ADD>
__global__ __launch_bounds__(BLOCK) void rms_norm_vec_kernel(
    float* x, const float* delta, const float* __restrict__ w, float* out,
    int hidden, float eps) {
  __shared__ float red[BLOCK / kWave];
  const int h4 = hidden >> 2;
  const size_t base = (size_t)blockIdx.x * (size_t)h4;
  float4 v[NV];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      float4 a = ld4(x, base + c);
      if constexpr (ADD) {
        const float4 d = ld4(delta, base + c);
        a.x += d.x; a.y += d.y; a.z += d.z; a.w += d.w;
        st4(x, base + c, a);
      }
      v[i] = a;
      ss += a.x * a.x;
      ss += a.y * a.y;
      ss += a.z * a.z;
      ss += a.w * a.w;
    }
  }
  ss = block_sum<BLOCK>(ss, red);
  const float rinv = 1.0f / sqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      const float4 wv = ld4(w, c);
      float4 o;
      o.x = (v[i].x * rinv) * wv.x;
      o.y = (v[i].y * rinv) * wv.y;
      o.z = (v[i].z * rinv) * wv.z;
      o.w = (v[i].w * rinv) * wv.w;
      st4(out, base + c, o);
    }
  }
}

// Scalar fallback for any hidden / alignment: two sweeps over the row.
template <bool ADD>
__global__ __launch_bounds__(256) void rms_norm_scalar_kernel(
    float* x, const float* delta, const float* __restrict__ w, float* out,
    int hidden, float eps) {
  __shared__ float red[256 / kWave];
  const size_t base = (size_t)blockIdx.x * (size_t)hidden;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < hidden; c += 256) {
    float a = x[base + c];
    if constexpr (ADD) {
      a += delta[base + c];
      x[base + c] = a;
    }
    ss += a * a;
  }
  ss = block_sum<256>(ss, red);
  const float rinv = 1.0f / sqrtf(ss / (float)hidden + eps);
  for (int c = threadIdx.x; c < hidden; c += 256) {
    out[base + c] = (x[base + c] * rinv) * w[c];
  }
}

// ---------------------------------------------------------------------------
// LayerNorm, kernels/mod.rs:866-895 + avx.rs:417-481:
//   mean = sum(x)/H; var = sum((x-mean)^2); inv = 1/sqrt(var/H + eps)
//   out = fma((x-mean)*inv, w, b) for columns in whole 8-blocks, and
//   ((x-mean)*inv)*w + b for the hidden % 8 tail (the reference's scalar tail).
// ---------------------------------------------------------------------------
QASR_DEV float ln_out(float xv, float mean, float inv, float w, float b, bool fused) {
  const float t = (xv - mean) * inv;
  return fused ? __builtin_fmaf(t, w, b) : t * w + b;
}

template <int BLOCK, int NV>
__global__ __launch_bounds__(BLOCK) void layer_norm_vec_kernel(
    float* out, const float* x, const float* __restrict__ w,
    const float* __restrict__ b, int hidden, float eps) {
  __shared__ float red[BLOCK / kWave];
  const int h4 = hidden >> 2;
  const int fused_end = hidden & ~7;
  const size_t base = (size_t)blockIdx.x * (size_t)h4;
  float4 v[NV];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      v[i] = ld4(x, base + c);
      s += v[i].x;
      s += v[i].y;
      s += v[i].z;
      s += v[i].w;
    }
  }
  s = block_sum<BLOCK>(s, red);
  const float mean = s / (float)hidden;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      float d;
      d = v[i].x - mean; q += d * d;
      d = v[i].y - mean; q += d * d;
      d = v[i].z - mean; q += d * d;
      d = v[i].w - mean; q += d * d;
    }
  }
  q = block_sum<BLOCK>(q, red);
  const float inv = 1.0f / sqrtf(q / (float)hidden + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      const float4 wv = ld4(w, c);
      const float4 bv = ld4(b, c);
      const bool f = 4 * c < fused_end;  // 4-blocks never straddle an 8-block edge
      float4 o;
      o.x = ln_out(v[i].x, mean, inv, wv.x, bv.x, f);
      o.y = ln_out(v[i].y, mean, inv, wv.y, bv.y, f);
      o.z = ln_out(v[i].z, mean, inv, wv.z, bv.z, f);
      o.w = ln_out(v[i].w, mean, inv, wv.w, bv.w, f);
      st4(out, base + c, o);
    }
  }
}

__global__ __launch_bounds__(256) void layer_norm_scalar_kernel(
    float* out, const float* x, const float* __restrict__ w,
    const float* __restrict__ b, int hidden, float eps) {
  __shared__ float red[256 / kWave];
  const size_t base = (size_t)blockIdx.x * (size_t)hidden;
  const int fused_end = hidden & ~7;
  float s = 0.0f;
  for (int c = threadIdx.x; c < hidden; c += 256) s += x[base + c];
  s = block_sum<256>(s, red);
  const float mean = s / (float)hidden;
  float q = 0.0f;
  for (int c = threadIdx.x; c < hidden; c += 256) {
    const float d = x[base + c] - mean;
    q += d * d;
  }
  q = block_sum<256>(q, red);
  const float inv = 1.0f / sqrtf(q / (float)hidden + eps);
  for (int c = threadIdx.x; c < hidden; c += 256) {
    out[base + c] = ln_out(x[base + c], mean, inv, w[c], b[c], c < fused_end);
  }
}

// ---------------------------------------------------------------------------
// a[i] += b[i]
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void add_vec_kernel(float* a, const float* b, size_t n4) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    float4 x = ld4(a, i);
    const float4 y = ld4(b, i);
    x.x += y.x; x.y += y.y; x.z += y.z; x.w += y.w;
    st4(a, i, x);
  }
}

__global__ __launch_bounds__(256) void add_scalar_kernel(float* a, const float* b, size_t begin, size_t n) {
  for (size_t i = begin + (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    a[i] += b[i];
  }
}

// Picks (BLOCK, NV) so that BLOCK*NV float4 cover a row of h4 float4.
// Returns false when the row is too long for the register-resident kernel.
struct RowShape {
  int block;
  int nv;
};

bool pick_row_shape(int h4, RowShape* s) {
  if (h4 <= 64) { *s = {64, 1}; return true; }
  if (h4 <= 128) { *s = {128, 1}; return true; }
  if (h4 <= 256) { *s = {256, 1}; return true; }
  if (h4 <= 512) { *s = {256, 2}; return true; }
  if (h4 <= 1024) { *s = {256, 4}; return true; }
  if (h4 <= 2048) { *s = {256, 8}; return true; }
  return false;
}

template <bool ADD>
int launch_rms(float* x, const float* delta, const float* w, float* out,
               size_t seq_len, size_t hidden, float eps, hipStream_t st) {
  const int h = (int)hidden;
  const dim3 grid((unsigned)seq_len);
  RowShape rs{};
  const bool vec = hidden % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(out) &&
                   (!ADD || aligned16(delta)) && pick_row_shape(h / 4, &rs);
  if (!vec) {
    rms_norm_scalar_kernel<ADD><<<grid, 256, 0, st>>>(x, delta, w, out, h, eps);
  } else if (rs.block == 64) {
    rms_norm_vec_kernel<64, 1, ADD><<<grid, 64, 0, st>>>(x, delta, w, out, h, eps);
  } else if (rs.block == 128) {
    rms_norm_vec_kernel<128, 1, ADD><<<grid, 128, 0, st>>>(x, delta, w, out, h, eps);
  } else if (rs.nv == 1) {
    rms_norm_vec_kernel<256, 1, ADD><<<grid, 256, 0, st>>>(x, delta, w, out, h, eps);
  } else if (rs.nv == 2) {
    rms_norm_vec_kernel<256, 2, ADD><<<grid, 256, 0, st>>>(x, delta, w, out, h, eps);
  } else if (rs.nv == 4) {
    rms_norm_vec_kernel<256, 4, ADD><<<grid, 256, 0, st>>>(x, delta, w, out, h, eps);
  } else {
    rms_norm_vec_kernel<256, 8, ADD><<<grid, 256, 0, st>>>(x, delta, w, out, h, eps);
  }
  return launch_status(ADD ? "add_rms_norm" : "rms_norm");
}

int check_rows(size_t seq_len, size_t hidden) {
  size_t n;
  QASR_REQUIRE(mul_ok(seq_len, hidden, &n), "seq_len * hidden overflows");
  QASR_REQUIRE(seq_len <= 0x7fffffffu, "seq_len exceeds the grid limit (2^31-1 rows)");
  QASR_REQUIRE(hidden <= 0x7fffffffu, "hidden exceeds 2^31-1");
  return QASR_OK;
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_add_inplace_f32(float* a, const float* b, size_t n, void* stream) {
  if (n == 0) return QASR_OK;
  QASR_REQUIRE(a && b, "add_inplace: null pointer");
  QASR_REQUIRE(n <= kMaxElems, "add_inplace: n too large");
  hipStream_t st = as_stream(stream);
  size_t done = 0;
  if (aligned16(a) && aligned16(b)) {
    const size_t n4 = n / 4;
    if (n4) add_vec_kernel<<<grid_for(n4, 256), 256, 0, st>>>(a, b, n4);
    done = n4 * 4;
  }
  if (done < n) add_scalar_kernel<<<grid_for(n - done, 256), 256, 0, st>>>(a, b, done, n);
  return launch_status("add_inplace");
}

extern "C" int qasr_rms_norm_f32(float* out, const float* x, const float* weight,
                                 size_t seq_len, size_t hidden, float eps, void* stream) {
  if (seq_len == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(out && x && weight, "rms_norm: null pointer");
  int rc = check_rows(seq_len, hidden);
  if (rc) return rc;
  return launch_rms<false>(const_cast<float*>(x), nullptr, weight, out, seq_len, hidden, eps,
                           as_stream(stream));
}

extern "C" int qasr_add_rms_norm_f32(float* x, const float* delta, const float* weight,
                                     float* out, size_t seq_len, size_t hidden, float eps,
                                     void* stream) {
  if (seq_len == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(x && delta && weight && out, "add_rms_norm: null pointer");
  QASR_REQUIRE(out != x, "add_rms_norm: out must not alias the residual x");
  int rc = check_rows(seq_len, hidden);
  if (rc) return rc;
  return launch_rms<true>(x, delta, weight, out, seq_len, hidden, eps, as_stream(stream));
}

extern "C" int qasr_layer_norm_f32(float* out, const float* x, const float* weight,
                                   const float* bias, size_t seq_len, size_t hidden, float eps,
                                   void* stream) {
  if (seq_len == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(out && x && weight && bias, "layer_norm: null pointer");
  int rc = check_rows(seq_len, hidden);
  if (rc) return rc;
  hipStream_t st = as_stream(stream);
  const int h = (int)hidden;
  const dim3 grid((unsigned)seq_len);
  RowShape rs{};
  const bool vec = hidden % 4 == 0 && aligned16(x) && aligned16(out) && aligned16(weight) &&
                   aligned16(bias) && pick_row_shape(h / 4, &rs);
  if (!vec) {
    layer_norm_scalar_kernel<<<grid, 256, 0, st>>>(out, x, weight, bias, h, eps);
  } else if (rs.block == 64) {
    layer_norm_vec_kernel<64, 1><<<grid, 64, 0, st>>>(out, x, weight, bias, h, eps);
  } else if (rs.block == 128) {
    layer_norm_vec_kernel<128, 1><<<grid, 128, 0, st>>>(out, x, weight, bias, h, eps);
  } else if (rs.nv == 1) {
    layer_norm_vec_kernel<256, 1><<<grid, 256, 0, st>>>(out, x, weight, bias, h, eps);
  } else if (rs.nv == 2) {
    layer_norm_vec_kernel<256, 2><<<grid, 256, 0, st>>>(out, x, weight, bias, h, eps);
  } else if (rs.nv == 4) {
    layer_norm_vec_kernel<256, 4><<<grid, 256, 0, st>>>(out, x, weight, bias, h, eps);
  } else {
    layer_norm_vec_kernel<256, 8><<<grid, 256, 0, st>>>(out, x, weight, bias, h, eps);
  }
  return launch_status("layer_norm");
}
