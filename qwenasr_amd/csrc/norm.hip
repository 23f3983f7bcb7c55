// Row normalisations: residual add + RMSNorm, RMSNorm, LayerNorm, add_inplace.
//
// Layout: row-major [seq_len, hidden] fp32. One workgroup owns one row; each
// thread keeps NV float4 of the row in registers, so a row crosses HBM exactly
// once in each direction (read x [+ delta], write [x and] out). The sum of
// squares (or mean/variance) is reduced with wave shuffles and one LDS step.
// Row data moves with nontemporal 16-byte accesses (the LayerNorm at
// [3000,896] measured 7.1 us with cached accesses, 6.0 us with these), except
// in the add+RMSNorm+quantize kernel, where they measured slower ([256,2048]:
// 4.1 -> 4.6 us); gains and biases, read by every row, stay cached.
#include "common.hpp"

namespace qasr {
namespace {


// ---------------------------------------------------------------------------
// RMSNorm (optionally fused with the residual add), vectorised row kernel.
// Arithmetic per row, as kernels/mod.rs:897-918 + avx.rs:374-415:
//   rinv = 1 / sqrt(sum(x^2) / hidden + eps);  out = (x * rinv) * w
// ---------------------------------------------------------------------------
template <int BLOCK, int NV, bool ADD, bool QUANT>
__global__ __launch_bounds__(BLOCK) void rms_norm_vec_kernel(
    float* x, const float* delta, const float* __restrict__ w, float* out, int8_t* q,
    float* q_scales, int hidden, float eps) {
  __shared__ float red[BLOCK / kWave];
  const int h4 = hidden >> 2;
  const size_t base = (size_t)blockIdx.x * (size_t)h4;
  float4 v[NV], wv[NV];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      // the gain is independent of the row statistics: load it with the row
      wv[i] = ld4(w, c);
      float4 a = QUANT ? ld4(x, base + c) : ld4_nt(x, base + c);
      if constexpr (ADD) {
        const float4 d = QUANT ? ld4(delta, base + c) : ld4_nt(delta, base + c);
        a.x += d.x; a.y += d.y; a.z += d.z; a.w += d.w;
        if constexpr (QUANT) st4(x, base + c, a); else st4_nt(x, base + c, a);
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
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      float4 o;
      o.x = (v[i].x * rinv) * wv[i].x;
      o.y = (v[i].y * rinv) * wv[i].y;
      o.z = (v[i].z * rinv) * wv[i].z;
      o.w = (v[i].w * rinv) * wv[i].w;
      if (out) {
        if constexpr (QUANT) st4(out, base + c, o); else st4_nt(out, base + c, o);
      }
      v[i] = o;
      if constexpr (QUANT) {
        // absmax as quantize.rs:646-652 (`if abs > absmax`: NaN never wins)
        const float a0 = fabsf(o.x), a1 = fabsf(o.y), a2 = fabsf(o.z), a3 = fabsf(o.w);
        if (a0 > amax) amax = a0;
        if (a1 > amax) amax = a1;
        if (a2 > amax) amax = a2;
        if (a3 > amax) amax = a3;
      }
    }
  }
  if constexpr (QUANT) {
    // Per-row int8 quantization of the normalised row, quantize.rs:633-662.
    amax = block_max<BLOCK>(amax, red);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (threadIdx.x == 0) q_scales[blockIdx.x] = amax / 127.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = threadIdx.x + i * BLOCK;
      if (c < h4) {
        const uint32_t b = (uint32_t)(quant_i8(v[i].x, inv) & 0xff) |
                           ((uint32_t)(quant_i8(v[i].y, inv) & 0xff) << 8) |
                           ((uint32_t)(quant_i8(v[i].z, inv) & 0xff) << 16) |
                           ((uint32_t)(quant_i8(v[i].w, inv) & 0xff) << 24);
        reinterpret_cast<uint32_t*>(q)[base + c] = b;
      }
    }
  }
}

// Scalar fallback for any hidden / alignment: sweeps over the row.
template <bool ADD, bool QUANT>
__global__ __launch_bounds__(256) void rms_norm_scalar_kernel(
    float* x, const float* delta, const float* __restrict__ w, float* out, int8_t* q,
    float* q_scales, int hidden, float eps) {
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
  float amax = 0.0f;
  for (int c = threadIdx.x; c < hidden; c += 256) {
    const float o = (x[base + c] * rinv) * w[c];
    if (out) out[base + c] = o;
    if constexpr (QUANT) {
      const float a = fabsf(o);
      if (a > amax) amax = a;
    }
  }
  if constexpr (QUANT) {
    amax = block_max<256>(amax, red);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (threadIdx.x == 0) q_scales[blockIdx.x] = amax / 127.0f;
    for (int c = threadIdx.x; c < hidden; c += 256) {
      q[base + c] = (int8_t)quant_i8((x[base + c] * rinv) * w[c], inv);
    }
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
  float4 v[NV], wv[NV], bv[NV];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + i * BLOCK;
    if (c < h4) {
      wv[i] = ld4(w, c);  // gain and bias: independent of the statistics
      bv[i] = ld4(b, c);
      v[i] = ld4_nt(x, base + c);
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
      const bool f = 4 * c < fused_end;  // 4-blocks never straddle an 8-block edge
      float4 o;
      o.x = ln_out(v[i].x, mean, inv, wv[i].x, bv[i].x, f);
      o.y = ln_out(v[i].y, mean, inv, wv[i].y, bv[i].y, f);
      o.z = ln_out(v[i].z, mean, inv, wv[i].z, bv[i].z, f);
      o.w = ln_out(v[i].w, mean, inv, wv[i].w, bv[i].w, f);
      st4_nt(out, base + c, o);
    }
  }
}

// One wave per row (4 rows per workgroup): the row's NV float4 per lane stay
// in registers and both statistics are wave reductions (no LDS, no barrier).
// With a pre-add the row first takes an addition and is written back to x_out
// before it is normalised, with the fp32 adds of the standalone kernels:
//   kLnAddPe:    x[r] += pe[r mod n_pos] (pe_add_vec_kernel): the encoder's PE
//                add (encoder.rs:341-343) and layer 0's LayerNorm of the same
//                rows (encoder.rs:370-371) in one pass;
//   kLnAddDelta: x[r] += delta[r] (add_vec_kernel): each residual add of the
//                encoder layer and the LayerNorm that reads its rows next
//                (encoder.rs:386 + 389-390, 397 + 370-371, 397 + 401-402).
enum LnAdd { kLnPlain = 0, kLnAddPe = 1, kLnAddDelta = 2 };

template <int NV, int ADD = kLnPlain>
__global__ __launch_bounds__(256) void layer_norm_wave_kernel(
    float* out, const float* x, const float* __restrict__ w, const float* __restrict__ b,
    int rows, int hidden, float eps, float* x_out = nullptr, const float* add = nullptr,
    int n_pos = 1) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const int h4 = hidden >> 2;
  const int fused_end = hidden & ~7;
  const size_t base = (size_t)row * (size_t)h4;
  const size_t abase = ADD == kLnAddPe ? (size_t)(row % n_pos) * (size_t)h4 : base;
  float4 v[NV], wv[NV], bv[NV];
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * kWave;
    if (c < h4) {
      wv[i] = ld4(w, c);  // gain and bias: independent of the statistics
      bv[i] = ld4(b, c);
      v[i] = ld4_nt(x, base + c);
      if constexpr (ADD != kLnPlain) {
        // the 13 PE table rows are shared by all rows (cached); delta streams
        const float4 p = ADD == kLnAddPe ? ld4(add, abase + c) : ld4_nt(add, abase + c);
        v[i].x += p.x; v[i].y += p.y; v[i].z += p.z; v[i].w += p.w;
        st4_nt(x_out, base + c, v[i]);
      }
      s += v[i].x;
      s += v[i].y;
      s += v[i].z;
      s += v[i].w;
    }
  }
  s = wave_sum(s);
  const float mean = s / (float)hidden;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * kWave;
    if (c < h4) {
      float d;
      d = v[i].x - mean; q += d * d;
      d = v[i].y - mean; q += d * d;
      d = v[i].z - mean; q += d * d;
      d = v[i].w - mean; q += d * d;
    }
  }
  q = wave_sum(q);
  const float inv = 1.0f / sqrtf(q / (float)hidden + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + i * kWave;
    if (c < h4) {
      const bool f = 4 * c < fused_end;
      float4 o;
      o.x = ln_out(v[i].x, mean, inv, wv[i].x, bv[i].x, f);
      o.y = ln_out(v[i].y, mean, inv, wv[i].y, bv[i].y, f);
      o.z = ln_out(v[i].z, mean, inv, wv[i].z, bv[i].z, f);
      o.w = ln_out(v[i].w, mean, inv, wv[i].w, bv[i].w, f);
      st4_nt(out, base + c, o);
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

template <bool ADD, bool QUANT>
int launch_rms(float* x, const float* delta, const float* w, float* out, int8_t* q,
               float* qs, size_t seq_len, size_t hidden, float eps, hipStream_t st) {
  const int h = (int)hidden;
  const dim3 grid((unsigned)seq_len);
  RowShape rs{};
  const bool vec = hidden % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(out) &&
                   (!ADD || aligned16(delta)) && (!QUANT || aligned4(q)) &&
                   pick_row_shape(h / 4, &rs);
  if (!vec) {
    rms_norm_scalar_kernel<ADD, QUANT><<<grid, 256, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  } else if (rs.block == 64) {
    rms_norm_vec_kernel<64, 1, ADD, QUANT><<<grid, 64, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  } else if (rs.block == 128) {
    rms_norm_vec_kernel<128, 1, ADD, QUANT><<<grid, 128, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  } else if (rs.nv == 1) {
    rms_norm_vec_kernel<256, 1, ADD, QUANT><<<grid, 256, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  } else if (rs.nv == 2) {
    // Rows of 1025-2048 floats take eight waves of one float4 each: the row's
    // loads leave from all four SIMDs at once ([256,2048] with the int8
    // epilogue: 5.8 us with four waves of two float4, 5.5 us with eight).
    rms_norm_vec_kernel<512, 1, ADD, QUANT><<<grid, 512, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  } else if (rs.nv == 4) {
    rms_norm_vec_kernel<256, 4, ADD, QUANT><<<grid, 256, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  } else {
    rms_norm_vec_kernel<256, 8, ADD, QUANT><<<grid, 256, 0, st>>>(x, delta, w, out, q, qs, h, eps);
  }
  return launch_status(QUANT ? "add_rms_norm_quant" : (ADD ? "add_rms_norm" : "rms_norm"));
}

int check_rows(size_t seq_len, size_t hidden) {
  size_t n;
  QASR_REQUIRE(mul_ok(seq_len, hidden, &n), "seq_len * hidden overflows");
  QASR_REQUIRE(seq_len <= kMaxRows, "seq_len exceeds the grid limit (2^24 rows per launch)");
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
  return launch_rms<false, false>(const_cast<float*>(x), nullptr, weight, out, nullptr, nullptr,
                                  seq_len, hidden, eps, as_stream(stream));
}

extern "C" int qasr_add_rms_norm_f32(float* x, const float* delta, const float* weight,
                                     float* out, size_t seq_len, size_t hidden, float eps,
                                     void* stream) {
  if (seq_len == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(x && delta && weight && out, "add_rms_norm: null pointer");
  QASR_REQUIRE(out != x, "add_rms_norm: out must not alias the residual x");
  int rc = check_rows(seq_len, hidden);
  if (rc) return rc;
  return launch_rms<true, false>(x, delta, weight, out, nullptr, nullptr, seq_len, hidden, eps,
                                 as_stream(stream));
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
  const int h4 = h / 4;
  if (vec && h4 <= 8 * kWave) {
    const unsigned wgrid = (unsigned)((seq_len + 3) / 4);
    const int r = (int)seq_len;
    if (h4 <= kWave) layer_norm_wave_kernel<1><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps);
    else if (h4 <= 2 * kWave) layer_norm_wave_kernel<2><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps);
    else if (h4 <= 4 * kWave) layer_norm_wave_kernel<4><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps);
    else layer_norm_wave_kernel<8><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps);
  } else if (!vec) {
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

static bool spans_overlap(const void* a, size_t an, const void* b, size_t bn) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + bn && pb < pa + an;
}

extern "C" int qasr_pe_add_layer_norm_f32(float* x, const float* pe, float* out,
                                          const float* weight, const float* bias, size_t rows,
                                          size_t d_model, size_t n_pos, float eps, void* stream) {
  if (rows == 0 || d_model == 0) return QASR_OK;
  QASR_REQUIRE(x && pe && out && weight && bias, "pe_add_layer_norm: null pointer");
  QASR_REQUIRE(n_pos > 0 && n_pos < 0x7fffffffu, "pe_add_layer_norm: n_pos must be in [1, 2^31)");
  int rc = check_rows(rows, d_model);
  if (rc) return rc;
  const size_t xb = rows * d_model * sizeof(float), pb = n_pos * d_model * sizeof(float);
  QASR_REQUIRE(!spans_overlap(out, xb, x, xb) && !spans_overlap(pe, pb, x, xb),
               "pe_add_layer_norm: out and pe must not overlap x");
  const int h = (int)d_model, h4 = h / 4;
  const bool vec = d_model % 4 == 0 && h4 <= 8 * kWave && aligned16(x) && aligned16(out) &&
                   aligned16(pe) && aligned16(weight) && aligned16(bias);
  if (!vec) {  // any other shape: the two passes, with the same results
    rc = qasr_pe_add_f32(x, pe, rows, d_model, n_pos, stream);
    if (rc != QASR_OK) return rc;
    return qasr_layer_norm_f32(out, x, weight, bias, rows, d_model, eps, stream);
  }
  hipStream_t st = as_stream(stream);
  const unsigned wgrid = (unsigned)((rows + 3) / 4);
  const int r = (int)rows, np = (int)n_pos;
  if (h4 <= kWave)
    layer_norm_wave_kernel<1, kLnAddPe><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, pe, np);
  else if (h4 <= 2 * kWave)
    layer_norm_wave_kernel<2, kLnAddPe><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, pe, np);
  else if (h4 <= 4 * kWave)
    layer_norm_wave_kernel<4, kLnAddPe><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, pe, np);
  else
    layer_norm_wave_kernel<8, kLnAddPe><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, pe, np);
  return launch_status("pe_add_layer_norm");
}

extern "C" int qasr_add_layer_norm_f32(float* x, const float* delta, const float* weight,
                                       const float* bias, float* out, size_t seq_len,
                                       size_t hidden, float eps, void* stream) {
  if (seq_len == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(x && delta && weight && bias && out, "add_layer_norm: null pointer");
  int rc = check_rows(seq_len, hidden);
  if (rc) return rc;
  const size_t xb = seq_len * hidden * sizeof(float);
  QASR_REQUIRE(!spans_overlap(out, xb, x, xb) && !spans_overlap(delta, xb, x, xb) &&
                   !spans_overlap(delta, xb, out, xb),
               "add_layer_norm: x, delta and out must not overlap");
  const int h = (int)hidden, h4 = h / 4;
  const bool vec = hidden % 4 == 0 && h4 <= 8 * kWave && aligned16(x) && aligned16(out) &&
                   aligned16(delta) && aligned16(weight) && aligned16(bias);
  if (!vec) {  // any other shape: the two passes, with the same results
    rc = qasr_add_inplace_f32(x, delta, seq_len * hidden, stream);
    if (rc != QASR_OK) return rc;
    return qasr_layer_norm_f32(out, x, weight, bias, seq_len, hidden, eps, stream);
  }
  hipStream_t st = as_stream(stream);
  const unsigned wgrid = (unsigned)((seq_len + 3) / 4);
  const int r = (int)seq_len;
  if (h4 <= kWave)
    layer_norm_wave_kernel<1, kLnAddDelta><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, delta);
  else if (h4 <= 2 * kWave)
    layer_norm_wave_kernel<2, kLnAddDelta><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, delta);
  else if (h4 <= 4 * kWave)
    layer_norm_wave_kernel<4, kLnAddDelta><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, delta);
  else
    layer_norm_wave_kernel<8, kLnAddDelta><<<wgrid, 256, 0, st>>>(out, x, weight, bias, r, h, eps, x, delta);
  return launch_status("add_layer_norm");
}

extern "C" int qasr_add_rms_norm_quant_f32(float* x, const float* delta, const float* weight,
                                           float* out, int8_t* q, float* q_scales,
                                           size_t seq_len, size_t hidden, float eps,
                                           void* stream) {
  if (seq_len == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(x && weight && q && q_scales, "add_rms_norm_quant: null pointer");
  QASR_REQUIRE(out != x, "add_rms_norm_quant: out must not alias the residual x");
  int rc = check_rows(seq_len, hidden);
  if (rc) return rc;
  if (delta) {
    return launch_rms<true, true>(x, delta, weight, out, q, q_scales, seq_len, hidden, eps,
                                  as_stream(stream));
  }
  return launch_rms<false, true>(x, nullptr, weight, out, q, q_scales, seq_len, hidden, eps,
                                 as_stream(stream));
}
