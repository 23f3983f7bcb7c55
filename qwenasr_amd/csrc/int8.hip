// INT8 path: per-row quantizer, W8A32 linear (drop-in for linear_nobias_int8),
// gate/up interleave, and the W8A8 gate/up projection fused with SwiGLU.
//
// Weight layout is the .qint8 one: int8 row-major [out_dim, in_dim] with one f32
// scale per output row (quantize.rs:77-84). The fused gate/up matrix has its
// rows interleaved g0,u0,g1,u1,... (decoder.rs:701-719), so one gate/up pair is
// 2*in_dim contiguous bytes and its SwiGLU output needs no cross-wave exchange.
#include "common.hpp"

#include <climits>

#include "gemm_w8a8.hpp"

namespace qasr {
namespace {


// ---------------------------------------------------------------------------
// Per-row quantizer, quantize.rs:633-662.
// ---------------------------------------------------------------------------
// Register-resident variant: one workgroup per row, NV float4 per thread,
// one read of x and one write of q.
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_vec_kernel(int8_t* q, float* scales,
                                                                const float* x, int cols) {
  __shared__ float red[256 / kWave];
  const int c4 = cols >> 2;
  const size_t base = (size_t)blockIdx.x * c4;
  float4 v[NV];
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < c4) {
      v[i] = ld4(x, base + c);
      const float a0 = fabsf(v[i].x), a1 = fabsf(v[i].y), a2 = fabsf(v[i].z), a3 = fabsf(v[i].w);
      if (a0 > m) m = a0;
      if (a1 > m) m = a1;
      if (a2 > m) m = a2;
      if (a3 > m) m = a3;
    }
  }
  m = block_max<256>(m, red);
  const float inv = m > 0.0f ? 127.0f / m : 0.0f;
  if (threadIdx.x == 0) scales[blockIdx.x] = m / 127.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < c4) {
      const uint32_t b = (uint32_t)(quant_i8(v[i].x, inv) & 0xff) |
                         ((uint32_t)(quant_i8(v[i].y, inv) & 0xff) << 8) |
                         ((uint32_t)(quant_i8(v[i].z, inv) & 0xff) << 16) |
                         ((uint32_t)(quant_i8(v[i].w, inv) & 0xff) << 24);
      reinterpret_cast<uint32_t*>(q)[base + c] = b;
    }
  }
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(int8_t* q, float* scales,
                                                            const float* x, int cols) {
  __shared__ float red[256 / kWave];
  const size_t base = (size_t)blockIdx.x * cols;
  float m = 0.0f;
  for (int c = threadIdx.x; c < cols; c += 256) {
    const float a = fabsf(x[base + c]);
    if (a > m) m = a;  // NaN never wins, as in `if abs > absmax`
  }
  m = block_max<256>(m, red);
  const float inv = m > 0.0f ? 127.0f / m : 0.0f;
  if (threadIdx.x == 0) scales[blockIdx.x] = m / 127.0f;
  for (int c = threadIdx.x; c < cols; c += 256) q[base + c] = (int8_t)quant_i8(x[base + c], inv);
}

// ---------------------------------------------------------------------------
// W8A32 linear: y[s,o] = (sum_k (f32)w[o,k] * x[s,k]) * scale[o] (+ bias[o]).
// One wave per output row; each lane owns 16-byte slices of the row, keeps
// them in registers and reuses them for every token s.
// ---------------------------------------------------------------------------
template <int KCH>  // in_dim / 1024 chunks held in registers (1..8)
__global__ __launch_bounds__(256) void w8a32_vec_kernel(float* y, const float* x, const int8_t* w,
                                                        const float* scales, const float* bias,
                                                        int seq, int in_dim, int out_dim) {
  const int lane = threadIdx.x & (kWave - 1);
  const int o = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (o >= out_dim) return;
  const int8_t* wr = w + (size_t)o * in_dim;
  int4 wv[KCH];
#pragma unroll
  for (int c = 0; c < KCH; ++c) wv[c] = reinterpret_cast<const int4*>(wr)[c * kWave + lane];
  const float sc = scales[o];
  const float bs = bias ? bias[o] : 0.0f;
  for (int s = 0; s < seq; ++s) {
    const float* xs = x + (size_t)s * in_dim;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const int k0 = (c * kWave + lane) * 16;
      const int wq[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float4 xv = ld4(xs + k0 + 4 * t, 0);
        acc = __builtin_fmaf((float)(int8_t)(wq[t] & 0xff), xv.x, acc);
        acc = __builtin_fmaf((float)(int8_t)((wq[t] >> 8) & 0xff), xv.y, acc);
        acc = __builtin_fmaf((float)(int8_t)((wq[t] >> 16) & 0xff), xv.z, acc);
        acc = __builtin_fmaf((float)(int8_t)((wq[t] >> 24) & 0xff), xv.w, acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      float r = acc * sc;
      if (bias) r += bs;
      y[(size_t)s * out_dim + o] = r;
    }
  }
}

// Decode shape (one token): each wave owns R consecutive output rows, issues
// all R x KCH weight loads before the first FMA (so R KiB per chunk are in
// flight per wave instead of one), and keeps x in registers across its rows.
// With PART, the workgroup also reduces its rows' results to the best
// (value, index) in the lm_head argmax order and writes it to part[blockIdx.x];
// waves past the last row then stay to the end (their loads clamp to the last
// row and they offer no candidate).
// Epilogues of the one-token matvec: plain rows, rows + per-workgroup argmax
// candidate (lm_head), or the decode loop's SwiGLU on interleaved gate/up rows.
enum RowsEpi { kEpiRows = 0, kEpiArgmax = 1, kEpiSwiglu = 2 };

// With NORM the input row is not read as given: every workgroup first forms
// h = x (+ delta) and the RMSNorm h * rinv * gain of it in LDS, with the
// element order of the standalone kernel for that row length
// (rms_norm_vec_kernel<256, KCH>: thread t sums float4s t, t + 256, ...; at
// 2048 floats rms_norm_vec_kernel<512, 1>), so the row equals that kernel's
// output bit for bit; workgroup 0 also writes h to h_out.
struct RowNorm {
  const float* x;
  const float* delta;  // nullable: plain RMSNorm of x
  const float* gain;
  float* h_out;        // nullable; never x or delta (other workgroups still read them)
  float eps;
};

template <int KCH, int R, int EPI, bool NORM = false>
QASR_DEV void w8a32_rows_body(float* y, const float* x, const int8_t* w, const float* scales,
                              const float* bias, int in_dim, int out_dim, unsigned block,
                              float2* part, const RowNorm& rn = RowNorm{}) {
  constexpr bool PART = EPI == kEpiArgmax;
  static_assert(EPI != kEpiSwiglu || R % 2 == 0, "SwiGLU pairs sit in one wave");
  static_assert(!(NORM && PART), "no normalised input on the argmax path");
  const int lane = threadIdx.x & (kWave - 1);
  const int o0 = (int)(block * (256 / kWave) + threadIdx.x / kWave) * R;

  // the row statistics' inputs are loaded before the weights: the wait for
  // them then leaves the weight loads in flight
  float4 nx[NORM ? KCH : 1], nd[NORM ? KCH : 1], ng[NORM ? KCH : 1];
  float4 xg[NORM ? 1 : KCH];
  if constexpr (!NORM) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) xg[i] = ld4(x, threadIdx.x + 256 * i);
  }
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = threadIdx.x + 256 * i;
      ng[i] = ld4(rn.gain, c);
      nx[i] = ld4(rn.x, c);
      if (rn.delta) nd[i] = ld4(rn.delta, c);
    }
  }
  // the epilogue's row scale (and bias) of lane r < R, loaded with the
  // inputs: after the dot products it would be one more memory round trip
  const int o_ep = min(o0 + (lane < R ? lane : 0), out_dim - 1);
  const float sc_ep = scales[o_ep];
  const float bias_ep = bias ? bias[o_ep] : 0.0f;
  v4i wv[R][KCH];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int o = o0 + r < out_dim ? o0 + r : out_dim - 1;  // tail rows recompute the last row
    const v4i* wr = reinterpret_cast<const v4i*>(w + (size_t)o * in_dim);
#pragma unroll
    for (int c = 0; c < KCH; ++c) wv[r][c] = __builtin_nontemporal_load(wr + c * kWave + lane);
  }
  float4 xv[KCH][4];
  if constexpr (NORM) {
    __shared__ float4 xs[256 * KCH];
    __shared__ float red[2 * 256 / kWave];
    float ss = 0.0f, ss_hi = 0.0f;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = threadIdx.x + 256 * i;
      float4 a = nx[i];
      if (rn.delta) {
        a.x += nd[i].x; a.y += nd[i].y; a.z += nd[i].z; a.w += nd[i].w;
      }
      if (rn.h_out && blockIdx.x == 0) st4(rn.h_out, c, a);
      nx[i] = a;
      float& s = KCH == 2 && i == 1 ? ss_hi : ss;
      s += a.x * a.x;
      s += a.y * a.y;
      s += a.z * a.z;
      s += a.w * a.w;
    }
    if constexpr (KCH == 2) {
      // A 2048-float row: rms_norm_vec_kernel<512, 1>'s order, where float4 c
      // is lane c % 64 of wave c / 64 and the eight wave sums are added in
      // wave order. Here wave w's two float4 halves are that kernel's waves w
      // and w + 4.
      ss = wave_sum(ss);
      ss_hi = wave_sum(ss_hi);
      if ((threadIdx.x & (kWave - 1)) == 0) {
        red[threadIdx.x / kWave] = ss;
        red[256 / kWave + threadIdx.x / kWave] = ss_hi;
      }
      __syncthreads();
      ss = red[0];
#pragma unroll
      for (int i = 1; i < 2 * 256 / kWave; ++i) ss += red[i];
    } else {
      ss = block_sum<256>(ss, red);
    }
    const float rinv = 1.0f / sqrtf(ss / (float)in_dim + rn.eps);
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      float4 o;
      o.x = (nx[i].x * rinv) * ng[i].x;
      o.y = (nx[i].y * rinv) * ng[i].y;
      o.z = (nx[i].z * rinv) * ng[i].z;
      o.w = (nx[i].w * rinv) * ng[i].w;
      xs[threadIdx.x + 256 * i] = o;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < KCH; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) xv[c][t] = xs[(c * kWave + lane) * 4 + t];
    if (o0 >= out_dim) return;  // after the workgroup's barrier
  } else {
    // x through LDS: loaded as consecutive 16-byte pieces per lane (a lane's
    // own 64-byte piece, read straight from global memory, put every lane of
    // a load instruction on a different line: 4x the line lookups of the
    // weight loads for a quarter of the bytes), once per workgroup. The
    // barrier waits for LDS only, so the weight loads stay in flight.
    __shared__ float4 xs[256 * KCH];
#pragma unroll
    for (int i = 0; i < KCH; ++i) xs[threadIdx.x + 256 * i] = xg[i];
    lds_barrier();
#pragma unroll
    for (int c = 0; c < KCH; ++c)
#pragma unroll
      for (int t = 0; t < 4; ++t) xv[c][t] = xs[(c * kWave + lane) * 4 + t];
    if constexpr (!PART) {
      if (o0 >= out_dim) return;  // after the workgroup's barrier
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const int wq[4] = {wv[r][c][0], wv[r][c][1], wv[r][c][2], wv[r][c][3]};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        a = __builtin_fmaf((float)(int8_t)(wq[t] & 0xff), xv[c][t].x, a);
        a = __builtin_fmaf((float)(int8_t)((wq[t] >> 8) & 0xff), xv[c][t].y, a);
        a = __builtin_fmaf((float)(int8_t)((wq[t] >> 16) & 0xff), xv[c][t].z, a);
        a = __builtin_fmaf((float)(int8_t)((wq[t] >> 24) & 0xff), xv[c][t].w, a);
      }
    }
    acc[r] = wave_sum(a);
  }
  const bool mine = lane < R && o0 + lane < out_dim;
  float res = 0.0f;
  if (mine) {
    float a = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r)
      if (lane == r) a = acc[r];
    const int o = o0 + lane;
    res = a * sc_ep;
    if (bias) res += bias_ep;
    if constexpr (EPI != kEpiSwiglu) y[o] = res;
  }
  if constexpr (EPI == kEpiSwiglu) {
    // rows o0 + 2i and o0 + 2i + 1 are gate_i and up_i (decoder.rs:916-921):
    // out[(o0 + lane) / 2] = g / (1 + expf(-g)) * u
    const float u = __shfl_down(res, 1, kWave);
    if (mine && (lane & 1) == 0) y[(o0 + lane) >> 1] = silu_expf(res) * u;
  }
  if constexpr (PART) {
    __shared__ float sv[256 / kWave];
    __shared__ int si[256 / kWave];
    float bv = -__builtin_inff();
    int bi = INT_MAX;
    if (mine) argmax_consider(res, o0 + lane, bv, bi);
#pragma unroll
    for (int m = R / 2; m >= 1; m >>= 1) {  // candidates sit in lanes 0..R-1
      const float ov = __shfl_xor(bv, m, kWave);
      const int oi = __shfl_xor(bi, m, kWave);
      if (argmax_better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      sv[threadIdx.x / kWave] = bv;
      si[threadIdx.x / kWave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
      for (int k = 1; k < 256 / kWave; ++k)
        if (argmax_better(sv[k], si[k], bv, bi)) {
          bv = sv[k];
          bi = si[k];
        }
      part[block] = make_float2(bv, __int_as_float(bi));
    }
  }
}

template <int KCH, int R, int EPI = kEpiRows, bool NORM = false>
__global__ __launch_bounds__(256) void w8a32_rows_kernel(float* y, const float* x, const int8_t* w,
                                                         const float* scales, const float* bias,
                                                         int in_dim, int out_dim,
                                                         float2* part = nullptr, RowNorm rn = RowNorm{}) {
  w8a32_rows_body<KCH, R, EPI, NORM>(y, x, w, scales, bias, in_dim, out_dim, blockIdx.x, part, rn);
}

// Several matrices of the same input in one launch (the q/k/v projections):
// workgroups [wg_begin[m], wg_begin[m + 1]) compute matrix m.
constexpr int kMaxMats = 4;
struct MatSet {
  float* y[kMaxMats];
  const int8_t* w[kMaxMats];
  const float* s[kMaxMats];
  int out[kMaxMats];
  unsigned wg_begin[kMaxMats + 1];
  int n;
};

template <int KCH, int R, bool NORM = false>
__global__ __launch_bounds__(256) void w8a32_rows_multi_kernel(MatSet ms, const float* x,
                                                               int in_dim, RowNorm rn = RowNorm{}) {
  float* y = ms.y[0];
  const int8_t* w = ms.w[0];
  const float* sc = ms.s[0];
  int out = ms.out[0];
  unsigned b0 = 0;
#pragma unroll
  for (int m = 1; m < kMaxMats; ++m)
    if (m < ms.n && blockIdx.x >= ms.wg_begin[m]) {
      y = ms.y[m];
      w = ms.w[m];
      sc = ms.s[m];
      out = ms.out[m];
      b0 = ms.wg_begin[m];
    }
  w8a32_rows_body<KCH, R, kEpiRows, NORM>(y, x, w, sc, nullptr, in_dim, out, blockIdx.x - b0, nullptr, rn);
}

// Gate/up pairs for any shape: one wave per (token, output j) takes the dots
// of interleaved rows 2j (gate) and 2j + 1 (up) and applies the decode SwiGLU
// (libm expf) or, with PREFILL, the prefill one (swiglu_ref).
template <bool PREFILL = false>
__global__ __launch_bounds__(256) void gate_up_swiglu_w8a32_pairs_kernel(
    float* out, const float* x, const int8_t* w, const float* scales, int seq, int in_dim,
    int inter) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long item = (long long)blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (item >= (long long)seq * inter) return;
  const int s = (int)(item / inter), j = (int)(item % inter);
  const int8_t* wg = w + (size_t)(2 * j) * in_dim;
  const int8_t* wu = wg + in_dim;
  const float* xs = x + (size_t)s * in_dim;
  float ag = 0.0f, au = 0.0f;
  for (int k = lane; k < in_dim; k += kWave) {
    ag = __builtin_fmaf((float)wg[k], xs[k], ag);
    au = __builtin_fmaf((float)wu[k], xs[k], au);
  }
  ag = wave_sum(ag);
  au = wave_sum(au);
  if (lane == 0) {
    const float g = ag * scales[2 * j], u = au * scales[2 * j + 1];
    if constexpr (PREFILL)
      out[(size_t)s * inter + j] = swiglu_ref(g, u, j < (inter & ~7));
    else
      out[(size_t)s * inter + j] = silu_expf(g) * u;
  }
}

// Rows per wave of a one-token matvec: the largest power of two that leaves
// at least 1024 waves (an even spread over the 1024 SIMDs) and keeps the
// weight registers of a wave at most 8-16 KiB in flight.
int rows_per_wave(size_t in_dim, size_t out_rows) {
  const size_t kch = in_dim / 1024;
  const int cap = kch == 1 ? 8 : kch == 2 ? 4 : 2;
  int r = 1;
  while (r < cap && out_rows / (2 * (size_t)r) >= 1024) r *= 2;
  return r;
}

bool w8a32_rows_shape(size_t in_dim, const void* w, const void* x) {
  return in_dim >= 1024 && in_dim % 1024 == 0 && in_dim <= 8192 && aligned16(w) && aligned16(x);
}

// Launches the one-token kernel for (in_dim / 1024, r) on `grid` workgroups
// (with NORM, the input row is rn's normalised h and x is not read).
template <int EPI, bool NORM = false>
void launch_rows(int kch, int r, unsigned grid, hipStream_t st, float* y, const float* x,
                 const int8_t* w, const float* scales, const float* bias, int k, int o,
                 float2* part, const RowNorm& rn = RowNorm{}) {
#define QASR_ROWS(KCH, R)                                                                            \
  if (kch == KCH && r == R) {                                                                        \
    w8a32_rows_kernel<KCH, R, EPI, NORM><<<grid, 256, 0, st>>>(y, x, w, scales, bias, k, o, part, rn); \
    return;                                                                                          \
  }
  if constexpr (EPI != kEpiSwiglu) {
    QASR_ROWS(1, 1) QASR_ROWS(2, 1) QASR_ROWS(3, 1) QASR_ROWS(4, 1)
    QASR_ROWS(5, 1) QASR_ROWS(6, 1) QASR_ROWS(7, 1) QASR_ROWS(8, 1)
  }
  QASR_ROWS(1, 2) QASR_ROWS(1, 4) QASR_ROWS(1, 8)
  QASR_ROWS(2, 2) QASR_ROWS(2, 4)
  QASR_ROWS(3, 2) QASR_ROWS(4, 2)
  QASR_ROWS(5, 2) QASR_ROWS(6, 2)
  QASR_ROWS(7, 2) QASR_ROWS(8, 2)
#undef QASR_ROWS
}

template <bool NORM = false>
void launch_rows_multi(int kch, int r, unsigned grid, hipStream_t st, const MatSet& ms,
                       const float* x, int k, const RowNorm& rn = RowNorm{}) {
#define QASR_ROWS(KCH, R)                                                      \
  if (kch == KCH && r == R) {                                                  \
    w8a32_rows_multi_kernel<KCH, R, NORM><<<grid, 256, 0, st>>>(ms, x, k, rn); \
    return;                                                                    \
  }
  QASR_ROWS(1, 1) QASR_ROWS(1, 2) QASR_ROWS(1, 4) QASR_ROWS(1, 8)
  QASR_ROWS(2, 1) QASR_ROWS(2, 2) QASR_ROWS(2, 4)
  QASR_ROWS(3, 1) QASR_ROWS(3, 2) QASR_ROWS(4, 1) QASR_ROWS(4, 2)
  QASR_ROWS(5, 1) QASR_ROWS(5, 2) QASR_ROWS(6, 1) QASR_ROWS(6, 2)
  QASR_ROWS(7, 1) QASR_ROWS(7, 2) QASR_ROWS(8, 1) QASR_ROWS(8, 2)
#undef QASR_ROWS
}

__global__ __launch_bounds__(256) void w8a32_scalar_kernel(float* y, const float* x, const int8_t* w,
                                                           const float* scales, const float* bias,
                                                           int seq, int in_dim, int out_dim) {
  const int lane = threadIdx.x & (kWave - 1);
  const int o = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (o >= out_dim) return;
  const int8_t* wr = w + (size_t)o * in_dim;
  for (int s = 0; s < seq; ++s) {
    const float* xs = x + (size_t)s * in_dim;
    float acc = 0.0f;
    for (int k = lane; k < in_dim; k += kWave) acc = __builtin_fmaf((float)wr[k], xs[k], acc);
    acc = wave_sum(acc);
    if (lane == 0) {
      float r = acc * scales[o];
      if (bias) r += bias[o];
      y[(size_t)s * out_dim + o] = r;
    }
  }
}

// ---------------------------------------------------------------------------
// Gate/up row interleave (decoder.rs:701-719).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void interleave_kernel(int8_t* wgu, float* sgu, const int8_t* wg,
                                                         const float* sg, const int8_t* wu,
                                                         const float* su, size_t inter,
                                                         size_t hidden) {
  const size_t n = inter * hidden;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const size_t r = i / hidden, c = i - r * hidden;
    wgu[(2 * r) * hidden + c] = wg[i];
    wgu[(2 * r + 1) * hidden + c] = wu[i];
    if (c == 0) {
      sgu[2 * r] = sg[r];
      sgu[2 * r + 1] = su[r];
    }
  }
}

// ---------------------------------------------------------------------------
// W8A8 gate/up + SwiGLU, batch 1: a bandwidth-bound matvec.
//
// A wave owns NP consecutive gate/up pairs (NP * 2 * in_dim contiguous bytes).
// Lane l reads 16-byte slices at byte 1024*c + 16*l of each row, so every load
// instruction of the wave covers 1 KiB contiguous. The lane's matching 16*KCH
// activation bytes live in registers for the whole kernel. All NP*2*KCH weight
// loads are issued before the first v_dot4, then the 2*NP int32 sums are
// reduced across the wave and NP lanes finish the SwiGLU epilogue.
// ---------------------------------------------------------------------------
QASR_DEV int dot16(v4i a, v4i b, int acc) {
  acc = __builtin_amdgcn_sdot4(a[0], b[0], acc, false);
  acc = __builtin_amdgcn_sdot4(a[1], b[1], acc, false);
  acc = __builtin_amdgcn_sdot4(a[2], b[2], acc, false);
  acc = __builtin_amdgcn_sdot4(a[3], b[3], acc, false);
  return acc;
}

template <int KCH, int NP, bool F32IN>
__global__ __launch_bounds__(256) void gateup_matvec_kernel(float* out, const int8_t* w,
                                                            const float* scales, const int8_t* xq8,
                                                            const float* xsc, const float* xf,
                                                            int inter) {
  constexpr int K = KCH * 1024;
  const int lane = threadIdx.x & (kWave - 1);
  const int pair0 = (blockIdx.x * (256 / kWave) + threadIdx.x / kWave) * NP;
  // With F32IN the workgroup quantizes x together (two barriers), so no wave
  // leaves early: waves past the last pair clamp their loads and store nothing.
  if (!F32IN && pair0 >= inter) return;

  // Activations first: their loads (L2-resident) retire before the weight
  // stream's, since a wave's vector loads complete in issue order. fp32 input
  // is read once per workgroup with consecutive 16-byte pieces per lane
  // (thread t: float4 t + 256c); a lane's own 64-byte run of x would put the
  // 64 lanes of one load on 32 different lines.
  v4i xq[KCH];
  float xs = 0.0f;
  float4 xf4[F32IN ? KCH : 1];
  if constexpr (F32IN) {
#pragma unroll
    for (int c = 0; c < KCH; ++c) xf4[c] = ld4(xf, threadIdx.x + 256 * c);
  } else {
#pragma unroll
    for (int c = 0; c < KCH; ++c) xq[c] = reinterpret_cast<const v4i*>(xq8)[c * kWave + lane];
    xs = xsc[0];
  }
  // the epilogue's gate/up scales of lane p < NP, loaded with the activations
  // (after the dot products they would be one more memory round trip)
  const int j_ep = min(pair0 + (lane < NP ? lane : 0), inter - 1);
  const float2 sc_ep = make_float2(scales[2 * j_ep], scales[2 * j_ep + 1]);

  // Then the weight stream: NP pairs x 2 rows x KCH slices, all in flight.
  v4i wv[NP][2][KCH];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int pr = pair0 + p < inter ? pair0 + p : inter - 1;  // clamp the tail, result discarded
    const v4i* row = reinterpret_cast<const v4i*>(w + (size_t)pr * 2 * K);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int c = 0; c < KCH; ++c) wv[p][r][c] = __builtin_nontemporal_load(row + r * (K / 16) + c * kWave + lane);
  }

  // All weight loads stay issued before any use (the scheduler would otherwise
  // sink them next to their dot products and serialise their latency).
  __builtin_amdgcn_sched_barrier(0);

  // Per-vector quantization of x (quantize.rs:633-662) overlaps the weight
  // stream: the workgroup's absmax (NaN never wins, as `if abs > absmax`),
  // the int8 vector into LDS, then each lane's 16*KCH bytes back out. The
  // barriers wait on LDS only, so the weight loads stay in flight.
  if constexpr (F32IN) {
    __shared__ float red[256 / kWave];
    __shared__ int xq_lds[KCH * 256];
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
      const float a[4] = {fabsf(xf4[c].x), fabsf(xf4[c].y), fabsf(xf4[c].z), fabsf(xf4[c].w)};
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (a[t] > m) m = a[t];
    }
    m = wave_max(m);
    if (lane == 0) red[threadIdx.x / kWave] = m;
    lds_barrier();
    m = red[0];
#pragma unroll
    for (int i = 1; i < 256 / kWave; ++i) m = red[i] > m ? red[i] : m;
    const float inv = m > 0.0f ? 127.0f / m : 0.0f;
#pragma unroll
    for (int c = 0; c < KCH; ++c)
      xq_lds[threadIdx.x + 256 * c] = (quant_i8(xf4[c].x, inv) & 0xff) | ((quant_i8(xf4[c].y, inv) & 0xff) << 8) |
                                      ((quant_i8(xf4[c].z, inv) & 0xff) << 16) |
                                      ((quant_i8(xf4[c].w, inv) & 0xff) << 24);
    lds_barrier();
#pragma unroll
    for (int c = 0; c < KCH; ++c) xq[c] = reinterpret_cast<const v4i*>(xq_lds)[c * kWave + lane];
    xs = m / 127.0f;
  }

  int acc[NP][2];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      int a = 0;
#pragma unroll
      for (int c = 0; c < KCH; ++c) a = dot16(wv[p][r][c], xq[c], a);
      acc[p][r] = group_sum_i32<kWave>(a);
    }
  if (lane < NP && pair0 + lane < inter) {
    int dg = acc[0][0], du = acc[0][1];
#pragma unroll
    for (int p = 1; p < NP; ++p)
      if (lane == p) { dg = acc[p][0]; du = acc[p][1]; }
    const int j = pair0 + lane;
    out[j] = swiglu_w8a8(dg, du, xs, sc_ep.x, sc_ep.y);
  }
}

// Any in_dim % 16 == 0 (and batch >= 1) without the register budget of the
// matvec kernel: one wave per (pair, token), weight slices re-read per token.
__global__ __launch_bounds__(256) void gateup_generic_kernel(float* out, const int8_t* w,
                                                             const float* scales,
                                                             const int8_t* xq, const float* xs,
                                                             int batch, int in_dim, int inter) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long item = (long long)blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (item >= (long long)batch * inter) return;
  const int b = (int)(item / inter), j = (int)(item % inter);
  const v4i* g = reinterpret_cast<const v4i*>(w + (size_t)(2 * j) * in_dim);
  const v4i* u = reinterpret_cast<const v4i*>(w + (size_t)(2 * j + 1) * in_dim);
  const v4i* xv = reinterpret_cast<const v4i*>(xq + (size_t)b * in_dim);
  int dg = 0, du = 0;
  for (int c = lane; c < in_dim / 16; c += kWave) {
    const v4i xx = xv[c];
    dg = dot16(g[c], xx, dg);
    du = dot16(u[c], xx, du);
  }
  dg = group_sum_i32<kWave>(dg);
  du = group_sum_i32<kWave>(du);
  if (lane == 0) out[(size_t)b * inter + j] = swiglu_w8a8(dg, du, xs[b], scales[2 * j], scales[2 * j + 1]);
}

constexpr int kMatvecPairs = 3;  // pairs per wave: 12 per 4-wave workgroup

template <bool F32IN>
int launch_matvec(float* out, const int8_t* w, const float* scales, const int8_t* xq,
                  const float* xs, const float* xf, size_t in_dim, size_t inter, hipStream_t st) {
  const unsigned grid =
      (unsigned)((inter + kMatvecPairs * 4 - 1) / (kMatvecPairs * 4));
  switch (in_dim / 1024) {
    case 1: gateup_matvec_kernel<1, kMatvecPairs, F32IN><<<grid, 256, 0, st>>>(out, w, scales, xq, xs, xf, (int)inter); break;
    case 2: gateup_matvec_kernel<2, kMatvecPairs, F32IN><<<grid, 256, 0, st>>>(out, w, scales, xq, xs, xf, (int)inter); break;
    case 3: gateup_matvec_kernel<3, kMatvecPairs, F32IN><<<grid, 256, 0, st>>>(out, w, scales, xq, xs, xf, (int)inter); break;
    case 4: gateup_matvec_kernel<4, 4, F32IN><<<(unsigned)((inter + 15) / 16), 256, 0, st>>>(out, w, scales, xq, xs, xf, (int)inter); break;
    default: return fail(QASR_ERR_UNSUPPORTED, "gate_up matvec: in_dim must be 1024..4096 in steps of 1024");
  }
  return launch_status("gate_up_swiglu_w8a8 (matvec)");
}

bool matvec_shape(size_t in_dim) { return in_dim % 1024 == 0 && in_dim >= 1024 && in_dim <= 4096; }

// ---------------------------------------------------------------------------
// W8A32 linear for many tokens (prefill) on the bf16 matrix cores, fp32-exact
// products: the reference's T matvecs (kernels/mod.rs:655-660) as one GEMM
//   y[t, n] = (sum_k (f32)w[n, k] * x[t, k]) * scales[n] (+ bias[n]).
// An int8 weight is exact in bf16, and an fp32 activation is exactly
// hi + mid + lo with three bf16 terms (truncation: 8 + 8 + 8 mantissa bits),
// so every product w * x = w*hi + w*mid + w*lo is formed exactly and summed in
// fp32 by v_mfma_f32_16x16x32_bf16 -- the same fp32-sum arithmetic as the
// reference, only in another order.
// Two kernels. The LDS-staged one: a workgroup owns 128 weight rows x 64
// tokens and walks K in chunks of 64; the chunk's weights (as bf16) and
// activations (as the three bf16 terms) are staged in LDS, then each of the 4
// waves (64 rows x 32 tokens) runs 2 k-steps x 3 terms x 4 x 2 MFMA tiles. The
// split-K one (smaller grids): the 4 waves share a smaller tile, split K
// between them and load their fragments straight into registers.
// MFMA operands: A[i][k] (lane i + 16*(k/8), element k%8) = weight row i,
// B[k][j] = token j; the result lane l holds rows 4*(l/16)+v of token l%16.
// ---------------------------------------------------------------------------
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
constexpr int kGmBK = 64;           // K granularity of the GEMM path
// GEMM epilogues: y = acc * scale; + bias; or the SwiGLU of each interleaved
// (gate, up) row pair, y[t, n/2] = swiglu(y[t, n], y[t, n + 1]), an output row
// of N/2 -- in the prefill form (kernels::swiglu_multiply's fast_exp blocks and
// expf tail after the gate/up projection) or the decode loop's form
// (g / (1 + expf(-g)) * u, decoder.rs:916-921) for batched decode streams;
// or the q/k/v heads of a prefill chunk (head norms, RoPE, KV-cache rows)
// or, in the split-K kernel only, the prefill residual add: h[t, n] += y and
// each token's sum of squares of its updated 64-row slice (kGemmResidual).
// kGemmXNorm added to an epilogue of the LDS-staged kernels folds the prefill
// RMSNorm into their activation staging (see GemmXNorm).
enum GemmEpi { kGemmRows = 0, kGemmBias = 1, kGemmSwiglu = 2, kGemmSwigluLibm = 3, kGemmHeads = 4,
               kGemmResidual = 5 };
constexpr int kGemmXNorm = 8;
// K chunks in flight per thread in the single-buffered LDS-staged kernel (2
// and 3 measured slower: 1.7B gate/up at T = 512 86.0 -> 88.2 / 97.5 us), and
// register sets of the double-buffered one (4 sets measured the same as 2)
constexpr int kGemmPrefetch = 1;
constexpr int kGemmSets = 2;
constexpr int kGemmPcSets = 4;  // the producer/consumer kernel's register sets (chunks in flight)

QASR_DEV unsigned short bf16_bits_trunc(float v) { return (unsigned short)(__float_as_uint(v) >> 16); }
QASR_DEV float bf16_trunc(float v) { return __uint_as_float(__float_as_uint(v) & 0xffff0000u); }
// bf16 bits of two floats, truncated, packed low element first
QASR_DEV unsigned bf16_pair(float lo_elem, float hi_elem) {
  return __builtin_amdgcn_perm(__float_as_uint(hi_elem), __float_as_uint(lo_elem), 0x07060302u);
}

// BN weight rows x BT tokens per workgroup (BN in {64, 128}, BT in {32, 64});
// the 4 waves form a 2 x 2 grid of (BN/2) x (BT/2) tiles.
// Up to 4 weight matrices of the same activations (q/k/v) in one launch:
// column-of-workgroups ranges [bx_begin[m], bx_begin[m + 1]) compute matrix m.
struct GemmSet {
  float* y[4];
  const int8_t* w[4];
  const float* s[4];
  const float* b[4];
  int N[4];
  unsigned bx_begin[5];
  int n;
  float* ss;          // kGemmResidual: [T][ceil(N / 64)] sums of squares of the updated rows
  float* hg;          // kGemmResidual (optional): the updated rows times gain[n], the next norm's input
  const float* gain;
};

// Workgroup -> tile map. The grid is one-dimensional over cols x rows tiles
// and workgroup b runs on XCD b % 8. With split_cols = a > 0, XCD c owns the
// rectangle of cols/a column blocks x rows/(8/a) token blocks at (c % a, c / a),
// so the weights and activations it reads fit its own L2; split_cols = 0 keeps
// the row-major order (column block fastest).
struct TileMap {
  unsigned cols, rows, split_cols;
};

QASR_DEV void tile_of(const TileMap& m, unsigned b, unsigned& bx, unsigned& by) {
  if (m.split_cols == 0) {
    bx = b % m.cols;
    by = b / m.cols;
    return;
  }
  const unsigned xcd = b % 8, slot = b / 8;
  const unsigned ca = m.cols / m.split_cols, rb = m.rows / (8 / m.split_cols);
  bx = (xcd % m.split_cols) * ca + slot % ca;
  by = (xcd / m.split_cols) * rb + slot / ca;
}

// NPF chunks of weights and activations are in flight in registers: the loads
// of chunk c + NPF are issued right after chunk c is staged into LDS.
// Rows n..n+3 (n a multiple of 4) of token t are the interleaved pairs of
// outputs n/2 and n/2 + 1 of the SwiGLU row (N/2 wide).
template <int EPI>
QASR_DEV void swiglu_store(float* y, const float (&res)[4], int t, int n, int N) {
  const int inter = N >> 1, j = n >> 1, fast_end = EPI == kGemmSwiglu ? inter & ~7 : 0;
  float* row = y + (size_t)t * inter;
  if (n + 1 < N) row[j] = swiglu_ref(res[0], res[1], j < fast_end);
  if (n + 3 < N) row[j + 1] = swiglu_ref(res[2], res[3], j + 1 < fast_end);
}

// The kGemmHeads epilogue: the q/k/v projections of a prefill chunk (one
// sequence, token t at position start_pos + t) with the steps after them,
// decoder.rs:799-810. The launch's matrices are q, k and v (set index 0, 1,
// 2), every tile is one 128-row head x BT tokens, and per token:
//   q head: per-head RMSNorm (q_norm_w) + NeoX RoPE, written to y (in place
//           of the plain projection's output);
//   k head: the same with k_norm_w, written to k_cache row start_pos + t;
//   v head: written to v_cache row start_pos + t.
// A position outside the RoPE table or the cache gives a NaN q row and no
// cache write. The dequantized products are the plain epilogue's (acc *
// scale) and the heads go through head_norm_rope, so the results equal the
// GEMM followed by qasr_head_rms_norm_rope_kv_f32 bit for bit.
struct GemmHeadEpi {
  float* k_cache;  // [cache_rows][n_kv_heads * 128]
  float* v_cache;
  const float* q_norm_w;
  const float* k_norm_w;
  const float* cos_tab;  // [table_rows][128]
  const float* sin_tab;
  long long start_pos;
  long long table_rows;
  long long cache_rows;
  int n_kv_heads;
  float eps;
};

// The prefill RMSNorm folded into the LDS-staged GEMMs (kGemmXNorm). The
// activations are hg = h * gain, the residual stream times the norm's gain
// (written by the kGemmResidual epilogue that produced h), staged like any
// activations; token t's 1 / rms = 1 / sqrt(sum / K + eps), with sum the
// `slices` partial sums of squares ss[t][0..slices-1] of h added in slice
// order, multiplies the token's outputs in the epilogue: y = (acc * scale) *
// rinv, the reference's rms_norm (kernels/mod.rs:897-918) + projection with
// the scalar factored out of the dot product. Each lane loads its epilogue
// tokens' partials when the kernel starts and adds them after the k loop.
struct GemmXNorm {
  const float* ss;
  int slices;  // a multiple of 4, at most kXnMaxSlices
  float eps;
};
constexpr int kXnMaxSlices = 32;  // in_dim <= 2048

QASR_DEV void xnorm_load(float (&p)[kXnMaxSlices], const GemmXNorm& xn, int t) {
  const float* row = xn.ss + (size_t)t * (size_t)xn.slices;
#pragma unroll
  for (int u = 0; u < kXnMaxSlices; u += 4) {
    const float4 v = u < xn.slices ? *reinterpret_cast<const float4*>(row + u) : make_float4(0.f, 0.f, 0.f, 0.f);
    p[u] = v.x;
    p[u + 1] = v.y;
    p[u + 2] = v.z;
    p[u + 3] = v.w;
  }
}
QASR_DEV float xnorm_rinv(const float (&p)[kXnMaxSlices], int K, float eps) {
  float sum = 0.0f;
#pragma unroll
  for (int u = 0; u < kXnMaxSlices; ++u) sum += p[u];  // the zero slots past `slices` add nothing
  return 1.0f / sqrtf(sum / (float)K + eps);
}

constexpr int kHeadTilePitch = 136;  // floats per token row of the staged head tile (pad: banks)

// acc: the 4 waves' MI x MJ blocks of 32 x 32 (lane l, register 4q + v of
// block (i, j) = row 64 wr + 32i + 8q + 4(l/32) + v of token 32 wc + 32j +
// l%32 of the tile). Called after the k loop's last barrier (LDS free). RT:
// the outputs of token column j are also multiplied by rt[j].
template <int BT, int MI, int MJ, bool RT>
QASR_DEV void gemm_heads_epilogue(const v16f (&acc)[MI][MJ], float* tile, int mat, float* y,
                                  const float* __restrict__ scales, int N, int n0, int t0, int T,
                                  const GemmHeadEpi& he, const float (&rt)[MJ]) {
  static_assert(MI == 2 && BT == 64 * MJ, "a 128-row head per tile");
  static_assert(BT * kHeadTilePitch * 4 <= (size_t)(128 + 3 * BT) * (kGmBK + 8) * 2, "the tile fits one stage");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave & 1, wc = wave >> 1;
  const int r = lane & 31, g = lane >> 5;
#pragma unroll
  for (int j = 0; j < MJ; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = 64 * wr + 32 * i + 8 * q + 4 * g;
        const float4 s = *reinterpret_cast<const float4*>(scales + n0 + nl);
        float4 v = make_float4(acc[i][j][4 * q] * s.x, acc[i][j][4 * q + 1] * s.y,
                               acc[i][j][4 * q + 2] * s.z, acc[i][j][4 * q + 3] * s.w);
        if constexpr (RT) {  // the folded RMSNorm's 1 / rms of the lane's token
          v.x *= rt[j];
          v.y *= rt[j];
          v.z *= rt[j];
          v.w *= rt[j];
        }
        *reinterpret_cast<float4*>(tile + ((BT / 2) * wc + 32 * j + r) * kHeadTilePitch + nl) = v;
      }
  lds_barrier();
  // 16 threads per token, in head_norm_rope's lane layout: dims 4sub.. and 64 + 4sub..
  const int sub = tid & 15;
  float4 w1, w2;
  if (mat < 2) {
    const float* w = mat == 0 ? he.q_norm_w : he.k_norm_w;
    w1 = ld4(w, sub);
    w2 = ld4(w + 64, sub);
  }
  const int head = n0 / 128;
  const size_t kv_dim = (size_t)he.n_kv_heads * 128;
#pragma unroll
  for (int p = 0; p < BT / 16; ++p) {
    const int tl = 16 * p + (tid >> 4), t = t0 + tl;
    float4 x1 = *reinterpret_cast<const float4*>(tile + tl * kHeadTilePitch + 4 * sub);
    float4 x2 = *reinterpret_cast<const float4*>(tile + tl * kHeadTilePitch + 64 + 4 * sub);
    const long long pos = he.start_pos + t;
    const bool pos_ok = pos < he.table_rows && pos < he.cache_rows;
    if (mat < 2) {
      const long long pr = pos_ok ? pos : 0;  // out-of-table rows read row 0, then become NaN
      const float* cr = he.cos_tab + pr * 128;
      const float* sr = he.sin_tab + pr * 128;
      const float4 c1 = ld4(cr, sub), c2 = ld4(cr + 64, sub);
      const float4 s1 = ld4(sr, sub), s2 = ld4(sr + 64, sub);
      // every lane of the group joins the reduction, past T or not
      head_norm_rope<128, true, true>(x1, x2, w1, w2, c1, c2, s1, s2, pos_ok, he.eps);
    }
    if (t >= T) continue;
    float* dst = nullptr;
    if (mat == 0) {
      dst = y + (size_t)t * N + n0;
    } else if (pos_ok) {  // a row outside the cache is not written
      dst = (mat == 1 ? he.k_cache : he.v_cache) + (size_t)pos * kv_dim + (size_t)head * 128;
    }
    if (dst) {
      st4(dst, sub, x1);
      st4(dst + 64, sub, x2);
    }
  }
}

// Row scales (and biases) of a wave's 32 MI rows r0 .. r0 + 32 MI - 1, loaded
// before the k loop so that the epilogue does not wait on memory after it.
// Lane l, register k holds row r0 + 64k + l (clamped to the last row past the
// end); the accumulator element for row offset 32i + 8q + 4g + v is read from
// lane (32i + 8q + 4g + v) % 64, register i / 2, with a cross-lane permute.
template <int MI, bool BIAS>
struct GemmEpiRows {
  static constexpr int R = (32 * MI + 63) / 64;
  float s[R];
  float b[R];
  QASR_DEV void load(const float* scales, const float* bias, int N, int r0, int lane) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const int nv = min(r0 + 64 * k + lane, N - 1);
      s[k] = scales[nv];
      if constexpr (BIAS) b[k] = bias[nv];
    }
  }
  QASR_DEV float scale(int i, int off) const { return __shfl(s[i >> 1], 32 * (i & 1) + off, kWave); }
  QASR_DEV float shift(int i, int off) const { return __shfl(b[i >> 1], 32 * (i & 1) + off, kWave); }
};

// The epilogue of the LDS-staged kernels, run by the 4 waves that hold the
// accumulators (threads 0..255) after the k loop's last barrier: 1 / rms of
// the folded RMSNorm, then the heads epilogue or the row scales (and biases)
// with a plain, SwiGLU or bias store.
template <int BN, int BT, int EPI, int MI, int MJ>
QASR_DEV void gemm_tile_epilogue(const v16f (&acc)[MI][MJ], const GemmEpiRows<MI, (EPI & 7) == kGemmBias>& ep,
                                 const float (&xp)[MJ][kXnMaxSlices], const GemmXNorm& xn, int K,
                                 unsigned short* lds, int mat, float* y, const float* __restrict__ scales, int N,
                                 int n0, int t0, int T, const GemmHeadEpi& he) {
  constexpr int EP = EPI & 7;
  constexpr bool XN = (EPI & kGemmXNorm) != 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wr = wave & 1, wc = wave >> 1;
  const int r = lane & 31, g = lane >> 5;
  [[maybe_unused]] float rt[MJ];  // XN: 1 / rms of the lane's tokens
  if constexpr (XN) {
#pragma unroll
    for (int j = 0; j < MJ; ++j) rt[j] = xnorm_rinv(xp[j], K, xn.eps);
  }
  if constexpr (EP == kGemmHeads) {
    static_assert(BN == 128, "one head per tile");
    gemm_heads_epilogue<BT, MI, MJ, XN>(acc, reinterpret_cast<float*>(lds), mat, y, scales, N, n0, t0, T, he,
                                        rt);
    return;
  }
  // lane l, register 4q + v of block (i, j) holds row n0 + (BN/2)wr + 32i + 8q + 4(l/32) + v
  // of token t0 + (BT/2)wc + 32j + l%32
  const bool vec_out = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
#pragma unroll
  for (int j = 0; j < MJ; ++j) {
    const int t = t0 + (BT / 2) * wc + 32 * j + r;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + (BN / 2) * wr + 32 * i + 8 * q + 4 * g;
        float res[4];
        // the cross-lane reads run with every lane active (an inactive source
        // lane reads as 0); lanes past the last token only skip the stores
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          res[v] = acc[i][j][4 * q + v] * ep.scale(i, 8 * q + 4 * g + v);
          if constexpr (XN) res[v] *= rt[j];
          if constexpr (EP == kGemmBias) res[v] += ep.shift(i, 8 * q + 4 * g + v);
        }
        if (t < T) {
          if constexpr (EP == kGemmSwiglu || EP == kGemmSwigluLibm) {
            swiglu_store<EP>(y, res, t, n, N);
          } else if (vec_out && n + 3 < N) {
            *reinterpret_cast<float4*>(&y[(size_t)t * N + n]) = make_float4(res[0], res[1], res[2], res[3]);
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (n + v < N) y[(size_t)t * N + n + v] = res[v];
          }
        }
      }
  }
}

template <int BN, int BT, int BK, int NPF, int EPI>
__global__ __launch_bounds__(256) void w8a32_gemm_bf16x3_kernel(GemmSet set, TileMap map,
                                                                const float* __restrict__ x, int T, int K,
                                                                GemmHeadEpi he, GemmXNorm xn) {
  constexpr int kGmRow = BK + 8;  // LDS row in bf16 (16-byte pad)
  constexpr int EP = EPI & 7;                       // the epilogue
  constexpr bool XN = (EPI & kGemmXNorm) != 0;      // RMSNorm folded in (1 / rms in the epilogue)
  extern __shared__ __align__(16) unsigned short gm_lds[];  // [BN][kGmRow] weights, [3][BT][kGmRow] terms
  unsigned bx, by;
  tile_of(map, blockIdx.x, bx, by);
  float* y = set.y[0];
  const int8_t* w = set.w[0];
  const float* scales = set.s[0];
  const float* bias = set.b[0];
  int N = set.N[0];
  unsigned bx0 = 0;
  int mat = 0;
#pragma unroll
  for (int m = 1; m < 4; ++m)
    if (m < set.n && bx >= set.bx_begin[m]) {
      y = set.y[m];
      w = set.w[m];
      scales = set.s[m];
      bias = set.b[m];
      N = set.N[m];
      bx0 = set.bx_begin[m];
      mat = m;
    }
  // 32x32x16 products: a wave's (BN/2) x (BT/2) tile is MI x MJ blocks of 32 x 32
  // (the 16x16x32 form needs twice the independent accumulators to keep the
  // matrix pipe full at one wave per SIMD)
  constexpr int MI = BN / 64, MJ = BT / 64;
  static_assert(BN % 64 == 0 && BT % 64 == 0, "32 x 32 blocks per wave");
  constexpr int TPW = 256 / BN, WB = BK / TPW;       // weight staging: threads per row, bytes each
  constexpr int TPX = 256 / BT, XF = BK / TPX;       // activation staging: threads per token, floats each
  auto wl = reinterpret_cast<unsigned short (*)[kGmRow]>(gm_lds);
  auto xl = reinterpret_cast<unsigned short (*)[BT][kGmRow]>(gm_lds + BN * kGmRow);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave & 1, wc = wave >> 1;
  const int r = lane & 31, g = lane >> 5;
  const int n0 = (int)(bx - bx0) * BN, t0 = (int)by * BT;
  v16f acc[MI][MJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[i][j] = v16f{};
  [[maybe_unused]] GemmEpiRows<MI, EP == kGemmBias> ep;
  if constexpr (EP != kGemmHeads) ep.load(scales, bias, N, n0 + (BN / 2) * wr, lane);

  // rows and tokens past the end re-read the last one (valid memory; not stored)
  // Staging items: weight item c is 16 bytes of row 64c + tid / 4 at byte
  // 16 (tid % 4) of the chunk; activation item c is 4 floats of token
  // 16c + tid / 16 at float 4 (tid % 16). A wave's load then covers 16 rows x
  // 64 bytes or 4 tokens x 256 bytes: 16 or 8 cache lines per instruction, not
  // one line per lane pair.
  static_assert(BK == 64 && WB / 16 == BN / 64 && XF / 4 == BT / 16, "item counts of the staging map");
  const int w_part = tid & 3, x_part = tid & 15;
  const int8_t* wsrc[WB / 16];
  const float* xsrc[XF / 4];
#pragma unroll
  for (int c = 0; c < WB / 16; ++c) wsrc[c] = w + (size_t)min(n0 + 64 * c + (tid >> 2), N - 1) * K + 16 * w_part;
#pragma unroll
  for (int c = 0; c < XF / 4; ++c) xsrc[c] = x + (size_t)min(t0 + 16 * c + (tid >> 4), T - 1) * K + 4 * x_part;
  [[maybe_unused]] float xp[MJ][kXnMaxSlices];  // XN: the partial sums of squares of the lane's epilogue tokens
  if constexpr (XN) {
#pragma unroll
    for (int j = 0; j < MJ; ++j) xnorm_load(xp[j], xn, min(t0 + (BT / 2) * wc + 32 * j + r, T - 1));
  }

  v4i wv[NPF][WB / 16];
  v4f xv[NPF][XF / 4];
#pragma unroll
  for (int q = 0; q < NPF; ++q)
    if (q * BK < K) {
#pragma unroll
      for (int c = 0; c < WB / 16; ++c) wv[q][c] = *reinterpret_cast<const v4i*>(wsrc[c] + q * BK);
#pragma unroll
      for (int c = 0; c < XF / 4; ++c) xv[q][c] = *reinterpret_cast<const v4f*>(xsrc[c] + q * BK);
    }
  for (int kb = 0; kb < K; kb += NPF * BK) {
#pragma unroll
    for (int q = 0; q < NPF; ++q) {
      const int k0 = kb + q * BK;
      if (k0 >= K) break;
#pragma unroll
      for (int c = 0; c < WB / 16; ++c) {
        v4i wc = wv[q][c];
        asm volatile("" : "+v"(wc));  // keeps the conversion from being hoisted next to the load
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // int8 -> bf16 is exact (at most 8 significant bits)
          const int v = wc[e];
          const uint2 h = make_uint2(bf16_pair((float)(int8_t)(v & 0xff), (float)(int8_t)((v >> 8) & 0xff)),
                                     bf16_pair((float)(int8_t)((v >> 16) & 0xff), (float)(int8_t)((v >> 24) & 0xff)));
          *reinterpret_cast<uint2*>(&wl[64 * c + (tid >> 2)][16 * w_part + 4 * e]) = h;
        }
      }
#pragma unroll
      for (int c = 0; c < XF / 4; ++c) {  // x = hi + mid + lo exactly
        v4f xc = xv[q][c];
        asm volatile("" : "+v"(xc));
        const float ev[4] = {xc.x, xc.y, xc.z, xc.w};
        float r1[4], r2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r1[e] = ev[e] - bf16_trunc(ev[e]);
          r2[e] = r1[e] - bf16_trunc(r1[e]);  // at most 8 significant bits
        }
        const int tok = 16 * c + (tid >> 4), col = 4 * x_part;
        *reinterpret_cast<uint2*>(&xl[0][tok][col]) = make_uint2(bf16_pair(ev[0], ev[1]), bf16_pair(ev[2], ev[3]));
        *reinterpret_cast<uint2*>(&xl[1][tok][col]) = make_uint2(bf16_pair(r1[0], r1[1]), bf16_pair(r1[2], r1[3]));
        *reinterpret_cast<uint2*>(&xl[2][tok][col]) = make_uint2(bf16_pair(r2[0], r2[1]), bf16_pair(r2[2], r2[3]));
      }
      lds_barrier();  // the staged chunk is visible to every wave
      if (k0 + NPF * BK < K) {
#pragma unroll
        for (int c = 0; c < WB / 16; ++c)
          wv[q][c] = *reinterpret_cast<const v4i*>(wsrc[c] + k0 + NPF * BK);
#pragma unroll
        for (int c = 0; c < XF / 4; ++c) xv[q][c] = *reinterpret_cast<const v4f*>(xsrc[c] + k0 + NPF * BK);
      }
#pragma unroll
      for (int kk = 0; kk < BK; kk += 16) {
        v8bf a[MI], b[3][MJ];
#pragma unroll
        for (int i = 0; i < MI; ++i)
          a[i] = *reinterpret_cast<const v8bf*>(&wl[(BN / 2) * wr + 32 * i + r][kk + 8 * g]);
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
          for (int j = 0; j < MJ; ++j)
            b[term][j] = *reinterpret_cast<const v8bf*>(&xl[term][(BT / 2) * wc + 32 * j + r][kk + 8 * g]);
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < MJ; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[term][j], acc[i][j], 0, 0, 0);
      }
      lds_barrier();  // LDS only: the prefetched chunk's global loads stay in flight
    }
  }

  gemm_tile_epilogue<BN, BT, EPI>(acc, ep, xp, xn, K, gm_lds, mat, y, scales, N, n0, t0, T, he);
}

template <int BN, int BT, int BK>
constexpr size_t gemm_lds_bytes() {
  return (size_t)(BN + 3 * BT) * (BK + 8) * 2;
}

// Double-buffered form of the LDS-staged kernel, same tiles, same products in
// the same order per accumulator (so the same results bit for bit). Two LDS
// stages: while the MFMAs of chunk c read one stage, chunk c + 1 is converted
// (int8 -> bf16, fp32 -> three bf16 terms) and written to the other, a slice
// of that work after each 16-wide k step, so the conversion's VALU work issues
// while the matrix pipe is busy instead of after it. Chunk c + 2's global
// loads are in flight meanwhile in a second register set. One barrier per
// chunk: it both publishes the staged chunk and retires the reads of the stage
// the next chunk overwrites.
template <int BN, int BT, int BK, int NS, int EPI>
__global__ __launch_bounds__(256) void w8a32_gemm_bf16x3_db_kernel(GemmSet set, TileMap map,
                                                                   const float* __restrict__ x, int T, int K,
                                                                   GemmHeadEpi he, GemmXNorm xn) {
  constexpr int kGmRow = BK + 8;                   // LDS row in bf16 (16-byte pad)
  constexpr int STAGE = (BN + 3 * BT) * kGmRow;    // bf16 per LDS stage
  extern __shared__ __align__(16) unsigned short gm_lds[];  // 2 x ([BN][kGmRow] weights, [3][BT][kGmRow] terms)
  unsigned bx, by;
  tile_of(map, blockIdx.x, bx, by);
  float* y = set.y[0];
  const int8_t* w = set.w[0];
  const float* scales = set.s[0];
  const float* bias = set.b[0];
  int N = set.N[0];
  unsigned bx0 = 0;
  int mat = 0;
#pragma unroll
  for (int m = 1; m < 4; ++m)
    if (m < set.n && bx >= set.bx_begin[m]) {
      y = set.y[m];
      w = set.w[m];
      scales = set.s[m];
      bias = set.b[m];
      N = set.N[m];
      bx0 = set.bx_begin[m];
      mat = m;
    }
  constexpr int MI = BN / 64, MJ = BT / 64;
  static_assert(BN % 64 == 0 && BT % 64 == 0, "32 x 32 blocks per wave");
  constexpr int EP = EPI & 7;                       // the epilogue
  constexpr bool XN = (EPI & kGemmXNorm) != 0;      // RMSNorm folded in (1 / rms in the epilogue)
  constexpr int NW = BN / 64, NX = BT / 16;         // 16-byte staging items per thread
  constexpr int KSTEPS = BK / 16;                    // MFMA k steps per chunk
  static_assert(NW >= 1 && NX >= 1, "each thread stages whole 16-byte items");
  static_assert(NS >= 2 && NS % 2 == 0, "an even number of register sets");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave & 1, wc = wave >> 1;
  const int r = lane & 31, g = lane >> 5;
  const int n0 = (int)(bx - bx0) * BN, t0 = (int)by * BT;
  v16f acc[MI][MJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[i][j] = v16f{};
  [[maybe_unused]] GemmEpiRows<MI, EP == kGemmBias> ep;
  if constexpr (EP != kGemmHeads) ep.load(scales, bias, N, n0 + (BN / 2) * wr, lane);

  // rows and tokens past the end re-read the last one (valid memory; not stored)
  // staging items as in the single-buffered kernel (16 or 8 lines per load instruction)
  static_assert(BK == 64 && NW == BN / 64 && NX == BT / 16, "item counts of the staging map");
  const int w_part = tid & 3, x_part = tid & 15;
  const int8_t* wsrc[NW];
  const float* xsrc[NX];
#pragma unroll
  for (int c = 0; c < NW; ++c) wsrc[c] = w + (size_t)min(n0 + 64 * c + (tid >> 2), N - 1) * K + 16 * w_part;
#pragma unroll
  for (int c = 0; c < NX; ++c) xsrc[c] = x + (size_t)min(t0 + 16 * c + (tid >> 4), T - 1) * K + 4 * x_part;
  [[maybe_unused]] float xp[MJ][kXnMaxSlices];  // XN: the partial sums of squares of the lane's epilogue tokens
  if constexpr (XN) {
#pragma unroll
    for (int j = 0; j < MJ; ++j) xnorm_load(xp[j], xn, min(t0 + (BT / 2) * wc + 32 * j + r, T - 1));
  }

  auto load = [&](v4i (&wv)[NW], v4f (&xv)[NX], int k0) {
#pragma unroll
    for (int c = 0; c < NW; ++c) wv[c] = *reinterpret_cast<const v4i*>(wsrc[c] + k0);
#pragma unroll
    for (int c = 0; c < NX; ++c) xv[c] = *reinterpret_cast<const v4f*>(xsrc[c] + k0);
  };
  // The staging items that go after k step `part` (item c of N after step c * KSTEPS / N).
  // Each item passes through an empty asm first: the conversion cannot then be
  // hoisted next to the item's load, which would wait for the load right there.
  auto stage = [&](const v4i (&wv)[NW], const v4f (&xv)[NX], unsigned short* st, int part) {
    auto wl = reinterpret_cast<unsigned short (*)[kGmRow]>(st);
    auto xl = reinterpret_cast<unsigned short (*)[BT][kGmRow]>(st + BN * kGmRow);
#pragma unroll
    for (int c = 0; c < NW; ++c) {
      if (part >= 0 && c * KSTEPS / NW != part) continue;
      v4i wc = wv[c];
      asm volatile("" : "+v"(wc));
#pragma unroll
      for (int e = 0; e < 4; ++e) {  // int8 -> bf16 is exact (at most 8 significant bits)
        const int v = wc[e];
        const uint2 h = make_uint2(bf16_pair((float)(int8_t)(v & 0xff), (float)(int8_t)((v >> 8) & 0xff)),
                                   bf16_pair((float)(int8_t)((v >> 16) & 0xff), (float)(int8_t)((v >> 24) & 0xff)));
        *reinterpret_cast<uint2*>(&wl[64 * c + (tid >> 2)][16 * w_part + 4 * e]) = h;
      }
    }
#pragma unroll
    for (int c = 0; c < NX; ++c) {  // x = hi + mid + lo exactly
      if (part >= 0 && c * KSTEPS / NX != part) continue;
      v4f xc = xv[c];
      asm volatile("" : "+v"(xc));
      const float ev[4] = {xc.x, xc.y, xc.z, xc.w};
      float r1[4], r2[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r1[e] = ev[e] - bf16_trunc(ev[e]);
        r2[e] = r1[e] - bf16_trunc(r1[e]);  // at most 8 significant bits
      }
      const int tok = 16 * c + (tid >> 4), col = 4 * x_part;
      *reinterpret_cast<uint2*>(&xl[0][tok][col]) = make_uint2(bf16_pair(ev[0], ev[1]), bf16_pair(ev[2], ev[3]));
      *reinterpret_cast<uint2*>(&xl[1][tok][col]) = make_uint2(bf16_pair(r1[0], r1[1]), bf16_pair(r1[2], r1[3]));
      *reinterpret_cast<uint2*>(&xl[2][tok][col]) = make_uint2(bf16_pair(r2[0], r2[1]), bf16_pair(r2[2], r2[3]));
    }
  };
  // k step s of the chunk staged in `st`: every product term in the order of
  // the single-buffered kernel (term, then row block, then token block).
  auto mfma_step = [&](const unsigned short* st, int s) {
    auto wl = reinterpret_cast<const unsigned short (*)[kGmRow]>(st);
    auto xl = reinterpret_cast<const unsigned short (*)[BT][kGmRow]>(st + BN * kGmRow);
    const int kk = 16 * s;
    v8bf a[MI], b[3][MJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) a[i] = *reinterpret_cast<const v8bf*>(&wl[(BN / 2) * wr + 32 * i + r][kk + 8 * g]);
#pragma unroll
    for (int term = 0; term < 3; ++term)
#pragma unroll
      for (int j = 0; j < MJ; ++j)
        b[term][j] = *reinterpret_cast<const v8bf*>(&xl[term][(BT / 2) * wc + 32 * j + r][kk + 8 * g]);
#pragma unroll
    for (int term = 0; term < 3; ++term)
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[term][j], acc[i][j], 0, 0, 0);
  };
  // One chunk: its MFMAs from stage `cur`, the next chunk staged into `nxt` a
  // slice per k step (straight-line code, so the scheduler can interleave the
  // slice's VALU work with the MFMAs).
  auto chunk = [&](const unsigned short* cur, unsigned short* nxt, const v4i (&wv)[NW],
                   const v4f (&xv)[NX]) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      mfma_step(cur, s);
      stage(wv, xv, nxt, s);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Register set u holds chunks u, u + NS, ...: chunk j is loaded as soon as
  // chunk j - NS has been staged, so NS - 1 chunks of MFMAs hide its latency.
  // Chunks past the end re-load the last one (valid memory) and the final
  // chunk stages it into the idle stage: the loop stays free of branches.
  // The caller guarantees K % (NS * BK) == 0.
  unsigned short* st0 = gm_lds;
  unsigned short* st1 = gm_lds + STAGE;
  const int nch = K / BK;
  v4i wreg[NS][NW];
  v4f xreg[NS][NX];
#pragma unroll
  for (int u = 0; u < NS; ++u) load(wreg[u], xreg[u], min(u, nch - 1) * BK);
  stage(wreg[0], xreg[0], st0, -1);
  load(wreg[0], xreg[0], min(NS, nch - 1) * BK);
  lds_barrier();
  for (int c = 0; c < nch; c += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {  // chunk c + u from stage u % 2 (NS is even)
      chunk((u & 1) ? st1 : st0, (u & 1) ? st0 : st1, wreg[(u + 1) % NS], xreg[(u + 1) % NS]);
      load(wreg[(u + 1) % NS], xreg[(u + 1) % NS], min(c + u + 1 + NS, nch - 1) * BK);
      lds_barrier();
    }
  }

  gemm_tile_epilogue<BN, BT, EPI>(acc, ep, xp, xn, K, gm_lds, mat, y, scales, N, n0, t0, T, he);
}

// Producer/consumer form of the double-buffered kernel: 8 waves, the same
// tiles, stages and products in the same order per accumulator (so the same
// results bit for bit). Waves 0-3 hold the accumulators: each chunk they only
// read the staged operands and issue the MFMAs. Waves 4-7, the converters (one
// per SIMD beside an MFMA wave), load the chunks NS ahead into registers,
// convert them (int8 -> bf16, fp32 -> three bf16 terms) and write them to the
// stage the MFMA waves read next. The conversion's VALU work and the waits for
// the loads then sit on other waves than the products: the SIMD issues a
// converter's VALU instructions while its MFMA wave's products run, and an
// MFMA wave never waits on global memory. One barrier per chunk publishes the
// next stage and retires the reads of the stage the converters overwrite
// after it. The converters return after the loop's last barrier; the
// epilogue's barriers then count the 4 MFMA waves only.
template <int BN, int BT, int BK, int NS, int EPI>
__global__ __launch_bounds__(512) void w8a32_gemm_bf16x3_pc_kernel(GemmSet set, TileMap map,
                                                                   const float* __restrict__ x, int T, int K,
                                                                   GemmHeadEpi he, GemmXNorm xn) {
  constexpr int kGmRow = BK + 8;                   // LDS row in bf16 (16-byte pad)
  constexpr int STAGE = (BN + 3 * BT) * kGmRow;    // bf16 per LDS stage
  extern __shared__ __align__(16) unsigned short gm_lds[];  // 2 x ([BN][kGmRow] weights, [3][BT][kGmRow] terms)
  unsigned bx, by;
  tile_of(map, blockIdx.x, bx, by);
  float* y = set.y[0];
  const int8_t* w = set.w[0];
  const float* scales = set.s[0];
  const float* bias = set.b[0];
  int N = set.N[0];
  unsigned bx0 = 0;
  int mat = 0;
#pragma unroll
  for (int m = 1; m < 4; ++m)
    if (m < set.n && bx >= set.bx_begin[m]) {
      y = set.y[m];
      w = set.w[m];
      scales = set.s[m];
      bias = set.b[m];
      N = set.N[m];
      bx0 = set.bx_begin[m];
      mat = m;
    }
  constexpr int MI = BN / 64, MJ = BT / 64;
  static_assert(BN % 64 == 0 && BT % 64 == 0, "32 x 32 blocks per wave");
  constexpr int EP = EPI & 7;
  constexpr bool XN = (EPI & kGemmXNorm) != 0;
  constexpr int NW = BN / 64, NX = BT / 16;         // 16-byte staging items per converter thread
  constexpr int KSTEPS = BK / 16;                    // MFMA k steps per chunk
  static_assert(BK == 64 && NW >= 1 && NX >= 1, "the staging map of the double-buffered kernel");
  static_assert(NS >= 2 && NS % 2 == 0, "an even number of register sets");
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // uniform: scalar branches
  const int n0 = (int)(bx - bx0) * BN, t0 = (int)by * BT;
  const int nch = K / BK;
  unsigned short* st0 = gm_lds;
  unsigned short* st1 = gm_lds + STAGE;

  if (wave >= 4) {
    // Converter thread ct stages the items of thread ct of the 256-thread kernel.
    const int ct = (int)threadIdx.x - 256;
    const int w_part = ct & 3, x_part = ct & 15;
    const int8_t* wsrc[NW];
    const float* xsrc[NX];
    // rows and tokens past the end re-read the last one (valid memory; not stored)
#pragma unroll
    for (int c = 0; c < NW; ++c) wsrc[c] = w + (size_t)min(n0 + 64 * c + (ct >> 2), N - 1) * K + 16 * w_part;
#pragma unroll
    for (int c = 0; c < NX; ++c) xsrc[c] = x + (size_t)min(t0 + 16 * c + (ct >> 4), T - 1) * K + 4 * x_part;
    auto load = [&](v4i (&wv)[NW], v4f (&xv)[NX], int k0) {
#pragma unroll
      for (int c = 0; c < NW; ++c) wv[c] = *reinterpret_cast<const v4i*>(wsrc[c] + k0);
#pragma unroll
      for (int c = 0; c < NX; ++c) xv[c] = *reinterpret_cast<const v4f*>(xsrc[c] + k0);
    };
    auto stage = [&](const v4i (&wv)[NW], const v4f (&xv)[NX], unsigned short* st) {
      auto wl = reinterpret_cast<unsigned short (*)[kGmRow]>(st);
      auto xl = reinterpret_cast<unsigned short (*)[BT][kGmRow]>(st + BN * kGmRow);
#pragma unroll
      for (int c = 0; c < NW; ++c) {
        const v4i wc = wv[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // int8 -> bf16 is exact (at most 8 significant bits)
          const int v = wc[e];
          const uint2 h = make_uint2(bf16_pair((float)(int8_t)(v & 0xff), (float)(int8_t)((v >> 8) & 0xff)),
                                     bf16_pair((float)(int8_t)((v >> 16) & 0xff), (float)(int8_t)((v >> 24) & 0xff)));
          *reinterpret_cast<uint2*>(&wl[64 * c + (ct >> 2)][16 * w_part + 4 * e]) = h;
        }
      }
#pragma unroll
      for (int c = 0; c < NX; ++c) {  // x = hi + mid + lo exactly
        const v4f xc = xv[c];
        const float ev[4] = {xc.x, xc.y, xc.z, xc.w};
        float r1[4], r2[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r1[e] = ev[e] - bf16_trunc(ev[e]);
          r2[e] = r1[e] - bf16_trunc(r1[e]);  // at most 8 significant bits
        }
        const int tok = 16 * c + (ct >> 4), col = 4 * x_part;
        *reinterpret_cast<uint2*>(&xl[0][tok][col]) = make_uint2(bf16_pair(ev[0], ev[1]), bf16_pair(ev[2], ev[3]));
        *reinterpret_cast<uint2*>(&xl[1][tok][col]) = make_uint2(bf16_pair(r1[0], r1[1]), bf16_pair(r1[2], r1[3]));
        *reinterpret_cast<uint2*>(&xl[2][tok][col]) = make_uint2(bf16_pair(r2[0], r2[1]), bf16_pair(r2[2], r2[3]));
      }
    };
    // Register set u holds chunks u, u + NS, ...: chunk j is loaded as soon as
    // chunk j - NS has been staged, NS - 1 chunks of products ahead of its use.
    // Chunks past the end re-load the last one (valid memory) and the final
    // pass stages it into the idle stage: the loop stays free of branches.
    // The caller guarantees K % (NS * BK) == 0.
    v4i wreg[NS][NW];
    v4f xreg[NS][NX];
#pragma unroll
    for (int u = 0; u < NS; ++u) load(wreg[u], xreg[u], min(u, nch - 1) * BK);
    stage(wreg[0], xreg[0], st0);
    load(wreg[0], xreg[0], min(NS, nch - 1) * BK);
    lds_barrier();
    for (int c = 0; c < nch; c += NS) {
#pragma unroll
      for (int u = 0; u < NS; ++u) {  // while chunk c + u is multiplied from stage u % 2, stage chunk c + u + 1
        stage(wreg[(u + 1) % NS], xreg[(u + 1) % NS], (u & 1) ? st0 : st1);
        load(wreg[(u + 1) % NS], xreg[(u + 1) % NS], min(c + u + 1 + NS, nch - 1) * BK);
        lds_barrier();
      }
    }
    return;
  }

  const int lane = threadIdx.x & 63;
  const int wr = wave & 1, wc = wave >> 1;
  const int r = lane & 31, g = lane >> 5;
  v16f acc[MI][MJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[i][j] = v16f{};
  [[maybe_unused]] GemmEpiRows<MI, EP == kGemmBias> ep;
  if constexpr (EP != kGemmHeads) ep.load(scales, bias, N, n0 + (BN / 2) * wr, lane);
  [[maybe_unused]] float xp[MJ][kXnMaxSlices];  // XN: the partial sums of squares of the lane's epilogue tokens
  if constexpr (XN) {
#pragma unroll
    for (int j = 0; j < MJ; ++j) xnorm_load(xp[j], xn, min(t0 + (BT / 2) * wc + 32 * j + r, T - 1));
  }
  // The operand fragments of k step s of the chunk staged in `st`, and the
  // step's products in the order of the single-buffered kernel (term, then
  // row block, then token block). The fragments of step s + 1 are read before
  // the products of step s issue (two register sets), so each step's products
  // wait only for their own fragments.
  auto read_step = [&](const unsigned short* st, int s, v8bf (&a)[MI], v8bf (&b)[3][MJ]) {
    auto wl = reinterpret_cast<const unsigned short (*)[kGmRow]>(st);
    auto xl = reinterpret_cast<const unsigned short (*)[BT][kGmRow]>(st + BN * kGmRow);
    const int kk = 16 * s;
#pragma unroll
    for (int i = 0; i < MI; ++i) a[i] = *reinterpret_cast<const v8bf*>(&wl[(BN / 2) * wr + 32 * i + r][kk + 8 * g]);
#pragma unroll
    for (int term = 0; term < 3; ++term)
#pragma unroll
      for (int j = 0; j < MJ; ++j)
        b[term][j] = *reinterpret_cast<const v8bf*>(&xl[term][(BT / 2) * wc + 32 * j + r][kk + 8 * g]);
  };
  auto mfma_step = [&](const v8bf (&a)[MI], const v8bf (&b)[3][MJ]) {
#pragma unroll
    for (int term = 0; term < 3; ++term)
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[term][j], acc[i][j], 0, 0, 0);
  };
  auto chunk = [&](const unsigned short* st) {
    v8bf a[2][MI], b[2][3][MJ];
    read_step(st, 0, a[0], b[0]);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      if (s + 1 < KSTEPS) read_step(st, s + 1, a[(s + 1) & 1], b[(s + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      mfma_step(a[s & 1], b[s & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  lds_barrier();  // chunk 0 staged
  for (int c = 0; c < nch; c += 2) {  // nch is even (a multiple of NS)
    chunk(st0);
    lds_barrier();
    chunk(st1);
    lds_barrier();
  }
  gemm_tile_epilogue<BN, BT, EPI>(acc, ep, xp, xn, K, gm_lds, mat, y, scales, N, n0, t0, T, he);
}

// Column split of the XCD map that minimises the bytes one XCD reads
// (cols/a weight blocks of BN x K int8 + rows/(8/a) token blocks of BT x K fp32);
// 0 when no split divides the tile grid evenly.
inline unsigned xcd_split_cols(unsigned cols, unsigned rows, int BN, int BT) {
  unsigned best = 0;
  double best_cost = 0;
  for (unsigned a = 1; a <= 8; a *= 2) {
    const unsigned b = 8 / a;
    if (cols % a || rows % b) continue;
    const double cost = (double)(cols / a) * BN + (double)(rows / b) * BT * 4;
    if (best == 0 || cost < best_cost) {
      best = a;
      best_cost = cost;
    }
  }
  return best;
}

// Split-K variant: the KW waves of a workgroup share one BN x BT output tile
// and take interleaved 64-wide K steps (wave w: steps w, w + KW, ...). Each
// wave loads its weight and activation fragments straight into registers in
// the operand layout of v_mfma_f32_32x32x16_bf16 (A[i][k] in lane i + 32(k/8),
// element k%8; B alike), so the main loop has no LDS traffic and no barriers;
// each weight and activation element is converted once per workgroup. Within
// a 32-wide K chunk, lane group g (lanes 32g..32g+31) covers k = 16g..16g+15:
// the first 8 feed MFMA slots 8g..8g+7 of one 16-slot product and the next 8
// those of the other (the same permutation of k for both operands, so the dot
// product is unchanged). With a single 32 x 32 block per wave each bf16 term
// gets its own accumulator (three independent chains for the matrix pipe),
// added hi + mid + lo at the end. The KW partial tiles are added in LDS in
// wave order.
QASR_DEV unsigned bf16_pair_i8(int v, int byte) {  // bytes byte, byte + 1 of v as two bf16
  return bf16_pair((float)(int8_t)((v >> (8 * byte)) & 0xff), (float)(int8_t)((v >> (8 * byte + 8)) & 0xff));
}

template <int MI, int MJ>
struct KsplitRaw {
  v4i w[MI][2];          // per 32-wide chunk: 16 int8 of one weight row
  v4f x[MJ][8];          // load q: floats 4(lane % 16).. of token 4q + lane / 16 (coalesced)
};
// Row pitch (floats) of a wave's staged activation block [32 tokens][64 k]:
// the 16-byte pad spreads the fragment reads of 32 rows over the banks.
constexpr int kKsPitch = 68;

// Lane l, register 4q + v of block (i, j) holds row n0 + 32i + 8q + 4(l/32) + v
// of token t0 + 32j + l%32; the KW waves' partial tiles are added in LDS in
// wave order (deterministic), the blocks split over the waves; epilogue
// y = sum * scale (+ bias), or (kGemmResidual) y += sum * scale with each
// token's sum of squares of its updated 64 rows written to ss[t][n0 / 64]
// (per lane in item order, then the two lanes of a token, then the waves in
// order through LDS) and, with hg, hg = the updated y * gain[n].
template <int MI, int MJ, int KW, int EPI>
QASR_DEV void ksplit_reduce_store(const v16f (&acc)[MI][MJ], float* red, int wave, int lane, float* y,
                                  const float* scales, const float* bias, int N, int T, int n0, int t0,
                                  float* ss, float* hg, const float* gain) {
  const int r = lane & 31, g = lane >> 5;
  constexpr int PER_WAVE = MI * MJ * 16 * 64;  // floats
  // Wave w reduces and stores the (block, register quad) items w, w + KW, ...
  // Their row scales (and biases) are loaded before the partial tiles go
  // through LDS, so that exchange hides their latency.
  constexpr int ITEMS = (MI * MJ * 4 + KW - 1) / KW;
  float es[ITEMS][4], eb[ITEMS][4];
  [[maybe_unused]] float hv[ITEMS][4], gv[ITEMS][4];  // kGemmResidual: the rows to add to, the gains
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int p = min(wave + KW * it, MI * MJ * 4 - 1);
    const int n = n0 + 32 * ((p >> 2) / MJ) + 8 * (p & 3) + 4 * g;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int nv = min(n + v, N - 1);
      es[it][v] = scales[nv];
      eb[it][v] = EPI == kGemmBias ? bias[nv] : 0.0f;
    }
    if constexpr (EPI == kGemmResidual) {
      const int t = min(t0 + 32 * ((p >> 2) % MJ) + r, T - 1);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        hv[it][v] = y[(size_t)t * N + min(n + v, N - 1)];
        gv[it][v] = hg ? gain[min(n + v, N - 1)] : 0.0f;
      }
    }
  }
  float* mine = red + (size_t)wave * PER_WAVE;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) mine[((i * MJ + j) * 16 + e) * 64 + lane] = acc[i][j][e];
  __syncthreads();
  const bool vec_out = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  static_assert(EPI != kGemmResidual || (KW == 4 && MI == 2), "residual slices: 64 rows, item it = block it");
  [[maybe_unused]] float sq[MJ];
#pragma unroll
  for (int j = 0; j < MJ; ++j) sq[j] = 0.0f;
#pragma unroll
  for (int it = 0; it < ITEMS; ++it) {
    const int p = wave + KW * it;
    if (p < MI * MJ * 4) {
      const int blk = p >> 2, q = p & 3;
      const int i = blk / MJ, j = blk % MJ;
      const int t = t0 + 32 * j + r;
      const int n = n0 + 32 * i + 8 * q + 4 * g;
      float res[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int e = (blk * 16 + 4 * q + v) * 64 + lane;
        float sum = red[e];
#pragma unroll
        for (int ww = 1; ww < KW; ++ww) sum += red[(size_t)ww * PER_WAVE + e];
        res[v] = sum * es[it][v];
        if constexpr (EPI == kGemmBias) res[v] += eb[it][v];
      }
      if constexpr (EPI == kGemmResidual) {
        // h + y in the residual add's order (decoder.rs:829, 843)
        float hn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (t < T) {
          float* hp = &y[(size_t)t * N + n];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < N) hn[v] = hv[it][v] + res[v];
          if (vec_out && n + 3 < N) {
            *reinterpret_cast<float4*>(hp) = make_float4(hn[0], hn[1], hn[2], hn[3]);
            if (hg)
              *reinterpret_cast<float4*>(&hg[(size_t)t * N + n]) =
                  make_float4(hn[0] * gv[it][0], hn[1] * gv[it][1], hn[2] * gv[it][2], hn[3] * gv[it][3]);
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (n + v < N) {
                hp[v] = hn[v];
                if (hg) hg[(size_t)t * N + n + v] = hn[v] * gv[it][v];
              }
          }
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) sq[it % MJ] += hn[v] * hn[v];
      } else if (t < T) {
        if constexpr (EPI == kGemmSwiglu || EPI == kGemmSwigluLibm) {
          swiglu_store<EPI>(y, res, t, n, N);
        } else if (vec_out && n + 3 < N) {
          *reinterpret_cast<float4*>(&y[(size_t)t * N + n]) = make_float4(res[0], res[1], res[2], res[3]);
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (n + v < N) y[(size_t)t * N + n + v] = res[v];
        }
      }
    }
  }
  if constexpr (EPI == kGemmResidual) {
    __shared__ float ssl[KW][MJ][32];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
      const float both = sq[j] + __shfl_xor(sq[j], 32, kWave);  // rows 4g..4g+3 of each quad: g = 0, 1
      if (g == 0) ssl[wave][j][r] = both;
    }
    __syncthreads();
    if (wave == 0 && g == 0) {
      const int slices = (N + 63) / 64;
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        float sum = ssl[0][j][r];
#pragma unroll
        for (int ww = 1; ww < KW; ++ww) sum += ssl[ww][j][r];
        const int t = t0 + 32 * j + r;
        if (t < T) ss[(size_t)t * slices + n0 / 64] = sum;
      }
    }
  }
}

template <int BN, int BT, int KW, int EPI>
__global__ __launch_bounds__(64 * KW) void w8a32_gemm_ksplit_kernel(GemmSet set, TileMap map,
                                                                    const float* __restrict__ x, int T, int K) {
  constexpr int MI = BN / 32, MJ = BT / 32;
  constexpr int NT = MI * MJ == 1 ? 3 : 1;  // accumulators per block: one per term for a single block
  static_assert(BN % 32 == 0 && BT % 32 == 0, "32 x 32 blocks");
  // [KW][MI * MJ * 16][64] partial tiles after the loop; during it each
  // wave's staged activations, [KW][MJ][32][kKsPitch]
  extern __shared__ __align__(16) float gk_red[];
  unsigned bx, by;
  tile_of(map, blockIdx.x, bx, by);
  float* y = set.y[0];
  const int8_t* w = set.w[0];
  const float* scales = set.s[0];
  const float* bias = set.b[0];
  int N = set.N[0];
  unsigned bx0 = 0;
#pragma unroll
  for (int m = 1; m < 4; ++m)
    if (m < set.n && bx >= set.bx_begin[m]) {
      y = set.y[m];
      w = set.w[m];
      scales = set.s[m];
      bias = set.b[m];
      N = set.N[m];
      bx0 = set.bx_begin[m];
    }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches
  const int r = lane & 31, g = lane >> 5;
  const int n0 = (int)(bx - bx0) * BN, t0 = (int)by * BT;
  // rows and tokens past the end re-read the last one (valid memory; not stored)
  const int8_t* wp[MI];
  const float* xp[MJ][8];
#pragma unroll
  for (int i = 0; i < MI; ++i) wp[i] = w + (size_t)min(n0 + 32 * i + r, N - 1) * K + 16 * g;
#pragma unroll
  for (int j = 0; j < MJ; ++j)
#pragma unroll
    for (int q = 0; q < 8; ++q)
      xp[j][q] = x + (size_t)min(t0 + 32 * j + 4 * q + (lane >> 4), T - 1) * K + 4 * (lane & 15);
  float* xs = gk_red + (size_t)wave * MJ * 32 * kKsPitch;  // this wave's staged activations

  v16f acc[NT][MI][MJ];
#pragma unroll
  for (int u = 0; u < NT; ++u)
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j) acc[u][i][j] = v16f{};

  auto load = [&](KsplitRaw<MI, MJ>& raw, int step) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int k = step * 64 + 32 * c;
#pragma unroll
      for (int i = 0; i < MI; ++i) raw.w[i][c] = *reinterpret_cast<const v4i*>(wp[i] + k);
    }
    // the activations as 1 KiB contiguous pieces (four tokens' 64 k each):
    // lanes one 128-byte line apart cost the load path 8x the line lookups
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) raw.x[j][q] = *reinterpret_cast<const v4f*>(xp[j][q] + step * 64);
  };
  // Every loaded register passes through an empty asm first, so no part of
  // the conversion is hoisted next to its load (which would wait for the load
  // there instead of one step later).
  // The activations go through the wave's LDS block into the MFMA layout:
  // lane (r, g) takes floats 32c + 16g .. +15 of token r (only this wave
  // touches the block, and its LDS accesses complete in order).
  auto compute = [&](const KsplitRaw<MI, MJ>& in) {
    KsplitRaw<MI, MJ> raw = in;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int i = 0; i < MI; ++i) asm volatile("" : "+v"(raw.w[i][c]));
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        asm volatile("" : "+v"(raw.x[j][q]));
        *reinterpret_cast<v4f*>(xs + (j * 32 + 4 * q + (lane >> 4)) * kKsPitch + 4 * (lane & 15)) = raw.x[j][q];
      }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
    v4f xf[MJ][2][4];
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int f = 0; f < 4; ++f)
          xf[j][c][f] = *reinterpret_cast<const v4f*>(xs + (j * 32 + r) * kKsPitch + 32 * c + 16 * g + 4 * f);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // k = 32c + 16g + 8h + (0..7): MFMA slots 8g..8g+7
        // weights: int8 -> bf16 is exact (at most 8 significant bits)
        v4u a[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const int v0 = raw.w[i][c][2 * h], v1 = raw.w[i][c][2 * h + 1];
          a[i] = v4u{bf16_pair_i8(v0, 0), bf16_pair_i8(v0, 2), bf16_pair_i8(v1, 0), bf16_pair_i8(v1, 2)};
        }
        // activations: x = hi + mid + lo exactly (three truncated bf16 terms)
        v4u b[3][MJ];
#pragma unroll
        for (int j = 0; j < MJ; ++j)
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            const v4f xv = xf[j][c][2 * h + f];
            const float e[4] = {xv.x, xv.y, xv.z, xv.w};
            float r1[4], r2[4];
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
              r1[qq] = e[qq] - bf16_trunc(e[qq]);
              r2[qq] = r1[qq] - bf16_trunc(r1[qq]);  // at most 8 significant bits
            }
            b[0][j][2 * f] = bf16_pair(e[0], e[1]);
            b[0][j][2 * f + 1] = bf16_pair(e[2], e[3]);
            b[1][j][2 * f] = bf16_pair(r1[0], r1[1]);
            b[1][j][2 * f + 1] = bf16_pair(r1[2], r1[3]);
            b[2][j][2 * f] = bf16_pair(r2[0], r2[1]);
            b[2][j][2 * f + 1] = bf16_pair(r2[2], r2[3]);
          }
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
          for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < MJ; ++j) {
              v16f& d = acc[NT == 3 ? term : 0][i][j];
              d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[i]),
                                                          __builtin_bit_cast(v8bf, b[term][j]), d, 0, 0, 0);
            }
      }
  };

  // Wave `wave` takes steps wave, wave + KW, ... (n_mine of them). Two
  // register sets in turn: step n + 1's loads are in flight while step n is
  // converted and multiplied. The loads are unconditional (indices past the
  // wave's last step re-load it), so the loop body is branch-free and the
  // compiler's waits stay exact.
  const int steps = K / 64;
  const int n_mine = wave < steps ? (steps - wave + KW - 1) / KW : 0;  // wave-uniform
  auto step_of = [&](int n) { return wave + KW * min(n, n_mine - 1); };
  if (n_mine > 0) {
    KsplitRaw<MI, MJ> ra, rb;
    load(ra, step_of(0));
    load(rb, step_of(1));
    for (int n = 0; n + 2 <= n_mine; n += 2) {
      compute(ra);
      load(ra, step_of(n + 2));
      compute(rb);
      load(rb, step_of(n + 3));
    }
    if (n_mine & 1) compute(ra);
  }
  if constexpr (NT == 3) {
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[0][0][0][e] = (acc[0][0][0][e] + acc[1][0][0][e]) + acc[2][0][0][e];
  }
  __syncthreads();  // every wave's staged activations read: the partial tiles reuse the LDS
  ksplit_reduce_store<MI, MJ, KW, EPI>(acc[0], gk_red, wave, lane, y, scales, bias, N, T, n0, t0, set.ss, set.hg,
                                       set.gain);
}

template <int BN, int BT, int KW, int EPI>
bool try_gemm_ksplit(const GemmSet& set, unsigned cols, const float* x, int T, int K, hipStream_t st) {
  constexpr size_t red = (size_t)KW * BN * BT * sizeof(float);                 // partial tiles
  constexpr size_t stage = (size_t)KW * (BT / 32) * 32 * kKsPitch * sizeof(float);  // staged activations
  constexpr size_t lds = red > stage ? red : stage;
  if (K % 64 != 0) return false;
  if (lds > 65536 && !raise_lds_limit<&w8a32_gemm_ksplit_kernel<BN, BT, KW, EPI>>(lds)) return false;
  TileMap map;
  map.cols = cols;
  map.rows = (unsigned)((T + BT - 1) / BT);
  map.split_cols = xcd_split_cols(map.cols, map.rows, BN, BT);
  w8a32_gemm_ksplit_kernel<BN, BT, KW, EPI><<<map.cols * map.rows, 64 * KW, lds, st>>>(set, map, x, T, K);
  return true;
}

template <int BN, int BT, int BK, int NPF, int EPI>
bool try_gemm(const GemmSet& set, unsigned cols, const float* x, int T, int K, hipStream_t st,
              const GemmHeadEpi& he = GemmHeadEpi{}, const GemmXNorm& xn = GemmXNorm{}) {
  constexpr size_t lds = gemm_lds_bytes<BN, BT, BK>();
  if (K % BK != 0) return false;
  if (lds > 65536 && !raise_lds_limit<&w8a32_gemm_bf16x3_kernel<BN, BT, BK, NPF, EPI>>(lds)) return false;
  TileMap map;
  map.cols = cols;
  map.rows = (unsigned)((T + BT - 1) / BT);
  map.split_cols = xcd_split_cols(map.cols, map.rows, BN, BT);
  w8a32_gemm_bf16x3_kernel<BN, BT, BK, NPF, EPI><<<map.cols * map.rows, 256, lds, st>>>(set, map, x, T, K, he, xn);
  return true;
}

template <int BN, int BT, int BK, int NS, int EPI>
bool try_gemm_db(const GemmSet& set, unsigned cols, const float* x, int T, int K, hipStream_t st,
                 const GemmHeadEpi& he = GemmHeadEpi{}, const GemmXNorm& xn = GemmXNorm{}) {
  constexpr size_t lds = 2 * gemm_lds_bytes<BN, BT, BK>();
  if (K % (NS * BK) != 0) return false;
  if (lds > 65536 && !raise_lds_limit<&w8a32_gemm_bf16x3_db_kernel<BN, BT, BK, NS, EPI>>(lds)) return false;
  TileMap map;
  map.cols = cols;
  map.rows = (unsigned)((T + BT - 1) / BT);
  map.split_cols = xcd_split_cols(map.cols, map.rows, BN, BT);
  w8a32_gemm_bf16x3_db_kernel<BN, BT, BK, NS, EPI><<<map.cols * map.rows, 256, lds, st>>>(set, map, x, T, K, he,
                                                                                         xn);
  return true;
}

template <int BN, int BT, int BK, int NS, int EPI>
bool try_gemm_pc(const GemmSet& set, unsigned cols, const float* x, int T, int K, hipStream_t st,
                 const GemmHeadEpi& he = GemmHeadEpi{}, const GemmXNorm& xn = GemmXNorm{}) {
  constexpr size_t lds = 2 * gemm_lds_bytes<BN, BT, BK>();
  if (K % (NS * BK) != 0) return false;
  if (lds > 65536 && !raise_lds_limit<&w8a32_gemm_bf16x3_pc_kernel<BN, BT, BK, NS, EPI>>(lds)) return false;
  TileMap map;
  map.cols = cols;
  map.rows = (unsigned)((T + BT - 1) / BT);
  map.split_cols = xcd_split_cols(map.cols, map.rows, BN, BT);
  w8a32_gemm_bf16x3_pc_kernel<BN, BT, BK, NS, EPI><<<map.cols * map.rows, 512, lds, st>>>(set, map, x, T, K, he,
                                                                                         xn);
  return true;
}

// Kernel and tile: the LDS-staged 256 x 64 tile where it still gives at least
// 512 workgroups (a 256-stream lm_head: each workgroup's activation rows then
// serve twice the weight rows, 634.7 -> 579.9 us at [256,2048]x[2048,151936];
// 256 x 128 measured slower, one workgroup per CU), the 128 x 64 tile where it
// gives at least 256 (its staged operands are shared by 4 waves: 128 B loaded
// per MFMA) -- double-buffered when that is one workgroup per CU (T = 512
// q/k/v: 25.7 -> 24.9 us at K = 1024, 40.4 -> 37.4 us at K = 2048); with more
// workgroups the single-buffered kernel is faster (two or three share a CU and
// overlap each other's staging and MFMAs; the double-buffered one's LDS allows
// only one: 0.6B gate/up at T = 512 33.5 against 42-45 us), except where the
// 128-row tiles would give some CUs two workgroups and others one while
// 192-row tiles give at most one per CU: those run double-buffered (0.6B
// gate/up at T = 512: 384 tiles of 128 rows 29.3 us, 256 of 192 27.3 us).
// Where the double-buffered kernel would run, its producer/consumer form runs
// instead when K is a multiple of 4 chunks (0.6B at T = 512, one box, cold
// inputs: q/k/v 24.7 -> 21.8 us, gate/up 29.6 -> 26.8 us; the prefill step
// 3004 -> 2861 us); otherwise the split-K kernel with the largest of 64 x 64, 64 x 32 and
// 32 x 32 that fills the chip (measured at T = 512: o [1024, 2048] 20.0 ->
// 16.7 us, down [1024, 3072] 27.4 -> 20.9 us against the LDS-staged 64 x 32).
// Returns false when the chosen kernel cannot run the shape (K not a multiple
// of its K step, or its LDS size refused), or when it is the split-K kernel
// and the epilogue asks for the folded RMSNorm (kGemmXNorm, which only the
// LDS-staged kernels stage): nothing was launched.
template <int EPI>
bool launch_w8a32_gemm(GemmSet set, const float* x, int T, int K, hipStream_t st,
                       const GemmXNorm& xn = GemmXNorm{}) {
  auto cols = [&](int bn) {
    unsigned c = 0;
    for (int m = 0; m < set.n; ++m) {
      set.bx_begin[m] = c;
      c += (unsigned)((set.N[m] + bn - 1) / bn);
    }
    for (int m = set.n; m <= 4; ++m) set.bx_begin[m] = c;
    return c;
  };
  const long long rows64 = (T + 63) / 64, rows32 = (T + 31) / 32;
  const GemmHeadEpi he{};
  unsigned c = cols(256);
  if (c * rows64 >= 512) return try_gemm<256, 64, 64, kGemmPrefetch, EPI>(set, c, x, T, K, st, he, xn);
  const unsigned c128 = cols(128);
  c = cols(192);
  if (c128 * rows64 > 256 && c * rows64 <= 256 &&
      (try_gemm_pc<192, 64, 64, kGemmPcSets, EPI>(set, c, x, T, K, st, he, xn) ||
       try_gemm_db<192, 64, 64, kGemmSets, EPI>(set, c, x, T, K, st, he, xn)))
    return true;
  c = cols(128);
  if (c * rows64 >= 256) {
    if (c * rows64 <= 256 && (try_gemm_pc<128, 64, 64, kGemmPcSets, EPI>(set, c, x, T, K, st, he, xn) ||
                              try_gemm_db<128, 64, 64, kGemmSets, EPI>(set, c, x, T, K, st, he, xn)))
      return true;
    return try_gemm<128, 64, 64, kGemmPrefetch, EPI>(set, c, x, T, K, st, he, xn);
  }
  if constexpr ((EPI & kGemmXNorm) != 0) {
    return false;
  } else {
    c = cols(64);
    if (c * rows64 >= 256) return try_gemm_ksplit<64, 64, 4, EPI>(set, c, x, T, K, st);
    if (c * rows32 >= 256) return try_gemm_ksplit<64, 32, 4, EPI>(set, c, x, T, K, st);
    return try_gemm_ksplit<32, 32, 4, EPI>(set, cols(32), x, T, K, st);
  }
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_quantize_rows_i8(int8_t* q, float* scales, const float* x, size_t rows,
                                     size_t cols, void* stream) {
  if (rows == 0) return QASR_OK;
  QASR_REQUIRE(q && scales && x, "quantize_rows_i8: null pointer");
  QASR_REQUIRE(rows <= kMaxRows && cols <= 0x7fffffffu, "quantize_rows_i8: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(rows, cols, &n), "quantize_rows_i8: rows * cols overflows");
  hipStream_t st = as_stream(stream);
  const int c = (int)cols;
  if (cols % 4 == 0 && cols / 4 <= 8 * 256 && aligned16(x) && aligned4(q)) {
    const size_t c4 = cols / 4;
    if (c4 <= 256) quantize_rows_vec_kernel<1><<<(unsigned)rows, 256, 0, st>>>(q, scales, x, c);
    else if (c4 <= 512) quantize_rows_vec_kernel<2><<<(unsigned)rows, 256, 0, st>>>(q, scales, x, c);
    else if (c4 <= 1024) quantize_rows_vec_kernel<4><<<(unsigned)rows, 256, 0, st>>>(q, scales, x, c);
    else quantize_rows_vec_kernel<8><<<(unsigned)rows, 256, 0, st>>>(q, scales, x, c);
  } else {
    quantize_rows_kernel<<<(unsigned)rows, 256, 0, st>>>(q, scales, x, c);
  }
  return launch_status("quantize_rows_i8");
}

// From this many tokens the linear runs as one matrix-core GEMM instead of
// per-token matvecs.
constexpr size_t kGemmMinTokens = 8;

// The q/k/v GEMM with the heads epilogue: 128-row tiles (one head), the
// producer/consumer (else double-buffered) kernel where that is one workgroup
// per CU, as for the plain projection.
static bool launch_w8a32_heads(GemmSet set, const float* x, int T, int K, const GemmHeadEpi& he,
                               hipStream_t st, const GemmXNorm& xn = GemmXNorm{}) {
  unsigned c = 0;
  for (int m = 0; m < set.n; ++m) {
    set.bx_begin[m] = c;
    c += (unsigned)(set.N[m] / 128);
  }
  for (int m = set.n; m <= 4; ++m) set.bx_begin[m] = c;
  const long long rows64 = (T + 63) / 64;
  constexpr int kFold = kGemmHeads | kGemmXNorm;
  if (xn.ss) {
    if (c * rows64 <= 256 && (try_gemm_pc<128, 64, 64, kGemmPcSets, kFold>(set, c, x, T, K, st, he, xn) ||
                              try_gemm_db<128, 64, 64, kGemmSets, kFold>(set, c, x, T, K, st, he, xn)))
      return true;
    return try_gemm<128, 64, 64, kGemmPrefetch, kFold>(set, c, x, T, K, st, he, xn);
  }
  if (c * rows64 <= 256 && (try_gemm_pc<128, 64, 64, kGemmPcSets, kGemmHeads>(set, c, x, T, K, st, he) ||
                            try_gemm_db<128, 64, 64, kGemmSets, kGemmHeads>(set, c, x, T, K, st, he)))
    return true;
  return try_gemm<128, 64, 64, kGemmPrefetch, kGemmHeads>(set, c, x, T, K, st, he);
}

static bool w8a32_gemm_shape(size_t seq_len, size_t in_dim, const void* w, const void* x) {
  return seq_len >= kGemmMinTokens && in_dim % kGmBK == 0 && aligned16(w) && aligned16(x);
}

static int launch_w8a32(float* y, const float* x, const int8_t* w, const float* scales,
                        const float* bias, size_t seq_len, size_t in_dim, size_t out_dim,
                        void* stream) {
  if (seq_len == 0 || out_dim == 0) return QASR_OK;
  QASR_REQUIRE(y && x && w && scales, "linear_int8: null pointer");
  QASR_REQUIRE(seq_len <= 0x7fffffffu && in_dim <= 0x7fffffffu && out_dim <= 0x7fffffffu,
               "linear_int8: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(in_dim, out_dim, &n) && mul_ok(seq_len, in_dim, &n) &&
                   mul_ok(seq_len, out_dim, &n),
               "linear_int8: size overflows");
  hipStream_t st = as_stream(stream);
  const unsigned grid = (unsigned)((out_dim + 3) / 4);
  const int s = (int)seq_len, k = (int)in_dim, o = (int)out_dim;
  const bool vec = w8a32_rows_shape(in_dim, w, x);
  if (vec && seq_len == 1) {
    const int r = rows_per_wave(in_dim, out_dim);
    launch_rows<kEpiRows>((int)(in_dim / 1024), r, (unsigned)((out_dim + 4 * r - 1) / (4 * r)), st,
                          y, x, w, scales, bias, k, o, nullptr);
  } else if (w8a32_gemm_shape(seq_len, in_dim, w, x)) {
    GemmSet set{};
    set.y[0] = y;
    set.w[0] = w;
    set.s[0] = scales;
    set.b[0] = bias;
    set.N[0] = o;
    set.n = 1;
    const bool ran = bias ? launch_w8a32_gemm<kGemmBias>(set, x, s, k, st)
                          : launch_w8a32_gemm<kGemmRows>(set, x, s, k, st);
    if (!ran) return fail(QASR_ERR_UNSUPPORTED, "linear_int8: the GEMM kernel cannot run this shape");
  } else if (vec) {
    switch (in_dim / 1024) {
      case 1: w8a32_vec_kernel<1><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      case 2: w8a32_vec_kernel<2><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      case 3: w8a32_vec_kernel<3><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      case 4: w8a32_vec_kernel<4><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      case 5: w8a32_vec_kernel<5><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      case 6: w8a32_vec_kernel<6><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      case 7: w8a32_vec_kernel<7><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
      default: w8a32_vec_kernel<8><<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o); break;
    }
  } else {
    w8a32_scalar_kernel<<<grid, 256, 0, st>>>(y, x, w, scales, bias, s, k, o);
  }
  return launch_status("linear_int8");
}

namespace qasr {
bool launch_w8a32_argmax_partials(float* y, const float* x, const int8_t* w, const float* scales,
                                  size_t in_dim, size_t out_dim, float2* part, size_t part_cap,
                                  hipStream_t st, unsigned* n_part) {
  if (!w8a32_rows_shape(in_dim, w, x)) return false;
  if (out_dim == 0 || out_dim > 0x7fffffffu - 64) return false;
  const int r = rows_per_wave(in_dim, out_dim);
  const size_t grid = (out_dim + 4 * r - 1) / (4 * r);
  if (grid > part_cap) return false;
  launch_rows<kEpiArgmax>((int)(in_dim / 1024), r, (unsigned)grid, st, y, x, w, scales, nullptr,
                         (int)in_dim, (int)out_dim, part);
  *n_part = (unsigned)grid;
  return true;
}
}  // namespace qasr

extern "C" int qasr_linear_nobias_int8_f32(float* y, const float* x, const int8_t* w,
                                           const float* scales, size_t seq_len, size_t in_dim,
                                           size_t out_dim, void* stream) {
  return launch_w8a32(y, x, w, scales, nullptr, seq_len, in_dim, out_dim, stream);
}

extern "C" int qasr_gate_up_swiglu_int8_f32(float* out, const float* x, const int8_t* w_gate_up,
                                            const float* scales_gate_up, size_t seq_len,
                                            size_t in_dim, size_t intermediate, void* stream) {
  if (seq_len == 0 || intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && x && w_gate_up && scales_gate_up, "gate_up_swiglu_int8: null pointer");
  QASR_REQUIRE(in_dim > 0 && in_dim <= 0x7fffffffu && seq_len <= 0x7fffffffu &&
                   intermediate <= 0x3fffffffu - 64,
               "gate_up_swiglu_int8: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(2 * intermediate, in_dim, &n) && mul_ok(seq_len, in_dim, &n) &&
                   mul_ok(seq_len, intermediate, &n) && n < ((size_t)1 << 33),
               "gate_up_swiglu_int8: size overflows");
  hipStream_t st = as_stream(stream);
  const size_t rows = 2 * intermediate;
  if (seq_len == 1 && w8a32_rows_shape(in_dim, w_gate_up, x)) {
    const int r = rows_per_wave(in_dim, rows) < 2 ? 2 : rows_per_wave(in_dim, rows);
    launch_rows<kEpiSwiglu>((int)(in_dim / 1024), r, (unsigned)((rows + 4 * r - 1) / (4 * r)), st,
                            out, x, w_gate_up, scales_gate_up, nullptr, (int)in_dim, (int)rows,
                            nullptr);
  } else if (w8a32_gemm_shape(seq_len, in_dim, w_gate_up, x)) {
    // several decode streams: the matrix-core GEMM with the loop's SwiGLU in its epilogue
    GemmSet set{};
    set.y[0] = out;
    set.w[0] = w_gate_up;
    set.s[0] = scales_gate_up;
    set.b[0] = nullptr;
    set.N[0] = (int)rows;
    set.n = 1;
    if (!launch_w8a32_gemm<kGemmSwigluLibm>(set, x, (int)seq_len, (int)in_dim, st))
      return fail(QASR_ERR_UNSUPPORTED, "gate_up_swiglu_int8: the GEMM kernel cannot run this shape");
  } else {
    const long long items = (long long)seq_len * (long long)intermediate;
    gate_up_swiglu_w8a32_pairs_kernel<false><<<(unsigned)((items + 3) / 4), 256, 0, st>>>(
        out, x, w_gate_up, scales_gate_up, (int)seq_len, (int)in_dim, (int)intermediate);
  }
  return launch_status("gate_up_swiglu_int8");
}

extern "C" int qasr_gate_up_swiglu_multiply_int8_f32(float* out, const float* x, const int8_t* w_gate_up,
                                                     const float* scales_gate_up, size_t seq_len,
                                                     size_t in_dim, size_t intermediate, void* stream) {
  if (seq_len == 0 || intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && x && w_gate_up && scales_gate_up, "gate_up_swiglu_multiply_int8: null pointer");
  QASR_REQUIRE(in_dim > 0 && in_dim <= 0x7fffffffu && seq_len <= 0x7fffffffu &&
                   intermediate <= 0x3fffffffu - 64,
               "gate_up_swiglu_multiply_int8: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(2 * intermediate, in_dim, &n) && mul_ok(seq_len, in_dim, &n) &&
                   mul_ok(seq_len, 2 * intermediate, &n) && n < ((size_t)1 << 33),
               "gate_up_swiglu_multiply_int8: size overflows");
  hipStream_t st = as_stream(stream);
  if (w8a32_gemm_shape(seq_len, in_dim, w_gate_up, x)) {
    GemmSet set{};
    set.y[0] = out;
    set.w[0] = w_gate_up;
    set.s[0] = scales_gate_up;
    set.b[0] = nullptr;
    set.N[0] = (int)(2 * intermediate);
    set.n = 1;
    if (!launch_w8a32_gemm<kGemmSwiglu>(set, x, (int)seq_len, (int)in_dim, st))
      return fail(QASR_ERR_UNSUPPORTED, "gate_up_swiglu_multiply_int8: the GEMM kernel cannot run this shape");
  } else {
    const long long items = (long long)seq_len * (long long)intermediate;
    gate_up_swiglu_w8a32_pairs_kernel<true><<<(unsigned)((items + 3) / 4), 256, 0, st>>>(
        out, x, w_gate_up, scales_gate_up, (int)seq_len, (int)in_dim, (int)intermediate);
  }
  return launch_status("gate_up_swiglu_multiply_int8");
}

// The q/k/v + heads launch; with xn the activations are the residual stream
// and the input RMSNorm is folded into the staging.
static int qkv_heads_impl(float* q, float* k_cache, float* v_cache, size_t cache_rows, const int8_t* wq,
                          const float* sq, const int8_t* wk, const float* sk, const int8_t* wv,
                          const float* sv, const float* x, size_t seq_len, size_t in_dim, size_t n_heads,
                          size_t n_kv_heads, size_t head_dim, const float* q_norm_w, const float* k_norm_w,
                          const float* cos_tab, const float* sin_tab, size_t table_rows, size_t start_pos,
                          float eps, void* stream, const GemmXNorm* xn) {
  if (seq_len == 0) return QASR_OK;
  QASR_REQUIRE(q && k_cache && v_cache && wq && sq && wk && sk && wv && sv && x && q_norm_w && k_norm_w &&
                   cos_tab && sin_tab,
               "qkv_heads_int8: null pointer");
  QASR_REQUIRE(n_heads >= 1 && n_kv_heads >= 1 && n_heads <= 65536 && n_kv_heads <= 65536,
               "qkv_heads_int8: head counts must be in [1, 65536]");
  QASR_REQUIRE(start_pos <= cache_rows && seq_len <= cache_rows - start_pos && start_pos <= table_rows &&
                   seq_len <= table_rows - start_pos,
               "qkv_heads_int8: rows start_pos..start_pos+seq_len exceed the cache or the RoPE table");
  if (head_dim != 128) return fail(QASR_ERR_UNSUPPORTED, "qkv_heads_int8: head_dim must be 128");
  const size_t rows = (n_heads + 2 * n_kv_heads) * 128, kv_dim = n_kv_heads * 128;
  size_t n;
  QASR_REQUIRE(rows <= 0x7fffffffu && in_dim <= 0x7fffffffu && seq_len <= 0x7fffffffu &&
                   start_pos <= 0x3fffffffffffffffull && table_rows <= 0x3fffffffffffffffull &&
                   cache_rows <= 0x3fffffffffffffffull,
               "qkv_heads_int8: size too large");
  QASR_REQUIRE(mul_ok(rows, in_dim, &n) && mul_ok(seq_len, in_dim, &n) && mul_ok(seq_len, rows, &n) &&
                   mul_ok(cache_rows, kv_dim, &n) && mul_ok(rows / 128, (seq_len + 63) / 64, &n) &&
                   n <= 0x7fffffffu,
               "qkv_heads_int8: size overflows");
  const bool aligned = aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(sq) &&
                       aligned16(sk) && aligned16(sv) && aligned16(q_norm_w) && aligned16(k_norm_w) &&
                       aligned16(cos_tab) && aligned16(sin_tab) && aligned16(wk) && aligned16(wv);
  if (!aligned || !w8a32_gemm_shape(seq_len, in_dim, wq, x))
    return fail(QASR_ERR_UNSUPPORTED,
                "qkv_heads_int8: needs seq_len >= 8, in_dim % 64 == 0 and 16-byte aligned buffers");
  GemmSet set{};
  const int8_t* ws[3] = {wq, wk, wv};
  const float* ss[3] = {sq, sk, sv};
  const size_t outs[3] = {n_heads * 128, kv_dim, kv_dim};
  for (int m = 0; m < 3; ++m) {
    set.y[m] = m == 0 ? q : nullptr;
    set.w[m] = ws[m];
    set.s[m] = ss[m];
    set.b[m] = nullptr;
    set.N[m] = (int)outs[m];
  }
  set.n = 3;
  GemmHeadEpi he{};
  he.k_cache = k_cache;
  he.v_cache = v_cache;
  he.q_norm_w = q_norm_w;
  he.k_norm_w = k_norm_w;
  he.cos_tab = cos_tab;
  he.sin_tab = sin_tab;
  he.start_pos = (long long)start_pos;
  he.table_rows = (long long)table_rows;
  he.cache_rows = (long long)cache_rows;
  he.n_kv_heads = (int)n_kv_heads;
  he.eps = eps;
  if (!launch_w8a32_heads(set, x, (int)seq_len, (int)in_dim, he, as_stream(stream), xn ? *xn : GemmXNorm{}))
    return fail(QASR_ERR_UNSUPPORTED, "qkv_heads_int8: the GEMM kernel cannot run this shape");
  return launch_status("qkv_heads_int8");
}

extern "C" int qasr_qkv_heads_int8_f32(float* q, float* k_cache, float* v_cache, size_t cache_rows,
                                       const int8_t* wq, const float* sq, const int8_t* wk,
                                       const float* sk, const int8_t* wv, const float* sv,
                                       const float* x, size_t seq_len, size_t in_dim, size_t n_heads,
                                       size_t n_kv_heads, size_t head_dim, const float* q_norm_w,
                                       const float* k_norm_w, const float* cos_tab,
                                       const float* sin_tab, size_t table_rows, size_t start_pos,
                                       float eps, void* stream) {
  return qkv_heads_impl(q, k_cache, v_cache, cache_rows, wq, sq, wk, sk, wv, sv, x, seq_len, in_dim, n_heads,
                        n_kv_heads, head_dim, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, start_pos, eps,
                        stream, nullptr);
}

namespace qasr {
namespace {
// x_norm = hg * rinv per row, rinv from the row's `slices` partial sums of
// squares added in slice order (as the folded GEMMs do): the normalised rows
// for the shapes the folded GEMMs do not take. In place (x_norm == hg) is fine.
__global__ __launch_bounds__(256) void xnorm_rows_kernel(float* x_norm, const float* hg, const float* __restrict__ ss,
                                                         int slices, int K, float eps) {
  const size_t row = blockIdx.x;
  const float* p = ss + row * (size_t)slices;
  float sum = 0.0f;
  for (int u = 0; u < slices; ++u) sum += p[u];
  const float rinv = 1.0f / sqrtf(sum / (float)K + eps);
  for (int k = threadIdx.x; k < K; k += 256) x_norm[row * K + k] = hg[row * K + k] * rinv;
}
}  // namespace
}  // namespace qasr

// Whether the folded GEMMs take these partial sums (their per-lane registers
// hold at most kXnMaxSlices, loaded 4 at a time).
static bool xnorm_fold_ok(const float* ss, size_t ss_slices) {
  return ss_slices % 4 == 0 && ss_slices <= (size_t)kXnMaxSlices && aligned16(ss);
}

static int xnorm_rows(float* x_norm, const float* hg, const float* ss, size_t slices, size_t rows, size_t K,
                      float eps, hipStream_t st) {
  xnorm_rows_kernel<<<(unsigned)rows, 256, 0, st>>>(x_norm, hg, ss, (int)slices, (int)K, eps);
  return launch_status("rms_norm fold: normalised rows");
}

extern "C" int qasr_rms_norm_qkv_heads_int8_f32(float* q, float* k_cache, float* v_cache, size_t cache_rows,
                                                const int8_t* wq, const float* sq, const int8_t* wk,
                                                const float* sk, const int8_t* wv, const float* sv,
                                                const float* hg, const float* ss, size_t ss_slices,
                                                float norm_eps, float* x_norm, size_t seq_len, size_t in_dim,
                                                size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                                const float* q_norm_w, const float* k_norm_w,
                                                const float* cos_tab, const float* sin_tab, size_t table_rows,
                                                size_t start_pos, float eps, void* stream) {
  if (seq_len == 0) return QASR_OK;
  QASR_REQUIRE(hg && ss && x_norm, "rms_norm_qkv_heads_int8: null pointer");
  QASR_REQUIRE(ss_slices == (in_dim + 63) / 64 && in_dim <= 0x7fffffffu && seq_len <= 0x7fffffffu,
               "rms_norm_qkv_heads_int8: ss_slices must be ceil(in_dim / 64)");
  if (xnorm_fold_ok(ss, ss_slices)) {
    const GemmXNorm xn{ss, (int)ss_slices, norm_eps};
    return qkv_heads_impl(q, k_cache, v_cache, cache_rows, wq, sq, wk, sk, wv, sv, hg, seq_len, in_dim, n_heads,
                          n_kv_heads, head_dim, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, start_pos, eps,
                          stream, &xn);
  }
  const int rc = xnorm_rows(x_norm, hg, ss, ss_slices, seq_len, in_dim, norm_eps, as_stream(stream));
  if (rc != QASR_OK) return rc;
  return qkv_heads_impl(q, k_cache, v_cache, cache_rows, wq, sq, wk, sk, wv, sv, x_norm, seq_len, in_dim, n_heads,
                        n_kv_heads, head_dim, q_norm_w, k_norm_w, cos_tab, sin_tab, table_rows, start_pos, eps,
                        stream, nullptr);
}

extern "C" int qasr_linear_int8_residual_f32(float* h, float* ss, float* hg, const float* gain, const float* x,
                                             const int8_t* w, const float* scales, size_t seq_len, size_t in_dim,
                                             size_t out_dim, void* stream) {
  if (seq_len == 0 || out_dim == 0) return QASR_OK;
  QASR_REQUIRE(h && ss && x && w && scales, "linear_int8_residual: null pointer");
  QASR_REQUIRE((hg == nullptr) == (gain == nullptr), "linear_int8_residual: hg and gain go together");
  QASR_REQUIRE(seq_len <= 0x7fffffffu && in_dim <= 0x7fffffffu && out_dim <= 0x7fffffffu,
               "linear_int8_residual: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(in_dim, out_dim, &n) && mul_ok(seq_len, in_dim, &n) && mul_ok(seq_len, out_dim, &n),
               "linear_int8_residual: size overflows");
  if (!w8a32_gemm_shape(seq_len, in_dim, w, x) || !aligned16(h) || (hg && !aligned16(hg)))
    return fail(QASR_ERR_UNSUPPORTED,
                "linear_int8_residual: needs seq_len >= 8, in_dim % 64 == 0 and 16-byte aligned h, hg, x, w");
  GemmSet set{};
  set.y[0] = h;
  set.w[0] = w;
  set.s[0] = scales;
  set.b[0] = nullptr;
  set.N[0] = (int)out_dim;
  set.n = 1;
  set.ss = ss;
  set.hg = hg;
  set.gain = gain;
  const unsigned c = (unsigned)((out_dim + 63) / 64);
  set.bx_begin[0] = 0;
  for (int m = 1; m <= 4; ++m) set.bx_begin[m] = c;
  const long long rows64 = (long long)((seq_len + 63) / 64);
  hipStream_t st = as_stream(stream);
  const bool ran = c * rows64 >= 256
                       ? try_gemm_ksplit<64, 64, 4, kGemmResidual>(set, c, x, (int)seq_len, (int)in_dim, st)
                       : try_gemm_ksplit<64, 32, 4, kGemmResidual>(set, c, x, (int)seq_len, (int)in_dim, st);
  if (!ran) return fail(QASR_ERR_UNSUPPORTED, "linear_int8_residual: the GEMM kernel cannot run this shape");
  return launch_status("linear_int8_residual");
}

extern "C" int qasr_rms_norm_gate_up_swiglu_multiply_int8_f32(float* out, const float* hg, const float* ss,
                                                             size_t ss_slices, float norm_eps, float* x_norm,
                                                             const int8_t* w_gate_up, const float* scales_gate_up,
                                                             size_t seq_len, size_t in_dim, size_t intermediate,
                                                             void* stream) {
  if (seq_len == 0 || intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && hg && ss && x_norm && w_gate_up && scales_gate_up,
               "rms_norm_gate_up_swiglu_multiply_int8: null pointer");
  QASR_REQUIRE(in_dim > 0 && in_dim <= 0x7fffffffu && seq_len <= 0x7fffffffu && intermediate <= 0x3fffffffu - 64,
               "rms_norm_gate_up_swiglu_multiply_int8: size too large");
  QASR_REQUIRE(ss_slices == (in_dim + 63) / 64,
               "rms_norm_gate_up_swiglu_multiply_int8: ss_slices must be ceil(in_dim / 64)");
  size_t n;
  QASR_REQUIRE(mul_ok(2 * intermediate, in_dim, &n) && mul_ok(seq_len, in_dim, &n) &&
                   mul_ok(seq_len, 2 * intermediate, &n) && n < ((size_t)1 << 33),
               "rms_norm_gate_up_swiglu_multiply_int8: size overflows");
  if (w8a32_gemm_shape(seq_len, in_dim, w_gate_up, hg) && xnorm_fold_ok(ss, ss_slices)) {
    GemmSet set{};
    set.y[0] = out;
    set.w[0] = w_gate_up;
    set.s[0] = scales_gate_up;
    set.b[0] = nullptr;
    set.N[0] = (int)(2 * intermediate);
    set.n = 1;
    const GemmXNorm xn{ss, (int)ss_slices, norm_eps};
    if (launch_w8a32_gemm<kGemmSwiglu | kGemmXNorm>(set, hg, (int)seq_len, (int)in_dim, as_stream(stream), xn))
      return launch_status("rms_norm_gate_up_swiglu_multiply_int8");
  }
  // a shape the folded kernels do not take: the normalised rows into x_norm, then the plain launch
  const int rc = xnorm_rows(x_norm, hg, ss, ss_slices, seq_len, in_dim, norm_eps, as_stream(stream));
  if (rc != QASR_OK) return rc;
  return qasr_gate_up_swiglu_multiply_int8_f32(out, x_norm, w_gate_up, scales_gate_up, seq_len, in_dim,
                                               intermediate, stream);
}

extern "C" int qasr_linear_nobias_int8_multi_f32(size_t n_mats, float* const* ys,
                                                 const int8_t* const* ws,
                                                 const float* const* scales,
                                                 const size_t* out_dims, const float* x,
                                                 size_t seq_len, size_t in_dim, void* stream) {
  if (n_mats == 0 || seq_len == 0) return QASR_OK;
  QASR_REQUIRE(ys && ws && scales && out_dims && x, "linear_nobias_int8_multi: null pointer");
  QASR_REQUIRE(n_mats <= (size_t)kMaxMats, "linear_nobias_int8_multi: at most 4 matrices");
  bool one_launch = seq_len == 1;
  size_t total = 0;
  for (size_t m = 0; m < n_mats; ++m) {
    QASR_REQUIRE(ys[m] && ws[m] && scales[m], "linear_nobias_int8_multi: null pointer");
    QASR_REQUIRE(out_dims[m] <= 0x7fffffffu - 64 && in_dim <= 0x7fffffffu,
                 "linear_nobias_int8_multi: size too large");
    size_t n;
    QASR_REQUIRE(mul_ok(in_dim, out_dims[m], &n) && mul_ok(seq_len, in_dim, &n) &&
                     mul_ok(seq_len, out_dims[m], &n),
                 "linear_nobias_int8_multi: size overflows");
    one_launch = one_launch && w8a32_rows_shape(in_dim, ws[m], x);
    total += out_dims[m];
  }
  QASR_REQUIRE(total <= 0x7fffffffu, "linear_nobias_int8_multi: size too large");
  if (total == 0) return QASR_OK;
  bool gemm = !one_launch;
  for (size_t m = 0; m < n_mats; ++m) gemm = gemm && w8a32_gemm_shape(seq_len, in_dim, ws[m], x);
  if (gemm) {
    GemmSet set{};
    for (size_t m = 0; m < n_mats; ++m) {
      set.y[m] = ys[m];
      set.w[m] = ws[m];
      set.s[m] = scales[m];
      set.b[m] = nullptr;
      set.N[m] = (int)out_dims[m];
    }
    set.n = (int)n_mats;
    if (!launch_w8a32_gemm<kGemmRows>(set, x, (int)seq_len, (int)in_dim, as_stream(stream)))
      return fail(QASR_ERR_UNSUPPORTED, "linear_nobias_int8_multi: the GEMM kernel cannot run this shape");
    return launch_status("linear_nobias_int8_multi");
  }
  if (!one_launch) {
    for (size_t m = 0; m < n_mats; ++m) {
      const int rc = launch_w8a32(ys[m], x, ws[m], scales[m], nullptr, seq_len, in_dim, out_dims[m],
                                  stream);
      if (rc != QASR_OK) return rc;
    }
    return QASR_OK;
  }
  const int r = rows_per_wave(in_dim, total);
  MatSet ms{};
  unsigned wg = 0;
  for (size_t m = 0; m < n_mats; ++m) {
    ms.y[m] = ys[m];
    ms.w[m] = ws[m];
    ms.s[m] = scales[m];
    ms.out[m] = (int)out_dims[m];
    ms.wg_begin[m] = wg;
    wg += (unsigned)((out_dims[m] + 4 * r - 1) / (4 * r));
  }
  for (size_t m = n_mats; m <= (size_t)kMaxMats; ++m) ms.wg_begin[m] = wg;
  ms.n = (int)n_mats;
  launch_rows_multi((int)(in_dim / 1024), r, wg, as_stream(stream), ms, x, (int)in_dim);
  return launch_status("linear_nobias_int8_multi");
}

// [a, a + an) and [b, b + bn) share a byte (null never overlaps)
static bool bytes_overlap(const void* a, size_t an, const void* b, size_t bn) {
  if (!a || !b) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + bn && pb < pa + an;
}

// Checks shared by the fused add + RMSNorm + projection entry points: the row
// is in_dim floats on the one-token vector path, h_out overlaps neither input.
static int check_row_norm(const char* what, float* h_out, const float* x, const float* delta,
                          const float* norm_w, size_t in_dim, float eps) {
  QASR_REQUIRE(x && norm_w, std::string(what) + ": null pointer");
  if (!(in_dim >= 1024 && in_dim % 1024 == 0 && in_dim <= 8192))
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": in_dim must be 1024..8192 in steps of 1024");
  if (!(aligned16(x) && aligned16(norm_w) && aligned16(delta) && aligned16(h_out)))
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": rows must be 16-byte aligned");
  const size_t nb = in_dim * sizeof(float);
  QASR_REQUIRE(!bytes_overlap(h_out, nb, x, nb) && !bytes_overlap(h_out, nb, delta, nb),
               std::string(what) + ": h_out must not overlap x or delta");
  QASR_REQUIRE(eps >= 0.0f, std::string(what) + ": eps must be non-negative");
  return QASR_OK;
}

extern "C" int qasr_add_rms_norm_linear_nobias_int8_multi_f32(
    size_t n_mats, float* const* ys, const int8_t* const* ws, const float* const* scales,
    const size_t* out_dims, float* h_out, const float* x, const float* delta, const float* norm_w,
    size_t in_dim, float eps, void* stream) {
  const char* what = "add_rms_norm_linear_nobias_int8_multi";
  if (n_mats == 0) return QASR_OK;
  QASR_REQUIRE(ys && ws && scales && out_dims, std::string(what) + ": null pointer");
  QASR_REQUIRE(n_mats <= (size_t)kMaxMats, std::string(what) + ": at most 4 matrices");
  int rc = check_row_norm(what, h_out, x, delta, norm_w, in_dim, eps);
  if (rc != QASR_OK) return rc;
  size_t total = 0;
  for (size_t m = 0; m < n_mats; ++m) {
    QASR_REQUIRE(ys[m] && ws[m] && scales[m], std::string(what) + ": null pointer");
    QASR_REQUIRE(out_dims[m] <= 0x7fffffffu - 64, std::string(what) + ": size too large");
    size_t n;
    QASR_REQUIRE(mul_ok(in_dim, out_dims[m], &n), std::string(what) + ": size overflows");
    if (!aligned16(ws[m])) return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": weights must be 16-byte aligned");
    const size_t yb = out_dims[m] * sizeof(float), nb = in_dim * sizeof(float);
    QASR_REQUIRE(!bytes_overlap(ys[m], yb, x, nb) && !bytes_overlap(ys[m], yb, delta, nb) &&
                     !bytes_overlap(ys[m], yb, h_out, nb),
                 std::string(what) + ": outputs must not overlap the row");
    total += out_dims[m];
  }
  QASR_REQUIRE(total <= 0x7fffffffu, std::string(what) + ": size too large");
  const int r = rows_per_wave(in_dim, total);
  MatSet ms{};
  unsigned wg = 0;
  for (size_t m = 0; m < n_mats; ++m) {
    ms.y[m] = ys[m];
    ms.w[m] = ws[m];
    ms.s[m] = scales[m];
    ms.out[m] = (int)out_dims[m];
    ms.wg_begin[m] = wg;
    wg += (unsigned)((out_dims[m] + 4 * r - 1) / (4 * r));
  }
  for (size_t m = n_mats; m <= (size_t)kMaxMats; ++m) ms.wg_begin[m] = wg;
  ms.n = (int)n_mats;
  if (wg == 0) return QASR_OK;
  const RowNorm rn{x, delta, norm_w, h_out, eps};
  launch_rows_multi<true>((int)(in_dim / 1024), r, wg, as_stream(stream), ms, x, (int)in_dim, rn);
  return launch_status(what);
}

extern "C" int qasr_add_rms_norm_gate_up_swiglu_int8_f32(float* out, float* h_out, const float* x,
                                                         const float* delta, const float* norm_w,
                                                         const int8_t* w_gate_up,
                                                         const float* scales_gate_up, size_t in_dim,
                                                         size_t intermediate, float eps,
                                                         void* stream) {
  const char* what = "add_rms_norm_gate_up_swiglu_int8";
  if (intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && w_gate_up && scales_gate_up, std::string(what) + ": null pointer");
  int rc = check_row_norm(what, h_out, x, delta, norm_w, in_dim, eps);
  if (rc != QASR_OK) return rc;
  QASR_REQUIRE(intermediate <= 0x3fffffffu - 64, std::string(what) + ": size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(2 * intermediate, in_dim, &n), std::string(what) + ": size overflows");
  if (!aligned16(w_gate_up)) return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": weights must be 16-byte aligned");
  const size_t ob = intermediate * sizeof(float), nb = in_dim * sizeof(float);
  QASR_REQUIRE(!bytes_overlap(out, ob, x, nb) && !bytes_overlap(out, ob, delta, nb) &&
                   !bytes_overlap(out, ob, h_out, nb),
               std::string(what) + ": out must not overlap the row");
  const size_t rows = 2 * intermediate;
  const int r = rows_per_wave(in_dim, rows) < 2 ? 2 : rows_per_wave(in_dim, rows);
  const RowNorm rn{x, delta, norm_w, h_out, eps};
  launch_rows<kEpiSwiglu, true>((int)(in_dim / 1024), r, (unsigned)((rows + 4 * r - 1) / (4 * r)),
                                as_stream(stream), out, x, w_gate_up, scales_gate_up, nullptr,
                                (int)in_dim, (int)rows, nullptr, rn);
  return launch_status(what);
}

extern "C" int qasr_linear_int8_f32(float* y, const float* x, const int8_t* w, const float* scales,
                                    const float* bias, size_t seq_len, size_t in_dim,
                                    size_t out_dim, void* stream) {
  return launch_w8a32(y, x, w, scales, bias, seq_len, in_dim, out_dim, stream);
}

extern "C" int qasr_interleave_gate_up_i8(int8_t* w_gate_up, float* scales_gate_up,
                                          const int8_t* w_gate, const float* s_gate,
                                          const int8_t* w_up, const float* s_up,
                                          size_t intermediate, size_t hidden, void* stream) {
  if (intermediate == 0 || hidden == 0) return QASR_OK;
  QASR_REQUIRE(w_gate_up && scales_gate_up && w_gate && s_gate && w_up && s_up,
               "interleave_gate_up_i8: null pointer");
  size_t n;
  QASR_REQUIRE(mul_ok(2 * intermediate, hidden, &n), "interleave_gate_up_i8: size overflows");
  interleave_kernel<<<grid_for(intermediate * hidden, 256), 256, 0, as_stream(stream)>>>(
      w_gate_up, scales_gate_up, w_gate, s_gate, w_up, s_up, intermediate, hidden);
  return launch_status("interleave_gate_up_i8");
}

extern "C" int qasr_gate_up_swiglu_w8a8(float* out, const int8_t* w, const float* scales,
                                        const int8_t* xq, const float* x_scales, size_t batch,
                                        size_t in_dim, size_t intermediate, void* stream) {
  if (batch == 0 || intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && w && scales && xq && x_scales, "gate_up_swiglu_w8a8: null pointer");
  QASR_REQUIRE(in_dim > 0 && in_dim % 16 == 0, "gate_up_swiglu_w8a8: in_dim must be a positive multiple of 16");
  QASR_REQUIRE(aligned16(w) && aligned16(xq), "gate_up_swiglu_w8a8: w and xq must be 16-byte aligned");
  QASR_REQUIRE(batch <= 0x7fffffffu && intermediate <= 0x3fffffffu && in_dim <= 0x7fffffffu,
               "gate_up_swiglu_w8a8: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(2 * intermediate, in_dim, &n) && mul_ok(batch, in_dim, &n) &&
                   mul_ok(batch, intermediate, &n),
               "gate_up_swiglu_w8a8: size overflows");
  hipStream_t st = as_stream(stream);
  if (batch == 1 && matvec_shape(in_dim)) {
    return launch_matvec<false>(out, w, scales, xq, x_scales, nullptr, in_dim, intermediate, st);
  }
  if (batch > 1 && gemm_w8a8_supported(batch, in_dim, intermediate)) {
    return gemm_w8a8_swiglu(out, w, scales, xq, x_scales, batch, in_dim, intermediate, st);
  }
  const long long items = (long long)batch * (long long)intermediate;
  gateup_generic_kernel<<<(unsigned)((items + 3) / 4), 256, 0, st>>>(
      out, w, scales, xq, x_scales, (int)batch, (int)in_dim, (int)intermediate);
  return launch_status("gate_up_swiglu_w8a8 (generic)");
}

extern "C" int qasr_gate_up_swiglu_w8a8_f32in(float* out, const int8_t* w, const float* scales,
                                              const float* x, size_t in_dim, size_t intermediate,
                                              void* stream) {
  if (intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && w && scales && x, "gate_up_swiglu_w8a8_f32in: null pointer");
  QASR_REQUIRE(aligned16(w) && aligned16(x), "gate_up_swiglu_w8a8_f32in: w and x must be 16-byte aligned");
  QASR_REQUIRE(intermediate <= 0x3fffffffu, "gate_up_swiglu_w8a8_f32in: size too large");
  if (!matvec_shape(in_dim)) {
    return fail(QASR_ERR_UNSUPPORTED,
                "gate_up_swiglu_w8a8_f32in: in_dim must be 1024..4096 in steps of 1024");
  }
  return launch_matvec<true>(out, w, scales, nullptr, nullptr, x, in_dim, intermediate,
                             as_stream(stream));
}

extern "C" int qasr_pack_w8a8_tiles(int8_t* packed, const int8_t* w, size_t rows, size_t cols,
                                    void* stream) {
  if (rows == 0 || cols == 0) return QASR_OK;
  QASR_REQUIRE(packed && w, "pack_w8a8_tiles: null pointer");
  QASR_REQUIRE(packed != w, "pack_w8a8_tiles: packing is out of place");
  QASR_REQUIRE(rows % kPackRows == 0 && cols % kPackK == 0,
               "pack_w8a8_tiles: rows must be a multiple of 16 and cols of 64");
  QASR_REQUIRE(aligned16(packed) && aligned16(w), "pack_w8a8_tiles: 16-byte alignment required");
  size_t n;
  QASR_REQUIRE(mul_ok(rows, cols, &n), "pack_w8a8_tiles: size overflows");
  const size_t slices = n / 16;
  pack_w8a8_tiles_kernel<<<grid_for(slices, 256), 256, 0, as_stream(stream)>>>(
      packed, w, slices, (int)(cols / kPackK), cols);
  return launch_status("pack_w8a8_tiles");
}

extern "C" int qasr_gate_up_swiglu_w8a8_packed(float* out, const int8_t* w_packed,
                                               const float* scales, const int8_t* xq,
                                               const float* x_scales, size_t batch,
                                               size_t in_dim, size_t intermediate,
                                               void* stream) {
  if (batch == 0 || intermediate == 0) return QASR_OK;
  QASR_REQUIRE(out && w_packed && scales && xq && x_scales,
               "gate_up_swiglu_w8a8_packed: null pointer");
  QASR_REQUIRE(aligned16(w_packed) && aligned16(xq) && aligned16(scales),
               "gate_up_swiglu_w8a8_packed: w, xq and scales must be 16-byte aligned");
  QASR_REQUIRE((reinterpret_cast<uintptr_t>(out) & 7u) == 0,
               "gate_up_swiglu_w8a8_packed: out must be 8-byte aligned");
  QASR_REQUIRE(batch <= 0x7fffffffu - 63, "gate_up_swiglu_w8a8_packed: batch too large");
  QASR_REQUIRE(batch <= 0x7fffffffu && intermediate <= 0x3fffffffu,
               "gate_up_swiglu_w8a8_packed: size too large");
  if (!packed_gemm_shape(in_dim, intermediate)) {
    return fail(QASR_ERR_UNSUPPORTED,
                "gate_up_swiglu_w8a8_packed: needs in_dim 1024 or 2048 and 2*intermediate % 192 == 0");
  }
  if (!try_packed_gemm(out, w_packed, scales, xq, x_scales, batch, in_dim, intermediate,
                       as_stream(stream))) {
    return fail(QASR_ERR_UNSUPPORTED,
                "gate_up_swiglu_w8a8_packed: the device cannot give a workgroup 128 KiB of LDS");
  }
  return launch_status("gate_up_swiglu_w8a8_packed");
}
