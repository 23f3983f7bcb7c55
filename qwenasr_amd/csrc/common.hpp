// Shared device helpers and C-ABI glue for the gfx950 kernels.
//
// All kernels are written for 64-lane wavefronts. Reductions inside a wave use
// cross-lane shuffles; reductions across the waves of a workgroup go through
// LDS. Nothing here depends on any other GPU family.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stddef.h>

#include <string>

#include "../../include/qasr.h"

#define QASR_DEV __device__ __forceinline__

namespace qasr {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Cross-lane reductions
// ---------------------------------------------------------------------------

// Sum over groups of WIDTH consecutive lanes (WIDTH a power of two <= 64).
// Every lane of a group ends with the same value.
template <int WIDTH>
QASR_DEV float group_sum(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

template <int WIDTH>
QASR_DEV float group_max(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) {
    float o = __shfl_xor(v, m, kWave);
    v = o > v ? o : v;
  }
  return v;
}

template <int WIDTH>
QASR_DEV int group_sum_i32(int v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

QASR_DEV float wave_sum(float v) { return group_sum<kWave>(v); }
QASR_DEV float wave_max(float v) { return group_max<kWave>(v); }

// Sum over a workgroup of BLOCK threads; every thread gets the same result
// (the per-wave partials are added in wave order by every thread).
// `lds` needs BLOCK/64 floats. Ends with a barrier so `lds` can be reused.
template <int BLOCK>
QASR_DEV float block_sum(float v, float* lds) {
  v = wave_sum(v);
  if constexpr (BLOCK == kWave) {
    return v;
  } else {
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x / kWave;
    if (lane == 0) lds[w] = v;
    __syncthreads();
    float t = lds[0];
#pragma unroll
    for (int i = 1; i < BLOCK / kWave; ++i) t += lds[i];
    __syncthreads();
    return t;
  }
}

template <int BLOCK>
QASR_DEV float block_max(float v, float* lds) {
  v = wave_max(v);
  if constexpr (BLOCK == kWave) {
    return v;
  } else {
    const int lane = threadIdx.x & (kWave - 1);
    const int w = threadIdx.x / kWave;
    if (lane == 0) lds[w] = v;
    __syncthreads();
    float t = lds[0];
#pragma unroll
    for (int i = 1; i < BLOCK / kWave; ++i) t = lds[i] > t ? lds[i] : t;
    __syncthreads();
    return t;
  }
}

// ---------------------------------------------------------------------------
// 16-byte streaming loads/stores. The nontemporal forms mark the lines for
// early eviction, which suits data each kernel touches exactly once.
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));

QASR_DEV float4 ld4(const float* p, size_t i) { return reinterpret_cast<const float4*>(p)[i]; }
QASR_DEV void st4(float* p, size_t i, float4 v) { reinterpret_cast<float4*>(p)[i] = v; }

QASR_DEV float4 ld4_nt(const float* p, size_t i) {
  const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p) + i);
  return make_float4(v[0], v[1], v[2], v[3]);
}

QASR_DEV void st4_nt(float* p, size_t i, float4 v) {
  const v4f o = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(o, reinterpret_cast<v4f*>(p) + i);
}

// ---------------------------------------------------------------------------
// Scalar math shared by several kernels
// ---------------------------------------------------------------------------

// silu(g) = g / (1 + exp(-g)), the libm form of decoder.rs:571-576.
QASR_DEV float silu_expf(float g) { return g / (1.0f + expf(-g)); }

// The x86_64 reference's degree-5 exp polynomial (avx.rs:483-514), one lane:
// clamp x*log2(e) to [-126, 126], split into nearest integer i (round half to
// even, as cvtps_epi32 does) and fraction f, then 2^i * P(f*ln2) with P the
// Taylor polynomial of exp to degree 5 evaluated by fused multiply-adds.
QASR_DEV float ref_fast_exp(float x) {
  float val = x * 1.442695041f;
  val = (val < 126.0f) ? val : 126.0f;   // minps(val, 126): NaN -> 126
  val = (val > -126.0f) ? val : -126.0f; // maxps(val, -126)
  const int ip = (int)__builtin_rintf(val);
  const float fp = val - (float)ip;
  const float e = __int_as_float((ip + 127) << 23);
  const float f = fp * 0.6931471806f;
  float p = __builtin_fmaf(1.0f / 120.0f, f, 1.0f / 24.0f);
  p = __builtin_fmaf(p, f, 1.0f / 6.0f);
  p = __builtin_fmaf(p, f, 0.5f);
  p = __builtin_fmaf(p, f, 1.0f);
  p = __builtin_fmaf(p, f, 1.0f);
  return e * p;
}

// One output of the prefill SwiGLU (kernels::swiglu_multiply, x86 arithmetic
// avx.rs:565-599): silu(g) * u with silu from fast_exp for columns below
// inter & ~7 (fast) and from expf for the row tail. Shared by the SwiGLU
// kernel and the gate/up GEMM's SwiGLU epilogue, which agree bit for bit.
QASR_DEV float swiglu_ref(float g, float u, bool fast) {
  const float s = fast ? g / (1.0f + ref_fast_exp(0.0f - g)) : g / (1.0f + expf(-g));
  return s * u;
}

QASR_DEV float qnan() { return __int_as_float(0x7fc00000); }

// s_waitcnt lgkmcnt(0) with vmcnt and expcnt left at their maxima (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
constexpr int kWaitLgkm0 = 15 | (7 << 4) | (0 << 8) | (3 << 14);
// s_waitcnt immediate that waits until at most n vector memory operations of
// this wave are outstanding (LDS and export counters left free).
constexpr int vmcnt_at_most(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// Workgroup barrier without a global-memory fence: the workgroup's LDS writes
// are complete (lgkmcnt(0)) and visible after it; outstanding global loads and
// stores keep flying (__syncthreads would wait for them: gfx9 counts both in
// vmcnt).
QASR_DEV void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  asm volatile("s_barrier" ::: "memory");
}

// Per-head RMSNorm (NORM) and NeoX RoPE (ROPE) of one head held by a group of
// HD/8 consecutive lanes: lane `sub` holds dims 4sub..4sub+3 in x1 and
// HD/2 + 4sub..4sub+3 in x2, with the gains (w1, w2) and the position's table
// entries (c1, c2, s1, s2) for the same dims.
//   kernels/mod.rs:927-932: rms_inv = 1/sqrt(sum(v^2)/head_dim + eps); v = v*rms_inv*w
//   kernels/mod.rs:1262-1263: v[d] = x1*c[d] + (-x2)*s[d]; v[d+h] = x2*c[d+h] + x1*s[d+h]
// A position outside the table (pos_ok false) turns the head to NaN. Every
// kernel that normalises or rotates heads calls this, so they agree bit for bit.
template <int HD, bool NORM, bool ROPE>
QASR_DEV void head_norm_rope(float4& x1, float4& x2, const float4& w1, const float4& w2,
                             const float4& c1, const float4& c2, const float4& s1,
                             const float4& s2, bool pos_ok, float eps) {
  if constexpr (NORM) {
    float ss = x1.x * x1.x;
    ss += x1.y * x1.y;
    ss += x1.z * x1.z;
    ss += x1.w * x1.w;
    ss += x2.x * x2.x;
    ss += x2.y * x2.y;
    ss += x2.z * x2.z;
    ss += x2.w * x2.w;
    ss = group_sum<HD / 8>(ss);
    const float rinv = 1.0f / sqrtf(ss / (float)HD + eps);
    x1.x = (x1.x * rinv) * w1.x; x1.y = (x1.y * rinv) * w1.y;
    x1.z = (x1.z * rinv) * w1.z; x1.w = (x1.w * rinv) * w1.w;
    x2.x = (x2.x * rinv) * w2.x; x2.y = (x2.y * rinv) * w2.y;
    x2.z = (x2.z * rinv) * w2.z; x2.w = (x2.w * rinv) * w2.w;
  }
  if constexpr (ROPE) {
    if (!pos_ok) {
      const float n = qnan();
      x1 = make_float4(n, n, n, n);
      x2 = x1;
    } else {
      float4 o1, o2;
      o1.x = x1.x * c1.x + (-x2.x) * s1.x; o2.x = x2.x * c2.x + x1.x * s2.x;
      o1.y = x1.y * c1.y + (-x2.y) * s1.y; o2.y = x2.y * c2.y + x1.y * s2.y;
      o1.z = x1.z * c1.z + (-x2.z) * s1.z; o2.z = x2.z * c2.z + x1.z * s2.z;
      o1.w = x1.w * c1.w + (-x2.w) * s1.w; o2.w = x2.w * c2.w + x1.w * s2.w;
      x1 = o1;
      x2 = o2;
    }
  }
}

// Round half away from zero, then clamp to int8 (NaN -> 0), the arithmetic of
// quantize.rs:657-658: `(v * inv).round().clamp(-128, 127) as i8`.
QASR_DEV int quant_i8(float v, float inv) {
  float r = roundf(v * inv);
  r = r < -128.0f ? -128.0f : r;
  r = r > 127.0f ? 127.0f : r;
  return (r == r) ? (int)r : 0;
}

// Number of workgroups for a grid-stride elementwise launch: enough to keep
// every CU busy with several waves, never more than the work needs.
inline unsigned grid_for(size_t items, unsigned block, unsigned cap = 256 * 16) {
  size_t g = (items + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

// ---------------------------------------------------------------------------
// C-ABI error plumbing
// ---------------------------------------------------------------------------

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Checks hipGetLastError after a launch and converts it to a status.
int launch_status(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Largest size any kernel indexes with 64-bit arithmetic; guards products of
// dimensions against overflow.
constexpr size_t kMaxElems = (size_t)1 << 40;

// A launch's total work-item count (grid x workgroup size) must fit in 32
// bits; exact-cover grids of 256-thread workgroups stay below this bound.
constexpr size_t kMaxGridItems = ((size_t)1 << 32) - 256;
inline bool exact_grid_ok(size_t items) { return items <= kMaxGridItems; }
// Most rows one row-per-workgroup launch may cover.
constexpr size_t kMaxRows = (size_t)1 << 24;

inline bool mul_ok(size_t a, size_t b, size_t* out) {
  if (a != 0 && b > kMaxElems / a) return false;
  *out = a * b;
  return true;
}

// Argmax order of the reference's lm_head scan (decoder.rs:941-949): a larger
// value wins, equal values go to the lower index, a NaN never wins.
QASR_DEV bool argmax_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}
QASR_DEV void argmax_consider(float v, int i, float& bv, int& bi) {
  if (v == v && argmax_better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

// Logits of one token through the W8A32 decode kernel, which also writes one
// (best value, index bits) pair per workgroup to `part` (int8.hip). Returns
// false, launching nothing, when the shape has no such kernel; *n_part is the
// number of pairs written.
bool launch_w8a32_argmax_partials(float* y, const float* x, const int8_t* w, const float* scales,
                                  size_t in_dim, size_t out_dim, float2* part, size_t part_cap,
                                  hipStream_t st, unsigned* n_part);
// Most pairs any shape writes: one per 4 output rows.
inline size_t lm_head_partials_max(size_t vocab) { return (vocab + 3) / 4; }

}  // namespace qasr

#define QASR_REQUIRE(cond, msg)                                   \
  do {                                                            \
    if (!(cond)) return ::qasr::fail(QASR_ERR_INVALID_ARG, msg); \
  } while (0)
