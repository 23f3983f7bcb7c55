// Batched W8A8 gate/up GEMM fused with SwiGLU on CDNA4 int8 MFMA.
//
//   C[n, m] = sum_k W[n, k] * Xq[m, k]       (int32, exact)
//   out[m, p] = silu(g) * u,  g = ((f32)C[2p, m] * xs[m]) * s[2p],
//                             u = ((f32)C[2p+1, m] * xs[m]) * s[2p+1]
//
// W is the row-interleaved gate/up matrix [N = 2*inter, K], Xq the per-row
// quantized activations [M = batch, K]. Both are K-contiguous, so each lane's
// MFMA operand is one 16-byte load.
//
// v_mfma_i32_16x16x64_i8: lane l supplies 16 int8 of A row (l % 16) and 16 int8
// of B column (l % 16) for k-group (l / 16); the result lane l holds
// D[4*(l/16) + v][l % 16], v = 0..3. The order of k inside an MFMA does not
// matter as long as A and B use the same one, which they do: lane l loads bytes
// [k0 + 16*(l/16), +16) of its W row and of its Xq row. With A = W and B = Xq^T a
// lane's four results are four consecutive W rows for one token -- two complete
// gate/up pairs -- so the SwiGLU epilogue needs no data exchange.
//
// Row-major kernel (gemm_w8a8_swiglu_lds_kernel, K = 1024 or 2048): a workgroup
// owns 192 W rows x 64 tokens. The 64 token rows of Xq (64 x K bytes) are
// staged once in LDS by direct global->LDS loads, with a 16-byte row pad
// (conflict-free b128 reads); each of the 4 waves owns 48 distinct W rows and
// streams them from HBM into registers with a PREFETCH-deep software pipeline,
// so W never touches LDS. The 4 workgroups that share a W tile (one per 64-token block) are
// dispatched to the same XCD back to back, so 3 of their 4 W reads hit that
// XCD's L2. gemm_w8a8_swiglu_kernel is the shape-generic fallback.
#pragma once

#include "common.hpp"

#include <atomic>

namespace qasr {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmK = 64;  // k per MFMA

// SwiGLU epilogue of every W8A8 kernel (matvec and GEMM alike, so their
// results agree bit for bit): g = (dg * xs) * sg, u = (du * xs) * su,
// out = silu(g) * u. silu uses the hardware exp2 (__expf) and reciprocal:
// a few ulp from g / (1 + expf(-g)), far inside the 1e-5 tolerance, at a third
// of the VALU cost of the IEEE exp + divide. g >> 0 gives exactly g (exp
// underflows to 0, rcp(1) = 1); g << 0 gives -0 (rcp(inf) = 0).
QASR_DEV float swiglu_w8a8(int dg, int du, float xs, float sg, float su) {
  const float g = ((float)dg * xs) * sg;
  const float u = ((float)du * xs) * su;
  return (g * __builtin_amdgcn_rcpf(1.0f + __expf(-g))) * u;
}

// ---------------------------------------------------------------------------
// Main kernel
// ---------------------------------------------------------------------------
constexpr int kLdsBN = 192;           // W rows per workgroup
constexpr int kLdsBM = 64;            // tokens per workgroup
constexpr int kLdsWaveRows = 48;      // W rows per wave (3 MFMA row tiles)
constexpr int kLdsMaxK = 2048;        // X tile must fit LDS: 64 x (2048 + 16) B
constexpr int kLdsRowPad = 16;
constexpr int kPrefetch = 12;         // k-steps of W in flight per wave
constexpr int kNumXcd = 8;

// MFMA tile layout of a weight matrix ("packed") for v_mfma_i32_16x16x64_i8:
// for each block of 16 rows rb and each 64-byte k-step s, one contiguous 1 KiB
// tile whose byte 16*lane + b is W[16*rb + lane % 16][64*s + 16*(lane / 16) + b],
// i.e. exactly the A operand lane `lane` feeds the MFMA. Tiles are ordered
// [rb][s], so a wave's operand load is one fully used 1 KiB span (8 cache
// lines) instead of 16 row fragments of 64 bytes.
constexpr int kPackRows = 16;
constexpr int kPackK = 64;

QASR_DEV size_t packed_tile_offset(int rb, int s, int ksteps) {
  return ((size_t)rb * ksteps + s) * 1024;
}

template <int KSTEPS>  // K / 64
__global__ __launch_bounds__(256) void gemm_w8a8_swiglu_lds_kernel(
    float* __restrict__ out, const int8_t* __restrict__ w, const float* __restrict__ scales,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int batch, int inter,
    int n_tiles, int m_tiles) {
  constexpr int K = KSTEPS * kGemmK;
  constexpr int LDS_STRIDE = K + kLdsRowPad;
  extern __shared__ __align__(16) int8_t xlds[];  // [64][K + 16]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;

  // XCD-aware tile order: consecutive blocks go to consecutive XCDs, so block
  // b runs on XCD b % 8. Put the m_tiles blocks of one W tile on one XCD.
  const int b = blockIdx.x;
  const int xcd = b % kNumXcd;
  const int slot = b / kNumXcd;
  int tile_n, tile_m;
  if (n_tiles % kNumXcd == 0) {
    tile_m = slot % m_tiles;
    tile_n = xcd + kNumXcd * (slot / m_tiles);
  } else {
    tile_m = b % m_tiles;
    tile_n = b / m_tiles;
  }
  const int n_wave = tile_n * kLdsBN + wave * kLdsWaveRows;
  const int m0 = tile_m * kLdsBM;

  // W operand pointers for this wave's three 16-row tiles (lane row r, group
  // g) and the byte step between consecutive k-steps.
  const int8_t* wp[3];
  constexpr int WSTEP = kGemmK;
#pragma unroll
  for (int i = 0; i < 3; ++i) wp[i] = w + (size_t)(n_wave + 16 * i + r) * K + 16 * g;

  // Stage Xq rows m0..m0+63 into LDS with direct global->LDS loads: each wave
  // instruction moves 64 lanes x 16 bytes into 1 KiB of contiguous LDS (half or
  // all of a K=2048 / K=1024 row), so the 128 KiB tile is in flight at once with
  // no register round trip. Rows past the batch re-read row batch-1 (valid
  // memory); their results are never stored.
  {
    constexpr int CHUNKS_PER_ROW = K / 1024;
    constexpr int CHUNKS = kLdsBM * CHUNKS_PER_ROW;
#pragma unroll 4
    for (int c = wave; c < CHUNKS; c += 4) {
      const int row = c / CHUNKS_PER_ROW, half = c - row * CHUNKS_PER_ROW;
      const int src_row = m0 + row < batch ? m0 + row : batch - 1;
      const int8_t* src = xq + (size_t)src_row * K + 1024 * half + 16 * lane;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(xlds + row * LDS_STRIDE + 1024 * half), 16, 0, 0);
    }
  }

  // Start the W stream; its HBM latency overlaps the LDS fill.
  v4i wbuf[kPrefetch][3];
#pragma unroll
  for (int d = 0; d < kPrefetch; ++d)
#pragma unroll
    for (int i = 0; i < 3; ++i)
      if (d < KSTEPS) wbuf[d][i] = *reinterpret_cast<const v4i*>(wp[i] + d * WSTEP);

  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0);  // the LDS fill (and the W prefetch) have landed
  __syncthreads();

  v4i acc[3][4];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  const int8_t* xl = xlds + r * LDS_STRIDE + 16 * g;
#pragma unroll
  for (int s0 = 0; s0 < KSTEPS; s0 += kPrefetch) {
#pragma unroll
    for (int d = 0; d < kPrefetch; ++d) {
      const int s = s0 + d;
      if (s < KSTEPS) {
        v4i a[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          a[i] = wbuf[d][i];
          if (s + kPrefetch < KSTEPS)
            wbuf[d][i] = *reinterpret_cast<const v4i*>(wp[i] + (s + kPrefetch) * WSTEP);
        }
        // Keep the prefetch issue here: without this fence the scheduler sinks
        // each load next to its use and the pipeline collapses to one load in
        // flight per k-step.
        __builtin_amdgcn_sched_barrier(0);
        v4i bx[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bx[j] = *reinterpret_cast<const v4i*>(xl + 16 * j * LDS_STRIDE + s * kGemmK);
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], bx[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // Epilogue: lane holds W rows n_wave + 16i + 4g + {0..3} for token m0 + 16j + r.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + 16 * j + r;
    if (m >= batch) continue;
    const float xsm = xs[m];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int n = n_wave + 16 * i + 4 * g;
      const float4 sc = *reinterpret_cast<const float4*>(scales + n);
      float2 o;
      o.x = swiglu_w8a8(acc[i][j][0], acc[i][j][1], xsm, sc.x, sc.y);
      o.y = swiglu_w8a8(acc[i][j][2], acc[i][j][3], xsm, sc.z, sc.w);
      *reinterpret_cast<float2*>(out + (size_t)m * inter + (n >> 1)) = o;
    }
  }
}

// ---------------------------------------------------------------------------
// Shape-generic fallback: 64 x 64 tiles, operands straight from global memory.
// ---------------------------------------------------------------------------
constexpr int kGemmBN = 64;  // W rows per workgroup (32 gate/up pairs)
constexpr int kGemmBM = 64;  // tokens per workgroup

__global__ __launch_bounds__(256) void gemm_w8a8_swiglu_kernel(
    float* __restrict__ out, const int8_t* __restrict__ w, const float* __restrict__ scales,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int batch, int K, int inter) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n_tiles = (2 * inter) / kGemmBN;
  const int tile_n = blockIdx.x % n_tiles;
  const int tile_m = blockIdx.x / n_tiles;
  const int n0 = tile_n * kGemmBN + (wave & 1) * 32;
  const int m0 = tile_m * kGemmBM + (wave >> 1) * 32;
  const int r = lane & 15;
  const int g = lane >> 4;

  const int8_t* a_ptr[2];
  const int8_t* b_ptr[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    a_ptr[i] = w + (size_t)(n0 + 16 * i + r) * K + 16 * g;
    int m = m0 + 16 * i + r;
    m = m < batch ? m : batch - 1;  // padded tokens read a valid row; never stored
    b_ptr[i] = xq + (size_t)m * K + 16 * g;
  }

  v4i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  for (int k0 = 0; k0 < K; k0 += kGemmK) {
    v4i a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      a[i] = *reinterpret_cast<const v4i*>(a_ptr[i] + k0);
      b[i] = *reinterpret_cast<const v4i*>(b_ptr[i] + k0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
  }

#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int m = m0 + 16 * j + r;
    if (m >= batch) continue;
    const float xsm = xs[m];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int n = n0 + 16 * i + 4 * g;
      const int p = n >> 1;
      float2 o;
      o.x = swiglu_w8a8(acc[i][j][0], acc[i][j][1], xsm, scales[n], scales[n + 1]);
      o.y = swiglu_w8a8(acc[i][j][2], acc[i][j][3], xsm, scales[n + 2], scales[n + 3]);
      *reinterpret_cast<float2*>(out + (size_t)m * inter + p) = o;
    }
  }
}

inline bool gemm_w8a8_supported(size_t batch, size_t K, size_t inter) {
  return batch >= 1 && K % kGemmK == 0 && (2 * inter) % kGemmBN == 0;
}

inline bool gemm_w8a8_lds_shape(size_t K, size_t inter) {
  return (K == 1024 || K == 2048) && (2 * inter) % kLdsBN == 0;
}

// Raises kernel Fn's dynamic-LDS limit (64 KiB by default) to `bytes` on the
// current device. The attribute is per device, so the outcome is remembered
// per device (0 unknown, 1 set, -1 unavailable); concurrent first calls may
// both set it, which is harmless. Returns false if the device cannot give a
// workgroup that much LDS.
template <auto Fn>
bool raise_lds_limit(size_t bytes) {
  constexpr int kMaxDevices = 64;
  static std::atomic<signed char> state[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  const signed char known = state[dev].load(std::memory_order_acquire);
  if (known != 0) return known > 0;
  int max_lds = 0;
  const bool ok =
      hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
      (size_t)max_lds >= bytes &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(Fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) == hipSuccess;
  state[dev].store(ok ? 1 : -1, std::memory_order_release);
  return ok;
}

// The staged X tile needs up to 64 x 2064 bytes.
template <int KSTEPS>
bool lds_kernel_ready(size_t lds) {
  (void)lds;
  return raise_lds_limit<&gemm_w8a8_swiglu_lds_kernel<KSTEPS>>((size_t)kLdsBM * (kLdsMaxK + kLdsRowPad));
}

template <int KSTEPS>
bool launch_lds_gemm(float* out, const int8_t* w, const float* scales, const int8_t* xq,
                     const float* xs, int batch, int inter, int n_tiles, int m_tiles,
                     size_t lds, hipStream_t st) {
  if (!lds_kernel_ready<KSTEPS>(lds)) return false;
  gemm_w8a8_swiglu_lds_kernel<KSTEPS><<<(unsigned)(n_tiles * m_tiles), 256, lds, st>>>(
      out, w, scales, xq, xs, batch, inter, n_tiles, m_tiles);
  return true;
}

// Launches the LDS-staged kernel when the shape allows; returns false if it
// did not launch (shape or device LDS), leaving the choice to the caller.
inline bool try_lds_gemm(float* out, const int8_t* w, const float* scales, const int8_t* xq,
                  const float* xs, size_t batch, size_t K, size_t inter, hipStream_t st) {
  if (!gemm_w8a8_lds_shape(K, inter) || !aligned16(scales) ||
      (2 * inter / kLdsBN) * ((batch + kLdsBM - 1) / kLdsBM) > 0x7fffffffu) {
    return false;
  }
  const int n_tiles = (int)((2 * inter) / kLdsBN);
  const int m_tiles = (int)((batch + kLdsBM - 1) / kLdsBM);
  const size_t lds = (size_t)kLdsBM * (K + kLdsRowPad);
  if (K == 1024) {
    return launch_lds_gemm<16>(out, w, scales, xq, xs, (int)batch, (int)inter, n_tiles,
                                       m_tiles, lds, st);
  }
  return launch_lds_gemm<32>(out, w, scales, xq, xs, (int)batch, (int)inter, n_tiles,
                                     m_tiles, lds, st);
}

inline int gemm_w8a8_swiglu(float* out, const int8_t* w, const float* scales, const int8_t* xq,
                            const float* xs, size_t batch, size_t K, size_t inter,
                            hipStream_t st) {
  // Each lane stores two adjacent outputs as one float2; inter % 32 == 0 keeps
  // every row start 8-byte aligned once out is.
  if ((reinterpret_cast<uintptr_t>(out) & 7u) != 0) {
    return fail(QASR_ERR_INVALID_ARG, "gate_up_swiglu_w8a8: out must be 8-byte aligned");
  }
  if (try_lds_gemm(out, w, scales, xq, xs, batch, K, inter, st)) {
    return launch_status("gate_up_swiglu_w8a8 (mfma, lds)");
  }
  const size_t n_tiles = (2 * inter) / kGemmBN;
  const size_t m_tiles = (batch + kGemmBM - 1) / kGemmBM;
  const size_t grid = n_tiles * m_tiles;
  if (grid > 0x7fffffffu) return fail(QASR_ERR_INVALID_ARG, "gate_up_swiglu_w8a8: grid too large");
  gemm_w8a8_swiglu_kernel<<<(unsigned)grid, 256, 0, st>>>(out, w, scales, xq, xs, (int)batch,
                                                          (int)K, (int)inter);
  return launch_status("gate_up_swiglu_w8a8 (mfma)");
}

}  // namespace qasr

namespace qasr {

// Row-major [rows, cols] int8 -> MFMA tile layout (see packed_tile_offset).
// One thread moves one 16-byte lane slice.
__global__ __launch_bounds__(256) void pack_w8a8_tiles_kernel(int8_t* __restrict__ packed,
                                                              const int8_t* __restrict__ w,
                                                              size_t n_slices, int ksteps,
                                                              size_t cols) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n_slices;
       i += (size_t)gridDim.x * 256) {
    const int lane = (int)(i & 63);
    const size_t tile = i >> 6;
    const size_t rb = tile / (size_t)ksteps;
    const int s = (int)(tile - rb * ksteps);
    const size_t row = rb * kPackRows + (lane & 15);
    const size_t col = (size_t)s * kPackK + 16 * (lane >> 4);
    *reinterpret_cast<v4i*>(packed + i * 16) = *reinterpret_cast<const v4i*>(w + row * cols + col);
  }
}

// ---------------------------------------------------------------------------
// Packed-weight kernel: one 8-wave workgroup per CU, K split in two halves.
//
// A workgroup owns 192 W rows x 64 tokens. Wave w = 4*kq + rg owns row group
// rg (48 rows = 3 MFMA tiles of 16) for all 64 tokens (4 tiles, 12
// accumulators) over K half kq, so every W tile and every Xq slice is read
// once per workgroup, and two waves share each SIMD: a single wave cannot
// issue v_mfma_i32_16x16x64_i8 back to back at full rate, two interleaved
// waves can.
//
// Xq is staged in LDS in 16 KiB chunks of [64 rows][256 bytes] (4 k-steps);
// the 16-byte slot p of a row holds the row's logical slot p ^ (row & 15), so
// the b128 fragment reads of 16 rows at one k offset hit 16 distinct bank
// groups. Every chunk is loaded into registers in the prologue, the first
// chunk of each K half first; those two are written to LDS before the loop,
// so the first MFMA waits for 32 KiB of Xq instead of all of it, and chunk
// c + 1 of each half is written at step 4c + 1 and first read at step 4c + 4
// (a barrier at step 4c + 3). 256-byte chunks measured 0.2-0.4 us faster than
// 512-byte ones (bit-identical: int32 sums are exact in any order). Plain loads are used rather than the direct global->LDS form: the
// compiler cannot tell which LDS bytes a pending direct load writes, so it
// drains every outstanding load (the whole W window) at the first LDS read;
// with register staging its per-load waits stay exact. The workgroup barriers
// of the staging are bare s_barrier after lgkmcnt(0), since __syncthreads()
// would also wait for the outstanding W loads. W streams from the tile-packed
// layout straight into registers, PF k-steps ahead, with non-temporal loads;
// the per-row and per-token scales of the epilogue are loaded before the loop
// so their latency hides under it.
//
// After the loop the two waves of a row group exchange halves through LDS:
// wave kq keeps token tiles 2kq, 2kq+1, adds its partner's partial sums for
// them (exact int32) and runs the SwiGLU epilogue on them. The results are
// staged as a [64][96] fp32 tile in LDS and written with 16-byte stores, each
// token's 96 outputs (384 bytes) contiguous.
// ---------------------------------------------------------------------------
constexpr int kPkBN = 192;       // W rows per workgroup
constexpr int kPkBM = 64;        // tokens per workgroup
constexpr int kPkWaves = 8;      // 4 row groups x 2 K halves
constexpr int kPkChunk = 256;    // bytes of K per staged X chunk
constexpr int kPkPrefetch = 3;   // k-steps of W in flight per wave
constexpr size_t kPkLds = 131072;


// Wave `wave`'s share of X chunk c: 2 four-row groups t, each lane one 16-byte slot.
// Rows past the batch re-read row batch - 1 (valid memory); their results are
// never stored.
template <int K>
QASR_DEV const v4i* x_chunk_src(const int8_t* __restrict__ xq, int c, int t, int wave, int lane,
                                int m0, int batch) {
  const int d = wave * 2 + t;          // 4-row group: rows 4d .. 4d+3, 16 slots each
  const int row = 4 * d + (lane >> 4);
  const int slot = (lane & 15) ^ (row & 15);
  const int src_row = m0 + row < batch ? m0 + row : batch - 1;
  return reinterpret_cast<const v4i*>(xq + (size_t)src_row * K + kPkChunk * c + 16 * slot);
}
QASR_DEV v4i* x_chunk_dst(int8_t* lds, int c, int t, int wave, int lane) {
  return reinterpret_cast<v4i*>(lds + c * 16384 + (wave * 2 + t) * 1024 + 16 * lane);
}

template <int KS, bool VEC_OUT>  // KS = K / 64 (16 or 32)
__global__ __launch_bounds__(64 * kPkWaves) void gemm_w8a8_swiglu_packed_kernel(
    float* __restrict__ out, const int8_t* __restrict__ wpk, const float* __restrict__ scales,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int batch, int inter,
    int n_tiles, int m_tiles) {
  constexpr int K = KS * kPackK;
  constexpr int KW = KS / 2;                // k-steps per wave
  constexpr int NCH = K / kPkChunk;         // X chunks (4 or 8)
  constexpr int CH_HALF = NCH / 2;          // chunks per K half
  constexpr int PF = kPkPrefetch;
  static_assert(kPkWaves * 2 * 4 == 64, "a chunk is 64 rows: 8 waves x 2 four-row groups");
  extern __shared__ __align__(16) int8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = wave & 3, kq = wave >> 2;
  const int r = lane & 15, g = lane >> 4;

  // XCD-aware order: block b runs on XCD b % 8; the m_tiles blocks that share
  // a W tile go to the same XCD back to back, so 3 of 4 W reads hit its L2.
  const int b = blockIdx.x;
  int tile_n, tile_m;
  if (n_tiles % kNumXcd == 0) {
    const int slot = b / kNumXcd;
    tile_m = slot % m_tiles;
    tile_n = b % kNumXcd + kNumXcd * (slot / m_tiles);
  } else {
    tile_m = b % m_tiles;
    tile_n = b / m_tiles;
  }
  const int n_wave = tile_n * kPkBN + rg * 48;
  const int m0 = tile_m * kPkBM;
  const int k0 = kq * KW;

  // Issue order: first X chunks, W window, epilogue operands, second X
  // chunks; sched_barriers keep it (loads complete in issue order).
  v4i xa[4], xr[CH_HALF > 1 ? (CH_HALF - 1) * 4 : 1];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    xa[t] = *x_chunk_src<K>(xq, 0, t, wave, lane, m0, batch);
    xa[2 + t] = *x_chunk_src<K>(xq, CH_HALF, t, wave, lane, m0, batch);
  }
  __builtin_amdgcn_sched_barrier(0);

  const int8_t* wp = wpk + packed_tile_offset(n_wave / kPackRows, k0, KS) + 16 * lane;
  constexpr size_t ROW_TILE = (size_t)KS * 1024;
  v4i wbuf[PF][3];
#pragma unroll
  for (int d = 0; d < PF; ++d)
#pragma unroll
    for (int i = 0; i < 3; ++i)
      wbuf[d][i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + i * ROW_TILE + d * 1024));
  __builtin_amdgcn_sched_barrier(0);
  float4 sc[3];
  float xsv[2];
#pragma unroll
  for (int i = 0; i < 3; ++i) sc[i] = *reinterpret_cast<const float4*>(scales + n_wave + 16 * i + 4 * g);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int m = m0 + 16 * (2 * kq + jj) + r;
    xsv[jj] = xs[m < batch ? m : batch - 1];
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (CH_HALF > 1) {
#pragma unroll
    for (int c = 1; c < CH_HALF; ++c)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        xr[(c - 1) * 4 + t] = *x_chunk_src<K>(xq, c, t, wave, lane, m0, batch);
        xr[(c - 1) * 4 + 2 + t] = *x_chunk_src<K>(xq, CH_HALF + c, t, wave, lane, m0, batch);
      }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    *x_chunk_dst(lds, 0, t, wave, lane) = xa[t];
    *x_chunk_dst(lds, CH_HALF, t, wave, lane) = xa[2 + t];
  }
  lds_barrier();

  v4i acc[3][4];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

  // B fragment of token tile j at global k-step s
  auto xfrag = [&](int s, int j) -> v4i {
    const int c = s >> 2;
    const int slot = 4 * (s & 3) + g;
    return *reinterpret_cast<const v4i*>(lds + c * 16384 + (16 * j + r) * kPkChunk + 16 * (slot ^ r));
  };
  v4i bcur[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) bcur[j] = xfrag(k0, j);

#pragma unroll
  for (int s0 = 0; s0 < KW; s0 += PF) {
#pragma unroll
    for (int d = 0; d < PF; ++d) {
      const int s = s0 + d;
      if (s < KW) {
        if (CH_HALF > 1 && (s & 3) == 1 && (s >> 2) + 1 < CH_HALF) {  // the next chunk of each half into LDS
          const int c = (s >> 2) + 1;
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int cc = 1; cc < CH_HALF; ++cc)
            if (cc == c) {
#pragma unroll
              for (int t = 0; t < 2; ++t) {
                *x_chunk_dst(lds, cc, t, wave, lane) = xr[(cc - 1) * 4 + t];
                *x_chunk_dst(lds, CH_HALF + cc, t, wave, lane) = xr[(cc - 1) * 4 + 2 + t];
              }
            }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (CH_HALF > 1 && (s & 3) == 3 && (s >> 2) + 1 < CH_HALF) {  // step s+1 reads the next chunk
          __builtin_amdgcn_sched_barrier(0);
          lds_barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
        v4i a[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          a[i] = wbuf[d][i];
          if (s + PF < KW)
            wbuf[d][i] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(wp + i * ROW_TILE + (s + PF) * 1024));
        }
        // Keep the prefetch and the next B fragments issued here: without the
        // fences the scheduler sinks each load next to its use.
        __builtin_amdgcn_sched_barrier(0);
        v4i bn[4];
        if (s + 1 < KW) {
#pragma unroll
          for (int j = 0; j < 4; ++j) bn[j] = xfrag(k0 + s + 1, j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 3; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], bcur[j], acc[i][j], 0, 0, 0);
        if (s + 1 < KW) {
#pragma unroll
          for (int j = 0; j < 4; ++j) bcur[j] = bn[j];
        }
      }
    }
  }

  // Exchange K-half partial sums. Register arrays take constant indices only
  // (a runtime index would move acc to scratch memory).
  __syncthreads();  // X no longer read
  v4i give[3][2], mine[3][2];
  if (kq == 0) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) { give[i][jj] = acc[i][2 + jj]; mine[i][jj] = acc[i][jj]; }
  } else {
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) { give[i][jj] = acc[i][jj]; mine[i][jj] = acc[i][2 + jj]; }
  }
  v4i* ex = reinterpret_cast<v4i*>(lds);  // [rg][receiver kq][i][jj][lane]
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) ex[(((rg * 2 + (1 - kq)) * 3 + i) * 2 + jj) * 64 + lane] = give[i][jj];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) mine[i][jj] += ex[(((rg * 2 + kq) * 3 + i) * 2 + jj) * 64 + lane];

  // Epilogue: lane holds W rows n_wave + 16i + 4g + {0..3} (two gate/up pairs)
  // for token m0 + 16*(2kq + jj) + r. The output tile is staged past the
  // exchange area (no barrier needed between them) with a row pitch of 100
  // floats: at 96 the 16 tokens of one write instruction would share a bank.
  if constexpr (VEC_OUT) {
    constexpr int OP = 100;  // staged row pitch (floats)
    float* ot = reinterpret_cast<float*>(lds + 65536);  // [64 tokens][OP]
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int t = 16 * (2 * kq + jj) + r;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        float2 o;
        o.x = swiglu_w8a8(mine[i][jj][0], mine[i][jj][1], xsv[jj], sc[i].x, sc[i].y);
        o.y = swiglu_w8a8(mine[i][jj][2], mine[i][jj][3], xsv[jj], sc[i].z, sc[i].w);
        *reinterpret_cast<float2*>(ot + t * OP + rg * 24 + 8 * i + 2 * g) = o;
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kPkBM * 24 / (64 * kPkWaves); ++t) {
      const int q = t * 64 * kPkWaves + threadIdx.x;
      const int row = q / 24, c4 = q - row * 24;
      const int m = m0 + row;
      if (m < batch)
        __builtin_nontemporal_store(*reinterpret_cast<const v4f*>(ot + row * OP + 4 * c4),
                                    reinterpret_cast<v4f*>(out + (size_t)m * inter + tile_n * 96 + 4 * c4));
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int m = m0 + 16 * (2 * kq + jj) + r;
      if (m >= batch) continue;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const int n = n_wave + 16 * i + 4 * g;
        float2 o;
        o.x = swiglu_w8a8(mine[i][jj][0], mine[i][jj][1], xsv[jj], sc[i].x, sc[i].y);
        o.y = swiglu_w8a8(mine[i][jj][2], mine[i][jj][3], xsv[jj], sc[i].z, sc[i].w);
        *reinterpret_cast<float2*>(out + (size_t)m * inter + (n >> 1)) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 96 x 128 tile (batch > 128). A workgroup owns 96 W rows x 128 tokens, so a CU
// reads 192 KiB of W and 256 KiB of Xq: 448 KiB against the 192 x 64 tile's
// 384 + 128 = 512 KiB. The 2 workgroups of a W tile sit on one XCD.
//
// Three MFMA waves each own two 16-row blocks over all 8 token tiles and the
// whole K: every W byte is loaded by one wave, each B fragment read from LDS
// feeds two MFMAs, and no partial sums change hands. The Xq tile (256 KiB) does
// not fit in LDS: two loader waves stream it in 32 KiB chunks (4 k-steps x 128
// tokens) through a ring of 3, with direct global->LDS loads. Each chunk is one
// barrier: barrier c means chunk c has landed and every MFMA wave is done with
// chunk c - 1, whose slot then takes chunk c + 2. A loader waits on its own
// loads (vmcnt) before each barrier. The MFMA waves issue no direct LDS load,
// so the compiler puts no drain of their W prefetch in front of their LDS
// reads, and their barrier waits on LDS only.
//
// Chunk layout: token row t of a chunk is 256 bytes (16 slots of 16 bytes), and
// LDS slot l of row t holds the row's data slot l ^ (t & 15), so the 16 tokens
// of one B-fragment read hit 16 different bank groups. The SwiGLU epilogue is
// the 192-row kernel's; results equal it bit for bit (int32 sums are exact).
//
// Measured at [256,2048] x [2048,12288]: 11.45 us against 12.1 us for the
// 192 x 64 tile. Timing-only copies put 1.25 us on the W loads, 1.7 us on the
// Xq loads, ~1 us on the MFMAs (the busiest SIMD issues a third of them: 6
// row blocks do not split over 4 SIMDs without loading W twice; most of their
// 3.4 us hides under the loads) and 0.65 us on the SwiGLU arithmetic; the rest
// is the launch, the wait for the first chunk and the stores.
// ---------------------------------------------------------------------------
constexpr int kT9BN = 96;                                // W rows per workgroup
constexpr int kT9BM = 128;                               // tokens per workgroup
constexpr int kT9BlocksPerWave = 2;                      // 16-row blocks per MFMA wave
constexpr int kT9MfmaWaves = kT9BN / kPackRows / kT9BlocksPerWave;
constexpr int kT9Loaders = 2;                            // loader waves
constexpr int kT9Waves = kT9MfmaWaves + kT9Loaders;
constexpr int kT9Ring = 3;                               // chunk slots
constexpr int kT9ChunkBytes = kT9BM * kPkChunk;          // 32 KiB
constexpr int kT9PiecesPerLoader = kT9ChunkBytes / 1024 / kT9Loaders;  // 1 KiB direct loads per chunk
constexpr size_t kT9Lds = (size_t)kT9Ring * kT9ChunkBytes;
constexpr int kT9Prefetch = 3;                           // k-steps of W in flight per MFMA wave
constexpr int kT9OutPitch = 52;                          // staged output row pitch (floats)

template <int KS>  // KS = K / 64 (16 or 32)
__global__ __launch_bounds__(64 * kT9Waves) void gemm_w8a8_swiglu_t96_kernel(
    float* __restrict__ out, const int8_t* __restrict__ wpk, const float* __restrict__ scales,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int batch, int inter,
    int n_tiles, int m_tiles) {
  constexpr int K = KS * kPackK;
  constexpr int NCH = K / kPkChunk;          // chunks (8 or 4)
  constexpr int SPC = kPkChunk / kPackK;     // k-steps per chunk (4)
  constexpr int PF = kT9Prefetch;
  constexpr int RB = kT9BlocksPerWave;
  static_assert(NCH >= kT9Ring - 1 && kT9Ring >= 2 && kT9Ring <= 4 &&
                    kT9PiecesPerLoader * 1024 * kT9Loaders == kT9ChunkBytes &&
                    (kT9Ring - 2) * kT9PiecesPerLoader <= 63,
                "ring schedule: the chunks outstanding behind the one waited for fit vmcnt");
  static_assert(kT9BM * kT9OutPitch * 4 <= (int)kT9Lds, "output staging fits the ring");
  extern __shared__ __align__(16) int8_t lds[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;

  // Block b runs on XCD b % 8; the m_tiles blocks of one W tile share an XCD.
  const int b = blockIdx.x;
  int tile_n, tile_m;
  if (n_tiles % kNumXcd == 0) {
    const int slot = b / kNumXcd;
    tile_m = slot % m_tiles;
    tile_n = b % kNumXcd + kNumXcd * (slot / m_tiles);
  } else {
    tile_m = b % m_tiles;
    tile_n = b / m_tiles;
  }
  const int m0 = tile_m * kT9BM;

  v4i acc[RB][8];
  float4 sc[RB];
  float xsv[8];
  if (wave >= kT9MfmaWaves) {
    // Loader: 1 KiB piece p of a chunk is token rows 4p .. 4p + 3; lane l fills
    // LDS slot l & 15 of row 4p + l / 16. Rows past the batch re-read row
    // batch - 1 (valid memory); their results are never stored.
    const int pw = wave - kT9MfmaWaves;
    auto issue = [&](int c) {
      int8_t* slot_base = lds + (c % kT9Ring) * kT9ChunkBytes;
#pragma unroll
      for (int i = 0; i < kT9PiecesPerLoader; ++i) {
        const int piece = kT9PiecesPerLoader * pw + i;
        const int row = 4 * piece + (lane >> 4);
        const int data_slot = (lane & 15) ^ (row & 15);
        const int src_row = m0 + row < batch ? m0 + row : batch - 1;
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(xq + (size_t)src_row * K + kPkChunk * c + 16 * data_slot),
            (__attribute__((address_space(3))) void*)(slot_base + piece * 1024), 16, 0, 0);
      }
    };
    constexpr int AHEAD = kT9Ring - 1;  // chunks issued beyond the one being read
#pragma unroll
    for (int c = 0; c < AHEAD; ++c) issue(c);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // chunk c has landed once at most the chunks issued after it are outstanding
      const int after = (c + AHEAD - 1 < NCH - 1 ? c + AHEAD - 1 : NCH - 1) - c;
      if (after >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_at_most(2 * kT9PiecesPerLoader));
      else if (after == 1) __builtin_amdgcn_s_waitcnt(vmcnt_at_most(kT9PiecesPerLoader));
      else __builtin_amdgcn_s_waitcnt(vmcnt_at_most(0));
      asm volatile("s_barrier" ::: "memory");
      // into the slot of chunk c - 1, which every MFMA wave has left
      if (c + AHEAD < NCH) issue(c + AHEAD);
    }
  } else {
    const int rb0 = tile_n * (kT9BN / kPackRows) + RB * wave;  // this wave's first 16-row block
    const int8_t* wp = wpk + packed_tile_offset(rb0, 0, KS) + 16 * lane;
    constexpr size_t ROW_TILE = (size_t)KS * 1024;
    v4i wbuf[PF][RB];
#pragma unroll
    for (int d = 0; d < PF; ++d)
#pragma unroll
      for (int i = 0; i < RB; ++i)
        wbuf[d][i] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wp + i * ROW_TILE + d * 1024));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RB; ++i) sc[i] = *reinterpret_cast<const float4*>(scales + 16 * (rb0 + i) + 4 * g);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int m = m0 + 16 * j + r;
      xsv[j] = xs[m < batch ? m : batch - 1];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // B fragment of token tile j at k-step s
    auto bfrag = [&](int s, int j) -> v4i {
      const int slot = SPC * (s % SPC) + g;
      return *reinterpret_cast<const v4i*>(lds + ((s / SPC) % kT9Ring) * kT9ChunkBytes +
                                           (16 * j + r) * kPkChunk + 16 * (slot ^ r));
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      lds_barrier();  // chunk c is in LDS; chunk c - 1's slot is released
      v4i bcur[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) bcur[j] = bfrag(SPC * c, j);
#pragma unroll
      for (int q = 0; q < SPC; ++q) {
        const int s = SPC * c + q;
        v4i a[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          a[i] = wbuf[s % PF][i];
          if (s + PF < KS)
            wbuf[s % PF][i] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(wp + i * ROW_TILE + (s + PF) * 1024));
        }
        // keep the prefetch and the next B fragments issued here (the
        // scheduler would otherwise sink each load next to its use)
        __builtin_amdgcn_sched_barrier(0);
        v4i bn[8];
        if (q + 1 < SPC) {
#pragma unroll
          for (int j = 0; j < 8; ++j) bn[j] = bfrag(s + 1, j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int i = 0; i < RB; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], bcur[j], acc[i][j], 0, 0, 0);
        if (q + 1 < SPC) {
#pragma unroll
          for (int j = 0; j < 8; ++j) bcur[j] = bn[j];
        }
      }
    }
  }

  // Epilogue: MFMA wave w, lane (r, g), block i holds W rows 16 rb + 4g + {0..3}
  // (rb = 6 tile_n + RB w + i: two gate/up pairs, outputs 48 tile_n + 8 (RB w + i)
  // + 2g + {0, 1}) for tokens m0 + 16j + r. Staged as a [128][52] fp32 tile over
  // the ring, then written with 16-byte stores, each token's 48 outputs (192
  // bytes) contiguous.
  lds_barrier();  // every X read is done (MFMA waves) and every load has landed (loaders)
  float* ot = reinterpret_cast<float*>(lds);
  if (wave < kT9MfmaWaves) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float2 o;
        o.x = swiglu_w8a8(acc[i][j][0], acc[i][j][1], xsv[j], sc[i].x, sc[i].y);
        o.y = swiglu_w8a8(acc[i][j][2], acc[i][j][3], xsv[j], sc[i].z, sc[i].w);
        *reinterpret_cast<float2*>(ot + (16 * j + r) * kT9OutPitch + 8 * (RB * wave + i) + 2 * g) = o;
      }
  }
  lds_barrier();
  constexpr int V4_PER_ROW = kT9BN / 2 / 4;  // 12
  constexpr int NV4 = kT9BM * V4_PER_ROW;
#pragma unroll
  for (int t = 0; t < (NV4 + 64 * kT9Waves - 1) / (64 * kT9Waves); ++t) {
    const int q = t * 64 * kT9Waves + threadIdx.x;
    const int row = q / V4_PER_ROW, c4 = q - row * V4_PER_ROW;
    const int m = m0 + row;
    if (q < NV4 && m < batch)
      __builtin_nontemporal_store(*reinterpret_cast<const v4f*>(ot + row * kT9OutPitch + 4 * c4),
                                  reinterpret_cast<v4f*>(out + (size_t)m * inter + tile_n * (kT9BN / 2) + 4 * c4));
  }
}

// ---------------------------------------------------------------------------
// Small-batch packed kernel (batch <= 64): one 8-wave workgroup per 48 W rows.
//
// With a single 64-token tile the 192-row kernel launches only 2*inter/192
// workgroups (64 at the 1.7B shape, a quarter of the CUs). Here a workgroup
// owns 48 rows x all tokens and wave w owns k-steps [w*KW, (w+1)*KW) (KW =
// K/64/8): its W tiles and X fragments go straight to registers (every W and
// X byte is loaded once per workgroup, no LDS staging), its 12 accumulators
// are int32 partial sums over its K slice, and the 8 partials of each
// accumulator tile are added in LDS (exact) by the wave that runs that tile's
// SwiGLU epilogue -- the same epilogue, so the outputs equal the 192-row
// kernel's bit for bit. The epilogue's token and row scales are loaded with
// the operands, not after the partial-sum barrier (a dependent memory round
// trip on the tail: B=32 9.27 -> 8.87 us).
// ---------------------------------------------------------------------------
constexpr int kSbRows = 48;
constexpr int kSbWaves = 8;
constexpr size_t kSbLds = (size_t)kSbWaves * 12 * 64 * 16;  // 96 KiB of partial sums

template <int KS>
__global__ __launch_bounds__(64 * kSbWaves) void gemm_w8a8_swiglu_small_kernel(
    float* __restrict__ out, const int8_t* __restrict__ wpk, const float* __restrict__ scales,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int batch, int inter) {
  constexpr int KW = KS / kSbWaves;
  constexpr int K = KS * kPackK;
  extern __shared__ __align__(16) int8_t lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * kSbRows;
  const int s0 = wave * KW;

  v4i wv[KW][3], xv[KW][4];
  const int8_t* wp = wpk + 16 * lane;
#pragma unroll
  for (int s = 0; s < KW; ++s)
#pragma unroll
    for (int i = 0; i < 3; ++i)
      wv[s][i] = __builtin_nontemporal_load(
          reinterpret_cast<const v4i*>(wp + packed_tile_offset(n0 / kPackRows + i, s0 + s, KS)));
  // token tiles past the batch are neither loaded nor multiplied (uniform tests)
#pragma unroll
  for (int s = 0; s < KW; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = 16 * j + r;
      const int row = m < batch ? m : batch - 1;  // rows past the batch: valid memory, dropped
      xv[s][j] = v4i{0, 0, 0, 0};
      if (16 * j < batch)
        xv[s][j] = *reinterpret_cast<const v4i*>(xq + (size_t)row * K + kPackK * (s0 + s) + 16 * g);
    }
  // the epilogue's scales for this wave's tiles (wave and wave + 8), loaded with the operands
  float ep_xs[2];
  float4 ep_sc[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int t = wave + kSbWaves * e;
    const int i = (t < 12 ? t : 0) >> 2, j = (t < 12 ? t : 0) & 3;
    const int m = 16 * j + r;
    ep_xs[e] = xs[m < batch ? m : batch - 1];
    ep_sc[e] = *reinterpret_cast<const float4*>(scales + n0 + 16 * i + 4 * g);
  }
  __builtin_amdgcn_sched_barrier(0);
  v4i acc[3][4];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KW; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (16 * j < batch) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[s][i], xv[s][j], acc[i][j], 0, 0, 0);
      }

  v4i* part = reinterpret_cast<v4i*>(lds);  // [wave][tile 4i + j][lane]
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) part[(wave * 12 + 4 * i + j) * 64 + lane] = acc[i][j];
  __syncthreads();
  // wave w finishes accumulator tiles w and w + 8: lane holds W rows
  // n0 + 16i + 4g + {0..3} (two gate/up pairs) for token 16j + r
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int t = wave + kSbWaves * e;
    if (t >= 12) break;
    const int i = t >> 2, j = t & 3;
    if (16 * j >= batch) continue;
    v4i sum = part[t * 64 + lane];
#pragma unroll
    for (int u = 1; u < kSbWaves; ++u) sum += part[(u * 12 + t) * 64 + lane];
    const int m = 16 * j + r;
    if (m < batch) {
      const float xsv = ep_xs[e];
      const int n = n0 + 16 * i + 4 * g;
      const float4 sc = ep_sc[e];
      float2 o;
      o.x = swiglu_w8a8(sum[0], sum[1], xsv, sc.x, sc.y);
      o.y = swiglu_w8a8(sum[2], sum[3], xsv, sc.z, sc.w);
      *reinterpret_cast<float2*>(out + (size_t)m * inter + (n >> 1)) = o;
    }
  }
}

template <int KS>
bool small_kernel_ready() {
  return raise_lds_limit<&gemm_w8a8_swiglu_small_kernel<KS>>(kSbLds);
}

inline bool packed_gemm_shape(size_t K, size_t inter) {
  return (K == 1024 || K == 2048) && (2 * inter) % kPkBN == 0;
}

template <int KS>
bool t96_kernel_ready() {
  return raise_lds_limit<&gemm_w8a8_swiglu_t96_kernel<KS>>(kT9Lds);
}

template <int KS, bool VEC_OUT>
bool packed_kernel_ready() {
  return raise_lds_limit<&gemm_w8a8_swiglu_packed_kernel<KS, VEC_OUT>>(kPkLds);
}

template <int KS, bool VEC_OUT>
bool launch_packed(float* out, const int8_t* wpk, const float* scales, const int8_t* xq,
                   const float* xs, int batch, int inter, int n_tiles, int m_tiles, hipStream_t st) {
  if (!packed_kernel_ready<KS, VEC_OUT>()) return false;
  gemm_w8a8_swiglu_packed_kernel<KS, VEC_OUT><<<(unsigned)(n_tiles * m_tiles), 64 * kPkWaves, kPkLds, st>>>(
      out, wpk, scales, xq, xs, batch, inter, n_tiles, m_tiles);
  return true;
}

// Launches the packed-weight kernel; returns false if the shape or the device
// LDS does not allow it (nothing launched). 16-byte aligned outputs take the
// LDS-staged 16-byte store path.
inline bool try_packed_gemm(float* out, const int8_t* wpk, const float* scales, const int8_t* xq,
                            const float* xs, size_t batch, size_t K, size_t inter, hipStream_t st) {
  if (!packed_gemm_shape(K, inter)) return false;
  const size_t n_tiles = 2 * inter / kPkBN, m_tiles = (batch + kPkBM - 1) / kPkBM;
  if (n_tiles * m_tiles > 0x7fffffffu) return false;
  const bool vec = aligned16(out);
  const int B = (int)batch, I = (int)inter, NT = (int)n_tiles, MT = (int)m_tiles;
  if (batch <= 64 && (2 * inter) % kSbRows == 0) {  // one token tile: 48-row workgroups
    const unsigned grid = (unsigned)(2 * inter / kSbRows);
    if (K == 1024 && small_kernel_ready<16>()) {
      gemm_w8a8_swiglu_small_kernel<16><<<grid, 64 * kSbWaves, kSbLds, st>>>(out, wpk, scales, xq, xs, B, I);
      return true;
    }
    if (K == 2048 && small_kernel_ready<32>()) {
      gemm_w8a8_swiglu_small_kernel<32><<<grid, 64 * kSbWaves, kSbLds, st>>>(out, wpk, scales, xq, xs, B, I);
      return true;
    }
  }
  if (vec && batch > (size_t)kT9BM && (2 * inter) % kT9BN == 0) {  // two or more 128-token tiles
    const size_t nt = 2 * inter / kT9BN, mt = (batch + kT9BM - 1) / kT9BM;
    if (nt * mt <= 0x7fffffffu) {
      if (K == 1024 && t96_kernel_ready<16>()) {
        gemm_w8a8_swiglu_t96_kernel<16><<<(unsigned)(nt * mt), 64 * kT9Waves, kT9Lds, st>>>(
            out, wpk, scales, xq, xs, B, I, (int)nt, (int)mt);
        return true;
      }
      if (K == 2048 && t96_kernel_ready<32>()) {
        gemm_w8a8_swiglu_t96_kernel<32><<<(unsigned)(nt * mt), 64 * kT9Waves, kT9Lds, st>>>(
            out, wpk, scales, xq, xs, B, I, (int)nt, (int)mt);
        return true;
      }
    }
  }
  if (K == 1024)
    return vec ? launch_packed<16, true>(out, wpk, scales, xq, xs, B, I, NT, MT, st)
               : launch_packed<16, false>(out, wpk, scales, xq, xs, B, I, NT, MT, st);
  return vec ? launch_packed<32, true>(out, wpk, scales, xq, xs, B, I, NT, MT, st)
             : launch_packed<32, false>(out, wpk, scales, xq, xs, B, I, NT, MT, st);
}

}  // namespace qasr
