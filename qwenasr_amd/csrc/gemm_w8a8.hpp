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
// D[4*(l/16) + v][l % 16], v = 0..3. The exact k order inside a group does not
// matter as long as A and B use the same one, which they do: lane l loads bytes
// [k0 + 16*(l/16), +16) of its W row and of its Xq row. With A = W and B = Xq^T a
// lane's four results are four consecutive W rows for one token -- two complete
// gate/up pairs -- so the SwiGLU epilogue needs no data exchange.
#pragma once

#include "common.hpp"

namespace qasr {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmBN = 64;  // W rows per workgroup (32 gate/up pairs)
constexpr int kGemmBM = 64;  // tokens per workgroup
constexpr int kGemmK = 64;   // k per MFMA

// Workgroup = 4 waves in a 2x2 layout; each wave owns 32 W rows x 32 tokens =
// 2 x 2 MFMA tiles. Operands come straight from global memory (the W slice is
// shared with the neighbouring wave through L1/L2).
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

  // Epilogue: lane holds rows n0 + 16i + 4g + {0,1,2,3} for token m0 + 16j + r.
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
      {
        const float gg = ((float)acc[i][j][0] * xsm) * scales[n];
        const float uu = ((float)acc[i][j][1] * xsm) * scales[n + 1];
        o.x = (gg / (1.0f + expf(-gg))) * uu;
      }
      {
        const float gg = ((float)acc[i][j][2] * xsm) * scales[n + 2];
        const float uu = ((float)acc[i][j][3] * xsm) * scales[n + 3];
        o.y = (gg / (1.0f + expf(-gg))) * uu;
      }
      *reinterpret_cast<float2*>(out + (size_t)m * inter + p) = o;
    }
  }
}

inline bool gemm_w8a8_supported(size_t batch, size_t K, size_t inter) {
  return batch >= 1 && K % kGemmK == 0 && (2 * inter) % kGemmBN == 0;
}

inline int gemm_w8a8_swiglu(float* out, const int8_t* w, const float* scales, const int8_t* xq,
                            const float* xs, size_t batch, size_t K, size_t inter,
                            hipStream_t st) {
  // Each lane stores two adjacent outputs as one float2; inter % 32 == 0 keeps
  // every row start 8-byte aligned once out is.
  if ((reinterpret_cast<uintptr_t>(out) & 7u) != 0) {
    return fail(QASR_ERR_INVALID_ARG, "gate_up_swiglu_w8a8: out must be 8-byte aligned");
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
