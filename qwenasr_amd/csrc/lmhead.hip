// lm_head argmax: the greedy-decode token choice at the end of every decode
// step (decoder.rs:929-963): logits = W8A32 matvec of the final hidden state,
// then the index of the largest logit.
//
// The reference scans the logits in order with a strict `>` starting from
// element 0, so the first maximum wins, a NaN never replaces the running
// best, and a NaN in element 0 is never replaced (result 0). The parallel
// scan here keeps, per thread and then per wave and workgroup, the best
// non-NaN (value, index) with ties going to the lower index, and returns 0
// when element 0 is NaN -- the same index as the sequential loop for every
// input.
#include "common.hpp"

#include <climits>

namespace qasr {
namespace {

QASR_DEV bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

QASR_DEV void consider(float v, int i, float& bv, int& bi) {
  if (v == v && better(v, i, bv, bi)) {  // v == v: NaN never wins
    bv = v;
    bi = i;
  }
}

constexpr int kArgmaxBlock = 1024;

template <bool VEC>
__global__ __launch_bounds__(kArgmaxBlock) void argmax_rows_kernel(int32_t* idx, const float* x,
                                                                   int cols) {
  __shared__ float sv[kArgmaxBlock / kWave];
  __shared__ int si[kArgmaxBlock / kWave];
  const float* row = x + (size_t)blockIdx.x * (size_t)cols;
  float bv = -__builtin_inff();
  int bi = INT_MAX;
  if constexpr (VEC) {
    const int c4 = cols >> 2;
    for (int c = threadIdx.x; c < c4; c += kArgmaxBlock) {
      const float4 v = ld4(row, c);
      consider(v.x, 4 * c, bv, bi);
      consider(v.y, 4 * c + 1, bv, bi);
      consider(v.z, 4 * c + 2, bv, bi);
      consider(v.w, 4 * c + 3, bv, bi);
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += kArgmaxBlock) consider(row[c], c, bv, bi);
  }
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  if (lane == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kArgmaxBlock / kWave; ++k)
      if (better(sv[k], si[k], bv, bi)) {
        bv = sv[k];
        bi = si[k];
      }
    const float first = row[0];
    // element 0 NaN: the reference's running best stays NaN at index 0;
    // a row of NaN and -inf only: bi is the first -inf, or INT_MAX if all NaN
    idx[blockIdx.x] = (first != first || bi == INT_MAX) ? 0 : bi;
  }
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_argmax_rows_f32(int32_t* idx, const float* x, size_t rows, size_t cols,
                                    void* stream) {
  if (rows == 0) return QASR_OK;
  QASR_REQUIRE(idx && x, "argmax_rows: null pointer");
  QASR_REQUIRE(cols > 0 && cols <= 0x7fffffffu, "argmax_rows: cols must be in [1, 2^31)");
  QASR_REQUIRE(rows <= kMaxRows, "argmax_rows: too many rows");
  size_t n;
  QASR_REQUIRE(mul_ok(rows, cols, &n), "argmax_rows: size overflows");
  hipStream_t st = as_stream(stream);
  if (cols % 4 == 0 && aligned16(x))
    argmax_rows_kernel<true><<<(unsigned)rows, kArgmaxBlock, 0, st>>>(idx, x, (int)cols);
  else
    argmax_rows_kernel<false><<<(unsigned)rows, kArgmaxBlock, 0, st>>>(idx, x, (int)cols);
  return launch_status("argmax_rows");
}

extern "C" int qasr_lm_head_int8_argmax_f32(int32_t* idx, float* logits, const float* x,
                                            const int8_t* w, const float* scales, size_t rows,
                                            size_t in_dim, size_t vocab, void* stream) {
  if (rows == 0) return QASR_OK;
  QASR_REQUIRE(idx && logits, "lm_head_int8_argmax: null pointer");
  QASR_REQUIRE(vocab > 0, "lm_head_int8_argmax: vocab must be positive");
  const int rc = qasr_linear_nobias_int8_f32(logits, x, w, scales, rows, in_dim, vocab, stream);
  if (rc != QASR_OK) return rc;
  return qasr_argmax_rows_f32(idx, logits, rows, vocab, stream);
}
