// lm_head argmax: the greedy-decode token choice at the end of every decode
// step (decoder.rs:929-963): logits = W8A32 matvec of the final hidden state,
// then the index of the largest logit.
//
// The reference scans the logits in order with a strict `>` starting from
// element 0, so the first maximum wins, a NaN never replaces the running
// best, and a NaN in element 0 is never replaced (result 0). The parallel
// scans here keep the best non-NaN (value, index) with ties going to the
// lower index (argmax_better in common.hpp) and return 0 when element 0 is
// NaN -- the same index as the sequential loop for every input.
//
// One token (the decode step): the matvec kernel reduces each workgroup's
// rows to one (value, index) pair in a caller workspace, and one workgroup
// merges the pairs, so the logits are not read a second time. Otherwise the
// logits are written first and scanned by one workgroup per row.
#include "common.hpp"

#include <atomic>
#include <climits>
#include <mutex>

namespace qasr {
namespace {

constexpr int kArgmaxBlock = 1024;
constexpr int kArgmaxLoads = 8;  // loads in flight per thread

QASR_DEV void block_argmax(float& bv, int& bi) {
  __shared__ float sv[kArgmaxBlock / kWave];
  __shared__ int si[kArgmaxBlock / kWave];
#pragma unroll
  for (int m = kWave / 2; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m, kWave);
    const int oi = __shfl_xor(bi, m, kWave);
    if (argmax_better(ov, oi, bv, bi)) {
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
      if (argmax_better(sv[k], si[k], bv, bi)) {
        bv = sv[k];
        bi = si[k];
      }
  }
}

// element 0 NaN: the reference's running best stays NaN at index 0; a row of
// NaN only leaves bi == INT_MAX
QASR_DEV int32_t argmax_result(float first, int bi) {
  return (first != first || bi == INT_MAX) ? 0 : bi;
}

template <bool VEC>
__global__ __launch_bounds__(kArgmaxBlock) void argmax_rows_kernel(int32_t* idx, const float* x,
                                                                   int cols) {
  const float* row = x + (size_t)blockIdx.x * (size_t)cols;
  float bv = -__builtin_inff();
  int bi = INT_MAX;
  if constexpr (VEC) {
    const int c4 = cols >> 2;
    for (int c = threadIdx.x; c < c4; c += kArgmaxBlock * kArgmaxLoads) {
      float4 v[kArgmaxLoads];
#pragma unroll
      for (int k = 0; k < kArgmaxLoads; ++k) {
        const int ck = c + k * kArgmaxBlock;
        v[k] = ck < c4 ? ld4(row, ck) : make_float4(__int_as_float(0x7fc00000), 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int k = 0; k < kArgmaxLoads; ++k) {
        const int ck = c + k * kArgmaxBlock;
        if (ck < c4) {
          argmax_consider(v[k].x, 4 * ck, bv, bi);
          argmax_consider(v[k].y, 4 * ck + 1, bv, bi);
          argmax_consider(v[k].z, 4 * ck + 2, bv, bi);
          argmax_consider(v[k].w, 4 * ck + 3, bv, bi);
        }
      }
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += kArgmaxBlock) argmax_consider(row[c], c, bv, bi);
  }
  block_argmax(bv, bi);
  if (threadIdx.x == 0) idx[blockIdx.x] = argmax_result(row[0], bi);
}

// Merges n (value, index bits) pairs; values are never NaN.
__global__ __launch_bounds__(kArgmaxBlock) void argmax_partials_kernel(int32_t* idx,
                                                                       const float2* part, int n,
                                                                       const float* logits) {
  float bv = -__builtin_inff();
  int bi = INT_MAX;
  for (int c = threadIdx.x; c < n; c += kArgmaxBlock * kArgmaxLoads) {
    float2 p[kArgmaxLoads];
#pragma unroll
    for (int k = 0; k < kArgmaxLoads; ++k) {
      const int ck = c + k * kArgmaxBlock;
      p[k] = ck < n ? part[ck] : make_float2(-__builtin_inff(), __int_as_float(INT_MAX));
    }
#pragma unroll
    for (int k = 0; k < kArgmaxLoads; ++k) {
      const int pi = __float_as_int(p[k].y);
      if (argmax_better(p[k].x, pi, bv, bi)) {
        bv = p[k].x;
        bi = pi;
      }
    }
  }
  block_argmax(bv, bi);
  if (threadIdx.x == 0) idx[0] = argmax_result(logits[0], bi);
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_argmax_rows_f32(int32_t* idx, const float* x, size_t rows, size_t cols,
                                    void* stream) {
  if (rows == 0) return QASR_OK;
  QASR_REQUIRE(idx && x, "argmax_rows: null pointer");
  QASR_REQUIRE(cols > 0 && cols <= 0x7fffffffu - kArgmaxBlock * kArgmaxLoads * 4,
               "argmax_rows: cols must be in [1, 2^31 - 32768)");
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

extern "C" size_t qasr_lm_head_argmax_workspace_bytes(size_t vocab) {
  return lm_head_partials_max(vocab) * sizeof(float2);
}

extern "C" int qasr_lm_head_int8_argmax_f32(int32_t* idx, float* logits, const float* x,
                                            const int8_t* w, const float* scales, size_t rows,
                                            size_t in_dim, size_t vocab, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  if (rows == 0) return QASR_OK;
  QASR_REQUIRE(idx && logits && x && w && scales, "lm_head_int8_argmax: null pointer");
  QASR_REQUIRE(vocab > 0, "lm_head_int8_argmax: vocab must be positive");
  QASR_REQUIRE(!workspace || (reinterpret_cast<uintptr_t>(workspace) & 7u) == 0,
               "lm_head_int8_argmax: workspace must be 8-byte aligned");
  if (rows == 1 && workspace) {
    hipStream_t st = as_stream(stream);
    unsigned n_part = 0;
    if (launch_w8a32_argmax_partials(logits, x, w, scales, in_dim, vocab,
                                     static_cast<float2*>(workspace),
                                     workspace_bytes / sizeof(float2), st, &n_part)) {
      int rc = launch_status("lm_head_int8_argmax");
      if (rc != QASR_OK) return rc;
      argmax_partials_kernel<<<1, kArgmaxBlock, 0, st>>>(idx, static_cast<const float2*>(workspace),
                                                         (int)n_part, logits);
      return launch_status("lm_head_int8_argmax");
    }
  }
  const int rc = qasr_linear_nobias_int8_f32(logits, x, w, scales, rows, in_dim, vocab, stream);
  if (rc != QASR_OK) return rc;
  return qasr_argmax_rows_f32(idx, logits, rows, vocab, stream);
}

// ---------------------------------------------------------------------------
// No-allocation variant: the per-workgroup candidates live in a file-scope
// device array instead of a caller workspace, for callers that cannot
// allocate (code under HIP graph capture, serving loops that forbid
// hipMalloc). Each GPU the library runs on holds its own copy of the array
// (512 KiB) until the process ends. The array's address differs per device
// and is only known to the runtime, so it is looked up once per device
// (hipGetSymbolAddress with that device current) and the device pointer --
// never the host-side name of the array -- is what the kernels receive.
// Every workgroup writes its candidate before the merge reads it, so nothing
// needs clearing between calls. Calls on one GPU share the array: calls that
// overlap in time on one GPU (two streams, two threads) race.
// ---------------------------------------------------------------------------
namespace qasr {
namespace {

// one candidate per matvec workgroup, at most one per 4 vocabulary rows
constexpr size_t kNoAllocPairs = QASR_LM_HEAD_NOALLOC_MAX_VOCAB / 4;
static __device__ __align__(256) float2 scratch[kNoAllocPairs];

constexpr int kMaxScratchDevices = 64;
std::atomic<float2*> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// The current device's copy of `scratch`, looked up on its first use.
int scratch_for_current_device(float2** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(QASR_ERR_HIP, "lm_head_int8_argmax_noalloc: no current device (or more than 64)");
  float2* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !addr)
        return fail(QASR_ERR_HIP, std::string("lm_head_int8_argmax_noalloc: hipGetSymbolAddress: ") +
                                      hipGetErrorString(e));
      p = static_cast<float2*>(addr);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return QASR_OK;
}

}  // namespace
}  // namespace qasr

extern "C" int qasr_lm_head_int8_argmax_noalloc_f32(int32_t* idx, float* logits, const float* x,
                                                    const int8_t* w, const float* scales, size_t rows,
                                                    size_t in_dim, size_t vocab, void* stream) {
  if (rows == 0) return QASR_OK;
  QASR_REQUIRE(idx && logits && x && w && scales, "lm_head_int8_argmax_noalloc: null pointer");
  QASR_REQUIRE(vocab > 0, "lm_head_int8_argmax_noalloc: vocab must be positive");
  if (rows != 1) {  // several rows: logits then a scan, no scratch used
    const int rc = qasr_linear_nobias_int8_f32(logits, x, w, scales, rows, in_dim, vocab, stream);
    if (rc != QASR_OK) return rc;
    return qasr_argmax_rows_f32(idx, logits, rows, vocab, stream);
  }
  QASR_REQUIRE(lm_head_partials_max(vocab) <= kNoAllocPairs,
               "lm_head_int8_argmax_noalloc: vocab above QASR_LM_HEAD_NOALLOC_MAX_VOCAB (262144)");
  float2* part = nullptr;
  const int rc0 = scratch_for_current_device(&part);
  if (rc0 != QASR_OK) return rc0;
  hipStream_t st = as_stream(stream);
  unsigned n_part = 0;
  if (!launch_w8a32_argmax_partials(logits, x, w, scales, in_dim, vocab, part, kNoAllocPairs, st, &n_part))
    return fail(QASR_ERR_UNSUPPORTED,
                "lm_head_int8_argmax_noalloc: one row needs in_dim 1024..8192 in steps of 1024 and "
                "16-byte aligned x and w");
  const int rc = launch_status("lm_head_int8_argmax_noalloc");
  if (rc != QASR_OK) return rc;
  argmax_partials_kernel<<<1, kArgmaxBlock, 0, st>>>(idx, part, (int)n_part, logits);
  return launch_status("lm_head_int8_argmax_noalloc");
}
