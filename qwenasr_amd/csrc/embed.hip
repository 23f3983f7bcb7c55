// Token-embedding gather for fp32, bf16 and int8+row-scale tables.
//
// One workgroup per token: the row is copied with 16-byte loads (fp32: 4
// values, bf16: 8 values, int8: 16 values per lane) and 16-byte stores of fp32.
// The conversions are exact: bf16 -> f32 is a 16-bit left shift
// (decoder.rs:631-636), int8 -> f32 is one multiply by the row scale
// (decoder.rs:639-646). An id outside [0, vocab) yields a NaN row.
#include "common.hpp"

namespace qasr {
namespace {

template <int MODE>  // 0 = f32, 1 = bf16, 2 = int8
__global__ __launch_bounds__(256) void gather_vec_kernel(float* out, const void* table,
                                                         const float* scales, const int32_t* ids,
                                                         int dim, long long vocab) {
  const long long id = ids[blockIdx.x];
  float* dst = out + (size_t)blockIdx.x * dim;
  const bool bad = id < 0 || id >= vocab;
  if constexpr (MODE == 0) {
    const float* src = static_cast<const float*>(table) + (bad ? 0 : id) * dim;
    for (int c = threadIdx.x; c < dim / 4; c += 256) {
      float4 v = ld4_nt(src, c);
      if (bad) v = make_float4(qnan(), qnan(), qnan(), qnan());
      st4_nt(dst, c, v);
    }
  } else if constexpr (MODE == 1) {
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(table) + (bad ? 0 : id) * dim);
    for (int c = threadIdx.x; c < dim / 8; c += 256) {
      const uint4 r = src[c];
      float4 lo, hi;
      lo.x = __uint_as_float(r.x << 16); lo.y = __uint_as_float(r.x & 0xffff0000u);
      lo.z = __uint_as_float(r.y << 16); lo.w = __uint_as_float(r.y & 0xffff0000u);
      hi.x = __uint_as_float(r.z << 16); hi.y = __uint_as_float(r.z & 0xffff0000u);
      hi.z = __uint_as_float(r.w << 16); hi.w = __uint_as_float(r.w & 0xffff0000u);
      if (bad) { lo = make_float4(qnan(), qnan(), qnan(), qnan()); hi = lo; }
      st4_nt(dst, 2 * c, lo);
      st4_nt(dst, 2 * c + 1, hi);
    }
  } else {
    const int4* src = reinterpret_cast<const int4*>(static_cast<const int8_t*>(table) + (bad ? 0 : id) * dim);
    const float s = bad ? qnan() : scales[id];
    for (int c = threadIdx.x; c < dim / 16; c += 256) {
      const int4 r = src[c];
      const int w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float4 o;
        o.x = (float)(int8_t)(w[k] & 0xff) * s;
        o.y = (float)(int8_t)((w[k] >> 8) & 0xff) * s;
        o.z = (float)(int8_t)((w[k] >> 16) & 0xff) * s;
        o.w = (float)(int8_t)((w[k] >> 24) & 0xff) * s;
        st4_nt(dst, 4 * c + k, o);
      }
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(256) void gather_scalar_kernel(float* out, const void* table,
                                                            const float* scales, const int32_t* ids,
                                                            int dim, long long vocab) {
  const long long id = ids[blockIdx.x];
  float* dst = out + (size_t)blockIdx.x * dim;
  const bool bad = id < 0 || id >= vocab;
  const size_t row = (size_t)(bad ? 0 : id) * dim;
  for (int c = threadIdx.x; c < dim; c += 256) {
    float v;
    if constexpr (MODE == 0) {
      v = static_cast<const float*>(table)[row + c];
    } else if constexpr (MODE == 1) {
      v = __uint_as_float((uint32_t)static_cast<const uint16_t*>(table)[row + c] << 16);
    } else {
      v = (float)static_cast<const int8_t*>(table)[row + c] * scales[bad ? 0 : id];
    }
    dst[c] = bad ? qnan() : v;
  }
}

template <int MODE>
int launch_gather(float* out, const void* table, const float* scales, const int32_t* ids,
                  size_t n, size_t dim, size_t vocab, void* stream) {
  const char* name = MODE == 0 ? "embed_gather_f32" : (MODE == 1 ? "embed_gather_bf16" : "embed_gather_i8");
  if (n == 0 || dim == 0) return QASR_OK;
  QASR_REQUIRE(out && table && ids && (MODE != 2 || scales), "embed_gather: null pointer");
  QASR_REQUIRE(vocab > 0, "embed_gather: vocab must be positive");
  QASR_REQUIRE(n <= kMaxRows && dim <= 0x7fffffffu, "embed_gather: size too large");
  size_t tab;
  QASR_REQUIRE(mul_ok(vocab, dim, &tab), "embed_gather: vocab * dim overflows");
  const int per = MODE == 0 ? 4 : (MODE == 1 ? 8 : 16);
  const bool vec = dim % per == 0 && aligned16(out) && aligned16(table);
  hipStream_t st = as_stream(stream);
  if (vec) {
    gather_vec_kernel<MODE><<<(unsigned)n, 256, 0, st>>>(out, table, scales, ids, (int)dim, (long long)vocab);
  } else {
    gather_scalar_kernel<MODE><<<(unsigned)n, 256, 0, st>>>(out, table, scales, ids, (int)dim, (long long)vocab);
  }
  return launch_status(name);
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_embed_gather_f32(float* out, const float* table, const int32_t* ids, size_t n,
                                     size_t dim, size_t vocab, void* stream) {
  return launch_gather<0>(out, table, nullptr, ids, n, dim, vocab, stream);
}

extern "C" int qasr_embed_gather_bf16(float* out, const uint16_t* table, const int32_t* ids,
                                      size_t n, size_t dim, size_t vocab, void* stream) {
  return launch_gather<1>(out, table, nullptr, ids, n, dim, vocab, stream);
}

extern "C" int qasr_embed_gather_i8(float* out, const int8_t* table, const float* row_scales,
                                    const int32_t* ids, size_t n, size_t dim, size_t vocab,
                                    void* stream) {
  return launch_gather<2>(out, table, row_scales, ids, n, dim, vocab, stream);
}
