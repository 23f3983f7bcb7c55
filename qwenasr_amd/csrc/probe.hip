// Measurement aid, no counterpart in the reference: a read-only kernel that
// shows how fast one CU can pull bytes in, which is what bounds the matrix-core
// kernels of this library (bench.py --probe runs it).
//
// Every workgroup (512 threads, as the W8A8 GEMMs) reads `bytes_per_wg` bytes
// with 16-byte loads, DEPTH loads in flight per thread, and XORs them into one
// int per thread (written to out, so nothing is optimised away):
//   mode 0: one region of bytes_per_wg per XCD (workgroup b on XCD b % 8),
//           read by all of that XCD's workgroups in the same order;
//   mode 1: as 0, each workgroup starting at its own rotation of the region;
//   mode 2: a private region of priv_bytes per workgroup, read repeatedly
//           (L2-resident after the first pass);
//   mode 3: a private region of bytes_per_wg per workgroup, read once, at
//           offset shift * grid * bytes_per_wg (an HBM stream);
//   mode 4: as 2, and waves w and w + 4 read the same addresses;
//   mode 5: as 3, and waves w and w + 4 read the same addresses.
// The host checks every region against buf_bytes before launching.
#include "common.hpp"

namespace qasr {
namespace {

typedef int v4i_p __attribute__((ext_vector_type(4)));

template <int DEPTH>
__global__ __launch_bounds__(512) void probe_read_kernel(const int8_t* __restrict__ buf, int* __restrict__ out,
                                                         int mode, long long total, long long priv,
                                                         long long shift) {
  const int b = blockIdx.x;
  long long base, span, off;
  if (mode == 0 || mode == 1) {
    base = (long long)(b % 8) * total;
    span = total;
    off = mode == 1 ? (long long)((b / 8) % 32) * (total / 32) : 0;
  } else if (mode == 2 || mode == 4) {
    base = (long long)b * priv;
    span = priv;
    off = 0;
  } else {
    base = ((long long)b + shift * gridDim.x) * total;
    span = total;
    off = 0;
  }
  const bool pairs = mode == 4 || mode == 5;
  const int tid = pairs ? (int)(threadIdx.x & 255) : (int)threadIdx.x;
  const long long step = pairs ? 256LL * 16 : 512LL * 16;  // bytes between a thread's loads
  off += (long long)tid * 16;
  if (off >= span) off -= span;
  v4i_p acc = {0, 0, 0, 0};
  const long long n = total / (512LL * 16);  // loads per thread
  for (long long i = 0; i < n; i += DEPTH) {
    v4i_p v[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      v[d] = *reinterpret_cast<const v4i_p*>(buf + base + off);
      off += step;
      if (off >= span) off -= span;
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) acc ^= v[d];
  }
  out[(size_t)b * 512 + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace
}  // namespace qasr

extern "C" int qasr_probe_read(int mode, int depth, unsigned grid, const void* buf, size_t buf_bytes, int* out,
                               size_t out_ints, size_t bytes_per_wg, size_t priv_bytes, size_t shift,
                               void* stream) {
  using namespace qasr;
  QASR_REQUIRE(buf && out, "probe_read: null pointer");
  QASR_REQUIRE(mode >= 0 && mode <= 5, "probe_read: mode must be 0..5");
  QASR_REQUIRE(depth == 4 || depth == 8 || depth == 16, "probe_read: depth must be 4, 8 or 16");
  QASR_REQUIRE(grid >= 1 && grid <= 4096, "probe_read: grid must be 1..4096");
  QASR_REQUIRE(bytes_per_wg >= 8192u * (size_t)depth && bytes_per_wg % (8192u * (size_t)depth) == 0,
               "probe_read: bytes_per_wg must be a multiple of 8192 * depth");
  QASR_REQUIRE(out_ints >= (size_t)grid * 512, "probe_read: out needs grid * 512 ints");
  QASR_REQUIRE(shift < 64, "probe_read: shift must be below 64");
  size_t need = 0;
  if (mode == 0 || mode == 1) {
    need = 8 * bytes_per_wg;
  } else if (mode == 2 || mode == 4) {
    QASR_REQUIRE(priv_bytes >= 8192 && priv_bytes % 16 == 0, "probe_read: priv_bytes must be >= 8192, 16-aligned");
    need = (size_t)grid * priv_bytes;
  } else {
    need = (shift + 1) * (size_t)grid * bytes_per_wg;
  }
  QASR_REQUIRE(need <= buf_bytes, "probe_read: the mode's regions exceed buf_bytes");
  QASR_REQUIRE(aligned16(buf), "probe_read: buf must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const int8_t* b8 = static_cast<const int8_t*>(buf);
  const long long tot = (long long)bytes_per_wg, pv = (long long)priv_bytes, sh = (long long)shift;
  if (depth == 4)
    probe_read_kernel<4><<<grid, 512, 0, st>>>(b8, out, mode, tot, pv, sh);
  else if (depth == 8)
    probe_read_kernel<8><<<grid, 512, 0, st>>>(b8, out, mode, tot, pv, sh);
  else
    probe_read_kernel<16><<<grid, 512, 0, st>>>(b8, out, mode, tot, pv, sh);
  return launch_status("probe_read");
}
