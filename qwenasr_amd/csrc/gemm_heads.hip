// Batched W8A8 projection on CDNA4 int8 MFMA with a per-head epilogue: the
// q/k/v projections of B decode streams, each stream at its own position.
//
//   dot[m, n] = sum_k W[n, k] * Xq[m, k]                 (int32, exact)
//   y[m, n]   = ((f32)dot[m, n] * xs[m]) * s[n]          (the W8A8 dequantization)
//
// W is tile-packed (qasr_pack_w8a8_tiles): [N, K] with N = (n_heads +
// 2 n_kv_heads) * 128 rows, the q heads, then the k heads, then the v heads
// (decoder.rs:881-886 as one matrix). A workgroup owns one 128-row head x TOK
// streams (32, or 16 where 32 would leave fewer than 256 workgroups or the
// staged rows would not fit the LDS), so the epilogue sees whole heads:
//   q heads: per-head RMSNorm (q_norm) + NeoX RoPE at the stream's position,
//            written to q_out[m, head] (decoder.rs:888, 891);
//   k heads: the same with k_norm, written into the stream's cache row
//            k_cache[m][pos][kv_head] (decoder.rs:889, 892, 894);
//   v heads: written into v_cache[m][pos][kv_head] (decoder.rs:895).
// The norm and rotation are head_norm_rope, the device function of the
// standalone head kernel, so the results equal the plain projection
// (qasr_linear_w8a8_packed) followed by qasr_head_rms_norm_rope_kv_f32 bit for
// bit. MODE 0 is that plain projection: y[m, n] in fp32.
//
// Structure (8 waves, 512 threads): wave w = 4*kq + rg owns rows 32*rg ..
// 32*rg + 31 (two 16-row MFMA tiles) for the TOK/16 stream tiles over K half
// kq. The TOK streams' int8 rows (TOK x K bytes) are staged once in LDS with the
// 16-byte slot of row r at slot ^ (r % 16), so the b128 fragment reads of 16
// rows at one k offset hit distinct banks; W streams from the packed tiles
// into registers PF k-steps ahead, with cached loads: each W tile is read by
// every stream tile of the batch (8 or 16), and non-temporal loads, which
// lose that reuse in the L2, measured 10-23% slower (o [2048,2048]: 6.8 ->
// 5.9 us as cached). After the loop the two K halves of a row
// group are added through LDS (exact int32), the dequantized tile goes to LDS
// as [TOK streams][128 dims], and groups of 16 threads -- one stream each, in
// the lane layout head_norm_rope expects -- finish the heads.
#include "common.hpp"

#include <atomic>

namespace qasr {
namespace {

typedef int v4i_t __attribute__((ext_vector_type(4)));

constexpr int kHdRows = 128;   // W rows per workgroup: one head
constexpr int kHdWaves = 8;
constexpr int kHdPF = 3;       // k-steps of W in flight per wave
constexpr int kHdTPitch = 136; // floats per stream row of the dequantized tile (pad: banks)
constexpr int kNumXcdH = 8;

struct HeadsArgs {
  float* y;               // MODE 0: [batch, N]
  float* q_out;           // MODE 1: [batch, n_heads * 128]
  float* k_cache;         // MODE 1: stream m's block at k_cache + m * cache_rows * kv_dim
  float* v_cache;
  const int8_t* w;        // packed [N, K]
  const float* scales;    // [N]
  const int8_t* xq;       // [batch, K]
  const float* xs;        // [batch]
  const float* q_norm_w;  // [128]
  const float* k_norm_w;
  const float* cos_tab;   // [table_rows, 128]
  const float* sin_tab;
  const int32_t* positions;  // [batch]
  long long table_rows;
  long long cache_rows;
  int batch;
  int N;
  int n_heads;
  int n_kv_heads;
  int n_tiles;
  int m_tiles;
  float eps;
};

template <int KS, int MODE, int TOK>  // K = 64 KS; TOK streams per workgroup (16 or 32)
__global__ __launch_bounds__(64 * kHdWaves) void gemm_w8a8_heads_kernel(HeadsArgs a) {
  constexpr int K = KS * 64;
  constexpr int KW = KS / 2;           // k-steps per wave (one K half)
  constexpr int MT = TOK / 16;         // 16-stream MFMA tiles
  constexpr int SLOTS = K / 16;        // 16-byte slots per staged row
  constexpr int XU = TOK * SLOTS / (64 * kHdWaves);  // staging loads per thread
  constexpr int PF = kHdPF;
  constexpr size_t ROW_TILE = (size_t)KS * 1024;  // bytes of one 16-row block of packed W
  static_assert(KS % 2 == 0 && (MT == 1 || MT == 2), "K halves; one or two stream tiles");
  static_assert(XU * 64 * kHdWaves == TOK * SLOTS, "the staging covers the tile");
  extern __shared__ __align__(16) int8_t lds[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave & 3, kq = wave >> 2;
  const int r = lane & 15, g = lane >> 4;

  // XCD-aware order: block b runs on XCD b % 8; the m_tiles blocks sharing a
  // W tile go to the same XCD back to back, so later ones hit its L2.
  const int b = blockIdx.x;
  int tile_n, tile_m;
  if (a.n_tiles % kNumXcdH == 0) {
    const int slot = b / kNumXcdH;
    tile_m = slot % a.m_tiles;
    tile_n = b % kNumXcdH + kNumXcdH * (slot / a.m_tiles);
  } else {
    tile_m = b % a.m_tiles;
    tile_n = b / a.m_tiles;
  }
  const int n0 = tile_n * kHdRows, m0 = tile_m * TOK;

  // Issue order: the stream rows, the W window, the epilogue operands.
  v4i_t xr[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int c = threadIdx.x + 64 * kHdWaves * u;
    const int row = c / SLOTS, slot = c % SLOTS;
    const int src = m0 + row < a.batch ? m0 + row : a.batch - 1;  // past the batch: valid row, dropped
    xr[u] = *reinterpret_cast<const v4i_t*>(a.xq + (size_t)src * K + 16 * slot);
  }
  __builtin_amdgcn_sched_barrier(0);
  const int8_t* wp = a.w + ((size_t)((n0 + 32 * rg) / 16) * KS + (size_t)kq * KW) * 1024 + 16 * lane;
  v4i_t wbuf[PF][2];
#pragma unroll
  for (int d = 0; d < PF; ++d)
#pragma unroll
    for (int i = 0; i < 2; ++i)
      wbuf[d][i] = *reinterpret_cast<const v4i_t*>(wp + i * ROW_TILE + d * 1024);
  __builtin_amdgcn_sched_barrier(0);
  float4 sc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) sc[i] = *reinterpret_cast<const float4*>(a.scales + n0 + 32 * rg + 16 * i + 4 * g);
  const int mt = m0 + (MT == 2 ? 16 * kq : 0) + r;
  const float xsv = a.xs[mt < a.batch ? mt : a.batch - 1];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int c = threadIdx.x + 64 * kHdWaves * u;
    const int row = c / SLOTS, slot = c % SLOTS;
    *reinterpret_cast<v4i_t*>(lds + row * K + 16 * (slot ^ (row & 15))) = xr[u];
  }
  lds_barrier();

  v4i_t acc[2][MT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = v4i_t{0, 0, 0, 0};
  // B fragment of stream tile j at global k-step s: stream row 16j + r, bytes
  // [64s + 16g, +16) = slot 4s + g
  auto xfrag = [&](int s, int j) -> v4i_t {
    return *reinterpret_cast<const v4i_t*>(lds + (16 * j + r) * K + 16 * ((4 * s + g) ^ r));
  };
  const int k0 = kq * KW;
  v4i_t bcur[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) bcur[j] = xfrag(k0, j);
#pragma unroll
  for (int s0 = 0; s0 < KW; s0 += PF) {
#pragma unroll
    for (int d = 0; d < PF; ++d) {
      const int s = s0 + d;
      if (s < KW) {
        v4i_t av[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          av[i] = wbuf[d][i];
          if (s + PF < KW)
            wbuf[d][i] = *reinterpret_cast<const v4i_t*>(wp + i * ROW_TILE + (s + PF) * 1024);
        }
        // keep the prefetch and the next fragments issued here (the scheduler
        // would sink each load next to its use)
        __builtin_amdgcn_sched_barrier(0);
        v4i_t bn[MT];
        if (s + 1 < KW) {
#pragma unroll
          for (int j = 0; j < MT; ++j) bn[j] = xfrag(k0 + s + 1, j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < MT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bcur[j], acc[i][j], 0, 0, 0);
        if (s + 1 < KW) {
#pragma unroll
          for (int j = 0; j < MT; ++j) bcur[j] = bn[j];
        }
      }
    }
  }

  // The two K halves of a row group: with two stream tiles wave kq keeps
  // tile kq and adds its partner's partial sums for it; with one, wave 0 of
  // the pair adds wave 1's (constant register indices only).
  __syncthreads();  // X no longer read
  v4i_t mine[2];
  v4i_t* ex = reinterpret_cast<v4i_t*>(lds);  // [rg][receiver kq][i][lane]
  if constexpr (MT == 2) {
    v4i_t give[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      give[i] = kq == 0 ? acc[i][1] : acc[i][0];
      mine[i] = kq == 0 ? acc[i][0] : acc[i][MT - 1];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) ex[((rg * 2 + (1 - kq)) * 2 + i) * 64 + lane] = give[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) mine[i] += ex[((rg * 2 + kq) * 2 + i) * 64 + lane];
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) mine[i] = acc[i][0];
    if (kq == 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i) ex[(rg * 2 + i) * 64 + lane] = mine[i];
    }
    __syncthreads();
    if (kq == 0) {
#pragma unroll
      for (int i = 0; i < 2; ++i) mine[i] += ex[(rg * 2 + i) * 64 + lane];
    }
  }
  __syncthreads();  // exchange area free

  // Dequantize into the [TOK streams][128 dims] tile: lane holds rows
  // 32rg + 16i + 4g + {0..3} of stream tile row (MT == 2 ? 16kq : 0) + r.
  float* T = reinterpret_cast<float*>(lds);
  if (MT == 2 || kq == 0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      float4 v;
      v.x = ((float)mine[i][0] * xsv) * sc[i].x;
      v.y = ((float)mine[i][1] * xsv) * sc[i].y;
      v.z = ((float)mine[i][2] * xsv) * sc[i].z;
      v.w = ((float)mine[i][3] * xsv) * sc[i].w;
      *reinterpret_cast<float4*>(T + ((MT == 2 ? 16 * kq : 0) + r) * kHdTPitch + 32 * rg + 16 * i + 4 * g) = v;
    }
  }
  lds_barrier();

  // One stream per group of 16 threads: dims 4sub..4sub+3 and 64+4sub..
  const int tok = threadIdx.x >> 4, sub = threadIdx.x & 15;
  if (tok >= TOK) return;  // whole waves past the tile (TOK = 16): nothing left to do
  const int m = m0 + tok;
  const bool live = m < a.batch;
  float4 x1 = *reinterpret_cast<const float4*>(T + tok * kHdTPitch + 4 * sub);
  float4 x2 = *reinterpret_cast<const float4*>(T + tok * kHdTPitch + 64 + 4 * sub);
  if constexpr (MODE == 0) {
    if (live) {
      float* yr = a.y + (size_t)m * a.N + n0;
      st4(yr, sub, x1);
      st4(yr + 64, sub, x2);
    }
  } else {
    const int h = tile_n;
    const int kind = h < a.n_heads ? 0 : (h < a.n_heads + a.n_kv_heads ? 1 : 2);
    const long long pos = live ? (long long)a.positions[m] : 0;
    const bool pos_ok = pos >= 0 && pos < a.table_rows && pos < a.cache_rows;
    const int kv_dim = a.n_kv_heads * 128;
    if (kind < 2) {
      const float* w = kind == 0 ? a.q_norm_w : a.k_norm_w;
      const float4 w1 = ld4(w, sub), w2 = ld4(w + 64, sub);
      const long long pr = pos_ok ? pos : 0;  // out-of-table rows read row 0, then become NaN
      const float* cr = a.cos_tab + pr * 128;
      const float* sr = a.sin_tab + pr * 128;
      const float4 c1 = ld4(cr, sub), c2 = ld4(cr + 64, sub);
      const float4 s1 = ld4(sr, sub), s2 = ld4(sr + 64, sub);
      // every lane of the group joins the reduction, live or not
      head_norm_rope<128, true, true>(x1, x2, w1, w2, c1, c2, s1, s2, pos_ok, a.eps);
    }
    if (live) {
      float* dst = nullptr;
      if (kind == 0) {
        dst = a.q_out + (size_t)m * a.n_heads * 128 + (size_t)h * 128;
      } else if (pos_ok) {  // a row outside the cache is not written
        float* cache = kind == 1 ? a.k_cache : a.v_cache;
        const int kvh = kind == 1 ? h - a.n_heads : h - a.n_heads - a.n_kv_heads;
        dst = cache + ((size_t)m * a.cache_rows + (size_t)pos) * kv_dim + (size_t)kvh * 128;
      }
      if (dst) {
        st4(dst, sub, x1);
        st4(dst + 64, sub, x2);
      }
    }
  }
}

// Streamed form of the q/k/v + heads kernel for 32-stream tiles (K = 1024 or
// 2048). Eight MFMA waves each own one 16-row block of the head over the whole
// K (no K halves to add up), and two loader waves bring the 32 stream rows in
// with direct global->LDS loads, in chunks of 4 k-steps (32 rows x 256 bytes,
// token row t's LDS slot l holding its data slot l ^ (t & 15)). All chunks are
// issued at once and the whole tile stays in LDS; barrier c means chunk c has
// landed, so the MFMAs start on the first 8 KiB instead of the whole tile. The
// epilogue's position is loaded at entry and its gains and table rows under
// the first chunk. Same dots, dequantization and head_norm_rope as
// gemm_w8a8_heads_kernel<KS, 1, 32>: the results equal it bit for bit.
constexpr int kHsMfma = kHdRows / 16;                     // 8: one 16-row block each
constexpr int kHsLoaders = 2;
constexpr int kHsWaves = kHsMfma + kHsLoaders;
constexpr int kHsTok = 32;
constexpr int kHsChunk = 256;                             // bytes of K per chunk
constexpr int kHsChunkBytes = kHsTok * kHsChunk;          // 8 KiB
constexpr int kHsPieces = kHsChunkBytes / 1024 / kHsLoaders;  // 1 KiB direct loads per chunk per loader
constexpr int kHsPF = 8;                                  // k-steps of W in flight per MFMA wave

template <int KS>
constexpr size_t heads_stream_lds() {
  return (size_t)kHsTok * KS * 64 + (size_t)kHsTok * kHdTPitch * sizeof(float);
}

// Waits until at most 4n of this wave's vector memory operations are
// outstanding (n < 16; the immediate must be a constant).
QASR_DEV void wait_vm_pieces(int n) {
  static_assert(kHsPieces == 4, "the cases below count 4 loads per chunk");
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(4)); break;
    case 2: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(8)); break;
    case 3: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(12)); break;
    case 4: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(16)); break;
    case 5: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(20)); break;
    case 6: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(24)); break;
    default: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(28)); break;
  }
}

template <int KS>  // K = 64 KS (16 or 32)
__global__ __launch_bounds__(64 * kHsWaves) void gemm_w8a8_heads_stream_kernel(HeadsArgs a) {
  constexpr int K = KS * 64;
  constexpr int NCH = K / kHsChunk;       // chunks (4 or 8)
  constexpr int SPC = kHsChunk / 64;      // k-steps per chunk
  constexpr int PF = kHsPF;
  static_assert(NCH * kHsPieces <= 63 && NCH <= 8, "every chunk in flight at once");
  static_assert(kHsTok * 16 == 64 * kHsMfma, "one 16-thread group per stream in the MFMA waves");
  extern __shared__ __align__(16) int8_t lds[];
  float* T = reinterpret_cast<float*>(lds + (size_t)NCH * kHsChunkBytes);  // [32 streams][kHdTPitch]

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int b = blockIdx.x;
  int tile_n, tile_m;
  if (a.n_tiles % kNumXcdH == 0) {
    const int slot = b / kNumXcdH;
    tile_m = slot % a.m_tiles;
    tile_n = b % kNumXcdH + kNumXcdH * (slot / a.m_tiles);
  } else {
    tile_m = b % a.m_tiles;
    tile_n = b / a.m_tiles;
  }
  const int n0 = tile_n * kHdRows, m0 = tile_m * kHsTok;
  const int h = tile_n;
  const int kind = h < a.n_heads ? 0 : (h < a.n_heads + a.n_kv_heads ? 1 : 2);

  // epilogue: one stream per group of 16 threads of the MFMA waves
  const int tok = threadIdx.x >> 4, sub = threadIdx.x & 15;
  const int m = m0 + tok;
  const bool live = wave < kHsMfma && m < a.batch;
  float4 w1, w2, c1, c2, s1, s2;
  int pos32 = 0;  // widened where it is used, after the first barrier
  bool pos_ok = false;

  v4i_t acc[2];
  float4 sc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float xsv[2];
  if (wave >= kHsMfma) {
    // Loader: 1 KiB piece p of a chunk is stream rows 4p .. 4p + 3; lane l
    // fills LDS slot l & 15 of row 4p + l / 16. Rows past the batch re-read
    // row batch - 1 (valid memory); their results are never stored.
    const int pw = wave - kHsMfma;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < kHsPieces; ++i) {
        const int piece = kHsPieces * pw + i;
        const int row = 4 * piece + (lane >> 4);
        const int data_slot = (lane & 15) ^ (row & 15);
        const int src = m0 + row < a.batch ? m0 + row : a.batch - 1;
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(a.xq + (size_t)src * K + kHsChunk * c + 16 * data_slot),
            (__attribute__((address_space(3))) void*)(lds + c * kHsChunkBytes + piece * 1024), 16, 0, 0);
      }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      wait_vm_pieces(NCH - 1 - c);  // chunk c has landed
      asm volatile("s_barrier" ::: "memory");
    }
  } else {
    // the position first: waiting for it then leaves every later load in flight.
    // Unconditional (a clamped, valid index): a load under a branch is waited
    // for, with everything issued before it, where the branch ends.
    pos32 = a.positions[m < a.batch ? m : a.batch - 1];
    const int8_t* wp = a.w + ((size_t)(n0 / 16 + wave) * KS) * 1024 + 16 * lane;
    v4i_t wbuf[PF];
#pragma unroll
    for (int d = 0; d < PF; ++d) wbuf[d] = *reinterpret_cast<const v4i_t*>(wp + d * 1024);
    __builtin_amdgcn_sched_barrier(0);
    sc = *reinterpret_cast<const float4*>(a.scales + n0 + 16 * wave + 4 * g);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int mt = m0 + 16 * j + r;
      xsv[j] = a.xs[mt < a.batch ? mt : a.batch - 1];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[j] = v4i_t{0, 0, 0, 0};

    // B fragment of stream tile j at k-step s
    auto xfrag = [&](int s, int j) -> v4i_t {
      const int slot = SPC * (s % SPC) + g;
      return *reinterpret_cast<const v4i_t*>(lds + (s / SPC) * kHsChunkBytes + (16 * j + r) * kHsChunk +
                                             16 * (slot ^ r));
    };
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      lds_barrier();  // chunk c is in LDS
      if (c == 0 && kind < 2) {
        // the epilogue's gains and table rows, under the stream rows' loads
        asm volatile("" : "+v"(pos32));  // first use here: the compiler would hoist the widening above the barrier
        const long long pos = pos32;
        pos_ok = m < a.batch && pos >= 0 && pos < a.table_rows && pos < a.cache_rows;
        const long long pr = pos_ok ? pos : 0;  // out-of-table rows read row 0, then become NaN
        const float* w = kind == 0 ? a.q_norm_w : a.k_norm_w;
        w1 = ld4(w, sub);
        w2 = ld4(w + 64, sub);
        c1 = ld4(a.cos_tab + pr * 128, sub);
        c2 = ld4(a.cos_tab + pr * 128 + 64, sub);
        s1 = ld4(a.sin_tab + pr * 128, sub);
        s2 = ld4(a.sin_tab + pr * 128 + 64, sub);
      }
      v4i_t bcur[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) bcur[j] = xfrag(SPC * c, j);
#pragma unroll
      for (int q = 0; q < SPC; ++q) {
        const int s = SPC * c + q;
        const v4i_t av = wbuf[s % PF];
        if (s + PF < KS) wbuf[s % PF] = *reinterpret_cast<const v4i_t*>(wp + (s + PF) * 1024);
        // keep the prefetch and the next fragments issued here (the scheduler
        // would sink each load next to its use)
        __builtin_amdgcn_sched_barrier(0);
        v4i_t bn[2];
        if (q + 1 < SPC) {
#pragma unroll
          for (int j = 0; j < 2; ++j) bn[j] = xfrag(s + 1, j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bcur[j], acc[j], 0, 0, 0);
        if (q + 1 < SPC) {
#pragma unroll
          for (int j = 0; j < 2; ++j) bcur[j] = bn[j];
        }
      }
    }
    // Dequantize into the [32 streams][128 dims] tile (past the staged rows:
    // no barrier needed before it): lane holds rows 16 wave + 4g + {0..3} of
    // stream 16j + r.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float4 v;
      v.x = ((float)acc[j][0] * xsv[j]) * sc.x;
      v.y = ((float)acc[j][1] * xsv[j]) * sc.y;
      v.z = ((float)acc[j][2] * xsv[j]) * sc.z;
      v.w = ((float)acc[j][3] * xsv[j]) * sc.w;
      *reinterpret_cast<float4*>(T + (16 * j + r) * kHdTPitch + 16 * wave + 4 * g) = v;
    }
  }
  lds_barrier();
  if (wave >= kHsMfma) return;  // loaders: done (no barrier follows)

  float4 x1 = *reinterpret_cast<const float4*>(T + tok * kHdTPitch + 4 * sub);
  float4 x2 = *reinterpret_cast<const float4*>(T + tok * kHdTPitch + 64 + 4 * sub);
  const long long pos = pos32;
  if (kind < 2) {
    // every lane of the group joins the reduction, live or not
    head_norm_rope<128, true, true>(x1, x2, w1, w2, c1, c2, s1, s2, pos_ok, a.eps);
  } else {
    pos_ok = m < a.batch && pos >= 0 && pos < a.table_rows && pos < a.cache_rows;
  }
  if (live) {
    const int kv_dim = a.n_kv_heads * 128;
    float* dst = nullptr;
    if (kind == 0) {
      dst = a.q_out + (size_t)m * a.n_heads * 128 + (size_t)h * 128;
    } else if (pos_ok) {  // a row outside the cache is not written
      float* cache = kind == 1 ? a.k_cache : a.v_cache;
      const int kvh = kind == 1 ? h - a.n_heads : h - a.n_heads - a.n_kv_heads;
      dst = cache + ((size_t)m * a.cache_rows + (size_t)pos) * kv_dim + (size_t)kvh * 128;
    }
    if (dst) {
      st4(dst, sub, x1);
      st4(dst + 64, sub, x2);
    }
  }
}

// Persistent form of the plain projection (MODE 0) for outputs many times
// wider than the GPU (a batch's lm_head: [256,2048]x[2048,151936] is 9496
// one-tile workgroups of 128 rows x 32 streams, 363 us). Each workgroup keeps
// one stream tile's rows in LDS and walks a contiguous range of column tiles,
// the next tile's W window loading under the current tile's last k-steps and
// epilogue, and takes 64 streams where their rows fit the LDS (K <= 2048):
// every W byte pulled into a CU then serves twice the outputs. Workgroup b
// runs on XCD b % 8; the m_tiles workgroups of one range sit on one XCD, so
// each W tile is fetched into that L2 once. The exchange area lies past the
// staged rows, which stay put; each lane stores its four dequantized rows of
// a stream directly. Per output the arithmetic is the one-tile kernel's, so
// the results are the same bit for bit.
template <int KS, int TOK>
__global__ __launch_bounds__(64 * kHdWaves) void gemm_w8a8_rows_persistent_kernel(HeadsArgs a, int groups) {
  constexpr int K = KS * 64;
  constexpr int KW = KS / 2;
  constexpr int MT = TOK / 16;        // 16-stream MFMA tiles
  constexpr int HT = MT > 1 ? MT / 2 : 1;  // stream tiles a wave finishes
  constexpr int SLOTS = K / 16;
  constexpr int XU = TOK * SLOTS / (64 * kHdWaves);
  // k-steps of W in flight per wave; a divisor of KW, so the next tile's first
  // steps land in the register slots its loop starts from
  constexpr int PF = 4;
  constexpr size_t ROW_TILE = (size_t)KS * 1024;
  constexpr int X_BYTES = TOK * K;
  static_assert(KS % 2 == 0 && (MT == 1 || MT == 2 || MT == 4), "K halves; 1, 2 or 4 stream tiles");
  static_assert(XU * 64 * kHdWaves == TOK * SLOTS, "the staging covers the tile");
  static_assert(KW % PF == 0, "the W window wraps into the next tile's slots");
  extern __shared__ __align__(16) int8_t lds[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave & 3, kq = wave >> 2;
  const int r = lane & 15, g = lane >> 4;
  const int b = blockIdx.x, xcd = b % kNumXcdH, j32 = b / kNumXcdH;
  const int tile_m = j32 % a.m_tiles, group = j32 / a.m_tiles;
  if (group >= groups) return;  // uniform, before any barrier
  const int ranges = kNumXcdH * groups, rho = xcd + kNumXcdH * group;
  const int nt_begin = (int)((long long)rho * a.n_tiles / ranges);
  const int nt_end = (int)((long long)(rho + 1) * a.n_tiles / ranges);
  if (nt_begin >= nt_end) return;
  const int m0 = tile_m * TOK;

  v4i_t xr[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int c = threadIdx.x + 64 * kHdWaves * u;
    const int row = c / SLOTS, slot = c % SLOTS;
    const int src = m0 + row < a.batch ? m0 + row : a.batch - 1;  // past the batch: valid row, dropped
    xr[u] = *reinterpret_cast<const v4i_t*>(a.xq + (size_t)src * K + 16 * slot);
  }
  __builtin_amdgcn_sched_barrier(0);
  auto wptr = [&](int tn) {
    return a.w + ((size_t)((tn * kHdRows + 32 * rg) / 16) * KS + (size_t)kq * KW) * 1024 + 16 * lane;
  };
  const int8_t* wp = wptr(nt_begin);
  v4i_t wbuf[PF][2];
#pragma unroll
  for (int d = 0; d < PF; ++d)
#pragma unroll
    for (int i = 0; i < 2; ++i)
      wbuf[d][i] = *reinterpret_cast<const v4i_t*>(wp + i * ROW_TILE + d * 1024);
  __builtin_amdgcn_sched_barrier(0);
  // the stream scales of the tiles this wave finishes: stream tile
  // (MT > 1 ? kq * HT + jj : 0), row r
  float xsv[HT];
  int mrow[HT];
#pragma unroll
  for (int jj = 0; jj < HT; ++jj) {
    mrow[jj] = m0 + 16 * (MT > 1 ? kq * HT + jj : 0) + r;
    xsv[jj] = a.xs[mrow[jj] < a.batch ? mrow[jj] : a.batch - 1];
  }
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int c = threadIdx.x + 64 * kHdWaves * u;
    const int row = c / SLOTS, slot = c % SLOTS;
    *reinterpret_cast<v4i_t*>(lds + row * K + 16 * (slot ^ (row & 15))) = xr[u];
  }
  lds_barrier();

  v4i_t* ex = reinterpret_cast<v4i_t*>(lds + X_BYTES);  // [rg][receiver kq][i][jj][lane]
  auto xfrag = [&](int s, int jt) -> v4i_t {
    return *reinterpret_cast<const v4i_t*>(lds + (16 * jt + r) * K + 16 * ((4 * s + g) ^ r));
  };
  const int k0 = kq * KW;
  const bool vec = (a.N & 3) == 0;  // (y is 16-byte aligned: checked by the entry point)
  for (int tn = nt_begin; tn < nt_end; ++tn) {
    const int n0 = tn * kHdRows;
    const int8_t* wn = wptr(tn + 1 < nt_end ? tn + 1 : tn);  // the next tile's window (the last re-loads itself)
    float4 sc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) sc[i] = *reinterpret_cast<const float4*>(a.scales + n0 + 32 * rg + 16 * i + 4 * g);
    v4i_t acc[2][MT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int jt = 0; jt < MT; ++jt) acc[i][jt] = v4i_t{0, 0, 0, 0};
    v4i_t bcur[MT];
#pragma unroll
    for (int jt = 0; jt < MT; ++jt) bcur[jt] = xfrag(k0, jt);
#pragma unroll
    for (int s0 = 0; s0 < KW; s0 += PF) {
#pragma unroll
      for (int d = 0; d < PF; ++d) {
        const int s = s0 + d;
        v4i_t av[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          av[i] = wbuf[d][i];
          const int8_t* src = s + PF < KW ? wp + i * ROW_TILE + (s + PF) * 1024
                                          : wn + i * ROW_TILE + (s + PF - KW) * 1024;
          wbuf[d][i] = *reinterpret_cast<const v4i_t*>(src);
        }
        __builtin_amdgcn_sched_barrier(0);
        v4i_t bn[MT];
        if (s + 1 < KW) {
#pragma unroll
          for (int jt = 0; jt < MT; ++jt) bn[jt] = xfrag(k0 + s + 1, jt);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jt = 0; jt < MT; ++jt)
            acc[i][jt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[i], bcur[jt], acc[i][jt], 0, 0, 0);
        if (s + 1 < KW) {
#pragma unroll
          for (int jt = 0; jt < MT; ++jt) bcur[jt] = bn[jt];
        }
      }
    }
    wp = wn;

    // K halves: wave kq keeps stream tiles kq * HT .. and adds its partner's
    // partial sums for them (with one stream tile, wave 0 of the pair adds
    // wave 1's); constant register indices only. The barriers wait for LDS
    // only, so the next tile's W window stays in flight.
    v4i_t mine[2][HT];
    if constexpr (MT > 1) {
      v4i_t give[2][HT];
      if (kq == 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jj = 0; jj < HT; ++jj) { give[i][jj] = acc[i][HT + jj]; mine[i][jj] = acc[i][jj]; }
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jj = 0; jj < HT; ++jj) { give[i][jj] = acc[i][jj]; mine[i][jj] = acc[i][HT + jj]; }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < HT; ++jj) ex[(((rg * 2 + (1 - kq)) * 2 + i) * HT + jj) * 64 + lane] = give[i][jj];
      lds_barrier();
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < HT; ++jj) mine[i][jj] += ex[(((rg * 2 + kq) * 2 + i) * HT + jj) * 64 + lane];
      lds_barrier();  // the exchange area is free for the next tile
    } else {
#pragma unroll
      for (int i = 0; i < 2; ++i) mine[i][0] = acc[i][0];
      if (kq == 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i) ex[(rg * 2 + i) * 64 + lane] = mine[i][0];
      }
      lds_barrier();
      if (kq == 0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) mine[i][0] += ex[(rg * 2 + i) * 64 + lane];
      }
      lds_barrier();
    }
    // lane: rows n0 + 32rg + 16i + 4g + {0..3} of stream mrow[jj]
    if (MT > 1 || kq == 0) {
#pragma unroll
      for (int jj = 0; jj < HT; ++jj) {
        if (mrow[jj] >= a.batch) continue;
        float* yr = a.y + (size_t)mrow[jj] * a.N + n0 + 32 * rg + 4 * g;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          float4 v;
          v.x = ((float)mine[i][jj][0] * xsv[jj]) * sc[i].x;
          v.y = ((float)mine[i][jj][1] * xsv[jj]) * sc[i].y;
          v.z = ((float)mine[i][jj][2] * xsv[jj]) * sc[i].z;
          v.w = ((float)mine[i][jj][3] * xsv[jj]) * sc[i].w;
          if (vec) {
            *reinterpret_cast<float4*>(yr + 16 * i) = v;
          } else {
            yr[16 * i] = v.x;
            yr[16 * i + 1] = v.y;
            yr[16 * i + 2] = v.z;
            yr[16 * i + 3] = v.w;
          }
        }
      }
    }
  }
}

// The staged rows (32 x K bytes) need more than the default 64 KiB of LDS at
// K = 2048; the limit is raised once per device.
template <auto Fn>
bool heads_lds_ok(size_t bytes) {
  if (bytes <= 65536) return true;
  constexpr int kMaxDev = 64;
  static std::atomic<signed char> state[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
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

template <int KS, int MODE, int TOK>
int launch_heads_tile(const HeadsArgs& a, unsigned grid, hipStream_t st, const char* what) {
  const size_t lds = (size_t)TOK * KS * 64 > 16384 ? (size_t)TOK * KS * 64 : 16384;  // >= exchange + fp32 tile
  if (!heads_lds_ok<&gemm_w8a8_heads_kernel<KS, MODE, TOK>>(lds))
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": device LDS too small");
  gemm_w8a8_heads_kernel<KS, MODE, TOK><<<grid, 64 * kHdWaves, lds, st>>>(a);
  return launch_status(what);
}

template <int KS>
int launch_heads_stream(const HeadsArgs& a, unsigned grid, hipStream_t st, const char* what) {
  constexpr size_t lds = heads_stream_lds<KS>();
  if (!heads_lds_ok<&gemm_w8a8_heads_stream_kernel<KS>>(lds))
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": device LDS too small");
  gemm_w8a8_heads_stream_kernel<KS><<<grid, 64 * kHsWaves, lds, st>>>(a);
  return launch_status(what);
}

// The persistent projection: 256 workgroups (32 per XCD), the stream tile's
// rows plus the exchange area and the dequantized tile in LDS.
template <int KS, int TOK>
constexpr size_t rows_persistent_lds() {  // staged rows + exchange area
  return (size_t)TOK * KS * 64 + (size_t)4 * 2 * 2 * (TOK >= 32 ? TOK / 32 : 1) * 64 * 16;
}

template <int KS, int TOK>
int launch_rows_persistent(const HeadsArgs& a, int groups, hipStream_t st, const char* what) {
  constexpr size_t lds = rows_persistent_lds<KS, TOK>();
  if (!heads_lds_ok<&gemm_w8a8_rows_persistent_kernel<KS, TOK>>(lds))
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": device LDS too small");
  gemm_w8a8_rows_persistent_kernel<KS, TOK><<<kNumXcdH * 32, 64 * kHdWaves, lds, st>>>(a, groups);
  return launch_status(what);
}

// 32-stream tiles (the staged rows shared by twice the outputs) when K <= 2048
// and they still give at least 256 workgroups; otherwise 16-stream tiles
// (32 x K would not fit the LDS, or the grid would leave CUs idle).
template <int KS, int MODE>
int launch_heads_k(HeadsArgs a, hipStream_t st, const char* what) {
  a.n_tiles = a.N / kHdRows;
  const size_t m32 = ((size_t)a.batch + 31) / 32, m16 = ((size_t)a.batch + 15) / 16;
  const bool tok32 = KS <= 32 && (size_t)a.n_tiles * m32 >= 256;
  a.m_tiles = (int)(tok32 ? m32 : m16);
  const size_t grid = (size_t)a.n_tiles * (size_t)a.m_tiles;
  QASR_REQUIRE(grid <= 0x7fffffffu, std::string(what) + ": grid too large");
  if constexpr (MODE == 0) {
    // 4+ one-tile workgroups per CU: the persistent form, with the widest
    // stream tile whose rows fit the LDS and whose count divides an XCD's 32
    // workgroups
    if (grid >= 1024) {
      const size_t m64 = ((size_t)a.batch + 63) / 64;
      HeadsArgs p = a;
      if constexpr (rows_persistent_lds<KS, 64>() <= 163840) {
        if (32 % m64 == 0) {
          p.m_tiles = (int)m64;
          return launch_rows_persistent<KS, 64>(p, (int)(32 / m64), st, what);
        }
      }
      if constexpr (rows_persistent_lds<KS, 32>() <= 163840) {
        if (32 % m32 == 0) {
          p.m_tiles = (int)m32;
          return launch_rows_persistent<KS, 32>(p, (int)(32 / m32), st, what);
        }
      }
      if (32 % m16 == 0) {
        p.m_tiles = (int)m16;
        return launch_rows_persistent<KS, 16>(p, (int)(32 / m16), st, what);
      }
    }
  }
  if constexpr (KS <= 32) {
    if constexpr (MODE == 1) {
      if (tok32) return launch_heads_stream<KS>(a, (unsigned)grid, st, what);
    }
    if (tok32) return launch_heads_tile<KS, MODE, 32>(a, (unsigned)grid, st, what);
  }
  return launch_heads_tile<KS, MODE, 16>(a, (unsigned)grid, st, what);
}

template <int MODE>
int launch_heads_gemm(HeadsArgs a, size_t K, hipStream_t st, const char* what) {
  switch (K) {
    case 1024: return launch_heads_k<16, MODE>(a, st, what);
    case 2048: return launch_heads_k<32, MODE>(a, st, what);
    case 3072: return launch_heads_k<48, MODE>(a, st, what);
    case 4096: return launch_heads_k<64, MODE>(a, st, what);
    default: return launch_heads_k<96, MODE>(a, st, what);  // 6144
  }
}

int check_w8a8_common(const int8_t* w, const float* scales, const int8_t* xq, const float* xs,
                      size_t batch, size_t in_dim, size_t out_dim, const char* what) {
  QASR_REQUIRE(w && scales && xq && xs, std::string(what) + ": null pointer");
  if (in_dim != 1024 && in_dim != 2048 && in_dim != 3072 && in_dim != 4096 && in_dim != 6144)
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": in_dim must be 1024, 2048, 3072, 4096 or 6144");
  if (out_dim % kHdRows != 0)
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": out_dim must be a multiple of 128");
  QASR_REQUIRE(batch <= 0x7fffffffu && out_dim <= 0x7fffffffu, std::string(what) + ": size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(batch, out_dim, &n) && mul_ok(batch, in_dim, &n) && mul_ok(out_dim, in_dim, &n),
               std::string(what) + ": size overflows");
  if (!aligned16(w) || !aligned16(scales) || !aligned16(xq))
    return fail(QASR_ERR_UNSUPPORTED, std::string(what) + ": w, scales and xq must be 16-byte aligned");
  return QASR_OK;
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_linear_w8a8_packed(float* y, const int8_t* w_packed, const float* scales,
                                       const int8_t* xq, const float* x_scales, size_t batch,
                                       size_t in_dim, size_t out_dim, void* stream) {
  if (batch == 0 || out_dim == 0) return QASR_OK;
  QASR_REQUIRE(y, "linear_w8a8_packed: null pointer");
  const int rc = check_w8a8_common(w_packed, scales, xq, x_scales, batch, in_dim, out_dim, "linear_w8a8_packed");
  if (rc != QASR_OK) return rc;
  if (!aligned16(y) || (out_dim * 4) % 16 != 0)
    return fail(QASR_ERR_UNSUPPORTED, "linear_w8a8_packed: y must be 16-byte aligned");
  HeadsArgs a{};
  a.y = y;
  a.w = w_packed;
  a.scales = scales;
  a.xq = xq;
  a.xs = x_scales;
  a.batch = (int)batch;
  a.N = (int)out_dim;
  return launch_heads_gemm<0>(a, in_dim, as_stream(stream), "linear_w8a8_packed");
}

extern "C" int qasr_qkv_heads_w8a8_packed(float* q_out, float* k_cache, float* v_cache, size_t cache_rows,
                                          const int8_t* w_packed, const float* scales, const int8_t* xq,
                                          const float* x_scales, const float* q_norm_w,
                                          const float* k_norm_w, const float* cos_tab,
                                          const float* sin_tab, size_t table_rows,
                                          const int32_t* positions, size_t batch, size_t in_dim,
                                          size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                          float eps, void* stream) {
  if (batch == 0) return QASR_OK;
  QASR_REQUIRE(q_out && k_cache && v_cache && q_norm_w && k_norm_w && cos_tab && sin_tab && positions,
               "qkv_heads_w8a8_packed: null pointer");
  if (head_dim != 128)
    return fail(QASR_ERR_UNSUPPORTED, "qkv_heads_w8a8_packed: head_dim must be 128");
  QASR_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads <= 4096 && n_kv_heads <= 4096,
               "qkv_heads_w8a8_packed: head counts must be in [1, 4096]");
  const size_t N = (n_heads + 2 * n_kv_heads) * head_dim;
  const int rc = check_w8a8_common(w_packed, scales, xq, x_scales, batch, in_dim, N, "qkv_heads_w8a8_packed");
  if (rc != QASR_OK) return rc;
  size_t n;
  QASR_REQUIRE(cache_rows > 0 && mul_ok(batch, cache_rows, &n) && mul_ok(n, n_kv_heads * head_dim, &n),
               "qkv_heads_w8a8_packed: cache size overflows");
  if (!aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(q_norm_w) ||
      !aligned16(k_norm_w) || !aligned16(cos_tab) || !aligned16(sin_tab))
    return fail(QASR_ERR_UNSUPPORTED, "qkv_heads_w8a8_packed: buffers must be 16-byte aligned");
  HeadsArgs a{};
  a.q_out = q_out;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.w = w_packed;
  a.scales = scales;
  a.xq = xq;
  a.xs = x_scales;
  a.q_norm_w = q_norm_w;
  a.k_norm_w = k_norm_w;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.positions = positions;
  a.table_rows = (long long)table_rows;
  a.cache_rows = (long long)cache_rows;
  a.batch = (int)batch;
  a.N = (int)N;
  a.n_heads = (int)n_heads;
  a.n_kv_heads = (int)n_kv_heads;
  a.eps = eps;
  return launch_heads_gemm<1>(a, in_dim, as_stream(stream), "qkv_heads_w8a8_packed");
}
