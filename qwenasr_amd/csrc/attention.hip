// Causal grouped-query attention over a key/value block, the decoder's
// attention step (kernels/mod.rs:1124-1207):
//   for query row i (global position q_offset + i) and head h, with
//   kv head h / (n_heads / n_kv_heads) and keys j < min(q_offset + i + 1, seq_k):
//   out[i, h, :] = sum_j softmax_j(q[i,h,:] . k[j,kvh,:] * scale) v[j,kvh,:]
// q, out: [seq_q, n_heads * head_dim]; k, v: [seq_k, n_kv_heads * head_dim]
// (a KvCache layer block).
//
// The reference runs one online softmax per (row, head) over the keys in
// order, starting from a running max of -1e30, and scales by 1/sum at the
// end (no scaling when the sum is 0). Here keys are processed in tiles of 64:
//   - QK: lane l owns key 64t + l and dots it with the q rows of all heads of
//     the kv group (q broadcast from LDS), one 16-byte k load at a time;
//   - the tile's max and sum come from wave reductions, and the running
//     (max, sum, out) of each head is rescaled once per tile;
//   - PV: lanes own head dimensions; the tile's keys are walked in order, each
//     v row read with one coalesced wave load and its probability broadcast
//     with readlane.
// A workgroup holds R query rows of one kv head, S waves per row splitting the
// key tiles; the S partial (max, sum, out) triples of a row are merged in LDS.
// Prefill uses R = 4, S = 1 (the 4 rows' waves share k/v lines in L1); decode
// uses R = 1, S = 8.
#include "common.hpp"

namespace qasr {
namespace {

constexpr int kPvBatch = 16;  // v rows in flight per lane in the PV product

QASR_DEV float bcast_lane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// PARTIAL: workgroup z covers keys [z * keys_per_split, (z + 1) * keys_per_split)
// and writes its unnormalised (max, sum, out) per head to the workspace
// (ws_o [seq_q][n_heads][nsplit][HD], ws_ml [seq_q][n_heads][nsplit][2]).
template <int HD, int G, int R, int S, bool PARTIAL = false>
__global__ __launch_bounds__(64 * R * S) void causal_attention_kernel(
    float* __restrict__ out, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, int seq_q, int seq_k, int nk, float scale, int q_offset,
    int keys_per_split = 0, float* __restrict__ ws_o = nullptr, float* __restrict__ ws_ml = nullptr) {
  constexpr int DPL = HD / 64;  // head dims per lane in the PV product
  constexpr int NW = R * S;
  __shared__ __align__(16) float qs[R][G][HD];
  __shared__ float cm[NW][G];
  __shared__ float cl[NW][G];
  __shared__ __align__(16) float co[S > 1 ? NW : 1][G][HD];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rr = wave / S, sp = wave % S;
  const int kh = blockIdx.y;
  const int i = blockIdx.x * R + rr;
  const bool row_ok = i < seq_q;
  int k_end = row_ok ? min(q_offset + i + 1, seq_k) : 0;
  int k_begin = 0;
  if constexpr (PARTIAL) {
    k_begin = min(k_end, (int)blockIdx.z * keys_per_split);
    k_end = min(k_end, k_begin + keys_per_split);
  }
  const size_t q_stride = (size_t)nk * G * HD, kv_stride = (size_t)nk * HD;

  if (sp == 0 && row_ok) {
    const float* qr = q + (size_t)i * q_stride + (size_t)kh * G * HD;
    for (int t = lane; t < G * HD; t += 64) qs[rr][t / HD][t % HD] = qr[t];
  }
  __syncthreads();

  float m[G], l[G], o[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -1e30f;  // the reference's initial running max
    l[g] = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[g][d] = 0.0f;
  }

  const int ntiles = (k_end - k_begin + 63) / 64;
  for (int t = sp; t < ntiles; t += S) {
    const int j = k_begin + t * 64 + lane;
    const bool kv = j < k_end;
    // QK: this lane's key against every head of the group
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = 0.0f;
    const float* kr = k + (size_t)(kv ? j : 0) * kv_stride + (size_t)kh * HD;
#pragma unroll 8
    for (int c = 0; c < HD / 4; ++c) {
      const float4 kk = ld4(kr, c);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 qq = *reinterpret_cast<const float4*>(&qs[rr][g][4 * c]);
        s[g] = __builtin_fmaf(qq.x, kk.x, s[g]);
        s[g] = __builtin_fmaf(qq.y, kk.y, s[g]);
        s[g] = __builtin_fmaf(qq.z, kk.z, s[g]);
        s[g] = __builtin_fmaf(qq.w, kk.w, s[g]);
      }
    }
    // online softmax update, one rescale per tile
    float p[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float sc = kv ? s[g] * scale : -__builtin_inff();
      const float mn = fmaxf(m[g], wave_max(sc));
      const float corr = expf(m[g] - mn);
      p[g] = kv ? expf(sc - mn) : 0.0f;
      l[g] = l[g] * corr + wave_sum(p[g]);
#pragma unroll
      for (int d = 0; d < DPL; ++d) o[g][d] *= corr;
      m[g] = mn;
    }
    // PV: keys of the tile in order, lanes over head dims. The v rows of 16
    // keys are loaded before their FMAs so their latencies overlap (past the
    // tile's last key the loads repeat that key and are not accumulated).
    const int nkeys = min(64, k_end - (k_begin + t * 64));
    const float* vr = v + (size_t)(k_begin + t * 64) * kv_stride + (size_t)kh * HD + lane * DPL;
    for (int j0 = 0; j0 < nkeys; j0 += kPvBatch) {
      float vv[kPvBatch][DPL];
#pragma unroll
      for (int u = 0; u < kPvBatch; ++u) {
        const size_t jj = (size_t)min(j0 + u, nkeys - 1);
        if constexpr (DPL == 2) {
          const float2 t2 = *reinterpret_cast<const float2*>(vr + jj * kv_stride);
          vv[u][0] = t2.x;
          vv[u][1] = t2.y;
        } else {
          vv[u][0] = vr[jj * kv_stride];
        }
      }
#pragma unroll
      for (int u = 0; u < kPvBatch; ++u) {
        if (j0 + u < nkeys) {  // uniform across the wave
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float pj = bcast_lane(p[g], j0 + u);
#pragma unroll
            for (int d = 0; d < DPL; ++d) o[g][d] = __builtin_fmaf(pj, vv[u][d], o[g][d]);
          }
        }
      }
    }
  }

  // merge the S key splits of a row
  if constexpr (S > 1) {
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        cm[wave][g] = m[g];
        cl[wave][g] = l[g];
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int d = 0; d < DPL; ++d) co[wave][g][lane * DPL + d] = o[g][d];
    __syncthreads();
    if (sp == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mx = cm[rr * S][g];
        for (int w = 1; w < S; ++w) mx = fmaxf(mx, cm[rr * S + w][g]);
        float lsum = 0.0f, acc[DPL];
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] = 0.0f;
        for (int w = 0; w < S; ++w) {
          const float f = expf(cm[rr * S + w][g] - mx);
          lsum = __builtin_fmaf(cl[rr * S + w][g], f, lsum);
#pragma unroll
          for (int d = 0; d < DPL; ++d) acc[d] = __builtin_fmaf(co[rr * S + w][g][lane * DPL + d], f, acc[d]);
        }
        m[g] = mx;  // the merged triple is relative to the row's overall max
        l[g] = lsum;
#pragma unroll
        for (int d = 0; d < DPL; ++d) o[g][d] = acc[d];
      }
    }
  }
  if constexpr (PARTIAL) {
    if (sp == 0 && row_ok) {
      const int nsplit = gridDim.z;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const size_t slot = ((size_t)i * nk * G + (size_t)kh * G + g) * nsplit + blockIdx.z;
#pragma unroll
        for (int d = 0; d < DPL; ++d) ws_o[slot * HD + lane * DPL + d] = o[g][d];
        if (lane == 0) {
          ws_ml[2 * slot] = m[g];
          ws_ml[2 * slot + 1] = l[g];
        }
      }
    }
    return;
  }
  if (sp == 0 && row_ok) {
    float* orow = out + (size_t)i * q_stride + (size_t)kh * G * HD;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float inv = l[g] > 0.0f ? 1.0f / l[g] : 1.0f;  // no scaling when the sum is 0
#pragma unroll
      for (int d = 0; d < DPL; ++d) orow[g * HD + lane * DPL + d] = o[g][d] * inv;
    }
  }
}

// Sum over the 4 lanes of a quad (lanes 4a..4a+3), every lane gets it.
QASR_DEV float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));  // lane ^ 1
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));  // lane ^ 2
  return v;
}

// Merges the nsplit (<= 64) partials of one (row, head) with one wave: lane z
// reads split z's (max, sum) so the overall max and the rescaled sum are wave
// reductions; the outputs are then summed with lanes over head dims, B
// splits' rows in flight at a time (the same sum in the same order for any
// B). Splits with no keys carry sum 0 and max -1e30 and drop out. `o` points
// at the (row, head) output row.
template <int HD, int B = 16>
QASR_DEV void merge_splits(float* o, const float* ws_o, const float* ml, int nsplit, int lane) {
  constexpr int DPL = HD / 64;
  const float* ob = ws_o + lane * DPL;
  // the first B splits' output rows do not depend on the maxima: their loads
  // go out with the (max, sum) loads, one memory round trip for both
  float ov[B][DPL];
#pragma unroll
  for (int u = 0; u < B; ++u) {
    const size_t z = (size_t)min(u, nsplit - 1);
#pragma unroll
    for (int d = 0; d < DPL; ++d) ov[u][d] = ob[z * HD + d];
  }
  const bool has = lane < nsplit;
  const float mz = has ? ml[2 * lane] : -__builtin_inff();
  const float lz = has ? ml[2 * lane + 1] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
  const float mx = wave_max(mz);
  const float f = has ? expf(mz - mx) : 0.0f;
  const float lsum = wave_sum(lz * f);
  float acc[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] = 0.0f;
  for (int z0 = 0; z0 < nsplit; z0 += B) {
    if (z0 > 0) {
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const size_t z = (size_t)min(z0 + u, nsplit - 1);
#pragma unroll
        for (int d = 0; d < DPL; ++d) ov[u][d] = ob[z * HD + d];
      }
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (z0 + u < nsplit) {  // uniform
        const float fz = bcast_lane(f, z0 + u);
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] = __builtin_fmaf(ov[u][d], fz, acc[d]);
      }
    }
  }
  const float inv = lsum > 0.0f ? 1.0f / lsum : 1.0f;
#pragma unroll
  for (int d = 0; d < DPL; ++d) o[lane * DPL + d] = acc[d] * inv;
}

// Decode-shaped split: one 4-wave workgroup per (row, kv head, key split)
// walks whole 64-key tiles; wave w owns keys 16w .. 16w+15 of each tile, so
// every SIMD of the CU has its own loads in flight. Each wave issues all k and
// v loads of its 16 keys before using any (one memory round trip per tile).
// QK: a quad of lanes owns a key; load instruction c gives lane l the head
// dims 16c + 4(l%4) .. +3 of key l/4, so the quad reads 64 contiguous bytes
// of its key row (the 16 keys of an instruction touch 16 cache lines, each
// line completed by the next instruction), and the quad's partial dots meet
// with two DPP adds. PV: lanes over head dims,
// probabilities broadcast with readlane. The 4 waves' (max, sum, out) merge in
// LDS; the workgroup writes its unnormalised partial to the workspace.
// The decode step's q/k head RMSNorm + RoPE and KV-cache store, done inside
// the split kernel (PRE): q, k, v are the raw projection outputs of the one
// token at position pos; cos_row/sin_row the RoPE table rows of pos; k_row,
// v_row the layer's cache rows of pos.
struct DecodePre {
  const float* k;
  const float* v;
  const float* q_norm_w;
  const float* k_norm_w;
  const float* cos_row;
  const float* sin_row;
  float* k_row;
  float* v_row;
  float eps;
};

// Batched decode streams (BATCH): row i is stream i, its keys are rows
// 0..positions[i] of its own cache block (k + i * cache_rows * kv_dim), cut
// into chunks of keys_per_split keys (blockIdx.z = chunk; a chunk past the
// stream's last key has no work and returns at once). A stream whose keys
// fit one chunk gets its normalised output row written by that workgroup;
// a longer one leaves one partial per chunk in the workspace (gridDim.z
// slots per (stream, head)) for attention_combine_batch_kernel. A position
// outside the cache gives NaN rows.
struct DecodeBatch {
  const int32_t* positions;
  long long cache_rows;
  float* out;
  const int32_t* order;  // optional: [batch][2] (stream, position), the longest streams first
};

template <int HD, int G, bool PRE = false, bool BATCH = false>
__global__ __launch_bounds__(256) void attention_decode_split_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    int seq_q, int seq_k, int nk, float scale, int q_offset, int keys_per_split,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, DecodePre pre = DecodePre{},
    DecodeBatch batch = DecodeBatch{}) {
  static_assert(!(PRE && BATCH), "one decode stream or a batch of them");
  constexpr int DPL = HD / 64;
  constexpr int DQ = HD / 4;   // head dims per lane of a quad
  constexpr int C4 = DQ / 4;   // float4 loads per key per lane
  __shared__ float cm[4][G], cl[4][G];
  __shared__ __align__(16) float co[4][G][HD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quarter = lane & 3, kq = lane >> 2;  // dim quarter, key within the wave's 16
  // BATCH: blockIdx.x = rank * nk + kv head. Workgroup n runs on XCD n % 8,
  // so with the head fastest one stream's heads fall on different XCDs and
  // every XCD gets the same share of each stream's keys (stream-fastest put
  // all of stream m on XCD m % 8: 15% slower at positions U[0,2047]). The
  // rank is the stream itself, or with batch.order the stream of that rank
  // in longest-first order (its position comes with it: one 8-byte load), so
  // the longest walks are dispatched first and the short ones fill the tail.
  // The stream's entry in `positions` is loaded beside it (off the critical
  // path): an order computed for other positions (stale) makes this stream's
  // rows and chunk partials NaN, since the merge counts chunks from
  // `positions`.
  const int rank = BATCH ? (int)(blockIdx.x / (unsigned)nk) : 0;
  [[maybe_unused]] long long order_pos = 0;
  [[maybe_unused]] bool stale = false;
  int i = BATCH ? rank : (int)blockIdx.x;
  if constexpr (BATCH) {
    if (batch.order) {
      const int2 e = reinterpret_cast<const int2*>(batch.order)[rank];
      if ((unsigned)e.x >= gridDim.x / (unsigned)nk) return;  // not an order of this batch: nothing read
      i = e.x;
      order_pos = e.y;
      stale = (long long)batch.positions[i] != order_pos;  // waited for where it is used
    }
  }
  const int kh = BATCH ? (int)(blockIdx.x % (unsigned)nk) : (int)blockIdx.y;
  const size_t q_stride = (size_t)nk * G * HD, kv_stride = (size_t)nk * HD;
  float4 qv[G][C4];
  [[maybe_unused]] bool bad_pos = false;
  int k_lim;
  if constexpr (BATCH) {
    const long long p = batch.order ? order_pos : (long long)batch.positions[i];
    bad_pos = p < 0 || p >= batch.cache_rows;
    k_lim = bad_pos ? 0 : (int)p + 1;
    if ((int)blockIdx.z * keys_per_split >= max(k_lim, 1)) {  // uniform: a chunk with no keys
      if (stale && gridDim.z > 1 && wave == 0) {  // the merge may read this chunk: make it NaN
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const size_t slot = ((size_t)i * nk * G + (size_t)kh * G + g) * gridDim.z + blockIdx.z;
#pragma unroll
          for (int d = 0; d < DPL; ++d) ws_o[slot * HD + lane * DPL + d] = qnan();
          if (lane == 0) ws_ml[2 * slot] = ws_ml[2 * slot + 1] = qnan();
        }
      }
      return;
    }
    k += (size_t)i * (size_t)batch.cache_rows * kv_stride;
    v += (size_t)i * (size_t)batch.cache_rows * kv_stride;
  } else {
    k_lim = min(q_offset + i + 1, seq_k);
  }
  const int k_begin = min(k_lim, (int)blockIdx.z * keys_per_split);
  const int k_end = min(k_lim, k_begin + keys_per_split);
  float m[G], l[G], o[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -1e30f;
    l[g] = 0.0f;
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[g][d] = 0.0f;
  }

  // A tile: this wave's keys t0 .. t0 + 15 (past k_end: repeat the last key,
  // masked in process_tile).
  // Cached loads: the K/V rows of all layers (235 MB at 28 layers x 1024
  // positions of the 1.7B shape) stay in the last-level cache from one decode
  // step to the next while the weights stream past it nontemporally;
  // nontemporal K/V loads measured 895 -> 956 us per decoded token.
  auto load_tile = [&](int t0, float4 (&kk)[C4], float (&vv)[16][DPL]) {
    const int nkeys = min(16, k_end - t0);
    const int j = min(kq, nkeys - 1);
    const float* kr = k + (size_t)(t0 + j) * kv_stride + (size_t)kh * HD + 4 * quarter;
#pragma unroll
    for (int c = 0; c < C4; ++c) kk[c] = ld4(kr, 4 * c);
    const float* vr = v + (size_t)t0 * kv_stride + (size_t)kh * HD + lane * DPL;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const size_t jj = (size_t)min(u, nkeys - 1);
      if constexpr (DPL == 2) {
        const float2 t2 = *reinterpret_cast<const float2*>(vr + jj * kv_stride);
        vv[u][0] = t2.x;
        vv[u][1] = t2.y;
      } else {
        vv[u][0] = vr[jj * kv_stride];
      }
    }
  };
  // with use_vlast, the tile's last key takes its v row from vlast
  auto process_tile = [&](int t0, const float4 (&kk)[C4], const float (&vv)[16][DPL], bool use_vlast,
                          const float (&vlast)[DPL]) {
    const int nkeys = min(16, k_end - t0);
    const bool key_ok = kq < nkeys;
    float p[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < C4; ++c) {
        a = __builtin_fmaf(qv[g][c].x, kk[c].x, a);
        a = __builtin_fmaf(qv[g][c].y, kk[c].y, a);
        a = __builtin_fmaf(qv[g][c].z, kk[c].z, a);
        a = __builtin_fmaf(qv[g][c].w, kk[c].w, a);
      }
      a = quad_sum(a);
      const float sc = key_ok ? a * scale : -__builtin_inff();
      const float mn = fmaxf(m[g], wave_max(sc));
      const float corr = expf(m[g] - mn);
      p[g] = key_ok ? expf(sc - mn) : 0.0f;
      l[g] = l[g] * corr + wave_sum(quarter == 0 ? p[g] : 0.0f);  // one copy of each key per quad
#pragma unroll
      for (int d = 0; d < DPL; ++d) o[g][d] *= corr;
      m[g] = mn;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (u < nkeys) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float pj = bcast_lane(p[g], 4 * u);
#pragma unroll
          for (int d = 0; d < DPL; ++d) {
            const float vx = (use_vlast && u == nkeys - 1) ? vlast[d] : vv[u][d];
            o[g][d] = __builtin_fmaf(pj, vx, o[g][d]);
          }
        }
      }
    }
  };

  int t0 = k_begin + 16 * wave;
  [[maybe_unused]] const int pos = k_lim - 1;  // PRE: the new key, the last of the last split
  [[maybe_unused]] const bool last = blockIdx.z == gridDim.z - 1;
  // PRE: the tile holding key pos takes that row from LDS (kpos, vpos). Key
  // pos is the last of the last split, so it is the last key of its tile:
  // the lanes whose key it is get kpos, and the PV sum takes vpos (vlast)
  // for the tile's last key. Returns whether the tile holds key pos.
  auto patch = [&](int t, float4 (&kk)[C4], float (&vlast)[DPL], const float* kpos, const float* vpos) {
    if (!(last && pos >= t && pos < t + 16)) return false;  // uniform
    const int nkeys = min(16, k_end - t);
    if (min(kq, nkeys - 1) == nkeys - 1) {
#pragma unroll
      for (int c = 0; c < C4; ++c) kk[c] = *reinterpret_cast<const float4*>(&kpos[16 * c + 4 * quarter]);
    }
#pragma unroll
    for (int d = 0; d < DPL; ++d) vlast[d] = vpos[lane * DPL + d];
    return true;
  };
  [[maybe_unused]] const float* kpos_p = nullptr;
  [[maybe_unused]] const float* vpos_p = nullptr;
  if constexpr (PRE) {
    // One token (i == 0). The wave's first tile is loaded before the
    // prologue (it does not depend on it). Groups of HD/8 lanes, in the
    // layout of the head kernel: groups 0..G-1 normalise and rotate this kv
    // head's q heads into LDS; in the split that holds key pos (the last),
    // group G writes the normalised, rotated k row into the cache and group
    // G+1 the v row, both also into LDS. The tile holding key pos takes that
    // row from LDS (its loads may predate the cache writes), so nothing in
    // this launch reads the new cache rows (no other workgroup reads them
    // either) and the barrier waits for LDS only, not for the global loads
    // and stores in flight.
    constexpr int L = HD / 8, HALF = HD / 2;
    static_assert((G + 2) * L <= 256, "prologue groups fit the workgroup");
    __shared__ __align__(16) float qs[G][HD];
    __shared__ __align__(16) float kpos[HD], vpos[HD];
    float4 kk0[C4];
    float vv0[16][DPL];
    const bool first = t0 < k_end;  // uniform per wave
    if (first) load_tile(t0, kk0, vv0);
    __builtin_amdgcn_sched_barrier(0);
    const int grp = threadIdx.x / L, sub = threadIdx.x % L;
    kpos_p = kpos;
    vpos_p = vpos;
    if (grp < G || (last && grp == G)) {
      const bool is_q = grp < G;
      const float* src = is_q ? q + (size_t)(kh * G + grp) * HD : pre.k + (size_t)kh * HD;
      const float* w = is_q ? pre.q_norm_w : pre.k_norm_w;
      const float4 w1 = ld4(w, sub), w2 = ld4(w + HALF, sub);
      const float4 c1 = ld4(pre.cos_row, sub), c2 = ld4(pre.cos_row + HALF, sub);
      const float4 s1 = ld4(pre.sin_row, sub), s2 = ld4(pre.sin_row + HALF, sub);
      float4 x1 = ld4(src, sub), x2 = ld4(src + HALF, sub);
      head_norm_rope<HD, true, true>(x1, x2, w1, w2, c1, c2, s1, s2, true, pre.eps);
      float* dst = is_q ? &qs[grp][0] : kpos;
      st4(dst, sub, x1);
      st4(dst + HALF, sub, x2);
      if (!is_q) {
        float* kr = pre.k_row + (size_t)kh * HD;
        st4(kr, sub, x1);
        st4(kr + HALF, sub, x2);
      }
    } else if (last && grp == G + 1) {
      const float* src = pre.v + (size_t)kh * HD;
      float* dst = pre.v_row + (size_t)kh * HD;
      const float4 v1 = ld4(src, sub), v2 = ld4(src + HALF, sub);
      st4(dst, sub, v1);
      st4(dst + HALF, sub, v2);
      st4(vpos, sub, v1);
      st4(vpos + HALF, sub, v2);
    }
    lds_barrier();
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int c = 0; c < C4; ++c) qv[g][c] = *reinterpret_cast<const float4*>(&qs[g][16 * c + 4 * quarter]);
    if (first) {
      float vlast[DPL];
      const bool hit = patch(t0, kk0, vlast, kpos, vpos);
      process_tile(t0, kk0, vv0, hit, vlast);
      t0 += 64;
    }
  } else {
    const float* qr = q + (size_t)i * q_stride + (size_t)kh * G * HD + 4 * quarter;
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int c = 0; c < C4; ++c) qv[g][c] = ld4(qr + g * HD, 4 * c);
  }
  // The remaining tiles, two register buffers deep: the next tile's loads are
  // issued before the current tile is processed, so a wave keeps a tile in
  // flight while it computes (a stream's many tiles in the batched form).
  // Every load of a tile is issued before its first use (the scheduler would
  // otherwise sink the v loads below the QK arithmetic: two round trips).
  auto run_tile = [&](int t, float4 (&kk)[C4], float (&vv)[16][DPL]) {
    float vlast[DPL];
    bool hit = false;
    if constexpr (PRE) hit = patch(t, kk, vlast, kpos_p, vpos_p);
    process_tile(t, kk, vv, hit, vlast);
  };
  if (t0 < k_end) {
    float4 kka[C4], kkb[C4];
    float vva[16][DPL], vvb[16][DPL];
    load_tile(t0, kka, vva);
    for (; t0 < k_end; t0 += 128) {
      const bool more = t0 + 64 < k_end;  // uniform per wave
      if (more) load_tile(t0 + 64, kkb, vvb);
      __builtin_amdgcn_sched_barrier(0);
      run_tile(t0, kka, vva);
      if (!more) break;
      if (t0 + 128 < k_end) load_tile(t0 + 128, kka, vva);
      __builtin_amdgcn_sched_barrier(0);
      run_tile(t0 + 64, kkb, vvb);
    }
  }
  // merge the 4 waves
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      cm[wave][g] = m[g];
      cl[wave][g] = l[g];
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int d = 0; d < DPL; ++d) co[wave][g][lane * DPL + d] = o[g][d];
  __syncthreads();
  const int nsplit = gridDim.z;
  if (wave == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mx = fmaxf(fmaxf(cm[0][g], cm[1][g]), fmaxf(cm[2][g], cm[3][g]));
      float lsum = 0.0f, acc[DPL];
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = expf(cm[w][g] - mx);
        lsum = __builtin_fmaf(cl[w][g], f, lsum);
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] = __builtin_fmaf(co[w][g][lane * DPL + d], f, acc[d]);
      }
      if (BATCH && stale) {  // the row and (if there are chunks) this chunk's partial are NaN
        float* orow = batch.out + ((size_t)i * nk * G + (size_t)kh * G + g) * HD;
#pragma unroll
        for (int d = 0; d < DPL; ++d) orow[lane * DPL + d] = qnan();
        if (nsplit > 1) {
          const size_t slot = ((size_t)i * nk * G + (size_t)kh * G + g) * nsplit + blockIdx.z;
#pragma unroll
          for (int d = 0; d < DPL; ++d) ws_o[slot * HD + lane * DPL + d] = qnan();
          if (lane == 0) ws_ml[2 * slot] = ws_ml[2 * slot + 1] = qnan();
        }
      } else if (BATCH && k_lim <= keys_per_split) {  // the whole key range: normalise as the merge kernel does
        const float inv = lsum > 0.0f ? 1.0f / lsum : 1.0f;
        float* orow = batch.out + ((size_t)i * nk * G + (size_t)kh * G + g) * HD;
#pragma unroll
        for (int d = 0; d < DPL; ++d) orow[lane * DPL + d] = bad_pos ? qnan() : acc[d] * inv;
      } else {
        const size_t slot = ((size_t)i * nk * G + (size_t)kh * G + g) * nsplit + blockIdx.z;
#pragma unroll
        for (int d = 0; d < DPL; ++d) ws_o[slot * HD + lane * DPL + d] = acc[d];
        if (lane == 0) {
          ws_ml[2 * slot] = mx;
          ws_ml[2 * slot + 1] = lsum;
        }
      }
    }
  }
}

// Merges the chunk partials of the batched decode streams whose keys span
// more than one chunk, one wave per (stream, q head); the rows of the other
// streams were written by the attention kernel itself.
template <int HD>
__global__ __launch_bounds__(256) void attention_combine_batch_kernel(float* __restrict__ out,
                                                                      const float* __restrict__ ws_o,
                                                                      const float* __restrict__ ws_ml,
                                                                      const int32_t* __restrict__ positions,
                                                                      long long cache_rows, int heads,
                                                                      long long rows_heads, int nchunk,
                                                                      int keys_per_chunk) {
  const int lane = threadIdx.x & 63;
  const long long rh = (long long)blockIdx.x * 4 + threadIdx.x / 64;  // stream * heads + head
  if (rh >= rows_heads) return;
  const long long p = positions[rh / heads];
  if (p < 0 || p >= cache_rows || p + 1 <= keys_per_chunk) return;
  const int used = (int)((p + keys_per_chunk) / keys_per_chunk);
  merge_splits<HD>(out + (size_t)rh * HD, ws_o + (size_t)rh * nchunk * HD, ws_ml + (size_t)rh * nchunk * 2,
                   used, lane);
}

// The batched attention with each stream's row quantized per row (the W8A8
// o projection's input): one workgroup per stream, one wave per q head (up to
// 16, then looping). A wave merges its head's chunk partials as
// attention_combine_batch_kernel does, or reads back the row the attention
// kernel normalised itself (one chunk, or a NaN row for a position outside the
// cache), into an LDS copy of the stream's row (and out); then the row's int8
// values and scale follow quantize.rs:633-662 exactly as qasr_quantize_rows_i8
// computes them (absmax where NaN never wins, scale = absmax / 127, the same
// rounding), so q and scale equal that kernel's on out.
template <int HD>
__global__ __launch_bounds__(1024) void attention_combine_quant_kernel(
    float* __restrict__ out, int8_t* __restrict__ out_q, float* __restrict__ out_scales,
    const float* __restrict__ ws_o, const float* __restrict__ ws_ml, const int32_t* __restrict__ positions,
    long long cache_rows, int heads, int nchunk, int keys_per_chunk) {
  extern __shared__ __align__(16) float q_row[];  // [heads * HD]
  __shared__ float red[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int m = blockIdx.x;
  const long long p = positions[m];
  const bool bad = p < 0 || p >= cache_rows;
  const int used = bad ? 1 : (int)((p + keys_per_chunk) / keys_per_chunk);
  const size_t row0 = (size_t)m * heads;
  for (int h = wave; h < heads; h += nwaves) {
    float* o = out + (row0 + h) * HD;
    if (used > 1) {
      merge_splits<HD>(q_row + h * HD, ws_o + (row0 + h) * nchunk * HD, ws_ml + (row0 + h) * nchunk * 2, used,
                       lane);
      constexpr int DPL = HD / 64;  // merge_splits' lane mapping: each lane copies out the values it wrote
#pragma unroll
      for (int d = 0; d < DPL; ++d) o[lane * DPL + d] = q_row[h * HD + lane * DPL + d];
    } else {
      for (int d = lane; d < HD; d += 64) q_row[h * HD + d] = o[d];
    }
  }
  __syncthreads();
  const int n = heads * HD;
  float mx = 0.0f;
  for (int c = threadIdx.x; c < n; c += blockDim.x) {
    const float a = fabsf(q_row[c]);
    if (a > mx) mx = a;  // NaN never wins
  }
  mx = wave_max(mx);  // then over the nwaves waves present (the max is exact in any order)
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
  for (int w = 1; w < nwaves; ++w) mx = red[w] > mx ? red[w] : mx;
  const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
  if (threadIdx.x == 0) out_scales[m] = mx / 127.0f;
  for (int c = threadIdx.x; c < n; c += blockDim.x) out_q[(size_t)m * n + c] = (int8_t)quant_i8(q_row[c], inv);
}

// Merges the partials of every (row, head), one one-wave workgroup each: a
// decode token's 16 heads then load their partials on 16 CUs, in one round
// trip each, instead of four heads' worth per CU (1.7B decode step at
// position 1023: 834.7 -> 824.6 us).
template <int HD>
__global__ __launch_bounds__(64) void attention_combine_kernel(float* __restrict__ out,
                                                                const float* __restrict__ ws_o,
                                                                const float* __restrict__ ws_ml,
                                                                long long rows_heads, int nsplit) {
  const int lane = threadIdx.x & 63;
  const long long rh = (long long)blockIdx.x;  // row * n_heads + head
  if (rh >= rows_heads) return;
  // every split's row in one memory round trip: 32 in flight past 16 splits
  // (attn_decode at position 2047, 32 splits: 308.5 -> 299.3 us for 28
  // layers; 32 in flight at 16 splits re-load the last one and cost 1%)
  if (nsplit > 16)
    merge_splits<HD, 32>(out + (size_t)rh * HD, ws_o + (size_t)rh * nsplit * HD,
                         ws_ml + (size_t)rh * nsplit * 2, nsplit, lane);
  else
    merge_splits<HD>(out + (size_t)rh * HD, ws_o + (size_t)rh * nsplit * HD, ws_ml + (size_t)rh * nsplit * 2,
                     nsplit, lane);
}

template <int HD, int G>
void launch_attention_split(float* out, const float* q, const float* k, const float* v, int seq_q,
                            int seq_k, int nk, float scale, int q_offset, int nsplit,
                            int keys_per_split, float* ws_o, float* ws_ml, hipStream_t st,
                            const DecodePre* pre = nullptr) {
  const dim3 grid((unsigned)seq_q, (unsigned)nk, (unsigned)nsplit);
  if constexpr (G * HD <= 256) {  // the wave's loads fit the register file
    if (pre)
      attention_decode_split_kernel<HD, G, true><<<grid, 256, 0, st>>>(
          q, k, v, seq_q, seq_k, nk, scale, q_offset, keys_per_split, ws_o, ws_ml, *pre);
    else
      attention_decode_split_kernel<HD, G><<<grid, 256, 0, st>>>(q, k, v, seq_q, seq_k, nk, scale,
                                                                q_offset, keys_per_split, ws_o, ws_ml);
  } else {
    causal_attention_kernel<HD, G, 1, 1, true><<<grid, 64, 0, st>>>(
        out, q, k, v, seq_q, seq_k, nk, scale, q_offset, keys_per_split, ws_o, ws_ml);
  }
  const long long rows_heads = (long long)seq_q * nk * G;
  attention_combine_kernel<HD><<<(unsigned)rows_heads, 64, 0, st>>>(out, ws_o, ws_ml,
                                                                               rows_heads, nsplit);
}

// Prefill attention on the fp32 matrix cores (v_mfma_f32_16x16x4f32), for
// head_dim 128. Products and sums stay fp32; only the order of the terms of
// each dot product and of the key sum differ from the reference's sequential
// loops.
//
// The 16 columns of the products are (query row, head) pairs: R = 16 / G
// consecutive rows x the G q heads of one kv head, column c = g * R + i, so
// the heads sharing a kv head share every k and v load. A workgroup of NW
// waves takes one such block; wave w walks the 64-key tiles w, w + NW, ... of
// the block's causal range as a complete online softmax of its own, and the
// NW (max, sum, out) triples are merged at the end. Per tile and wave:
//   QK, as S^T = K Q^T, one 16-key block kb at a time: A[i][k] (lane i+16k) =
//     K[key 16kb+i][dim d] and B[k][c] (lane c+16k) = Q[column c][dim d] at
//     step s = 0..31 with d = 16(s/4) + 4k + s%4 (a bijection of the 128
//     dims; each load instruction reads 64 contiguous bytes of a row). The
//     result sits at lane c+16h, register r = S[column c][key 16kb+4h+r].
//   softmax per column over the tile: 16 scores per lane, then lanes c, c+16,
//     c+32, c+48; the running (max, sum, out) are rescaled once per tile from
//     the reference's initial max -1e30.
//   PV, as O = P V: step (kb, r) consumes keys 16kb+4h+r (h = the lane
//     group), so A[c][h] = P[column c][that key] is the probability the lane
//     already holds, and B[h][j] = V[that key][dim 4j + jt%4 + 64(jt/4)] for
//     the 8 output tiles jt (whole 128-byte lines per load instruction); the
//     result sits at lane j+16h, register r = O[column 4h+r][that dim].
typedef float v4f __attribute__((ext_vector_type(4)));
// Key-tile streams per workgroup. Two waves per SIMD, so a CU holds two 4-wave
// workgroups (measured at T=512, 0.6B: 30.5 us; 8 waves per workgroup, one
// workgroup per CU: 47.7 us). The kernel asks for that occupancy explicitly:
// the compiler then keeps the accumulators in VGPRs (222, no AGPRs) instead
// of 190 VGPRs + 64 AGPRs with accumulator copies between the two files
// (prefill step 3004 -> 2985 us). Loading all of a tile's V rows where the
// source issues them (pinned with scheduling fences) takes the last registers
// and measured slower in the step (3006 us): the compiler loads each V block
// just before its products, which the step's L2-resident K/V rows tolerate.
constexpr int kPrefillWaves = 4;

// dims 16c + 4h .. 16c + 4h + 3 (c = 0..7) of a row, for lane group h (p points
// at dim 4h): one load instruction reads 64 contiguous bytes per row
QASR_DEV void ld_row32(float (&dst)[32], const float* p) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float4 t = ld4(p, 4 * c);
    dst[4 * c] = t.x;
    dst[4 * c + 1] = t.y;
    dst[4 * c + 2] = t.z;
    dst[4 * c + 3] = t.w;
  }
}

// v rows of keys key0 + r (r = 0..3), dims 4j..4j+3 and 64+4j..64+4j+3 for
// lane j (vbase points at dim 4j): dst[8r + jt]
QASR_DEV void ld_v_block(float (&dst)[32], const float* vbase, size_t kv_stride, int key0,
                         int last_key) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float* p = vbase + (size_t)min(key0 + r, last_key) * kv_stride;
    const float4 a = ld4(p, 0), b = ld4(p, 16);
    dst[8 * r] = a.x;
    dst[8 * r + 1] = a.y;
    dst[8 * r + 2] = a.z;
    dst[8 * r + 3] = a.w;
    dst[8 * r + 4] = b.x;
    dst[8 * r + 5] = b.y;
    dst[8 * r + 6] = b.z;
    dst[8 * r + 7] = b.w;
  }
}

template <int G, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_prefill_mfma_kernel(
    float* __restrict__ out, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, int seq_q, int seq_k, int nk, float scale, int q_offset) {
  constexpr int HD = 128;
  constexpr int R = 16 / G;  // query rows per block
  __shared__ float ml[NW][16][2];
  __shared__ __align__(16) float ol[NW - 1][16][HD];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int lo = lane & 15, hi = lane >> 4;
  // Items (row block, kv head) ranked heaviest first; workgroups i and i + n/2
  // take ranks i and n-1-i, so the two workgroups a CU holds at once pair a
  // long causal range with a short one.
  const int n_items = (int)gridDim.x, half = (n_items + 1) / 2, wid = (int)blockIdx.x;
  const int rank = wid < half ? wid : n_items - 1 - (wid - half);
  const int nblk = n_items / nk;
  const int i0 = (nblk - 1 - rank / nk) * R;
  const int kh = rank % nk;
  const size_t q_stride = (size_t)nk * G * HD, kv_stride = (size_t)nk * HD;

  // keys [0, k_hi) cover every row of the block
  const int k_hi = min(q_offset + min(i0 + R, seq_q), seq_k);
  const int ntiles = (k_hi + 63) / 64;
  // this lane's QK column: row i0 + lo % R, head lo / R
  const int k_lim = min(q_offset + i0 + lo % R + 1, seq_k);
  const int last_key = seq_k > 0 ? seq_k - 1 : 0;

  float m_run = -1e30f;  // the reference's initial running max
  float l_run = 0.0f;
  v4f o[8];
#pragma unroll
  for (int jt = 0; jt < 8; ++jt) o[jt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  if (w < ntiles) {
    float qf[32];
    ld_row32(qf, q + (size_t)min(i0 + lo % R, seq_q - 1) * q_stride + (size_t)(kh * G + lo / R) * HD + 4 * hi);
    const float* kbase = k + (size_t)kh * HD + 4 * hi;
    const float* vbase = v + (size_t)kh * HD + 4 * lo;
    float ka[32], kb1[32];
    ld_row32(ka, kbase + (size_t)min(w * 64 + lo, last_key) * kv_stride);
    ld_row32(kb1, kbase + (size_t)min(w * 64 + 16 + lo, last_key) * kv_stride);
    for (int t = w; t < ntiles; t += NW) {
      const int key0 = t * 64;
      // QK: key blocks 0 and 1 from the prefetched rows, 2 and 3 loaded meanwhile
      float kc[32], kd[32];
      ld_row32(kc, kbase + (size_t)min(key0 + 32 + lo, last_key) * kv_stride);
      ld_row32(kd, kbase + (size_t)min(key0 + 48 + lo, last_key) * kv_stride);
      v4f sacc[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) sacc[b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 32; ++st) {
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[st], qf[st], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kb1[st], qf[st], sacc[1], 0, 0, 0);
      }
      float va[32], vb[32];
      ld_v_block(va, vbase, kv_stride, key0 + 4 * hi, last_key);
      ld_v_block(vb, vbase, kv_stride, key0 + 16 + 4 * hi, last_key);
#pragma unroll
      for (int st = 0; st < 32; ++st) {
        sacc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[st], qf[st], sacc[2], 0, 0, 0);
        sacc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(kd[st], qf[st], sacc[3], 0, 0, 0);
      }
      float vc[32], vd[32];
      ld_v_block(vc, vbase, kv_stride, key0 + 32 + 4 * hi, last_key);
      ld_v_block(vd, vbase, kv_stride, key0 + 48 + 4 * hi, last_key);

      // online softmax over the tile's 64 keys, per column
      float sv[4][4];
      float mx = -__builtin_inff();
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = key0 + 16 * b + 4 * hi + r;
          sv[b][r] = key < k_lim ? sacc[b][r] * scale : -__builtin_inff();
          mx = fmaxf(mx, sv[b][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const float corr = expf(m_run - m_new);
      float sum = 0.0f;
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[b][r] = sv[b][r] == -__builtin_inff() ? 0.0f : expf(sv[b][r] - m_new);
          sum += sv[b][r];
        }
      sum += __shfl_xor(sum, 16, 64);
      sum += __shfl_xor(sum, 32, 64);
      l_run = __builtin_fmaf(l_run, corr, sum);
      m_run = m_new;
      // The tile's P V goes into a zeroed accumulator and is added to the
      // corrected running O after the tile (O = O corr + P V per column; O =
      // P V on the wave's first tile), so the matrix-core chain never waits
      // on the VALU correction of registers it is accumulating into.
      v4f ot[8];
#pragma unroll
      for (int jt = 0; jt < 8; ++jt) ot[jt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      // next tile's first two key blocks while PV runs
      const int tn = t + NW < ntiles ? t + NW : t;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) ot[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[0][r], va[8 * r + jt], ot[jt], 0, 0, 0);
      ld_row32(ka, kbase + (size_t)min(tn * 64 + lo, last_key) * kv_stride);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) ot[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[1][r], vb[8 * r + jt], ot[jt], 0, 0, 0);
      ld_row32(kb1, kbase + (size_t)min(tn * 64 + 16 + lo, last_key) * kv_stride);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) ot[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[2][r], vc[8 * r + jt], ot[jt], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) ot[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[3][r], vd[8 * r + jt], ot[jt], 0, 0, 0);
      if (t == w) {
#pragma unroll
        for (int jt = 0; jt < 8; ++jt) o[jt] = ot[jt];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float c = __shfl(corr, 4 * hi + r, 64);
#pragma unroll
          for (int jt = 0; jt < 8; ++jt) o[jt][r] = __builtin_fmaf(o[jt][r], c, ot[jt][r]);
        }
      }
    }
  }

  // merge the NW waves' (max, sum, out) in wave 0; a wave without tiles
  // carries max -1e30 and sum 0 and drops out
  if (hi == 0) {
    ml[w][lo][0] = m_run;
    ml[w][lo][1] = l_run;
  }
  if (w > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = &ol[w - 1][4 * hi + r][4 * lo];
      *reinterpret_cast<float4*>(dst) = make_float4(o[0][r], o[1][r], o[2][r], o[3][r]);
      *reinterpret_cast<float4*>(dst + 64) = make_float4(o[4][r], o[5][r], o[6][r], o[7][r]);
    }
  }
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = 4 * hi + r;
      float mx = ml[0][col][0];
#pragma unroll
      for (int u = 1; u < NW; ++u) mx = fmaxf(mx, ml[u][col][0]);
      const float f0 = expf(ml[0][col][0] - mx);
      float lsum = ml[0][col][1] * f0;
      float acc[8];
#pragma unroll
      for (int jt = 0; jt < 8; ++jt) acc[jt] = o[jt][r] * f0;
#pragma unroll
      for (int u = 1; u < NW; ++u) {
        const float f = expf(ml[u][col][0] - mx);
        lsum = __builtin_fmaf(ml[u][col][1], f, lsum);
        const float4 a = *reinterpret_cast<const float4*>(&ol[u - 1][col][4 * lo]);
        const float4 b = *reinterpret_cast<const float4*>(&ol[u - 1][col][4 * lo + 64]);
        acc[0] = __builtin_fmaf(a.x, f, acc[0]);
        acc[1] = __builtin_fmaf(a.y, f, acc[1]);
        acc[2] = __builtin_fmaf(a.z, f, acc[2]);
        acc[3] = __builtin_fmaf(a.w, f, acc[3]);
        acc[4] = __builtin_fmaf(b.x, f, acc[4]);
        acc[5] = __builtin_fmaf(b.y, f, acc[5]);
        acc[6] = __builtin_fmaf(b.z, f, acc[6]);
        acc[7] = __builtin_fmaf(b.w, f, acc[7]);
      }
      const float inv = lsum > 0.0f ? 1.0f / lsum : 1.0f;  // no scaling when the sum is 0
      const int row = i0 + col % R, head = kh * G + col / R;
      if (row < seq_q) {
        float* dst = out + (size_t)row * q_stride + (size_t)head * HD + 4 * lo;
        st4(dst, 0, make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv));
        st4(dst, 16, make_float4(acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv));
      }
    }
  }
}

template <int HD, int G>
void launch_attention(float* out, const float* q, const float* k, const float* v, int seq_q,
                      int seq_k, int nk, float scale, int q_offset, hipStream_t st) {
  if constexpr (HD == 128) {
    if (seq_q >= 16 / G) {  // prefill: the matrix-core kernel, 16 / G rows per workgroup
      const unsigned items = (unsigned)((seq_q + 16 / G - 1) / (16 / G)) * (unsigned)nk;
      attention_prefill_mfma_kernel<G, kPrefillWaves><<<items, 64 * kPrefillWaves, 0, st>>>(
          out, q, k, v, seq_q, seq_k, nk, scale, q_offset);
      return;
    }
  }
  // enough (row, kv head) pairs to fill the chip: 4 rows per workgroup, one
  // wave each; otherwise 8 waves split every row's keys
  if ((long long)seq_q * nk >= 1024) {
    const dim3 grid((unsigned)((seq_q + 3) / 4), (unsigned)nk);
    causal_attention_kernel<HD, G, 4, 1><<<grid, 256, 0, st>>>(out, q, k, v, seq_q, seq_k, nk, scale, q_offset);
  } else {
    const dim3 grid((unsigned)seq_q, (unsigned)nk);
    causal_attention_kernel<HD, G, 1, 8><<<grid, 512, 0, st>>>(out, q, k, v, seq_q, seq_k, nk, scale, q_offset);
  }
}

struct SplitPlan {
  int nsplit = 0, keys_per_split = 0;
  float* ws_o = nullptr;
  float* ws_ml = nullptr;
};

template <int HD>
bool dispatch_group(int G, float* out, const float* q, const float* k, const float* v, int seq_q,
                    int seq_k, int nk, float scale, int q_offset, const SplitPlan& sp,
                    hipStream_t st) {
#define QASR_ATTN_CASE(GG)                                                                       \
  case GG:                                                                                       \
    if (sp.nsplit > 1)                                                                           \
      launch_attention_split<HD, GG>(out, q, k, v, seq_q, seq_k, nk, scale, q_offset, sp.nsplit, \
                                     sp.keys_per_split, sp.ws_o, sp.ws_ml, st);                 \
    else                                                                                         \
      launch_attention<HD, GG>(out, q, k, v, seq_q, seq_k, nk, scale, q_offset, st);            \
    return true;
  switch (G) {
    QASR_ATTN_CASE(1)
    QASR_ATTN_CASE(2)
    QASR_ATTN_CASE(4)
    QASR_ATTN_CASE(8)
    default: return false;
  }
#undef QASR_ATTN_CASE
}

// Key-split plan: workgroups of whole 64-key tiles, aiming at about 1024
// workgroups, at most kMaxSplits splits; nothing to gain when there are
// already many (row, kv head) pairs or few keys. Workspace layout: the
// partial outputs [seq_q][n_heads][nsplit][head_dim], then the (max, sum)
// pairs [seq_q][n_heads][nsplit][2]. (Merging in the last-finishing
// workgroup instead of a second kernel needs an agent-scope fence per
// workgroup -- a whole-L2 writeback and invalidate -- and measured 2x slower.)
constexpr int kMaxSplits = 64;

SplitPlan plan_split(size_t seq_q, size_t seq_k, size_t nk, size_t q_offset, size_t head_dim,
                     size_t n_heads, float* workspace, size_t workspace_floats) {
  SplitPlan p;
  const size_t k_max = seq_k < q_offset + seq_q ? seq_k : q_offset + seq_q;
  const size_t pairs = seq_q * nk;
  if (!workspace || pairs >= 512 || k_max < 256) return p;
  size_t want = (1024 + pairs - 1) / pairs;
  const size_t by_len = k_max / 64;
  if (want > by_len) want = by_len;
  if (want > (size_t)kMaxSplits) want = kMaxSplits;
  if (want < 2) return p;
  const size_t need = seq_q * n_heads * want * (head_dim + 2);
  if (need > workspace_floats) return p;
  p.nsplit = (int)want;
  p.keys_per_split = (int)(((k_max + want - 1) / want + 63) / 64 * 64);
  p.nsplit = (int)((k_max + p.keys_per_split - 1) / p.keys_per_split);
  p.ws_o = workspace;
  p.ws_ml = p.ws_o + seq_q * n_heads * (size_t)p.nsplit * head_dim;
  return p;
}

}  // namespace
}  // namespace qasr

using namespace qasr;

static int attention_impl(float* out, const float* q, const float* k, const float* v, size_t seq_q,
                          size_t seq_k, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                          float scale, size_t q_offset, float* workspace, size_t workspace_floats,
                          void* stream) {
  if (seq_q == 0 || n_heads == 0) return QASR_OK;
  QASR_REQUIRE(out && q, "causal_attention: null pointer");
  QASR_REQUIRE(seq_k == 0 || (k && v), "causal_attention: null k or v");
  QASR_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "causal_attention: n_heads must be a multiple of n_kv_heads");
  QASR_REQUIRE(seq_q < 0x40000000u && seq_k < 0x40000000u && q_offset < 0x40000000u &&
                   n_heads <= 65536,
               "causal_attention: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(seq_q, n_heads * head_dim, &n) && mul_ok(seq_k, n_kv_heads * head_dim, &n),
               "causal_attention: size overflows");
  const size_t G = n_heads / n_kv_heads;
  const bool ok_shape = (head_dim == 64 || head_dim == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
  if (!ok_shape || !aligned16(q) || !aligned16(out) || (seq_k && (!aligned16(k) || !aligned16(v)))) {
    return fail(QASR_ERR_UNSUPPORTED,
                "causal_attention: needs head_dim 64 or 128, n_heads/n_kv_heads in {1,2,4,8} "
                "and 16-byte aligned buffers");
  }
  QASR_REQUIRE(!workspace || aligned16(workspace), "causal_attention: workspace must be 16-byte aligned");
  hipStream_t st = as_stream(stream);
  const int sq = (int)seq_q, sk = (int)seq_k, nk = (int)n_kv_heads, qo = (int)q_offset;
  const SplitPlan sp = plan_split(seq_q, seq_k, n_kv_heads, q_offset, head_dim, n_heads, workspace,
                                  workspace_floats);
  if (head_dim == 64)
    dispatch_group<64>((int)G, out, q, k, v, sq, sk, nk, scale, qo, sp, st);
  else
    dispatch_group<128>((int)G, out, q, k, v, sq, sk, nk, scale, qo, sp, st);
  return launch_status("causal_attention");
}

extern "C" int qasr_causal_attention_f32(float* out, const float* q, const float* k, const float* v,
                                         size_t seq_q, size_t seq_k, size_t n_heads,
                                         size_t n_kv_heads, size_t head_dim, float scale,
                                         size_t q_offset, void* stream) {
  return attention_impl(out, q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset,
                        nullptr, 0, stream);
}

extern "C" int qasr_decode_attention_f32(float* out, float* q, const float* k, const float* v,
                                         const float* q_norm_w, const float* k_norm_w,
                                         const float* cos_tab, const float* sin_tab,
                                         size_t table_rows, size_t pos, size_t n_heads,
                                         size_t n_kv_heads, size_t head_dim, float eps, float scale,
                                         float* k_cache, float* v_cache, size_t cache_rows,
                                         float* workspace, size_t workspace_floats, void* stream) {
  if (n_heads == 0) return QASR_OK;
  QASR_REQUIRE(out && q && k && v && q_norm_w && k_norm_w && cos_tab && sin_tab && k_cache && v_cache,
               "decode_attention: null pointer");
  QASR_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "decode_attention: n_heads must be a multiple of n_kv_heads");
  QASR_REQUIRE(pos < table_rows && pos < cache_rows,
               "decode_attention: pos must lie inside the RoPE table and the cache");
  QASR_REQUIRE(pos < 0x40000000u && n_heads <= 65536 && head_dim <= 4096,
               "decode_attention: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(cache_rows, n_kv_heads * head_dim, &n), "decode_attention: size overflows");
  const size_t G = n_heads / n_kv_heads, kv_dim = n_kv_heads * head_dim;
  const SplitPlan sp = plan_split(1, pos + 1, n_kv_heads, pos, head_dim, n_heads, workspace,
                                  workspace_floats);
  const bool fused_shape = (head_dim == 128 && (G == 1 || G == 2)) ||
                           (head_dim == 64 && (G == 1 || G == 2 || G == 4));
  const bool aligned = aligned16(out) && aligned16(q) && aligned16(k) && aligned16(v) &&
                       aligned16(q_norm_w) && aligned16(k_norm_w) && aligned16(cos_tab) &&
                       aligned16(sin_tab) && aligned16(k_cache) && aligned16(v_cache) &&
                       (!workspace || aligned16(workspace));
  if (sp.nsplit > 1 && fused_shape && aligned) {
    DecodePre pre{k, v, q_norm_w, k_norm_w, cos_tab + pos * head_dim, sin_tab + pos * head_dim,
                  k_cache + pos * kv_dim, v_cache + pos * kv_dim, eps};
    hipStream_t st = as_stream(stream);
    const int nk = (int)n_kv_heads, sk = (int)pos + 1, qo = (int)pos;
#define QASR_PRE(HD, GG)                                                                         \
  if (head_dim == HD && G == GG) {                                                               \
    launch_attention_split<HD, GG>(out, q, k_cache, v_cache, 1, sk, nk, scale, qo, sp.nsplit,    \
                                   sp.keys_per_split, sp.ws_o, sp.ws_ml, st, &pre);             \
    return launch_status("decode_attention");                                                    \
  }
    QASR_PRE(128, 1) QASR_PRE(128, 2) QASR_PRE(64, 1) QASR_PRE(64, 2) QASR_PRE(64, 4)
#undef QASR_PRE
  }
  // short contexts and other shapes: the two calls this one stands for
  int rc = qasr_head_rms_norm_rope_kv_f32(q, k, v, q_norm_w, k_norm_w, cos_tab, sin_tab, nullptr, pos, 1,
                                          n_heads, n_kv_heads, head_dim, table_rows, eps, k_cache,
                                          v_cache, cache_rows, stream);
  if (rc != QASR_OK) return rc;
  return attention_impl(out, q, k_cache, v_cache, 1, pos + 1, n_heads, n_kv_heads, head_dim, scale, pos,
                        workspace, workspace_floats, stream);
}

// Keys per chunk of the batched decode attention: 512 (a 2 MB stream-head
// walk becomes at most 4 workgroups, which evens out streams at different
// positions), more for caches over 32768 rows so that a row has at most 64
// chunks (one merge wave's lanes).
static size_t batched_chunk_keys(size_t cache_rows) {
  const size_t c = (cache_rows + kMaxSplits - 1) / kMaxSplits;
  const size_t r = (c + 63) / 64 * 64;
  return r > 512 ? r : 512;
}

namespace qasr {
namespace {
// order[r] = (stream, position) of the stream of rank r when the streams are
// sorted by their number of keys (position + 1; 0 outside the cache),
// most first, ties by stream index: a strict total order, so the ranks are a
// permutation. Each thread ranks one stream against all of them, 1024
// positions at a time through LDS (batch^2 comparisons).
__global__ __launch_bounds__(256) void batched_order_kernel(int32_t* __restrict__ order,
                                                            const int32_t* __restrict__ positions, int batch,
                                                            long long cache_rows) {
  __shared__ __align__(16) int keys[1024];
  auto key_of = [&](int j) {
    const long long p = positions[j];
    return (p < 0 || p >= cache_rows) ? 0 : (int)p + 1;
  };
  const int i = (int)blockIdx.x * 256 + (int)threadIdx.x;
  const int ki = i < batch ? key_of(i) : 0;
  int rank = 0;
  for (int base = 0; base < batch; base += 1024) {
    const int n = min(1024, batch - base);
    __syncthreads();
    for (int t = (int)threadIdx.x; t < n; t += 256) keys[t] = key_of(base + t);
    __syncthreads();
    if (i < batch) {
      // four keys per LDS read (n is a multiple of 4 except in the last block)
      const int n4 = n & ~3;
#pragma unroll 4
      for (int t = 0; t < n4; t += 4) {
        const int4 kk = *reinterpret_cast<const int4*>(&keys[t]);
        const int j = base + t;
        rank += (kk.x > ki) || (kk.x == ki && j < i);
        rank += (kk.y > ki) || (kk.y == ki && j + 1 < i);
        rank += (kk.z > ki) || (kk.z == ki && j + 2 < i);
        rank += (kk.w > ki) || (kk.w == ki && j + 3 < i);
      }
      for (int t = n4; t < n; ++t) rank += (keys[t] > ki) || (keys[t] == ki && base + t < i);
    }
  }
  if (i < batch) {
    order[2 * rank] = i;
    order[2 * rank + 1] = positions[i];
  }
}
}  // namespace
}  // namespace qasr

extern "C" int qasr_batched_decode_order_i32(int32_t* order, const int32_t* positions, size_t batch,
                                             size_t cache_rows, void* stream) {
  if (batch == 0) return QASR_OK;
  QASR_REQUIRE(order && positions, "batched_decode_order: null pointer");
  QASR_REQUIRE(batch <= 65536 && cache_rows > 0 && cache_rows < 0x40000000u,
               "batched_decode_order: batch must be at most 65536 and cache_rows in [1, 2^30)");
  batched_order_kernel<<<(unsigned)((batch + 255) / 256), 256, 0, as_stream(stream)>>>(
      order, positions, (int)batch, (long long)cache_rows);
  return launch_status("batched_decode_order");
}

// 0 also when the size would overflow (such a call is rejected anyway).
extern "C" size_t qasr_batched_decode_attention_workspace_floats(size_t batch, size_t n_heads, size_t head_dim,
                                                                 size_t cache_rows) {
  if (cache_rows == 0 || cache_rows >= 0x40000000u) return 0;
  const size_t nchunk = (cache_rows + batched_chunk_keys(cache_rows) - 1) / batched_chunk_keys(cache_rows);
  size_t n = 0;
  if (nchunk <= 1 || !mul_ok(batch, n_heads, &n) || !mul_ok(n, nchunk, &n) || !mul_ok(n, head_dim + 2, &n))
    return 0;
  return n;
}

extern "C" int qasr_batched_decode_attention_f32(float* out, const float* q, const float* k_cache,
                                                 const float* v_cache, size_t cache_rows,
                                                 const int32_t* positions, size_t batch, size_t n_heads,
                                                 size_t n_kv_heads, size_t head_dim, float scale,
                                                 float* workspace, size_t workspace_floats, int8_t* out_q,
                                                 float* out_scales, const int32_t* order, void* stream) {
  if (batch == 0 || n_heads == 0) return QASR_OK;
  QASR_REQUIRE(out && q && k_cache && v_cache && positions, "batched_decode_attention: null pointer");
  QASR_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "batched_decode_attention: n_heads must be a multiple of n_kv_heads");
  QASR_REQUIRE(batch <= 0x7fffffffu && n_kv_heads <= 65535 && cache_rows > 0 && cache_rows < 0x40000000u,
               "batched_decode_attention: size too large");
  size_t n;
  QASR_REQUIRE(mul_ok(batch, cache_rows, &n) && mul_ok(n, n_kv_heads * head_dim, &n) &&
                   mul_ok(batch, n_heads * head_dim, &n),
               "batched_decode_attention: size overflows");
  const size_t G = n_heads / n_kv_heads;
  const bool shape = (head_dim == 128 && (G == 1 || G == 2)) || (head_dim == 64 && (G == 1 || G == 2 || G == 4));
  if (!shape || !aligned16(out) || !aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(QASR_ERR_UNSUPPORTED,
                "batched_decode_attention: needs head_dim 128 with n_heads/n_kv_heads <= 2 (or 64 with <= 4) "
                "and 16-byte aligned buffers");
  // chunked when a workspace is given, else one workgroup per (stream, kv head) over all its keys
  const size_t need = qasr_batched_decode_attention_workspace_floats(batch, n_heads, head_dim, cache_rows);
  QASR_REQUIRE(!workspace || workspace_floats >= need,
               "batched_decode_attention: workspace smaller than "
               "qasr_batched_decode_attention_workspace_floats()");
  QASR_REQUIRE(!out_q == !out_scales, "batched_decode_attention: out_q and out_scales go together");
  QASR_REQUIRE(!out_q || n_heads * head_dim * 4 <= 65536,
               "batched_decode_attention: a quantized row must fit 64 KiB of LDS");
  const bool chunked = workspace && need > 0;
  const int kpc = chunked ? (int)batched_chunk_keys(cache_rows) : (int)cache_rows;
  const int nchunk = (int)((cache_rows + kpc - 1) / kpc);
  const size_t rows_heads = batch * n_heads;
  float* ws_o = chunked ? workspace : nullptr;
  float* ws_ml = chunked ? workspace + rows_heads * nchunk * head_dim : nullptr;
  const DecodeBatch b{positions, (long long)cache_rows, out, order};
  QASR_REQUIRE(batch * n_kv_heads <= 0x7fffffffu, "batched_decode_attention: batch * n_kv_heads too large");
  const dim3 grid((unsigned)(batch * n_kv_heads), 1, (unsigned)nchunk);
  hipStream_t st = as_stream(stream);
  const int nk = (int)n_kv_heads;
  const unsigned qthreads = (unsigned)(64 * (n_heads < 16 ? n_heads : 16));
#define QASR_BATCH(HD, GG)                                                                                 \
  if (head_dim == HD && G == GG) {                                                                         \
    attention_decode_split_kernel<HD, GG, false, true><<<grid, 256, 0, st>>>(                             \
        q, k_cache, v_cache, 1, (int)cache_rows, nk, scale, 0, kpc, ws_o, ws_ml, DecodePre{}, b);          \
    if (out_q)                                                                                             \
      attention_combine_quant_kernel<HD><<<(unsigned)batch, qthreads, n_heads * HD * 4, st>>>(           \
          out, out_q, out_scales, ws_o, ws_ml, positions, (long long)cache_rows, (int)n_heads, nchunk,      \
          kpc);                                                                                            \
    else if (chunked)                                                                                      \
      attention_combine_batch_kernel<HD><<<(unsigned)((rows_heads + 3) / 4), 256, 0, st>>>(               \
          out, ws_o, ws_ml, positions, (long long)cache_rows, (int)n_heads, (long long)rows_heads, nchunk, \
          kpc);                                                                                            \
  }
  QASR_BATCH(128, 1) QASR_BATCH(128, 2) QASR_BATCH(64, 1) QASR_BATCH(64, 2) QASR_BATCH(64, 4)
#undef QASR_BATCH
  return launch_status("batched_decode_attention");
}

extern "C" size_t qasr_causal_attention_workspace_floats(size_t seq_q, size_t n_heads,
                                                         size_t head_dim) {
  return seq_q * n_heads * (size_t)kMaxSplits * (head_dim + 2);
}

extern "C" int qasr_causal_attention_split_f32(float* out, const float* q, const float* k,
                                               const float* v, size_t seq_q, size_t seq_k,
                                               size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                               float scale, size_t q_offset, float* workspace,
                                               size_t workspace_floats, void* stream) {
  return attention_impl(out, q, k, v, seq_q, seq_k, n_heads, n_kv_heads, head_dim, scale, q_offset,
                        workspace, workspace_floats, stream);
}
