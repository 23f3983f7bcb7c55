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
// reductions; the outputs are then summed with lanes over head dims, 16
// splits' rows in flight at a time. Splits with no keys carry sum 0 and max
// -1e30 and drop out. `o` points at the (row, head) output row.
template <int HD>
QASR_DEV void merge_splits(float* o, const float* ws_o, const float* ml, int nsplit, int lane) {
  constexpr int DPL = HD / 64;
  constexpr int B = 16;
  const bool has = lane < nsplit;
  const float mz = has ? ml[2 * lane] : -__builtin_inff();
  const float lz = has ? ml[2 * lane + 1] : 0.0f;
  const float mx = wave_max(mz);
  const float f = has ? expf(mz - mx) : 0.0f;
  const float lsum = wave_sum(lz * f);
  float acc[DPL];
#pragma unroll
  for (int d = 0; d < DPL; ++d) acc[d] = 0.0f;
  const float* ob = ws_o + lane * DPL;
  for (int z0 = 0; z0 < nsplit; z0 += B) {
    float ov[B][DPL];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const size_t z = (size_t)min(z0 + u, nsplit - 1);
#pragma unroll
      for (int d = 0; d < DPL; ++d) ov[u][d] = ob[z * HD + d];
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
// QK: a quad of lanes owns a key (lane l covers head dims 32*(l%4) .. +31 of
// key l/4), so each load instruction reads 16 keys x 64 contiguous bytes and
// the quad's partial dots meet with two DPP adds. PV: lanes over head dims,
// probabilities broadcast with readlane. The 4 waves' (max, sum, out) merge in
// LDS; the workgroup writes its unnormalised partial to the workspace.
template <int HD, int G>
__global__ __launch_bounds__(256) void attention_decode_split_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    int seq_q, int seq_k, int nk, float scale, int q_offset, int keys_per_split,
    float* __restrict__ ws_o, float* __restrict__ ws_ml) {
  constexpr int DPL = HD / 64;
  constexpr int DQ = HD / 4;   // head dims per lane of a quad
  constexpr int C4 = DQ / 4;   // float4 loads per key per lane
  __shared__ float cm[4][G], cl[4][G];
  __shared__ __align__(16) float co[4][G][HD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quarter = lane & 3, kq = lane >> 2;  // dim quarter, key within the wave's 16
  const int i = blockIdx.x, kh = blockIdx.y;
  const size_t q_stride = (size_t)nk * G * HD, kv_stride = (size_t)nk * HD;
  float4 qv[G][C4];
  const float* qr = q + (size_t)i * q_stride + (size_t)kh * G * HD + quarter * DQ;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int c = 0; c < C4; ++c) qv[g][c] = ld4(qr + g * HD, c);

  const int k_lim = min(q_offset + i + 1, seq_k);
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
  for (int t0 = k_begin + 16 * wave; t0 < k_end; t0 += 64) {
    const int nkeys = min(16, k_end - t0);  // this wave's keys in the tile (>= 1)
    const int j = min(kq, nkeys - 1);       // past them: repeat the last key, masked below
    const float* kr = k + (size_t)(t0 + j) * kv_stride + (size_t)kh * HD + quarter * DQ;
    float4 kk[C4];
#pragma unroll
    for (int c = 0; c < C4; ++c) kk[c] = ld4(kr, c);
    const float* vr = v + (size_t)t0 * kv_stride + (size_t)kh * HD + lane * DPL;
    float vv[16][DPL];
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
    // every load issued before the first use (the scheduler would otherwise
    // sink the v loads below the QK arithmetic: two round trips)
    __builtin_amdgcn_sched_barrier(0);
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
          for (int d = 0; d < DPL; ++d) o[g][d] = __builtin_fmaf(pj, vv[u][d], o[g][d]);
        }
      }
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

// Merges the partials of every (row, head), one wave each.
template <int HD>
__global__ __launch_bounds__(256) void attention_combine_kernel(float* __restrict__ out,
                                                                const float* __restrict__ ws_o,
                                                                const float* __restrict__ ws_ml,
                                                                long long rows_heads, int nsplit) {
  const int lane = threadIdx.x & 63;
  const long long rh = (long long)blockIdx.x * 4 + threadIdx.x / 64;  // row * n_heads + head
  if (rh >= rows_heads) return;
  merge_splits<HD>(out + (size_t)rh * HD, ws_o + (size_t)rh * nsplit * HD, ws_ml + (size_t)rh * nsplit * 2,
                   nsplit, lane);
}

template <int HD, int G>
void launch_attention_split(float* out, const float* q, const float* k, const float* v, int seq_q,
                            int seq_k, int nk, float scale, int q_offset, int nsplit,
                            int keys_per_split, float* ws_o, float* ws_ml, hipStream_t st) {
  const dim3 grid((unsigned)seq_q, (unsigned)nk, (unsigned)nsplit);
  if constexpr (G * HD <= 256) {  // the wave's loads fit the register file
    attention_decode_split_kernel<HD, G><<<grid, 256, 0, st>>>(q, k, v, seq_q, seq_k, nk, scale,
                                                              q_offset, keys_per_split, ws_o, ws_ml);
  } else {
    causal_attention_kernel<HD, G, 1, 1, true><<<grid, 64, 0, st>>>(
        out, q, k, v, seq_q, seq_k, nk, scale, q_offset, keys_per_split, ws_o, ws_ml);
  }
  const long long rows_heads = (long long)seq_q * nk * G;
  attention_combine_kernel<HD><<<(unsigned)((rows_heads + 3) / 4), 256, 0, st>>>(out, ws_o, ws_ml,
                                                                               rows_heads, nsplit);
}

// Prefill attention on the fp32 matrix cores (v_mfma_f32_16x16x4f32), for
// head_dim 128 and 1 or 2 q heads per kv head. Products and sums stay fp32;
// only the order of the terms of each dot product and of the key sum differ
// from the reference's sequential loops.
//
// A workgroup takes 16 query rows x the G heads of one kv head with 8 waves:
// group z (waves 4z..4z+3) walks the 64-key tiles z, z+2, ... of the rows'
// causal range, and the two groups' (max, sum, out) are merged at the end.
// Within a group, wave w owns keys 16w..16w+15 of a tile in the QK product and
// head dims 32w..32w+31 in the PV product.
//   QK, as S^T = K Q^T: A[i][k] (lane i+16k) = K[key i][dim 32k+s] and
//     B[k][j] (lane j+16k) = Q[query j][dim 32k+s] at step s = 0..31, so each
//     lane reads 32 contiguous floats of its key and of its query. The result
//     sits at lane j+16c, register r = S[query j][key 16w+4c+r].
//   softmax per query row over the tile: the wave's max/sum over its 16 keys
//     (registers, then lanes j, j+16, j+32, j+48), the tile's across the 4
//     waves through LDS; the running (max, sum, out) are rescaled once per tile
//     from the reference's initial max -1e30.
//   PV, as O = P V: step (kb, r) consumes keys 16kb+4c+r (c = the lane group),
//     A[i][c] = P[query i][that key] (one float4 LDS read covers r = 0..3) and
//     B[c][j] = V[that key][dim 32w+2j+jt]; the result sits at lane j+16c,
//     register r = O[query 4c+r][dim 32w+2j+jt].
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kPfStride = 68;  // LDS row of the P tile in floats (64 keys + pad)

QASR_DEV void ld_row32(float (&dst)[32], const float* p) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const float4 t = ld4(p, c);
    dst[4 * c] = t.x;
    dst[4 * c + 1] = t.y;
    dst[4 * c + 2] = t.z;
    dst[4 * c + 3] = t.w;
  }
}

template <int G>
__global__ __launch_bounds__(512) void attention_prefill_mfma_kernel(
    float* __restrict__ out, const float* __restrict__ q, const float* __restrict__ k,
    const float* __restrict__ v, int seq_q, int seq_k, int nk, float scale, int q_offset) {
  constexpr int HD = 128;
  __shared__ float red_max[2][4][G][16];
  __shared__ float red_sum[2][4][G][16];
  __shared__ float corr_l[2][G][16];
  __shared__ __align__(16) float pl[2][G][16][kPfStride];
  __shared__ float ml[2][G][16][2];
  __shared__ __align__(16) float ol[G][16][HD];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave >> 2, w = wave & 3;
  const int lo = lane & 15, hi = lane >> 4;
  const int i0 = ((int)gridDim.x - 1 - (int)blockIdx.x) * 16;  // longest rows first
  const int kh = blockIdx.y;
  const size_t q_stride = (size_t)nk * G * HD, kv_stride = (size_t)nk * HD;

  // keys [0, k_hi) cover every row of the block; tiles alternate between groups
  const int k_hi = min(q_offset + min(i0 + 16, seq_q), seq_k);
  const int ntiles = (k_hi + 63) / 64;
  const int nit = (ntiles + 1) / 2;
  const int k_lim = min(q_offset + i0 + lo + 1, seq_k);  // keys of this lane's query (QK side)

  float qf[G][32];
#pragma unroll
  for (int g = 0; g < G; ++g)
    ld_row32(qf[g], q + (size_t)min(i0 + lo, seq_q - 1) * q_stride + (size_t)(kh * G + g) * HD + 32 * hi);

  float m_run[G], l_run[G];
  v4f o[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -1e30f;  // the reference's initial running max
    l_run[g] = 0.0f;
    o[g][0] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    o[g][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const int last_key = seq_k > 0 ? seq_k - 1 : 0;
  const float* kbase = k + (size_t)kh * HD + 32 * hi;
  const float* vbase = v + (size_t)kh * HD + 32 * w + 2 * lo;
  float kf[32];
  if (nit > 0) ld_row32(kf, kbase + (size_t)min(min(grp, ntiles - 1) * 64 + 16 * w + lo, last_key) * kv_stride);

  for (int it = 0; it < nit; ++it) {
    const int t = 2 * it + grp;
    const bool tile_ok = t < ntiles;  // the odd group's last turn may have no tile
    const int tc = tile_ok ? t : ntiles - 1;
    float2 vf[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {  // u = 4 kb + r: key 16kb + 4hi + r of the tile
      const int key = min(tc * 64 + 16 * (u >> 2) + 4 * hi + (u & 3), last_key);
      vf[u] = *reinterpret_cast<const float2*>(vbase + (size_t)key * kv_stride);
    }
    v4f sacc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) sacc[g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 32; ++st)
#pragma unroll
      for (int g = 0; g < G; ++g) sacc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[st], qf[g][st], sacc[g], 0, 0, 0);
    if (it + 1 < nit)  // next tile's keys while the softmax and PV run
      ld_row32(kf, kbase + (size_t)min(min(t + 2, ntiles - 1) * 64 + 16 * w + lo, last_key) * kv_stride);

    float sv[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mx = -__builtin_inff();
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = t * 64 + 16 * w + 4 * hi + r;
        sv[g][r] = (tile_ok && key < k_lim) ? sacc[g][r] * scale : -__builtin_inff();
        mx = fmaxf(mx, sv[g][r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      if (hi == 0) red_max[grp][w][g][lo] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float tmax = red_max[grp][0][g][lo];
#pragma unroll
      for (int ww = 1; ww < 4; ++ww) tmax = fmaxf(tmax, red_max[grp][ww][g][lo]);
      const float m_new = fmaxf(m_run[g], tmax);
      const float corr = expf(m_run[g] - m_new);
      float p[4], sum = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = sv[g][r] == -__builtin_inff() ? 0.0f : expf(sv[g][r] - m_new);
        sum += p[r];
      }
      sum += __shfl_xor(sum, 16, 64);
      sum += __shfl_xor(sum, 32, 64);
      if (hi == 0) red_sum[grp][w][g][lo] = sum;
      *reinterpret_cast<float4*>(&pl[grp][g][lo][16 * w + 4 * hi]) = make_float4(p[0], p[1], p[2], p[3]);
      if (w == 0 && hi == 0) corr_l[grp][g][lo] = corr;
      m_run[g] = m_new;
      l_run[g] *= corr;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) l_run[g] += red_sum[grp][ww][g][lo];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float c = corr_l[grp][g][4 * hi + r];
        o[g][0][r] *= c;
        o[g][1][r] *= c;
      }
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 a4 = *reinterpret_cast<const float4*>(&pl[grp][g][lo][16 * kb + 4 * hi]);
        const float a[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[g][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], vf[4 * kb + r].x, o[g][0], 0, 0, 0);
          o[g][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], vf[4 * kb + r].y, o[g][1], 0, 0, 0);
        }
      }
  }

  // merge the two groups: group 1 hands its (max, sum) and outputs to group 0
  if (w == 0 && hi == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      ml[grp][g][lo][0] = m_run[g];
      ml[grp][g][lo][1] = l_run[g];
    }
  }
  if (grp == 1) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<float2*>(&ol[g][4 * hi + r][32 * w + 2 * lo]) = make_float2(o[g][0][r], o[g][1][r]);
  }
  __syncthreads();
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * hi + r;
        const float m0 = ml[0][g][row][0], l0 = ml[0][g][row][1];
        const float m1 = ml[1][g][row][0], l1 = ml[1][g][row][1];
        const float mx = fmaxf(m0, m1);
        const float f0 = expf(m0 - mx), f1 = expf(m1 - mx);
        const float lsum = __builtin_fmaf(l1, f1, l0 * f0);
        const float inv = lsum > 0.0f ? 1.0f / lsum : 1.0f;  // no scaling when the sum is 0
        const float2 o1 = *reinterpret_cast<const float2*>(&ol[g][row][32 * w + 2 * lo]);
        const float a0 = __builtin_fmaf(o1.x, f1, o[g][0][r] * f0) * inv;
        const float a1 = __builtin_fmaf(o1.y, f1, o[g][1][r] * f0) * inv;
        if (i0 + row < seq_q)
          *reinterpret_cast<float2*>(out + (size_t)(i0 + row) * q_stride + (size_t)(kh * G + g) * HD +
                                     32 * w + 2 * lo) = make_float2(a0, a1);
      }
  }
}

template <int HD, int G>
void launch_attention(float* out, const float* q, const float* k, const float* v, int seq_q,
                      int seq_k, int nk, float scale, int q_offset, hipStream_t st) {
  if constexpr (HD == 128 && (G == 1 || G == 2)) {
    if (seq_q >= 16) {  // prefill: the matrix-core kernel
      const dim3 grid((unsigned)((seq_q + 15) / 16), (unsigned)nk);
      attention_prefill_mfma_kernel<G><<<grid, 512, 0, st>>>(out, q, k, v, seq_q, seq_k, nk, scale, q_offset);
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
