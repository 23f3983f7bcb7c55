// Per-head q/k RMSNorm, NeoX RoPE, their fusion, and RoPE table fill.
//
// Layout: q [seq, n_heads, head_dim], k [seq, n_kv_heads, head_dim], fp32,
// row-major. RoPE tables are RopeCache rows [pos, head_dim] with duplicated
// halves ([c(0..half) | c(0..half)]), built by rope_table_kernel.
//
// Vector path (head_dim in {64,128,256,512}): L = head_dim/8 lanes own one head;
// lane j of a head holds elements [4j, 4j+4) and [half+4j, half+4j+4) as two
// float4, which are exactly the NeoX rotation partners. A wave covers 64/L
// heads (4 heads at head_dim 128) and a head's sum of squares is a log2(L)-step
// shuffle reduction inside its lane group; no LDS and no barrier.
#include "common.hpp"

namespace qasr {
namespace {


struct HeadArgs {
  float* q;
  float* k;
  const float* qw;
  const float* kw;
  const float* cos_tab;
  const float* sin_tab;
  const int32_t* positions;
  long long q_heads;      // seq * n_heads
  long long total_heads;  // seq * (n_heads + n_kv_heads)
  int nq;
  int nk;
  long long table_rows;
  float eps;
  // KV-cache epilogue (head_rms_norm_rope_kv): k and v rows are read from
  // k_src/v and written to the cache at row (stream * cache_rows + pos), with
  // pos = positions[s] and stream = s when positions are given, else
  // pos = start_pos + s and stream = 0 (the reference's single sequence).
  const float* k_src;
  const float* v;
  float* k_cache;
  float* v_cache;
  long long kv_heads_end;  // q_heads + seq * n_kv_heads
  long long start_pos;
  long long cache_rows;
};

// Resolves global head index gh to its base pointer, norm weight and row.
QASR_DEV void head_of(const HeadArgs& a, long long gh, int hd, float** base, const float** w,
                      long long* row) {
  if (gh < a.q_heads) {
    *base = a.q + gh * hd;
    *w = a.qw;
    *row = gh / a.nq;
  } else {
    const long long g = gh - a.q_heads;
    *base = a.k + g * hd;
    *w = a.kw;
    *row = g / a.nk;
  }
}

// KV mode: head gh is a q head (in place), a k head (read k_src, write the
// cache) or a v head (copied to the cache). head_kv_src resolves the source,
// gain, row and kv head h without touching memory and returns the kind (0 q,
// 1 k, 2 v); head_kv_dst places the result once the row's position p is known.
QASR_DEV int head_kv_src(const HeadArgs& a, long long gh, int hd, const float** src,
                         const float** w, long long* row, long long* h) {
  *h = 0;
  if (gh < a.q_heads) {
    *row = gh / a.nq;
    *src = a.q + gh * hd;
    *w = a.qw;
    return 0;
  }
  const bool k = gh < a.kv_heads_end;
  const long long g = gh - (k ? a.q_heads : a.kv_heads_end);
  *row = g / a.nk;
  *h = g - *row * a.nk;
  *src = k ? a.k_src + g * hd : a.v + g * hd;
  *w = k ? a.kw : nullptr;
  return k ? 1 : 2;
}

QASR_DEV float* head_kv_dst(const HeadArgs& a, int kind, long long gh, int hd, long long row,
                            long long h, long long p, bool ok) {
  if (kind == 0) return a.q + gh * hd;
  const long long stream = a.positions ? row : 0;
  const long long cache_off = ((stream * a.cache_rows + (ok ? p : 0)) * a.nk + h) * hd;
  return (kind == 1 ? a.k_cache : a.v_cache) + cache_off;
}

constexpr int kHeadBlock = 128;  // threads per workgroup of the vector head kernel

template <int HD, bool NORM, bool ROPE, bool KV = false>
__global__ __launch_bounds__(kHeadBlock) void head_vec_kernel(HeadArgs a) {
  constexpr int L = HD / 8;
  constexpr int HPW = kWave / L;
  constexpr int HALF = HD / 2;
  const int lane = threadIdx.x & (kWave - 1);
  const int sub = lane & (L - 1);
  const long long gh =
      ((long long)blockIdx.x * (kHeadBlock / kWave) + threadIdx.x / kWave) * HPW + lane / L;
  if (gh >= a.total_heads) return;  // whole lane groups leave together
  float* base;        // where the result goes
  const float* src;   // where the head is read
  const float* w;
  long long row;
  long long pos = 0;
  bool pos_ok = true;
  int kind = 0;
  long long kvh = 0;
  if constexpr (KV) {
    kind = head_kv_src(a, gh, HD, &src, &w, &row, &kvh);
  } else {
    head_of(a, gh, HD, &base, &w, &row);
    src = base;
  }

  // Two memory round trips: the head row, gains and position together, then
  // the table rows, the only loads that depend on another. The row and gains
  // are issued first because the wait on the position (a load under a branch
  // on `positions`) covers everything issued before it. The fences keep the
  // scheduler from sinking the table loads next to the rotation.
  float4 x1 = ld4_nt(src, sub);
  float4 x2 = ld4_nt(src + HALF, sub);
  float4 w1, w2;
  if constexpr (NORM) {
    if (!KV || kind != 2) {
      w1 = ld4(w, sub);
      w2 = ld4(w + HALF, sub);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (KV) {
    pos = a.positions ? (long long)a.positions[row] : a.start_pos + row;
  } else if constexpr (ROPE) {
    pos = a.positions ? (long long)a.positions[row] : row;
  }
  float4 c1, c2, s1, s2;
  if constexpr (KV) {
    pos_ok = pos >= 0 && pos < a.table_rows && pos < a.cache_rows;
    base = head_kv_dst(a, kind, gh, HD, row, kvh, pos, pos_ok);
  } else if constexpr (ROPE) {
    pos_ok = pos >= 0 && pos < a.table_rows;
  }
  if (ROPE && (!KV || kind != 2)) {
    const long long pr = pos_ok ? pos : 0;  // out-of-table rows read row 0, then become NaN
    const float* cr = a.cos_tab + pr * HD;
    const float* sr = a.sin_tab + pr * HD;
    c1 = ld4(cr, sub); c2 = ld4(cr + HALF, sub);
    s1 = ld4(sr, sub); s2 = ld4(sr + HALF, sub);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (KV) {
    if (kind == 2) {  // v: a plain copy into the cache (decoder.rs:550, 895)
      if (pos_ok) {
        st4_nt(base, sub, x1);
        st4_nt(base + HALF, sub, x2);
      }
      return;  // the head's lane group leaves together
    }
  }
  // The rotation runs on every row (an out-of-table row rotates by table row
  // 0) and is then replaced by NaN, so the table loads are used on every path.
  head_norm_rope<HD, NORM, ROPE>(x1, x2, w1, w2, c1, c2, s1, s2, true, a.eps);
  if (ROPE && !pos_ok) {
    const float n = qnan();
    x1 = make_float4(n, n, n, n);
    x2 = x1;
  }
  if (KV && !pos_ok && base != src) return;  // k head outside the cache: nothing written
  st4_nt(base, sub, x1);
  st4_nt(base + HALF, sub, x2);
}

// Any head_dim (even when ROPE), any alignment: one wave per head.
template <bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void head_scalar_kernel(HeadArgs a, int hd) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long gh = (long long)blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
  if (gh >= a.total_heads) return;
  float* base;
  const float* w;
  long long row;
  head_of(a, gh, hd, &base, &w, &row);
  float rinv = 1.0f;
  if constexpr (NORM) {
    float ss = 0.0f;
    for (int d = lane; d < hd; d += kWave) ss += base[d] * base[d];
    ss = wave_sum(ss);
    rinv = 1.0f / sqrtf(ss / (float)hd + a.eps);
  }
  if constexpr (ROPE) {
    const int half = hd / 2;
    const long long pos = a.positions ? (long long)a.positions[row] : row;
    const bool bad = pos < 0 || pos >= a.table_rows;
    const float* cr = a.cos_tab + (bad ? 0 : pos) * hd;
    const float* sr = a.sin_tab + (bad ? 0 : pos) * hd;
    for (int d = lane; d < half; d += kWave) {
      float v1 = base[d], v2 = base[d + half];
      if constexpr (NORM) {
        v1 = (v1 * rinv) * w[d];
        v2 = (v2 * rinv) * w[d + half];
      }
      if (bad) {
        base[d] = qnan();
        base[d + half] = qnan();
      } else {
        base[d] = v1 * cr[d] + (-v2) * sr[d];
        base[d + half] = v2 * cr[d + half] + v1 * sr[d + half];
      }
    }
  } else {
    for (int d = lane; d < hd; d += kWave) base[d] = (base[d] * rinv) * w[d];
  }
}

template <bool NORM, bool ROPE>
int launch_heads(const HeadArgs& a, int hd, hipStream_t st) {
  const bool vec = (hd == 64 || hd == 128 || hd == 256 || hd == 512) && aligned16(a.q) &&
                   (a.total_heads == a.q_heads || aligned16(a.k)) &&
                   (!NORM || (aligned16(a.qw) && (a.total_heads == a.q_heads || aligned16(a.kw)))) &&
                   (!ROPE || (aligned16(a.cos_tab) && aligned16(a.sin_tab)));
  if (vec) {
    const long long hpw = kWave / (hd / 8);
    const long long heads_per_block = hpw * (kHeadBlock / kWave);
    const unsigned grid = (unsigned)((a.total_heads + heads_per_block - 1) / heads_per_block);
    switch (hd) {
      case 64: head_vec_kernel<64, NORM, ROPE><<<grid, kHeadBlock, 0, st>>>(a); break;
      case 128: head_vec_kernel<128, NORM, ROPE><<<grid, kHeadBlock, 0, st>>>(a); break;
      case 256: head_vec_kernel<256, NORM, ROPE><<<grid, kHeadBlock, 0, st>>>(a); break;
      default: head_vec_kernel<512, NORM, ROPE><<<grid, kHeadBlock, 0, st>>>(a); break;
    }
  } else {
    const unsigned grid = (unsigned)((a.total_heads + 3) / 4);
    head_scalar_kernel<NORM, ROPE><<<grid, 256, 0, st>>>(a, hd);
  }
  return launch_status(NORM ? (ROPE ? "head_rms_norm_rope" : "rms_norm_per_head")
                            : "apply_rope_neox");
}

int check_heads(size_t seq, size_t nh, size_t nk, size_t hd, bool rope) {
  QASR_REQUIRE(hd > 0 && hd <= 65536, "head_dim must be in [1, 65536]");
  QASR_REQUIRE(!rope || hd % 2 == 0, "RoPE needs an even head_dim");
  QASR_REQUIRE(nh <= 65536 && nk <= 65536, "head count too large");
  size_t heads, n;
  QASR_REQUIRE(mul_ok(seq, nh + nk, &heads), "seq * heads overflows");
  QASR_REQUIRE(mul_ok(heads, hd, &n), "seq * heads * head_dim overflows");
  QASR_REQUIRE(heads / 4 < 0x7fffffffu, "too many heads for one launch");
  return QASR_OK;
}

// RoPE table rows [pos_begin, pos_end). inv_freq comes from the host by value.
struct InvFreq {
  float v[256];
};

__global__ __launch_bounds__(256) void rope_table_kernel(float* cos_tab, float* sin_tab,
                                                         long long pos_begin, long long n_items,
                                                         int hd, InvFreq inv) {
  const int half = hd / 2;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n_items;
       i += (long long)gridDim.x * 256) {
    const long long p = pos_begin + i / half;
    const int d = (int)(i % half);
    // decoder.rs:279-285: angle = (pos as f32) * inv_freq[d] in f32; cos/sin of
    // that f32 angle, here evaluated in double and rounded once.
    const float angle = (float)p * inv.v[d];
    const float c = (float)cos((double)angle);
    const float s = (float)sin((double)angle);
    cos_tab[p * hd + d] = c;
    cos_tab[p * hd + half + d] = c;
    sin_tab[p * hd + d] = s;
    sin_tab[p * hd + half + d] = s;
  }
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_rms_norm_per_head_f32(float* x, const float* weight, size_t seq_len,
                                          size_t n_heads, size_t head_dim, float eps,
                                          void* stream) {
  if (seq_len == 0 || n_heads == 0 || head_dim == 0) return QASR_OK;
  QASR_REQUIRE(x && weight, "rms_norm_per_head: null pointer");
  int rc = check_heads(seq_len, n_heads, 0, head_dim, false);
  if (rc) return rc;
  HeadArgs a{};
  a.q = x;
  a.qw = weight;
  a.q_heads = (long long)(seq_len * n_heads);
  a.total_heads = a.q_heads;
  a.nq = (int)n_heads;
  a.nk = 1;
  a.eps = eps;
  return launch_heads<true, false>(a, (int)head_dim, as_stream(stream));
}

extern "C" int qasr_apply_rope_neox_f32(float* x, const float* cos_vals, const float* sin_vals,
                                        size_t seq, size_t n_heads, size_t head_dim,
                                        void* stream) {
  if (seq == 0 || n_heads == 0 || head_dim == 0) return QASR_OK;
  QASR_REQUIRE(x && cos_vals && sin_vals, "apply_rope_neox: null pointer");
  int rc = check_heads(seq, n_heads, 0, head_dim, true);
  if (rc) return rc;
  HeadArgs a{};
  a.q = x;
  a.cos_tab = cos_vals;
  a.sin_tab = sin_vals;
  a.positions = nullptr;
  a.q_heads = (long long)(seq * n_heads);
  a.total_heads = a.q_heads;
  a.nq = (int)n_heads;
  a.nk = 1;
  a.table_rows = (long long)seq;
  return launch_heads<false, true>(a, (int)head_dim, as_stream(stream));
}

extern "C" int qasr_head_rms_norm_rope_f32(float* q, float* k, const float* q_norm_w,
                                           const float* k_norm_w, const float* cos_tab,
                                           const float* sin_tab, const int32_t* positions,
                                           size_t seq, size_t n_heads, size_t n_kv_heads,
                                           size_t head_dim, size_t table_rows, float eps,
                                           void* stream) {
  if (seq == 0 || head_dim == 0 || n_heads + n_kv_heads == 0) return QASR_OK;
  QASR_REQUIRE(cos_tab && sin_tab, "head_rms_norm_rope: null table");
  QASR_REQUIRE(table_rows > 0, "head_rms_norm_rope: the RoPE table has no rows");
  QASR_REQUIRE(n_heads == 0 || (q && q_norm_w), "head_rms_norm_rope: null q");
  QASR_REQUIRE(n_kv_heads == 0 || (k && k_norm_w), "head_rms_norm_rope: null k");
  int rc = check_heads(seq, n_heads, n_kv_heads, head_dim, true);
  if (rc) return rc;
  HeadArgs a{};
  a.q = q;
  a.k = k;
  a.qw = q_norm_w;
  a.kw = k_norm_w;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.positions = positions;
  a.q_heads = (long long)(seq * n_heads);
  a.total_heads = (long long)(seq * (n_heads + n_kv_heads));
  a.nq = n_heads ? (int)n_heads : 1;
  a.nk = n_kv_heads ? (int)n_kv_heads : 1;
  a.table_rows = (long long)table_rows;
  a.eps = eps;
  return launch_heads<true, true>(a, (int)head_dim, as_stream(stream));
}

extern "C" int qasr_head_rms_norm_rope_kv_f32(float* q, const float* k, const float* v,
                                              const float* q_norm_w, const float* k_norm_w,
                                              const float* cos_tab, const float* sin_tab,
                                              const int32_t* positions, size_t start_pos,
                                              size_t seq, size_t n_heads, size_t n_kv_heads,
                                              size_t head_dim, size_t table_rows, float eps,
                                              float* k_cache, float* v_cache, size_t cache_rows,
                                              void* stream) {
  if (seq == 0 || n_heads + n_kv_heads == 0) return QASR_OK;
  QASR_REQUIRE(cos_tab && sin_tab, "head_rms_norm_rope_kv: null table");
  QASR_REQUIRE(n_heads == 0 || (q && q_norm_w), "head_rms_norm_rope_kv: null q");
  QASR_REQUIRE(n_kv_heads == 0 || (k && v && k_norm_w && k_cache && v_cache),
               "head_rms_norm_rope_kv: null k, v or cache");
  QASR_REQUIRE(table_rows > 0 && cache_rows > 0, "head_rms_norm_rope_kv: empty table or cache");
  QASR_REQUIRE(positions || (start_pos <= cache_rows && seq <= cache_rows - start_pos &&
                             start_pos + seq <= table_rows),
               "head_rms_norm_rope_kv: rows start_pos..start_pos+seq exceed the cache or the RoPE table");
  int rc = check_heads(seq, n_heads, 2 * n_kv_heads, head_dim, true);
  if (rc) return rc;
  size_t cache_elems;
  QASR_REQUIRE(mul_ok(cache_rows, n_kv_heads * head_dim, &cache_elems) &&
                   (!positions || mul_ok(cache_elems, seq, &cache_elems)),
               "head_rms_norm_rope_kv: cache size overflows");
  const bool vec = (head_dim == 64 || head_dim == 128 || head_dim == 256 || head_dim == 512) &&
                   aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_norm_w) &&
                   aligned16(k_norm_w) && aligned16(cos_tab) && aligned16(sin_tab) &&
                   aligned16(k_cache) && aligned16(v_cache);
  if (!vec) {
    return fail(QASR_ERR_UNSUPPORTED,
                "head_rms_norm_rope_kv: needs head_dim 64/128/256/512 and 16-byte aligned buffers");
  }
  HeadArgs a{};
  a.q = q;
  a.qw = q_norm_w;
  a.kw = k_norm_w;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.positions = positions;
  a.q_heads = (long long)(seq * n_heads);
  a.kv_heads_end = a.q_heads + (long long)(seq * n_kv_heads);
  a.total_heads = a.kv_heads_end + (long long)(seq * n_kv_heads);
  a.nq = n_heads ? (int)n_heads : 1;
  a.nk = n_kv_heads ? (int)n_kv_heads : 1;
  a.table_rows = (long long)table_rows;
  a.eps = eps;
  a.k_src = k;
  a.v = v;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.start_pos = (long long)start_pos;
  a.cache_rows = (long long)cache_rows;
  const int hd = (int)head_dim;
  const long long heads_per_block = (kWave / (hd / 8)) * (kHeadBlock / kWave);
  const unsigned grid = (unsigned)((a.total_heads + heads_per_block - 1) / heads_per_block);
  hipStream_t st = as_stream(stream);
  switch (hd) {
    case 64: head_vec_kernel<64, true, true, true><<<grid, kHeadBlock, 0, st>>>(a); break;
    case 128: head_vec_kernel<128, true, true, true><<<grid, kHeadBlock, 0, st>>>(a); break;
    case 256: head_vec_kernel<256, true, true, true><<<grid, kHeadBlock, 0, st>>>(a); break;
    default: head_vec_kernel<512, true, true, true><<<grid, kHeadBlock, 0, st>>>(a); break;
  }
  return launch_status("head_rms_norm_rope_kv");
}

extern "C" int qasr_rope_table_fill_f32(float* cos_tab, float* sin_tab, size_t pos_begin,
                                        size_t pos_end, size_t head_dim, float theta,
                                        void* stream) {
  if (pos_end <= pos_begin) return QASR_OK;
  QASR_REQUIRE(cos_tab && sin_tab, "rope_table_fill: null pointer");
  QASR_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 512,
               "rope_table_fill: head_dim must be even and <= 512");
  QASR_REQUIRE(pos_end <= ((size_t)1 << 24), "rope_table_fill: positions must be < 2^24");
  // RopeCache::ensure (decoder.rs:262-266): inv_freq[d] = 1 / theta.powf((2d) as f32 / hd as f32)
  InvFreq inv{};
  const int half = (int)head_dim / 2;
  for (int d = 0; d < half; ++d) {
    inv.v[d] = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
  }
  const long long items = (long long)(pos_end - pos_begin) * half;
  rope_table_kernel<<<grid_for((size_t)items, 256), 256, 0, as_stream(stream)>>>(
      cos_tab, sin_tab, (long long)pos_begin, items, (int)head_dim, inv);
  return launch_status("rope_table_fill");
}
