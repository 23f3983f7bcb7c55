/*
 * qasr_oracle.c -- CPU restatement of the QwenASR (ZhaoChaoqun/QwenASR, Rust)
 * x86_64 kernels on the fused-layer path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity oracle: only tests/, the
 * smoke check and bench.py's cpu_baseline leg load it. The product library
 * (qwenasr_amd/libqasr_hip.so) never links or calls it.
 *
 * Each function restates the arithmetic of the reference function it cites
 * (paths relative to crates/qwen-asr/src/), in the same order of operations:
 *   - the AVX2 paths (kernels/avx.rs) are restated lane by lane: an 8-wide
 *     register becomes a float[8], _mm256_fmadd_ps becomes fmaf per lane,
 *     hsum_ps becomes hsum8() with the same pairing;
 *   - Rust scalar loops never contract a*b+c, so this file is compiled with
 *     -ffp-contract=off and uses fmaf only where the reference uses an FMA;
 *   - Rust f32::{exp,sin,cos,powf,ln,sqrt,round} lower to glibc
 *     expf/sinf/cosf/powf/logf, IEEE sqrtf and roundf on x86_64 Linux, which
 *     this file calls directly.
 *
 * Functions with no reference counterpart (erf-GELU, W8A8) are marked NEW and
 * state the definition they implement.
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* hsum_ps (kernels/avx.rs:36-51): (lo+hi) then movehdup/movehl pairing:
 * ((s0+s1) + (s2+s3)) with s_i = v[i] + v[i+4]. */
static float hsum8(const float v[8]) {
  float s[4];
  for (int i = 0; i < 4; ++i) s[i] = v[i] + v[i + 4];
  const float a = s[0] + s[1];
  const float b = s[2] + s[3];
  return a + b;
}

/* ------------------------------------------------------------------------ */
/* add_inplace, kernels/mod.rs:486-488                                       */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_add_inplace(float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; ++i) a[i] += b[i];
}

/* ------------------------------------------------------------------------ */
/* rms_norm, kernels/mod.rs:897-918 -> avx::rms_norm_row, avx.rs:374-415     */
/* ------------------------------------------------------------------------ */
static void rms_norm_row(float* out, const float* x, const float* w, size_t hidden, float eps) {
  float acc0[8] = {0}, acc1[8] = {0};
  size_t i = 0;
  while (i + 16 <= hidden) {
    for (int l = 0; l < 8; ++l) {
      acc0[l] = fmaf(x[i + l], x[i + l], acc0[l]);
      acc1[l] = fmaf(x[i + 8 + l], x[i + 8 + l], acc1[l]);
    }
    i += 16;
  }
  while (i + 8 <= hidden) {
    for (int l = 0; l < 8; ++l) acc0[l] = fmaf(x[i + l], x[i + l], acc0[l]);
    i += 8;
  }
  float sum[8];
  for (int l = 0; l < 8; ++l) sum[l] = acc0[l] + acc1[l];
  float ss = hsum8(sum);
  while (i < hidden) {
    ss += x[i] * x[i];
    ++i;
  }
  const float rinv = 1.0f / sqrtf(ss / (float)hidden + eps);
  for (i = 0; i < hidden; ++i) out[i] = (x[i] * rinv) * w[i];
}

ORACLE_API void ref_rms_norm(float* out, const float* x, const float* w, size_t seq_len,
                             size_t hidden, float eps) {
  for (size_t s = 0; s < seq_len; ++s) rms_norm_row(out + s * hidden, x + s * hidden, w, hidden, eps);
}

/* The pair add_inplace + rms_norm the fused GPU kernel replaces
 * (decoder.rs:908+910, 924->878). */
ORACLE_API void ref_add_rms_norm(float* x, const float* delta, const float* w, float* out,
                                 size_t seq_len, size_t hidden, float eps) {
  ref_add_inplace(x, delta, seq_len * hidden);
  ref_rms_norm(out, x, w, seq_len, hidden, eps);
}

/* ------------------------------------------------------------------------ */
/* layer_norm, kernels/mod.rs:866-895 -> avx::layer_norm_row, avx.rs:417-481 */
/* ------------------------------------------------------------------------ */
static void layer_norm_row(float* out, const float* x, const float* w, const float* b,
                           size_t hidden, float eps) {
  float s0[8] = {0}, s1[8] = {0};
  size_t i = 0;
  while (i + 16 <= hidden) {
    for (int l = 0; l < 8; ++l) {
      s0[l] = s0[l] + x[i + l];
      s1[l] = s1[l] + x[i + 8 + l];
    }
    i += 16;
  }
  while (i + 8 <= hidden) {
    for (int l = 0; l < 8; ++l) s0[l] = s0[l] + x[i + l];
    i += 8;
  }
  float t[8];
  for (int l = 0; l < 8; ++l) t[l] = s0[l] + s1[l];
  float mean = hsum8(t);
  while (i < hidden) {
    mean += x[i];
    ++i;
  }
  mean /= (float)hidden;

  float v0[8] = {0}, v1[8] = {0};
  i = 0;
  while (i + 16 <= hidden) {
    for (int l = 0; l < 8; ++l) {
      const float d0 = x[i + l] - mean;
      const float d1 = x[i + 8 + l] - mean;
      v0[l] = fmaf(d0, d0, v0[l]);
      v1[l] = fmaf(d1, d1, v1[l]);
    }
    i += 16;
  }
  while (i + 8 <= hidden) {
    for (int l = 0; l < 8; ++l) {
      const float d = x[i + l] - mean;
      v0[l] = fmaf(d, d, v0[l]);
    }
    i += 8;
  }
  for (int l = 0; l < 8; ++l) t[l] = v0[l] + v1[l];
  float var = hsum8(t);
  while (i < hidden) {
    const float d = x[i] - mean;
    var += d * d;
    ++i;
  }
  const float inv_std = 1.0f / sqrtf(var / (float)hidden + eps);

  i = 0;
  while (i + 8 <= hidden) {
    for (int l = 0; l < 8; ++l) out[i + l] = fmaf((x[i + l] - mean) * inv_std, w[i + l], b[i + l]);
    i += 8;
  }
  while (i < hidden) {
    out[i] = (x[i] - mean) * inv_std * w[i] + b[i];
    ++i;
  }
}

ORACLE_API void ref_layer_norm(float* out, const float* x, const float* w, const float* b,
                               size_t seq_len, size_t hidden, float eps) {
  for (size_t s = 0; s < seq_len; ++s)
    layer_norm_row(out + s * hidden, x + s * hidden, w, b, hidden, eps);
}

/* ------------------------------------------------------------------------ */
/* rms_norm_per_head, kernels/mod.rs:920-935 (scalar; `iter().sum()` folds   */
/* left to right)                                                            */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_rms_norm_per_head(float* x, const float* w, size_t seq_len, size_t n_heads,
                                      size_t head_dim, float eps) {
  for (size_t s = 0; s < seq_len; ++s) {
    for (size_t h = 0; h < n_heads; ++h) {
      float* v = x + (s * n_heads + h) * head_dim;
      float ss = -0.0f;
      for (size_t d = 0; d < head_dim; ++d) ss = ss + v[d] * v[d];
      const float rinv = 1.0f / sqrtf(ss / (float)head_dim + eps);
      for (size_t d = 0; d < head_dim; ++d) v[d] = v[d] * rinv * w[d];
    }
  }
}

/* ------------------------------------------------------------------------ */
/* RopeCache::ensure table rows, decoder.rs:253-289. Rows do not depend on   */
/* the capacity-doubling history, so rows [0, n_pos) are filled directly.    */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_rope_inv_freq(float* inv_freq, size_t head_dim, float theta) {
  const size_t half = head_dim / 2;
  for (size_t d = 0; d < half; ++d)
    inv_freq[d] = 1.0f / powf(theta, (float)(2 * d) / (float)head_dim);
}

ORACLE_API void ref_rope_table(float* cos_tab, float* sin_tab, size_t n_pos, size_t head_dim,
                               float theta) {
  float inv[512];
  const size_t half = head_dim / 2;
  ref_rope_inv_freq(inv, head_dim, theta);
  for (size_t p = 0; p < n_pos; ++p) {
    const float pf = (float)p;
    for (size_t d = 0; d < half; ++d) {
      const float angle = pf * inv[d];
      const float c = cosf(angle);
      const float s = sinf(angle);
      cos_tab[p * head_dim + d] = c;
      cos_tab[p * head_dim + half + d] = c;
      sin_tab[p * head_dim + d] = s;
      sin_tab[p * head_dim + half + d] = s;
    }
  }
}

/* apply_rope_neox, kernels/mod.rs:1247-1267: row s uses cos/sin row s. */
ORACLE_API void ref_apply_rope_neox(float* x, const float* cos_vals, const float* sin_vals,
                                    size_t seq, size_t n_heads, size_t head_dim) {
  const size_t half = head_dim / 2;
  const size_t hidden = n_heads * head_dim;
  for (size_t s = 0; s < seq; ++s) {
    const float* c = cos_vals + s * head_dim;
    const float* sn = sin_vals + s * head_dim;
    for (size_t h = 0; h < n_heads; ++h) {
      float* v = x + s * hidden + h * head_dim;
      for (size_t d = 0; d < half; ++d) {
        const float x1 = v[d];
        const float x2 = v[half + d];
        v[d] = x1 * c[d] + (-x2) * sn[d];
        v[half + d] = x2 * c[half + d] + x1 * sn[half + d];
      }
    }
  }
}

/* The decoder's q/k sequence (decoder.rs:888-892 per token; 799-803 per
 * prefill) with a per-row position: head norm, then RoPE with table row
 * positions[s]. Batched multi-stream decode is this, looped over streams. */
ORACLE_API void ref_head_rms_norm_rope(float* q, float* k, const float* qw, const float* kw,
                                       const float* cos_tab, const float* sin_tab,
                                       const int32_t* positions, size_t seq, size_t n_heads,
                                       size_t n_kv_heads, size_t head_dim, float eps) {
  for (size_t s = 0; s < seq; ++s) {
    const size_t pos = positions ? (size_t)positions[s] : s;
    if (n_heads) {
      float* qs = q + s * n_heads * head_dim;
      ref_rms_norm_per_head(qs, qw, 1, n_heads, head_dim, eps);
      ref_apply_rope_neox(qs, cos_tab + pos * head_dim, sin_tab + pos * head_dim, 1, n_heads,
                          head_dim);
    }
    if (n_kv_heads) {
      float* ks = k + s * n_kv_heads * head_dim;
      ref_rms_norm_per_head(ks, kw, 1, n_kv_heads, head_dim, eps);
      ref_apply_rope_neox(ks, cos_tab + pos * head_dim, sin_tab + pos * head_dim, 1, n_kv_heads,
                          head_dim);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* fast_exp_avx, kernels/avx.rs:483-514, one lane                            */
/* ------------------------------------------------------------------------ */
ORACLE_API float ref_fast_exp(float x) {
  float val = x * 1.442695041f;
  val = (val < 126.0f) ? val : 126.0f;   /* _mm256_min_ps(val, 126) */
  val = (val > -126.0f) ? val : -126.0f; /* _mm256_max_ps(val, -126) */
  const int ip = (int)rintf(val);        /* _mm256_cvtps_epi32: nearest-even */
  const float fp = val - (float)ip;
  uint32_t bits = (uint32_t)(ip + 127) << 23;
  float e;
  memcpy(&e, &bits, sizeof e);
  const float f = fp * 0.6931471806f;
  float p = fmaf(1.0f / 120.0f, f, 1.0f / 24.0f);
  p = fmaf(p, f, 1.0f / 6.0f);
  p = fmaf(p, f, 0.5f);
  p = fmaf(p, f, 1.0f);
  p = fmaf(p, f, 1.0f);
  return e * p;
}

/* ------------------------------------------------------------------------ */
/* swiglu_multiply, kernels/mod.rs:965-985 -> avx::swiglu_interleaved,       */
/* avx.rs:565-599. Lanes of an 8-block are columns j..j+7 after the          */
/* deinterleave; the row tail uses libm expf.                                */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_swiglu_multiply(float* out, const float* gate_up, size_t seq_len,
                                    size_t inter) {
  for (size_t s = 0; s < seq_len; ++s) {
    const float* gu = gate_up + s * 2 * inter;
    float* o = out + s * inter;
    size_t j = 0;
    while (j + 8 <= inter) {
      for (int l = 0; l < 8; ++l) {
        const float g = gu[2 * (j + l)];
        const float u = gu[2 * (j + l) + 1];
        const float e = ref_fast_exp(0.0f - g);
        const float silu = g / (1.0f + e);
        o[j + l] = silu * u;
      }
      j += 8;
    }
    while (j < inter) {
      const float g = gu[2 * j];
      const float u = gu[2 * j + 1];
      o[j] = (g / (1.0f + expf(-g))) * u;
      ++j;
    }
  }
}

/* Decode-loop SwiGLU on split buffers with libm expf: decoder.rs:916-921
 * (there on the interleaved buffer), kernels/mod.rs:988-994. */
ORACLE_API void ref_swiglu_split(float* out, const float* gate, const float* up, size_t n) {
  for (size_t j = 0; j < n; ++j) {
    const float g = gate[j];
    out[j] = (g / (1.0f + expf(-g))) * up[j];
  }
}

/* silu, kernels/mod.rs:941-946 */
ORACLE_API void ref_silu(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* ------------------------------------------------------------------------ */
/* gelu (tanh form), kernels/mod.rs:948-963 -> avx::gelu_inplace,            */
/* avx.rs:533-563                                                            */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_gelu_tanh(float* x, size_t n) {
  size_t i = 0;
  while (i + 8 <= n) {
    for (int l = 0; l < 8; ++l) {
      const float v = x[i + l];
      const float v2 = v * v;
      const float v3 = v2 * v;
      const float inner = 0.7978845608028654f * fmaf(0.044715f, v3, v);
      const float e = ref_fast_exp(2.0f * inner);
      const float th = 1.0f - 2.0f / (e + 1.0f);
      x[i + l] = 0.5f * (v * (1.0f + th));
    }
    i += 8;
  }
  while (i < n) {
    const float v = x[i];
    const float x3 = v * v * v;
    const float inner = 0.7978845608028654f * (v + 0.044715f * x3);
    x[i] = 0.5f * v * (1.0f + tanhf(inner));
    ++i;
  }
}

/* NEW: exact GELU, 0.5*x*(1 + erf(x/sqrt(2))) evaluated in double as
 * 0.5*x*erfc(-x/sqrt(2)) and rounded once to f32. The reference's only erf
 * GELU is candle's Metal gelu_erf (encoder_gpu.rs:470,480). */
ORACLE_API void ref_gelu_erf(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const double v = (double)x[i];
    x[i] = (float)(0.5 * v * erfc(-v / sqrt(2.0)));
  }
}

/* ------------------------------------------------------------------------ */
/* sinusoidal_pe, kernels/mod.rs:1213-1226                                   */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_sinusoidal_pe(float* pe, size_t n_pos, size_t d_model) {
  const size_t half = d_model / 2;
  const float log_ts = logf(10000.0f) / (float)(half - 1);
  for (size_t p = 0; p < n_pos; ++p) {
    float* row = pe + p * d_model;
    for (size_t d = 0; d < half; ++d) {
      const float inv = expf(-(float)d * log_ts);
      const float angle = (float)p * inv;
      row[d] = sinf(angle);
      row[half + d] = cosf(angle);
    }
  }
}

/* Per-chunk PE add of encoder.rs:340-343: x[r] += pe[r mod n_pos]. */
ORACLE_API void ref_pe_add(float* x, const float* pe, size_t rows, size_t d_model, size_t n_pos) {
  for (size_t r = 0; r < rows; ++r)
    for (size_t c = 0; c < d_model; ++c) x[r * d_model + c] += pe[(r % n_pos) * d_model + c];
}

/* ------------------------------------------------------------------------ */
/* Token-embedding gather, decoder.rs:631-646                                */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_embed_gather_f32(float* out, const float* table, const int32_t* ids, size_t n,
                                     size_t dim) {
  for (size_t i = 0; i < n; ++i) memcpy(out + i * dim, table + (size_t)ids[i] * dim, dim * 4);
}

ORACLE_API void ref_embed_gather_bf16(float* out, const uint16_t* table, const int32_t* ids,
                                      size_t n, size_t dim) {
  for (size_t i = 0; i < n; ++i) {
    const uint16_t* src = table + (size_t)ids[i] * dim;
    for (size_t c = 0; c < dim; ++c) {
      const uint32_t bits = (uint32_t)src[c] << 16;
      memcpy(out + i * dim + c, &bits, 4);
    }
  }
}

ORACLE_API void ref_embed_gather_i8(float* out, const int8_t* table, const float* scales,
                                    const int32_t* ids, size_t n, size_t dim) {
  for (size_t i = 0; i < n; ++i) {
    const size_t row = (size_t)ids[i];
    const float s = scales[row];
    for (size_t c = 0; c < dim; ++c) out[i * dim + c] = (float)table[row * dim + c] * s;
  }
}

/* ------------------------------------------------------------------------ */
/* quantize_f32_to_int8, quantize.rs:633-662 (quantize_bf16_to_int8,         */
/* :599-630, is the same after the exact bf16 -> f32 shift)                  */
/* ------------------------------------------------------------------------ */
static int8_t q_i8(float v, float inv) {
  float r = roundf(v * inv);
  if (r < -128.0f) r = -128.0f; /* f32::clamp */
  if (r > 127.0f) r = 127.0f;
  if (r != r) return 0; /* `as i8` of NaN */
  return (int8_t)r;
}

ORACLE_API void ref_quantize_f32_to_int8(int8_t* q, float* scales, const float* x, size_t out_dim,
                                         size_t in_dim) {
  for (size_t o = 0; o < out_dim; ++o) {
    const float* row = x + o * in_dim;
    float absmax = 0.0f;
    for (size_t k = 0; k < in_dim; ++k) {
      const float a = fabsf(row[k]);
      if (a > absmax) absmax = a;
    }
    scales[o] = absmax / 127.0f;
    const float inv = absmax > 0.0f ? 127.0f / absmax : 0.0f;
    for (size_t k = 0; k < in_dim; ++k) q[o * in_dim + k] = q_i8(row[k], inv);
  }
}

ORACLE_API void ref_quantize_bf16_to_int8(int8_t* q, float* scales, const uint16_t* x,
                                          size_t out_dim, size_t in_dim) {
  for (size_t o = 0; o < out_dim; ++o) {
    float absmax = 0.0f;
    for (size_t k = 0; k < in_dim; ++k) {
      const uint32_t bits = (uint32_t)x[o * in_dim + k] << 16;
      float v;
      memcpy(&v, &bits, 4);
      const float a = fabsf(v);
      if (a > absmax) absmax = a;
    }
    scales[o] = absmax / 127.0f;
    const float inv = absmax > 0.0f ? 127.0f / absmax : 0.0f;
    for (size_t k = 0; k < in_dim; ++k) {
      const uint32_t bits = (uint32_t)x[o * in_dim + k] << 16;
      float v;
      memcpy(&v, &bits, 4);
      q[o * in_dim + k] = q_i8(v, inv);
    }
  }
}

/* ------------------------------------------------------------------------ */
/* W8A32 matvec: generic::int8_matvec_fused, kernels/generic.rs:37-49,       */
/* threaded as int8_matvec_threaded (kernels/mod.rs:622-647): nt contiguous  */
/* row chunks of ceil(out/nt); T > 1 runs T matvecs (mod.rs:655-660).        */
/* ------------------------------------------------------------------------ */
static void int8_matvec_rows(float* y, const float* x, const int8_t* w, const float* scales,
                             size_t in_dim, size_t begin, size_t end) {
  for (size_t o = begin; o < end; ++o) {
    const int8_t* wr = w + o * in_dim;
    float sum = 0.0f;
    for (size_t k = 0; k < in_dim; ++k) sum += (float)wr[k] * x[k];
    y[o] = sum * scales[o];
  }
}

typedef struct {
  float* y;
  const float* x;
  const int8_t* w;
  const float* scales;
  size_t in_dim, begin, end;
} mv_job;

static void* mv_worker(void* p) {
  const mv_job* j = (const mv_job*)p;
  int8_matvec_rows(j->y, j->x, j->w, j->scales, j->in_dim, j->begin, j->end);
  return NULL;
}

ORACLE_API void ref_linear_nobias_int8(float* y, const float* x, const int8_t* w,
                                       const float* scales, size_t seq_len, size_t in_dim,
                                       size_t out_dim, int n_threads) {
  if (n_threads < 1) n_threads = 1;
  if (n_threads > 16) n_threads = 16; /* MAX_THREADS, kernels/mod.rs:177 */
  for (size_t s = 0; s < seq_len; ++s) {
    float* ys = y + s * out_dim;
    const float* xs = x + s * in_dim;
    if (n_threads == 1) {
      int8_matvec_rows(ys, xs, w, scales, in_dim, 0, out_dim);
      continue;
    }
    pthread_t th[16];
    mv_job jobs[16];
    const size_t chunk = (out_dim + (size_t)n_threads - 1) / (size_t)n_threads;
    int started = 0;
    for (int t = 0; t < n_threads; ++t) {
      const size_t b = (size_t)t * chunk;
      size_t e = b + chunk;
      if (e > out_dim) e = out_dim;
      if (b >= e) continue;
      jobs[started] = (mv_job){ys, xs, w, scales, in_dim, b, e};
      if (pthread_create(&th[started], NULL, mv_worker, &jobs[started]) != 0) {
        mv_worker(&jobs[started]);
        continue;
      }
      ++started;
    }
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
  }
}

/* linear_int8, kernels/mod.rs:664-673: linear_nobias_int8, then += bias. */
ORACLE_API void ref_linear_int8(float* y, const float* x, const int8_t* w, const float* scales,
                                const float* bias, size_t seq_len, size_t in_dim, size_t out_dim,
                                int n_threads) {
  ref_linear_nobias_int8(y, x, w, scales, seq_len, in_dim, out_dim, n_threads);
  if (bias)
    for (size_t s = 0; s < seq_len; ++s)
      for (size_t o = 0; o < out_dim; ++o) y[s * out_dim + o] += bias[o];
}

/* Gate/up row interleave, decoder.rs:701-719. */
ORACLE_API void ref_interleave_gate_up(int8_t* wgu, float* sgu, const int8_t* wg, const float* sg,
                                       const int8_t* wu, const float* su, size_t inter,
                                       size_t hidden) {
  for (size_t r = 0; r < inter; ++r) {
    memcpy(wgu + (2 * r) * hidden, wg + r * hidden, hidden);
    memcpy(wgu + (2 * r + 1) * hidden, wu + r * hidden, hidden);
    sgu[2 * r] = sg[r];
    sgu[2 * r + 1] = su[r];
  }
}

/* ------------------------------------------------------------------------ */
/* NEW: W8A8 gate/up + SwiGLU.                                               */
/*   dg = sum_k w[2j,k]*xq[b,k], du = sum_k w[2j+1,k]*xq[b,k] (exact, int64) */
/*   g = ((f32)dg * xs[b]) * s[2j]; u = ((f32)du * xs[b]) * s[2j+1]          */
/*   out[b,j] = (g / (1 + expf(-g))) * u   (decode SwiGLU, decoder.rs:916-921)*/
/* dots (optional) receives the int32 sums [batch, 2*inter] for bit-exact    */
/* comparison.                                                               */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_gate_up_swiglu_w8a8(float* out, int32_t* dots, const int8_t* w,
                                        const float* scales, const int8_t* xq,
                                        const float* x_scales, size_t batch, size_t in_dim,
                                        size_t inter) {
  for (size_t b = 0; b < batch; ++b) {
    const int8_t* xb = xq + b * in_dim;
    for (size_t j = 0; j < inter; ++j) {
      const int8_t* g = w + (2 * j) * in_dim;
      const int8_t* u = w + (2 * j + 1) * in_dim;
      int64_t dg = 0, du = 0;
      for (size_t k = 0; k < in_dim; ++k) {
        dg += (int64_t)g[k] * (int64_t)xb[k];
        du += (int64_t)u[k] * (int64_t)xb[k];
      }
      if (dots) {
        dots[b * 2 * inter + 2 * j] = (int32_t)dg;
        dots[b * 2 * inter + 2 * j + 1] = (int32_t)du;
      }
      const float gg = ((float)(int32_t)dg * x_scales[b]) * scales[2 * j];
      const float uu = ((float)(int32_t)du * x_scales[b]) * scales[2 * j + 1];
      out[b * inter + j] = (gg / (1.0f + expf(-gg))) * uu;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Batched W8A8 projection (new; the reference's linear_nobias_int8,          */
/* kernels/mod.rs:650-661, with each stream's activation row quantized per    */
/* row by quantize_f32_to_int8, quantize.rs:633-662):                         */
/*   dot[m,n] = sum_k w[n,k] * xq[m,k] (exact), y = ((f32)dot * xs[m]) * s[n] */
/* -- the same dequantization as the gate/up epilogue above. dots optional.   */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_linear_w8a8(float* y, int32_t* dots, const int8_t* w, const float* scales,
                                const int8_t* xq, const float* x_scales, size_t batch,
                                size_t in_dim, size_t out_dim) {
  for (size_t m = 0; m < batch; ++m) {
    const int8_t* xm = xq + m * in_dim;
    for (size_t n = 0; n < out_dim; ++n) {
      const int8_t* wn = w + n * in_dim;
      int64_t d = 0;
      for (size_t k = 0; k < in_dim; ++k) d += (int64_t)wn[k] * (int64_t)xm[k];
      if (dots) dots[m * out_dim + n] = (int32_t)d;
      y[m * out_dim + n] = ((float)(int32_t)d * x_scales[m]) * scales[n];
    }
  }
}

/* ------------------------------------------------------------------------ */
/* lm_head argmax, decoder.rs:941-949 (and 955-962):                         */
/*   best = 0; best_val = logits[0];                                         */
/*   for i in 1..n { if logits[i] > best_val { best_val = logits[i]; best = i } } */
/* applied to each of `rows` rows.                                           */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_argmax_rows(int32_t* idx, const float* x, size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    size_t best = 0;
    float best_val = row[0];
    for (size_t i = 1; i < cols; ++i) {
      if (row[i] > best_val) {
        best_val = row[i];
        best = i;
      }
    }
    idx[r] = (int32_t)best;
  }
}

/* ------------------------------------------------------------------------ */
/* causal attention, kernels/mod.rs:1124-1168 (causal_attention_heads) with  */
/* the x86_64 helpers: dot_f32 avx.rs:247-295 (four 8-lane FMA accumulators  */
/* over 32-strides, an 8-stride tail into acc0, hsum of (acc0+acc1)+(acc2+acc3),*/
/* scalar tail), vec_scale_add avx.rs:351-372 (dst = fma(dst, c, src)),      */
/* vec_axpy_inplace avx.rs:326-349 (dst = fma(src, a, dst)),                 */
/* vec_scale_inplace avx.rs:301-324 (dst *= s). Scalar tails as written.     */
/* ------------------------------------------------------------------------ */
static float dot_f32_avx(const float* a, const float* b, size_t n) {
  float acc[4][8] = {{0}};
  size_t i = 0;
  while (i + 32 <= n) {
    for (int r = 0; r < 4; ++r)
      for (int l = 0; l < 8; ++l) acc[r][l] = fmaf(a[i + 8 * r + l], b[i + 8 * r + l], acc[r][l]);
    i += 32;
  }
  while (i + 8 <= n) {
    for (int l = 0; l < 8; ++l) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
    i += 8;
  }
  float s01[8], s23[8], t[8];
  for (int l = 0; l < 8; ++l) {
    s01[l] = acc[0][l] + acc[1][l];
    s23[l] = acc[2][l] + acc[3][l];
    t[l] = s01[l] + s23[l];
  }
  float sum = hsum8(t);
  while (i < n) {
    sum += a[i] * b[i];
    ++i;
  }
  return sum;
}

static void vec_scale_add_avx(float* dst, const float* src, float c, size_t n) {
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) dst[i + l] = fmaf(dst[i + l], c, src[i + l]);
  for (; i < n; ++i) dst[i] = dst[i] * c + src[i];
}

static void vec_axpy_avx(float* dst, const float* src, float a, size_t n) {
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) dst[i + l] = fmaf(src[i + l], a, dst[i + l]);
  for (; i < n; ++i) dst[i] += a * src[i];
}

ORACLE_API void ref_causal_attention(float* out, const float* q, const float* k, const float* v,
                                     size_t seq_q, size_t seq_k, size_t n_heads,
                                     size_t n_kv_heads, size_t head_dim, float scale,
                                     size_t q_offset) {
  const size_t heads_per_kv = n_heads / n_kv_heads;
  const size_t q_hidden = n_heads * head_dim, kv_hidden = n_kv_heads * head_dim;
  for (size_t h = 0; h < n_heads; ++h) {
    const size_t kv_h = h / heads_per_kv;
    for (size_t i = 0; i < seq_q; ++i) {
      const float* q_row = q + i * q_hidden + h * head_dim;
      float* o_row = out + i * q_hidden + h * head_dim;
      const size_t global_pos = q_offset + i;
      const size_t k_end = global_pos + 1 < seq_k ? global_pos + 1 : seq_k;
      float max_score = -1e30f, sum_exp = 0.0f;
      for (size_t d = 0; d < head_dim; ++d) o_row[d] = 0.0f;
      for (size_t j = 0; j < k_end; ++j) {
        const float* k_row = k + j * kv_hidden + kv_h * head_dim;
        const float* v_row = v + j * kv_hidden + kv_h * head_dim;
        const float score = dot_f32_avx(q_row, k_row, head_dim) * scale;
        if (score > max_score) {
          const float correction = expf(max_score - score);
          sum_exp = sum_exp * correction + 1.0f;
          vec_scale_add_avx(o_row, v_row, correction, head_dim);
          max_score = score;
        } else {
          const float wt = expf(score - max_score);
          sum_exp += wt;
          vec_axpy_avx(o_row, v_row, wt, head_dim);
        }
      }
      if (sum_exp > 0.0f) {
        const float inv_sum = 1.0f / sum_exp;
        for (size_t d = 0; d < head_dim; ++d) o_row[d] *= inv_sum;
      }
    }
  }
}

/* ------------------------------------------------------------------------ */
/* CPU-baseline driver (timing only): the batch-1 decode chain of one layer   */
/* -- add_inplace + rms_norm (decoder.rs:908+910), the q/k head norms + RoPE   */
/* at one position (decoder.rs:888-892), the decode loop's SwiGLU             */
/* (decoder.rs:916-921) -- repeated `iters` times over `sets` rotating input  */
/* sets, so a microsecond-scale chain is timed without a per-call foreign     */
/* function overhead. Set s uses x + s*hidden, q + s*nq*hd, etc.              */
/* ------------------------------------------------------------------------ */
ORACLE_API void ref_decode_chain_repeat(size_t iters, size_t sets, float* x, const float* delta,
                                        const float* w, float* out, float* q, float* k,
                                        const float* qw, const float* kw, const float* cos_tab,
                                        const float* sin_tab, const int32_t* positions,
                                        float* act, const float* gate, const float* up,
                                        size_t hidden, size_t n_heads, size_t n_kv_heads,
                                        size_t head_dim, size_t inter, float eps) {
  for (size_t i = 0; i < iters; ++i) {
    const size_t s = i % sets;
    ref_add_rms_norm(x + s * hidden, delta + s * hidden, w, out + s * hidden, 1, hidden, eps);
    ref_head_rms_norm_rope(q + s * n_heads * head_dim, k + s * n_kv_heads * head_dim, qw, kw,
                           cos_tab, sin_tab, positions + s, 1, n_heads, n_kv_heads, head_dim, eps);
    ref_swiglu_split(act + s * inter, gate + s * inter, up + s * inter, inter);
  }
}
