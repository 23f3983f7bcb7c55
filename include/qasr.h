/*
 * qasr.h — C-ABI of the MI355X (gfx950) fused-layer kernel library for the
 * QwenASR decoder/encoder hot path.
 *
 * Every entry point:
 *   - takes DEVICE pointers (memory from hipMalloc or a torch CUDA tensor),
 *     the dimensions in the same order as the Rust function it replaces, and a
 *     HIP stream passed as `void*` (NULL = the default stream);
 *   - only enqueues work: it never synchronises, never copies to the host and
 *     never allocates (the RoPE-table helpers are the one documented exception:
 *     they are setup calls, like RopeCache::ensure);
 *   - returns a qasr_status; on failure qasr_last_error() gives a message
 *     (thread-local, valid until the next failing call on that thread).
 *
 * The Rust reference returns `()` and panics on bad dimensions (slice bounds).
 * Here a bad dimension or null pointer is QASR_ERR_INVALID_ARG and nothing is
 * launched. Data-dependent faults that the reference would panic on (a token id
 * or RoPE position outside its table) cannot be checked on the host without a
 * synchronisation, so the kernels poison that row with NaN instead of reading
 * out of bounds.
 *
 * Reference citations are relative to crates/qwen-asr/src/ of
 * ZhaoChaoqun/QwenASR.
 */
#ifndef QASR_H
#define QASR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum qasr_status {
  QASR_OK = 0,
  QASR_ERR_INVALID_ARG = 1, /* null pointer, zero-size contract breach, overflow */
  QASR_ERR_UNSUPPORTED = 2, /* a shape the kernels do not implement */
  QASR_ERR_HIP = 3          /* the HIP runtime rejected the launch */
} qasr_status;

/* Library version, (major << 16) | (minor << 8) | patch. */
int qasr_version(void);

/* Message describing the last failing call on this thread ("" if none). */
const char* qasr_last_error(void);

/* ------------------------------------------------------------------------ */
/* Elementwise and normalisation (decoder + encoder)                         */
/* ------------------------------------------------------------------------ */

/* a[i] += b[i], i < n.  Replaces kernels::add_inplace (kernels/mod.rs:486-488). */
int qasr_add_inplace_f32(float* a, const float* b, size_t n, void* stream);

/* out[s,:] = x[s,:] * (1/sqrt(sum(x^2)/hidden + eps)) * weight.
 * Replaces kernels::rms_norm (kernels/mod.rs:897-918, x86 body avx.rs:374-415).
 * out may alias x. */
int qasr_rms_norm_f32(float* out, const float* x, const float* weight,
                      size_t seq_len, size_t hidden, float eps, void* stream);

/* Fused residual add + RMSNorm: x[s,:] += delta[s,:]; out[s,:] = rms_norm(x[s,:]).
 * Replaces the pair add_inplace + rms_norm at decoder.rs:908+910, 924->878,
 * 823+827 and 838->789 (kernels/mod.rs:486-488 then 897-918). x is updated
 * in place (the residual stream); out may alias delta. */
int qasr_add_rms_norm_f32(float* x, const float* delta, const float* weight,
                          float* out, size_t seq_len, size_t hidden, float eps,
                          void* stream);

/* Fused residual add + RMSNorm + per-row int8 quantization of the normalised
 * row (the activation side of a W8A8 projection):
 *   x[s,:] += delta[s,:] (skipped when delta == NULL); y = rms_norm(x[s,:]);
 *   q[s,:], q_scales[s] = quantize_rows_i8(y) (qasr_quantize_rows_i8 arithmetic).
 * out (may be NULL) receives y in fp32. Replaces add_inplace + rms_norm +
 * the activation quantization feeding the gate/up projection
 * (decoder.rs:908-914; kernels/mod.rs:486-488, 897-918; quantize.rs:633-662). */
int qasr_add_rms_norm_quant_f32(float* x, const float* delta, const float* weight,
                                float* out, int8_t* q, float* q_scales, size_t seq_len,
                                size_t hidden, float eps, void* stream);

/* LayerNorm: out = ((x - mean) * inv_std) * weight + bias (fused multiply-add),
 * inv_std = 1/sqrt(var + eps), two-pass mean/variance per row.
 * Replaces kernels::layer_norm (kernels/mod.rs:866-895, avx.rs:417-481). */
int qasr_layer_norm_f32(float* out, const float* x, const float* weight,
                        const float* bias, size_t seq_len, size_t hidden,
                        float eps, void* stream);

/* In-place per-head RMSNorm with a shared head_dim-long weight (q_norm/k_norm).
 * Replaces kernels::rms_norm_per_head (kernels/mod.rs:920-935). */
int qasr_rms_norm_per_head_f32(float* x, const float* weight, size_t seq_len,
                               size_t n_heads, size_t head_dim, float eps,
                               void* stream);

/* In-place NeoX half-rotation RoPE; row s uses cos_vals/sin_vals row s
 * (each row head_dim long: [c(0..half) | c(0..half)]).
 * Replaces kernels::apply_rope_neox (kernels/mod.rs:1247-1267). */
int qasr_apply_rope_neox_f32(float* x, const float* cos_vals,
                             const float* sin_vals, size_t seq,
                             size_t n_heads, size_t head_dim, void* stream);

/* Fused q/k head RMSNorm + RoPE with per-row positions:
 *   q[s,h,:] = rope(rms_norm_head(q[s,h,:], q_norm_w), positions[s])
 *   k[s,h,:] = rope(rms_norm_head(k[s,h,:], k_norm_w), positions[s])
 * cos_tab/sin_tab are RopeCache tables of table_rows rows of head_dim floats
 * (decoder.rs:253-289). positions == NULL means row s uses position s.
 * table_rows must be at least 1; a position outside [0, table_rows) poisons
 * that row's q and k with NaN.
 * Replaces rms_norm_per_head x2 + apply_rope_neox x2 at decoder.rs:455-459,
 * 543-547, 799-803, 888-892 (kernels/mod.rs:920-935, 1247-1267). k may be NULL
 * when n_kv_heads == 0. */
int qasr_head_rms_norm_rope_f32(float* q, float* k, const float* q_norm_w,
                                const float* k_norm_w, const float* cos_tab,
                                const float* sin_tab, const int32_t* positions,
                                size_t seq, size_t n_heads, size_t n_kv_heads,
                                size_t head_dim, size_t table_rows, float eps,
                                void* stream);

/* qasr_head_rms_norm_rope_f32 with the KV-cache store fused in (the step
 * after q/k norm + RoPE in every decoder layer):
 *   q[s,h,:]  = rope(rms_norm_head(q[s,h,:], q_norm_w), p)        (in place)
 *   k_cache[row, h, :] = rope(rms_norm_head(k[s,h,:], k_norm_w), p)
 *   v_cache[row, h, :] = v[s,h,:]
 * with p = start_pos + s and row = p when positions == NULL (one sequence:
 * k_cache/v_cache point at the layer's [cache_rows][n_kv_heads*head_dim]
 * block, KvCache::k_at/v_at of decoder.rs:194-202), or p = positions[s] and
 * row = s * cache_rows + p otherwise (row s is its own decode stream with its
 * own [cache_rows][kv_dim] block). k and v are read, not modified.
 * A row whose p lies outside the RoPE table or the cache gets a NaN q row and
 * no cache write. Replaces rms_norm_per_head x2 + apply_rope_neox x2 + the
 * k_at/v_at copies at decoder.rs:455-462, 543-550, 799-810, 888-895.
 * head_dim 64/128/256/512 and 16-byte aligned buffers (else UNSUPPORTED). */
int qasr_head_rms_norm_rope_kv_f32(float* q, const float* k, const float* v,
                                   const float* q_norm_w, const float* k_norm_w,
                                   const float* cos_tab, const float* sin_tab,
                                   const int32_t* positions, size_t start_pos, size_t seq,
                                   size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                   size_t table_rows, float eps, float* k_cache,
                                   float* v_cache, size_t cache_rows, void* stream);

/* Fill RoPE table rows [pos_begin, pos_end) for theta and head_dim:
 *   inv_freq[d] = 1 / theta^((2d)/head_dim)   (f32 powf, computed on the host
 *   once per call exactly as RopeCache::ensure does, decoder.rs:262-266)
 *   angle = (f32)pos * inv_freq[d]; row = [cos(angle) | cos(angle)], same for sin.
 * cos_tab/sin_tab must hold pos_end rows of head_dim floats. This is the
 * table-growth step of RopeCache::ensure (decoder.rs:253-289); head_dim even,
 * head_dim <= 512. */
int qasr_rope_table_fill_f32(float* cos_tab, float* sin_tab, size_t pos_begin,
                             size_t pos_end, size_t head_dim, float theta,
                             void* stream);

/* out[s,j] = silu(gate_up[s,2j]) * gate_up[s,2j+1] on the row-interleaved
 * gate/up buffer. Arithmetic follows the x86_64 reference: blocks of 8 use the
 * degree-5 fast_exp polynomial, the row tail uses expf.
 * Replaces kernels::swiglu_multiply (kernels/mod.rs:965-985, avx.rs:483-514,
 * 565-599). */
int qasr_swiglu_multiply_f32(float* out, const float* gate_up, size_t seq_len,
                             size_t intermediate, void* stream);

/* out[j] = silu(gate[j]) * up[j] with silu(g) = g / (1 + expf(-g)) on split
 * gate/up buffers. out may alias gate (then it is swiglu_multiply_inplace,
 * kernels/mod.rs:988-994); the decode loop's inline SwiGLU uses the same
 * arithmetic (decoder.rs:571-576, 916-921). */
int qasr_swiglu_split_f32(float* out, const float* gate, const float* up,
                          size_t n, void* stream);

/* x[i] = x[i] / (1 + expf(-x[i])).  Replaces kernels::silu (kernels/mod.rs:941-946). */
int qasr_silu_f32(float* x, size_t n, void* stream);

/* tanh-approximation GELU in place, x86_64 reference arithmetic (blocks of 8 via
 * fast_exp, tail via tanhf). Replaces kernels::gelu (kernels/mod.rs:948-963,
 * avx.rs:533-563). */
int qasr_gelu_tanh_f32(float* x, size_t n, void* stream);

/* Exact GELU in place: x = 0.5 * x * (1 + erf(x / sqrt(2))), evaluated as
 * 0.5 * x * erfc(-x / sqrt(2)). The reference CPU path has only the tanh form;
 * erf-GELU is what its Metal path calls (encoder_gpu.rs:470,480). */
int qasr_gelu_erf_f32(float* x, size_t n, void* stream);

/* pe[p, d] = sin(p * inv[d]), pe[p, half + d] = cos(p * inv[d]),
 * inv[d] = exp(-d * ln(10000) / (half - 1)).
 * Replaces kernels::sinusoidal_pe (kernels/mod.rs:1213-1226). */
int qasr_sinusoidal_pe_f32(float* pe, size_t n_pos, size_t d_model, void* stream);

/* x[r,:] += pe[r mod n_pos, :] for r < rows. Replaces the per-chunk
 * sinusoidal_pe + add_inplace at encoder.rs:340-343 and 599-601, with the PE
 * table built once by qasr_sinusoidal_pe_f32. */
int qasr_pe_add_f32(float* x, const float* pe, size_t rows, size_t d_model,
                    size_t n_pos, void* stream);

/* x[r,:] += pe[r mod n_pos, :], then out = layer_norm(x) (the arithmetic of
 * qasr_layer_norm_f32), in one pass over the rows. Replaces the encoder's PE
 * add (encoder.rs:341-343, 599-601) together with layer 0's attention
 * LayerNorm of the same rows (encoder.rs:370-371, 625-626; kernels/mod.rs:866-895).
 * x and out equal those of qasr_pe_add_f32 followed by qasr_layer_norm_f32 bit
 * for bit. out and pe must not overlap x. */
int qasr_pe_add_layer_norm_f32(float* x, const float* pe, float* out, const float* weight,
                               const float* bias, size_t rows, size_t d_model, size_t n_pos,
                               float eps, void* stream);

/* x += delta, then out = layer_norm(x) (the arithmetic of qasr_add_inplace_f32
 * and qasr_layer_norm_f32) in one pass over the rows. Replaces each encoder
 * residual add together with the LayerNorm that reads its rows next:
 * add_inplace (encoder.rs:386, 397; kernels/mod.rs:486-488) + layer_norm
 * (encoder.rs:389-390 and the next layer's 370-371, or the final 401-402;
 * kernels/mod.rs:866-895). x and out equal those of the two calls bit for bit.
 * x, delta and out must not overlap. */
int qasr_add_layer_norm_f32(float* x, const float* delta, const float* weight, const float* bias,
                            float* out, size_t seq_len, size_t hidden, float eps, void* stream);

/* ------------------------------------------------------------------------ */
/* Token-embedding gather (decoder.rs:631-646, context.rs:115-124)           */
/* ------------------------------------------------------------------------ */

/* out[i,:] = table[ids[i],:] (fp32 table of vocab rows). An id outside
 * [0, vocab) poisons out[i,:] with NaN. */
int qasr_embed_gather_f32(float* out, const float* table, const int32_t* ids,
                          size_t n, size_t dim, size_t vocab, void* stream);

/* out[i,:] = bf16->f32(table[ids[i],:]) by a 16-bit shift.
 * Replaces tok_embed_bf16_to_f32 (decoder.rs:631-636) for n tokens at once. */
int qasr_embed_gather_bf16(float* out, const uint16_t* table,
                           const int32_t* ids, size_t n, size_t dim,
                           size_t vocab, void* stream);

/* out[i,:] = (f32)table[ids[i],:] * row_scales[ids[i]].
 * Replaces tok_embed_int8_to_f32 (decoder.rs:639-646) for n tokens at once. */
int qasr_embed_gather_i8(float* out, const int8_t* table,
                         const float* row_scales, const int32_t* ids, size_t n,
                         size_t dim, size_t vocab, void* stream);

/* ------------------------------------------------------------------------ */
/* INT8 (qwen-asr-quantize .qint8 format)                                    */
/* ------------------------------------------------------------------------ */

/* Per-row symmetric int8 quantization: absmax, scale = absmax/127,
 * inv = 127/absmax (0 if absmax == 0), q = clamp(roundf(v*inv), -128, 127)
 * (round half away from zero; NaN -> 0). Same routine as
 * quantize_f32_to_int8 (quantize.rs:633-662); applied to activations it is the
 * per-vector quantization of the W8A8 path. */
int qasr_quantize_rows_i8(int8_t* q, float* scales, const float* x,
                          size_t rows, size_t cols, void* stream);

/* W8A32 linear, no bias: y[s,o] = (sum_k (f32)w[o,k] * x[s,k]) * scales[o].
 * Replaces kernels::linear_nobias_int8 (kernels/mod.rs:650-661,
 * generic.rs:37-49). Products are exact and summed in fp32 on every path (the
 * reference's arithmetic, another summation order). From 8 tokens up (with
 * in_dim % 64 == 0 and 16-byte aligned w and x) the call is one matrix-core
 * GEMM instead of the reference's per-token matvecs: x is split exactly into
 * three bf16 terms and int8 weights are exact in bf16. On that path a
 * non-finite activation turns its output row to NaN (the reference may give
 * +-inf there); finite inputs give the same results as the other paths. */
int qasr_linear_nobias_int8_f32(float* y, const float* x, const int8_t* w,
                                const float* scales, size_t seq_len,
                                size_t in_dim, size_t out_dim, void* stream);

/* The INT8 decode step's gate/up projection and SwiGLU in one call
 * (decoder.rs:912-921): gate_up = linear_nobias_int8(x, w_gate_up) on the
 * row-interleaved fused weight [2*intermediate, in_dim] (g0, u0, g1, u1, ...,
 * with interleaved scales), then out[s, j] = g / (1 + expf(-g)) * u with
 * g = gate_up[s, 2j], u = gate_up[s, 2j + 1] -- the decode loop's libm SwiGLU,
 * not the prefill fast_exp form. The gate_up values are never written. Several
 * rows (decode streams, seq_len >= 8, in_dim % 64 == 0, 16-byte aligned x and
 * w) run the matrix-core GEMM of qasr_linear_nobias_int8_f32 with the SwiGLU
 * in its epilogue. */
int qasr_gate_up_swiglu_int8_f32(float* out, const float* x, const int8_t* w_gate_up,
                                 const float* scales_gate_up, size_t seq_len, size_t in_dim,
                                 size_t intermediate, void* stream);

/* The prefill's gate/up projection and SwiGLU in one call (decoder.rs:831-834):
 * gate_up = linear_nobias_int8(x, w_gate_up) on the row-interleaved fused
 * weight, then kernels::swiglu_multiply (kernels/mod.rs:965-985, the
 * fast_exp form of avx.rs:565-599: out[s, j] = silu(gate_up[s, 2j]) *
 * gate_up[s, 2j + 1]). The gate_up values are never written. From 8 tokens
 * (the matrix-core GEMM path of qasr_linear_nobias_int8_f32) equal bit for
 * bit to qasr_linear_nobias_int8_f32 followed by qasr_swiglu_multiply_f32;
 * below, one wave per (token, output) takes the two dots (fp32, another
 * order). No reference counterpart as one call. */
int qasr_gate_up_swiglu_multiply_int8_f32(float* out, const float* x, const int8_t* w_gate_up,
                                          const float* scales_gate_up, size_t seq_len,
                                          size_t in_dim, size_t intermediate, void* stream);

/* Up to 4 W8A32 projections of the same input in one launch: for m < n_mats,
 * ys[m][s, :] = qasr_linear_nobias_int8_f32(x[s, :], ws[m], scales[m]) with
 * out_dims[m] rows (the q/k/v calls of one decode step share x:
 * decoder.rs:881-886). Same results as the separate calls, bit for bit. ys, ws,
 * scales and out_dims are host arrays of n_mats device pointers / sizes. */
int qasr_linear_nobias_int8_multi_f32(size_t n_mats, float* const* ys,
                                      const int8_t* const* ws, const float* const* scales,
                                      const size_t* out_dims, const float* x, size_t seq_len,
                                      size_t in_dim, void* stream);

/* A prefill chunk's q/k/v projections with the steps after them in one launch
 * (decoder.rs:795-810: the three linear_nobias_int8 calls, per-head RMSNorm
 * of q and k, NeoX RoPE, and the k_at/v_at copies into the layer's cache).
 * Token s of x [seq_len, in_dim] is at position p = start_pos + s:
 *   q[s, :]            = rope(rms_norm_head(x[s] . wq^T * sq, q_norm_w), p)
 *   k_cache[p, :]      = rope(rms_norm_head(x[s] . wk^T * sk, k_norm_w), p)
 *   v_cache[p, :]      = x[s] . wv^T * sv
 * with wq [n_heads*head_dim, in_dim], wk/wv [n_kv_heads*head_dim, in_dim] and
 * the caches the layer's [cache_rows][n_kv_heads*head_dim] blocks. Rows
 * start_pos..start_pos+seq_len must lie inside the cache and the RoPE table
 * (QASR_ERR_INVALID_ARG otherwise, as qasr_head_rms_norm_rope_kv_f32).
 * Bit-identical to qasr_linear_nobias_int8_multi_f32 (q, k, v) followed by
 * qasr_head_rms_norm_rope_kv_f32 (positions NULL): the raw k and v rows are
 * never written. head_dim 128, seq_len >= 8, in_dim % 64 == 0 and 16-byte
 * aligned buffers (QASR_ERR_UNSUPPORTED otherwise). No reference counterpart
 * as one call. */
int qasr_qkv_heads_int8_f32(float* q, float* k_cache, float* v_cache, size_t cache_rows,
                            const int8_t* wq, const float* sq, const int8_t* wk, const float* sk,
                            const int8_t* wv, const float* sv, const float* x, size_t seq_len,
                            size_t in_dim, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            const float* q_norm_w, const float* k_norm_w, const float* cos_tab,
                            const float* sin_tab, size_t table_rows, size_t start_pos, float eps,
                            void* stream);

/* The prefill residual add folded into the o / down projection:
 * h[t, :] += linear_nobias_int8(x[t, :], w, scales) for t < seq_len, and
 * ss[t * ceil(out_dim / 64) + s] = the sum of squares of h[t, 64s .. 64s+63]
 * after the add; with hg (and gain, [out_dim]), also hg[t, n] = h[t, n] *
 * gain[n] -- the statistics and the gain-scaled rows the next RMSNorm needs
 * (the two qasr_rms_norm_* entry points below). Replaces linear_nobias_int8 +
 * add_inplace (decoder.rs:821-822, 837-838; kernels/mod.rs:486-488): h equals
 * them bit for bit. ss holds seq_len * ceil(out_dim / 64) floats; x must not
 * overlap h or hg; hg and gain are both NULL or both given. seq_len >= 8,
 * in_dim % 64 == 0 and 16-byte aligned h, hg, x, w (QASR_ERR_UNSUPPORTED
 * otherwise). No reference counterpart as one call. */
int qasr_linear_int8_residual_f32(float* h, float* ss, float* hg, const float* gain, const float* x,
                                  const int8_t* w, const float* scales, size_t seq_len, size_t in_dim,
                                  size_t out_dim, void* stream);

/* The prefill post-attention RMSNorm folded into the gate/up projection +
 * SwiGLU (decoder.rs:826-833): out = swiglu_multiply(gate/up(x_norm)) as
 * qasr_gate_up_swiglu_multiply_int8_f32, with x_norm[t] = rms_norm(h[t]) *
 * norm_w taken as hg[t] * rinv[t]: hg = h * norm_w and the ss_slices =
 * ceil(in_dim / 64) partial sums of squares from
 * qasr_linear_int8_residual_f32, added in slice order into rinv =
 * 1 / sqrt(sum / in_dim + norm_eps). The GEMM stages hg and multiplies each
 * token's outputs by rinv; shapes it does not take (few tokens, in_dim > 2048
 * or not a multiple of 256) write hg * rinv into x_norm ([seq_len, in_dim];
 * x_norm == hg is allowed) and run the plain launch. Results equal the
 * reference's rms_norm + gate/up + swiglu_multiply within fp32 rounding (rinv
 * is factored out of the dot products; the sum of squares is added in
 * another order). No reference counterpart as one call. */
int qasr_rms_norm_gate_up_swiglu_multiply_int8_f32(float* out, const float* hg, const float* ss,
                                                   size_t ss_slices, float norm_eps, float* x_norm,
                                                   const int8_t* w_gate_up,
                                                   const float* scales_gate_up, size_t seq_len,
                                                   size_t in_dim, size_t intermediate,
                                                   void* stream);

/* The prefill layer-input RMSNorm folded into qasr_qkv_heads_int8_f32
 * (decoder.rs:789-810): the activations are hg = h * input_norm, each token's
 * outputs multiplied by its rinv from ss, as in
 * qasr_rms_norm_gate_up_swiglu_multiply_int8_f32 (including the x_norm
 * fallback); the rest of the contract is qasr_qkv_heads_int8_f32's (eps is the
 * head norms'). No reference counterpart as one call. */
int qasr_rms_norm_qkv_heads_int8_f32(float* q, float* k_cache, float* v_cache, size_t cache_rows,
                                     const int8_t* wq, const float* sq, const int8_t* wk,
                                     const float* sk, const int8_t* wv, const float* sv,
                                     const float* hg, const float* ss, size_t ss_slices,
                                     float norm_eps, float* x_norm, size_t seq_len, size_t in_dim,
                                     size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                     const float* q_norm_w, const float* k_norm_w,
                                     const float* cos_tab, const float* sin_tab, size_t table_rows,
                                     size_t start_pos, float eps, void* stream);

/* One decode token's layer-input residual add + RMSNorm and the projections
 * that read it, in one launch: h = x + delta (delta may be NULL: h = x),
 * xn = rms_norm(h) * norm_w, ys[m] = linear_nobias_int8(xn, ws[m], scales[m]).
 * Replaces the pairs add_inplace + rms_norm (decoder.rs:924->878, 908+910,
 * kernels/mod.rs:486-488, 897-918) followed by the projections that consume
 * the normalised row (q/k/v decoder.rs:881-886). Every workgroup normalises
 * the row itself, in the element order of qasr_add_rms_norm_f32, so ys equal
 * qasr_add_rms_norm_f32 + qasr_linear_nobias_int8_multi_f32 at one token bit
 * for bit. h is written to h_out (NULL: not written), which must not overlap x
 * or delta: the residual stream alternates between two buffers. One token;
 * in_dim 1024..8192 in steps of 1024 (QASR_ERR_UNSUPPORTED otherwise). */
int qasr_add_rms_norm_linear_nobias_int8_multi_f32(size_t n_mats, float* const* ys,
                                                   const int8_t* const* ws,
                                                   const float* const* scales,
                                                   const size_t* out_dims, float* h_out,
                                                   const float* x, const float* delta,
                                                   const float* norm_w, size_t in_dim,
                                                   float eps, void* stream);

/* The post-attention residual add + RMSNorm and the gate/up projection +
 * SwiGLU of one decode token in one launch (decoder.rs:908-921): as
 * qasr_add_rms_norm_linear_nobias_int8_multi_f32, with the output of
 * qasr_gate_up_swiglu_int8_f32 on the normalised row; equal bit for bit to
 * qasr_add_rms_norm_f32 followed by qasr_gate_up_swiglu_int8_f32. */
int qasr_add_rms_norm_gate_up_swiglu_int8_f32(float* out, float* h_out, const float* x,
                                              const float* delta, const float* norm_w,
                                              const int8_t* w_gate_up,
                                              const float* scales_gate_up, size_t in_dim,
                                              size_t intermediate, float eps, void* stream);

/* W8A32 linear with optional bias (bias may be NULL): y = linear_nobias + bias.
 * Replaces kernels::linear_int8 (kernels/mod.rs:664-673). */
int qasr_linear_int8_f32(float* y, const float* x, const int8_t* w,
                         const float* scales, const float* bias,
                         size_t seq_len, size_t in_dim, size_t out_dim,
                         void* stream);

/* Row-interleave separate gate [inter,hidden] and up [inter,hidden] int8
 * matrices (and their scales) into the fused [2*inter,hidden] layout
 * g0,u0,g1,u1,... the decoder builds at load time (decoder.rs:701-719). */
int qasr_interleave_gate_up_i8(int8_t* w_gate_up, float* scales_gate_up,
                               const int8_t* w_gate, const float* s_gate,
                               const int8_t* w_up, const float* s_up,
                               size_t intermediate, size_t hidden, void* stream);

/* W8A8 gate/up projection fused with SwiGLU, int32-exact dot products:
 *   dg = sum_k w[2j,k]*xq[b,k],  du = sum_k w[2j+1,k]*xq[b,k]     (int32)
 *   g  = ((f32)dg * x_scales[b]) * scales[2j]
 *   u  = ((f32)du * x_scales[b]) * scales[2j+1]
 *   out[b,j] = (g / (1 + expf(-g))) * u
 * w is the row-interleaved fused gate/up matrix [2*inter, in_dim] and scales
 * its interleaved per-row scales (decoder.rs:701-719). batch == 1 runs a
 * bandwidth-bound matvec; batch > 1 runs an MFMA int8 GEMM. in_dim % 16 == 0.
 * No reference counterpart: the reference runs this projection W8A32
 * (decoder.rs:912-921 -> kernels/mod.rs:650-661) followed by SwiGLU. */
int qasr_gate_up_swiglu_w8a8(float* out, const int8_t* w, const float* scales,
                             const int8_t* xq, const float* x_scales,
                             size_t batch, size_t in_dim, size_t intermediate,
                             void* stream);

/* Re-lays a row-major int8 weight matrix [rows, cols] into MFMA A-operand
 * tiles (v_mfma_i32_16x16x64_i8): for each 16-row block rb and 64-byte k-step
 * s one contiguous 1 KiB tile whose byte 16*l + b is
 * W[16*rb + l%16][64*s + 16*(l/16) + b]; tiles are ordered [rb][s].
 * rows % 16 == 0, cols % 64 == 0, out of place. A one-time
 * load-time transform of the device weights, like the gate/up row interleave
 * the decoder builds at load (decoder.rs:701-719); scales are unchanged.
 * No reference counterpart (the reference reads .qint8 rows directly). */
int qasr_pack_w8a8_tiles(int8_t* packed, const int8_t* w, size_t rows,
                         size_t cols, void* stream);

/* qasr_gate_up_swiglu_w8a8 on tile-packed weights: w_packed is
 * qasr_pack_w8a8_tiles of the row-interleaved gate/up matrix. Same arithmetic
 * and results. Needs in_dim 1024 or 2048 and (2*intermediate) % 192 == 0
 * (QASR_ERR_UNSUPPORTED otherwise); out 8-byte aligned. */
int qasr_gate_up_swiglu_w8a8_packed(float* out, const int8_t* w_packed,
                                    const float* scales, const int8_t* xq,
                                    const float* x_scales, size_t batch,
                                    size_t in_dim, size_t intermediate,
                                    void* stream);

/* Batched W8A8 projection on tile-packed weights (qasr_pack_w8a8_tiles):
 *   y[m, n] = ((f32)dot[m, n] * x_scales[m]) * scales[n],
 *   dot[m, n] = sum_k w[n, k] * xq[m, k]   (int32, exact)
 * for m < batch streams (xq, x_scales: qasr_quantize_rows_i8 or
 * qasr_add_rms_norm_quant_f32 of each stream's row). The reference's
 * linear_nobias_int8 (kernels/mod.rs:650-661, one W8A32 matvec per token) with
 * the activation quantized per row, as the batched gate/up projection does;
 * the integer dots are exact, so y equals the oracle's bit for bit. in_dim
 * 1024, 2048, 3072, 4096 or 6144, out_dim % 128 == 0, 16-byte aligned buffers
 * (QASR_ERR_UNSUPPORTED otherwise). Outputs wide enough for 4+ tiles per CU
 * (a batch's lm_head) run persistent workgroups that each walk a range of
 * column tiles; the results are the same. */
int qasr_linear_w8a8_packed(float* y, const int8_t* w_packed, const float* scales,
                            const int8_t* xq, const float* x_scales, size_t batch,
                            size_t in_dim, size_t out_dim, void* stream);

/* The q/k/v projections of `batch` decode streams, each at its own position,
 * with the steps after them in one launch (decoder.rs:881-895 per stream):
 * w_packed is the packed [(n_heads + 2 n_kv_heads) * head_dim, in_dim] matrix
 * of the q rows, then the k rows, then the v rows (scales likewise). For
 * stream m at pos = positions[m]:
 *   q = the q rows of qasr_linear_w8a8_packed -> per-head RMSNorm (q_norm_w)
 *       -> NeoX RoPE with table row pos, written to q_out[m, :];
 *   k = likewise with k_norm_w, written to k_cache row pos of stream m;
 *   v = the v rows, written to v_cache row pos of stream m.
 * Stream m's cache block is k_cache + m * cache_rows * n_kv_heads * head_dim
 * (the reference's KvCache layer layout, one block per stream). A position
 * outside the RoPE table or the cache gives a NaN q row and no cache write.
 * Bit-identical to qasr_linear_w8a8_packed followed by
 * qasr_head_rms_norm_rope_kv_f32 with positions. head_dim 128, in_dim as for
 * qasr_linear_w8a8_packed, 16-byte aligned buffers (QASR_ERR_UNSUPPORTED
 * otherwise). No reference
 * counterpart as one call (the reference decodes one stream at a time). */
int qasr_qkv_heads_w8a8_packed(float* q_out, float* k_cache, float* v_cache, size_t cache_rows,
                               const int8_t* w_packed, const float* scales, const int8_t* xq,
                               const float* x_scales, const float* q_norm_w,
                               const float* k_norm_w, const float* cos_tab,
                               const float* sin_tab, size_t table_rows,
                               const int32_t* positions, size_t batch, size_t in_dim,
                               size_t n_heads, size_t n_kv_heads, size_t head_dim, float eps,
                               void* stream);

/* As qasr_gate_up_swiglu_w8a8 for batch == 1 with an fp32 input vector that
 * the kernel quantizes per-vector itself (qasr_quantize_rows_i8 arithmetic),
 * so one launch covers quantize + matvec + SwiGLU. */
int qasr_gate_up_swiglu_w8a8_f32in(float* out, const int8_t* w,
                                   const float* scales, const float* x,
                                   size_t in_dim, size_t intermediate,
                                   void* stream);

/* ------------------------------------------------------------------------ */
/* Attention (kernels/mod.rs:1124-1207)                                      */
/* ------------------------------------------------------------------------ */

/* Causal grouped-query attention: for query row i (global position
 * q_offset + i) and head h, keys j < min(q_offset + i + 1, seq_k) of kv head
 * h / (n_heads / n_kv_heads):
 *   out[i,h,:] = sum_j softmax_j(q[i,h,:] . k[j,kvh,:] * scale) * v[j,kvh,:]
 * q, out: [seq_q, n_heads*head_dim]; k, v: [seq_k, n_kv_heads*head_dim]
 * (a KvCache layer block, KvCache::k_layer_full of decoder.rs:212-222).
 * A row with no keys gets zeros. Replaces kernels::causal_attention
 * (kernels/mod.rs:1124-1207; calls decoder.rs:472-476, 561-564, 818-821,
 * 900-903). head_dim 64 or 128, n_heads / n_kv_heads in {1, 2, 4, 8},
 * 16-byte aligned buffers (else UNSUPPORTED). */
int qasr_causal_attention_f32(float* out, const float* q, const float* k, const float* v,
                              size_t seq_q, size_t seq_k, size_t n_heads, size_t n_kv_heads,
                              size_t head_dim, float scale, size_t q_offset, void* stream);

/* qasr_causal_attention_f32 for decode-shaped calls (few query rows, long
 * key ranges): the keys of each (row, kv head) are split over up to 64
 * workgroups whose partial (max, sum, output) triples go to the caller's
 * workspace and are merged by a second kernel, so a single decode stream
 * uses the whole GPU. Same results within rounding (the merge reorders the
 * softmax sums). workspace: 16-byte aligned, at least
 * qasr_causal_attention_workspace_floats(seq_q, n_heads, head_dim) floats for
 * the full split; with less (or NULL) it falls back to fewer or no splits.
 * Calls that share a workspace must not run concurrently (one stream).
 * No reference counterpart: the reference threads over heads
 * (kernels/mod.rs:1174-1203); this is its single-stream GPU shape. */
int qasr_causal_attention_split_f32(float* out, const float* q, const float* k, const float* v,
                                    size_t seq_q, size_t seq_k, size_t n_heads,
                                    size_t n_kv_heads, size_t head_dim, float scale,
                                    size_t q_offset, float* workspace, size_t workspace_floats,
                                    void* stream);

/* One decode token's attention block after the q/k/v projections, the
 * layer's steps of decoder.rs:888-903 in one call: q/k head RMSNorm + RoPE at
 * position pos, the K/V rows stored into the layer's cache block, and causal
 * attention of the token over cache rows 0..pos. Same results, bit for bit,
 * as qasr_head_rms_norm_rope_kv_f32(q, k, v, ..., positions = NULL,
 * start_pos = pos, seq = 1, ...) followed by
 * qasr_causal_attention_split_f32(out, q, k_cache, v_cache, 1, pos + 1, ...,
 * q_offset = pos, workspace, ...). When the keys are split over workgroups
 * (workspace large enough, pos >= 255, head_dim 128 with n_heads/n_kv_heads
 * <= 2 or head_dim 64 with <= 4) it is a single attention launch (+ merge):
 * every workgroup normalises and rotates its q heads itself and the one
 * holding key pos writes the cache rows; q is then left as given. Otherwise
 * it runs the two calls, and q holds its normalised, rotated rows: treat q
 * as scratch. pos must lie inside the RoPE table and the cache (INVALID_ARG
 * otherwise; the two-call form writes NaN rows instead). No reference
 * counterpart as one call. */
int qasr_decode_attention_f32(float* out, float* q, const float* k, const float* v,
                              const float* q_norm_w, const float* k_norm_w, const float* cos_tab,
                              const float* sin_tab, size_t table_rows, size_t pos, size_t n_heads,
                              size_t n_kv_heads, size_t head_dim, float eps, float scale,
                              float* k_cache, float* v_cache, size_t cache_rows, float* workspace,
                              size_t workspace_floats, void* stream);

/* Decode attention of `batch` streams, each over its own cache block
 * (decoder.rs:900-903 per stream): for stream m at pos = positions[m], out[m]
 * = causal attention of q[m] (n_heads*head_dim, already normalised and
 * rotated) over rows 0..pos of k_cache/v_cache + m * cache_rows *
 * n_kv_heads * head_dim (the block qasr_head_rms_norm_rope_kv_f32 with
 * positions writes). With a workspace of at least
 * qasr_batched_decode_attention_workspace_floats() floats, each stream's keys
 * are cut into chunks of 512 (streams at different positions then cost the
 * GPU evenly) and the chunks' partial results are merged in a second launch;
 * with workspace NULL one workgroup per (stream, kv head) walks all of its
 * keys. Both give the oracle's result within 1e-5 (the order of the key sums
 * differs). The workspace is scratch for one call at a time on a stream. A
 * position outside the cache gives a NaN row. head_dim 128 with
 * n_heads/n_kv_heads in {1, 2}, or 64 with {1, 2, 4}; 16-byte aligned
 * buffers (QASR_ERR_UNSUPPORTED otherwise); a workspace that is too small is
 * QASR_ERR_INVALID_ARG. With out_q and out_scales (both or neither; int8
 * [batch, n_heads * head_dim], f32 [batch]) each stream's row is also
 * quantized per row in the launch that merges the chunks, with the values
 * and scale qasr_quantize_rows_i8 gives on out (the input of a W8A8 o
 * projection; n_heads * head_dim * 4 <= 65536). With order (from
 * qasr_batched_decode_order_i32 on the same positions) the streams are
 * walked longest first, which evens out the tail of a batch at different
 * positions; the results are the same. An order that is not a permutation of
 * the batch leaves the rows of the streams it misses unwritten (never out of
 * bounds). No reference counterpart as one call (the reference decodes one
 * stream at a time). */
int qasr_batched_decode_attention_f32(float* out, const float* q, const float* k_cache,
                                      const float* v_cache, size_t cache_rows,
                                      const int32_t* positions, size_t batch, size_t n_heads,
                                      size_t n_kv_heads, size_t head_dim, float scale, float* workspace,
                                      size_t workspace_floats, int8_t* out_q, float* out_scales,
                                      const int32_t* order, void* stream);

/* order[2r], order[2r + 1] = the stream of rank r and its position, ranking
 * the batch's streams by their number of keys (positions[m] + 1; 0 for a
 * position outside [0, cache_rows)), most first, ties by stream index. One
 * launch; the same order serves every layer of a decode step (positions
 * change only between steps). batch <= 65536. No reference counterpart. */
int qasr_batched_decode_order_i32(int32_t* order, const int32_t* positions, size_t batch,
                                  size_t cache_rows, void* stream);

/* Workspace floats qasr_batched_decode_attention_f32 uses for these sizes (0:
 * the cache is one chunk, no workspace is needed). */
size_t qasr_batched_decode_attention_workspace_floats(size_t batch, size_t n_heads, size_t head_dim,
                                                      size_t cache_rows);

/* Workspace floats qasr_causal_attention_split_f32 can use for these sizes. */
size_t qasr_causal_attention_workspace_floats(size_t seq_q, size_t n_heads, size_t head_dim);

/* ------------------------------------------------------------------------ */
/* lm_head (decoder.rs:929-963)                                              */
/* ------------------------------------------------------------------------ */

/* idx[r] = index of the largest x[r, :] as the reference's greedy loop finds
 * it (decoder.rs:941-949: start at element 0, replace on a strict `>`): the
 * first maximum wins, NaN never wins, and a NaN in element 0 gives 0. */
int qasr_argmax_rows_f32(int32_t* idx, const float* x, size_t rows, size_t cols,
                         void* stream);

/* INT8 lm_head + argmax for `rows` hidden states: logits[r, :] =
 * linear_nobias_int8(x[r, :]) (qasr_linear_nobias_int8_f32 arithmetic, the
 * reference's kernels::linear_nobias_int8 call at decoder.rs:939 and 954),
 * then idx[r] = the qasr_argmax_rows_f32 index of logits[r, :]. logits is
 * caller-owned [rows, vocab] and keeps the logits.
 *
 * workspace (8-byte aligned, may be NULL): with rows == 1 and at least
 * qasr_lm_head_argmax_workspace_bytes(vocab) bytes, the matvec reduces its
 * rows to per-workgroup candidates there and one small kernel merges them
 * (no second pass over the logits). Without it, or for rows > 1, the logits
 * are scanned after the matvec. Same idx either way. Calls that share a
 * workspace must be ordered on one stream. */
int qasr_lm_head_int8_argmax_f32(int32_t* idx, float* logits, const float* x,
                                 const int8_t* w, const float* scales, size_t rows,
                                 size_t in_dim, size_t vocab, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Workspace bytes qasr_lm_head_int8_argmax_f32 can use for this vocab. */
size_t qasr_lm_head_argmax_workspace_bytes(size_t vocab);

/* qasr_lm_head_int8_argmax_f32 without a workspace and without allocating:
 * no counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * The one-row candidates go to a 512 KiB array the library holds on each GPU
 * it runs on until the process ends (looked up once per device on the first
 * call there; nothing is allocated, no call here allocates). Same results as
 * qasr_lm_head_int8_argmax_f32 with a workspace. One row needs in_dim
 * 1024..8192 in steps of 1024 and 16-byte aligned x and w (UNSUPPORTED
 * otherwise); vocab at most QASR_LM_HEAD_NOALLOC_MAX_VOCAB (INVALID_ARG
 * otherwise). rows > 1 writes the logits and scans them, as the workspace
 * form does. All calls on one GPU share the array: calls that overlap in time
 * on one GPU (two streams or threads) race; calls ordered on one stream do
 * not. */
#define QASR_LM_HEAD_NOALLOC_MAX_VOCAB 262144
int qasr_lm_head_int8_argmax_noalloc_f32(int32_t* idx, float* logits, const float* x,
                                         const int8_t* w, const float* scales, size_t rows,
                                         size_t in_dim, size_t vocab, void* stream);

/* ------------------------------------------------------------------------ */
/* .qint8 weight files (quantize.rs:1-34, QuantFile quantize.rs:114-300)     */
/* ------------------------------------------------------------------------ */

/* Tensor dtypes of a .qint8 file (the V2 dtype byte; V1 infers them). */
enum { QASR_QINT8_INT8 = 0, QASR_QINT8_F32 = 1, QASR_QINT8_BF16 = 2 };

typedef struct qasr_qint8_file qasr_qint8_file;

/* Maps `path` read-only and parses its tensor table as QuantFile::open does
 * (quantize.rs:122-245): V1 or V2 magic, V1 dtype from scale_offset, unknown
 * V2 dtype as INT8, a table cut short by the end of the file ends there.
 * Host-side setup call (no device work). */
int qasr_qint8_open(const char* path, qasr_qint8_file** out);
/* Unmaps the file. If any upload was queued from it, first waits for the
 * device (copies from the mapping may still be in flight). NULL is a no-op. */
int qasr_qint8_close(qasr_qint8_file* f);

/* Format version (1 or 2) and number of tensors parsed. */
int qasr_qint8_info(const qasr_qint8_file* f, int* version, size_t* n_tensors);

/* Index of the tensor named `name` (QuantFile::find, quantize.rs:247-249). */
int qasr_qint8_find(const qasr_qint8_file* f, const char* name, size_t* index);

/* Table entry of tensor `index`: name (not NUL-terminated; valid until close),
 * dtype, shape (shape_cap entries available), offsets into the data section.
 * Any output pointer may be NULL. */
int qasr_qint8_tensor(const qasr_qint8_file* f, size_t index, const char** name,
                      size_t* name_len, int* dtype, size_t* n_dims, uint64_t* shape,
                      size_t shape_cap, uint64_t* data_offset, uint64_t* scale_offset);

/* Copies tensor `index` to device memory: its data (numel bytes for INT8,
 * 4*numel for F32, 2*numel for BF16) to dev_data and, for INT8, its shape[0]
 * row scales to dev_scales (the mapping of QuantFile::get_quant_weight,
 * quantize.rs:252-268). Fails if the tensor extends past the file. Load-time
 * call: the copy is from pageable memory and may not be asynchronous. */
int qasr_qint8_upload(const qasr_qint8_file* f, size_t index, void* dev_data,
                      float* dev_scales, void* stream);

/* Uploads INT8 gate [inter, hidden] and up [inter, hidden] as the fused
 * row-interleaved matrix dev_w [2*inter, hidden] (g0, u0, g1, u1, ...) with
 * interleaved scales dev_scales [2*inter], directly by strided copies: the
 * fusion DecoderInt8::load does on the host (decoder.rs:697-719), which takes
 * inter and hidden from the model config. Both tensors must be INT8 and
 * exactly [inter, hidden]; the reference does not check this. */
int qasr_qint8_upload_gate_up(const qasr_qint8_file* f, const char* gate_name,
                              const char* up_name, size_t inter, size_t hidden,
                              int8_t* dev_w, float* dev_scales, void* stream);

/* ------------------------------------------------------------------------ */
/* Measurement aid                                                           */
/* ------------------------------------------------------------------------ */

/* No counterpart in the reference: a read-only probe of how fast one CU pulls
 * bytes in (bench.py --probe). `grid` workgroups of 512 threads each read
 * bytes_per_wg bytes of buf with 16-byte loads, `depth` (4, 8 or 16) in flight
 * per thread, and write one int per thread to out (grid * 512 ints). mode 0:
 * one region per XCD read by all its workgroups in the same order; 1: as 0 from
 * a per-workgroup rotation; 2: a private priv_bytes region per workgroup read
 * repeatedly (L2-resident); 3: a private region read once at offset
 * shift * grid * bytes_per_wg (HBM stream); 4 / 5: as 2 / 3 with waves w and
 * w + 4 reading the same addresses. bytes_per_wg must be a multiple of
 * 8192 * depth; every region is checked against buf_bytes on the host. */
int qasr_probe_read(int mode, int depth, unsigned grid, const void* buf, size_t buf_bytes, int* out,
                    size_t out_ints, size_t bytes_per_wg, size_t priv_bytes, size_t shift, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* QASR_H */
