// qwen_asr/kernels.hpp -- C++ host mirror of the Rust `qwen_asr::kernels`
// module (crates/qwen-asr/src/kernels/mod.rs) over device memory, built on the
// C-ABI in qasr.h.
//
// Every function keeps the reference's name and argument order; Rust slices
// become DevSlice<T> views of device memory (pointer + element count). Where
// the reference would panic on a slice that is too short, these throw Panic
// before anything is launched; a non-zero qasr_status throws QasrError.
// Calls enqueue on the thread's current stream (set_stream) and never
// synchronise.
//
// Header-only; link libqasr_hip.so or libqasr_hip.a plus amdhip64.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "../qasr.h"

namespace qwen_asr {
namespace kernels {

// The reference's panics (slice index out of range, dimension mismatch).
struct Panic : std::out_of_range {
  using std::out_of_range::out_of_range;
};

// A C-ABI call returned a non-zero status.
struct QasrError : std::runtime_error {
  int code;
  QasrError(const std::string& fn, int c)
      : std::runtime_error(fn + " failed (" + std::to_string(c) + "): " + qasr_last_error()),
        code(c) {}
};

// Non-owning view of `len` elements of device memory.
template <class T>
struct DevSlice {
  T* ptr = nullptr;
  size_t len = 0;

  DevSlice() = default;
  DevSlice(T* p, size_t n) : ptr(p), len(n) {}
  template <class U>
  DevSlice(const DevSlice<U>& o) : ptr(o.ptr), len(o.len) {}  // T* <- U* (adds const)

  // &s[start..start+n], panicking like a Rust range index.
  DevSlice sub(size_t start, size_t n) const {
    if (start > len || n > len - start) {
      throw Panic("range end index " + std::to_string(start + n) +
                  " out of range for slice of length " + std::to_string(len));
    }
    return DevSlice(ptr + start, n);
  }
};

// Owning device buffer (hipMalloc/hipFree), used by RopeCache and tests.
template <class T>
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t n) : n_(n) {
    if (n && hipMalloc(reinterpret_cast<void**>(&p_), n * sizeof(T)) != hipSuccess) {
      throw std::bad_alloc();
    }
  }
  ~DeviceBuffer() { reset(); }
  DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      reset();
      p_ = o.p_;
      n_ = o.n_;
      o.p_ = nullptr;
      o.n_ = 0;
    }
    return *this;
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;

  T* data() const { return p_; }
  size_t size() const { return n_; }
  DevSlice<T> slice() const { return DevSlice<T>(p_, n_); }
  operator DevSlice<T>() const { return slice(); }
  operator DevSlice<const T>() const { return DevSlice<const T>(p_, n_); }

 private:
  void reset() {
    if (p_) (void)hipFree(p_);
    p_ = nullptr;
    n_ = 0;
  }
  T* p_ = nullptr;
  size_t n_ = 0;
};

namespace detail {
inline hipStream_t& stream_ref() {
  thread_local hipStream_t s = nullptr;
  return s;
}
template <class T>
void need(const DevSlice<T>& s, size_t n, const char* name) {
  if (s.len < n) {
    throw Panic(std::string(name) + ": range end index " + std::to_string(n) +
                " out of range for slice of length " + std::to_string(s.len));
  }
}
inline void check(int rc, const char* fn) {
  if (rc != QASR_OK) throw QasrError(fn, rc);
}
inline void* st() { return reinterpret_cast<void*>(stream_ref()); }
}  // namespace detail

inline void set_stream(hipStream_t s) { detail::stream_ref() = s; }
inline hipStream_t current_stream() { return detail::stream_ref(); }

using F = DevSlice<float>;
using CF = DevSlice<const float>;

// ---- basic / normalisation (kernels/mod.rs:486-488, 866-935) -----------------
inline void add_inplace(F a, CF b, size_t n) {
  detail::need(a, n, "a");
  detail::need(b, n, "b");
  detail::check(qasr_add_inplace_f32(a.ptr, b.ptr, n, detail::st()), "add_inplace");
}

inline void rms_norm(F out, CF x, CF weight, size_t seq_len, size_t hidden, float eps) {
  detail::need(out, seq_len * hidden, "out");
  detail::need(x, seq_len * hidden, "x");
  detail::need(weight, hidden, "weight");
  detail::check(qasr_rms_norm_f32(out.ptr, x.ptr, weight.ptr, seq_len, hidden, eps, detail::st()),
                "rms_norm");
}

// add_inplace(x, delta) followed by rms_norm(out, x) in one pass.
inline void add_rms_norm(F x, CF delta, CF weight, F out, size_t seq_len, size_t hidden, float eps) {
  detail::need(x, seq_len * hidden, "x");
  detail::need(delta, seq_len * hidden, "delta");
  detail::need(weight, hidden, "weight");
  detail::need(out, seq_len * hidden, "out");
  detail::check(qasr_add_rms_norm_f32(x.ptr, delta.ptr, weight.ptr, out.ptr, seq_len, hidden, eps,
                                      detail::st()),
                "add_rms_norm");
}

inline void layer_norm(F out, CF x, CF weight, CF bias, size_t seq_len, size_t hidden, float eps) {
  detail::need(out, seq_len * hidden, "out");
  detail::need(x, seq_len * hidden, "x");
  detail::need(weight, hidden, "weight");
  detail::need(bias, hidden, "bias");
  detail::check(qasr_layer_norm_f32(out.ptr, x.ptr, weight.ptr, bias.ptr, seq_len, hidden, eps,
                                    detail::st()),
                "layer_norm");
}

inline void rms_norm_per_head(F x, CF weight, size_t seq_len, size_t n_heads, size_t head_dim,
                              float eps) {
  detail::need(x, seq_len * n_heads * head_dim, "x");
  detail::need(weight, head_dim, "weight");
  detail::check(qasr_rms_norm_per_head_f32(x.ptr, weight.ptr, seq_len, n_heads, head_dim, eps,
                                           detail::st()),
                "rms_norm_per_head");
}

// ---- RoPE (kernels/mod.rs:1247-1267, decoder.rs:234-306) --------------------------
inline void apply_rope_neox(F x, CF cos_vals, CF sin_vals, size_t seq, size_t n_heads,
                            size_t head_dim) {
  detail::need(x, seq * n_heads * head_dim, "x");
  detail::need(cos_vals, seq * head_dim, "cos_vals");
  detail::need(sin_vals, seq * head_dim, "sin_vals");
  detail::check(qasr_apply_rope_neox_f32(x.ptr, cos_vals.ptr, sin_vals.ptr, seq, n_heads, head_dim,
                                         detail::st()),
                "apply_rope_neox");
}

// Device RoPE table with the reference's growth rule: capacity doubles from
// 1024; new rows are filled on the device. A change of head_dim or theta
// rebuilds the table from row 0.
class RopeCache {
 public:
  void ensure(size_t required_pos, size_t head_dim, float theta) {
    if (head_dim != head_dim_ || theta != theta_) {
      cos_ = DeviceBuffer<float>();
      sin_ = DeviceBuffer<float>();
      cap_ = 0;
      head_dim_ = head_dim;
      theta_ = theta;
    }
    if (required_pos <= cap_) return;
    size_t new_cap = cap_ ? cap_ : 1024;
    while (new_cap < required_pos) new_cap *= 2;
    DeviceBuffer<float> c(new_cap * head_dim), s(new_cap * head_dim);
    if (cap_) {
      const size_t bytes = cap_ * head_dim * sizeof(float);
      if (hipMemcpyAsync(c.data(), cos_.data(), bytes, hipMemcpyDeviceToDevice, current_stream()) != hipSuccess ||
          hipMemcpyAsync(s.data(), sin_.data(), bytes, hipMemcpyDeviceToDevice, current_stream()) != hipSuccess) {
        throw std::runtime_error("RopeCache::ensure: device copy failed");
      }
    }
    detail::check(qasr_rope_table_fill_f32(c.data(), s.data(), cap_, new_cap, head_dim, theta,
                                           detail::st()),
                  "rope_table_fill");
    cos_ = std::move(c);
    sin_ = std::move(s);
    cap_ = new_cap;
  }
  size_t cap() const { return cap_; }
  size_t head_dim() const { return head_dim_; }
  CF cos() const { return cos_; }
  CF sin() const { return sin_; }
  CF cos_at(size_t pos) const { return cos().sub(pos * head_dim_, head_dim_); }
  CF sin_at(size_t pos) const { return sin().sub(pos * head_dim_, head_dim_); }
  CF cos_range(size_t start, size_t len) const { return cos().sub(start * head_dim_, len * head_dim_); }
  CF sin_range(size_t start, size_t len) const { return sin().sub(start * head_dim_, len * head_dim_); }

 private:
  DeviceBuffer<float> cos_, sin_;
  size_t cap_ = 0, head_dim_ = 0;
  float theta_ = 0.0f;
};

// q/k head RMSNorm + RoPE at per-row positions (positions.len == 0: row s at s).
inline void head_rms_norm_rope(F q, F k, CF q_norm_w, CF k_norm_w, const RopeCache& rope,
                               DevSlice<const int32_t> positions, size_t seq, size_t n_heads,
                               size_t n_kv_heads, size_t head_dim, float eps) {
  detail::need(q, seq * n_heads * head_dim, "q");
  detail::need(k, seq * n_kv_heads * head_dim, "k");
  detail::need(q_norm_w, head_dim, "q_norm_w");
  detail::need(k_norm_w, head_dim, "k_norm_w");
  if (positions.ptr) detail::need(positions, seq, "positions");
  if (rope.head_dim() != head_dim) throw Panic("head_rms_norm_rope: RopeCache head_dim mismatch");
  detail::check(qasr_head_rms_norm_rope_f32(q.ptr, k.ptr, q_norm_w.ptr, k_norm_w.ptr,
                                            rope.cos().ptr, rope.sin().ptr, positions.ptr, seq,
                                            n_heads, n_kv_heads, head_dim, rope.cap(), eps,
                                            detail::st()),
                "head_rms_norm_rope");
}

// Device KV cache with the reference's layout [n_layers][max_seq][kv_dim] and
// growth rule (decoder.rs:129-228): grow() doubles max_seq until it covers the
// request and keeps the first len rows of every layer.
class KvCache {
 public:
  KvCache(size_t n_layers, size_t max_seq, size_t kv_dim)
      : n_layers_(n_layers), max_seq_(max_seq), kv_dim_(kv_dim),
        k_(n_layers * max_seq * kv_dim), v_(n_layers * max_seq * kv_dim) {
    zero(k_);
    zero(v_);
  }
  size_t len = 0;
  size_t max_seq() const { return max_seq_; }
  size_t kv_dim() const { return kv_dim_; }
  void grow(size_t required) {
    if (required <= max_seq_) return;
    size_t new_max = max_seq_;
    while (new_max < required) new_max *= 2;
    DeviceBuffer<float> k(n_layers_ * new_max * kv_dim_), v(n_layers_ * new_max * kv_dim_);
    zero(k);
    zero(v);
    const size_t bytes = len * kv_dim_ * sizeof(float);
    for (size_t l = 0; l < n_layers_ && bytes; ++l) {
      const size_t src = l * max_seq_ * kv_dim_, dst = l * new_max * kv_dim_;
      if (hipMemcpyAsync(k.data() + dst, k_.data() + src, bytes, hipMemcpyDeviceToDevice, current_stream()) != hipSuccess ||
          hipMemcpyAsync(v.data() + dst, v_.data() + src, bytes, hipMemcpyDeviceToDevice, current_stream()) != hipSuccess) {
        throw std::runtime_error("KvCache::grow: device copy failed");
      }
    }
    k_ = std::move(k);
    v_ = std::move(v);
    max_seq_ = new_max;
  }
  // The layer's whole [max_seq][kv_dim] block (the store target) and its
  // first len rows (what attention reads: k_layer / v_layer).
  F k_block(size_t layer) const { return F(k_.data(), k_.size()).sub(layer * max_seq_ * kv_dim_, max_seq_ * kv_dim_); }
  F v_block(size_t layer) const { return F(v_.data(), v_.size()).sub(layer * max_seq_ * kv_dim_, max_seq_ * kv_dim_); }
  F k_layer(size_t layer) const { return k_block(layer).sub(0, len * kv_dim_); }
  F v_layer(size_t layer) const { return v_block(layer).sub(0, len * kv_dim_); }

 private:
  static void zero(DeviceBuffer<float>& b) {
    if (b.size() && hipMemsetAsync(b.data(), 0, b.size() * sizeof(float), current_stream()) != hipSuccess)
      throw std::runtime_error("KvCache: device memset failed");
  }
  size_t n_layers_, max_seq_, kv_dim_;
  DeviceBuffer<float> k_, v_;
};

// q/k head RMSNorm + RoPE with the KV store fused in: rows start_pos.. of one
// sequence go to the layer blocks k_cache/v_cache (k and v are read only).
inline void head_rms_norm_rope_kv(F q, CF k, CF v, CF q_norm_w, CF k_norm_w, const RopeCache& rope,
                                  size_t start_pos, size_t seq, size_t n_heads, size_t n_kv_heads,
                                  size_t head_dim, float eps, F k_cache, F v_cache, size_t cache_rows) {
  const size_t kv_dim = n_kv_heads * head_dim;
  detail::need(q, seq * n_heads * head_dim, "q");
  detail::need(k, seq * kv_dim, "k");
  detail::need(v, seq * kv_dim, "v");
  detail::need(q_norm_w, head_dim, "q_norm_w");
  detail::need(k_norm_w, head_dim, "k_norm_w");
  detail::need(k_cache, cache_rows * kv_dim, "k_cache");
  detail::need(v_cache, cache_rows * kv_dim, "v_cache");
  if (rope.head_dim() != head_dim) throw Panic("head_rms_norm_rope_kv: RopeCache head_dim mismatch");
  detail::check(qasr_head_rms_norm_rope_kv_f32(q.ptr, k.ptr, v.ptr, q_norm_w.ptr, k_norm_w.ptr,
                                               rope.cos().ptr, rope.sin().ptr, nullptr, start_pos,
                                               seq, n_heads, n_kv_heads, head_dim, rope.cap(), eps,
                                               k_cache.ptr, v_cache.ptr, cache_rows, detail::st()),
                "head_rms_norm_rope_kv");
}

// ---- activations (kernels/mod.rs:941-994) ------------------------------------
inline void silu(F x, size_t n) {
  detail::need(x, n, "x");
  detail::check(qasr_silu_f32(x.ptr, n, detail::st()), "silu");
}

inline void gelu(F x, size_t n) {  // tanh form, as the reference CPU path
  detail::need(x, n, "x");
  detail::check(qasr_gelu_tanh_f32(x.ptr, n, detail::st()), "gelu");
}

inline void gelu_erf(F x, size_t n) {  // exact erf form
  detail::need(x, n, "x");
  detail::check(qasr_gelu_erf_f32(x.ptr, n, detail::st()), "gelu_erf");
}

inline void swiglu_multiply(F out, CF gate_up, size_t seq_len, size_t intermediate) {
  detail::need(out, seq_len * intermediate, "out");
  detail::need(gate_up, seq_len * 2 * intermediate, "gate_up");
  detail::check(qasr_swiglu_multiply_f32(out.ptr, gate_up.ptr, seq_len, intermediate, detail::st()),
                "swiglu_multiply");
}

inline void swiglu_multiply_inplace(F gate, CF up) {
  detail::need(up, gate.len, "up");
  detail::check(qasr_swiglu_split_f32(gate.ptr, gate.ptr, up.ptr, gate.len, detail::st()),
                "swiglu_multiply_inplace");
}

// residual add + the LayerNorm that reads its rows (encoder.rs:386 + 389-390, 397 + 370-371)
inline void add_layer_norm(F x, CF delta, CF weight, CF bias, F out, size_t seq_len, size_t hidden,
                           float eps) {
  detail::need(x, seq_len * hidden, "x");
  detail::need(delta, seq_len * hidden, "delta");
  detail::need(weight, hidden, "weight");
  detail::need(bias, hidden, "bias");
  detail::need(out, seq_len * hidden, "out");
  detail::check(qasr_add_layer_norm_f32(x.ptr, delta.ptr, weight.ptr, bias.ptr, out.ptr, seq_len,
                                        hidden, eps, detail::st()),
                "add_layer_norm");
}

// ---- position embeddings (kernels/mod.rs:1213-1226) -------------------------------
inline void sinusoidal_pe(F pe, size_t n_pos, size_t d_model) {
  detail::need(pe, n_pos * d_model, "pe");
  detail::check(qasr_sinusoidal_pe_f32(pe.ptr, n_pos, d_model, detail::st()), "sinusoidal_pe");
}

// x[r] += pe[r mod n_pos] (the per-chunk add of encoder.rs:341-343 over all rows)
inline void pe_add(F x, CF pe, size_t rows, size_t d_model, size_t n_pos) {
  detail::need(x, rows * d_model, "x");
  detail::need(pe, n_pos * d_model, "pe");
  detail::check(qasr_pe_add_f32(x.ptr, pe.ptr, rows, d_model, n_pos, detail::st()), "pe_add");
}

// pe_add + layer 0's LayerNorm of the same rows (encoder.rs:341-343, 370-371) in one pass
inline void pe_add_layer_norm(F x, CF pe, F out, CF weight, CF bias, size_t rows, size_t d_model,
                              size_t n_pos, float eps) {
  detail::need(x, rows * d_model, "x");
  detail::need(pe, n_pos * d_model, "pe");
  detail::need(out, rows * d_model, "out");
  detail::need(weight, d_model, "weight");
  detail::need(bias, d_model, "bias");
  detail::check(qasr_pe_add_layer_norm_f32(x.ptr, pe.ptr, out.ptr, weight.ptr, bias.ptr, rows, d_model,
                                           n_pos, eps, detail::st()),
                "pe_add_layer_norm");
}

// ---- token embeddings (decoder.rs:631-646) ------------------------------------------
inline void tok_embed_bf16_to_f32(F dst, DevSlice<const uint16_t> tok_emb_bf16,
                                  DevSlice<const int32_t> token_id_on_device, size_t dim) {
  detail::need(dst, dim, "dst");
  detail::need(token_id_on_device, 1, "token_id");
  detail::check(qasr_embed_gather_bf16(dst.ptr, tok_emb_bf16.ptr, token_id_on_device.ptr, 1, dim,
                                       tok_emb_bf16.len / dim, detail::st()),
                "tok_embed_bf16_to_f32");
}

// ---- INT8 (kernels/mod.rs:650-673, quantize.rs:633-662) --------------------------------
inline void linear_nobias_int8(F y, CF x, DevSlice<const int8_t> w_int8, CF scales, size_t seq_len,
                               size_t in_dim, size_t out_dim) {
  detail::need(y, seq_len * out_dim, "y");
  detail::need(x, seq_len * in_dim, "x");
  detail::need(w_int8, out_dim * in_dim, "w_int8");
  detail::need(scales, out_dim, "scales");
  detail::check(qasr_linear_nobias_int8_f32(y.ptr, x.ptr, w_int8.ptr, scales.ptr, seq_len, in_dim,
                                            out_dim, detail::st()),
                "linear_nobias_int8");
}

// Several projections of the same x in one launch (decoder.rs:881-886's q/k/v):
// ys[m] = linear_nobias_int8(x, ws[m], scales[m]) with out_dims[m] rows.
inline void linear_nobias_int8_multi(const std::vector<F>& ys,
                                     const std::vector<DevSlice<const int8_t>>& ws,
                                     const std::vector<CF>& scales,
                                     const std::vector<size_t>& out_dims, CF x, size_t seq_len,
                                     size_t in_dim) {
  const size_t n = out_dims.size();
  if (ys.size() != n || ws.size() != n || scales.size() != n)
    throw Panic("linear_nobias_int8_multi: one output, weight and scale slice per matrix");
  std::vector<float*> yp(n);
  std::vector<const int8_t*> wp(n);
  std::vector<const float*> sp(n);
  for (size_t m = 0; m < n; ++m) {
    detail::need(ys[m], seq_len * out_dims[m], "y");
    detail::need(ws[m], out_dims[m] * in_dim, "w_int8");
    detail::need(scales[m], out_dims[m], "scales");
    yp[m] = ys[m].ptr;
    wp[m] = ws[m].ptr;
    sp[m] = scales[m].ptr;
  }
  detail::need(x, seq_len * in_dim, "x");
  detail::check(qasr_linear_nobias_int8_multi_f32(n, yp.data(), wp.data(), sp.data(),
                                                  out_dims.data(), x.ptr, seq_len, in_dim,
                                                  detail::st()),
                "linear_nobias_int8_multi");
}

inline void linear_int8(F y, CF x, DevSlice<const int8_t> w_int8, CF scales, CF bias,
                        size_t seq_len, size_t in_dim, size_t out_dim) {
  detail::need(y, seq_len * out_dim, "y");
  detail::need(x, seq_len * in_dim, "x");
  detail::need(w_int8, out_dim * in_dim, "w_int8");
  detail::need(scales, out_dim, "scales");
  if (bias.ptr) detail::need(bias, out_dim, "bias");
  detail::check(qasr_linear_int8_f32(y.ptr, x.ptr, w_int8.ptr, scales.ptr, bias.ptr, seq_len,
                                     in_dim, out_dim, detail::st()),
                "linear_int8");
}

inline void quantize_f32_to_int8(DevSlice<int8_t> q, F scales, CF f32_data, size_t out_dim,
                                 size_t in_dim) {
  detail::need(q, out_dim * in_dim, "q");
  detail::need(scales, out_dim, "scales");
  detail::need(f32_data, out_dim * in_dim, "f32_data");
  detail::check(qasr_quantize_rows_i8(q.ptr, scales.ptr, f32_data.ptr, out_dim, in_dim,
                                      detail::st()),
                "quantize_f32_to_int8");
}

inline void gate_up_swiglu_w8a8(F out, DevSlice<const int8_t> w_gate_up, CF scales,
                                DevSlice<const int8_t> xq, CF x_scales, size_t batch,
                                size_t in_dim, size_t intermediate) {
  detail::need(out, batch * intermediate, "out");
  detail::need(w_gate_up, 2 * intermediate * in_dim, "w_gate_up");
  detail::need(scales, 2 * intermediate, "scales");
  detail::need(xq, batch * in_dim, "xq");
  detail::need(x_scales, batch, "x_scales");
  detail::check(qasr_gate_up_swiglu_w8a8(out.ptr, w_gate_up.ptr, scales.ptr, xq.ptr, x_scales.ptr,
                                         batch, in_dim, intermediate, detail::st()),
                "gate_up_swiglu_w8a8");
}

// The decode loop's gate/up projection + SwiGLU (decoder.rs:912-921): out = silu(g) * u on the
// row-interleaved fused weight, gate/up values never stored.
inline void gate_up_swiglu_int8(F out, CF x, DevSlice<const int8_t> w_gate_up, CF scales,
                                size_t seq_len, size_t in_dim, size_t intermediate) {
  detail::need(out, seq_len * intermediate, "out");
  detail::need(x, seq_len * in_dim, "x");
  detail::need(w_gate_up, 2 * intermediate * in_dim, "w_gate_up");
  detail::need(scales, 2 * intermediate, "scales");
  detail::check(qasr_gate_up_swiglu_int8_f32(out.ptr, x.ptr, w_gate_up.ptr, scales.ptr, seq_len,
                                             in_dim, intermediate, detail::st()),
                "gate_up_swiglu_int8");
}

// The prefill's gate/up projection + swiglu_multiply (decoder.rs:831-834, the fast_exp SwiGLU).
inline void gate_up_swiglu_multiply_int8(F out, CF x, DevSlice<const int8_t> w_gate_up, CF scales,
                                         size_t seq_len, size_t in_dim, size_t intermediate) {
  detail::need(out, seq_len * intermediate, "out");
  detail::need(x, seq_len * in_dim, "x");
  detail::need(w_gate_up, 2 * intermediate * in_dim, "w_gate_up");
  detail::need(scales, 2 * intermediate, "scales");
  detail::check(qasr_gate_up_swiglu_multiply_int8_f32(out.ptr, x.ptr, w_gate_up.ptr, scales.ptr,
                                                      seq_len, in_dim, intermediate, detail::st()),
                "gate_up_swiglu_multiply_int8");
}

// Prefill q/k/v with the head norms, RoPE and K/V cache rows in one launch (decoder.rs:795-810):
// bit-identical to linear_nobias_int8_multi (q, k, v) + head_rms_norm_rope_kv without positions.
// k_cache/v_cache are the layer's [cache_rows][n_kv_heads*head_dim] blocks.
inline void qkv_heads_int8(F q, F k_cache, F v_cache, size_t cache_rows, DevSlice<const int8_t> wq, CF sq,
                           DevSlice<const int8_t> wk, CF sk, DevSlice<const int8_t> wv, CF sv, CF x,
                           size_t seq_len, size_t in_dim, size_t n_heads, size_t n_kv_heads,
                           size_t head_dim, CF q_norm_w, CF k_norm_w, const RopeCache& rope,
                           size_t start_pos, float eps) {
  const size_t qd = n_heads * head_dim, kv = n_kv_heads * head_dim;
  detail::need(q, seq_len * qd, "q");
  detail::need(k_cache, cache_rows * kv, "k_cache");
  detail::need(v_cache, cache_rows * kv, "v_cache");
  detail::need(wq, qd * in_dim, "wq");
  detail::need(sq, qd, "sq");
  detail::need(wk, kv * in_dim, "wk");
  detail::need(sk, kv, "sk");
  detail::need(wv, kv * in_dim, "wv");
  detail::need(sv, kv, "sv");
  detail::need(x, seq_len * in_dim, "x");
  detail::need(q_norm_w, head_dim, "q_norm_w");
  detail::need(k_norm_w, head_dim, "k_norm_w");
  if (rope.head_dim() != head_dim) throw Panic("qkv_heads_int8: RopeCache head_dim mismatch");
  detail::check(qasr_qkv_heads_int8_f32(q.ptr, k_cache.ptr, v_cache.ptr, cache_rows, wq.ptr, sq.ptr, wk.ptr,
                                        sk.ptr, wv.ptr, sv.ptr, x.ptr, seq_len, in_dim, n_heads, n_kv_heads,
                                        head_dim, q_norm_w.ptr, k_norm_w.ptr, rope.cos().ptr, rope.sin().ptr,
                                        rope.cap(), start_pos, eps, detail::st()),
                "qkv_heads_int8");
}

// Prefill folds: the residual add in the o / down GEMM (h += x W^T, plus each token's sums of
// squares over 64-column slices of the updated h in ss and, with hg/gain, hg = h * gain), and the
// next RMSNorm in the q/k/v or gate/up GEMM, which reads hg and multiplies each token's outputs by
// its 1 / rms from ss (x_norm receives hg * rinv only on shapes the folded kernels do not take).
inline size_t norm_slices(size_t hidden) { return (hidden + 63) / 64; }

inline void linear_int8_residual(F h, F ss, F hg, CF gain, CF x, DevSlice<const int8_t> w, CF scales,
                                 size_t seq_len, size_t in_dim, size_t out_dim) {
  detail::need(h, seq_len * out_dim, "h");
  detail::need(ss, seq_len * norm_slices(out_dim), "ss");
  if (hg.ptr || gain.ptr) {
    detail::need(hg, seq_len * out_dim, "hg");
    detail::need(gain, out_dim, "gain");
  }
  detail::need(x, seq_len * in_dim, "x");
  detail::need(w, out_dim * in_dim, "w");
  detail::need(scales, out_dim, "scales");
  detail::check(qasr_linear_int8_residual_f32(h.ptr, ss.ptr, hg.ptr, gain.ptr, x.ptr, w.ptr, scales.ptr, seq_len,
                                              in_dim, out_dim, detail::st()),
                "linear_int8_residual");
}

inline void rms_norm_gate_up_swiglu_multiply_int8(F out, CF hg, CF ss, float eps, F x_norm,
                                                  DevSlice<const int8_t> w_gate_up, CF scales_gate_up,
                                                  size_t seq_len, size_t in_dim, size_t intermediate) {
  detail::need(out, seq_len * intermediate, "out");
  detail::need(hg, seq_len * in_dim, "hg");
  detail::need(ss, seq_len * norm_slices(in_dim), "ss");
  detail::need(x_norm, seq_len * in_dim, "x_norm");
  detail::need(w_gate_up, 2 * intermediate * in_dim, "w_gate_up");
  detail::need(scales_gate_up, 2 * intermediate, "scales_gate_up");
  detail::check(qasr_rms_norm_gate_up_swiglu_multiply_int8_f32(out.ptr, hg.ptr, ss.ptr, norm_slices(in_dim), eps,
                                                               x_norm.ptr, w_gate_up.ptr, scales_gate_up.ptr,
                                                               seq_len, in_dim, intermediate, detail::st()),
                "rms_norm_gate_up_swiglu_multiply_int8");
}

inline void rms_norm_qkv_heads_int8(F q, F k_cache, F v_cache, size_t cache_rows, DevSlice<const int8_t> wq,
                                    CF sq, DevSlice<const int8_t> wk, CF sk, DevSlice<const int8_t> wv, CF sv,
                                    CF hg, CF ss, float norm_eps, F x_norm, size_t seq_len, size_t in_dim,
                                    size_t n_heads, size_t n_kv_heads, size_t head_dim, CF q_norm_w,
                                    CF k_norm_w, const RopeCache& rope, size_t start_pos, float eps) {
  const size_t qd = n_heads * head_dim, kv = n_kv_heads * head_dim;
  detail::need(q, seq_len * qd, "q");
  detail::need(k_cache, cache_rows * kv, "k_cache");
  detail::need(v_cache, cache_rows * kv, "v_cache");
  detail::need(wq, qd * in_dim, "wq");
  detail::need(sq, qd, "sq");
  detail::need(wk, kv * in_dim, "wk");
  detail::need(sk, kv, "sk");
  detail::need(wv, kv * in_dim, "wv");
  detail::need(sv, kv, "sv");
  detail::need(hg, seq_len * in_dim, "hg");
  detail::need(ss, seq_len * norm_slices(in_dim), "ss");
  detail::need(x_norm, seq_len * in_dim, "x_norm");
  detail::need(q_norm_w, head_dim, "q_norm_w");
  detail::need(k_norm_w, head_dim, "k_norm_w");
  if (rope.head_dim() != head_dim) throw Panic("rms_norm_qkv_heads_int8: RopeCache head_dim mismatch");
  detail::check(qasr_rms_norm_qkv_heads_int8_f32(
                    q.ptr, k_cache.ptr, v_cache.ptr, cache_rows, wq.ptr, sq.ptr, wk.ptr, sk.ptr, wv.ptr, sv.ptr,
                    hg.ptr, ss.ptr, norm_slices(in_dim), norm_eps, x_norm.ptr, seq_len, in_dim, n_heads,
                    n_kv_heads, head_dim, q_norm_w.ptr, k_norm_w.ptr, rope.cos().ptr, rope.sin().ptr, rope.cap(),
                    start_pos, eps, detail::st()),
                "rms_norm_qkv_heads_int8");
}

// Decode folds (one token): h = x + delta (delta empty: h = x), the RMSNorm of h and the
// projections of the normalised row in one launch, equal bit for bit to add_rms_norm followed by
// the projection; h goes to h_out (empty: not written), which must not overlap x or delta.
inline void add_rms_norm_linear_nobias_int8_multi(const std::vector<F>& ys,
                                                  const std::vector<DevSlice<const int8_t>>& ws,
                                                  const std::vector<CF>& scales,
                                                  const std::vector<size_t>& out_dims, F h_out, CF x,
                                                  CF delta, CF norm_w, size_t in_dim, float eps) {
  const size_t n = out_dims.size();
  if (ys.size() != n || ws.size() != n || scales.size() != n)
    throw Panic("add_rms_norm_linear_nobias_int8_multi: one output, weight and scale slice per matrix");
  std::vector<float*> yp(n);
  std::vector<const int8_t*> wp(n);
  std::vector<const float*> sp(n);
  for (size_t m = 0; m < n; ++m) {
    detail::need(ys[m], out_dims[m], "y");
    detail::need(ws[m], out_dims[m] * in_dim, "w_int8");
    detail::need(scales[m], out_dims[m], "scales");
    yp[m] = ys[m].ptr;
    wp[m] = ws[m].ptr;
    sp[m] = scales[m].ptr;
  }
  detail::need(x, in_dim, "x");
  detail::need(norm_w, in_dim, "norm_w");
  if (delta.ptr) detail::need(delta, in_dim, "delta");
  if (h_out.ptr) detail::need(h_out, in_dim, "h_out");
  detail::check(qasr_add_rms_norm_linear_nobias_int8_multi_f32(n, yp.data(), wp.data(), sp.data(),
                                                               out_dims.data(), h_out.ptr, x.ptr,
                                                               delta.ptr, norm_w.ptr, in_dim, eps,
                                                               detail::st()),
                "add_rms_norm_linear_nobias_int8_multi");
}

inline void add_rms_norm_gate_up_swiglu_int8(F out, F h_out, CF x, CF delta, CF norm_w,
                                             DevSlice<const int8_t> w_gate_up, CF scales,
                                             size_t in_dim, size_t intermediate, float eps) {
  detail::need(out, intermediate, "out");
  detail::need(x, in_dim, "x");
  detail::need(norm_w, in_dim, "norm_w");
  if (delta.ptr) detail::need(delta, in_dim, "delta");
  if (h_out.ptr) detail::need(h_out, in_dim, "h_out");
  detail::need(w_gate_up, 2 * intermediate * in_dim, "w_gate_up");
  detail::need(scales, 2 * intermediate, "scales");
  detail::check(qasr_add_rms_norm_gate_up_swiglu_int8_f32(out.ptr, h_out.ptr, x.ptr, delta.ptr,
                                                          norm_w.ptr, w_gate_up.ptr, scales.ptr,
                                                          in_dim, intermediate, eps, detail::st()),
                "add_rms_norm_gate_up_swiglu_int8");
}

// ---- attention (kernels/mod.rs:1124-1207) ---------------------------------------------
inline size_t attention_workspace_floats(size_t seq_q, size_t n_heads, size_t head_dim) {
  return qasr_causal_attention_workspace_floats(seq_q, n_heads, head_dim);
}

// kernels::causal_attention: q [seq_q, n_heads*hd], k/v [seq_k, n_kv_heads*hd] (a KvCache
// layer block), out [seq_q, n_heads*hd]; query i sees keys 0..=q_offset+i.
inline void causal_attention(F out, CF q, CF k, CF v, size_t seq_q, size_t seq_k, size_t n_heads,
                             size_t n_kv_heads, size_t head_dim, float scale, size_t q_offset) {
  detail::need(out, seq_q * n_heads * head_dim, "out");
  detail::need(q, seq_q * n_heads * head_dim, "q");
  detail::need(k, seq_k * n_kv_heads * head_dim, "k");
  detail::need(v, seq_k * n_kv_heads * head_dim, "v");
  detail::check(qasr_causal_attention_f32(out.ptr, q.ptr, k.ptr, v.ptr, seq_q, seq_k, n_heads,
                                          n_kv_heads, head_dim, scale, q_offset, detail::st()),
                "causal_attention");
}

// Same result with the keys split over workgroups (decode); workspace of
// attention_workspace_floats(seq_q, n_heads, head_dim) floats, reused across calls.
inline void causal_attention(F out, CF q, CF k, CF v, size_t seq_q, size_t seq_k, size_t n_heads,
                             size_t n_kv_heads, size_t head_dim, float scale, size_t q_offset,
                             F workspace) {
  detail::need(out, seq_q * n_heads * head_dim, "out");
  detail::need(q, seq_q * n_heads * head_dim, "q");
  detail::need(k, seq_k * n_kv_heads * head_dim, "k");
  detail::need(v, seq_k * n_kv_heads * head_dim, "v");
  detail::check(qasr_causal_attention_split_f32(out.ptr, q.ptr, k.ptr, v.ptr, seq_q, seq_k, n_heads,
                                                n_kv_heads, head_dim, scale, q_offset,
                                                workspace.ptr, workspace.len, detail::st()),
                "causal_attention");
}

// One decode token: q/k head RMSNorm + RoPE at pos, the K/V rows into the layer's cache block
// and causal attention over rows 0..pos (decoder.rs:888-903), equal bit for bit to
// head_rms_norm_rope_kv + causal_attention with a workspace; q is scratch.
inline void decode_attention(F out, F q, CF k, CF v, CF q_norm_w, CF k_norm_w, const RopeCache& rope,
                             size_t pos, size_t n_heads, size_t n_kv_heads, size_t head_dim, float eps,
                             float scale, F k_cache, F v_cache, size_t cache_rows, F workspace) {
  const size_t kv_dim = n_kv_heads * head_dim;
  detail::need(out, n_heads * head_dim, "out");
  detail::need(q, n_heads * head_dim, "q");
  detail::need(k, kv_dim, "k");
  detail::need(v, kv_dim, "v");
  detail::need(q_norm_w, head_dim, "q_norm_w");
  detail::need(k_norm_w, head_dim, "k_norm_w");
  detail::need(k_cache, cache_rows * kv_dim, "k_cache");
  detail::need(v_cache, cache_rows * kv_dim, "v_cache");
  if (rope.head_dim() != head_dim) throw Panic("decode_attention: RopeCache head_dim mismatch");
  detail::check(qasr_decode_attention_f32(out.ptr, q.ptr, k.ptr, v.ptr, q_norm_w.ptr, k_norm_w.ptr,
                                          rope.cos().ptr, rope.sin().ptr, rope.cap(), pos, n_heads,
                                          n_kv_heads, head_dim, eps, scale, k_cache.ptr, v_cache.ptr,
                                          cache_rows, workspace.ptr, workspace.len, detail::st()),
                "decode_attention");
}

// ---- lm_head (decoder.rs:929-963) ---------------------------------------------------
inline void argmax_rows(DevSlice<int32_t> idx, CF x, size_t rows, size_t cols) {
  detail::need(idx, rows, "idx");
  detail::need(x, rows * cols, "x");
  detail::check(qasr_argmax_rows_f32(idx.ptr, x.ptr, rows, cols, detail::st()), "argmax_rows");
}

inline size_t lm_head_workspace_bytes(size_t vocab) {
  return qasr_lm_head_argmax_workspace_bytes(vocab);
}

inline void lm_head_int8_argmax(DevSlice<int32_t> idx, F logits, CF x, DevSlice<const int8_t> w,
                                CF scales, size_t rows, size_t in_dim, size_t vocab,
                                DevSlice<uint8_t> workspace = {}) {
  detail::need(idx, rows, "idx");
  detail::need(logits, rows * vocab, "logits");
  detail::need(x, rows * in_dim, "x");
  detail::need(w, vocab * in_dim, "w");
  detail::need(scales, vocab, "scales");
  detail::check(qasr_lm_head_int8_argmax_f32(idx.ptr, logits.ptr, x.ptr, w.ptr, scales.ptr, rows,
                                             in_dim, vocab, workspace.ptr, workspace.len,
                                             detail::st()),
                "lm_head_int8_argmax");
}

// ---- .qint8 files (QuantFile, quantize.rs:108-330) ----------------------------------------
struct QuantTensorMeta {
  std::string name;
  int dtype = QASR_QINT8_INT8;
  std::vector<uint64_t> shape;
  uint64_t data_offset = 0, scale_offset = 0;
  size_t numel() const {
    size_t n = 1;
    for (uint64_t d : shape) n *= (size_t)d;
    return n;
  }
  size_t out_dim() const { return shape.empty() ? 0 : (size_t)shape[0]; }
  size_t in_dim() const { return shape.size() < 2 ? 0 : numel() / out_dim(); }
};

class QuantFile {
 public:
  // QuantFile::open: empty for a missing or malformed file.
  static std::optional<QuantFile> open(const std::string& path) {
    qasr_qint8_file* h = nullptr;
    if (qasr_qint8_open(path.c_str(), &h) != QASR_OK) return std::nullopt;
    return QuantFile(h);
  }
  QuantFile(QuantFile&& o) noexcept : h_(o.h_), tensors_(std::move(o.tensors_)) { o.h_ = nullptr; }
  QuantFile(const QuantFile&) = delete;
  QuantFile& operator=(const QuantFile&) = delete;
  ~QuantFile() { qasr_qint8_close(h_); }

  int version() const {
    int v = 0;
    detail::check(qasr_qint8_info(h_, &v, nullptr), "qint8_info");
    return v;
  }
  const std::vector<QuantTensorMeta>& tensors() const { return tensors_; }
  const QuantTensorMeta* find(const std::string& name) const {
    size_t i = 0;
    if (qasr_qint8_find(h_, name.c_str(), &i) != QASR_OK) return nullptr;
    return &tensors_[i];
  }
  // Copies a tensor's data (and INT8 row scales) to device memory.
  void upload(const std::string& name, void* data, size_t data_bytes, F scales = {}) const {
    const QuantTensorMeta* m = find(name);
    if (!m) throw Panic("qint8_upload: no tensor " + name);
    const size_t es = m->dtype == QASR_QINT8_F32 ? 4 : m->dtype == QASR_QINT8_BF16 ? 2 : 1;
    if (data_bytes < m->numel() * es) throw Panic("qint8_upload: data slice too short for " + name);
    if (m->dtype == QASR_QINT8_INT8) detail::need(scales, m->out_dim(), "scales");
    size_t i = 0;
    detail::check(qasr_qint8_find(h_, name.c_str(), &i), "qint8_find");
    detail::check(qasr_qint8_upload(h_, i, data, scales.ptr, detail::st()), "qint8_upload");
  }
  // DecoderInt8::load's fused gate/up (decoder.rs:697-719), built by the copy itself.
  void upload_gate_up(const std::string& gate, const std::string& up, size_t inter, size_t hidden,
                      DevSlice<int8_t> w, F scales) const {
    detail::need(w, 2 * inter * hidden, "w");
    detail::need(scales, 2 * inter, "scales");
    detail::check(qasr_qint8_upload_gate_up(h_, gate.c_str(), up.c_str(), inter, hidden, w.ptr,
                                            scales.ptr, detail::st()),
                  "qint8_upload_gate_up");
  }

 private:
  explicit QuantFile(qasr_qint8_file* h) : h_(h) {
    size_t n = 0;
    detail::check(qasr_qint8_info(h_, nullptr, &n), "qint8_info");
    for (size_t i = 0; i < n; ++i) {
      QuantTensorMeta m;
      const char* name = nullptr;
      size_t name_len = 0, n_dims = 0;
      uint64_t shape[256];
      detail::check(qasr_qint8_tensor(h_, i, &name, &name_len, &m.dtype, &n_dims, shape, 256,
                                      &m.data_offset, &m.scale_offset),
                    "qint8_tensor");
      m.name.assign(name, name_len);
      m.shape.assign(shape, shape + n_dims);
      tensors_.push_back(std::move(m));
    }
  }
  qasr_qint8_file* h_ = nullptr;
  std::vector<QuantTensorMeta> tensors_;
};

}  // namespace kernels
}  // namespace qwen_asr
