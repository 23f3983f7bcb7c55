// Reader for the `.qint8` quantized-weight files of qwen-asr-quantize
// (quantize.rs:1-34 format, QuantFile::open quantize.rs:122-245): maps the
// file read-only, parses the tensor table with the reference's rules, and
// uploads tensors to device memory. The fused gate/up upload interleaves the
// rows (g0, u0, g1, u1, ...) inside the copy itself with strided 2-D copies,
// as DecoderInt8::load builds the fused matrix on the host
// (decoder.rs:699-719).
//
// Format (little endian):
//   magic "QINT8\x01\0\0" (V1) or "QINT8\x02\0\0" (V2), u32 n_tensors, u32 0
//   per tensor: u16 name_len, name, [V2: u8 dtype 0=INT8 1=F32 2=BF16],
//               u8 n_dims, u32 shape[n_dims], u64 data_offset, u64 scale_offset
//   data section (offsets are relative to its start)
// V1 has no dtype byte: scale_offset 0 means F32, else INT8. An unknown V2
// dtype byte reads as INT8. A table cut short by the end of the file ends the
// table there (the tensors read so far stay), as the reference's loop does.
#include "common.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

struct qasr_qint8_file {
  const uint8_t* map = nullptr;
  size_t size = 0;
  size_t data_start = 0;
  int version = 0;
  mutable bool uploaded = false;  // a copy from the mapping was queued: close waits for it
  struct Tensor {
    std::string name;
    int dtype = 0;
    std::vector<uint64_t> shape;
    uint64_t data_offset = 0, scale_offset = 0;
  };
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> index;
};

namespace qasr {
namespace {

template <class T>
T rd(const uint8_t* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));  // little-endian host
  return v;
}

// Strict UTF-8 check (no overlong forms, no surrogates, nothing above
// U+10FFFF): a name that fails it makes QuantFile::open return None
// (quantize.rs:188, str::from_utf8).
bool valid_utf8(const uint8_t* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    if (c < 0x80) { ++i; continue; }
    size_t len;
    uint32_t cp, lo;
    if (c >= 0xC2 && c <= 0xDF) { len = 2; cp = c & 0x1F; lo = 0x80; }
    else if (c >= 0xE0 && c <= 0xEF) { len = 3; cp = c & 0x0F; lo = 0x800; }
    else if (c >= 0xF0 && c <= 0xF4) { len = 4; cp = c & 0x07; lo = 0x10000; }
    else return false;
    if (i + len > n) return false;
    for (size_t k = 1; k < len; ++k) {
      if ((s[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3F);
    }
    if (cp < lo || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return false;
    i += len;
  }
  return true;
}

size_t dtype_size(int dtype) { return dtype == QASR_QINT8_F32 ? 4 : (dtype == QASR_QINT8_BF16 ? 2 : 1); }

// numel and byte extents of tensor t; false if they overflow or leave the file
bool extents(const qasr_qint8_file* f, const qasr_qint8_file::Tensor& t, size_t* numel,
             size_t* data_bytes, size_t* out_dim) {
  size_t n = 1;
  for (uint64_t d : t.shape) {
    if (d && n > SIZE_MAX / d) return false;
    n *= (size_t)d;
  }
  *numel = n;
  *out_dim = t.shape.empty() ? 0 : (size_t)t.shape[0];
  const size_t es = dtype_size(t.dtype);
  if (n > SIZE_MAX / es) return false;
  *data_bytes = n * es;
  const size_t avail = f->size - f->data_start;
  if (t.data_offset > avail || *data_bytes > avail - t.data_offset) return false;
  if (t.dtype == QASR_QINT8_INT8) {
    if (*out_dim > SIZE_MAX / 4 || t.scale_offset > avail || *out_dim * 4 > avail - t.scale_offset)
      return false;
  }
  return true;
}

}  // namespace
}  // namespace qasr

using namespace qasr;

extern "C" int qasr_qint8_open(const char* path, qasr_qint8_file** out) {
  QASR_REQUIRE(path && out, "qint8_open: null argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(QASR_ERR_INVALID_ARG, std::string("qint8_open: cannot open ") + path);
  struct stat st {};
  if (fstat(fd, &st) < 0 || st.st_size < 16) {
    ::close(fd);
    return fail(QASR_ERR_INVALID_ARG, "qint8_open: not a .qint8 file (shorter than its header)");
  }
  const size_t size = (size_t)st.st_size;
  void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return fail(QASR_ERR_INVALID_ARG, "qint8_open: mmap failed");
  const uint8_t* d = static_cast<const uint8_t*>(m);
  int version = 0;
  if (std::memcmp(d, "QINT8\x02\x00\x00", 8) == 0) version = 2;
  else if (std::memcmp(d, "QINT8\x01\x00\x00", 8) == 0) version = 1;
  if (!version) {
    munmap(m, size);
    return fail(QASR_ERR_INVALID_ARG, "qint8_open: bad magic");
  }
  auto* f = new qasr_qint8_file;
  f->map = d;
  f->size = size;
  f->version = version;
  const uint32_t n = rd<uint32_t>(d + 8);
  size_t pos = 16;
  for (uint32_t t = 0; t < n; ++t) {
    if (pos + 2 > size) break;
    const size_t name_len = rd<uint16_t>(d + pos);
    pos += 2;
    if (pos + name_len > size) break;
    if (!valid_utf8(d + pos, name_len)) {
      delete f;
      munmap(m, size);
      return fail(QASR_ERR_INVALID_ARG, "qint8_open: tensor name is not UTF-8");
    }
    qasr_qint8_file::Tensor ten;
    ten.name.assign(reinterpret_cast<const char*>(d + pos), name_len);
    pos += name_len;
    int dtype = QASR_QINT8_INT8;
    if (version == 2) {
      if (pos + 1 > size) break;
      const uint8_t b = d[pos++];
      dtype = b == 1 ? QASR_QINT8_F32 : (b == 2 ? QASR_QINT8_BF16 : QASR_QINT8_INT8);
    }
    if (pos + 1 > size) break;
    const size_t n_dims = d[pos++];
    for (size_t k = 0; k < n_dims && pos + 4 <= size; ++k, pos += 4) ten.shape.push_back(rd<uint32_t>(d + pos));
    if (pos + 16 > size) break;
    ten.data_offset = rd<uint64_t>(d + pos);
    ten.scale_offset = rd<uint64_t>(d + pos + 8);
    pos += 16;
    if (version == 1) dtype = ten.scale_offset == 0 ? QASR_QINT8_F32 : QASR_QINT8_INT8;
    ten.dtype = dtype;
    f->index[ten.name] = f->tensors.size();  // a repeated name maps to its last entry
    f->tensors.push_back(std::move(ten));
  }
  f->data_start = pos;
  *out = f;
  return QASR_OK;
}

extern "C" int qasr_qint8_close(qasr_qint8_file* f) {
  if (!f) return QASR_OK;
  // queued copies may still read the mapping; only a file that uploaded
  // something touches the device here
  const bool sync_failed = f->uploaded && hipDeviceSynchronize() != hipSuccess;
  if (f->map) munmap(const_cast<uint8_t*>(f->map), f->size);
  delete f;
  return sync_failed ? fail(QASR_ERR_HIP, "qint8_close: device synchronize failed") : QASR_OK;
}

extern "C" int qasr_qint8_info(const qasr_qint8_file* f, int* version, size_t* n_tensors) {
  QASR_REQUIRE(f, "qint8_info: null file");
  if (version) *version = f->version;
  if (n_tensors) *n_tensors = f->tensors.size();
  return QASR_OK;
}

extern "C" int qasr_qint8_find(const qasr_qint8_file* f, const char* name, size_t* index) {
  QASR_REQUIRE(f && name && index, "qint8_find: null argument");
  const auto it = f->index.find(name);
  if (it == f->index.end()) return fail(QASR_ERR_INVALID_ARG, std::string("qint8_find: no tensor ") + name);
  *index = it->second;
  return QASR_OK;
}

extern "C" int qasr_qint8_tensor(const qasr_qint8_file* f, size_t index, const char** name,
                                 size_t* name_len, int* dtype, size_t* n_dims, uint64_t* shape,
                                 size_t shape_cap, uint64_t* data_offset, uint64_t* scale_offset) {
  QASR_REQUIRE(f, "qint8_tensor: null file");
  QASR_REQUIRE(index < f->tensors.size(), "qint8_tensor: index out of range");
  const auto& t = f->tensors[index];
  if (name) *name = t.name.data();
  if (name_len) *name_len = t.name.size();
  if (dtype) *dtype = t.dtype;
  if (n_dims) *n_dims = t.shape.size();
  if (shape) {
    QASR_REQUIRE(shape_cap >= t.shape.size(), "qint8_tensor: shape buffer too small");
    for (size_t k = 0; k < t.shape.size(); ++k) shape[k] = t.shape[k];
  }
  if (data_offset) *data_offset = t.data_offset;
  if (scale_offset) *scale_offset = t.scale_offset;
  return QASR_OK;
}

extern "C" int qasr_qint8_upload(const qasr_qint8_file* f, size_t index, void* dev_data,
                                 float* dev_scales, void* stream) {
  QASR_REQUIRE(f, "qint8_upload: null file");
  QASR_REQUIRE(index < f->tensors.size(), "qint8_upload: index out of range");
  const auto& t = f->tensors[index];
  size_t numel, bytes, out_dim;
  QASR_REQUIRE(extents(f, t, &numel, &bytes, &out_dim),
               "qint8_upload: tensor " + t.name + " extends past the end of the file");
  QASR_REQUIRE(dev_data || bytes == 0, "qint8_upload: null data destination");
  QASR_REQUIRE(t.dtype != QASR_QINT8_INT8 || dev_scales || out_dim == 0,
               "qint8_upload: INT8 tensors need a scales destination");
  hipStream_t st = as_stream(stream);
  const uint8_t* base = f->map + f->data_start;
  f->uploaded = true;
  if (bytes && hipMemcpyAsync(dev_data, base + t.data_offset, bytes, hipMemcpyHostToDevice, st) != hipSuccess)
    return fail(QASR_ERR_HIP, "qint8_upload: data copy failed");
  if (t.dtype == QASR_QINT8_INT8 && out_dim &&
      hipMemcpyAsync(dev_scales, base + t.scale_offset, out_dim * 4, hipMemcpyHostToDevice, st) != hipSuccess)
    return fail(QASR_ERR_HIP, "qint8_upload: scale copy failed");
  return QASR_OK;
}

extern "C" int qasr_qint8_upload_gate_up(const qasr_qint8_file* f, const char* gate_name,
                                         const char* up_name, size_t inter, size_t hidden,
                                         int8_t* dev_w, float* dev_scales, void* stream) {
  QASR_REQUIRE(f && gate_name && up_name && dev_w && dev_scales, "qint8_upload_gate_up: null argument");
  size_t gi, ui;
  int rc = qasr_qint8_find(f, gate_name, &gi);
  if (rc) return rc;
  rc = qasr_qint8_find(f, up_name, &ui);
  if (rc) return rc;
  const auto& g = f->tensors[gi];
  const auto& u = f->tensors[ui];
  QASR_REQUIRE(g.dtype == QASR_QINT8_INT8 && u.dtype == QASR_QINT8_INT8,
               "qint8_upload_gate_up: gate and up must be INT8 tensors");
  size_t gn, gb, go, un, ub, uo;  // numel, data bytes, shape[0]
  QASR_REQUIRE(extents(f, g, &gn, &gb, &go) && extents(f, u, &un, &ub, &uo),
               "qint8_upload_gate_up: tensor extends past the end of the file");
  QASR_REQUIRE(g.shape.size() == 2 && u.shape.size() == 2 && go == inter && uo == inter &&
                   g.shape[1] == hidden && u.shape[1] == hidden,
               "qint8_upload_gate_up: gate and up must both be [inter, hidden]");
  if (inter == 0 || hidden == 0) return QASR_OK;
  hipStream_t st = as_stream(stream);
  const uint8_t* base = f->map + f->data_start;
  f->uploaded = true;
  // rows of gate to fused rows 0, 2, 4, ...; rows of up to 1, 3, 5, ...
  if (hipMemcpy2DAsync(dev_w, 2 * hidden, base + g.data_offset, hidden, hidden, inter,
                       hipMemcpyHostToDevice, st) != hipSuccess ||
      hipMemcpy2DAsync(dev_w + hidden, 2 * hidden, base + u.data_offset, hidden, hidden, inter,
                       hipMemcpyHostToDevice, st) != hipSuccess ||
      hipMemcpy2DAsync(dev_scales, 8, base + g.scale_offset, 4, 4, inter, hipMemcpyHostToDevice, st) !=
          hipSuccess ||
      hipMemcpy2DAsync(dev_scales + 1, 8, base + u.scale_offset, 4, 4, inter, hipMemcpyHostToDevice, st) !=
          hipSuccess)
    return fail(QASR_ERR_HIP, "qint8_upload_gate_up: copy failed");
  return QASR_OK;
}
