// Reader of the reference's private weight files (host side): the
// quantized_f12 tensors written by quantize_weights.py:60-64,91 as
// little-endian int32 .npy, [rows = out][cols = in], C order.  Same checks as
// MappedWeights (artifacts.hpp:31-49): magic and version 1 or 2, header at
// most 64 KiB, descr '<i4', fortran_order False, the exact expected shape and
// file length.  The file is memory-mapped read-only; at() is the reference's
// ring word (sign-extended, & (2^59 - 1), artifacts.hpp:86-92), and upload()
// copies the int32 tensor to the device, where praghip_share_gemm takes it
// with w_bits = 32.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "praghip.h"

namespace praghip {
int set_error(int code, const std::string& text);
}

struct praghip_weights {
  void* memory = MAP_FAILED;
  size_t length = 0, offset = 0, rows = 0, cols = 0;
  ~praghip_weights() {
    if (memory != MAP_FAILED) munmap(memory, length);
  }
  const int32_t* data() const {
    return reinterpret_cast<const int32_t*>(static_cast<const unsigned char*>(memory) + offset);
  }
};

namespace {

using praghip::set_error;

// Parses the dims of "'shape': (a, b, )" into out; false when malformed.
bool parse_shape(const std::string& h, std::vector<size_t>& out) {
  const size_t at = h.find("'shape': (");
  if (at == std::string::npos) return false;
  const size_t open = at + 10, close = h.find(')', open);
  if (close == std::string::npos) return false;
  const std::string body = h.substr(open, close - open);
  size_t i = 0;
  while (i < body.size()) {
    while (i < body.size() && (body[i] == ' ' || body[i] == ',')) ++i;
    if (i == body.size()) break;
    if (body[i] < '0' || body[i] > '9') return false;
    size_t v = 0;
    while (i < body.size() && body[i] >= '0' && body[i] <= '9') {
      const size_t d = size_t(body[i] - '0');
      if (v > (SIZE_MAX - d) / 10) return false;
      v = v * 10 + d;
      ++i;
    }
    out.push_back(v);
    while (i < body.size() && body[i] == ' ') ++i;
    if (i < body.size() && body[i] != ',') return false;
  }
  return true;
}

int open_checked(const char* path, size_t r, size_t c, bool vector, praghip_weights* w) {
  if (r == 0 || (!vector && c == 0)) return set_error(PRAGHIP_E_SHAPE, "BAD_SHAPE");
  const int fd = open(path, O_RDONLY | O_CLOEXEC | O_NOFOLLOW);
  if (fd < 0) return set_error(PRAGHIP_E_ARGUMENT, "E_WEIGHT_FILE");
  struct stat st {};
  if (fstat(fd, &st) || !S_ISREG(st.st_mode)) {
    close(fd);
    return set_error(PRAGHIP_E_ARGUMENT, "E_WEIGHT_FILE");
  }
  w->length = size_t(st.st_size);
  w->memory = w->length ? mmap(nullptr, w->length, PROT_READ, MAP_PRIVATE, fd, 0) : MAP_FAILED;
  close(fd);
  if (w->memory == MAP_FAILED) return set_error(PRAGHIP_E_ARGUMENT, "E_WEIGHT_MAP");
  const auto* p = static_cast<const unsigned char*>(w->memory);
  if (w->length < 12 || std::memcmp(p, "\x93NUMPY", 6) || (p[6] != 1 && p[6] != 2) || p[7] != 0)
    return set_error(PRAGHIP_E_ARGUMENT, "E_NPY_FORMAT");
  size_t n = size_t(p[8]) | (size_t(p[9]) << 8), off = 10;
  if (p[6] == 2) {
    n |= (size_t(p[10]) << 16) | (size_t(p[11]) << 24);
    off = 12;
  }
  if (n > 65536 || off + n > w->length) return set_error(PRAGHIP_E_ARGUMENT, "E_NPY_FORMAT");
  const std::string h(reinterpret_cast<const char*>(p + off), n);
  off += n;
  if (h.find("'descr': '<i4'") == std::string::npos || h.find("'fortran_order': False") == std::string::npos)
    return set_error(PRAGHIP_E_ARGUMENT, "E_NPY_FORMAT");
  std::vector<size_t> dims;
  if (!parse_shape(h, dims)) return set_error(PRAGHIP_E_ARGUMENT, "E_NPY_FORMAT");
  const std::vector<size_t> want = vector ? std::vector<size_t>{r} : std::vector<size_t>{r, c};
  const size_t cc = vector ? 1 : c;
  if (dims != want || r > SIZE_MAX / cc || r * cc > (SIZE_MAX - off) / 4 || off + r * cc * 4 != w->length)
    return set_error(PRAGHIP_E_SHAPE, "E_NPY_SHAPE");
  w->offset = off;
  w->rows = r;
  w->cols = cc;
  return PRAGHIP_OK;
}

}  // namespace

extern "C" {

int praghip_weights_open(const char* path, size_t rows, size_t cols, int vector, praghip_weights** out) {
  if (!path || !out) return set_error(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = nullptr;
  auto* w = new praghip_weights();
  const int rc = open_checked(path, rows, cols, vector != 0, w);
  if (rc != PRAGHIP_OK) {
    delete w;
    return rc;
  }
  *out = w;
  return PRAGHIP_OK;
}

int praghip_weights_shape(const praghip_weights* w, size_t* rows, size_t* cols) {
  if (!w || !rows || !cols) return set_error(PRAGHIP_E_ARGUMENT, "E_NULL");
  *rows = w->rows;
  *cols = w->cols;
  return PRAGHIP_OK;
}

const int32_t* praghip_weights_data(const praghip_weights* w) { return w ? w->data() : nullptr; }

int praghip_weights_at(const praghip_weights* w, size_t r, size_t c, uint64_t* word) {
  if (!w || !word) return set_error(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (r >= w->rows || c >= w->cols) return set_error(PRAGHIP_E_SHAPE, "BAD_SHAPE");
  int32_t v;
  std::memcpy(&v, w->data() + r * w->cols + c, 4);  // little-endian host
  *word = uint64_t(int64_t(v)) & ((uint64_t(1) << 59) - 1);
  return PRAGHIP_OK;
}

int praghip_weights_max_abs(const praghip_weights* w, uint64_t* max_abs) {
  if (!w || !max_abs) return set_error(PRAGHIP_E_ARGUMENT, "E_NULL");
  const int32_t* d = w->data();
  uint64_t m = 0;
  for (size_t i = 0, n = w->rows * w->cols; i < n; ++i) {
    int32_t v;
    std::memcpy(&v, d + i, 4);
    const uint64_t a = v < 0 ? uint64_t(-int64_t(v)) : uint64_t(v);
    m = a > m ? a : m;
  }
  *max_abs = m;
  return PRAGHIP_OK;
}

int praghip_weights_upload(const praghip_weights* w, int device, int32_t* dst, void* stream) {
  if (!w || !dst) return set_error(PRAGHIP_E_ARGUMENT, "E_NULL");
  int previous = 0;
  hipError_t e = hipGetDevice(&previous);
  if (e == hipSuccess && previous != device) e = hipSetDevice(device);
  const auto s = static_cast<hipStream_t>(stream);
  if (e == hipSuccess) e = hipMemcpyAsync(dst, w->data(), w->rows * w->cols * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);  // the mapping may be closed right after
  if (previous != device) (void)hipSetDevice(previous);
  if (e != hipSuccess) return set_error(PRAGHIP_E_DEVICE, std::string("E_WEIGHT_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

// Host split into the three balanced signed bytes (w = sum_e b_e 256^e with
// b_e in [-128, 127]) of praghip_share_gemm's w_bits 24, then one copy.
int praghip_weights_upload_split(const praghip_weights* w, int device, int8_t* dst, void* stream) {
  if (!w || !dst) return set_error(PRAGHIP_E_ARGUMENT, "E_NULL");
  const size_t count = w->rows * w->cols;
  const int32_t* src = w->data();
  std::vector<int8_t> planes(3 * count);
  for (size_t i = 0; i < count; ++i) {
    int v = src[i];
    if (v < -0x808080 || v > 0x7F7F7F) return set_error(PRAGHIP_E_SHAPE, "E_WEIGHT_RANGE");
    for (int e = 0; e < 3; ++e) {
      const int8_t b = int8_t(v & 0xff);  // the low byte as a signed value
      planes[size_t(e) * count + i] = b;
      v = (v - b) >> 8;
    }
  }
  int previous = 0;
  hipError_t e = hipGetDevice(&previous);
  if (e == hipSuccess && previous != device) e = hipSetDevice(device);
  const auto s = static_cast<hipStream_t>(stream);
  if (e == hipSuccess) e = hipMemcpyAsync(dst, planes.data(), planes.size(), hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (previous != device) (void)hipSetDevice(previous);
  if (e != hipSuccess) return set_error(PRAGHIP_E_DEVICE, std::string("E_WEIGHT_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

void praghip_weights_close(praghip_weights* w) { delete w; }

}  // extern "C"
