// C ABI of praghip (include/praghip.h): the NTT and Switch plans, the share
// GEMM, the ring ops, lift, dyadic MAC and local dot, the seeded generators;
// the host helpers shared with plans.cpp (host.hpp).
//
// Plans mirror the reference's backend objects (NttBatch ntt.cu:99-171,
// Switch switch.cu:84-217): they own their device buffers and one stream,
// validate shapes and canonical inputs before touching the device, release
// themselves after any HIP error, and report Cleanup{first error, wiped bytes,
// freed bytes, closed} from an idempotent close().
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "praghip.h"
#include "host.hpp"
#include "kernels.hpp"

namespace praghip {
hipError_t launch_share_gemm(const uint64_t* x, const void* w, int w_bits, const int8_t* shifts, uint64_t* y,
                             int M, int K, int N, int mask_bits, hipStream_t s, bool y_zero = false);
bool share_gemm_adds_into_y(const void* x, const void* w, int w_bits, int M, int K, int N);
hipError_t launch_gemm_clear_list(const GemmClearList& l, hipStream_t s);
hipError_t launch_weight_split(const int32_t* w, int8_t* planes, size_t count, hipStream_t s);
hipError_t launch_share_gemm_valu(const uint64_t* x, const int8_t* w, const int8_t* shifts, uint64_t* y, int M,
                                  int K, int N, int mask_bits, hipStream_t s);
}

using namespace praghip;
using namespace praghip::host;

namespace {
thread_local std::string g_error;
}  // namespace

namespace praghip {
// The error slot, for the other host-side sources of the library.
int set_error(int code, const std::string& text) {
  g_error = text;
  return code;
}
}  // namespace praghip

namespace praghip::host {

int fail(int code, const std::string& text) { return set_error(code, text); }

// ------------------------------------------------------------ number theory
uint64_t mulmod(uint64_t a, uint64_t b, uint64_t q) { return uint64_t((u128)a * b % q); }
uint64_t powmod(uint64_t a, uint64_t e, uint64_t q) {
  uint64_t r = 1 % q;
  a %= q;
  for (; e; e >>= 1) {
    if (e & 1) r = mulmod(r, a, q);
    a = mulmod(a, a, q);
  }
  return r;
}
uint64_t invmod(uint64_t a, uint64_t q) { return powmod(a % q, q - 2, q); }  // q prime
bool is_prime(uint64_t n) {
  static const uint64_t bases[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return false;
  for (uint64_t b : bases) {
    if (n == b) return true;
    if (n % b == 0) return false;
  }
  uint64_t d = n - 1;
  int s = 0;
  while (!(d & 1)) {
    d >>= 1;
    ++s;
  }
  for (uint64_t b : bases) {
    uint64_t x = powmod(b, d, n);
    if (x == 1 || x == n - 1) continue;
    bool comp = true;
    for (int r = 1; r < s && comp; ++r) {
      x = mulmod(x, x, n);
      if (x == n - 1) comp = false;
    }
    if (comp) return false;
  }
  return true;
}
uint64_t shoup_q(uint64_t w, uint64_t q) { return uint64_t(((u128)w << 64) / q); }
uint64_t bitrev(uint64_t x, unsigned bits) {
  uint64_t r = 0;
  for (unsigned i = 0; i < bits; ++i) r |= ((x >> i) & 1) << (bits - 1 - i);
  return r;
}
// Smallest primitive 2N-th root of unity (SEAL try_minimal_primitive_root).
uint64_t minimal_root(uint64_t q, uint64_t two_n) {
  if ((q - 1) % two_n) return 0;
  uint64_t g = 0;
  for (uint64_t x = 2; x < q && !g; ++x) {
    const uint64_t c = powmod(x, (q - 1) / two_n, q);
    if (powmod(c, two_n / 2, q) == q - 1) g = c;
  }
  if (!g) return 0;
  const uint64_t g2 = mulmod(g, g, q);
  uint64_t cur = g, best = g;
  for (uint64_t i = 0; i < two_n; i += 2) {
    best = cur < best ? cur : best;
    cur = mulmod(cur, g2, q);
  }
  return best;
}
// SEAL NTTTables (seal_tables.cpp:22-33 exports them): forward[bitrev(i)] = psi^i,
// inverse[bitrev(i-1)+1] = psi^-i, invn = N^-1; each as (operand, quotient).
bool make_tables(uint64_t q, unsigned log_n, uint64_t* fwd, uint64_t* inv, uint64_t* invn, uint64_t* psi_out) {
  const uint64_t n = 1ull << log_n;
  const uint64_t psi = minimal_root(q, 2 * n);
  if (!psi) return false;
  const uint64_t psi_inv = invmod(psi, q);
  fwd[0] = 1;
  fwd[1] = shoup_q(1, q);
  inv[0] = 1;
  inv[1] = shoup_q(1, q);
  uint64_t p = psi, pi = psi_inv;
  for (uint64_t i = 1; i < n; ++i) {
    const uint64_t f = bitrev(i, log_n), r = bitrev(i - 1, log_n) + 1;
    fwd[2 * f] = p;
    fwd[2 * f + 1] = shoup_q(p, q);
    inv[2 * r] = pi;
    inv[2 * r + 1] = shoup_q(pi, q);
    p = mulmod(p, psi, q);
    pi = mulmod(pi, psi_inv, q);
  }
  const uint64_t ni = invmod(n % q, q);
  invn[0] = ni;
  invn[1] = shoup_q(ni, q);
  if (psi_out) *psi_out = psi;
  return true;
}

// --------------------------------------------------------------- device side

int check_device(int device) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return fail(PRAGHIP_E_DEVICE, "E_GFX950_REQUIRED: no HIP device");
  if (device < 0 || device >= count) return fail(PRAGHIP_E_ARGUMENT, "E_DEVICE_INDEX");
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return fail(PRAGHIP_E_DEVICE, "E_DEVICE_PROPERTIES");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(PRAGHIP_E_DEVICE, std::string("E_GFX950_REQUIRED: ") + prop.gcnArchName);
  return PRAGHIP_OK;
}


// Shared release: wipe sensitive buffers, synchronise, free everything.
void release_all(int device, Buffers& buf, hipStream_t& stream, hipEvent_t* events, int nevents, praghip_cleanup& c,
                 bool& closing) {
  closing = true;
  if (c.closed) return;
  auto ok = [&](hipError_t e) {
    if (e != hipSuccess && !c.first_hip_error) c.first_hip_error = int(e);
    return e == hipSuccess;
  };
  if (device < 0) {
    c.closed = 1;
    return;
  }
  DeviceScope scope(device);
  if (!ok(scope.status())) return;
  uint64_t queued = 0;
  for (auto& e : buf.entries)
    if (e.sensitive && *e.slot && ok(hipMemsetAsync(*e.slot, 0, e.bytes, stream))) queued += e.bytes;
  if (ok(stream ? hipStreamSynchronize(stream) : hipDeviceSynchronize())) c.wipe_synchronized_bytes += queued;
  bool all_freed = true;
  for (auto& e : buf.entries) {
    if (!*e.slot) continue;
    if (ok(hipFree(*e.slot))) {
      *e.slot = nullptr;
      if (e.sensitive) c.freed_bytes += e.bytes;
    } else {
      all_freed = false;
    }
  }
  bool events_gone = true;
  for (int i = 0; i < nevents; ++i)
    if (events[i]) {
      if (ok(hipEventDestroy(events[i]))) events[i] = nullptr;
      else events_gone = false;
    }
  if (stream && ok(hipStreamDestroy(stream))) stream = nullptr;
  c.closed = all_freed && events_gone && !stream;
}


// Builds the per-prime constants and device-format tables of a prime set.
int build_ntt_host(const uint64_t* q, size_t P, unsigned log_n, const uint64_t* fwd_in, const uint64_t* inv_in,
                   const uint64_t* invn_in, NttHost& h) {
  const size_t n = size_t(1) << log_n;
  h.primes.resize(P);
  h.fwd_u.resize(P * n);
  h.inv_u.resize(P * n);
  h.fwd_f.resize(P * n);
  h.inv_f.resize(P * n);
  std::vector<uint64_t> fwd(2 * n), inv(2 * n), invn(2);
  for (size_t p = 0; p < P; ++p) {
    const uint64_t qq = q[p];
    if (qq < 3 || qq >= (1ull << 62) || !is_prime(qq) || (qq - 1) % (2 * n))
      return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT: q must be a prime < 2^62 with q == 1 mod 2N");
    for (size_t p2 = 0; p2 < p; ++p2)
      if (q[p2] == qq) return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT: repeated prime");
    if (!make_tables(qq, log_n, fwd.data(), inv.data(), invn.data(), nullptr))
      return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT: no 2N-th root");
    if ((fwd_in && std::memcmp(fwd_in + p * 2 * n, fwd.data(), 16 * n)) ||
        (inv_in && std::memcmp(inv_in + p * 2 * n, inv.data(), 16 * n)) ||
        (invn_in && std::memcmp(invn_in + p * 2, invn.data(), 16)))
      return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT: tables are not the SEAL tables of q");
    NttPrime& pr = h.primes[p];
    std::memset(&pr, 0, sizeof(pr));
    pr.q = qq;
    pr.q2 = 2 * qq;
    pr.ninv = invn[0];
    pr.ninv_q = invn[1];
    const uint64_t w_last = inv[2 * (n - 1)];
    const uint64_t last = mulmod(w_last, invn[0], qq);
    pr.last = last;
    pr.last_q = shoup_q(last, qq);
    pr.one_q = shoup_q(1, qq);
    pr.use_f64 = qq < (1ull << 50);
    pr.qd = double(qq);
    pr.qinv = 1.0 / double(qq);
    pr.ninv_f = double(invn[0]);
    pr.last_f = double(last);
    for (size_t i = 0; i < n; ++i) {
      h.fwd_u[p * n + i] = make_ulonglong2(fwd[2 * i], fwd[2 * i + 1]);
      h.inv_u[p * n + i] = make_ulonglong2(inv[2 * i], inv[2 * i + 1]);
      h.fwd_f[p * n + i] = double(fwd[2 * i]);
      h.inv_f[p * n + i] = double(inv[2 * i]);
    }
  }
  return PRAGHIP_OK;
}

hipError_t upload_ntt(const NttHost& h, unsigned log_n, Buffers& buf, NttDevice& d, hipStream_t s) {
  const size_t P = h.primes.size(), n = size_t(1) << log_n;
  d.log_n = int(log_n);
  d.P = int(P);
  hipError_t e;
  if ((e = buf.alloc((void**)&d.primes, P * sizeof(NttPrime), false)) != hipSuccess) return e;
  if ((e = buf.alloc((void**)&d.tw_fwd_u, P * n * 16, false)) != hipSuccess) return e;
  if ((e = buf.alloc((void**)&d.tw_inv_u, P * n * 16, false)) != hipSuccess) return e;
  if ((e = buf.alloc((void**)&d.tw_fwd_f, P * n * 8, false)) != hipSuccess) return e;
  if ((e = buf.alloc((void**)&d.tw_inv_f, P * n * 8, false)) != hipSuccess) return e;
  for (size_t p = 0; p < P; ++p) {
    if (h.primes[p].use_f64)
      d.host_sel_f64[d.n_f64++] = int(p);
    else
      d.host_sel_u64[d.n_u64++] = int(p);
    if (!h.primes[p].use_f64 && h.primes[p].q >= (1ull << 60)) d.lazy_u64 = 0;
  }
  if ((e = buf.alloc((void**)&d.sel_f64, 64 * sizeof(int), false)) != hipSuccess) return e;
  if ((e = buf.alloc((void**)&d.sel_u64, 64 * sizeof(int), false)) != hipSuccess) return e;
  if ((e = hipMemcpyAsync(d.sel_f64, d.host_sel_f64, 64 * sizeof(int), hipMemcpyHostToDevice, s))) return e;
  if ((e = hipMemcpyAsync(d.sel_u64, d.host_sel_u64, 64 * sizeof(int), hipMemcpyHostToDevice, s))) return e;
  if ((e = hipMemcpyAsync(d.primes, h.primes.data(), P * sizeof(NttPrime), hipMemcpyHostToDevice, s))) return e;
  if ((e = hipMemcpyAsync(d.tw_fwd_u, h.fwd_u.data(), P * n * 16, hipMemcpyHostToDevice, s))) return e;
  if ((e = hipMemcpyAsync(d.tw_inv_u, h.inv_u.data(), P * n * 16, hipMemcpyHostToDevice, s))) return e;
  if ((e = hipMemcpyAsync(d.tw_fwd_f, h.fwd_f.data(), P * n * 8, hipMemcpyHostToDevice, s))) return e;
  if ((e = hipMemcpyAsync(d.tw_inv_f, h.inv_f.data(), P * n * 8, hipMemcpyHostToDevice, s))) return e;
  return hipStreamSynchronize(s);
}

// (pick: device-pointer entry points run on the caller's stream as given, NULL
// being the HIP null stream, so they order with the caller's own work.)

void wipe_host(std::vector<uint64_t>& v) {
  volatile uint64_t* p = v.data();
  for (size_t i = 0; i < v.size(); ++i) p[i] = 0;
}

}  // namespace praghip::host

// ============================================================== NttBatch plan
struct praghip_ntt_plan {
  int device = -1;
  unsigned log_n = 0;
  size_t P = 0, batches = 0, words = 0;
  std::vector<uint64_t> host_q;
  Buffers buf;
  NttDevice d;
  uint64_t* data = nullptr;
  ulonglong2* client_key = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t ev[4] = {};
  praghip_timing timing{};
  praghip_cleanup cleanup{};
  bool closing = false;
  void release() { release_all(device, buf, stream, ev, 4, cleanup, closing); }
  ~praghip_ntt_plan() { release(); }
};

namespace {
int device_failure(praghip_ntt_plan* p, hipError_t e, const char* what) {
  p->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_NTT_HIP: ") + what + ": " + hipGetErrorString(e));
}
}  // namespace

namespace praghip::host {
bool canonical(const uint64_t* v, size_t words, const std::vector<uint64_t>& q, unsigned log_n) {
  const size_t P = q.size();
  for (size_t i = 0; i < words; ++i)
    if (v[i] >= q[(i >> log_n) % P]) return false;
  return true;
}
}  // namespace praghip::host

extern "C" {

const char* praghip_last_error(void) { return g_error.c_str(); }
int praghip_version(void) { return 1; }

int praghip_device_count(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return 0;
  int good = 0;
  for (int i = 0; i < count; ++i) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, i) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++good;
  }
  return good;
}

}  // extern "C"

namespace {

bool is_hex_digit(char c) {
  return (c >= '0' && c <= '9') || (c >= 'a' && c <= 'f') || (c >= 'A' && c <= 'F');
}

// The binding strings of one device (empty on any runtime error).
bool device_identity(int device, std::string& uuid, std::string& pci) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return false;
  const char* b = prop.uuid.bytes;
  bool text = true;
  for (int i = 0; i < 16; ++i) text = text && is_hex_digit(b[i]);
  uuid = "GPU-";
  if (text) {
    uuid.append(b, 16);
  } else {
    static const char digits[] = "0123456789abcdef";
    for (int i = 0; i < 16; ++i) {
      if (i == 4 || i == 6 || i == 8 || i == 10) uuid += '-';
      const unsigned v = static_cast<unsigned char>(b[i]);
      uuid += digits[v >> 4];
      uuid += digits[v & 15];
    }
  }
  char bus[64] = {0};
  if (hipDeviceGetPCIBusId(bus, sizeof(bus) - 1, device) != hipSuccess) return false;
  pci = bus;
  return true;
}

bool same_id(const std::string& a, const char* b) {
  if (a.size() != std::strlen(b)) return false;
  for (size_t i = 0; i < a.size(); ++i) {
    char x = a[i], y = b[i];
    if (x >= 'A' && x <= 'F') x = char(x - 'A' + 'a');
    if (y >= 'A' && y <= 'F') y = char(y - 'A' + 'a');
    if (x != y) return false;
  }
  return true;
}

}  // namespace

extern "C" {

int praghip_device_identity(int device, char* uuid, size_t uuid_size, char* pci, size_t pci_size) {
  if (!uuid || !pci) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (uuid_size < 40 || pci_size < 16) return fail(PRAGHIP_E_ARGUMENT, "E_IDENTITY_BUFFER");
  uuid[0] = pci[0] = 0;
  if (int rc = check_device(device)) return rc;
  std::string u, p;
  if (!device_identity(device, u, p) || p.size() >= pci_size) return fail(PRAGHIP_E_DEVICE, "E_DEVICE_PROPERTIES");
  std::memcpy(uuid, u.c_str(), u.size() + 1);
  std::memcpy(pci, p.c_str(), p.size() + 1);
  return PRAGHIP_OK;
}

int praghip_device_bind(const char* uuid, const char* pci, int* device) {
  if (!device) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *device = -1;
  if (!uuid || !pci || !*uuid || !*pci) return fail(PRAGHIP_E_DEVICE, "E_PHASE_DEVICE_BINDING");
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) count = 0;
  for (int i = 0; i < count; ++i) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, i) != hipSuccess || std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) continue;
    std::string u, p;
    if (device_identity(i, u, p) && same_id(u, uuid) && same_id(p, pci)) {
      *device = i;
      return PRAGHIP_OK;
    }
  }
  return fail(PRAGHIP_E_DEVICE, "E_GFX950_REQUIRED: no gfx950 device with this UUID and PCI bus id");
}

int praghip_device_bind_env(const char* uuid_var, const char* pci_var, int* device) {
  if (!device) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *device = -1;
  const char* uuid = std::getenv(uuid_var ? uuid_var : "PRAG_ENC0_GPU_UUID");
  const char* pci = std::getenv(pci_var ? pci_var : "PRAG_ENC0_GPU_PCI");
  return praghip_device_bind(uuid, pci, device);
}

int praghip_ntt_tables(uint64_t q, uint32_t log_n, uint64_t* fwd_pairs, uint64_t* inv_pairs, uint64_t* invn_pair,
                       uint64_t* psi) {
  if (!fwd_pairs || !inv_pairs || !invn_pair) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (log_n < 1 || log_n > 17) return fail(PRAGHIP_E_SHAPE, "E_NTT_SHAPE");
  if (q < 3 || q >= (1ull << 62) || !is_prime(q)) return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT");
  if (!make_tables(q, log_n, fwd_pairs, inv_pairs, invn_pair, psi)) return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT");
  return PRAGHIP_OK;
}

int praghip_ntt_plan_create(int device, const uint64_t* q, size_t primes, uint32_t log_n, const uint64_t* fwd_pairs,
                            const uint64_t* inv_pairs, const uint64_t* invn_pairs, size_t batches,
                            praghip_ntt_plan** plan) {
  if (!plan || !q) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *plan = nullptr;
  if (log_n < 4 || log_n > 14 || primes < 1 || primes > 64) return fail(PRAGHIP_E_SHAPE, "E_NTT_SHAPE");
  NttHost h;
  if (int rc = build_ntt_host(q, primes, log_n, fwd_pairs, inv_pairs, invn_pairs, h)) return rc;
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_ntt_plan> p(new praghip_ntt_plan);
  p->device = device;
  p->log_n = log_n;
  p->P = primes;
  p->batches = batches;
  p->words = batches * primes << log_n;
  p->host_q.assign(q, q + primes);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  for (auto& ev : p->ev)
    if (e == hipSuccess) e = hipEventCreate(&ev);
  if (e == hipSuccess) e = upload_ntt(h, log_n, p->buf, p->d, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->data, p->words * 8, true);
  if (e != hipSuccess) return device_failure(p.get(), e, "create");
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  *plan = p.release();
  return PRAGHIP_OK;
}

static int ntt_device(praghip_ntt_plan* p, uint64_t* data, size_t limbs, void* stream, bool inverse) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_NTT_CLOSED");
  if (!data && limbs) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (reinterpret_cast<uintptr_t>(data) & 15) return fail(PRAGHIP_E_ARGUMENT, "E_NTT_ALIGNMENT: 16-byte aligned data");
  if (limbs > (1ull << 31)) return fail(PRAGHIP_E_SHAPE, "E_NTT_SHAPE");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ntt(inverse, data, limbs, p->d, pick(stream));
  if (e != hipSuccess) return device_failure(p, e, inverse ? "inverse" : "forward");
  return PRAGHIP_OK;
}

int praghip_ntt_forward(praghip_ntt_plan* plan, uint64_t* data, size_t limbs, void* stream) {
  return ntt_device(plan, data, limbs, stream, false);
}
int praghip_ntt_inverse(praghip_ntt_plan* plan, uint64_t* data, size_t limbs, void* stream) {
  return ntt_device(plan, data, limbs, stream, true);
}

static int ntt_host_run(praghip_ntt_plan* p, const uint64_t* input, uint64_t* output, int mode) {
  // mode 0 forward, 1 inverse, 2 client phase
  if (!p || !input || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_NTT_CLOSED");
  if (mode == 2 && !p->client_key) return fail(PRAGHIP_E_STATE, "E_CLIENT_KEY_STATE");
  if (!p->words) return fail(PRAGHIP_E_SHAPE, "E_NTT_SHAPE");
  if (!canonical(input, p->words, p->host_q, p->log_n)) return fail(PRAGHIP_E_CANONICAL, "E_NTT_CANONICAL_REQUIRED");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  const size_t bytes = p->words * 8, limbs = p->words >> p->log_n;
  hipStream_t s = p->stream;
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], s);
  if (e == hipSuccess) e = hipMemcpyAsync(p->data, input, bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], s);
  if (e == hipSuccess) e = launch_ntt(mode == 1, p->data, limbs, p->d, s);
  if (mode == 2) {
    if (e == hipSuccess) e = launch_dyadic_shoup(p->data, p->client_key, p->d, p->words, s);
    if (e == hipSuccess) e = launch_ntt(true, p->data, limbs, p->d, s);
  }
  if (e == hipSuccess) e = hipEventRecord(p->ev[2], s);
  if (e == hipSuccess) e = hipMemcpyAsync(output, p->data, bytes, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[3], s);
  if (e == hipSuccess) e = hipEventSynchronize(p->ev[3]);
  float t01 = 0, t12 = 0, t23 = 0;
  if (e == hipSuccess) e = hipEventElapsedTime(&t01, p->ev[0], p->ev[1]);
  if (e == hipSuccess) e = hipEventElapsedTime(&t12, p->ev[1], p->ev[2]);
  if (e == hipSuccess) e = hipEventElapsedTime(&t23, p->ev[2], p->ev[3]);
  if (e != hipSuccess) {
    std::memset(output, 0, bytes);
    return device_failure(p, e, "transform");
  }
  p->timing.upload_ms = t01;
  p->timing.kernel_ms = t12;
  p->timing.download_ms = t23;
  return PRAGHIP_OK;
}

int praghip_ntt_transform(praghip_ntt_plan* plan, const uint64_t* input, uint64_t* output, int inverse) {
  return ntt_host_run(plan, input, output, inverse ? 1 : 0);
}

int praghip_ntt_bind_client_key(praghip_ntt_plan* p, const uint64_t* key) {
  if (!p || !key) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing || p->client_key) return fail(PRAGHIP_E_STATE, "E_CLIENT_KEY_STATE");
  const size_t n = size_t(1) << p->log_n;
  std::vector<uint64_t> pairs(2 * p->P * n);
  for (size_t k = 0; k < p->P; ++k)
    for (size_t i = 0; i < n; ++i) {
      const uint64_t v = key[k * n + i];
      if (v >= p->host_q[k]) {
        wipe_host(pairs);
        return fail(PRAGHIP_E_CANONICAL, "E_CLIENT_KEY_CANONICAL");
      }
      pairs[2 * (k * n + i)] = v;
      pairs[2 * (k * n + i) + 1] = shoup_q(v, p->host_q[k]);
    }
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->client_key, pairs.size() * 8, true);
  if (e == hipSuccess) e = hipMemcpyAsync(p->client_key, pairs.data(), pairs.size() * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  wipe_host(pairs);
  if (e != hipSuccess) return device_failure(p, e, "bind_client_key");
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  return PRAGHIP_OK;
}

int praghip_ntt_client_phase(praghip_ntt_plan* plan, const uint64_t* input, uint64_t* output) {
  return ntt_host_run(plan, input, output, 2);
}

int praghip_ntt_sync(praghip_ntt_plan* p) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_NTT_CLOSED");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return device_failure(p, e, "sync");
  return PRAGHIP_OK;
}

int praghip_ntt_timing(const praghip_ntt_plan* p, praghip_timing* out) {
  if (!p || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = p->timing;
  return PRAGHIP_OK;
}

int praghip_ntt_close(praghip_ntt_plan* p, praghip_cleanup* out) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  p->release();
  if (out) *out = p->cleanup;
  return PRAGHIP_OK;
}

void praghip_ntt_destroy(praghip_ntt_plan* p) { delete p; }

}  // extern "C"

// ================================================================ Switch plan
struct praghip_switch_plan {
  int device = -1;
  unsigned log_n = 0;
  uint32_t element = 1;
  size_t L = 0, K = 0, dnum = 0, max_batch = 0;
  std::vector<uint64_t> host_q;
  Buffers buf;
  NttDevice d;
  KsConst kc{};
  KsConst* kc_dev = nullptr;
  uint64_t *key = nullptr, *acc = nullptr, *prod = nullptr, *in = nullptr, *out = nullptr, *inter = nullptr;
  unsigned* queue = nullptr;
  unsigned acc_slots = 0;
  size_t inter_cts = 0;
  hipStream_t stream = nullptr;
  // start, uploaded, the four kernel phases, downloaded
  static constexpr int kEvents = 7;
  hipEvent_t ev[kEvents] = {};
  praghip_timing timing{};
  praghip_switch_phases phases{};
  praghip_cleanup cleanup{};
  bool closing = false;
  void release() { release_all(device, buf, stream, ev, kEvents, cleanup, closing); }
  ~praghip_switch_plan() { release(); }
};

namespace {
int switch_failure(praghip_switch_plan* p, hipError_t e, const char* what) {
  p->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_SWITCH_HIP: ") + what + ": " + hipGetErrorString(e));
}
}  // namespace

namespace praghip::host {
// Galois element validity (keyswitch/seal_adapter.cpp:35): odd and < 2N.
bool galois_inverse(uint32_t g, unsigned log_n, uint32_t& ginv) {
  const uint64_t two_n = 2ull << log_n;
  if (!(g & 1) || g >= two_n) return false;
  // (Z/2N)* has order N, so g^-1 = g^(N-1) mod 2N
  uint64_t r = 1, b = g, e = (1ull << log_n) - 1;
  for (; e; e >>= 1) {
    if (e & 1) r = r * b % two_n;
    b = b * b % two_n;
  }
  ginv = uint32_t(r);
  return true;
}
int build_ks_const(const uint64_t* q, size_t L, size_t dnum, unsigned log_n, KsConst& kc) {
  const size_t K = L + 1;
  std::memset(&kc, 0, sizeof(kc));
  kc.L = int(L);
  kc.K = int(K);
  kc.dnum = int(dnum);
  kc.log_n = int(log_n);
  const size_t base = L / dnum, extra = L % dnum;
  for (size_t j = 0; j <= dnum; ++j) kc.dig_lo[j] = int(j * base + (j < extra ? j : extra));
  for (size_t j = 0; j < dnum; ++j)
    for (int i = kc.dig_lo[j]; i < kc.dig_lo[j + 1]; ++i) kc.digit_of[i] = int(j);
  for (size_t t = 0; t < K; ++t) {
    kc.q[t] = q[t];
    const u128 ratio = (~(u128)0) / q[t];
    kc.bar[t] = Barrett{q[t], uint64_t(ratio), uint64_t(ratio >> 64)};
    kc.one_q[t] = shoup_q(1, q[t]);
  }
  for (size_t i = 0; i < L; ++i) {
    const int j = kc.digit_of[i];
    uint64_t h = 1;
    for (int i2 = kc.dig_lo[j]; i2 < kc.dig_lo[j + 1]; ++i2)
      if (size_t(i2) != i) h = mulmod(h, q[i2] % q[i], q[i]);
    const uint64_t ih = invmod(h, q[i]);
    kc.inv_hat[i] = Shoup{ih, shoup_q(ih, q[i])};
    for (size_t t = 0; t < K; ++t) {
      uint64_t ht = 1;
      for (int i2 = kc.dig_lo[j]; i2 < kc.dig_lo[j + 1]; ++i2)
        if (size_t(i2) != i) ht = mulmod(ht, q[i2] % q[t], q[t]);
      kc.hat[i][t] = Shoup{ht, shoup_q(ht, q[t])};
    }
    const uint64_t p = q[L];
    const uint64_t ip = invmod(p % q[i], q[i]);
    kc.invp[i] = Shoup{ip, shoup_q(ip, q[i])};
    kc.half_mod[i] = (p >> 1) % q[i];
  }
  kc.lazy = 1;
  const uint64_t n = 1ull << log_n;
  std::vector<uint64_t> fwd(2 * n), inv(2 * n), invn(2);
  for (size_t t = 0; t < K; ++t) {
    kc.lazy &= q[t] < (1ull << 60) ? 1 : 0;
    uint64_t y = 1;  // q^-1 mod 2^64 by Newton's iteration (each step doubles the correct low bits)
    for (int it = 0; it < 6; ++it) y *= 2 - q[t] * y;
    kc.neg_qinv[t] = 0 - y;
    if (!make_tables(q[t], log_n, fwd.data(), inv.data(), invn.data(), nullptr)) return PRAGHIP_E_CONTEXT;
    const uint64_t r = uint64_t(((u128)1 << 64) % q[t]);  // 2^64 mod q_t
    const uint64_t nr = mulmod(invn[0], r, q[t]), lr = mulmod(inv[2 * (n - 1)], nr, q[t]);
    kc.ninv_r[t] = Shoup{nr, shoup_q(nr, q[t])};
    kc.last_r[t] = Shoup{lr, shoup_q(lr, q[t])};
  }
  return PRAGHIP_OK;
}
}  // namespace praghip::host

extern "C" {

int praghip_switch_plan_create(int device, const uint64_t* q, size_t data_primes, uint32_t log_n, size_t dnum,
                               const uint64_t* fwd_pairs, const uint64_t* inv_pairs, const uint64_t* invn_pairs,
                               const uint64_t* invp_pairs, const uint64_t* key, uint32_t element, size_t max_batch,
                               praghip_switch_plan** plan) {
  if (!plan || !q) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *plan = nullptr;
  const size_t L = data_primes, K = L + 1;
  if (log_n < 4 || log_n > 14 || L < 1 || K > size_t(kMaxKeyPrimes) || dnum < 1 || dnum > L || max_batch < 1)
    return fail(PRAGHIP_E_SHAPE, "E_SWITCH_SHAPE");
  uint32_t ginv = 1;
  if (!galois_inverse(element, log_n, ginv)) return fail(PRAGHIP_E_ARGUMENT, "E_SWITCH_ELEMENT");
  // the caller's SEAL tables (Switch::initialize, switch.hpp:24) are checked
  // against the ones derived from q
  NttHost h;
  if (int rc = build_ntt_host(q, K, log_n, fwd_pairs, inv_pairs, invn_pairs, h)) return rc;
  if (invp_pairs)
    for (size_t i = 0; i < L; ++i) {  // inv_q_last_mod_q (seal_adapter.cpp:40): q[L]^-1 mod q_i, Shoup quotient
      const uint64_t ip = invmod(q[L] % q[i], q[i]);
      if (invp_pairs[2 * i] != ip || invp_pairs[2 * i + 1] != shoup_q(ip, q[i]))
        return fail(PRAGHIP_E_CONTEXT, "E_NTT_CONTEXT: inv_q_last_mod_q is not q[L]^-1 mod q_i");
    }
  const size_t n = size_t(1) << log_n, key_words = dnum * 2 * K * n;
  if (key)
    for (size_t i = 0; i < key_words; ++i)
      if (key[i] >= q[(i >> log_n) % K]) return fail(PRAGHIP_E_CANONICAL, "E_SWITCH_KEY_CANONICAL");
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_switch_plan> p(new praghip_switch_plan);
  p->device = device;
  p->log_n = log_n;
  p->element = element;
  p->L = L;
  p->K = K;
  p->dnum = dnum;
  p->max_batch = max_batch;
  p->host_q.assign(q, q + K);
  build_ks_const(q, L, dnum, log_n, p->kc);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  for (auto& ev : p->ev)
    if (e == hipSuccess) e = hipEventCreate(&ev);
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], p->stream);
  if (e == hipSuccess) e = upload_ntt(h, log_n, p->buf, p->d, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->kc_dev, sizeof(KsConst), false);
  if (e == hipSuccess) e = hipMemcpyAsync(p->kc_dev, &p->kc, sizeof(KsConst), hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess && key) e = p->buf.alloc((void**)&p->key, key_words * 8, true);
  if (e == hipSuccess && key) e = hipMemcpyAsync(p->key, key, key_words * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], p->stream);
  // the fused kernel's running sums and work queue, only for shapes the
  // three-phase kernels do not take (they never touch either)
  const bool fused = !keyswitch_rows_supported(p->kc);
  if (e == hipSuccess && fused) {
    p->acc_slots = ks_acc_slots(int(log_n));
    e = p->acc_slots ? p->buf.alloc((void**)&p->acc, size_t(p->acc_slots) * 2 * n * 8, true) : hipErrorInvalidValue;
  }
  if (e == hipSuccess && fused) e = p->buf.alloc((void**)&p->queue, kQueueWords * 4, false);
  if (e == hipSuccess && fused) e = hipMemsetAsync(p->queue, 0, kQueueWords * 4, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->prod, max_batch * 2 * K * n * 8, true);
  if (e == hipSuccess && keyswitch_rows_supported(p->kc)) {
    p->inter_cts = std::min(max_batch, kKsRowsChunk);
    e = p->buf.alloc((void**)&p->inter, p->inter_cts * dnum * K * n * 8, true);
  }
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->in, 2 * L * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->out, 2 * L * n * 8, true);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  float setup_ms = 0;
  if (e == hipSuccess) e = hipEventElapsedTime(&setup_ms, p->ev[0], p->ev[1]);
  if (e != hipSuccess) return switch_failure(p.get(), e, "create");
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  p->phases.setup_upload_ms = setup_ms;
  p->phases.device_bytes = p->timing.device_bytes;
  p->phases.sensitive_bytes = p->timing.sensitive_bytes;
  *plan = p.release();
  return PRAGHIP_OK;
}

static hipError_t keyswitch_chunks(praghip_switch_plan* p, const uint64_t* in, uint64_t* out, size_t batch,
                                   const uint64_t* keys, size_t key_stride, uint32_t ginv, hipStream_t s,
                                   hipEvent_t* phase_events = nullptr) {
  const size_t n = size_t(1) << p->log_n, ct_words = 2 * p->L * n;
  for (size_t b0 = 0; b0 < batch; b0 += p->max_batch) {
    KsArgs a;
    a.batch = std::min(p->max_batch, batch - b0);
    a.in = in + b0 * ct_words;
    a.out = out + b0 * ct_words;
    a.key = keys + b0 * key_stride;
    a.key_stride = key_stride;
    a.acc = p->acc;
    a.acc_slots = p->acc_slots;
    a.prod = p->prod;
    a.galois_inv = ginv;
    a.queue = p->queue;
    a.inter = p->inter;
    a.inter_cts = p->inter_cts;
    a.phase_events = batch <= p->max_batch ? phase_events : nullptr;
    const hipError_t e = launch_keyswitch(a, p->kc_dev, p->kc, p->d, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int praghip_keyswitch(praghip_switch_plan* p, const uint64_t* input, uint64_t* output, size_t batch,
                      const uint64_t* keys, size_t key_stride, uint32_t galois_elt, void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  if (batch && (!input || !output)) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (input == output && batch) return fail(PRAGHIP_E_ARGUMENT, "E_SWITCH_ALIAS");
  if ((reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(output)) & 7 ||
      (reinterpret_cast<uintptr_t>(keys) & 15) || (key_stride & 1))
    return fail(PRAGHIP_E_ARGUMENT, "E_SWITCH_ALIGNMENT: 8-byte aligned ciphertexts, 16-byte aligned keys, even key_stride");
  if (!keys && !p->key) return fail(PRAGHIP_E_STATE, "E_SWITCH_NO_KEY");
  uint32_t ginv = 1;
  if (!galois_inverse(galois_elt, p->log_n, ginv)) return fail(PRAGHIP_E_ARGUMENT, "E_SWITCH_ELEMENT");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess)
    e = keyswitch_chunks(p, input, output, batch, keys ? keys : p->key, keys ? key_stride : 0, ginv,
                         pick(stream));
  if (e != hipSuccess) return switch_failure(p, e, "keyswitch");
  return PRAGHIP_OK;
}

// Host round trip on the plan's stream: upload, keyswitch with Galois inverse
// `ginv` (1: none), download, synchronous.
static int switch_host_run(praghip_switch_plan* p, const uint64_t* input, uint64_t* output, uint32_t ginv,
                           const char* what) {
  if (!p || !input || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  if (!p->key) return fail(PRAGHIP_E_STATE, "E_SWITCH_NO_KEY");
  const size_t n = size_t(1) << p->log_n, words = 2 * p->L * n;
  for (size_t i = 0; i < words; ++i)
    if (input[i] >= p->host_q[(i >> p->log_n) % p->L]) return fail(PRAGHIP_E_CANONICAL, "E_SWITCH_CIPHERTEXT");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  hipStream_t s = p->stream;
  // events: 0 start, 1 uploaded, 2..5 after the four kernel phases, 6 downloaded
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], s);
  if (e == hipSuccess) e = hipMemcpyAsync(p->in, input, words * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], s);
  if (e == hipSuccess) e = keyswitch_chunks(p, p->in, p->out, 1, p->key, 0, ginv, s, p->ev + 2);
  if (e == hipSuccess) e = hipMemcpyAsync(output, p->out, words * 8, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[6], s);
  if (e == hipSuccess) e = hipEventSynchronize(p->ev[6]);
  float t[6] = {};
  for (int i = 0; i < 6 && e == hipSuccess; ++i) e = hipEventElapsedTime(&t[i], p->ev[i], p->ev[i + 1]);
  if (e != hipSuccess) {
    std::memset(output, 0, words * 8);
    return switch_failure(p, e, what);
  }
  p->timing.upload_ms = t[0];
  p->timing.kernel_ms = double(t[1]) + t[2] + t[3] + t[4];
  p->timing.download_ms = t[5];
  p->phases.upload_ms = t[0];
  p->phases.rns_ntt_ms = t[1];
  p->phases.product_ms = t[2];
  p->phases.inverse_ms = t[3];
  p->phases.moddown_ms = t[4];
  p->phases.download_ms = t[5];
  return PRAGHIP_OK;
}

int praghip_switch_apply(praghip_switch_plan* p, const uint64_t* input, uint64_t* output) {
  uint32_t ginv = 1;
  if (p) galois_inverse(p->element, p->log_n, ginv);
  return switch_host_run(p, input, output, ginv, "apply");
}

int praghip_switch_evaluate(praghip_switch_plan* p, const uint64_t* input, uint64_t* output) {
  return switch_host_run(p, input, output, 1u, "evaluate");
}

int praghip_switch_sync(praghip_switch_plan* p) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return switch_failure(p, e, "sync");
  return PRAGHIP_OK;
}

int praghip_switch_timing(const praghip_switch_plan* p, praghip_timing* out) {
  if (!p || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = p->timing;
  return PRAGHIP_OK;
}

int praghip_switch_phase_timing(const praghip_switch_plan* p, praghip_switch_phases* out) {
  if (!p || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = p->phases;
  return PRAGHIP_OK;
}

int praghip_switch_close(praghip_switch_plan* p, praghip_cleanup* out) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  p->release();
  if (out) *out = p->cleanup;
  return PRAGHIP_OK;
}

void praghip_switch_destroy(praghip_switch_plan* p) { delete p; }

// ================================================================ share GEMM
int praghip_share_gemm(int device, const uint64_t* x, const void* w, int w_bits, const int8_t* shifts, uint64_t* y,
                       size_t m, size_t k, size_t n, int mask_bits, void* stream) {
  if (m == 0 || n == 0) return PRAGHIP_OK;
  if (!x || !w || !y) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (w_bits != 8 && w_bits != 24 && w_bits != 32) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_WEIGHT_DTYPE");
  if (mask_bits < 1 || mask_bits > 64) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_MASK");
  if (k >= (1u << 17) || m >= (1u << 31) || n >= (1u << 31)) return fail(PRAGHIP_E_SHAPE, "E_SHARE_SHAPE");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 7 ||
      (w_bits == 32 && (reinterpret_cast<uintptr_t>(w) & 3)))
    return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess)
    e = launch_share_gemm(x, w, w_bits, shifts, y, int(m), int(k), int(n), mask_bits, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_SHARE_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

int praghip_share_gemm_valu(int device, const uint64_t* x, const int8_t* w, const int8_t* shifts, uint64_t* y,
                            size_t m, size_t k, size_t n, int mask_bits, void* stream) {
  if (m == 0 || n == 0) return PRAGHIP_OK;
  if (!x || !w || !y) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (mask_bits < 1 || mask_bits > 64) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_MASK");
  if (k >= (1u << 17) || m >= (1u << 31) || n >= (1u << 31)) return fail(PRAGHIP_E_SHAPE, "E_SHARE_SHAPE");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 7)
    return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess)
    e = launch_share_gemm_valu(x, w, shifts, y, int(m), int(k), int(n), mask_bits, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_SHARE_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

int praghip_weights_split(int device, const int32_t* w, int8_t* planes, size_t count, void* stream) {
  if (count == 0) return PRAGHIP_OK;
  if (!w || !planes) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (reinterpret_cast<uintptr_t>(w) & 3) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_weight_split(w, planes, count, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_SHARE_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

int praghip_share_gemm_batch(int device, const praghip_gemm_desc* list, size_t count, void* stream) {
  if (count == 0) return PRAGHIP_OK;
  if (!list) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  for (size_t i = 0; i < count; ++i) {  // validate the whole list before the first launch
    const praghip_gemm_desc& d = list[i];
    if (d.m == 0 || d.n == 0) continue;
    if (!d.x || !d.w || !d.y) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
    if (d.w_bits != 8 && d.w_bits != 24 && d.w_bits != 32) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_WEIGHT_DTYPE");
    if (d.mask_bits < 1 || d.mask_bits > 64) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_MASK");
    if (d.k >= (1u << 17) || d.m >= (1u << 31) || d.n >= (1u << 31)) return fail(PRAGHIP_E_SHAPE, "E_SHARE_SHAPE");
    if ((reinterpret_cast<uintptr_t>(d.x) | reinterpret_cast<uintptr_t>(d.y)) & 7 ||
        (d.w_bits == 32 && (reinterpret_cast<uintptr_t>(d.w) & 3)))
      return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  }
  // the outputs that split-K products add into are zeroed together, one
  // launch per up to kGemmClearMax of them, when none of them overlaps any
  // other operand of the batch (an earlier product could read it); otherwise
  // each product clears its own output just before it runs
  std::vector<size_t> adds;
  for (size_t i = 0; i < count; ++i) {
    const praghip_gemm_desc& d = list[i];
    if (d.m && d.n && share_gemm_adds_into_y(d.x, d.w, d.w_bits, int(d.m), int(d.k), int(d.n))) adds.push_back(i);
  }
  const auto span = [](const void* p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    return std::pair<uintptr_t, uintptr_t>(a, a + bytes);
  };
  const auto overlaps = [](std::pair<uintptr_t, uintptr_t> a, std::pair<uintptr_t, uintptr_t> b) {
    return a.first < b.second && b.first < a.second;
  };
  bool together = adds.size() > 1;
  for (size_t a = 0; a < adds.size() && together; ++a) {
    const praghip_gemm_desc& da = list[adds[a]];
    const auto ya = span(da.y, da.m * da.n * 8);
    for (size_t j = 0; j < count && together; ++j) {
      const praghip_gemm_desc& d = list[j];
      if (!d.m || !d.n) continue;
      const size_t wbytes = d.n * d.k * (d.w_bits == 8 ? 1 : d.w_bits == 24 ? 3 : 4);
      if (overlaps(ya, span(d.x, d.m * d.k * 8)) || overlaps(ya, span(d.w, wbytes)) ||
          (d.shifts && overlaps(ya, span(d.shifts, d.n))) || (j != adds[a] && overlaps(ya, span(d.y, d.m * d.n * 8))))
        together = false;
    }
  }
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (together)
    for (size_t a0 = 0; a0 < adds.size() && e == hipSuccess; a0 += kGemmClearMax) {
      GemmClearList l{};
      for (size_t a = a0; a < adds.size() && l.count < kGemmClearMax; ++a) {
        l.ptr[l.count] = list[adds[a]].y;
        l.words[l.count++] = list[adds[a]].m * list[adds[a]].n;
      }
      e = launch_gemm_clear_list(l, static_cast<hipStream_t>(stream));
    }
  for (size_t i = 0; i < count && e == hipSuccess; ++i) {
    const praghip_gemm_desc& d = list[i];
    if (d.m == 0 || d.n == 0) continue;
    e = launch_share_gemm(d.x, d.w, d.w_bits, d.shifts, d.y, int(d.m), int(d.k), int(d.n), d.mask_bits,
                          static_cast<hipStream_t>(stream), together);
  }
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_SHARE_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

}  // extern "C"

// ========================================================= synthetic inputs
extern "C" {

int praghip_fill_residues(int device, uint64_t* data, size_t limbs, uint32_t log_n, const uint64_t* q,
                          size_t primes, uint64_t seed, void* stream) {
  if (!q || (!data && limbs)) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (primes < 1 || primes > size_t(kMaxKeyPrimes) || log_n > 20) return fail(PRAGHIP_E_SHAPE, "E_FILL_SHAPE");
  PrimeList pl{};
  for (size_t i = 0; i < primes; ++i) pl.q[i] = q[i];
  pl.count = int(primes);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess)
    e = launch_fill_residues(data, limbs << log_n, int(log_n), pl, seed, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_FILL_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

int praghip_fill_u64(int device, uint64_t* data, size_t count, uint64_t seed, void* stream) {
  if (!data && count) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_fill_u64(data, count, seed, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_FILL_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

int praghip_fill_shift(int device, int8_t* data, size_t count, uint64_t seed, void* stream) {
  if (!data && count) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_fill_shift(data, count, seed, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_FILL_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

int praghip_fill_i8(int device, int8_t* data, size_t count, uint64_t seed, void* stream) {
  if (!data && count) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_fill_i8(data, count, seed, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(PRAGHIP_E_DEVICE, std::string("E_FILL_HIP: ") + hipGetErrorString(e));
  return PRAGHIP_OK;
}

}  // extern "C"

// ======================================================== share-side kernels
namespace praghip::host {
// q must be an odd prime-sized modulus below 2^62 (Barrett-128 and the lift's
// q - 2^59 need q > 2^59 only for the reference's own primes; any q works).
bool valid_moduli(const uint64_t* q, size_t primes) {
  if (!q || primes < 1 || primes > size_t(kMaxKeyPrimes)) return false;
  for (size_t i = 0; i < primes; ++i)
    if (q[i] < 3 || q[i] >= (1ull << 62) || !(q[i] & 1)) return false;
  return true;
}
Barrett barrett_of(uint64_t q) {
  const u128 ratio = (~(u128)0) / q;
  return Barrett{q, uint64_t(ratio), uint64_t(ratio >> 64)};
}
int hip_fail(const char* what, hipError_t e) { return fail(PRAGHIP_E_DEVICE, std::string(what) + hipGetErrorString(e)); }
}  // namespace praghip::host

extern "C" {

int praghip_ring_add(int device, const uint64_t* a, const uint64_t* b, uint64_t* c, size_t n, int mask_bits,
                     void* stream) {
  if (n == 0) return PRAGHIP_OK;
  if (!a || !b || !c) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (mask_bits < 1 || mask_bits > 64) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_MASK");
  if (!aligned8(a) || !aligned8(b) || !aligned8(c) ||
      ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(c)) & 15))
    return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ring_add(a, b, c, n, mask_bits, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_CUDA_LOCAL: ", e);
}

int praghip_ring_scale(int device, const uint64_t* a, uint64_t factor, uint64_t* c, size_t n, int mask_bits,
                       void* stream) {
  if (n == 0) return PRAGHIP_OK;
  if (!a || !c) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (mask_bits < 1 || mask_bits > 64) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_MASK");
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(c)) & 15)
    return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ring_scale(a, factor, c, n, mask_bits, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_CUDA_LOCAL: ", e);
}

int praghip_ring_layout(int device, const uint64_t* a, size_t n_in, const uint64_t* map, uint64_t* c, size_t n_out,
                        void* stream) {
  if (n_out == 0) return PRAGHIP_OK;
  if (!a || !map || !c) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (n_in == 0) return fail(PRAGHIP_E_SHAPE, "E_CUDA_SHAPE");
  if (!aligned8(a) || !aligned8(map) || !aligned8(c)) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ring_layout(a, n_in, map, c, n_out, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_CUDA_LOCAL: ", e);
}

int praghip_ring_sum_rows(int device, const uint64_t* a, uint64_t* out, size_t rows, size_t cols, int mask_bits,
                          void* stream) {
  if (rows == 0) return PRAGHIP_OK;
  if (!a || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (cols == 0) return fail(PRAGHIP_E_SHAPE, "E_CUDA_SHAPE");
  if (mask_bits < 1 || mask_bits > 64) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_MASK");
  if (!aligned8(a) || !aligned8(out)) return fail(PRAGHIP_E_ARGUMENT, "E_SHARE_ALIGNMENT");
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ring_sum_rows(a, out, rows, cols, mask_bits, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_CUDA_LOCAL: ", e);
}

int praghip_lift59(int device, const uint64_t* ring, uint64_t* out, size_t blocks, uint32_t log_n, size_t width,
                   const uint64_t* q, size_t primes, void* stream) {
  if (blocks == 0) return PRAGHIP_OK;
  if (!ring || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (!valid_moduli(q, primes) || log_n < 1 || log_n > 17 || width > (size_t(1) << log_n))
    return fail(PRAGHIP_E_SHAPE, "E_LIFT_SHAPE");
  if (!aligned8(ring) || !aligned8(out)) return fail(PRAGHIP_E_ARGUMENT, "E_LIFT_ALIGNMENT");
  PrimeList pl{};
  for (size_t i = 0; i < primes; ++i) pl.q[i] = q[i];
  pl.count = int(primes);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_lift59(ring, out, blocks, int(log_n), width, pl, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_LIFT_HIP: ", e);
}

int praghip_dyadic_mac(int device, const uint64_t* a, const uint64_t* w, uint64_t* out, size_t blocks, size_t limbs,
                       uint32_t log_n, size_t w_limbs, const uint64_t* q, size_t primes, void* stream) {
  if (limbs == 0) return PRAGHIP_OK;
  if (!a || !w || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (!valid_moduli(q, primes) || blocks == 0 || w_limbs == 0 || log_n < 1 || log_n > 17)
    return fail(PRAGHIP_E_SHAPE, "E_DYADIC_SHAPE");
  if (!aligned8(a) || !aligned8(w) || !aligned8(out)) return fail(PRAGHIP_E_ARGUMENT, "E_DYADIC_ALIGNMENT");
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < primes; ++i) m[i] = barrett_of(q[i]);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess)
    e = launch_dyadic_mac(a, w, out, blocks, limbs, int(log_n), w_limbs, m, int(primes),
                          static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_DYADIC_HIP: ", e);
}

size_t praghip_local_dot_workspace_words(size_t slots) { return slots * kLocalTiles; }

int praghip_local_dot_scale(int device, const uint64_t* shares, const uint64_t* weights, size_t words, size_t slots,
                            const uint64_t* delta, uint64_t r, const uint64_t* q, size_t primes, uint64_t* scaled,
                            uint64_t* workspace, void* stream) {
  if (slots == 0) return PRAGHIP_OK;
  if (!shares || !weights || !delta || !scaled || !workspace) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (!valid_moduli(q, primes) || words == 0 || slots > 65535 || r >= (1ull << 59))
    return fail(PRAGHIP_E_SHAPE, "E_LOCAL_SHAPE");
  for (size_t k = 0; k < primes; ++k)
    if (delta[k] >= q[k]) return fail(PRAGHIP_E_CANONICAL, "E_LOCAL_DELTA");
  if (!aligned8(shares) || !aligned8(weights) || !aligned8(scaled) || !aligned8(workspace))
    return fail(PRAGHIP_E_ARGUMENT, "E_LOCAL_ALIGNMENT");
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < primes; ++i) m[i] = barrett_of(q[i]);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess)
    e = launch_local_dot_scale(shares, weights, words, slots, delta, r, m, int(primes), scaled, workspace,
                               static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_LOCAL_HIP: ", e);
}

// ============================================================ ShareStorage
// prag::model::ShareStorage from LocalShares::allocate (local_shares.hpp:12-17,
// 29; local_shares.cu:14-24): device words of one participant's shares,
// zero-filled on allocation; write/read are synchronous host copies on the
// storage's own stream; clear wipes, synchronises and frees.
}  // extern "C"

struct praghip_share_storage {
  int device = -1;
  size_t words = 0;
  Buffers buf;
  uint64_t* data = nullptr;
  hipStream_t stream = nullptr;
  praghip_cleanup cleanup{};
  uint64_t uploaded = 0, downloaded = 0;
  bool closing = false;
  void release() { release_all(device, buf, stream, nullptr, 0, cleanup, closing); }
  ~praghip_share_storage() { release(); }
};

namespace {
int storage_failure(praghip_share_storage* st, hipError_t e, const char* what) {
  st->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_CUDA_LOCAL: ") + what + ": " + hipGetErrorString(e));
}
int storage_range(const praghip_share_storage* st, size_t offset, size_t count) {
  if (!st) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (st->closing) return fail(PRAGHIP_E_CLOSED, "E_CUDA_STORAGE_CLOSED");
  if (offset > st->words || count > st->words - offset) return fail(PRAGHIP_E_SHAPE, "E_CUDA_SHAPE");
  return PRAGHIP_OK;
}
}  // namespace

extern "C" {

int praghip_storage_allocate(int device, size_t words, praghip_share_storage** out) {
  if (!out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = nullptr;
  if (words == 0 || words > SIZE_MAX / 8) return fail(PRAGHIP_E_SHAPE, "E_CUDA_SHAPE");
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_share_storage> st(new praghip_share_storage);
  st->device = device;
  st->words = words;
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&st->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = st->buf.alloc((void**)&st->data, words * 8, true);
  if (e == hipSuccess) e = hipMemsetAsync(st->data, 0, words * 8, st->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
  if (e != hipSuccess) return storage_failure(st.get(), e, "allocate");
  *out = st.release();
  return PRAGHIP_OK;
}

int praghip_storage_write(praghip_share_storage* st, size_t offset, const uint64_t* words, size_t count) {
  if (int rc = storage_range(st, offset, count)) return rc;
  if (count && !words) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  for (size_t i = 0; i < count; ++i)
    if (words[i] >> 59) return fail(PRAGHIP_E_CANONICAL, "E_CUDA_WORD");
  if (!count) return PRAGHIP_OK;
  DeviceScope scope(st->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipMemcpyAsync(st->data + offset, words, count * 8, hipMemcpyHostToDevice, st->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
  if (e != hipSuccess) return storage_failure(st, e, "write");
  st->uploaded += count * 8;
  return PRAGHIP_OK;
}

int praghip_storage_read(praghip_share_storage* st, size_t offset, size_t count, uint64_t* out) {
  if (int rc = storage_range(st, offset, count)) return rc;
  if (count && !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (!count) return PRAGHIP_OK;
  DeviceScope scope(st->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipMemcpyAsync(out, st->data + offset, count * 8, hipMemcpyDeviceToHost, st->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(st->stream);
  if (e != hipSuccess) {
    std::memset(out, 0, count * 8);
    return storage_failure(st, e, "read");
  }
  st->downloaded += count * 8;
  return PRAGHIP_OK;
}

int praghip_storage_data(praghip_share_storage* st, uint64_t** data, size_t* words) {
  if (!st || !data) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (st->closing) return fail(PRAGHIP_E_CLOSED, "E_CUDA_STORAGE_CLOSED");
  *data = st->data;
  if (words) *words = st->words;
  return PRAGHIP_OK;
}

int praghip_storage_stats(const praghip_share_storage* st, uint64_t* uploaded_bytes, uint64_t* downloaded_bytes) {
  if (!st) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (uploaded_bytes) *uploaded_bytes = st->uploaded;
  if (downloaded_bytes) *downloaded_bytes = st->downloaded;
  return PRAGHIP_OK;
}

int praghip_storage_clear(praghip_share_storage* st, praghip_cleanup* out) {
  if (!st) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  st->release();
  if (out) *out = st->cleanup;
  return PRAGHIP_OK;
}

void praghip_storage_destroy(praghip_share_storage* st) { delete st; }

int praghip_local_dot_scale_noalloc(int device, const uint64_t* shares, const uint64_t* weights, size_t words,
                                    size_t slots, const uint64_t* delta, uint64_t r, const uint64_t* q, size_t primes,
                                    uint64_t* scaled, void* stream) {
  if (slots == 0) return PRAGHIP_OK;
  if (!shares || !weights || !delta || !scaled) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (slots > kNoAllocSlots) return fail(PRAGHIP_E_SHAPE, "E_LOCAL_NOALLOC_SLOTS: at most 64 slots");
  if (!valid_moduli(q, primes) || words == 0 || r >= (1ull << 59)) return fail(PRAGHIP_E_SHAPE, "E_LOCAL_SHAPE");
  for (size_t k = 0; k < primes; ++k)
    if (delta[k] >= q[k]) return fail(PRAGHIP_E_CANONICAL, "E_LOCAL_DELTA");
  if (!aligned8(shares) || !aligned8(weights) || !aligned8(scaled)) return fail(PRAGHIP_E_ARGUMENT, "E_LOCAL_ALIGNMENT");
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < primes; ++i) m[i] = barrett_of(q[i]);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  uint64_t* work = nullptr;
  if (e == hipSuccess) e = local_dot_scratch(device, &work);
  if (e == hipSuccess)
    e = launch_local_dot_scale(shares, weights, words, slots, delta, r, m, int(primes), scaled, work,
                               static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PRAGHIP_OK : hip_fail("E_LOCAL_HIP: ", e);
}

}  // extern "C"

