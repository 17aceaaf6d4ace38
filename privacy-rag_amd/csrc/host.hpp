// Host-side helpers shared by the C ABI sources (api.cpp, plans.cpp): error
// slot, number theory for tables and constants, device scoping, the plans'
// allocation registry and wipe-on-release, NTT table upload, argument checks.
// Internal to the library; not part of include/praghip.h.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "praghip.h"
#include "kernels.hpp"

namespace praghip {
int set_error(int code, const std::string& text);
}

namespace praghip::host {

using u128 = unsigned __int128;

// Records `text` as praghip_last_error() and returns `code`.
int fail(int code, const std::string& text);

// ------------------------------------------------------------ number theory
uint64_t mulmod(uint64_t a, uint64_t b, uint64_t q);
uint64_t invmod(uint64_t a, uint64_t q);  // q prime
bool is_prime(uint64_t n);
uint64_t shoup_q(uint64_t w, uint64_t q);  // floor(w 2^64 / q)
// SEAL NTTTables of q at 2^log_n: [N][2] (operand, quotient) pairs; false
// without a 2N-th root.
bool make_tables(uint64_t q, unsigned log_n, uint64_t* fwd, uint64_t* inv, uint64_t* invn, uint64_t* psi_out);
Barrett barrett_of(uint64_t q);

// --------------------------------------------------------------- device side
class DeviceScope {
 public:
  explicit DeviceScope(int target) {
    status_ = hipGetDevice(&previous_);
    if (status_ == hipSuccess && previous_ != target) {
      status_ = hipSetDevice(target);
      restore_ = status_ == hipSuccess;
    }
  }
  ~DeviceScope() {
    if (restore_) (void)hipSetDevice(previous_);
  }
  hipError_t status() const { return status_; }

 private:
  int previous_ = 0;
  bool restore_ = false;
  hipError_t status_ = hipSuccess;
};

// E_GFX950_REQUIRED / E_DEVICE_INDEX unless `device` is a gfx950 device.
int check_device(int device);

// Allocation registry: every device buffer of a plan, sensitive or public.
struct Buffers {
  struct Entry {
    void** slot;
    size_t bytes;
    bool sensitive;
  };
  std::vector<Entry> entries;
  hipError_t alloc(void** slot, size_t bytes, bool sensitive) {
    *slot = nullptr;
    if (!bytes) return hipSuccess;
    const hipError_t e = hipMalloc(slot, bytes);
    if (e == hipSuccess) entries.push_back({slot, bytes, sensitive});
    return e;
  }
  size_t sensitive_bytes() const {
    size_t s = 0;
    for (auto& e : entries) s += e.sensitive ? e.bytes : 0;
    return s;
  }
  size_t total_bytes() const {
    size_t s = 0;
    for (auto& e : entries) s += e.bytes;
    return s;
  }
};

// Wipes the sensitive buffers, synchronises, frees everything, destroys the
// events and the stream; fills `c` (closed only if every step succeeded).
void release_all(int device, Buffers& buf, hipStream_t& stream, hipEvent_t* events, int nevents, praghip_cleanup& c,
                 bool& closing);

struct NttHost {
  std::vector<NttPrime> primes;
  std::vector<ulonglong2> fwd_u, inv_u;
  std::vector<double> fwd_f, inv_f;
};

int build_ntt_host(const uint64_t* q, size_t P, unsigned log_n, const uint64_t* fwd_in, const uint64_t* inv_in,
                   const uint64_t* invn_in, NttHost& h);
hipError_t upload_ntt(const NttHost& h, unsigned log_n, Buffers& buf, NttDevice& d, hipStream_t s);

// Device-pointer entry points run on the caller's stream as given.
inline hipStream_t pick(void* stream) { return static_cast<hipStream_t>(stream); }
void wipe_host(std::vector<uint64_t>& v);

// ------------------------------------------------------------------ checks
// every word below its limb's prime (limb l of 2^log_n words uses q[l % P])
bool canonical(const uint64_t* v, size_t words, const std::vector<uint64_t>& q, unsigned log_n);
// Galois element odd and < 2N; its inverse mod 2N
bool galois_inverse(uint32_t g, unsigned log_n, uint32_t& ginv);
int build_ks_const(const uint64_t* q, size_t L, size_t dnum, unsigned log_n, KsConst& kc);
bool valid_moduli(const uint64_t* q, size_t primes);
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }
int hip_fail(const char* what, hipError_t e);

}  // namespace praghip::host
