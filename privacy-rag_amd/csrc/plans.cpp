// C ABI of the plans composed from the kernels (include/praghip.h): the HE
// matrix product, the public-key encryption of zero, the token-resident path
// and the acyclic packing tree.  Same conventions as api.cpp: validation
// before any device work, release on a HIP error, idempotent close().
#include <hip/hip_runtime.h>

#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "praghip.h"
#include "host.hpp"
#include "kernels.hpp"

using namespace praghip;
using namespace praghip::host;

// ============================================================== Matrix plan
// matrix_gpu::Matrix (matrix.hpp:9-24, matrix.cu:48-81): ciphertext blocks
// held in NTT form; evaluate(ring) = INTT( sum_b NTT(ct_b) (.) NTT(lift(ring_b)) ).
struct praghip_matrix_plan {
  int device = -1;
  unsigned log_n = 0;
  size_t P = 0, blocks = 0;
  std::vector<uint64_t> host_q;
  Buffers buf;
  NttDevice d;
  uint64_t *input = nullptr, *ring = nullptr, *weight = nullptr, *output = nullptr;
  size_t batch_cap = 0;
  uint64_t* bweight = nullptr;  // [batch_cap][blocks][P][N] transformed weight limbs
  uint64_t* indices = nullptr;  // [512] target coefficients of a selective batch
  hipStream_t stream = nullptr;
  hipEvent_t ev[1] = {};
  praghip_cleanup cleanup{};
  bool closing = false;
  void release() { release_all(device, buf, stream, ev, 1, cleanup, closing); }
  ~praghip_matrix_plan() { release(); }
};

namespace {
int matrix_failure(praghip_matrix_plan* p, hipError_t e, const char* what) {
  p->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_MATRIX_HIP: ") + what + ": " + hipGetErrorString(e));
}
PrimeList host_primes(const praghip_matrix_plan* p) {
  PrimeList pl{};
  for (size_t i = 0; i < p->P; ++i) pl.q[i] = p->host_q[i];
  pl.count = int(p->P);
  return pl;
}
// lift + NTT (one pass) -> sum of products -> INTT, all on the plan's device buffers
hipError_t matrix_run(praghip_matrix_plan* p, const uint64_t* ring_dev, uint64_t* out_dev, hipStream_t s) {
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < p->P; ++i) m[i] = barrett_of(p->host_q[i]);
  hipError_t e = launch_ntt_lift(ring_dev, 0, p->weight, p->blocks, host_primes(p), p->d, s);
  if (e == hipSuccess)
    e = launch_dyadic_mac(p->input, p->weight, out_dev, p->blocks, 2 * p->P, int(p->log_n), p->P, m, int(p->P), s);
  if (e == hipSuccess) e = launch_ntt(true, out_dev, 2 * p->P, p->d, s);
  return e;
}
}  // namespace

extern "C" {

int praghip_matrix_plan_create(int device, const uint64_t* q, size_t primes, uint32_t log_n, const uint64_t* input,
                               size_t blocks, praghip_matrix_plan** plan) {
  if (!plan || !q || !input) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *plan = nullptr;
  if (log_n < 4 || log_n > 14 || primes < 1 || primes > size_t(kMaxKeyPrimes) || blocks < 1 || blocks > 4096)
    return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_SHAPE");
  NttHost h;
  if (int rc = build_ntt_host(q, primes, log_n, nullptr, nullptr, nullptr, h)) return rc;
  const size_t n = size_t(1) << log_n, in_words = blocks * 2 * primes * n;
  std::vector<uint64_t> qv(q, q + primes);
  if (!canonical(input, in_words, qv, log_n)) return fail(PRAGHIP_E_CANONICAL, "E_NTT_CANONICAL_REQUIRED");
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_matrix_plan> p(new praghip_matrix_plan);
  p->device = device;
  p->log_n = log_n;
  p->P = primes;
  p->blocks = blocks;
  p->host_q = qv;
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&p->ev[0]);
  if (e == hipSuccess) e = upload_ntt(h, log_n, p->buf, p->d, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->input, in_words * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->ring, blocks * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->weight, blocks * primes * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->output, 2 * primes * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->indices, kMaxTargets * 8, false);
  if (e == hipSuccess) e = hipMemcpyAsync(p->input, input, in_words * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = launch_ntt(false, p->input, blocks * 2 * primes, p->d, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return matrix_failure(p.get(), e, "create");
  *plan = p.release();
  return PRAGHIP_OK;
}

int praghip_matrix_evaluate(praghip_matrix_plan* p, const uint64_t* ring, uint64_t* output, const uint64_t* targets,
                            size_t count) {
  if (!p || !ring || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "MATRIX_GPU_CLOSED");
  const size_t n = size_t(1) << p->log_n, ring_words = p->blocks * n, out_words = 2 * p->P * n;
  if (targets) {  // evaluate_selective (matrix.cu:69-73)
    if (count == 0 || count > 512) return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_TARGET_COUNT");
    for (size_t i = 0; i < count; ++i)
      if (targets[i] >= n || (i && targets[i] <= targets[i - 1])) return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_TARGET_INDEX");
  }
  for (size_t i = 0; i < ring_words; ++i)
    if (ring[i] >> 59) return fail(PRAGHIP_E_CANONICAL, "MATRIX_GPU_RING");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipMemcpyAsync(p->ring, ring, ring_words * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = matrix_run(p, p->ring, p->output, p->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(output, p->output, out_words * 8, hipMemcpyDeviceToHost, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) {
    volatile uint64_t* o = output;
    for (size_t i = 0; i < out_words; ++i) o[i] = 0;
    return matrix_failure(p, e, "evaluate");
  }
  if (targets) {  // c0 keeps only the target coefficients; c1 is complete
    std::vector<uint8_t> keep(n, 0);
    for (size_t i = 0; i < count; ++i) keep[targets[i]] = 1;
    for (size_t k = 0; k < p->P; ++k)
      for (size_t z = 0; z < n; ++z)
        if (!keep[z]) output[k * n + z] = 0;
  }
  return PRAGHIP_OK;
}

int praghip_matrix_evaluate_device(praghip_matrix_plan* p, const uint64_t* ring, uint64_t* output, void* stream) {
  if (!p || !ring || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "MATRIX_GPU_CLOSED");
  if ((reinterpret_cast<uintptr_t>(ring) | reinterpret_cast<uintptr_t>(output)) & 15)
    return fail(PRAGHIP_E_ARGUMENT, "MATRIX_GPU_ALIGNMENT");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = matrix_run(p, ring, output, pick(stream));
  if (e != hipSuccess) return matrix_failure(p, e, "evaluate");
  return PRAGHIP_OK;
}

int praghip_matrix_reserve(praghip_matrix_plan* p, size_t groups) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "MATRIX_GPU_CLOSED");
  if (groups == 0 || groups > 4096) return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_BATCH");
  if (groups <= p->batch_cap) return PRAGHIP_OK;
  if (p->batch_cap) return fail(PRAGHIP_E_STATE, "MATRIX_GPU_BATCH_RESERVED");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->bweight, groups * p->blocks * p->P * (size_t(8) << p->log_n), true);
  if (e != hipSuccess) return matrix_failure(p, e, "reserve");
  p->batch_cap = groups;
  return PRAGHIP_OK;
}

}  // extern "C"

namespace {
// Target list of evaluate_selective (matrix.cu:65-68): 1..512 strictly
// increasing coefficient indices below N.
int check_targets(const uint64_t* targets, size_t count, size_t n) {
  if (count == 0 || count > kMaxTargets) return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_TARGET_COUNT");
  for (size_t i = 0; i < count; ++i)
    if (targets[i] >= n || (i && targets[i] <= targets[i - 1])) return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_TARGET_INDEX");
  return PRAGHIP_OK;
}
}  // namespace

// Many output groups per call: lift and transform every group's weight limbs,
// one column-batched sum of products over the resident blocks, one inverse
// transform over all outputs.  With targets: the device-side selective form
// (c0 kept at the targets only, gathered into `selected`).
static int matrix_batch(praghip_matrix_plan* p, const uint64_t* rings, uint64_t* output, size_t groups,
                        const uint64_t* targets, size_t count, uint64_t* selected, void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "MATRIX_GPU_CLOSED");
  if (targets)
    if (int rc = check_targets(targets, count, size_t(1) << p->log_n)) return rc;
  if (groups == 0) return PRAGHIP_OK;
  if (!rings || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (groups > p->batch_cap) return fail(PRAGHIP_E_SHAPE, "MATRIX_GPU_BATCH");
  if ((reinterpret_cast<uintptr_t>(rings) | reinterpret_cast<uintptr_t>(output) |
       reinterpret_cast<uintptr_t>(selected)) & 15)
    return fail(PRAGHIP_E_ARGUMENT, "MATRIX_GPU_ALIGNMENT");
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < p->P; ++i) m[i] = barrett_of(p->host_q[i]);
  const hipStream_t s = pick(stream);
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ntt_lift(rings, 0, p->bweight, groups * p->blocks, host_primes(p), p->d, s);
  if (e == hipSuccess)
    e = launch_token_mac(p->input, p->bweight, output, groups, p->blocks, 2 * p->P, int(p->log_n), m, int(p->P), s);
  if (e == hipSuccess) e = launch_ntt(true, output, groups * 2 * p->P, p->d, s);
  if (e == hipSuccess && targets) e = hipMemcpyAsync(p->indices, targets, count * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && targets)
    e = launch_select_c0(output, groups, int(p->P), int(p->log_n), p->indices, unsigned(count), selected, s);
  if (e != hipSuccess) return matrix_failure(p, e, "evaluate_device_batch");
  return PRAGHIP_OK;
}

extern "C" {

int praghip_matrix_evaluate_device_batch(praghip_matrix_plan* p, const uint64_t* rings, uint64_t* output,
                                         size_t groups, void* stream) {
  return matrix_batch(p, rings, output, groups, nullptr, 0, nullptr, stream);
}

int praghip_matrix_evaluate_device_batch_selective(praghip_matrix_plan* p, const uint64_t* rings, uint64_t* output,
                                                   size_t groups, const uint64_t* targets, size_t count,
                                                   uint64_t* selected, void* stream) {
  if (!targets) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  return matrix_batch(p, rings, output, groups, targets, count, selected, stream);
}

// The cost model that sizes a packed matrix product (bfv_layout.hpp:8-27):
// for a batch of b rows, inner dimension k and o outputs, every power-of-two
// reduction width d in [16, 8192/b] packs up to cap = min(512/b, 8192/(b d))
// output columns per returned ciphertext; the choice minimises the bytes moved,
// ceil(k/d) input ciphertexts of 1,572,960 B plus the returned ciphertexts of
// 786,528 B, the first (smallest) d winning ties.  qk_reverse64 is the
// dedicated single-output product of 128 terms, for b <= 64.
int praghip_matrix_packing(size_t batch, size_t inner, size_t outputs, int qk_reverse64, praghip_matrix_packing_t* out) {
  if (!out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = praghip_matrix_packing_t{0, 0, 0, 0};
  if (qk_reverse64) {
    if (batch == 0 || batch > 64) return fail(PRAGHIP_E_SHAPE, "E_QK_REVERSE64_SHAPE");
    *out = praghip_matrix_packing_t{128, 1, 1, 1};
    return PRAGHIP_OK;
  }
  if (batch == 0 || batch > 16 || inner == 0 || inner > 8192 || outputs == 0 || outputs > 155648)
    return fail(PRAGHIP_E_SHAPE, "E_MATRIX_SHAPE");
  const uint64_t kInputBytes = 1572960, kReturnBytes = 786528;
  const size_t per_group = 512 / batch;  // output columns one packed group holds
  const size_t whole = outputs / per_group, rest = outputs % per_group;
  uint64_t best = ~uint64_t(0);
  for (size_t width = 16; width <= 8192 / batch; width <<= 1) {
    const size_t cap = std::min(per_group, 8192 / (batch * width));
    const size_t returns = whole * ((per_group + cap - 1) / cap) + (rest ? (rest + cap - 1) / cap : 0);
    const size_t inputs = (inner + width - 1) / width;
    const uint64_t bytes = inputs * kInputBytes + returns * kReturnBytes;
    if (bytes < best) {
      best = bytes;
      *out = praghip_matrix_packing_t{width, cap, returns, inputs};
    }
  }
  return PRAGHIP_OK;
}

size_t praghip_matrix_device_bytes(const praghip_matrix_plan* p) { return p ? p->buf.total_bytes() : 0; }

int praghip_matrix_close(praghip_matrix_plan* p, praghip_cleanup* out) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  p->release();
  if (out) *out = p->cleanup;
  return PRAGHIP_OK;
}

void praghip_matrix_destroy(praghip_matrix_plan* p) { delete p; }

}  // extern "C"

// ================================================================ Enc0 plan
// prag::enc0_gpu::PublicZero (enc0.hpp:15-25, enc0.cu:99-114): the public key
// resident in NTT form; evaluate(samples) = ModDown(INTT(NTT(u) (.) pk) + e).
struct praghip_enc0_plan {
  int device = -1;
  unsigned log_n = 0;
  size_t L = 0, K = 0;
  std::vector<uint64_t> host_q;
  Buffers buf;
  NttDevice d;
  Enc0Const kc{};
  uint64_t *pk = nullptr, *samples = nullptr, *expanded = nullptr, *prod = nullptr, *out = nullptr;
  size_t batch_cap = 0;
  uint64_t *bu = nullptr, *bprod = nullptr;  // [batch_cap][K][N] NTT(u), [batch_cap][2][K][N] products
  hipStream_t stream = nullptr;
  hipEvent_t ev[1] = {};
  praghip_cleanup cleanup{};
  bool closing = false;
  void release() { release_all(device, buf, stream, ev, 1, cleanup, closing); }
  ~praghip_enc0_plan() { release(); }
};

namespace {
int enc0_failure(praghip_enc0_plan* p, hipError_t e, const char* what) {
  p->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_ENC0_HIP: ") + what + ": " + hipGetErrorString(e));
}
// samples [3][K][N] on the device -> out [2][L][N]
hipError_t enc0_run(praghip_enc0_plan* p, const uint64_t* samples, uint64_t* out, hipStream_t s) {
  const size_t n = size_t(1) << p->log_n, K = p->K;
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < K; ++i) m[i] = barrett_of(p->host_q[i]);
  hipError_t e = hipMemcpyAsync(p->expanded, samples, K * n * 8, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess) e = launch_ntt(false, p->expanded, K, p->d, s);
  // prod[c][t] = pk[c][t] (.) NTT(u)[t]: the MAC with one block, u broadcast over both components
  if (e == hipSuccess) e = launch_dyadic_mac(p->pk, p->expanded, p->prod, 1, 2 * K, int(p->log_n), K, m, int(K), s);
  if (e == hipSuccess) e = launch_ntt(true, p->prod, 2 * K, p->d, s);
  if (e == hipSuccess) e = launch_enc0_moddown(p->prod, samples + K * n, out, p->kc, s);
  return e;
}
}  // namespace

extern "C" {

int praghip_enc0_plan_create(int device, const uint64_t* q, size_t data_primes, uint32_t log_n, const uint64_t* pk,
                             praghip_enc0_plan** plan) {
  if (!plan || !q || !pk) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *plan = nullptr;
  const size_t L = data_primes, K = L + 1;
  if (log_n < 4 || log_n > 14 || L < 1 || K > size_t(kMaxKeyPrimes)) return fail(PRAGHIP_E_SHAPE, "E_SWITCH_SHAPE");
  NttHost h;
  if (int rc = build_ntt_host(q, K, log_n, nullptr, nullptr, nullptr, h)) return rc;
  const size_t n = size_t(1) << log_n;
  std::vector<uint64_t> qv(q, q + K);
  if (!canonical(pk, 2 * K * n, qv, log_n)) return fail(PRAGHIP_E_CANONICAL, "E_NTT_CANONICAL_REQUIRED");
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_enc0_plan> p(new praghip_enc0_plan);
  p->device = device;
  p->log_n = log_n;
  p->L = L;
  p->K = K;
  p->host_q = qv;
  p->kc.L = int(L);
  p->kc.log_n = int(log_n);
  const uint64_t sp = q[L];
  for (size_t i = 0; i < K; ++i) p->kc.q[i] = q[i];
  for (size_t i = 0; i < L; ++i) {
    const uint64_t ip = invmod(sp % q[i], q[i]);
    p->kc.invp[i] = Shoup{ip, shoup_q(ip, q[i])};
    p->kc.half_mod[i] = (sp >> 1) % q[i];
    p->kc.one_q[i] = shoup_q(1, q[i]);
  }
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&p->ev[0]);
  if (e == hipSuccess) e = upload_ntt(h, log_n, p->buf, p->d, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->pk, 2 * K * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->samples, 3 * K * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->expanded, K * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->prod, 2 * K * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->out, 2 * L * n * 8, true);
  if (e == hipSuccess) e = hipMemcpyAsync(p->pk, pk, 2 * K * n * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return enc0_failure(p.get(), e, "create");
  *plan = p.release();
  return PRAGHIP_OK;
}

int praghip_enc0_evaluate(praghip_enc0_plan* p, const uint64_t* samples, uint64_t* output) {
  if (!p || !samples || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  const size_t n = size_t(1) << p->log_n, words = 3 * p->K * n, out_words = 2 * p->L * n;
  if (!canonical(samples, words, p->host_q, p->log_n)) return fail(PRAGHIP_E_CANONICAL, "E_ENC0_SAMPLE_CANONICAL");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipMemcpyAsync(p->samples, samples, words * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = enc0_run(p, p->samples, p->out, p->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(output, p->out, out_words * 8, hipMemcpyDeviceToHost, p->stream);
  // the one-time samples and every intermediate are wiped after use (enc0.cu:112)
  for (uint64_t* b : {p->samples, p->expanded, p->prod, p->out}) {
    const size_t bytes = b == p->samples ? words * 8 : b == p->expanded ? p->K * n * 8
                         : b == p->prod  ? 2 * p->K * n * 8 : out_words * 8;
    if (e == hipSuccess) e = hipMemsetAsync(b, 0, bytes, p->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) {
    volatile uint64_t* o = output;
    for (size_t i = 0; i < out_words; ++i) o[i] = 0;
    return enc0_failure(p, e, "evaluate");
  }
  return PRAGHIP_OK;
}

int praghip_enc0_evaluate_device(praghip_enc0_plan* p, const uint64_t* samples, uint64_t* output, void* stream) {
  if (!p || !samples || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  if ((reinterpret_cast<uintptr_t>(samples) | reinterpret_cast<uintptr_t>(output)) & 15)
    return fail(PRAGHIP_E_ARGUMENT, "E_ENC0_ALIGNMENT");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = enc0_run(p, samples, output, pick(stream));
  if (e != hipSuccess) return enc0_failure(p, e, "evaluate");
  return PRAGHIP_OK;
}

int praghip_enc0_reserve(praghip_enc0_plan* p, size_t count) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  if (count == 0 || count > 4096) return fail(PRAGHIP_E_SHAPE, "E_ENC0_BATCH");
  if (count <= p->batch_cap) return PRAGHIP_OK;
  if (p->batch_cap) return fail(PRAGHIP_E_STATE, "E_ENC0_BATCH_RESERVED");
  const size_t limb = size_t(8) << p->log_n;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->bu, count * p->K * limb, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->bprod, count * 2 * p->K * limb, true);
  if (e != hipSuccess) return enc0_failure(p, e, "reserve");
  p->batch_cap = count;
  return PRAGHIP_OK;
}

// Many encryptions per call: every u transformed in one launch, the products
// with both key components as one column-batched product (the public key is
// the single resident block), one inverse transform, one noise-add + ModDown.
int praghip_enc0_evaluate_device_batch(praghip_enc0_plan* p, const uint64_t* samples, uint64_t* output, size_t count,
                                       void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_SWITCH_CLOSED");
  if (count == 0) return PRAGHIP_OK;
  if (!samples || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (count > p->batch_cap) return fail(PRAGHIP_E_SHAPE, "E_ENC0_BATCH");
  if ((reinterpret_cast<uintptr_t>(samples) | reinterpret_cast<uintptr_t>(output)) & 15)
    return fail(PRAGHIP_E_ARGUMENT, "E_ENC0_ALIGNMENT");
  const size_t n = size_t(1) << p->log_n, K = p->K, sample_words = 3 * K * n;
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < K; ++i) m[i] = barrett_of(p->host_q[i]);
  const hipStream_t s = pick(stream);
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  // u of every encryption: rows of K N words, sample_words apart
  if (e == hipSuccess)
    e = hipMemcpy2DAsync(p->bu, K * n * 8, samples, sample_words * 8, K * n * 8, count, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess) e = launch_ntt(false, p->bu, count * K, p->d, s);
  if (e == hipSuccess)
    e = launch_token_mac(p->pk, p->bu, p->bprod, count, 1, 2 * K, int(p->log_n), m, int(K), s);
  if (e == hipSuccess) e = launch_ntt(true, p->bprod, count * 2 * K, p->d, s);
  if (e == hipSuccess) e = launch_enc0_moddown(p->bprod, samples + K * n, output, p->kc, s, count, sample_words);
  if (e != hipSuccess) return enc0_failure(p, e, "evaluate_device_batch");
  return PRAGHIP_OK;
}

int praghip_enc0_close(praghip_enc0_plan* p, praghip_cleanup* out) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  p->release();
  if (out) *out = p->cleanup;
  return PRAGHIP_OK;
}

void praghip_enc0_destroy(praghip_enc0_plan* p) { delete p; }

}  // extern "C"

// ============================================================== Packing plan
// prag::experimental_full_switch::Packing (bfv_gpu_packing.hpp:10-45): the
// 2 x levels switching keys of the acyclic packing tree held on the device.
// A pair at level l is  ks_{l,0}(L + x^s R) + ks_{l,1}(sigma_g(L - x^s R)),
// s = N >> (l + 1), g = 2^(l+1) + 1 (switch.cu:49-61, 157-185).  Both switches
// of every pair in a call run as ONE batched keyswitch: the prepared sums
// first, then the Galois-mapped differences, each half sharing its key.
struct praghip_pack_plan {
  int device = -1;
  unsigned log_n = 0;
  size_t L = 0, K = 0, dnum = 0, levels = 0, max_pairs = 0, key_words = 0;
  std::vector<uint64_t> host_q;
  Buffers buf;
  NttDevice d;
  KsConst kc{};
  KsConst* kc_dev = nullptr;
  uint64_t *keys = nullptr, *work = nullptr, *ksout = nullptr, *prod = nullptr, *acc = nullptr, *inter = nullptr;
  uint64_t *host_in = nullptr, *host_out = nullptr;
  size_t inter_cts = 0;
  unsigned* queue = nullptr;
  unsigned acc_slots = 0;
  size_t merges = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev[2] = {};
  praghip_timing timing{};
  praghip_cleanup cleanup{};
  bool closing = false;
  void release() { release_all(device, buf, stream, ev, 2, cleanup, closing); }
  ~praghip_pack_plan() { release(); }
};

namespace {
int pack_failure(praghip_pack_plan* p, hipError_t e, const char* what) {
  p->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_PACK_HIP: ") + what + ": " + hipGetErrorString(e));
}
// `count` pairs at one level; pair e reads left/right at
// ((e / group) * stride + e % group) ciphertexts from its base and is written
// to out + e ciphertexts.  Chunks of max_pairs pairs; each chunk reads its
// inputs before writing its outputs, and chunk outputs never land on inputs
// of a later chunk when out <= left (the tree reduces in place).
hipError_t pack_run(praghip_pack_plan* p, const uint64_t* left, const uint64_t* right, size_t count, size_t group,
                    size_t stride, unsigned level, uint64_t* out, hipStream_t s) {
  const size_t n = size_t(1) << p->log_n, ct = 2 * p->L * n;
  PrimeList pl{};
  for (size_t i = 0; i < p->L; ++i) pl.q[i] = p->host_q[i];
  pl.count = int(p->L);
  const size_t shift = n >> (level + 1);
  uint32_t ginv = 1;
  galois_inverse((2u << level) + 1, p->log_n, ginv);  // g = 2^(level+1) + 1 is odd and < 2N
  hipError_t e = hipSuccess;
  for (size_t c0 = 0; c0 < count && e == hipSuccess; c0 += p->max_pairs) {
    const size_t c = std::min(p->max_pairs, count - c0);
    uint64_t* sum = p->work;
    uint64_t* diff = p->work + c * ct;
    e = launch_pack_prepare(left, right, sum, diff, c, c0, group, stride, pl, int(p->log_n), shift, ginv, s);
    if (e != hipSuccess) break;
    KsArgs a;
    a.in = p->work;
    a.out = p->ksout;
    a.key = p->keys + size_t(2 * level) * p->key_words;
    a.key_stride = p->key_words;
    a.key_group = c;
    a.acc = p->acc;
    a.acc_slots = p->acc_slots;
    a.prod = p->prod;
    a.batch = 2 * c;
    a.galois_inv = 1;  // the Galois map is applied by the prepare kernel
    a.queue = p->queue;
    a.inter = p->inter;
    a.inter_cts = p->inter_cts;
    e = launch_keyswitch(a, p->kc_dev, p->kc, p->d, s);
    if (e == hipSuccess) e = launch_pack_finish(p->ksout, p->ksout + c * ct, out + c0 * ct, c, pl, int(p->log_n), s);
  }
  return e;
}
}  // namespace

extern "C" {

// packed_target (bfv_acyclic_pack.hpp:53-56): the coefficient a coordinate's
// constant term reaches after the packing tree over 2^levels leaves, its low
// `levels` bits reversed, times N >> levels (the reference: 9 levels at
// N = 16384, spacing 32).
int praghip_packed_target(size_t coordinate, unsigned levels, uint32_t log_n, uint64_t* target) {
  if (!target) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (log_n < 1 || log_n > 14 || levels < 1 || levels > log_n) return fail(PRAGHIP_E_SHAPE, "E_PACK_KEY_LEVELS");
  uint64_t r = 0;
  for (unsigned j = 0; j < levels; ++j) r = (r << 1) | ((coordinate >> j) & 1);
  *target = r << (log_n - levels);
  return PRAGHIP_OK;
}

int praghip_pack_plan_create(int device, const uint64_t* q, size_t data_primes, uint32_t log_n, size_t dnum,
                             size_t levels, const uint64_t* keys, size_t max_pairs, praghip_pack_plan** plan) {
  if (!plan || !q || !keys) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *plan = nullptr;
  const size_t L = data_primes, K = L + 1;
  if (log_n < 4 || log_n > 14 || L < 1 || K > size_t(kMaxKeyPrimes) || dnum < 1 || dnum > L || max_pairs < 1 ||
      max_pairs > 4096)
    return fail(PRAGHIP_E_SHAPE, "E_SWITCH_SHAPE");
  if (levels < 1 || levels > log_n) return fail(PRAGHIP_E_SHAPE, "E_PACK_KEY_LEVELS");
  NttHost h;
  if (int rc = build_ntt_host(q, K, log_n, nullptr, nullptr, nullptr, h)) return rc;
  const size_t n = size_t(1) << log_n, key_words = dnum * 2 * K * n, ct = 2 * L * n;
  for (size_t i = 0, total = 2 * levels * key_words; i < total; ++i)
    if (keys[i] >= q[(i >> log_n) % K]) return fail(PRAGHIP_E_CANONICAL, "E_SWITCH_KEY_CANONICAL");
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_pack_plan> p(new praghip_pack_plan);
  p->device = device;
  p->log_n = log_n;
  p->L = L;
  p->K = K;
  p->dnum = dnum;
  p->levels = levels;
  p->max_pairs = max_pairs;
  p->key_words = key_words;
  p->host_q.assign(q, q + K);
  build_ks_const(q, L, dnum, log_n, p->kc);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  for (auto& ev : p->ev)
    if (e == hipSuccess) e = hipEventCreate(&ev);
  if (e == hipSuccess) e = upload_ntt(h, log_n, p->buf, p->d, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->kc_dev, sizeof(KsConst), false);
  if (e == hipSuccess) e = hipMemcpyAsync(p->kc_dev, &p->kc, sizeof(KsConst), hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->keys, 2 * levels * key_words * 8, true);
  if (e == hipSuccess) e = hipMemcpyAsync(p->keys, keys, 2 * levels * key_words * 8, hipMemcpyHostToDevice, p->stream);
  // the fused kernel's running sums and work queue, only for shapes the
  // three-phase kernels do not take (they never touch either)
  const bool fused = !keyswitch_rows_supported(p->kc);
  if (e == hipSuccess && fused) {
    p->acc_slots = ks_acc_slots(int(log_n));
    e = p->acc_slots ? p->buf.alloc((void**)&p->acc, size_t(p->acc_slots) * 2 * n * 8, true) : hipErrorInvalidValue;
  }
  if (e == hipSuccess && fused) e = p->buf.alloc((void**)&p->queue, kQueueWords * 4, false);
  if (e == hipSuccess && fused) e = hipMemsetAsync(p->queue, 0, kQueueWords * 4, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->work, 2 * max_pairs * ct * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->ksout, 2 * max_pairs * ct * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->prod, 2 * max_pairs * 2 * K * n * 8, true);
  if (e == hipSuccess && keyswitch_rows_supported(p->kc)) {
    p->inter_cts = std::min(2 * max_pairs, kKsRowsChunk);
    e = p->buf.alloc((void**)&p->inter, p->inter_cts * dnum * K * n * 8, true);
  }
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->host_in, 2 * ct * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->host_out, ct * 8, true);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return pack_failure(p.get(), e, "create");
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  *plan = p.release();
  return PRAGHIP_OK;
}

int praghip_pack_pair(praghip_pack_plan* p, const uint64_t* left, const uint64_t* right, unsigned level,
                      uint64_t* output) {
  if (!p || !left || !right || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_PACK_CLOSED");
  if (level >= p->levels) return fail(PRAGHIP_E_SHAPE, "E_PACK_LEVEL");
  const size_t n = size_t(1) << p->log_n, ct = 2 * p->L * n;
  const std::vector<uint64_t> dq(p->host_q.begin(), p->host_q.begin() + p->L);
  if (!canonical(left, ct, dq, p->log_n) || !canonical(right, ct, dq, p->log_n))
    return fail(PRAGHIP_E_CANONICAL, "E_PACK_CIPHERTEXT");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  hipStream_t s = p->stream;
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], s);
  if (e == hipSuccess) e = hipMemcpyAsync(p->host_in, left, ct * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipMemcpyAsync(p->host_in + ct, right, ct * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = pack_run(p, p->host_in, p->host_in + ct, 1, 1, 0, level, p->host_out, s);
  if (e == hipSuccess) e = hipMemcpyAsync(output, p->host_out, ct * 8, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], s);
  if (e == hipSuccess) e = hipEventSynchronize(p->ev[1]);
  float ms = 0;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, p->ev[0], p->ev[1]);
  if (e != hipSuccess) {
    volatile uint64_t* o = output;
    for (size_t i = 0; i < ct; ++i) o[i] = 0;
    return pack_failure(p, e, "pair");
  }
  p->timing.kernel_ms = ms;
  ++p->merges;
  return PRAGHIP_OK;
}

int praghip_pack_pair_device(praghip_pack_plan* p, const uint64_t* left, const uint64_t* right, size_t count,
                             unsigned level, uint64_t* output, void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing || level >= p->levels) return fail(p->closing ? PRAGHIP_E_CLOSED : PRAGHIP_E_SHAPE, "E_PACK_DEVICE_LEVEL");
  if (count == 0) return PRAGHIP_OK;
  if (!left || !right || !output || !aligned8(left) || !aligned8(right) || !aligned8(output))
    return fail(PRAGHIP_E_ARGUMENT, "E_PACK_DEVICE_VIEW");
  const size_t ct = 2 * p->L << p->log_n;
  const auto lo = reinterpret_cast<uintptr_t>(output), hi = lo + count * ct * 8;
  for (const uint64_t* v : {left, right}) {
    const auto a = reinterpret_cast<uintptr_t>(v), b = a + count * ct * 8;
    if (a < hi && lo < b) return fail(PRAGHIP_E_ARGUMENT, "E_PACK_DEVICE_VIEW: output overlaps an input");
  }
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = pack_run(p, left, right, count, count, 0, level, output, pick(stream));
  if (e != hipSuccess) return pack_failure(p, e, "pair_device");
  p->merges += count;
  return PRAGHIP_OK;
}

int praghip_pack_tree_device(praghip_pack_plan* p, uint64_t* nodes, size_t leaves, size_t slots, void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_PACK_CLOSED");
  if (leaves == 0 || (leaves & (leaves - 1)) || slots == 0 || leaves > (size_t(1) << p->levels))
    return fail(PRAGHIP_E_SHAPE, "E_PACK_LEVEL");
  if (!nodes || !aligned8(nodes)) return fail(PRAGHIP_E_ARGUMENT, "E_PACK_DEVICE_VIEW");
  const size_t ct = 2 * p->L << p->log_n;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  unsigned level = 0;
  for (size_t m = leaves; m > 1 && e == hipSuccess; m >>= 1, ++level) {
    // level `level`: node a of slot s is the pair of nodes 2a and 2a + 1
    const size_t pairs = (m >> 1) * slots;
    e = pack_run(p, nodes, nodes + slots * ct, pairs, slots, 2 * slots, level, nodes, pick(stream));
    p->merges += pairs;
  }
  if (e != hipSuccess) return pack_failure(p, e, "tree_device");
  return PRAGHIP_OK;
}

int praghip_pack_merges(const praghip_pack_plan* p, uint64_t* merges) {
  if (!p || !merges) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *merges = p->merges;
  return PRAGHIP_OK;
}

int praghip_pack_timing(const praghip_pack_plan* p, praghip_timing* out) {
  if (!p || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = p->timing;
  return PRAGHIP_OK;
}

int praghip_pack_close(praghip_pack_plan* p, praghip_cleanup* out) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  p->release();
  if (out) *out = p->cleanup;
  return PRAGHIP_OK;
}

void praghip_pack_destroy(praghip_pack_plan* p) { delete p; }

}  // extern "C"

// ============================================================ TokenWeights plan
// prag::experimental::resident::TokenWeights (resident.hpp:20-45,
// resident.cu:104-195, resident/seal_adapter.cpp:22-61): `blocks` coefficient-
// form ciphertexts per slot, held in NTT form.  One evaluation of a weight
// column (ring words [blocks][width]) is
//   lift (reversed into the low `width` coefficients) -> NTT ->
//   sum over blocks of products -> INTT -> + Delta-scaled local term at
//   x^(width-1) of c0 -> times x^-(width-1)
// and lands in `finished` [slots][2][P][N]; a stack of (levels + 1)
// ciphertexts per slot holds the packing tree's partial results.
struct praghip_token_plan {
  int device = -1;
  unsigned log_n = 0;
  size_t P = 0, slots = 0, blocks = 0, width = 0, levels = 0, words = 0;
  std::vector<uint64_t> host_q, delta;
  uint64_t r = 0;
  bool local_bound = false;
  Buffers buf;
  NttDevice d;
  uint64_t *input = nullptr, *ring = nullptr, *weight = nullptr, *output = nullptr, *finished = nullptr;
  uint64_t *scaled = nullptr, *stack = nullptr, *local_shares = nullptr, *local_partial = nullptr;
  // batch scratch (praghip_token_reserve): [cap][blocks][P][N] weights, [cap][slots][2][P][N] products,
  // [cap][slots][P] scaled terms, [cap * slots][kLocalTiles] local-dot partials
  size_t batch_cap = 0;
  uint64_t *bweight = nullptr, *boutput = nullptr, *bscaled = nullptr, *bpartial = nullptr;
  hipStream_t stream = nullptr;
  // start, uploaded, lifted, transformed, summed, finished, downloaded
  static constexpr int kEvents = 7;
  hipEvent_t ev[kEvents] = {};
  praghip_timing timing{};
  praghip_token_phases phases{};
  praghip_cleanup cleanup{};
  bool closing = false;
  void release() { release_all(device, buf, stream, ev, kEvents, cleanup, closing); }
  ~praghip_token_plan() { release(); }
};

namespace {
int token_failure(praghip_token_plan* p, hipError_t e, const char* what) {
  p->release();
  return fail(PRAGHIP_E_DEVICE, std::string("E_RESIDENT_HIP: ") + what + ": " + hipGetErrorString(e));
}
PrimeList token_primes(const praghip_token_plan* p) {
  PrimeList pl{};
  for (size_t i = 0; i < p->P; ++i) pl.q[i] = p->host_q[i];
  pl.count = int(p->P);
  return pl;
}
// lift + NTT (one pass) -> sum over blocks -> (INTT) into p->output.  ev
// (null: none) receives events after the lift (ev[0], only when the lift is a
// kernel of its own, i.e. a prime is on the float path), after the transform
// (ev[1]) and after the sum (ev[2]).
hipError_t token_product(praghip_token_plan* p, const uint64_t* ring_dev, bool inverse, hipStream_t s,
                         hipEvent_t* ev = nullptr) {
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < p->P; ++i) m[i] = barrett_of(p->host_q[i]);
  const size_t limbs = p->slots * 2 * p->P;
  hipError_t e = hipSuccess;
  if (ev && p->d.n_f64) {  // a float-path prime: the lift is its own kernel, timed apart
    e = launch_lift59(ring_dev, p->weight, p->blocks, int(p->log_n), p->width, token_primes(p), s);
    if (e == hipSuccess) e = hipEventRecord(ev[0], s);
    if (e == hipSuccess) e = launch_ntt(false, p->weight, p->blocks * p->P, p->d, s);
  } else {
    e = launch_ntt_lift(ring_dev, p->width, p->weight, p->blocks, token_primes(p), p->d, s);
  }
  if (e == hipSuccess && ev) e = hipEventRecord(ev[1], s);
  if (e == hipSuccess)
    e = launch_dyadic_mac(p->input, p->weight, p->output, p->blocks, limbs, int(p->log_n), p->P, m, int(p->P), s);
  if (e == hipSuccess && ev) e = hipEventRecord(ev[2], s);
  if (e == hipSuccess && inverse) e = launch_ntt(true, p->output, limbs, p->d, s);
  return e;
}
// the whole evaluate_device path; residues [slots][P] device, or null for the
// bound local shares
hipError_t token_finished(praghip_token_plan* p, const uint64_t* ring_dev, const uint64_t* residues, uint64_t* out,
                          hipStream_t s, hipEvent_t* ev = nullptr) {
  hipError_t e = token_product(p, ring_dev, true, s, ev);
  if (e == hipSuccess && !residues) {
    Barrett m[kMaxKeyPrimes];
    for (size_t i = 0; i < p->P; ++i) m[i] = barrett_of(p->host_q[i]);
    e = launch_local_dot_scale(p->local_shares, ring_dev, p->blocks * p->width, p->slots, p->delta.data(), p->r, m,
                               int(p->P), p->scaled, p->local_partial, s);
    residues = p->scaled;
  }
  if (e == hipSuccess)
    e = launch_token_finish(p->output, residues, out, p->slots, token_primes(p), int(p->log_n), p->width, s);
  return e;
}
// Delta_k = floor(Q / 2^59) mod q_k and r = Q mod 2^59, Q = prod q (the
// coeff_div_plain_modulus / coeff_modulus_mod_plain_modulus of a t = 2^59
// context, resident/seal_adapter.cpp:48-58).
void bfv_delta(const std::vector<uint64_t>& q, std::vector<uint64_t>& delta, uint64_t& r) {
  std::vector<uint64_t> big{1};
  for (uint64_t x : q) {
    u128 carry = 0;
    for (auto& limb : big) {
      const u128 v = (u128)limb * x + carry;
      limb = uint64_t(v);
      carry = v >> 64;
    }
    if (carry) big.push_back(uint64_t(carry));
  }
  r = big[0] & ((1ull << 59) - 1);
  std::vector<uint64_t> sh(big.size());
  for (size_t i = 0; i < big.size(); ++i)
    sh[i] = (big[i] >> 59) | (i + 1 < big.size() ? big[i + 1] << 5 : 0);
  delta.clear();
  for (uint64_t x : q) {
    u128 acc = 0;
    for (size_t i = sh.size(); i-- > 0;) acc = ((acc << 64) | sh[i]) % x;
    delta.push_back(uint64_t(acc));
  }
}
// Milliseconds between consecutive phase events 0..n of a host-buffer
// evaluation; without a lift kernel (event 2 not recorded) the lift takes 0
// and the transform runs from event 1.
hipError_t token_phase_times(praghip_token_plan* p, float* t, int n) {
  hipError_t e = hipSuccess;
  const bool lift_kernel = p->d.n_f64 != 0;
  for (int i = 0; i < n && e == hipSuccess; ++i) {
    if (!lift_kernel && i == 1) {
      t[i] = 0;
      continue;
    }
    e = hipEventElapsedTime(&t[i], p->ev[!lift_kernel && i == 2 ? 1 : i], p->ev[i + 1]);
  }
  return e;
}
bool ring_word_ok(uint64_t v) {
  constexpr uint64_t modulus = 1ull << 59, bound = 1ull << 20;
  return v < modulus && !(v > bound && v < modulus - bound);
}
bool in_plan(const praghip_token_plan* p, const uint64_t* view) {
  const size_t ct = 2 * p->P << p->log_n;
  const auto v = reinterpret_cast<uintptr_t>(view);
  auto inside = [&](const uint64_t* base, size_t words) {
    const auto b = reinterpret_cast<uintptr_t>(base);
    return base && v >= b && v + ct * 8 <= b + words * 8 && (v - b) % 8 == 0;
  };
  return inside(p->finished, p->words) || inside(p->stack, p->slots * (p->levels + 1) * ct);
}
}  // namespace

extern "C" {

int praghip_token_plan_create(int device, const uint64_t* q, size_t primes, uint32_t log_n, size_t slots,
                              size_t blocks, size_t width, size_t levels, const uint64_t* input,
                              praghip_token_plan** plan) {
  if (!plan || !q || !input) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *plan = nullptr;
  const size_t n = size_t(1) << log_n;
  if (log_n < 4 || log_n > 14 || primes < 1 || primes > size_t(kMaxKeyPrimes) || slots < 1 || slots > 64 ||
      blocks < 1 || blocks > 4096 || width < 1 || width > n || levels > log_n)
    return fail(PRAGHIP_E_SHAPE, "E_GPU_TOKEN_CONTEXT_LAYOUT");
  NttHost h;
  if (int rc = build_ntt_host(q, primes, log_n, nullptr, nullptr, nullptr, h)) return rc;
  const size_t words = slots * 2 * primes * n, in_words = blocks * words;
  std::vector<uint64_t> qv(q, q + primes);
  if (!canonical(input, in_words, qv, log_n)) return fail(PRAGHIP_E_CANONICAL, "E_GPU_TOKEN_CONTEXT_LAYOUT");
  if (int rc = check_device(device)) return rc;
  std::unique_ptr<praghip_token_plan> p(new praghip_token_plan);
  p->device = device;
  p->log_n = log_n;
  p->P = primes;
  p->slots = slots;
  p->blocks = blocks;
  p->width = width;
  p->levels = levels;
  p->words = words;
  p->host_q = qv;
  bfv_delta(qv, p->delta, p->r);
  DeviceScope scope(device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  for (auto& ev : p->ev)
    if (e == hipSuccess) e = hipEventCreate(&ev);
  if (e == hipSuccess) e = upload_ntt(h, log_n, p->buf, p->d, p->stream);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->input, in_words * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->ring, blocks * width * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->weight, blocks * primes * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->output, words * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->finished, words * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->scaled, slots * primes * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->stack, (levels + 1) * words * 8, true);
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], p->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(p->input, input, in_words * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], p->stream);
  // the reference transforms the inputs on the CPU at construction; here the
  // GPU does it
  if (e == hipSuccess) e = launch_ntt(false, p->input, blocks * slots * 2 * primes, p->d, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  float ms = 0;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, p->ev[0], p->ev[1]);
  if (e != hipSuccess) return token_failure(p.get(), e, "create");
  p->timing.upload_ms = ms;
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  p->phases.initial_input_upload_ms = ms;
  p->phases.input_bytes = in_words * 8;
  p->phases.ring_weight_bytes = blocks * width * 8;
  p->phases.ntt_weight_bytes = blocks * primes * n * 8;
  p->phases.output_bytes = words * 8;
  p->phases.device_bytes = p->timing.device_bytes;
  *plan = p.release();
  return PRAGHIP_OK;
}

int praghip_token_bind_local_shares(praghip_token_plan* p, const uint64_t* shares, size_t words) {
  if (!p || !shares) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing || p->local_bound || words != p->slots * p->blocks * p->width)
    return fail(PRAGHIP_E_STATE, "E_LOCAL_BINDING");
  for (size_t i = 0; i < words; ++i)
    if (shares[i] >> 59) return fail(PRAGHIP_E_STATE, "E_LOCAL_BINDING");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->local_shares, words * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->local_partial, p->slots * kLocalTiles * 8, true);
  if (e == hipSuccess) e = hipMemcpyAsync(p->local_shares, shares, words * 8, hipMemcpyHostToDevice, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return token_failure(p, e, "bind_local_shares");
  p->local_bound = true;
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  return PRAGHIP_OK;
}

static int token_check_ring(const praghip_token_plan* p, const uint64_t* ring, size_t words) {
  if (words != p->blocks * p->width) return fail(PRAGHIP_E_SHAPE, "E_RESIDENT_WEIGHT_SHAPE");
  for (size_t i = 0; i < words; ++i)
    if (!ring_word_ok(ring[i])) return fail(PRAGHIP_E_CANONICAL, "E_RESIDENT_WEIGHT_BOUND");
  return PRAGHIP_OK;
}

int praghip_token_evaluate(praghip_token_plan* p, const uint64_t* ring, size_t words, uint64_t* output) {
  if (!p || !ring || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_RESIDENT_CLOSED");
  if (int rc = token_check_ring(p, ring, words)) return rc;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  hipStream_t s = p->stream;
  // events: 0 start, 1 uploaded, 2 lifted, 3 transformed, 4 summed (= 5,
  // nothing to finish), 6 downloaded (resident.cu:152-166)
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], s);
  if (e == hipSuccess) e = hipMemcpyAsync(p->ring, ring, words * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], s);
  if (e == hipSuccess) e = token_product(p, p->ring, false, s, p->ev + 2);
  if (e == hipSuccess) e = hipEventRecord(p->ev[5], s);
  if (e == hipSuccess) e = hipMemcpyAsync(output, p->output, p->words * 8, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[6], s);
  if (e == hipSuccess) e = hipEventSynchronize(p->ev[6]);
  float t[6] = {};
  if (e == hipSuccess) e = token_phase_times(p, t, 6);
  if (e != hipSuccess) {
    volatile uint64_t* o = output;
    for (size_t i = 0; i < p->words; ++i) o[i] = 0;
    return token_failure(p, e, "evaluate");
  }
  p->timing.upload_ms = t[0];
  p->timing.kernel_ms = double(t[1]) + t[2] + t[3] + t[4];
  p->timing.download_ms = t[5];
  p->phases.weight_upload_ms = t[0];
  p->phases.lift_ms = t[1];
  p->phases.ntt_ms = t[2];
  p->phases.dyadic_ms = double(t[3]) + t[4];
  p->phases.finish_ms = 0;
  p->phases.download_ms = t[5];
  return PRAGHIP_OK;
}

static int token_finished_host(praghip_token_plan* p, const uint64_t* ring, size_t words, const uint64_t* residues,
                               const uint64_t** view) {
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  hipStream_t s = p->stream;
  // events: 0 start, 1 uploaded, 2 lifted, 3 transformed, 4 summed, 5
  // finished (resident.cu:167-184)
  if (e == hipSuccess) e = hipEventRecord(p->ev[0], s);
  if (e == hipSuccess) e = hipMemcpyAsync(p->ring, ring, words * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && residues)
    e = hipMemcpyAsync(p->scaled, residues, p->slots * p->P * 8, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipEventRecord(p->ev[1], s);
  if (e == hipSuccess) e = token_finished(p, p->ring, residues ? p->scaled : nullptr, p->finished, s, p->ev + 2);
  if (e == hipSuccess) e = hipEventRecord(p->ev[5], s);
  if (e == hipSuccess) e = hipEventSynchronize(p->ev[5]);
  float t[5] = {};
  if (e == hipSuccess) e = token_phase_times(p, t, 5);
  if (e != hipSuccess) return token_failure(p, e, "evaluate_finished");
  p->timing.upload_ms = t[0];
  p->timing.kernel_ms = double(t[1]) + t[2] + t[3] + t[4];
  p->timing.download_ms = 0;
  p->phases.weight_upload_ms = t[0];
  p->phases.lift_ms = t[1];
  p->phases.ntt_ms = t[2];
  p->phases.dyadic_ms = t[3];
  p->phases.finish_ms = t[4];
  p->phases.download_ms = 0;
  *view = p->finished;
  return PRAGHIP_OK;
}

int praghip_token_evaluate_finished(praghip_token_plan* p, const uint64_t* ring, size_t words, const uint64_t* local,
                                    const uint64_t** view) {
  if (!p || !ring || !local || !view) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_RESIDENT_CLOSED");
  if (int rc = token_check_ring(p, ring, words)) return rc;
  // SEAL scalingvariant: Delta_k m + floor((r m + 2^58) / 2^59) mod q_k
  std::vector<uint64_t> scaled(p->slots * p->P);
  for (size_t slot = 0; slot < p->slots; ++slot) {
    const uint64_t m = local[slot];
    if (m >> 59) {
      wipe_host(scaled);
      return fail(PRAGHIP_E_CANONICAL, "E_GPU_TOKEN_CONTEXT_LAYOUT");
    }
    const uint64_t fix = uint64_t(((u128)p->r * m + (1ull << 58)) >> 59);
    for (size_t k = 0; k < p->P; ++k) {
      const uint64_t qk = p->host_q[k];
      scaled[slot * p->P + k] = uint64_t(((u128)m * p->delta[k] + fix) % qk);
    }
  }
  const int rc = token_finished_host(p, ring, words, scaled.data(), view);
  wipe_host(scaled);
  return rc;
}

int praghip_token_evaluate_local_finished(praghip_token_plan* p, const uint64_t* ring, size_t words,
                                          const uint64_t** view) {
  if (!p || !ring || !view) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_RESIDENT_CLOSED");
  if (!p->local_bound) return fail(PRAGHIP_E_STATE, "E_RESIDENT_LOCAL_SHAPE");
  if (int rc = token_check_ring(p, ring, words)) return rc;
  return token_finished_host(p, ring, words, nullptr, view);
}

int praghip_token_reserve(praghip_token_plan* p, size_t coords) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_RESIDENT_CLOSED");
  if (coords == 0 || coords > 4096) return fail(PRAGHIP_E_SHAPE, "E_RESIDENT_BATCH");
  if (coords <= p->batch_cap) return PRAGHIP_OK;
  if (p->batch_cap) return fail(PRAGHIP_E_STATE, "E_RESIDENT_BATCH_RESERVED");
  const size_t n = size_t(1) << p->log_n;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->bweight, coords * p->blocks * p->P * n * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->boutput, coords * p->words * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->bscaled, coords * p->slots * p->P * 8, true);
  if (e == hipSuccess) e = p->buf.alloc((void**)&p->bpartial, coords * p->slots * kLocalTiles * 8, true);
  if (e != hipSuccess) return token_failure(p, e, "reserve");
  p->batch_cap = coords;
  p->timing.device_bytes = p->buf.total_bytes();
  p->timing.sensitive_bytes = p->buf.sensitive_bytes();
  return PRAGHIP_OK;
}

int praghip_token_evaluate_device_batch(praghip_token_plan* p, const uint64_t* rings, const uint64_t* residues,
                                        uint64_t* output, size_t coords, void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_RESIDENT_CLOSED");
  if (coords == 0) return PRAGHIP_OK;
  if (!rings || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (coords > p->batch_cap) return fail(PRAGHIP_E_SHAPE, "E_RESIDENT_BATCH");
  if (!residues && !p->local_bound) return fail(PRAGHIP_E_STATE, "E_RESIDENT_LOCAL_SHAPE");
  if (!aligned8(rings) || !aligned8(output) || (residues && !aligned8(residues)))
    return fail(PRAGHIP_E_ARGUMENT, "E_RESIDENT_ALIGNMENT");
  const hipStream_t s = pick(stream);
  const size_t limbs = p->slots * 2 * p->P, words = p->blocks * p->width;
  Barrett m[kMaxKeyPrimes];
  for (size_t i = 0; i < p->P; ++i) m[i] = barrett_of(p->host_q[i]);
  const PrimeList pl = token_primes(p);
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = launch_ntt_lift(rings, p->width, p->bweight, coords * p->blocks, pl, p->d, s);
  if (e == hipSuccess)
    e = launch_token_mac(p->input, p->bweight, p->boutput, coords, p->blocks, limbs, int(p->log_n), m, int(p->P), s);
  if (e == hipSuccess) e = launch_ntt(true, p->boutput, coords * limbs, p->d, s);
  if (e == hipSuccess && !residues) {
    e = launch_local_dot_scale(p->local_shares, rings, words, p->slots, p->delta.data(), p->r, m, int(p->P),
                               p->bscaled, p->bpartial, s, coords);
    residues = p->bscaled;
  }
  if (e == hipSuccess)
    e = launch_token_finish(p->boutput, residues, output, coords * p->slots, pl, int(p->log_n), p->width, s);
  if (e != hipSuccess) return token_failure(p, e, "evaluate_device_batch");
  return PRAGHIP_OK;
}

int praghip_token_evaluate_device(praghip_token_plan* p, const uint64_t* ring, const uint64_t* residues,
                                  uint64_t* output, void* stream) {
  if (!p || !ring || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing) return fail(PRAGHIP_E_CLOSED, "E_RESIDENT_CLOSED");
  if (!residues && !p->local_bound) return fail(PRAGHIP_E_STATE, "E_RESIDENT_LOCAL_SHAPE");
  if (!aligned8(ring) || !aligned8(output) || (residues && !aligned8(residues)))
    return fail(PRAGHIP_E_ARGUMENT, "E_RESIDENT_ALIGNMENT");
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = token_finished(p, ring, residues, output, pick(stream));
  if (e != hipSuccess) return token_failure(p, e, "evaluate_device");
  return PRAGHIP_OK;
}

int praghip_token_stack_store(praghip_token_plan* p, size_t slot, unsigned level, const uint64_t* view,
                              void* stream) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  const size_t ct = 2 * p->P << p->log_n;
  if (p->closing || slot >= p->slots || level > p->levels || !view || !aligned8(view))
    return fail(PRAGHIP_E_ARGUMENT, "E_DEVICE_STACK_VIEW");
  uint64_t* dst = p->stack + (slot * (p->levels + 1) + level) * ct;
  if (view == dst) return PRAGHIP_OK;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  // on the stream that produced the view (the reference waits on the view's
  // ready event, resident.cu:177), then waited for
  const hipStream_t s = pick(stream);
  if (e == hipSuccess) e = hipMemcpyAsync(dst, view, ct * 8, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return token_failure(p, e, "stack_store");
  return PRAGHIP_OK;
}

// stack_store waiting on the view's ready event (resident.cu:176-179): the
// plan's stream waits on `ready`, copies, and the copy is waited for.
int praghip_token_stack_store_ready(praghip_token_plan* p, size_t slot, unsigned level, const uint64_t* view,
                                    void* ready) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  const size_t ct = 2 * p->P << p->log_n;
  if (p->closing || slot >= p->slots || level > p->levels || !view || !ready || !aligned8(view))
    return fail(PRAGHIP_E_ARGUMENT, "E_DEVICE_STACK_VIEW");
  uint64_t* dst = p->stack + (slot * (p->levels + 1) + level) * ct;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess) e = hipStreamWaitEvent(p->stream, static_cast<hipEvent_t>(ready), 0);
  if (e == hipSuccess && view != dst) e = hipMemcpyAsync(dst, view, ct * 8, hipMemcpyDeviceToDevice, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return token_failure(p, e, "stack_store");
  return PRAGHIP_OK;
}

int praghip_token_stack_view(praghip_token_plan* p, size_t slot, unsigned level, const uint64_t** view) {
  if (!p || !view) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing || slot >= p->slots || level > p->levels) return fail(PRAGHIP_E_ARGUMENT, "E_DEVICE_STACK_INDEX");
  const size_t ct = 2 * p->P << p->log_n;
  *view = p->stack + (slot * (p->levels + 1) + level) * ct;
  return PRAGHIP_OK;
}

static int token_download(praghip_token_plan* p, const uint64_t* view, void* ready, bool need_ready,
                          uint64_t* output) {
  if (!p || !output) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  if (p->closing || !view || !in_plan(p, view) || (need_ready && !ready))
    return fail(PRAGHIP_E_ARGUMENT, "E_DEVICE_DOWNLOAD_VIEW");
  const size_t ct = 2 * p->P << p->log_n;
  DeviceScope scope(p->device);
  hipError_t e = scope.status();
  if (e == hipSuccess && ready) e = hipStreamWaitEvent(p->stream, static_cast<hipEvent_t>(ready), 0);
  if (e == hipSuccess) e = hipMemcpyAsync(output, view, ct * 8, hipMemcpyDeviceToHost, p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) {
    volatile uint64_t* o = output;
    for (size_t i = 0; i < ct; ++i) o[i] = 0;
    return token_failure(p, e, "download");
  }
  return PRAGHIP_OK;
}

int praghip_token_download(praghip_token_plan* p, const uint64_t* view, uint64_t* output) {
  return token_download(p, view, nullptr, false, output);
}

// download waiting on the view's ready event (resident.cu:187-189).
int praghip_token_download_ready(praghip_token_plan* p, const uint64_t* view, void* ready, uint64_t* output) {
  return token_download(p, view, ready, true, output);
}

int praghip_token_phase_timing(const praghip_token_plan* p, praghip_token_phases* out) {
  if (!p || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = p->phases;
  return PRAGHIP_OK;
}

int praghip_token_timing(const praghip_token_plan* p, praghip_timing* out) {
  if (!p || !out) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  *out = p->timing;
  return PRAGHIP_OK;
}

int praghip_token_close(praghip_token_plan* p, praghip_cleanup* out) {
  if (!p) return fail(PRAGHIP_E_ARGUMENT, "E_NULL");
  p->release();
  if (out) *out = p->cleanup;
  return PRAGHIP_OK;
}

void praghip_token_destroy(praghip_token_plan* p) { delete p; }

}  // extern "C"
