// Internal interface between the C ABI layer (api.cpp) and the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

#include "ntt_core.hpp"

namespace praghip {

// Device-resident NTT tables of one prime set.
struct NttDevice {
  int log_n = 0, P = 0;
  NttPrime* primes = nullptr;        // [P]
  ulonglong2* tw_fwd_u = nullptr;    // [P][N] (w, floor(w 2^64/q))
  ulonglong2* tw_inv_u = nullptr;    // [P][N]
  double* tw_fwd_f = nullptr;        // [P][N] w as a double, for q < 2^50
  double* tw_inv_f = nullptr;        // [P][N]
  // prime indices handled by the float path (q < 2^50) and by the integer path
  int* sel_f64 = nullptr;            // device [n_f64]
  int* sel_u64 = nullptr;            // device [n_u64]
  int n_f64 = 0, n_u64 = 0;
  int host_sel_f64[64] = {}, host_sel_u64[64] = {};
  int lazy_u64 = 1;  // every integer-path prime below 2^60: the lazy integer transforms (ArU64L)
};

hipError_t launch_ntt(bool inverse, uint64_t* data, size_t limbs, const NttDevice& d, hipStream_t s);
hipError_t launch_dyadic_shoup(uint64_t* data, const ulonglong2* key, const NttDevice& d, size_t words,
                               hipStream_t s);

// Keyswitch constants (device).  K = L + 1 key primes; prime L is the special
// prime p.  Digit j covers data primes [dig_lo[j], dig_lo[j+1]).
constexpr int kMaxKeyPrimes = 16;
struct KsConst {
  int L, K, dnum, log_n;
  int dig_lo[kMaxKeyPrimes + 1];
  int digit_of[kMaxKeyPrimes];           // data prime -> digit
  uint64_t q[kMaxKeyPrimes];
  Barrett bar[kMaxKeyPrimes];            // Barrett-128 ratios (product kernel)
  Shoup inv_hat[kMaxKeyPrimes];          // ((Q_j/q_i) mod q_i)^-1, mod q_i
  Shoup hat[kMaxKeyPrimes][kMaxKeyPrimes];  // (Q_j/q_i) mod q_t, mod q_t   [i][t]
  Shoup invp[kMaxKeyPrimes];             // p^-1 mod q_i
  uint64_t half_mod[kMaxKeyPrimes];      // floor(p/2) mod q_i
  uint64_t one_q[kMaxKeyPrimes];         // floor(2^64 / q_t): Shoup constant of 1, every key prime
  // lazy integer path (every key prime below 2^60): Montgomery key products,
  // whose factor 2^-64 the last inverse stage removes
  int lazy;
  uint64_t neg_qinv[kMaxKeyPrimes];      // -q_t^-1 mod 2^64
  Shoup ninv_r[kMaxKeyPrimes];           // N^-1 2^64 mod q_t
  Shoup last_r[kMaxKeyPrimes];           // w_last N^-1 2^64 mod q_t (w_last = inv[N-1])
};

struct KsArgs {
  const uint64_t* in;    // [batch][2][L][N] coefficient form
  uint64_t* out;         // [batch][2][L][N]
  const uint64_t* key;   // [dnum][2][K][N] NTT form, + b * key_stride
  size_t key_stride;     // words between consecutive keys (0 = one shared key)
  size_t key_group = 1;  // consecutive ciphertexts that share one key: ciphertext b uses key b / key_group
  uint64_t* acc;         // scratch [acc_slots][2][N]: per-workgroup running sums
  unsigned acc_slots;
  uint64_t* prod;        // scratch [batch][2][K][N]: products in coefficient form
  size_t batch;
  uint32_t galois_inv;   // g^-1 mod 2N (1 = identity)
  unsigned* queue;       // scratch [kQueueWords], zero before the first launch (the kernel leaves it zero)
  uint64_t* inter = nullptr;  // scratch [inter_cts][dnum][K][N]: expanded digits of the three-phase path
  size_t inter_cts = 0;       // ciphertexts per three-phase chunk (0: whole-limb path only)
  // four events recorded on the stream after the ModUp + forward columns, the
  // rows, the special prime's inverse columns and the ModDown columns (the
  // whole-limb path records the first at its start, the next two after its
  // kernel); null: none.  Only for a batch of one chunk.
  hipEvent_t* phase_events = nullptr;
};
// Work-queue counters of the fused keyswitch: one ticket per XCD group, then
// the count of finished workgroups.
constexpr unsigned kQueueGroups = 8;
constexpr unsigned kQueueWords = 16;

// ModDown constants of the encryption of zero (K = L + 1 primes, p = q[L]).
struct Enc0Const {
  int L, log_n;
  uint64_t q[kMaxKeyPrimes];
  Shoup invp[kMaxKeyPrimes];      // p^-1 mod q_i
  uint64_t half_mod[kMaxKeyPrimes];  // floor(p/2) mod q_i
  uint64_t one_q[kMaxKeyPrimes];     // floor(2^64 / q_i)
};
// out [2][L][N] = ModDown(prod + noise), prod and noise [2][K][N]; for `count`
// encryptions prod and out advance by their size and noise by noise_stride.
hipError_t launch_enc0_moddown(const uint64_t* prod, const uint64_t* noise, uint64_t* out, const Enc0Const& kc,
                               hipStream_t s, size_t count = 1, size_t noise_stride = 0);

// Prime list passed by value to the fill kernel.
struct PrimeList {
  uint64_t q[kMaxKeyPrimes];
  int count;
};
// Barrett-128 ratios of a prime list, passed by value.
struct BarrettList {
  Barrett m[kMaxKeyPrimes];
  int count;
};
hipError_t launch_fill_residues(uint64_t* out, size_t words, int log_n, const PrimeList& q, uint64_t seed,
                                hipStream_t s);
hipError_t launch_fill_u64(uint64_t* out, size_t count, uint64_t seed, hipStream_t s);
hipError_t launch_fill_i8(int8_t* out, size_t count, uint64_t seed, hipStream_t s);
hipError_t launch_fill_shift(int8_t* out, size_t count, uint64_t seed, hipStream_t s);

// Ring ops, lift, dyadic MAC and local dot (shares.hip).
constexpr unsigned kLocalTiles = 256;  // workgroups per slot of the local dot (workspace words per slot)
hipError_t launch_ring_add(const uint64_t* a, const uint64_t* b, uint64_t* c, size_t n, int bits, hipStream_t s);
hipError_t launch_ring_scale(const uint64_t* a, uint64_t factor, uint64_t* c, size_t n, int bits, hipStream_t s);
hipError_t launch_ring_layout(const uint64_t* a, size_t n_in, const uint64_t* map, uint64_t* c, size_t n_out,
                              hipStream_t s);
hipError_t launch_ring_sum_rows(const uint64_t* a, uint64_t* out, size_t rows, size_t cols, int bits,
                                hipStream_t s);
hipError_t launch_lift59(const uint64_t* ring, uint64_t* out, size_t blocks, int log_n, size_t width,
                         const PrimeList& q, hipStream_t s);
// Forward NTT of lifted ring words: limb l = b P + k of out is the lift of ring
// block b (lift59_residue mod q_k = pl.q[k], the layout of launch_lift59's
// width), then transformed; one pass over memory when every prime is on the
// integer path.
hipError_t launch_ntt_lift(const uint64_t* ring, size_t width, uint64_t* out, size_t blocks, const PrimeList& pl,
                           const NttDevice& d, hipStream_t s);
hipError_t launch_dyadic_mac(const uint64_t* a, const uint64_t* w, uint64_t* out, size_t blocks, size_t limbs,
                             int log_n, size_t w_limbs, const Barrett* m, int primes, hipStream_t s);
hipError_t launch_local_dot_scale(const uint64_t* shares, const uint64_t* weights, size_t words, size_t slots,
                                  const uint64_t* delta, uint64_t r, const Barrett* m, int primes, uint64_t* scaled,
                                  uint64_t* work, hipStream_t s, size_t coords = 1);
// Slot rows the allocation-free local dot takes: its scratch is
// kNoAllocSlots * kLocalTiles words (128 KiB) per device.
constexpr size_t kNoAllocSlots = 64;
// Device address of that scratch on `device` (the current device).
hipError_t local_dot_scratch(int device, uint64_t** address);

// Token-resident path and packing tree (token.hip).
hipError_t launch_token_finish(const uint64_t* in, const uint64_t* scaled, uint64_t* out, size_t slots,
                               const PrimeList& pl, int log_n, size_t width, hipStream_t s);
// out[c][l][N] = sum_b in[b][l] (.) w[c][b][l % P] over `coords` weight
// columns sharing the resident inputs in [blocks][limbs][N]; w is
// [coords][blocks][P][N], out [coords][limbs][N].
hipError_t launch_token_mac(const uint64_t* in, const uint64_t* w, uint64_t* out, size_t coords, size_t blocks,
                            size_t limbs, int log_n, const Barrett* m, int primes, hipStream_t s);
hipError_t launch_pack_prepare(const uint64_t* left, const uint64_t* right, uint64_t* sum, uint64_t* diff,
                               size_t count, size_t first, size_t group, size_t stride, const PrimeList& pl,
                               int log_n, size_t shift, uint32_t ginv, hipStream_t s);
// Selective batch output: c0 of each group [groups][2][primes][2^log_n] zero
// outside the `count` (<= kMaxTargets) sorted target coefficients idx[], and
// the targets gathered into selected [groups][primes][count] (if non-null).
constexpr unsigned kMaxTargets = 512;
hipError_t launch_select_c0(uint64_t* out, size_t groups, int primes, int log_n, const uint64_t* idx,
                            unsigned count, uint64_t* selected, hipStream_t s);
hipError_t launch_pack_finish(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t count, const PrimeList& pl,
                              int log_n, hipStream_t s);

hipError_t launch_keyswitch(const KsArgs& a, const KsConst* kc_dev, const KsConst& kc, const NttDevice& d,
                            hipStream_t s);
// Workgroups of the fused keyswitch kernel for 2^log_n (the acc slots a plan
// allocates); 0 for an unsupported size.
unsigned ks_acc_slots(int log_n);
// Three-phase keyswitch (columns, rows, columns) for N = 16384 with digits of
// equal size 1..3; hipErrorNotSupported for any other shape or without the
// `inter` scratch.  launch_keyswitch takes it when it applies.
bool keyswitch_rows_supported(const KsConst& kc);
hipError_t launch_keyswitch_rows(const KsArgs& a, const KsConst* kc_dev, const KsConst& kc, const NttDevice& d,
                                 hipStream_t s);
// Ciphertexts per three-phase chunk a plan sizes its `inter` scratch for.
constexpr size_t kKsRowsChunk = 64;

// Outputs a batched share GEMM zeroes in one launch before its split-K
// products (launch_gemm_clear_list, gemm.hip).
constexpr int kGemmClearMax = 64;
struct GemmClearList {
  uint64_t* ptr[kGemmClearMax];
  size_t words[kGemmClearMax];
  int count;
};

}  // namespace praghip
