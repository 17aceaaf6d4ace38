// Batched BFV keyswitch (Switch::evaluate, switch.cu:113-125, with the Galois
// step of keyswitch/seal_adapter.cpp:44-51 moved onto the GPU).
//
//   ModUp    : digit j = residues of c1 on its data primes, fast base
//              conversion to every other key prime (for one prime per digit
//              this is exactly decompose, switch.cu:63-68)
//   NTT      : forward transform of every expanded limb
//   product  : P[c][t] = sum_j E[j][t] * K[j][c][t] mod q_t (switch.cu:69-73)
//   INTT     : inverse transform of the 2 x K product limbs
//   ModDown  : divide by the special prime with rounding, + c0 (switch.cu:74-82)
//
// The Galois automorphism a(X) -> a(X^g) is applied as a gather when c1 and
// c0 are read: output coefficient k comes from i = k * g^-1 mod 2N, negated
// when i >= N.
#include <type_traits>

#include "kernels.hpp"

namespace praghip {

__device__ __forceinline__ uint64_t galois_read(const uint64_t* __restrict__ limb, unsigned k, uint32_t ginv,
                                                int log_n, uint64_t q) {
  // branch-free: ginv = 1 gives i = k and no negation
  const unsigned i = (k * ginv) & ((2u << log_n) - 1);
  const uint64_t v = limb[i & ((1u << log_n) - 1)];
  return ((i >> log_n) && v) ? q - v : v;
}

// One thread per (ciphertext, coefficient): ModDown of both components.
__global__ void __launch_bounds__(256)
    ks_moddown_kernel(const uint64_t* __restrict__ prod, const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                      const KsConst* __restrict__ kcp, size_t batch, uint32_t ginv) {
  const KsConst& kc = *kcp;
  const int L = kc.L, K = kc.K, log_n = kc.log_n;
  const size_t n = size_t(1) << log_n;
  const size_t total = batch * n;
  const uint64_t p = kc.q[L], half = p >> 1;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += size_t(gridDim.x) * blockDim.x) {
    const size_t b = idx >> log_n;
    const unsigned k = unsigned(idx & (n - 1));
    for (int c = 0; c < 2; ++c) {
      const uint64_t* pc = prod + (b * 2 + c) * K * n;
      uint64_t last = pc[size_t(L) * n + k] + half;
      last = last >= p ? last - p : last;
      for (int i = 0; i < L; ++i) {
        const uint64_t qi = kc.q[i];
        const uint64_t reduced = mul_shoup(last, 1, kc.one_q[i], qi);  // last mod q_i
        const uint64_t corr = sub_mod(reduced, kc.half_mod[i], qi);
        uint64_t val = mul_shoup(sub_mod(pc[size_t(i) * n + k], corr, qi), kc.invp[i].w, kc.invp[i].wq, qi);
        if (c == 0) val = add_mod(val, galois_read(in + (b * 2 * L + i) * n, k, ginv, log_n, qi), qi);
        out[((b * 2 + c) * L + i) * n + k] = val;
      }
    }
  }
}

// Noise add + ModDown of the public-key encryption of zero (PublicZero,
// enc0.cu:55-63 moddown after noise_add): one thread per (component, data
// prime, coefficient); x = prod + e for the data prime and for p, then
// switch.cu:74-82 without the c0 term.
__global__ void __launch_bounds__(256)
    enc0_moddown_kernel(const uint64_t* __restrict__ prod, const uint64_t* __restrict__ noise,
                        uint64_t* __restrict__ out, Enc0Const kc, size_t count, size_t noise_stride) {
  const int L = kc.L, K = L + 1, log_n = kc.log_n;
  const size_t n = size_t(1) << log_n, per = size_t(2 * L) << log_n, total = count * per;
  const uint64_t p = kc.q[L], half = p >> 1;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += size_t(gridDim.x) * blockDim.x) {
    // encryption e: prod + e [2][K][N], noise + e noise_stride, out + e [2][L][N]
    const size_t e = idx / per, r = idx - e * per;
    const size_t c = r / (size_t(L) << log_n), k = r & (n - 1);
    const int i = int((r >> log_n) % unsigned(L));
    const uint64_t qi = kc.q[i];
    const uint64_t* pe = prod + e * (size_t(2 * K) << log_n);
    const uint64_t* ne = noise + e * noise_stride;
    const size_t li = (c * K + i) * n + k, lp = (c * K + L) * n + k;
    const uint64_t x = add_mod(pe[li], ne[li], qi);
    uint64_t last = add_mod(pe[lp], ne[lp], p) + half;
    last = last >= p ? last - p : last;
    const uint64_t reduced = mul_shoup(last, 1, kc.one_q[i], qi);  // last mod q_i
    const uint64_t corr = sub_mod(reduced, kc.half_mod[i], qi);
    out[idx] = mul_shoup(sub_mod(x, corr, qi), kc.invp[i].w, kc.invp[i].wq, qi);
  }
}

hipError_t launch_enc0_moddown(const uint64_t* prod, const uint64_t* noise, uint64_t* out, const Enc0Const& kc,
                               hipStream_t s, size_t count, size_t noise_stride) {
  const size_t total = count * (size_t(2 * kc.L) << kc.log_n);
  const unsigned blocks = unsigned(std::min<size_t>((total + 255) / 256, 1u << 16));
  hipLaunchKernelGGL(enc0_moddown_kernel, dim3(blocks), dim3(256), 0, s, prod, noise, out, kc, count, noise_stride);
  return hipGetLastError();
}

// ------------------------------------------------------------------ fused
// One workgroup per (ciphertext b, key prime t): ModUp of every digit to prime
// t, its forward NTT, the key inner product and the inverse NTT of both
// product components, with the limb held in registers + LDS throughout.  The
// coefficient-form products go to `prod` for ModDown.  Per digit the two
// running sums live in a per-workgroup slot in global memory, in a
// thread-private layout (register r of thread th at [c][r][th]): coalesced,
// and re-read by the same workgroup shortly after, so they stay in cache.
//
// Arithmetic per prime: the float path when every data prime and t are below
// 2^50 (ModUp, product and transforms in exact FP64), otherwise the integer
// path (Shoup ModUp, Shoup key products exact like the Barrett-128 products of
// switch.cu:30-45, Harvey transforms).  The special prime (60 bits) takes the
// integer path.
struct KsFused {
  const uint64_t* in;      // [batch][2][L][N]
  const uint64_t* key;     // [dnum][2][K][N] per key, key_stride words apart
  size_t key_stride;
  unsigned key_group;      // ciphertext b uses key b / key_group
  uint64_t* prod;          // [batch][2][K][N] coefficient form
  uint64_t* acc;           // [gridDim.x][2][N] running sums
  const KsConst* kc;
  const NttPrime* primes;  // [K]
  const ulonglong2* tw_fwd_u;
  const ulonglong2* tw_inv_u;
  const double* tw_fwd_f;
  const double* tw_inv_f;
  unsigned batch, items;
  unsigned acc_slots;  // workgroups the acc buffer has room for
  uint32_t ginv;
  int data_f64;  // every data prime is below 2^50
  int xcd;       // items of one ciphertext on one XCD (batch and grid multiples of 8)
  unsigned* queue;  // [kQueueWords]: per-group tickets, then the finished-workgroup count; zero between launches
};

__device__ __forceinline__ uint64_t as_u64(double x) { return (uint64_t)__double_as_longlong(x); }
__device__ __forceinline__ double as_f64(uint64_t x) { return __longlong_as_double((long long)x); }

// ModUp of digit j to prime t for this thread's registers (forward-input
// layout): e[r] = c1_t when t is one of the digit's primes, else
// sum_i [c1_i (Q_j/q_i)^-1]_{q_i} (Q_j/q_i) mod q_t over the digit's primes
// (fast base conversion, no correction).  The per-prime constants are read
// once per digit prime, outside the loop over registers.
template <int LOGN>
__device__ __forceinline__ void modup_f64(double (&e)[kE], const KsFused& f, const KsConst& kc, const uint64_t* c1,
                                          int j, int t, const NttPrime& pt, unsigned th) {
  const int lo = kc.dig_lo[j], hi = kc.dig_lo[j + 1];
  if (t >= lo && t < hi) {
    const uint64_t* x = c1 + (size_t(t) << LOGN);
    const uint64_t q = kc.q[t];
#pragma unroll
    for (int r = 0; r < kE; ++r) e[r] = ArF64::from_u64(galois_read(x, fwd_in_index<LOGN>(th, r), f.ginv, LOGN, q));
    return;
  }
#pragma unroll
  for (int r = 0; r < kE; ++r) e[r] = 0.0;
  for (int i = lo, n = 0; i < hi; ++i, ++n) {
    const NttPrime pi = f.primes[i];
    const uint64_t* x = c1 + (size_t(i) << LOGN);
    const double ih = double(kc.inv_hat[i].w), ihq = ih * pi.qinv;
    const double hf = double(kc.hat[i][t].w), hfq = hf * pt.qinv;
    const uint64_t qi = kc.q[i];
#pragma unroll
    for (int r = 0; r < kE; ++r) {
      const double v = ArF64::from_u64(galois_read(x, fwd_in_index<LOGN>(th, r), f.ginv, LOGN, qi));
      const double y = canon_f64(mul_f64(v, ih, ihq, pi.qd), pi.qd);  // [x (Q_j/q_i)^-1]_{q_i}
      e[r] += mul_f64(y, hf, hfq, pt.qd);                             // |term| < 7q/8
    }
    if ((n & 3) == 3) {
#pragma unroll
      for (int r = 0; r < kE; ++r) e[r] = reduce_f64(e[r], pt.qd, pt.qinv);
    }
  }
#pragma unroll
  for (int r = 0; r < kE; ++r) e[r] = reduce_f64(e[r], pt.qd, pt.qinv);
}
template <int LOGN>
__device__ __forceinline__ void modup_u64(uint64_t (&e)[kE], const KsFused& f, const KsConst& kc, const uint64_t* c1,
                                          int j, int t, unsigned th) {
  const int lo = kc.dig_lo[j], hi = kc.dig_lo[j + 1];
  const uint64_t qt = kc.q[t], qt2 = 2 * qt;
  if (t >= lo && t < hi) {
    const uint64_t* x = c1 + (size_t(t) << LOGN);
#pragma unroll
    for (int r = 0; r < kE; ++r) e[r] = galois_read(x, fwd_in_index<LOGN>(th, r), f.ginv, LOGN, qt);
    return;
  }
#pragma unroll
  for (int r = 0; r < kE; ++r) e[r] = 0;
  for (int i = lo; i < hi; ++i) {
    const uint64_t* x = c1 + (size_t(i) << LOGN);
    const Shoup ih = kc.inv_hat[i], hf = kc.hat[i][t];
    const uint64_t qi = kc.q[i];
#pragma unroll
    for (int r = 0; r < kE; ++r) {
      const uint64_t y = mul_shoup(galois_read(x, fwd_in_index<LOGN>(th, r), f.ginv, LOGN, qi), ih.w, ih.wq, qi);
      const uint64_t a = e[r] + mul_shoup_lazy(y, hf.w, hf.wq, qt);  // [0, 4q_t)
      e[r] = a >= qt2 ? a - qt2 : a;
    }
  }
#pragma unroll
  for (int r = 0; r < kE; ++r) e[r] = e[r] >= qt ? e[r] - qt : e[r];
}

// Float path item.  acc0 stays in registers; component 1's running sum goes
// through the workgroup's slot.
template <int LOGN>
__device__ __forceinline__ void ks_item_f64(const KsFused& f, const KsConst& kc, unsigned b, int t, uint64_t* lds,
                                            uint64_t* slot) {
  using A = ArF64Lean;
  constexpr unsigned TH = ntt_threads<LOGN>();
  const NttPrime pr = f.primes[t];
  const A ar(pr);
  const int K = kc.K, L = kc.L, dnum = kc.dnum;
  const uint64_t* c1 = f.in + (((size_t(b) * 2 + 1) * size_t(L)) << LOGN);
  const uint64_t* kb = f.key + size_t(b / f.key_group) * f.key_stride + (size_t(t) << LOGN);
  double* xl = reinterpret_cast<double*>(lds);
  uint64_t* s1 = slot;
  double acc0[kE];
  for (int j = 0; j < dnum; ++j) {
    // thread index made loop-variant (j < 2^30): per-thread indices are
    // recomputed per digit instead of being hoisted and kept live (or
    // spilled) across the transforms
    const unsigned th = threadIdx.x + (unsigned(j) >> 30);
    double e[kE];
    modup_f64<LOGN>(e, f, kc, c1, j, t, pr, th);
    ntt_regs<LOGN, false>(e, xl, th, f.tw_fwd_f + (size_t(t) << LOGN), ar, pr);
    const uint64_t* k0 = kb + ((size_t(j) * 2 * K) << LOGN);
    const uint64_t* k1 = k0 + (size_t(K) << LOGN);
    const bool settle = (j & 3) == 3 || j + 1 == dnum;
#pragma unroll
    for (int r = 0; r < kE; r += 2) {
      // registers r and r + 1 sit at adjacent positions after the last
      // forward pass: one 16-byte load per key limb
      const unsigned pos = fwd_out_index<LOGN>(th, r);
      const ulonglong2 ka = *reinterpret_cast<const ulonglong2*>(k0 + pos);
      const ulonglong2 kb = *reinterpret_cast<const ulonglong2*>(k1 + pos);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int rr = r + h;
        const unsigned si = unsigned(rr) * TH + th;
        // |e| <= 3.44 q after the last forward stage: products |p| <= 1.8 q,
        // summed without re-centring and re-centred after every fourth
        // digit and after the last, so the sums stay within
        // q/2 + 1 + 4 (1.8 q) < 8 q < 2^53
        const double p0 = ar.mul(e[rr], ArF64::from_u64(h ? ka.y : ka.x));
        double p1 = ar.mul(e[rr], ArF64::from_u64(h ? kb.y : kb.x));
        acc0[rr] = j ? acc0[rr] + p0 : p0;
        if (j) p1 += as_f64(s1[si]);
        if (settle) {
          acc0[rr] = reduce_f64(acc0[rr], ar.q, ar.qinv);
          p1 = reduce_f64(p1, ar.q, ar.qinv);
        }
        s1[si] = as_u64(p1);
      }
      if ((r & 3) == 2) __builtin_amdgcn_sched_barrier(0);
    }
  }
  uint64_t* pb = f.prod + ((size_t(b) * 2 * K + t) << LOGN);
  {
    const unsigned th = threadIdx.x + (unsigned(dnum) >> 30);
    ntt_regs<LOGN, true>(acc0, xl, th, f.tw_inv_f + (size_t(t) << LOGN), ar, pr);
#pragma unroll
    for (int r = 0; r < kE; ++r) pb[inv_out_index<LOGN>(th, r)] = ar.to_u64_inv(acc0[r]);
  }
  {
    const unsigned th = threadIdx.x + (unsigned(dnum + 1) >> 30);
#pragma unroll
    for (int r = 0; r < kE; ++r) acc0[r] = as_f64(s1[unsigned(r) * TH + th]);
    ntt_regs<LOGN, true>(acc0, xl, th, f.tw_inv_f + (size_t(t) << LOGN), ar, pr);
    uint64_t* pc = pb + (size_t(K) << LOGN);
#pragma unroll
    for (int r = 0; r < kE; ++r) pc[inv_out_index<LOGN>(th, r)] = ar.to_u64_inv(acc0[r]);
  }
}

// Integer path item (special prime, primes of 50 bits or more): both running
// sums go through the workgroup's slot.
template <int LOGN>
__device__ __forceinline__ void ks_item_u64(const KsFused& f, const KsConst& kc, unsigned b, int t, uint64_t* lds,
                                            uint64_t* slot) {
  using A = ArU64;
  constexpr unsigned TH = ntt_threads<LOGN>();
  const NttPrime pr = f.primes[t];
  const A ar(pr);
  const int K = kc.K, L = kc.L, dnum = kc.dnum;
  const uint64_t* c1 = f.in + (((size_t(b) * 2 + 1) * size_t(L)) << LOGN);
  const uint64_t* kb = f.key + size_t(b / f.key_group) * f.key_stride + (size_t(t) << LOGN);
  uint64_t* s0 = slot;
  uint64_t* s1 = slot + (size_t(kE) * TH);
  const Barrett bar = kc.bar[t];
  for (int j = 0; j < dnum; ++j) {
    const unsigned th = threadIdx.x + (unsigned(j) >> 30);
    uint64_t e[kE];
    modup_u64<LOGN>(e, f, kc, c1, j, t, th);
    ntt_regs<LOGN, false>(e, lds, th, f.tw_fwd_u + (size_t(t) << LOGN), ar, pr);
    const uint64_t* k0 = kb + ((size_t(j) * 2 * K) << LOGN);
    const uint64_t* k1 = k0 + (size_t(K) << LOGN);
#pragma unroll
    for (int r = 0; r < kE; r += 2) {
      // keys in 16-byte pairs (registers r, r + 1 are adjacent); the
      // transformed digit meets two key words, so it gets a Shoup quotient
      // and both products are Shoup products
      const unsigned pos = fwd_out_index<LOGN>(th, r);
      const ulonglong2 ka = *reinterpret_cast<const ulonglong2*>(k0 + pos);
      const ulonglong2 kb2 = *reinterpret_cast<const ulonglong2*>(k1 + pos);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int rr = r + h;
        const unsigned si = unsigned(rr) * TH + th;
        const uint64_t x = ar.to_u64_fwd(e[rr]);
        const uint64_t xq = shoup_quotient(x, bar);
        uint64_t p0 = mul_shoup(h ? ka.y : ka.x, x, xq, pr.q);
        uint64_t p1 = mul_shoup(h ? kb2.y : kb2.x, x, xq, pr.q);
        if (j) {
          p0 = add_mod(p0, s0[si], pr.q);
          p1 = add_mod(p1, s1[si], pr.q);
        }
        s0[si] = p0;
        s1[si] = p1;
      }
      if ((r & 3) == 2) __builtin_amdgcn_sched_barrier(0);
    }
  }
  uint64_t* pb = f.prod + ((size_t(b) * 2 * K + t) << LOGN);
#pragma unroll 1
  for (int c = 0; c < 2; ++c) {
    const unsigned th = threadIdx.x + (unsigned(c + dnum) >> 30);
    const uint64_t* sc = c ? s1 : s0;
    uint64_t e[kE];
#pragma unroll
    for (int r = 0; r < kE; ++r) e[r] = sc[unsigned(r) * TH + th];
    ntt_regs<LOGN, true>(e, lds, th, f.tw_inv_u + (size_t(t) << LOGN), ar, pr);
    uint64_t* pc = pb + ((size_t(c) * K) << LOGN);
#pragma unroll
    for (int r = 0; r < kE; ++r) pc[inv_out_index<LOGN>(th, r)] = ar.to_u64_inv(e[r]);
  }
}

// Items are handed out from a ticket counter, so a workgroup that finishes
// early takes the next item instead of following a fixed stride.  With the
// float path the special-prime item (integer path) costs about 1.7 float
// items; those are issued first, so the long items start in the first wave of
// the grid and the short ones fill in behind them (longest first).  With xcd
// set, workgroup w (on XCD w % 8) serves only ciphertexts b == w (mod 8) from
// queue w % 8, keeping the K items that re-read a ciphertext's c1 on one L2.
// The last workgroup to leave zeroes the counters for the next launch.  Every
// workgroup exits once its ticket passes the item count, so the loop always
// ends.
template <int LOGN>
__global__ void __launch_bounds__(ntt_threads<LOGN>()) ks_fused_kernel(KsFused f) {
  __shared__ __attribute__((aligned(16))) uint64_t lds[(1 << LOGN) + (1 << LOGN) / 16];
  __shared__ unsigned ticket;
  const KsConst& kc = *f.kc;
  const unsigned K = unsigned(kc.K), L = unsigned(kc.L);
  uint64_t* slot = f.acc + (size_t(blockIdx.x) * 2 * kE * ntt_threads<LOGN>());
  const unsigned groups = f.xcd ? 8u : 1u, g = f.xcd ? (blockIdx.x & 7u) : 0u;
  const unsigned cts = f.batch / groups;  // ciphertexts of this group: b = i * groups + g
  const unsigned count = cts * K;
  const bool split = f.data_f64 && K > 1;  // integer-path items (t = L) first
  for (;;) {
    __syncthreads();  // the previous item's LDS use and ticket reads are over
    if (threadIdx.x == 0) ticket = atomicAdd(f.queue + g, 1u);
    __syncthreads();
    const unsigned k = ticket;
    if (k >= count) break;
    unsigned i, t;
    if (!split) {
      i = k / K;
      t = k % K;
    } else if (k < cts) {
      i = k;
      t = L;
    } else {
      i = (k - cts) / L;
      t = (k - cts) % L;
    }
    const unsigned b = i * groups + g;
    if (f.data_f64 && t < L)
      ks_item_f64<LOGN>(f, kc, b, int(t), lds, slot);
    else
      ks_item_u64<LOGN>(f, kc, b, int(t), lds, slot);
  }
  if (threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(f.queue + kQueueGroups, 1u) == gridDim.x - 1) {
      for (unsigned q = 0; q <= kQueueGroups; ++q) atomicExch(f.queue + q, 0u);
    }
  }
}

static unsigned grid_for(size_t work) { return unsigned(std::min<size_t>((work + 255) / 256, 1u << 20)); }

template <int LOGN>
static unsigned fused_grid() {
  static unsigned grid = 0;
  if (!grid) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ks_fused_kernel<LOGN>, ntt_threads<LOGN>(), 0) !=
            hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    grid = unsigned(cus * per_cu);
  }
  return grid;
}

#define PH_LOGN_SWITCH(EXPR)      \
  switch (log_n) {                \
    case 4: { constexpr int LG = 4; EXPR; } \
    case 5: { constexpr int LG = 5; EXPR; } \
    case 6: { constexpr int LG = 6; EXPR; } \
    case 7: { constexpr int LG = 7; EXPR; } \
    case 8: { constexpr int LG = 8; EXPR; } \
    case 9: { constexpr int LG = 9; EXPR; } \
    case 10: { constexpr int LG = 10; EXPR; } \
    case 11: { constexpr int LG = 11; EXPR; } \
    case 12: { constexpr int LG = 12; EXPR; } \
    case 13: { constexpr int LG = 13; EXPR; } \
    case 14: { constexpr int LG = 14; EXPR; } \
    default: break;               \
  }

unsigned ks_acc_slots(int log_n) {
  PH_LOGN_SWITCH(return fused_grid<LG>());
  return 0;
}

template <int LOGN>
static hipError_t launch_fused_n(KsFused f, hipStream_t s) {
  const unsigned blocks = std::min(f.items, std::min(fused_grid<LOGN>(), f.acc_slots));
  f.xcd = (f.batch % kQueueGroups == 0 && blocks % kQueueGroups == 0) ? 1 : 0;
  hipLaunchKernelGGL((ks_fused_kernel<LOGN>), dim3(blocks), dim3(ntt_threads<LOGN>()), 0, s, f);
  return hipGetLastError();
}

hipError_t launch_keyswitch(const KsArgs& a, const KsConst* kc_dev, const KsConst& kc, const NttDevice& d,
                            hipStream_t s) {
  if (a.batch == 0) return hipSuccess;
  if (a.inter && keyswitch_rows_supported(kc)) return launch_keyswitch_rows(a, kc_dev, kc, d, s);
  const size_t n = size_t(1) << kc.log_n;
  KsFused f;
  f.in = a.in;
  f.key = a.key;
  f.key_stride = a.key_stride;
  f.key_group = unsigned(a.key_group ? a.key_group : 1);
  f.prod = a.prod;
  f.acc = a.acc;
  f.kc = kc_dev;
  f.primes = d.primes;
  f.tw_fwd_u = d.tw_fwd_u;
  f.tw_inv_u = d.tw_inv_u;
  f.tw_fwd_f = d.tw_fwd_f;
  f.tw_inv_f = d.tw_inv_f;
  f.batch = unsigned(a.batch);
  f.items = unsigned(a.batch * kc.K);
  f.acc_slots = a.acc_slots;
  f.ginv = a.galois_inv;
  f.queue = a.queue;
  f.data_f64 = 1;
  for (int i = 0; i < kc.L; ++i) f.data_f64 &= kc.q[i] < (1ull << 50) ? 1 : 0;
  f.xcd = 0;
  hipError_t e = hipErrorInvalidValue;
  const int log_n = kc.log_n;
  if (a.phase_events) (void)hipEventRecord(a.phase_events[0], s);
  PH_LOGN_SWITCH(e = launch_fused_n<LG>(f, s); break);
  if (e != hipSuccess) return e;
  if (a.phase_events) {
    (void)hipEventRecord(a.phase_events[1], s);
    (void)hipEventRecord(a.phase_events[2], s);
  }
  hipLaunchKernelGGL(ks_moddown_kernel, dim3(grid_for(a.batch * n)), dim3(256), 0, s, a.prod, a.in, a.out, kc_dev,
                     a.batch, a.galois_inv);
  if (a.phase_events) (void)hipEventRecord(a.phase_events[3], s);
  return hipGetLastError();
}

}  // namespace praghip
