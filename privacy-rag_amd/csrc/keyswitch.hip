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
#include "kernels.hpp"

namespace praghip {

__device__ __forceinline__ uint64_t galois_read(const uint64_t* __restrict__ limb, unsigned k, uint32_t ginv,
                                                int log_n, uint64_t q) {
  if (ginv == 1) return limb[k];
  const unsigned two_n_mask = (2u << log_n) - 1;
  const unsigned i = (unsigned)(((uint64_t)k * ginv) & two_n_mask);
  const uint64_t v = limb[i & ((1u << log_n) - 1)];
  return ((i >> log_n) && v) ? q - v : v;
}

// One thread per (ciphertext, coefficient): reads the c1 residues once and
// writes every (digit, key prime) value of that coefficient.
__global__ void __launch_bounds__(256)
    ks_modup_kernel(const uint64_t* __restrict__ in, uint64_t* __restrict__ expanded,
                    const KsConst* __restrict__ kcp, size_t batch, uint32_t ginv) {
  const KsConst& kc = *kcp;
  const int L = kc.L, K = kc.K, log_n = kc.log_n;
  const size_t n = size_t(1) << log_n;
  const size_t total = batch * n;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += size_t(gridDim.x) * blockDim.x) {
    const size_t b = idx >> log_n;
    const unsigned k = unsigned(idx & (n - 1));
    const uint64_t* c1 = in + (b * 2 + 1) * L * n;
    uint64_t v[kMaxKeyPrimes];
#pragma unroll
    for (int i = 0; i < kMaxKeyPrimes; ++i)
      if (i < L) v[i] = galois_read(c1 + i * n, k, ginv, log_n, kc.q[i]);
    uint64_t* eb = expanded + b * size_t(kc.dnum) * K * n;
    for (int j = 0; j < kc.dnum; ++j) {
      const int lo = kc.dig_lo[j], hi = kc.dig_lo[j + 1];
      uint64_t y[kMaxKeyPrimes];
#pragma unroll
      for (int i = 0; i < kMaxKeyPrimes; ++i)
        if (i >= lo && i < hi) y[i] = mul_shoup(v[i], kc.inv_hat[i].w, kc.inv_hat[i].wq, kc.q[i]);
      for (int t = 0; t < K; ++t) {
        uint64_t e;
        if (t >= lo && t < hi) {
          e = v[t];
        } else {
          const uint64_t qt = kc.q[t], qt2 = 2 * qt;
          uint64_t acc = 0;
#pragma unroll
          for (int i = 0; i < kMaxKeyPrimes; ++i)
            if (i >= lo && i < hi) {
              acc += mul_shoup_lazy(y[i], kc.hat[i][t].w, kc.hat[i][t].wq, qt);  // [0, 2q_t)
              acc = acc >= qt2 ? acc - qt2 : acc;
            }
          e = acc >= qt ? acc - qt : acc;
        }
        eb[(size_t(j) * K + t) * n + k] = e;
      }
    }
  }
}

// One thread per (ciphertext, key prime, coefficient): both components.
__global__ void __launch_bounds__(256)
    ks_product_kernel(const uint64_t* __restrict__ expanded, const uint64_t* __restrict__ key, size_t key_stride,
                      uint64_t* __restrict__ prod, const KsConst* __restrict__ kcp, size_t batch) {
  const KsConst& kc = *kcp;
  const int K = kc.K, dnum = kc.dnum, log_n = kc.log_n;
  const size_t n = size_t(1) << log_n;
  const size_t total = batch * K * n;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += size_t(gridDim.x) * blockDim.x) {
    const size_t k = idx & (n - 1);
    const size_t bt = idx >> log_n;
    const int t = int(bt % unsigned(K));
    const size_t b = bt / unsigned(K);
    const Barrett m = kc.bar[t];
    const uint64_t* e = expanded + b * size_t(dnum) * K * n + size_t(t) * n + k;
    const uint64_t* kb = key + b * key_stride + size_t(t) * n + k;
    uint64_t s0 = 0, s1 = 0;
    for (int j = 0; j < dnum; ++j) {
      const uint64_t x = e[size_t(j) * K * n];
      s0 = add_mod(s0, mul_barrett(x, kb[(size_t(j) * 2 + 0) * K * n], m), m.q);
      s1 = add_mod(s1, mul_barrett(x, kb[(size_t(j) * 2 + 1) * K * n], m), m.q);
    }
    uint64_t* pb = prod + b * 2 * K * n + size_t(t) * n + k;
    pb[0] = s0;
    pb[size_t(K) * n] = s1;
  }
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

static unsigned grid_for(size_t work) { return unsigned(std::min<size_t>((work + 255) / 256, 1u << 20)); }

hipError_t launch_keyswitch(const KsArgs& a, const KsConst* kc_dev, const KsConst& kc, const NttDevice& d,
                            hipStream_t s) {
  if (a.batch == 0) return hipSuccess;
  const size_t n = size_t(1) << kc.log_n;
  hipLaunchKernelGGL(ks_modup_kernel, dim3(grid_for(a.batch * n)), dim3(256), 0, s, a.in, a.expanded, kc_dev,
                     a.batch, a.galois_inv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_ntt(false, a.expanded, a.batch * kc.dnum * kc.K, d, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ks_product_kernel, dim3(grid_for(a.batch * kc.K * n)), dim3(256), 0, s, a.expanded, a.key,
                     a.key_stride, a.prod, kc_dev, a.batch);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_ntt(true, a.prod, a.batch * 2 * kc.K, d, s);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ks_moddown_kernel, dim3(grid_for(a.batch * n)), dim3(256), 0, s, a.prod, a.in, a.out, kc_dev,
                     a.batch, a.galois_inv);
  return hipGetLastError();
}

}  // namespace praghip
