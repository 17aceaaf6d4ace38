// Element-wise kernels of the token-resident path and of the acyclic packing
// tree:
//   token_finish: the Delta-scaled local term added to coefficient
//     block_width-1 of c0, then the product multiplied by x^-(block_width-1)
//     (resident.cu:54-59 add_shift);
//   pack_prepare: right * x^shift, then the sum and the Galois image of the
//     difference of a packing pair (switch.cu:49-58 packing_prepare);
//   pack_finish: the two switched halves added (switch.cu:59-61).
// All residues stay canonical (< q < 2^62, so a + b never wraps).  Each kernel
// is a single HBM pass; one thread per output coefficient, contiguous in the
// coefficient index so reads and writes coalesce except the Galois-permuted
// reads, which stay inside one 2^log_n-word limb.
#include "kernels.hpp"

namespace praghip {

static unsigned elem_grid(size_t items) {
  return unsigned(std::min<size_t>(std::max<size_t>((items + 255) / 256, 1), 1u << 20));
}

// out[slot][c][p][d] = x^-(w-1) * (in[slot][c][p] + [c == 0] scaled[slot][p] x^(w-1)),
// negacyclic: source j = d + w - 1 (kept) or d + w - 1 - N (negated).
__global__ void __launch_bounds__(256)
    token_finish_kernel(const uint64_t* __restrict__ in, const uint64_t* __restrict__ scaled,
                        uint64_t* __restrict__ out, size_t slots, PrimeList pl, int log_n, size_t width) {
  const size_t n = size_t(1) << log_n, P = size_t(pl.count), total = slots * 2 * P * n;
  const size_t lift = width - 1;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += size_t(gridDim.x) * blockDim.x) {
    const size_t d = i & (n - 1), limb = i >> log_n, p = limb % P, c = (limb / P) & 1, slot = limb / (2 * P);
    const uint64_t q = pl.q[p];
    const bool wrap = d + lift >= n;
    const size_t j = wrap ? d + lift - n : d + lift;
    uint64_t v = in[(limb << log_n) + j];
    if (c == 0 && j == lift) v = add_mod(v, scaled[slot * P + p], q);
    out[i] = (wrap && v) ? q - v : v;
  }
}

hipError_t launch_token_finish(const uint64_t* in, const uint64_t* scaled, uint64_t* out, size_t slots,
                               const PrimeList& pl, int log_n, size_t width, hipStream_t s) {
  const size_t total = slots * 2 * size_t(pl.count) << log_n;
  hipLaunchKernelGGL(token_finish_kernel, dim3(elem_grid(total)), dim3(256), 0, s, in, scaled, out, slots, pl, log_n,
                     width);
  return hipGetLastError();
}

// Sum of products of a batch of weight columns against the resident inputs:
//   out[c][l][z] = sum_b in[b][l][z] * w[c][b][l % P][z]  mod q_{l % P}
// (resident.cu:38-45 accumulate), for every column c of the batch.  One thread
// per (coordinate group, prime p, coefficient z) walks all limbs l = p (mod P)
// and kMacCoords columns: each weight word is read once and each input word
// once per column group, instead of once per column.  A weight word meets up
// to KL inputs (KL limb slots per thread: 8 for the token path's slots x 2P
// limbs, 2 for a single ciphertext's 2P, so no slot multiplies zeros), so it
// gets a Shoup quotient (from the Barrett ratio)
// and the products are Shoup products: exact, like the reference's Barrett-128
// products, with fewer 64-bit multiplies.  LAZY (every prime below 2^60): the
// products are left in [0, 2q) and the sums reduced by 8q after every fourth
// block, so they stay below 16q < 2^64, and made canonical once at the end.
constexpr int kMacCoords = 4;
template <bool LAZY, int KL>
__global__ void __launch_bounds__(256)
    token_mac_kernel(const uint64_t* __restrict__ in, const uint64_t* __restrict__ w, uint64_t* __restrict__ out,
                     size_t coords, size_t blocks, size_t limbs, int log_n, BarrettList bl) {
  const size_t n = size_t(1) << log_n, P = size_t(bl.count), groups = (coords + kMacCoords - 1) / kMacCoords;
  const size_t words = limbs << log_n, wcol = blocks * P << log_n, total = groups * P << log_n;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += size_t(gridDim.x) * blockDim.x) {
    const size_t z = i & (n - 1), p = (i >> log_n) % P, c0 = ((i >> log_n) / P) * kMacCoords;
    const Barrett m = bl.m[p];
    const size_t cn = coords - c0 < size_t(kMacCoords) ? coords - c0 : size_t(kMacCoords);
    for (size_t l0 = p; l0 < limbs; l0 += KL * P) {
      uint64_t acc[kMacCoords][KL];
#pragma unroll
      for (int c = 0; c < kMacCoords; ++c)
#pragma unroll
        for (int k = 0; k < KL; ++k) acc[c][k] = 0;
      for (size_t b = 0; b < blocks; ++b) {
        uint64_t x[KL];
#pragma unroll
        for (int k = 0; k < KL; ++k) {
          const size_t l = l0 + size_t(k) * P;
          x[k] = l < limbs ? in[b * words + (l << log_n) + z] : 0;
        }
#pragma unroll
        for (int c = 0; c < kMacCoords; ++c) {
          if (size_t(c) >= cn) break;
          const uint64_t wv = w[(c0 + c) * wcol + ((b * P + p) << log_n) + z];
          const uint64_t wq = shoup_quotient(wv, m);
#pragma unroll
          for (int k = 0; k < KL; ++k) {
            if constexpr (LAZY) {
              acc[c][k] += mul_shoup_lazy(x[k], wv, wq, m.q);
            } else {
              const uint64_t v = acc[c][k] + mul_shoup(x[k], wv, wq, m.q);
              acc[c][k] = v >= m.q ? v - m.q : v;
            }
          }
        }
        if constexpr (LAZY) {
          if ((b & 3) == 3) {
            const uint64_t q8 = 8 * m.q;
#pragma unroll
            for (int c = 0; c < kMacCoords; ++c)
#pragma unroll
              for (int k = 0; k < KL; ++k) acc[c][k] = acc[c][k] >= q8 ? acc[c][k] - q8 : acc[c][k];
          }
        }
      }
#pragma unroll
      for (int c = 0; c < kMacCoords; ++c) {
        if (size_t(c) >= cn) break;
#pragma unroll
        for (int k = 0; k < KL; ++k) {
          const size_t l = l0 + size_t(k) * P;
          uint64_t v = acc[c][k];
          if constexpr (LAZY) {  // below 16q -> [0, q)
            v = v >= 8 * m.q ? v - 8 * m.q : v;
            v = v >= 4 * m.q ? v - 4 * m.q : v;
            v = v >= 2 * m.q ? v - 2 * m.q : v;
            v = v >= m.q ? v - m.q : v;
          }
          if (l < limbs) out[(c0 + c) * words + (l << log_n) + z] = v;
        }
      }
    }
  }
}

hipError_t launch_token_mac(const uint64_t* in, const uint64_t* w, uint64_t* out, size_t coords, size_t blocks,
                            size_t limbs, int log_n, const Barrett* m, int primes, hipStream_t s) {
  BarrettList bl{};
  for (int i = 0; i < primes; ++i) bl.m[i] = m[i];
  bl.count = primes;
  bool lazy = true;
  for (int i = 0; i < primes; ++i) lazy = lazy && m[i].q < (1ull << 60);
  const size_t total = ((coords + kMacCoords - 1) / kMacCoords * size_t(primes)) << log_n;
  // limb slots per thread: the limbs of one prime, rounded up to 2, 4 or 8
  const size_t per = (limbs + size_t(primes) - 1) / size_t(primes);
  const int kl = per <= 2 ? 2 : (per <= 4 ? 4 : 8);
  const auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(elem_grid(total)), dim3(256), 0, s, in, w, out, coords, blocks, limbs, log_n, bl);
  };
  if (lazy)
    kl == 2 ? go(token_mac_kernel<true, 2>) : kl == 4 ? go(token_mac_kernel<true, 4>) : go(token_mac_kernel<true, 8>);
  else
    kl == 2 ? go(token_mac_kernel<false, 2>) : kl == 4 ? go(token_mac_kernel<false, 4>) : go(token_mac_kernel<false, 8>);
  return hipGetLastError();
}

// Local pair i is pair e = first + i of the list; it reads
// left(e) = left + ((e / group) * stride + e % group) * ct and right(e) the
// same way from right (ct = 2 L N words), and writes
//   sum[i]  = left(e) + x^shift right(e)
//   diff[i] = sigma_g(left(e) - x^shift right(e)),  sigma_g: x -> x^g
// with x^shift right at j = right[j - shift], negated for j < shift.  Both
// outputs are written in coefficient order: diff at d takes the source
// coefficient u = d g^-1 mod 2N (negated when u >= N), gathered from inside
// the same limb, so no write is scattered.
__device__ __forceinline__ uint64_t shifted_diff(const uint64_t* __restrict__ l, const uint64_t* __restrict__ r,
                                                 size_t j, size_t n, size_t shift, uint64_t q, uint64_t& sum) {
  uint64_t v = r[(j + n - shift) & (n - 1)];
  v = (j < shift && v) ? q - v : v;
  const uint64_t a = l[j];
  sum = add_mod(a, v, q);
  return sub_mod(a, v, q);
}

__global__ void __launch_bounds__(256)
    pack_prepare_kernel(const uint64_t* __restrict__ left, const uint64_t* __restrict__ right,
                        uint64_t* __restrict__ sum, uint64_t* __restrict__ diff, size_t count, size_t first,
                        size_t group, size_t stride, PrimeList pl, int log_n, size_t shift, uint32_t ginv) {
  const size_t n = size_t(1) << log_n, L = size_t(pl.count), ct = 2 * L * n, total = count * ct;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += size_t(gridDim.x) * blockDim.x) {
    const size_t i = idx / ct, w = idx - i * ct, d = w & (n - 1), base = w - d, e = first + i;
    const size_t src = ((e / group) * stride + e % group) * ct + base;
    const uint64_t q = pl.q[(w >> log_n) % L];
    const uint64_t* l = left + src;
    const uint64_t* r = right + src;
    uint64_t s0;
    (void)shifted_diff(l, r, d, n, shift, q, s0);
    sum[i * ct + w] = s0;
    const size_t u = (d * size_t(ginv)) & (2 * n - 1);
    uint64_t unused;
    const uint64_t delta = shifted_diff(l, r, u & (n - 1), n, shift, q, unused);
    diff[i * ct + w] = (u >= n && delta) ? q - delta : delta;
  }
}

hipError_t launch_pack_prepare(const uint64_t* left, const uint64_t* right, uint64_t* sum, uint64_t* diff,
                               size_t count, size_t first, size_t group, size_t stride, const PrimeList& pl,
                               int log_n, size_t shift, uint32_t ginv, hipStream_t s) {
  const size_t total = count * 2 * size_t(pl.count) << log_n;
  hipLaunchKernelGGL(pack_prepare_kernel, dim3(elem_grid(total)), dim3(256), 0, s, left, right, sum, diff, count,
                     first, group, stride, pl, log_n, shift, ginv);
  return hipGetLastError();
}

// out[w] = a[w] + b[w] mod q over count ciphertexts [count][2][L][N].
__global__ void __launch_bounds__(256)
    pack_finish_kernel(const uint64_t* __restrict__ a, const uint64_t* __restrict__ b, uint64_t* __restrict__ out,
                       size_t count, PrimeList pl, int log_n) {
  const size_t L = size_t(pl.count), total = count * 2 * L << log_n;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += size_t(gridDim.x) * blockDim.x)
    out[i] = add_mod(a[i], b[i], pl.q[(i >> log_n) % L]);
}

hipError_t launch_pack_finish(const uint64_t* a, const uint64_t* b, uint64_t* out, size_t count, const PrimeList& pl,
                              int log_n, hipStream_t s) {
  const size_t total = count * 2 * size_t(pl.count) << log_n;
  hipLaunchKernelGGL(pack_finish_kernel, dim3(elem_grid(total)), dim3(256), 0, s, a, b, out, count, pl, log_n);
  return hipGetLastError();
}

// Selective evaluation of a batch (evaluate_selective, matrix.cu:65-81, with
// the c0 gather of matrix.cu:41-44): c0 of every output group keeps only the
// `count` target coefficients idx[] (strictly increasing, < N) and is zero
// elsewhere; selected[g][k][j] = c0[g][k][idx[j]] when selected is given.  One
// thread per c0 coefficient finds its coefficient among the targets by binary
// search over idx staged in LDS; c1 is left as it is.
__global__ void __launch_bounds__(256)
    select_c0_kernel(uint64_t* __restrict__ out, size_t groups, int primes, int log_n,
                     const uint64_t* __restrict__ idx, unsigned count, uint64_t* __restrict__ selected) {
  __shared__ uint64_t targets[kMaxTargets];
  for (unsigned j = threadIdx.x; j < count; j += blockDim.x) targets[j] = idx[j];
  __syncthreads();
  const size_t n = size_t(1) << log_n, per_group = size_t(primes) << log_n, total = groups * per_group;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += size_t(gridDim.x) * blockDim.x) {
    const size_t g = i / per_group, r = i % per_group, z = r & (n - 1);
    unsigned lo = 0, hi = count;  // first target >= z
    while (lo < hi) {
      const unsigned mid = (lo + hi) >> 1;
      if (targets[mid] < z)
        lo = mid + 1;
      else
        hi = mid;
    }
    uint64_t* c0 = out + g * 2 * per_group + r;  // c0 limb k, coefficient z
    if (lo < count && targets[lo] == z) {
      if (selected) selected[(g * size_t(primes) + (r >> log_n)) * count + lo] = *c0;
    } else {
      *c0 = 0;
    }
  }
}

hipError_t launch_select_c0(uint64_t* out, size_t groups, int primes, int log_n, const uint64_t* idx,
                            unsigned count, uint64_t* selected, hipStream_t s) {
  if (count == 0 || count > kMaxTargets) return hipErrorInvalidValue;
  const size_t total = groups * size_t(primes) << log_n;
  hipLaunchKernelGGL(select_c0_kernel, dim3(elem_grid(total)), dim3(256), 0, s, out, groups, primes, log_n, idx,
                     count, selected);
  return hipGetLastError();
}

}  // namespace praghip
