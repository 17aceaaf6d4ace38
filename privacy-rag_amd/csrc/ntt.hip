// Batched negacyclic NTT / INTT kernels (NttBatch::transform, ntt.cu:104-127,
// and the stage loops inside Switch / TokenWeights / Matrix / PublicZero).
//
// Layout: [limbs][N] u64, limb l uses prime index l % P (the reference's
// [batch][prime][coefficient], ntt.hpp:20).  One workgroup per limb; the
// whole limb is transformed in registers + LDS, so each launch reads and
// writes every coefficient once (the reference launches 14 stages, each a
// full HBM round trip).
#include "kernels.hpp"

namespace praghip {

template <int LOGN, bool INV, class A>
__device__ __forceinline__ void ntt_limb(uint64_t* __restrict__ x, const typename A::TW* __restrict__ tw,
                                         const NttPrime& pr, typename A::T* lds) {
  using T = typename A::T;
  const unsigned t = threadIdx.x;
  const A ar(pr);
  T v[16];
  if (!INV) {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = ar.from_u64(x[fwd_in_index<LOGN>(t, j)]);
    ntt_fwd_regs<LOGN>(v, lds, t, tw, ar);
    ulonglong2* out = reinterpret_cast<ulonglong2*>(x + (size_t(t) << 4));
#pragma unroll
    for (int j = 0; j < 16; j += 2) out[j / 2] = make_ulonglong2(ar.to_u64_fwd(v[j]), ar.to_u64_fwd(v[j + 1]));
  } else {
    const ulonglong2* in = reinterpret_cast<const ulonglong2*>(x + (size_t(t) << 4));
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      const ulonglong2 p = in[j / 2];
      v[j] = ar.from_u64(p.x);
      v[j + 1] = ar.from_u64(p.y);
    }
    ntt_inv_regs<LOGN>(v, lds, t, tw, ar, pr);
#pragma unroll
    for (int j = 0; j < 16; ++j) x[inv_out_index<LOGN>(t, j)] = ar.to_u64_inv(v[j]);
  }
}

template <int LOGN, bool INV>
__global__ void __launch_bounds__((1 << LOGN) / 16)
    ntt_kernel(uint64_t* __restrict__ data, const NttPrime* __restrict__ primes,
               const ulonglong2* __restrict__ tw_u, const double2* __restrict__ tw_f, int P) {
  __shared__ uint64_t lds[(1 << LOGN) + (1 << LOGN) / 16];
  const size_t limb = blockIdx.x;
  const int p = int(limb % unsigned(P));
  const NttPrime pr = primes[p];
  uint64_t* x = data + (limb << LOGN);
  const size_t toff = size_t(p) << LOGN;
  if (pr.use_f64)
    ntt_limb<LOGN, INV, ArF64>(x, tw_f + toff, pr, reinterpret_cast<double*>(lds));
  else
    ntt_limb<LOGN, INV, ArU64>(x, tw_u + toff, pr, lds);
}

template <int LOGN>
static hipError_t launch_ntt_n(bool inverse, uint64_t* data, size_t limbs, const NttDevice& d,
                               hipStream_t s) {
  const dim3 grid{unsigned(limbs)}, block{unsigned((1 << LOGN) / 16)};
  if (inverse)
    hipLaunchKernelGGL((ntt_kernel<LOGN, true>), grid, block, 0, s, data, d.primes, d.tw_inv_u, d.tw_inv_f, d.P);
  else
    hipLaunchKernelGGL((ntt_kernel<LOGN, false>), grid, block, 0, s, data, d.primes, d.tw_fwd_u, d.tw_fwd_f, d.P);
  return hipGetLastError();
}

hipError_t launch_ntt(bool inverse, uint64_t* data, size_t limbs, const NttDevice& d, hipStream_t s) {
  if (limbs == 0) return hipSuccess;
  switch (d.log_n) {
    case 4: return launch_ntt_n<4>(inverse, data, limbs, d, s);
    case 5: return launch_ntt_n<5>(inverse, data, limbs, d, s);
    case 6: return launch_ntt_n<6>(inverse, data, limbs, d, s);
    case 7: return launch_ntt_n<7>(inverse, data, limbs, d, s);
    case 8: return launch_ntt_n<8>(inverse, data, limbs, d, s);
    case 9: return launch_ntt_n<9>(inverse, data, limbs, d, s);
    case 10: return launch_ntt_n<10>(inverse, data, limbs, d, s);
    case 11: return launch_ntt_n<11>(inverse, data, limbs, d, s);
    case 12: return launch_ntt_n<12>(inverse, data, limbs, d, s);
    case 13: return launch_ntt_n<13>(inverse, data, limbs, d, s);
    case 14: return launch_ntt_n<14>(inverse, data, limbs, d, s);
    default: return hipErrorInvalidValue;
  }
}

// Pointwise product with a per-prime operand in Shoup form (client_dyadic,
// ntt.cu:55-57): data[l][k] = data[l][k] * key[l % P][k] mod q.
__global__ void dyadic_shoup_kernel(uint64_t* __restrict__ data, const ulonglong2* __restrict__ key,
                                    const NttPrime* __restrict__ primes, int P, int log_n, size_t words) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += size_t(gridDim.x) * blockDim.x) {
    const size_t limb = i >> log_n;
    const int p = int(limb % unsigned(P));
    const ulonglong2 w = key[(size_t(p) << log_n) + (i & ((size_t(1) << log_n) - 1))];
    data[i] = mul_shoup(data[i], w.x, w.y, primes[p].q);
  }
}

hipError_t launch_dyadic_shoup(uint64_t* data, const ulonglong2* key, const NttDevice& d, size_t words,
                               hipStream_t s) {
  if (!words) return hipSuccess;
  const unsigned blocks = unsigned(std::min<size_t>((words + 255) / 256, 65536));
  hipLaunchKernelGGL(dyadic_shoup_kernel, dim3(blocks), dim3(256), 0, s, data, key, d.primes, d.P, d.log_n, words);
  return hipGetLastError();
}

}  // namespace praghip
