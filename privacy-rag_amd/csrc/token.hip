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
// write, which stays inside one 2^log_n-word limb.
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

// Local pair i is pair e = first + i of the list; it reads
// left(e) = left + ((e / group) * stride + e % group) * ct and right(e) the
// same way from right (ct = 2 L N words), and writes
//   sum[i]  = left(e) + x^shift right(e)
//   diff[i] = sigma_g(left(e) - x^shift right(e)),  sigma_g: x -> x^g
// with x^shift right at j = right[j - shift], negated for j < shift.
__global__ void __launch_bounds__(256)
    pack_prepare_kernel(const uint64_t* __restrict__ left, const uint64_t* __restrict__ right,
                        uint64_t* __restrict__ sum, uint64_t* __restrict__ diff, size_t count, size_t first,
                        size_t group, size_t stride, PrimeList pl, int log_n, size_t shift, uint32_t g) {
  const size_t n = size_t(1) << log_n, L = size_t(pl.count), ct = 2 * L * n, total = count * ct;
  const size_t two_n_mask = 2 * n - 1;
  for (size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += size_t(gridDim.x) * blockDim.x) {
    const size_t i = idx / ct, w = idx - i * ct, j = w & (n - 1), base = w - j, e = first + i;
    const size_t src = ((e / group) * stride + e % group) * ct + base;
    const uint64_t q = pl.q[(w >> log_n) % L];
    const bool neg = j < shift;
    uint64_t v = right[src + ((j + n - shift) & (n - 1))];
    v = (neg && v) ? q - v : v;
    const uint64_t a = left[src + j];
    sum[i * ct + w] = add_mod(a, v, q);
    const uint64_t delta = sub_mod(a, v, q);
    const size_t dest = (j * size_t(g)) & two_n_mask;
    diff[i * ct + base + (dest & (n - 1))] = (dest >= n && delta) ? q - delta : delta;
  }
}

hipError_t launch_pack_prepare(const uint64_t* left, const uint64_t* right, uint64_t* sum, uint64_t* diff,
                               size_t count, size_t first, size_t group, size_t stride, const PrimeList& pl,
                               int log_n, size_t shift, uint32_t g, hipStream_t s) {
  const size_t total = count * 2 * size_t(pl.count) << log_n;
  hipLaunchKernelGGL(pack_prepare_kernel, dim3(elem_grid(total)), dim3(256), 0, s, left, right, sum, diff, count,
                     first, group, stride, pl, log_n, shift, g);
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

}  // namespace praghip
