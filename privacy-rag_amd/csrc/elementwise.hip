// Element-wise kernels of the BFV path: seeded synthetic inputs (the same
// counter-based splitmix64 stream on every platform), and the ring helpers.
#include "kernels.hpp"

namespace praghip {

__device__ __forceinline__ uint64_t splitmix64(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// limb l of a [limbs][N] buffer: uniform residues mod q[l % P] (Lemire mulhi)
__global__ void fill_residues_kernel(uint64_t* __restrict__ out, size_t words, int log_n, PrimeList q,
                                     uint64_t seed) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += size_t(gridDim.x) * blockDim.x)
    out[i] = __umul64hi(splitmix64(seed, i), q.q[(i >> log_n) % unsigned(q.count)]);
}
__global__ void fill_u64_kernel(uint64_t* __restrict__ out, size_t count, uint64_t seed) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x)
    out[i] = splitmix64(seed, i);
}
// int8 uniform in [-127, 127]
__global__ void fill_i8_kernel(int8_t* __restrict__ out, size_t count, uint64_t seed) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x)
    out[i] = int8_t(int64_t(__umul64hi(splitmix64(seed, i), 255)) - 127);
}

// Per-channel shifts in [0, 7]: mulhi(z, 8).
__global__ void fill_shift_kernel(int8_t* __restrict__ out, size_t count, uint64_t seed) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += size_t(gridDim.x) * blockDim.x)
    out[i] = int8_t(__umul64hi(splitmix64(seed, i), 8));
}

static unsigned grid_of(size_t n) { return unsigned(std::min<size_t>((n + 255) / 256, 1u << 16)); }

hipError_t launch_fill_residues(uint64_t* out, size_t words, int log_n, const PrimeList& q, uint64_t seed,
                                hipStream_t s) {
  if (!words) return hipSuccess;
  hipLaunchKernelGGL(fill_residues_kernel, dim3(grid_of(words)), dim3(256), 0, s, out, words, log_n, q, seed);
  return hipGetLastError();
}
hipError_t launch_fill_u64(uint64_t* out, size_t count, uint64_t seed, hipStream_t s) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(fill_u64_kernel, dim3(grid_of(count)), dim3(256), 0, s, out, count, seed);
  return hipGetLastError();
}
hipError_t launch_fill_i8(int8_t* out, size_t count, uint64_t seed, hipStream_t s) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(fill_i8_kernel, dim3(grid_of(count)), dim3(256), 0, s, out, count, seed);
  return hipGetLastError();
}

hipError_t launch_fill_shift(int8_t* out, size_t count, uint64_t seed, hipStream_t s) {
  if (!count) return hipSuccess;
  hipLaunchKernelGGL(fill_shift_kernel, dim3(grid_of(count)), dim3(256), 0, s, out, count, seed);
  return hipGetLastError();
}

}  // namespace praghip
