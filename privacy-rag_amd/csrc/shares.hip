// Element-wise and reduction kernels of the other hot-path backends:
//   ring ops of LocalShares (compute/local_shares.cu:9-12), mod 2^mask_bits;
//   the centred lift of ring words into Z_q (resident.cu:23-30, matrix.cu:23-26);
//   the dyadic multiply-accumulate (resident.cu:38-45 accumulate,
//   matrix.cu:34-38 product), Barrett-128 as in switch.cu:30-45;
//   the party-local dot product with BFV Delta scaling (resident.cu:60-74,
//   constants from resident/seal_adapter.cpp:43-53).
// All of it is HBM-bound integer work: one pass over the operands, 16-byte
// accesses where the layout allows, grid-stride loops over a grid sized to the
// chip.
#include "kernels.hpp"

#include <mutex>

namespace praghip {

static unsigned stream_grid(size_t items, unsigned per_block) {
  const size_t blocks = (items + per_block - 1) / per_block;
  return unsigned(std::min<size_t>(std::max<size_t>(blocks, 1), 8192));
}

__device__ __forceinline__ uint64_t ring_mask(int bits) { return bits >= 64 ? ~0ull : (1ull << bits) - 1; }

// ------------------------------------------------------------------ ring ops
// c = (a + b) mod 2^bits, two words per thread and step (16-byte accesses).
__global__ void ring_add_kernel(const uint64_t* __restrict__ a, const uint64_t* __restrict__ b,
                                uint64_t* __restrict__ c, size_t n, int bits) {
  const uint64_t m = ring_mask(bits);
  const size_t pairs = n >> 1, stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < pairs; i += stride) {
    const ulonglong2 x = reinterpret_cast<const ulonglong2*>(a)[i], y = reinterpret_cast<const ulonglong2*>(b)[i];
    reinterpret_cast<ulonglong2*>(c)[i] = make_ulonglong2((x.x + y.x) & m, (x.y + y.y) & m);
  }
  if ((n & 1) && blockIdx.x == 0 && threadIdx.x == 0) c[n - 1] = (a[n - 1] + b[n - 1]) & m;
}

// c = (a * factor) mod 2^bits.
__global__ void ring_scale_kernel(const uint64_t* __restrict__ a, uint64_t factor, uint64_t* __restrict__ c, size_t n,
                                  int bits) {
  const uint64_t m = ring_mask(bits);
  const size_t pairs = n >> 1, stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < pairs; i += stride) {
    const ulonglong2 x = reinterpret_cast<const ulonglong2*>(a)[i];
    reinterpret_cast<ulonglong2*>(c)[i] = make_ulonglong2((x.x * factor) & m, (x.y * factor) & m);
  }
  if ((n & 1) && blockIdx.x == 0 && threadIdx.x == 0) c[n - 1] = (a[n - 1] * factor) & m;
}

// c[i] = a[map[i]] (a public gather); an index outside [0, n_in) gives 0.
__global__ void ring_layout_kernel(const uint64_t* __restrict__ a, size_t n_in, const uint64_t* __restrict__ map,
                                   uint64_t* __restrict__ c, size_t n_out) {
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n_out; i += stride) {
    const uint64_t j = map[i];
    c[i] = j < n_in ? a[j] : 0;
  }
}

// out[r] = (sum_c a[r][c]) mod 2^bits: one wave per row, lanes stride over
// the columns, then a butterfly reduction across the wave (exact: sums of
// u64 words wrap mod 2^64 in any order).
__global__ void __launch_bounds__(256) ring_sum_rows_kernel(const uint64_t* __restrict__ a, uint64_t* __restrict__ out,
                                                            size_t rows, size_t cols, int bits) {
  const unsigned lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t waves = size_t(gridDim.x) * (blockDim.x >> 6);
  for (size_t r = size_t(blockIdx.x) * (blockDim.x >> 6) + wave; r < rows; r += waves) {
    const uint64_t* row = a + r * cols;
    uint64_t s = 0;
    for (size_t c = lane; c < cols; c += 64) s += row[c];
#pragma unroll
    for (int d = 32; d; d >>= 1) s += __shfl_xor(s, d, 64);
    if (lane == 0) out[r] = s & ring_mask(bits);
  }
}

hipError_t launch_ring_add(const uint64_t* a, const uint64_t* b, uint64_t* c, size_t n, int bits, hipStream_t s) {
  hipLaunchKernelGGL(ring_add_kernel, dim3(stream_grid(n / 2 + 1, 256)), dim3(256), 0, s, a, b, c, n, bits);
  return hipGetLastError();
}
hipError_t launch_ring_scale(const uint64_t* a, uint64_t factor, uint64_t* c, size_t n, int bits, hipStream_t s) {
  hipLaunchKernelGGL(ring_scale_kernel, dim3(stream_grid(n / 2 + 1, 256)), dim3(256), 0, s, a, factor, c, n, bits);
  return hipGetLastError();
}
hipError_t launch_ring_layout(const uint64_t* a, size_t n_in, const uint64_t* map, uint64_t* c, size_t n_out,
                              hipStream_t s) {
  hipLaunchKernelGGL(ring_layout_kernel, dim3(stream_grid(n_out, 256)), dim3(256), 0, s, a, n_in, map, c, n_out);
  return hipGetLastError();
}
hipError_t launch_ring_sum_rows(const uint64_t* a, uint64_t* out, size_t rows, size_t cols, int bits,
                                hipStream_t s) {
  hipLaunchKernelGGL(ring_sum_rows_kernel, dim3(stream_grid(rows, 4)), dim3(256), 0, s, a, out, rows, cols, bits);
  return hipGetLastError();
}

// ---------------------------------------------------------------------- lift
// out[b][k][z] = lift59_residue(v, q_k), the signed value of the ring-2^59 word
// v as a canonical residue mod q_k.  width = 0: v = ring[b][z] over all N
// coefficients (matrix.cu:23-26).  width > 0: the resident token layout
// (resident.cu:23-30), v = ring[b][width-1-z] for z < width, 0 above.  The
// plans fuse this into the forward NTT's loads (launch_ntt_lift); this kernel
// serves praghip_lift59.
__global__ void lift59_kernel(const uint64_t* __restrict__ ring, uint64_t* __restrict__ out, size_t blocks,
                              int log_n, size_t width, PrimeList q) {
  const size_t n = size_t(1) << log_n, P = size_t(q.count), total = blocks * P * n;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t z = i & (n - 1), k = (i >> log_n) % P, b = (i >> log_n) / P;
    uint64_t v = 0;
    if (width == 0)
      v = ring[(b << log_n) + z];
    else if (z < width)
      v = ring[b * width + (width - 1 - z)];
    else {
      out[i] = 0;
      continue;
    }
    out[i] = lift59_residue(v, q.q[k]);
  }
}

hipError_t launch_lift59(const uint64_t* ring, uint64_t* out, size_t blocks, int log_n, size_t width,
                         const PrimeList& q, hipStream_t s) {
  const size_t total = (blocks * size_t(q.count)) << log_n;
  hipLaunchKernelGGL(lift59_kernel, dim3(stream_grid(total, 256)), dim3(256), 0, s, ring, out, blocks, log_n, width,
                     q);
  return hipGetLastError();
}

// ------------------------------------------------------------- dyadic MAC
// out[l][z] = sum_b a[b][l][z] * w[b][l % wl][z] mod q_{l % P}: the Barrett-128
// products of resident.cu:38-45 / matrix.cu:34-38, summed with a conditional
// subtraction per block.  One thread per output word, the block loop inside.
__global__ void dyadic_mac_kernel(const uint64_t* __restrict__ a, const uint64_t* __restrict__ w,
                                  uint64_t* __restrict__ out, size_t blocks, size_t limbs, int log_n, size_t w_limbs,
                                  BarrettList bl) {
  const size_t n = size_t(1) << log_n, words = limbs << log_n;
  const size_t stride = size_t(gridDim.x) * blockDim.x;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) {
    const size_t l = i >> log_n, z = i & (n - 1);
    const Barrett m = bl.m[l % unsigned(bl.count)];
    const size_t wo = ((l % w_limbs) << log_n) + z;
    uint64_t sum = 0;
    for (size_t b = 0; b < blocks; ++b) {
      sum += mul_barrett(a[b * words + i], w[b * (w_limbs << log_n) + wo], m);
      sum = sum >= m.q ? sum - m.q : sum;
    }
    out[i] = sum;
  }
}

hipError_t launch_dyadic_mac(const uint64_t* a, const uint64_t* w, uint64_t* out, size_t blocks, size_t limbs,
                             int log_n, size_t w_limbs, const Barrett* m, int primes, hipStream_t s) {
  BarrettList bl{};
  for (int i = 0; i < primes; ++i) bl.m[i] = m[i];
  bl.count = primes;
  hipLaunchKernelGGL(dyadic_mac_kernel, dim3(stream_grid(limbs << log_n, 256)), dim3(256), 0, s, a, w, out, blocks,
                     limbs, log_n, w_limbs, bl);
  return hipGetLastError();
}

// ------------------------------------------------- local dot + Delta scaling
// Pass 1: partial[slot][g] = sum over this workgroup's words of s[j] * w[j]
// (mod 2^64), kLocalTiles workgroups per slot.  Pass 2, one workgroup per
// slot: m = (sum of the partials) & (2^59 - 1), then per prime
//   scaled_k = Delta_k * m + floor((r * m + 2^58) / 2^59)   mod q_k.
// The floor term is below 2^59 + 1; it is reduced mod q_k before the add, so
// primes below 2^59 are handled too (the reference's single conditional
// subtraction covers its 60-bit primes only, where both agree).
struct ScaleConst {
  Barrett m[kMaxKeyPrimes];
  uint64_t delta[kMaxKeyPrimes];
  int count;
  uint64_t r;
};

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* lds) {
#pragma unroll
  for (int d = 32; d; d >>= 1) v += __shfl_xor(v, d, 64);
  const unsigned lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  uint64_t s = 0;
  for (unsigned i = 0; i < (blockDim.x >> 6); ++i) s += lds[i];
  return s;
}

// Row y of the grid is (coordinate y / slots, slot y % slots): the slot's
// shares against that coordinate's weights (coordinate c at weights + c words).
__global__ void __launch_bounds__(256) local_dot_kernel(const uint64_t* __restrict__ shares,
                                                        const uint64_t* __restrict__ weights, size_t words,
                                                        size_t slots, uint64_t* __restrict__ partial) {
  __shared__ uint64_t lds[4];
  const size_t y = blockIdx.y, g = blockIdx.x;
  const uint64_t* s = shares + (y % slots) * words;
  const uint64_t* w = weights + (y / slots) * words;
  uint64_t acc = 0;
  for (size_t j = g * blockDim.x + threadIdx.x; j < words; j += size_t(gridDim.x) * blockDim.x) acc += s[j] * w[j];
  const uint64_t tot = block_sum_u64(acc, lds);
  if (threadIdx.x == 0) partial[y * gridDim.x + g] = tot;
}

__global__ void __launch_bounds__(256) local_scale_kernel(const uint64_t* __restrict__ partial, unsigned tiles,
                                                          ScaleConst sc, uint64_t* __restrict__ scaled) {
  __shared__ uint64_t lds[4];
  const size_t slot = blockIdx.x;
  uint64_t acc = 0;
  for (unsigned j = threadIdx.x; j < tiles; j += blockDim.x) acc += partial[slot * tiles + j];
  const uint64_t sum = block_sum_u64(acc, lds);
  if (threadIdx.x < unsigned(sc.count)) {
    const unsigned k = threadIdx.x;
    const uint64_t m = sum & ((1ull << 59) - 1);
    // floor((r m + 2^58) / 2^59) of the 128-bit r m: add the half to the low
    // word, carry into the high word, keep bits 59..122
    const uint64_t rm_lo = m * sc.r, rm_hi = __umul64hi(m, sc.r);
    const uint64_t half_lo = rm_lo + (1ull << 58), half_hi = rm_hi + (half_lo < rm_lo ? 1 : 0);
    const uint64_t fix = (half_hi << 5) | (half_lo >> 59);  // < 2^59 + 1
    const Barrett b = sc.m[k];
    const uint64_t z = mul_barrett(m, sc.delta[k], b);
    scaled[slot * unsigned(sc.count) + k] = add_mod(z, fix % b.q, b.q);
  }
}

// coords > 1: `coords` weight columns of `words` each, one after the other;
// scaled is [coords][slots][primes] and work [coords * slots][kLocalTiles].
hipError_t launch_local_dot_scale(const uint64_t* shares, const uint64_t* weights, size_t words, size_t slots,
                                  const uint64_t* delta, uint64_t r, const Barrett* m, int primes, uint64_t* scaled,
                                  uint64_t* work, hipStream_t s, size_t coords) {
  ScaleConst sc{};
  for (int i = 0; i < primes; ++i) {
    sc.m[i] = m[i];
    sc.delta[i] = delta[i];
  }
  sc.count = primes;
  sc.r = r;
  const unsigned tiles = unsigned(std::min<size_t>(kLocalTiles, std::max<size_t>(1, (words + 255) / 256)));
  const unsigned rows = unsigned(slots * coords);
  hipLaunchKernelGGL(local_dot_kernel, dim3(tiles, rows), dim3(256), 0, s, shares, weights, words, slots, work);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(local_scale_kernel, dim3(rows), dim3(256), 0, s, work, tiles, sc, scaled);
  return hipGetLastError();
}

// ------------------------------------------- allocation-free local dot scratch
// The per-tile partial sums of up to kNoAllocSlots slot rows of the local dot,
// for callers that cannot allocate device memory.  Each device holds its own
// copy until the process ends, and every call on a device shares it: calls that
// overlap on one device race.  Every word a call reads was written by the same
// call's first kernel, so nothing needs clearing.
static __device__ __align__(256) uint64_t scratch[kNoAllocSlots * kLocalTiles];

namespace {
constexpr int kScratchDevices = 64;
std::mutex scratch_mutex;
uint64_t* scratch_address[kScratchDevices] = {};
}  // namespace

// Device address of `scratch` on `device`, which must be the current device.
// Looked up once per device; the host-side name of the array is not a device
// address and is never passed to a kernel or a copy.
hipError_t local_dot_scratch(int device, uint64_t** address) {
  if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_address[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    scratch_address[device] = static_cast<uint64_t*>(p);
  }
  *address = scratch_address[device];
  return hipSuccess;
}

}  // namespace praghip
