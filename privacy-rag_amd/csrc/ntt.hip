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

// Kernel over the limbs whose prime uses arithmetic A: virtual index v maps to
// limb (v / C) * P + sel[v % C], where sel lists the C prime indices of that
// arithmetic.  Workgroup g transforms v = g, g + G, ... (G resident
// workgroups).  Each limb is loaded in the first pass's layout (coalesced),
// transformed in registers + LDS and stored in the last pass's layout.  The
// float-path forward kernel issues the next limb's loads as soon as the
// current limb no longer needs the LDS (before its last pass), so they overlap
// the last pass and the stores instead of starting after them.  The
// float-path inverse kernel loads the next limb's first-pass twiddles before
// the current limb's stores and its words after them; the other kernels have
// no registers to spare and load each limb at the top of its turn.
//
// LIFT (forward only): limb l = b P + k is not read from data but formed on
// load from ring block b, lift59_residue mod q_k (ring[b][z] when width = 0;
// ring[b][width-1-z] for z < width and 0 above otherwise), so the lifted limbs
// never pass through memory.
struct NttLift {
  const uint64_t* ring = nullptr;
  size_t width = 0;
};

template <int LOGN, bool INV, class A, bool LIFT = false>
__global__ void __launch_bounds__(ntt_threads<LOGN>())
    ntt_kernel(uint64_t* __restrict__ data, size_t count, const NttPrime* __restrict__ primes,
               const typename A::TW* __restrict__ tw, int P, const int* __restrict__ sel, int C, NttLift lift) {
  __shared__ __attribute__((aligned(16))) uint64_t lds[(1 << LOGN) + (1 << LOGN) / 16];
  using T = typename A::T;
  const unsigned t = threadIdx.x;
  const auto limb_of = [&](size_t v) { return (v / unsigned(C)) * unsigned(P) + unsigned(sel[v % unsigned(C)]); };
  const auto in_index = [&](int j) { return INV ? inv_in_index<LOGN>(t, j) : fwd_in_index<LOGN>(t, j); };
  // the input words of limb `limb` in the first pass's register layout (with
  // LIFT the ring words, lifted by `lifted` once the limb's turn comes)
  const auto load = [&](uint64_t (&raw)[kE], size_t limb) {
    if constexpr (LIFT) {
      // coefficient z reads base[sign * z]: base = ring[b] (sign +1), or the
      // last word of the token block ring[b][width - 1] (sign -1, z < width)
      const size_t b = limb / unsigned(P);
      const bool rev = lift.width != 0;
      const uint64_t* base = lift.ring + (rev ? b * lift.width + lift.width - 1 : b << LOGN);
      const long long sign = rev ? -1 : 1;
      const unsigned limit = rev ? unsigned(lift.width) : (1u << LOGN);
#pragma unroll
      for (int j = 0; j < kE; ++j) {
        const unsigned z = in_index(j);
        raw[j] = z < limit ? base[sign * (long long)z] : 0;
      }
    } else {
      const uint64_t* x = data + (limb << LOGN);
#pragma unroll
      for (int j = 0; j < kE; ++j) raw[j] = x[in_index(j)];
    }
  };
  const auto lifted = [&](uint64_t v, const NttPrime& pr) {
    if constexpr (LIFT)
      return lift59_residue(v, pr);
    else
      return v;
  };
  const auto store = [&](const A& ar, T (&x)[kE], size_t limb) {
    uint64_t* out = data + (limb << LOGN);
    if (!INV) {
#pragma unroll
      for (int j = 0; j < kE; j += 2)
        *reinterpret_cast<ulonglong2*>(out + fwd_out_index<LOGN>(t, j)) =
            make_ulonglong2(ar.to_u64_fwd(x[j]), ar.to_u64_fwd(x[j + 1]));
    } else {
#pragma unroll
      for (int j = 0; j < kE; ++j) out[inv_out_index<LOGN>(t, j)] = ar.to_u64_inv(x[j]);
    }
  };
  if constexpr (std::is_same<T, double>::value && !INV) {
    size_t v = blockIdx.x;
    if (v >= count) return;
    uint64_t raw[kE];
    load(raw, limb_of(v));
    for (; v < count; v += gridDim.x) {
      const size_t limb = limb_of(v);
      const int p = int(limb % unsigned(P));
      const NttPrime pr = primes[p];
      const A ar(pr);
      T x[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) x[j] = ar.from_u64(lifted(raw[j], pr));
      const size_t vn = v + gridDim.x;
      ntt_regs<LOGN, INV>(x, reinterpret_cast<T*>(lds), t, tw + (size_t(p) << LOGN), ar, pr, [&] {
        if (vn < count) load(raw, limb_of(vn));
      });
      store(ar, x, limb);
    }
  } else if constexpr (std::is_same<T, double>::value && INV) {
    // the next limb's first-pass twiddles are loaded before this limb's
    // stores (vector memory operations complete in order: issued behind the
    // stores they would wait for them, and the first pass waits for its
    // twiddles); its words after them (before the stores as well, they cost
    // registers and measured no faster)
    size_t v = blockIdx.x;
    if (v >= count) return;
    uint64_t raw[kE];
    typename A::TW w0[pass_twiddles<Passes<LOGN>::r(INV, 0)>()];
    {
      const size_t limb = limb_of(v);
      load(raw, limb);
      load_pass_twiddles<LOGN, INV, 0>(w0, t, tw + ((limb % unsigned(P)) << LOGN));
    }
    for (; v < count; v += gridDim.x) {
      const size_t limb = limb_of(v);
      const int p = int(limb % unsigned(P));
      const NttPrime pr = primes[p];
      const A ar(pr);
      T x[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) x[j] = ar.from_u64(raw[j]);
      run_passes<LOGN, INV, 0>(x, reinterpret_cast<T*>(lds), t, tw + (size_t(p) << LOGN), ar, pr, w0, [] {});
      const size_t vn = v + gridDim.x;
      if (vn < count) load_pass_twiddles<LOGN, INV, 0>(w0, t, tw + ((limb_of(vn) % unsigned(P)) << LOGN));
      store(ar, x, limb);
      if (vn < count) load(raw, limb_of(vn));
    }
  } else {
    for (size_t v = blockIdx.x; v < count; v += gridDim.x) {
      const size_t limb = limb_of(v);
      const int p = int(limb % unsigned(P));
      const NttPrime pr = primes[p];
      const A ar(pr);
      uint64_t raw[kE];
      load(raw, limb);
      T x[kE];
#pragma unroll
      for (int j = 0; j < kE; ++j) x[j] = ar.from_u64(lifted(raw[j], pr));
      ntt_regs<LOGN, INV>(x, reinterpret_cast<T*>(lds), t, tw + (size_t(p) << LOGN), ar, pr);
      store(ar, x, limb);
    }
  }
}

// Resident workgroups per CU times the CU count, cached per kernel.
template <int LOGN, bool INV, class A, bool LIFT>
static unsigned persistent_grid() {
  static unsigned grid = 0;
  if (!grid) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, ntt_kernel<LOGN, INV, A, LIFT>, ntt_threads<LOGN>(), 0) !=
            hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    grid = unsigned(cus * per_cu);
  }
  return grid;
}

// Number of limbs among the first `limbs` whose prime index is in sel[0..C).
static size_t subset_count(size_t limbs, int P, const int* host_sel, int C) {
  size_t count = (limbs / unsigned(P)) * unsigned(C);
  const size_t tail = limbs % unsigned(P);
  for (int c = 0; c < C; ++c) count += size_t(host_sel[c]) < tail ? 1 : 0;
  return count;
}

template <int LOGN, bool INV, class A, bool LIFT = false>
static hipError_t launch_subset(uint64_t* data, size_t limbs, const NttDevice& d, const typename A::TW* tw,
                                const int* sel_dev, const int* sel_host, int C, hipStream_t s, NttLift lift = {}) {
  if (!C) return hipSuccess;
  const size_t count = subset_count(limbs, d.P, sel_host, C);
  if (!count) return hipSuccess;
  const dim3 block{unsigned(ntt_threads<LOGN>())};
  const dim3 grid{unsigned(std::min<size_t>(count, persistent_grid<LOGN, INV, A, LIFT>()))};
  hipLaunchKernelGGL((ntt_kernel<LOGN, INV, A, LIFT>), grid, block, 0, s, data, count, d.primes, tw, d.P, sel_dev, C,
                     lift);
  return hipGetLastError();
}

template <class A>
struct TypeTag {
  using type = A;
};

template <int LOGN>
static hipError_t launch_ntt_n(bool inverse, uint64_t* data, size_t limbs, const NttDevice& d,
                               hipStream_t s) {
  // integer-path primes all below 2^60: the lazy transforms (ArU64L)
  const auto u64 = [&](auto tag, bool inv) {
    using A = typename decltype(tag)::type;
    return inv ? launch_subset<LOGN, true, A>(data, limbs, d, d.tw_inv_u, d.sel_u64, d.host_sel_u64, d.n_u64, s)
               : launch_subset<LOGN, false, A>(data, limbs, d, d.tw_fwd_u, d.sel_u64, d.host_sel_u64, d.n_u64, s);
  };
  hipError_t e;
  if (inverse)
    e = launch_subset<LOGN, true, ArF64T>(data, limbs, d, d.tw_inv_f, d.sel_f64, d.host_sel_f64, d.n_f64, s);
  else
    e = launch_subset<LOGN, false, ArF64T>(data, limbs, d, d.tw_fwd_f, d.sel_f64, d.host_sel_f64, d.n_f64, s);
  if (e == hipSuccess && d.n_u64) e = d.lazy_u64 ? u64(TypeTag<ArU64L>{}, inverse) : u64(TypeTag<ArU64>{}, inverse);
  return e;
}

template <int LOGN>
static hipError_t launch_ntt_lift_n(const uint64_t* ring, size_t width, uint64_t* out, size_t limbs,
                                    const NttDevice& d, hipStream_t s) {
  const NttLift lift{ring, width};
  return d.lazy_u64 ? launch_subset<LOGN, false, ArU64L, true>(out, limbs, d, d.tw_fwd_u, d.sel_u64, d.host_sel_u64,
                                                               d.n_u64, s, lift)
                    : launch_subset<LOGN, false, ArU64, true>(out, limbs, d, d.tw_fwd_u, d.sel_u64, d.host_sel_u64,
                                                              d.n_u64, s, lift);
}

// Every prime on the integer path: the lift is done by the transform's loads.
// With float-path primes (whose kernel has no registers left for the lift's
// arithmetic) the lift kernel writes the limbs first and the transform runs
// in place.
hipError_t launch_ntt_lift(const uint64_t* ring, size_t width, uint64_t* out, size_t blocks, const PrimeList& pl,
                           const NttDevice& d, hipStream_t s) {
  const size_t limbs = blocks * size_t(d.P);
  if (limbs == 0) return hipSuccess;
  if (d.n_f64) {
    const hipError_t e = launch_lift59(ring, out, blocks, d.log_n, width, pl, s);
    return e == hipSuccess ? launch_ntt(false, out, limbs, d, s) : e;
  }
  switch (d.log_n) {
    case 4: return launch_ntt_lift_n<4>(ring, width, out, limbs, d, s);
    case 5: return launch_ntt_lift_n<5>(ring, width, out, limbs, d, s);
    case 6: return launch_ntt_lift_n<6>(ring, width, out, limbs, d, s);
    case 7: return launch_ntt_lift_n<7>(ring, width, out, limbs, d, s);
    case 8: return launch_ntt_lift_n<8>(ring, width, out, limbs, d, s);
    case 9: return launch_ntt_lift_n<9>(ring, width, out, limbs, d, s);
    case 10: return launch_ntt_lift_n<10>(ring, width, out, limbs, d, s);
    case 11: return launch_ntt_lift_n<11>(ring, width, out, limbs, d, s);
    case 12: return launch_ntt_lift_n<12>(ring, width, out, limbs, d, s);
    case 13: return launch_ntt_lift_n<13>(ring, width, out, limbs, d, s);
    case 14: return launch_ntt_lift_n<14>(ring, width, out, limbs, d, s);
    default: return hipErrorInvalidValue;
  }
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
