// Negacyclic NTT / INTT core for gfx950: one workgroup per limb of N = 2^LOGN
// coefficients, N/16 threads, 16 coefficients per thread held in registers.
//
// The transform is the reference's radix-2 stage sequence (ntt.cu:104-127,
// stage() ntt.cu:42-53): forward stage s has gap N>>(s+1) and twiddle
// fwd[(1<<s) + group]; inverse stage l has gap 1<<l and twiddle
// inv[N-(N>>l)+1+group], and the last inverse stage scales by N^-1.  Those
// stages are grouped four at a time into radix-16 register passes: a pass
// over the gap bits [LO, LO+R) gives each thread the 2^R coefficients that
// differ only in those bits.  Between passes the limb is exchanged through LDS
// (one 8-byte slot per coefficient plus one pad slot per 16, which keeps every
// pass's access pattern free of bank conflicts).
//
// Arithmetic policies:
//   ArU64 - any q < 2^62: Harvey's lazy butterflies (forward values in [0,4q),
//           inverse in [0,2q)) over Shoup twiddles, canonicalised at the end;
//   ArF64 - q < 2^50: residues as exact doubles, FMA-based products, centred
//           values re-centred every second stage.
// Both produce the canonical residue of the same transform, so the result is
// bit-identical to the reference whatever the path.
#pragma once
#include "modarith.hpp"

namespace praghip {

// Per-prime constants of a plan (device copy).
struct NttPrime {
  uint64_t q, q2;             // q, 2q
  uint64_t ninv, ninv_q;      // N^-1 mod q (Shoup pair)
  uint64_t last, last_q;      // w_last * N^-1 (Shoup pair), w_last = inv[N-1]
  double qd, qinv;            // q and 1/q as doubles (float path)
  double ninv_f, ninv_fq;     // N^-1 as (w, w/q)
  double last_f, last_fq;     // w_last * N^-1 as (w, w/q)
  int use_f64;                // q < 2^50: the float path is exact
  int pad;
};

__device__ __forceinline__ unsigned lds_pos(unsigned x) { return x + (x >> 4); }

// Index of the j-th register coefficient of thread t in a pass over the gap
// bits [LO, LO+R).  When R < 4 each thread runs 16>>R independent radix-2^R
// blocks; SUB_MINOR puts the block number in the low bits of the thread's
// identity (16 consecutive coefficients per thread), otherwise in the high bits
// (consecutive threads on consecutive coefficients).
template <int LOGN, int LO, int R, bool SUB_MINOR>
__device__ __forceinline__ unsigned elem_index(unsigned t, int j) {
  constexpr int SUB = 16 >> R;
  constexpr unsigned THREADS = (1u << LOGN) / 16;
  const int b = j >> R, jl = j & ((1 << R) - 1);
  const unsigned T = SUB_MINOR ? (t * SUB + b) : (t + unsigned(b) * THREADS);
  const unsigned lo = T & ((1u << LO) - 1), hi = T >> LO;
  return (hi << (LO + R)) | (unsigned(jl) << LO) | lo;
}

// ---------------------------------------------------------------- policies
struct ArU64 {
  using T = uint64_t;
  using TW = ulonglong2;
  uint64_t q, q2;
  __device__ explicit ArU64(const NttPrime& p) : q(p.q), q2(p.q2) {}
  __device__ __forceinline__ T from_u64(uint64_t x) const { return x; }
  __device__ __forceinline__ uint64_t to_u64_fwd(T x) const {  // [0,4q) -> [0,q)
    x = x >= q2 ? x - q2 : x;
    return x >= q ? x - q : x;
  }
  __device__ __forceinline__ uint64_t to_u64_inv(T x) const { return x >= q ? x - q : x; }  // [0,2q)
  __device__ __forceinline__ void fwd(T& x, T& y, TW w) const {  // CT, values in [0,4q)
    T a = x >= q2 ? x - q2 : x;
    const T t = mul_shoup_lazy(y, w.x, w.y, q);
    x = a + t;
    y = a - t + q2;
  }
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {  // GS, values in [0,2q)
    T s = x + y;
    s = s >= q2 ? s - q2 : s;
    const T d = x - y + q2;
    x = s;
    y = mul_shoup_lazy(d, w.x, w.y, q);
  }
  __device__ __forceinline__ void inv_last(T& x, T& y, const NttPrime& p) const {
    const T s = x + y, d = x - y + q2;
    x = mul_shoup_lazy(s, p.ninv, p.ninv_q, q);
    y = mul_shoup_lazy(d, p.last, p.last_q, q);
  }
  __device__ __forceinline__ void settle(T&) const {}
};

struct ArF64 {
  using T = double;
  using TW = double2;
  double q, qinv;
  __device__ explicit ArF64(const NttPrime& p) : q(p.qd), qinv(p.qinv) {}
  __device__ __forceinline__ T from_u64(uint64_t x) const { return (double)x; }
  __device__ __forceinline__ uint64_t to_u64(T x) const {
    x = reduce_f64(x, q, qinv);
    x = x < 0.0 ? x + q : x;
    return (uint64_t)x;
  }
  __device__ __forceinline__ uint64_t to_u64_fwd(T x) const { return to_u64(x); }
  __device__ __forceinline__ uint64_t to_u64_inv(T x) const { return to_u64(x); }
  __device__ __forceinline__ void fwd(T& x, T& y, TW w) const {
    const T t = mul_f64(y, w.x, w.y, q);
    const T a = x;
    x = a + t;
    y = a - t;
  }
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {
    const T s = x + y, d = x - y;
    x = reduce_f64(s, q, qinv);
    y = mul_f64(d, w.x, w.y, q);
  }
  __device__ __forceinline__ void inv_last(T& x, T& y, const NttPrime& p) const {
    const T s = x + y, d = x - y;
    x = mul_f64(s, p.ninv_f, p.ninv_fq, q);
    y = mul_f64(d, p.last_f, p.last_fq, q);
  }
  __device__ __forceinline__ void settle(T& x) const { x = reduce_f64(x, q, qinv); }
};

// ------------------------------------------------------------------ passes
// Forward radix-2^R pass over gap bits [LO, LO+R): global stages
// s = LOGN-LO-R .. LOGN-LO-1.
template <int LOGN, int LO, int R, bool SUB_MINOR, class A>
__device__ __forceinline__ void fwd_pass(typename A::T (&v)[16], unsigned t,
                                         const typename A::TW* __restrict__ tw, const A& ar) {
  constexpr int SUB = 16 >> R;
  constexpr unsigned THREADS = (1u << LOGN) / 16;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
    const unsigned T = SUB_MINOR ? (t * SUB + b) : (t + unsigned(b) * THREADS);
    const unsigned hi = T >> LO;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int s = LOGN - LO - R + i, g = R - 1 - i;
#pragma unroll
      for (int k = 0; k < (1 << i); ++k) {
        const typename A::TW w = tw[(1u << s) + (hi << i) + k];
#pragma unroll
        for (int m = 0; m < (1 << g); ++m) {
          const int j0 = (b << R) | (k << (g + 1)) | m, j1 = j0 | (1 << g);
          ar.fwd(v[j0], v[j1], w);
        }
      }
      if (s & 1) {
#pragma unroll
        for (int m = 0; m < (1 << R); ++m) ar.settle(v[(b << R) | m]);
      }
    }
  }
}

// Inverse radix-2^R pass over gap bits [LO, LO+R): stages l = LO .. LO+R-1.
template <int LOGN, int LO, int R, bool SUB_MINOR, class A>
__device__ __forceinline__ void inv_pass(typename A::T (&v)[16], unsigned t,
                                         const typename A::TW* __restrict__ tw, const A& ar,
                                         const NttPrime& pr) {
  constexpr int SUB = 16 >> R;
  constexpr unsigned N = 1u << LOGN, THREADS = N / 16;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
    const unsigned T = SUB_MINOR ? (t * SUB + b) : (t + unsigned(b) * THREADS);
    const unsigned hi = T >> LO;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int l = LO + i;
      if (l == LOGN - 1) {  // last stage: one group, twiddle and N^-1 folded
#pragma unroll
        for (int m = 0; m < (1 << i); ++m) {
          const int j0 = (b << R) | m, j1 = j0 | (1 << i);
          ar.inv_last(v[j0], v[j1], pr);
        }
      } else {
#pragma unroll
        for (int k = 0; k < (1 << (R - 1 - i)); ++k) {
          const unsigned group = (hi << (R - 1 - i)) + k;
          const typename A::TW w = tw[N - (N >> l) + 1 + group];
#pragma unroll
          for (int m = 0; m < (1 << i); ++m) {
            const int j0 = (b << R) | (k << (i + 1)) | m, j1 = j0 | (1 << i);
            ar.inv(v[j0], v[j1], w);
          }
        }
      }
    }
  }
}

template <int LOGN, int LO0, int R0, bool SM0, int LO1, int R1, bool SM1, class T>
__device__ __forceinline__ void exchange(T (&v)[16], T* lds, unsigned t) {
#pragma unroll
  for (int j = 0; j < 16; ++j) lds[lds_pos(elem_index<LOGN, LO0, R0, SM0>(t, j))] = v[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = lds[lds_pos(elem_index<LOGN, LO1, R1, SM1>(t, j))];
  __syncthreads();
}

template <int LOGN>
struct Passes {
  static constexpr int NP = (LOGN + 3) / 4;
  static constexpr int RLAST = LOGN - 4 * (NP - 1);
  // forward: high bits first; the last pass is [0, RLAST) with SUB_MINOR
  static constexpr int fwd_lo(int p) { return p < NP - 1 ? LOGN - 4 * (p + 1) : 0; }
  static constexpr int fwd_r(int p) { return p < NP - 1 ? 4 : RLAST; }
  static constexpr bool fwd_sm(int p) { return p == NP - 1; }
  // inverse: low bits first; the last pass is [LOGN-RLAST, LOGN) block-major
  static constexpr int inv_lo(int p) { return 4 * p; }
  static constexpr int inv_r(int p) { return p < NP - 1 ? 4 : RLAST; }
  static constexpr bool inv_sm(int p) { return p == 0; }
};

template <int LOGN, int P, class A>
__device__ __forceinline__ void fwd_from(typename A::T (&v)[16], typename A::T* lds, unsigned t,
                                         const typename A::TW* tw, const A& ar) {
  using S = Passes<LOGN>;
  fwd_pass<LOGN, S::fwd_lo(P), S::fwd_r(P), S::fwd_sm(P)>(v, t, tw, ar);
  if constexpr (P + 1 < S::NP) {
    exchange<LOGN, S::fwd_lo(P), S::fwd_r(P), S::fwd_sm(P), S::fwd_lo(P + 1), S::fwd_r(P + 1),
             S::fwd_sm(P + 1)>(v, lds, t);
    fwd_from<LOGN, P + 1>(v, lds, t, tw, ar);
  }
}
template <int LOGN, int P, class A>
__device__ __forceinline__ void inv_from(typename A::T (&v)[16], typename A::T* lds, unsigned t,
                                         const typename A::TW* tw, const A& ar, const NttPrime& pr) {
  using S = Passes<LOGN>;
  inv_pass<LOGN, S::inv_lo(P), S::inv_r(P), S::inv_sm(P)>(v, t, tw, ar, pr);
  if constexpr (P + 1 < S::NP) {
    exchange<LOGN, S::inv_lo(P), S::inv_r(P), S::inv_sm(P), S::inv_lo(P + 1), S::inv_r(P + 1),
             S::inv_sm(P + 1)>(v, lds, t);
    inv_from<LOGN, P + 1>(v, lds, t, tw, ar, pr);
  }
}

// Register layouts at the boundaries of a transform:
//   forward input  : element (j << (LOGN-4)) | t   (coalesced across threads)
//   forward output : element (t << 4) | j          (16 consecutive per thread)
//   inverse input  : element (t << 4) | j
//   inverse output : block-major last pass (coalesced across threads)
template <int LOGN>
__device__ __forceinline__ unsigned fwd_in_index(unsigned t, int j) {
  using S = Passes<LOGN>;
  return elem_index<LOGN, S::fwd_lo(0), S::fwd_r(0), S::fwd_sm(0)>(t, j);
}
template <int LOGN>
__device__ __forceinline__ unsigned fwd_out_index(unsigned t, int j) {
  using S = Passes<LOGN>;
  return elem_index<LOGN, S::fwd_lo(S::NP - 1), S::fwd_r(S::NP - 1), S::fwd_sm(S::NP - 1)>(t, j);
}
template <int LOGN>
__device__ __forceinline__ unsigned inv_in_index(unsigned t, int j) {
  using S = Passes<LOGN>;
  return elem_index<LOGN, S::inv_lo(0), S::inv_r(0), S::inv_sm(0)>(t, j);
}
template <int LOGN>
__device__ __forceinline__ unsigned inv_out_index(unsigned t, int j) {
  using S = Passes<LOGN>;
  return elem_index<LOGN, S::inv_lo(S::NP - 1), S::inv_r(S::NP - 1), S::inv_sm(S::NP - 1)>(t, j);
}

// Whole-limb transforms on register data (v holds the input layout on entry
// and the output layout on exit; values stay in the policy's lazy form).
template <int LOGN, class A>
__device__ __forceinline__ void ntt_fwd_regs(typename A::T (&v)[16], typename A::T* lds, unsigned t,
                                             const typename A::TW* tw, const A& ar) {
  fwd_from<LOGN, 0>(v, lds, t, tw, ar);
}
template <int LOGN, class A>
__device__ __forceinline__ void ntt_inv_regs(typename A::T (&v)[16], typename A::T* lds, unsigned t,
                                             const typename A::TW* tw, const A& ar, const NttPrime& pr) {
  inv_from<LOGN, 0>(v, lds, t, tw, ar, pr);
}

constexpr size_t lds_bytes(int log_n) { return (((size_t)1 << log_n) + ((size_t)1 << log_n) / 16) * 8; }

}  // namespace praghip
