// Keyswitch at N = 16384 in three phases (Switch::evaluate, switch.cu:113-125):
// the same radix-2 stage sequence as the whole-limb path, split where a
// transform changes from stride-1024 columns to contiguous 1024-coefficient
// rows, so every phase runs at high occupancy instead of one limb per CU.
//
//   A  columns  ModUp of digit j to every key prime t, then forward stages
//               0-3 (gaps 8192..1024): thread c holds coefficients
//               c + 1024 k, k = 0..15, and every twiddle is the same for all
//               threads.  Out: E[b][j][t][N] (lazy, per-policy form).
//   B  rows     two waves per (ciphertext, prime t, row r): forward stages
//               4-13 of each digit's row, the key product summed over the
//               digits in registers, inverse stages 0-9 of both sums.
//               Out: the products' rows, [b][2][K][N] (lazy).
//   C  columns  inverse stages 10-13 (N^-1 folded into the last): first the
//               special prime's, leaving the ModDown rounding term in place,
//               then every data prime's with ModDown and the c0 term
//               (switch.cu:74-82).
//
// Each phase keeps the stage order, the butterflies and the re-centring
// points of the whole-limb transform, so the values - and the canonical
// result - are the same.  E and the products pass through HBM, about twice
// the algorithmic bytes.  The ciphertexts go in chunks of up to 64 (the
// scratch a plan sizes E for); smaller chunks, which would keep E in the
// last-level cache, leave too few workgroups per launch and are slower.
#include "kernels.hpp"
#include "ntt_core.hpp"

namespace praghip {

namespace {

constexpr int kLog = 14;                 // N = 16384
constexpr int kRowLog = 10;              // rows of 1024
constexpr unsigned kN = 1u << kLog;
constexpr unsigned kCols = 1u << kRowLog;  // columns of stride 1024
constexpr unsigned kRowLds = (1u << kRowLog) + (1u << kRowLog) / 16;  // padded LDS words per wave

struct KsRows {
  const uint64_t* in;   // [batch][2][L][N]
  uint64_t* out;        // [batch][2][L][N]
  const uint64_t* key;  // [dnum][2][K][N] per key
  size_t key_stride;
  unsigned key_group;
  uint64_t* e;          // [chunk][dnum][K][N]
  uint64_t* prod;       // [batch][2][K][N]
  const KsConst* kc;
  const NttPrime* primes;
  const ulonglong2* tw_fwd_u;
  const ulonglong2* tw_inv_u;
  const double* tw_fwd_f;
  const double* tw_inv_f;
  uint32_t ginv;
  int data_f64;     // every data prime below 2^50: data primes take the float path
  int moddown_f64;  // every data prime in (2^32, 2^50): ModDown in FP64 too
  int narrow;       // every key prime below twice every other: x mod q_t by one subtraction
  unsigned b0, cts;  // chunk: ciphertexts b0 .. b0 + cts - 1
};

template <class A>
struct TypeTag {
  using type = A;
};
typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint64_t bits_of(double x) { return (uint64_t)__double_as_longlong(x); }
__device__ __forceinline__ double double_of(uint64_t x) { return __longlong_as_double((long long)x); }

__device__ __forceinline__ uint64_t gather(const uint64_t* __restrict__ limb, unsigned k, uint32_t ginv, uint64_t q) {
  const unsigned i = (k * ginv) & (2 * kN - 1);
  const uint64_t v = limb[i & (kN - 1)];
  return ((i >> kLog) && v) ? q - v : v;
}

// Column c (coefficients c + 1024 k, k < 16) of a limb after the Galois
// gather; a plain strided read when the element is the identity (ginv is a
// launch argument, so the branch is uniform).
__device__ __forceinline__ void gather_column(uint64_t (&y)[kE], const uint64_t* __restrict__ limb, unsigned c,
                                              uint32_t ginv, uint64_t q) {
  if (ginv == 1) {
#pragma unroll
    for (int k = 0; k < kE; ++k) y[k] = limb[c + (unsigned(k) << kRowLog)];
  } else {
#pragma unroll
    for (int k = 0; k < kE; ++k) y[k] = gather(limb, c + (unsigned(k) << kRowLog), ginv, q);
  }
}

// Stored form of a policy value: doubles by their bits, integers as they are.
template <class A>
__device__ __forceinline__ uint64_t store_form(typename A::T x) {
  if constexpr (std::is_same<typename A::T, double>::value)
    return bits_of(x);
  else
    return x;
}
template <class A>
__device__ __forceinline__ typename A::T load_form(uint64_t x) {
  if constexpr (std::is_same<typename A::T, double>::value)
    return double_of(x);
  else
    return x;
}

template <class A>
__device__ __forceinline__ const typename A::TW* fwd_table(const KsRows& f, int t) {
  if constexpr (std::is_same<typename A::T, double>::value)
    return f.tw_fwd_f + (size_t(t) << kLog);
  else
    return f.tw_fwd_u + (size_t(t) << kLog);
}
template <class A>
__device__ __forceinline__ const typename A::TW* inv_table(const KsRows& f, int t) {
  if constexpr (std::is_same<typename A::T, double>::value)
    return f.tw_inv_f + (size_t(t) << kLog);
  else
    return f.tw_inv_u + (size_t(t) << kLog);
}

// ------------------------------------------------------------------ phase A
// Waves per SIMD the forward column kernels are compiled for (the twiddles
// live in scalar registers): one-prime digits need only the 16 values, four
// fit; the base conversion of two- and three-prime digits needs the registers
// of two.
template <int D>
constexpr int kColFwdWaves() {
  return D == 1 ? 4 : 2;
}

// Twiddles of forward stages 0-3 in the order fwd_pass consumes them: one
// group per stage (stage s uses fwd[2^s + k], k < 2^s), i.e. fwd[1..15].
// kScalar: the twiddles are moved to scalar registers (the table index is
// wave-uniform), which frees their VGPRs where the SGPRs are not needed for
// more than one target's values.
template <class A, bool kScalar>
__device__ __forceinline__ void top_fwd(typename A::T (&v)[kE], const typename A::TW* __restrict__ tab, const A& ar) {
  typename A::TW w[pass_twiddles<kLogE>()];
#pragma unroll
  for (int n = 0; n < pass_twiddles<kLogE>(); ++n) w[n] = kScalar ? to_sgpr(tab[1 + n]) : tab[1 + n];
  fwd_pass<kLog, kLog - kLogE, kLogE>(v, w, ar, [] {});
}

// Modup of one target for the float path: y holds [x_i (Q_j/q_i)^-1]_{q_i}
// for the digit's primes.
template <int D>
__device__ __forceinline__ void cols_target_f64(double (&v)[kE], const uint64_t (&y)[D][kE], const KsConst& kc,
                                                int lo, int t, const NttPrime& pt) {
#pragma unroll
  for (int k = 0; k < kE; ++k) v[k] = 0.0;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const double hf = double(kc.hat[lo + d][t].w), hfq = hf * pt.qinv;
#pragma unroll
    for (int k = 0; k < kE; ++k) v[k] += mul_f64(ArF64::from_u64(y[d][k]), hf, hfq, pt.qd);  // |term| < 7q/8
  }
#pragma unroll
  for (int k = 0; k < kE; ++k) v[k] = reduce_f64(v[k], pt.qd, pt.qinv);
}
template <int D>
__device__ __forceinline__ void cols_target_u64(uint64_t (&v)[kE], const uint64_t (&y)[D][kE], const KsConst& kc,
                                                int lo, int t) {
  const uint64_t qt = kc.q[t], qt2 = 2 * qt;
#pragma unroll
  for (int k = 0; k < kE; ++k) v[k] = 0;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const Shoup hf = kc.hat[lo + d][t];
#pragma unroll
    for (int k = 0; k < kE; ++k) {
      const uint64_t a = v[k] + mul_shoup_lazy(y[d][k], hf.w, hf.wq, qt);  // [0, 4 q_t)
      v[k] = a >= qt2 ? a - qt2 : a;
    }
  }
#pragma unroll
  for (int k = 0; k < kE; ++k) v[k] = v[k] >= qt ? v[k] - qt : v[k];
}

// y = [x_i (Q_j/q_i)^-1]_{q_i} for the digit's primes at this thread's
// coefficients, by the policy's arithmetic (exact either way).
template <int D, class A>
__device__ __forceinline__ void digit_factors(uint64_t (&y)[D][kE], const KsRows& f, const KsConst& kc,
                                              const uint64_t* c1, int lo, unsigned c) {
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int i = lo + d;
    const uint64_t qi = kc.q[i];
    const Shoup ih = kc.inv_hat[i];
    const uint64_t* x = c1 + (size_t(i) << kLog);
    if constexpr (std::is_same<typename A::T, double>::value) {
      const NttPrime pi = f.primes[i];
      const double w = double(ih.w), wq = w * pi.qinv;
#pragma unroll
      for (int k = 0; k < kE; ++k) {
        const double v = ArF64::from_u64(gather(x, c + (unsigned(k) << kRowLog), f.ginv, qi));
        y[d][k] = (uint64_t)canon_f64(mul_f64(v, w, wq, pi.qd), pi.qd);
      }
    } else {
#pragma unroll
      for (int k = 0; k < kE; ++k) y[d][k] = mul_shoup(gather(x, c + (unsigned(k) << kRowLog), f.ginv, qi), ih.w, ih.wq, qi);
    }
  }
}

// Targets per integer-path column-forward thread (cols_fwd_body): the
// digit's column is read and its factors y computed once for G targets.
// One-prime digits take every key prime (their stores then overlap the next
// target's stages: 123 -> 103 us at dnum = 6, batch 64); larger digits one
// target, since their factors would not fit the registers beside a second
// target's values.  (The float-path data primes take every target of a digit
// in cols_fwd_float_body.)
template <class A, int D>
constexpr unsigned kColTargets() {
  return std::is_same<typename A::T, double>::value ? 6u : (D == 1 ? 7u : 1u);
}

// x mod q_t for a canonical residue x of another key prime: one conditional
// subtraction when every key prime is below twice every other (`narrow`; the
// reference's decomposition at switch.cu:63-68 and its ModDown at :74-82 rely
// on it for the locked primes), a Shoup product by 1 otherwise.
__device__ __forceinline__ uint64_t reduce_to(uint64_t x, const KsConst& kc, int t, int narrow) {
  const uint64_t qt = kc.q[t];
  if (narrow) return x >= qt ? x - qt : x;
  return mul_shoup(x, 1, kc.one_q[t], qt);
}

// One thread per (ciphertext, digit, group of up to G targets, column), for
// the targets t_lo .. t_lo + t_n - 1 of one arithmetic policy (A = ArF64Lean:
// float-path data primes; ArU64: the integer-path primes); digits of exactly
// D primes.
template <int D, class A, unsigned G>
__device__ __forceinline__ void cols_fwd_body(const KsRows& f, unsigned t_lo, unsigned t_n, unsigned blk) {
  using T = typename A::T;
  const KsConst& kc = *f.kc;
  const unsigned dnum = unsigned(kc.dnum), K = unsigned(kc.K), L = unsigned(kc.L);
  const unsigned groups = (t_n + G - 1) / G;
  const unsigned gid = blk * blockDim.x + threadIdx.x;
  if (gid >= f.cts * dnum * groups * kCols) return;
  // kCols is a multiple of the wave size, so w is the same for every lane of
  // a wave; on the integer path readfirstlane lets the targets' twiddle pairs
  // live in scalar registers (the float path keeps its six targets' in VGPRs)
  unsigned w = gid >> kRowLog;
  if constexpr (!std::is_same<typename A::T, double>::value) w = __builtin_amdgcn_readfirstlane(w);
  const unsigned c = gid & (kCols - 1);
  const unsigned g = w % groups, j = (w / groups) % dnum, bl = w / (groups * dnum), b = f.b0 + bl;
  const int lo = kc.dig_lo[j];
  const uint64_t* c1 = f.in + ((size_t(b) * 2 + 1) * L << kLog);
  uint64_t y[D][kE];
  const unsigned t_first = t_lo + g * G, t_end = t_lo + (g * G + G < t_n ? g * G + G : t_n);
  if constexpr (D == 1) {
    // one prime per digit: (Q_j / q_i) = 1, so the digit expands to its own
    // canonical residues, reduced mod each target below
    gather_column(y[0], c1 + (size_t(lo) << kLog), c, f.ginv, kc.q[lo]);
  } else if (G > 1) {
    digit_factors<D, A>(y, f, kc, c1, lo, c);
  }
  for (unsigned t = t_first; t < t_end; ++t) {
    const NttPrime pt = f.primes[t];
    const A ar(pt);
    T v[kE];
    if constexpr (D == 1) {
      if (int(t) == lo) {
#pragma unroll
        for (int k = 0; k < kE; ++k) v[k] = ar.from_u64(y[0][k]);
      } else {
#pragma unroll
        for (int k = 0; k < kE; ++k) v[k] = ar.from_u64(reduce_to(y[0][k], kc, int(t), f.narrow));
      }
    } else if (int(t) >= lo && int(t) < lo + D) {  // a prime of the digit: its own residues
#pragma unroll
      for (int k = 0; k < kE; ++k)
        v[k] = ar.from_u64(gather(c1 + (size_t(t) << kLog), c + (unsigned(k) << kRowLog), f.ginv, pt.q));
    } else {
      if (G == 1) digit_factors<D, A>(y, f, kc, c1, lo, c);
      if constexpr (std::is_same<T, double>::value)
        cols_target_f64<D>(v, y, kc, lo, int(t), pt);
      else
        cols_target_u64<D>(v, y, kc, lo, int(t));
    }
    top_fwd<A, D == 1>(v, fwd_table<A>(f, int(__builtin_amdgcn_readfirstlane(t))), ar);  // t is wave-uniform
    uint64_t* et = f.e + ((size_t(bl) * dnum + j) * K + t) * kN + c;
#pragma unroll
    for (int k = 0; k < kE; ++k) et[unsigned(k) << kRowLog] = store_form<A>(v[k]);
  }
}

// One policy per launch (every prime on the integer path).
template <int D, class A, unsigned G>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kColFwdWaves<D>())))
    ks_cols_fwd_kernel(KsRows f, unsigned t_lo, unsigned t_n) {
  cols_fwd_body<D, A, G>(f, t_lo, t_n, blockIdx.x);
}

// The float-path data primes of one digit column in one thread: thread
// (ciphertext, digit j, column c) reads the digit's D residues at its column
// once, transforms them as the digit's own targets, turns them into the
// factors [x (Q_j/q_i)^-1]_{q_i} in place and base-converts them to every
// other data prime.  `w` names the (ciphertext, digit, 256 columns) the
// workgroup takes, as in cols_fwd_body with one target group.
template <int D>
__device__ __forceinline__ void cols_fwd_float_body(const KsRows& f, unsigned w_blk) {
  const KsConst& kc = *f.kc;
  const unsigned dnum = unsigned(kc.dnum), K = unsigned(kc.K), L = unsigned(kc.L);
  const unsigned gid = w_blk * blockDim.x + threadIdx.x;
  if (gid >= f.cts * dnum * kCols) return;
  const unsigned w = __builtin_amdgcn_readfirstlane(gid >> kRowLog);  // kCols is a multiple of the wave size
  const unsigned c = gid & (kCols - 1), j = w % dnum, bl = w / dnum, b = f.b0 + bl;
  const int lo = kc.dig_lo[j];
  const uint64_t* c1 = f.in + ((size_t(b) * 2 + 1) * L << kLog);
  uint64_t* eb = f.e + (size_t(bl) * dnum + j) * K * kN + c;
  const auto store = [&](int t, const double (&v)[kE]) {
    uint64_t* et = eb + (size_t(t) << kLog);
#pragma unroll
    for (int k = 0; k < kE; ++k) et[unsigned(k) << kRowLog] = bits_of(v[k]);
  };
  uint64_t y[D][kE];
#pragma unroll
  for (int d = 0; d < D; ++d) gather_column(y[d], c1 + (size_t(lo + d) << kLog), c, f.ginv, kc.q[lo + d]);
  // the digit's own primes: their residues as they are
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const ArF64Lean ar(f.primes[lo + d]);
    double v[kE];
#pragma unroll
    for (int k = 0; k < kE; ++k) v[k] = ArF64::from_u64(y[d][k]);
    top_fwd<ArF64Lean, true>(v, f.tw_fwd_f + (size_t(lo + d) << kLog), ar);
    store(lo + d, v);
  }
  if constexpr (D > 1) {  // factors in place (exact FP64 products, canonical)
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const NttPrime pi = f.primes[lo + d];
      const double iw = double(kc.inv_hat[lo + d].w), iwq = iw * pi.qinv;
#pragma unroll
      for (int k = 0; k < kE; ++k)
        y[d][k] = (uint64_t)canon_f64(mul_f64(ArF64::from_u64(y[d][k]), iw, iwq, pi.qd), pi.qd);
    }
  }
  for (int t = 0; t < int(L); ++t) {  // the other data primes
    if (t >= lo && t < lo + D) continue;
    const NttPrime pt = f.primes[t];
    const ArF64Lean ar(pt);
    double v[kE];
    if constexpr (D == 1) {
#pragma unroll
      for (int k = 0; k < kE; ++k) v[k] = ArF64::from_u64(reduce_to(y[0][k], kc, t, f.narrow));
    } else {
      cols_target_f64<D>(v, y, kc, lo, t, pt);
    }
    top_fwd<ArF64Lean, true>(v, f.tw_fwd_f + (size_t(t) << kLog), ar);
    store(t, v);
  }
}

// Float-path data primes with an integer-path special prime: a workgroup
// takes the float targets or the special prime of one (ciphertext, digit, 256
// columns); workgroups go to the XCDs round robin, so in every run of 16 the
// first eight take the float targets of eight column groups and the next
// eight the special prime of the same eight, on the same XCDs and dispatched
// together - the special prime's read of the digit's columns finds them in
// that XCD's L2.  Each digit column is read from memory once.
template <int D, class AU>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 1 ? 3 : 2)))
    ks_cols_fwd_pair(KsRows f, unsigned works) {
  const unsigned r = blockIdx.x & 15u, w = (blockIdx.x >> 4) * 8u + (r & 7u);
  if (w >= works) return;
  if (r < 8)
    cols_fwd_float_body<D>(f, w);
  else
    cols_fwd_body<D, AU, 1>(f, unsigned(f.kc->L), 1u, w);
}

// ------------------------------------------------------------------ phase B
// One item = (ciphertext, key prime t, row of 1024 coefficients) on the two
// waves of a workgroup, 8 coefficients per lane (radix-8 register passes, one
// exchange crossing the two waves, the others within a wave): forward stages
// 4-13 of each digit's row, the key products summed over the digits in
// registers, inverse stages 0-9 of both sums.  Eight coefficients per lane
// keep a wave within 168 VGPRs, so a SIMD holds three waves.  The row's
// forward twiddles are staged in LDS once per item (16 KiB beside the 8.5 KiB
// exchange buffer: six items fit a CU's 160 KiB), so the digits' passes issue
// no vector-memory loads, and the next digit's row and this digit's key words
// are in flight while the passes run (vector loads complete in order: a
// twiddle load behind them would wait for them).  E is read with
// nontemporal loads, and so are the keys when every ciphertext has its own:
// each of those words is read once, and streamed through L2 as ordinary
// loads they evict the twiddle tables that every item's copy reads (a key
// shared by a batch is re-read by its other items and stays cached).
constexpr int kRowLE = 3;                           // 8 coefficients per lane
constexpr unsigned kRow2Threads = 1u << (kRowLog - kRowLE);  // 128: the item's two waves

// Twiddles of row pass P (a 1024-coefficient transform's pass map with 2^LE
// coefficients per thread, the row's bits above it): global group index =
// (row << 10 | local) >> (LO + R); t is the thread of the item.
template <bool INV, int P, int LE, class TW>
__device__ __forceinline__ void row_twiddles_e(TW (&w)[(pass_tw_count<kRowLog, INV, P, LE>())], unsigned t,
                                               unsigned row, const TW* __restrict__ tab) {
  using M = PassMap<kRowLog, INV, P, LE>;
  constexpr int LO = M::LO, R = M::R, SUB = (1 << LE) >> R;
  int n = 0;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
    const unsigned hi_lane = ((row << kRowLog) | M::elem(t, b << R)) >> (LO + R);
    const unsigned hi = M::uniform_groups() ? __builtin_amdgcn_readfirstlane(hi_lane) : hi_lane;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!INV) {
        const int s = kLog - LO - R + i;
#pragma unroll
        for (int k = 0; k < (1 << i); ++k) w[n++] = tab[(1u << s) + (hi << i) + k];
      } else {
        const int l = LO + i;
#pragma unroll
        for (int k = 0; k < (1 << (R - 1 - i)); ++k) w[n++] = tab[kN - (kN >> l) + 1 + (hi << (R - 1 - i)) + k];
      }
    }
  }
}

// Passes P .. NP - 1 of a row on 2^LE coefficients per thread, each pass's
// twiddles loaded when it starts; stage numbers are the N = 16384
// transform's.
template <bool INV, int P, class A, int E>
__device__ __forceinline__ void row_passes_e(typename A::T (&v)[E], typename A::T* lds, unsigned t, unsigned row,
                                             const typename A::TW* __restrict__ tab, const A& ar, const NttPrime& pr) {
  constexpr int LE = ilog2(E);
  using S = Passes<kRowLog, LE>;
  constexpr int LO = S::lo(INV, P), R = S::r(INV, P);
  typename A::TW w[pass_tw_count<kRowLog, INV, P, LE>()];
  row_twiddles_e<INV, P, LE>(w, t, row, tab);
  if constexpr (INV)
    inv_pass<kLog, LO, R>(v, w, ar, pr, [] {});
  else
    fwd_pass<kLog, LO, R>(v, w, ar, [] {});
  if constexpr (P + 1 < S::NP) {
    exchange<kRowLog, INV, P>(v, lds, t);
    row_passes_e<INV, P + 1>(v, lds, t, row, tab, ar, pr);
  }
}

// The forward twiddles of one row in LDS: stage s (4 <= s < 14) of the N =
// 16384 transform has 2^(s-4) groups inside a row, the table entries
// (1 << s) + (row << (s - 4)) + k; they sit at [2^(s-4) - 1, 2^(s-3) - 1),
// 1023 entries in all.  An item loads them once, with its 128 threads, and
// every digit's forward passes read them there, so no vector-memory load
// stands between a digit's row and key loads and their use.
constexpr unsigned kRowTw = (1u << kRowLog) - 1;
constexpr int kRowKeyPass = 3;

template <class TW>
__device__ __forceinline__ void row_twiddles_fill(TW* ltw, const TW* __restrict__ tab, unsigned row, unsigned t2) {
#pragma unroll
  for (unsigned i = 0; i < (kRowTw + kRow2Threads - 1) / kRow2Threads; ++i) {
    const unsigned e = t2 + i * kRow2Threads;
    if (e < kRowTw) {
      const unsigned m = e + 1, sl = 31u - unsigned(__builtin_clz(m));  // s - 4
      ltw[e] = tab[(1u << (sl + 4)) + (row << sl) + (m - (1u << sl))];
    }
  }
}

// Twiddles of forward row pass P from the row's LDS copy: the group index
// inside the row is local >> (LO + R).
template <int P, int LE, class TW>
__device__ __forceinline__ void row_twiddles_lds(TW (&w)[(pass_tw_count<kRowLog, false, P, LE>())], unsigned t,
                                                 const TW* ltw) {
  using M = PassMap<kRowLog, false, P, LE>;
  constexpr int LO = M::LO, R = M::R, SUB = (1 << LE) >> R;
  int n = 0;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
    const unsigned hi_lane = M::elem(t, b << R) >> (LO + R);
    const unsigned hi = M::uniform_groups() ? __builtin_amdgcn_readfirstlane(hi_lane) : hi_lane;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int sl = kRowLog - LO - R + i;
#pragma unroll
      for (int k = 0; k < (1 << i); ++k) w[n++] = ltw[(1u << sl) - 1 + (hi << i) + k];
    }
  }
}

// Forward passes P .. NP - 1 of a row, twiddles from LDS; at_kp() runs at
// the start of pass KP (the item issues its key loads there).
template <int P, int KP, class A, int E, class F>
__device__ __forceinline__ void row_passes_fwd_lds(typename A::T (&v)[E], typename A::T* lds, unsigned t,
                                                   const typename A::TW* ltw, const A& ar, F&& at_kp) {
  constexpr int LE = ilog2(E);
  using S = Passes<kRowLog, LE>;
  constexpr int LO = S::lo(false, P), R = S::r(false, P);
  if constexpr (P == KP) at_kp();
  typename A::TW w[pass_tw_count<kRowLog, false, P, LE>()];
  row_twiddles_lds<P, LE>(w, t, ltw);
  fwd_pass<kLog, LO, R>(v, w, ar, [] {});
  if constexpr (P + 1 < S::NP) {
    exchange<kRowLog, false, P>(v, lds, t);
    row_passes_fwd_lds<P + 1, KP>(v, lds, t, ltw, ar, at_kp);
  }
}

// Item (ciphertext bl, prime t, row) on the two waves of the workgroup
// (thread t2 < 128).  Policy A:
//   ArU64L    - every key prime below 2^60: Montgomery key products x k 2^-64
//               of the transformed digit word (x < 12q after stage 13) and
//               the canonical key words (x k < 12 q^2 < q 2^64, each product
//               below 2q), added without reduction from zero and reduced by 8q
//               after every fourth digit, so the sums stay below 16q; the last
//               inverse stage multiplies the factor 2^64 back in
//               (product_prime);
//   ArU64     - Harvey bounds: the transformed digit word meets two key words,
//               so it gets one Shoup quotient and two Shoup products;
//   ArF64Lean - the float data primes (q < 2^50), exact FP64 products.
template <class A>
__device__ __forceinline__ void row_item2(const KsRows& f, const KsConst& kc, unsigned bl, unsigned t,
                                          unsigned row, unsigned t2, typename A::T* lds, typename A::TW* ltw) {
  using T = typename A::T;
  constexpr int E = 1 << kRowLE;
  constexpr bool kF64 = std::is_same<T, double>::value;
  constexpr bool kMont = std::is_same<A, ArU64L>::value;
  const unsigned dnum = unsigned(kc.dnum), K = unsigned(kc.K);
  const unsigned b = f.b0 + bl;
  const NttPrime pr = f.primes[t];
  const A ar(pr);
  const typename A::TW* ti = inv_table<A>(f, int(t));
  const uint64_t* kb = f.key + size_t(b / f.key_group) * f.key_stride + (size_t(t) << kLog);
  const bool own_keys = f.key_group == 1;  // shared keys are re-read by other items: leave them cached
  const uint64_t* e0 = f.e + (size_t(bl) * dnum * K + t) * kN + (row << kRowLog);
  const size_t e_step = size_t(K) * kN;  // digit to digit in E
  // the row's forward twiddles into LDS, then the first digit's row (the
  // twiddle loads are issued first, so their wait before the LDS writes
  // leaves the row's loads in flight)
  row_twiddles_fill(ltw, fwd_table<A>(f, int(t)), row, t2);
  uint64_t en[E];
#pragma unroll
  for (int k = 0; k < E; ++k) en[k] = __builtin_nontemporal_load(&e0[fwd_in_index<kRowLog, kRowLE>(t2, k)]);
  __syncthreads();
  T a0[E], a1[E];
  if constexpr (kMont || kF64) {
#pragma unroll
    for (int k = 0; k < E; ++k) a0[k] = a1[k] = 0;
  }
  for (unsigned j = 0; j < dnum; ++j) {
    T v[E];
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = load_form<A>(en[k]);
    if (j + 1 < dnum) {  // the next digit's row, in flight during this digit's passes
      const uint64_t* src = e0 + (j + 1) * e_step;
#pragma unroll
      for (int k = 0; k < E; ++k) en[k] = __builtin_nontemporal_load(&src[fwd_in_index<kRowLog, kRowLE>(t2, k)]);
    }
    // the digit's key words, issued at the start of forward pass kRowKeyPass:
    // registers r, r + 1 hold adjacent coefficients after the last forward
    // pass, so one 16-byte load per key limb and pair
    const uint64_t* k0 = kb + ((size_t(j) * 2 * K) << kLog);
    const uint64_t* k1 = k0 + (size_t(K) << kLog);
    ulonglong2 kav[E / 2], kkv[E / 2];
    row_passes_fwd_lds<0, kRowKeyPass>(v, lds, t2, ltw, ar, [&] {
#pragma unroll
      for (int r = 0; r < E; r += 2) {
        const unsigned pos = (row << kRowLog) | fwd_out_index<kRowLog, kRowLE>(t2, r);
        if (own_keys) {
          const u64x2 a = __builtin_nontemporal_load(reinterpret_cast<const u64x2*>(k0 + pos));
          const u64x2 c = __builtin_nontemporal_load(reinterpret_cast<const u64x2*>(k1 + pos));
          kav[r / 2] = make_ulonglong2(a.x, a.y);
          kkv[r / 2] = make_ulonglong2(c.x, c.y);
        } else {
          kav[r / 2] = *reinterpret_cast<const ulonglong2*>(k0 + pos);
          kkv[r / 2] = *reinterpret_cast<const ulonglong2*>(k1 + pos);
        }
      }
    });
#pragma unroll
    for (int r = 0; r < E; r += 2) {
      const ulonglong2 ka = kav[r / 2], kk = kkv[r / 2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int rr = r + h;
        const uint64_t w0 = h ? ka.y : ka.x, w1 = h ? kk.y : kk.x;
        if constexpr (kF64) {
          // |v| <= 3.44 q after the last forward stage: products |p| <= 1.8 q,
          // added from zero without re-centring; the sums are re-centred
          // after every fourth digit and after the last, so they stay within
          // q/2 + 1 + 4 (1.8 q) < 8 q < 2^53
          a0[rr] += ar.mul(v[rr], ArF64::from_u64(w0));
          a1[rr] += ar.mul(v[rr], ArF64::from_u64(w1));
        } else if constexpr (kMont) {
          // x < 12q after stage 13, canonical key words: each product < 2q
          a0[rr] += mul_mont(v[rr], w0, ar.q, kc.neg_qinv[t]);
          a1[rr] += mul_mont(v[rr], w1, ar.q, kc.neg_qinv[t]);
        } else {
          const uint64_t x = ar.to_u64_fwd(v[rr]);
          const uint64_t xq = shoup_quotient(x, kc.bar[t]);
          const uint64_t p0 = mul_shoup(w0, x, xq, ar.q), p1 = mul_shoup(w1, x, xq, ar.q);
          a0[rr] = j ? add_mod(a0[rr], p0, ar.q) : p0;
          a1[rr] = j ? add_mod(a1[rr], p1, ar.q) : p1;
        }
      }
    }
    if constexpr (kMont) {
      if ((j & 3) == 3) {  // sums below 16q: reduced by 8q every fourth digit
#pragma unroll
        for (int k = 0; k < E; ++k) {
          a0[k] = a0[k] >= ar.q8 ? a0[k] - ar.q8 : a0[k];
          a1[k] = a1[k] >= ar.q8 ? a1[k] - ar.q8 : a1[k];
        }
      }
    } else if constexpr (kF64) {
      if ((j & 3) == 3) {
#pragma unroll
        for (int k = 0; k < E; ++k) {
          a0[k] = reduce_f64(a0[k], ar.q, ar.qinv);
          a1[k] = reduce_f64(a1[k], ar.q, ar.qinv);
        }
      }
    }
    // the next digit's first exchange writes the LDS this digit's last one
    // read, and crosses the waves: it starts with a workgroup barrier
  }
  if constexpr (kF64) {  // re-centred, |x| <= q/2 + 1: the inverse passes' input bound
#pragma unroll
    for (int k = 0; k < E; ++k) {
      a0[k] = reduce_f64(a0[k], ar.q, ar.qinv);
      a1[k] = reduce_f64(a1[k], ar.q, ar.qinv);
    }
  }
  if constexpr (kMont) {  // below 16q -> below 4q, the lazy inverse's input bound
#pragma unroll
    for (int k = 0; k < E; ++k) {
      a0[k] = a0[k] >= ar.q8 ? a0[k] - ar.q8 : a0[k];
      a0[k] = a0[k] >= ar.q4 ? a0[k] - ar.q4 : a0[k];
      a1[k] = a1[k] >= ar.q8 ? a1[k] - ar.q8 : a1[k];
      a1[k] = a1[k] >= ar.q4 ? a1[k] - ar.q4 : a1[k];
    }
  }
  uint64_t* pb = f.prod + ((size_t(b) * 2 * K + t) << kLog) + (row << kRowLog);
  // the integer paths' inverse passes with the compiler's Shoup product
  // (ArU64LC, ArU64C)
  using AI = std::conditional_t<kMont, ArU64LC, std::conditional_t<std::is_same<A, ArU64>::value, ArU64C, A>>;
  const AI ari(pr);
  row_passes_e<true, 0>(a0, lds, t2, row, ti, ari, pr);
#pragma unroll
  for (int k = 0; k < E; ++k) pb[inv_out_index<kRowLog, kRowLE>(t2, k)] = store_form<A>(a0[k]);
  __syncthreads();  // the second transform's first exchange reuses the LDS
  row_passes_e<true, 0>(a1, lds, t2, row, ti, ari, pr);
  uint64_t* pc = pb + (size_t(K) << kLog);
#pragma unroll
  for (int k = 0; k < E; ++k) pc[inv_out_index<kRowLog, kRowLE>(t2, k)] = store_form<A>(a1[k]);
}

// One workgroup (two waves) per item; items [0, u64_items) are the
// integer-path primes t_u64 .. K - 1 (policy AU), the rest the float-path data
// primes 0 .. t_u64 - 1.
template <class AU>
__global__ void __launch_bounds__(kRow2Threads) __attribute__((amdgpu_waves_per_eu(3)))
    ks_rows2_kernel(KsRows f, unsigned t_u64) {
  __shared__ __attribute__((aligned(16))) uint64_t lds[kRowLds];
  __shared__ ulonglong2 ltw[kRowTw];  // the row's forward twiddles (doubles on the float path)
  const KsConst& kc = *f.kc;
  const unsigned K = unsigned(kc.K);
  const unsigned item = blockIdx.x, t2 = threadIdx.x;
  constexpr unsigned rows = kN >> kRowLog;
  const unsigned n_u64 = K - t_u64, u64_items = f.cts * n_u64 * rows;
  if (item >= f.cts * K * rows) return;
  if (item < u64_items) {
    const unsigned row = item % rows, t = t_u64 + (item / rows) % n_u64, bl = item / (rows * n_u64);
    row_item2<AU>(f, kc, bl, t, row, t2, lds, ltw);
  } else {
    const unsigned x = item - u64_items;
    const unsigned row = x % rows, t = (x / rows) % t_u64, bl = x / (rows * t_u64);
    row_item2<ArF64Lean>(f, kc, bl, t, row, t2, reinterpret_cast<double*>(lds), reinterpret_cast<double*>(ltw));
  }
}

// ------------------------------------------------------------------ phase C
template <class A>
__device__ __forceinline__ void top_inv(typename A::T (&v)[kE], const typename A::TW* __restrict__ tab, const A& ar,
                                        const NttPrime& pr) {
  // inverse stages 10-13: stage l uses inv[N - (N >> l) + 1 + k], k < 2^(13-l);
  // stage 13 (one group) takes N^-1 and its twiddle from the prime constants
  typename A::TW w[pass_twiddles<kLogE>()];
  int n = 0;
#pragma unroll
  for (int i = 0; i < kLogE; ++i) {
    const int l = kLog - kLogE + i;
#pragma unroll
    for (int k = 0; k < (1 << (kLogE - 1 - i)); ++k) {
      if (l != kLog - 1) w[n] = to_sgpr(tab[kN - (kN >> l) + 1 + k]);
      ++n;
    }
  }
  inv_pass<kLog, kLog - kLogE, kLogE>(v, w, ar, pr, [] {});
}

// Constants of key prime t for the last inverse stage of a product formed
// by Montgomery key products (the lazy integer path): N^-1 and w_last N^-1
// carry the factor 2^64 that the products lack.
template <class A>
__device__ __forceinline__ NttPrime product_prime(const KsRows& f, const KsConst& kc, int t) {
  NttPrime r = f.primes[t];
  if constexpr (std::is_same<A, ArU64L>::value) {
    r.ninv = kc.ninv_r[t].w;
    r.ninv_q = kc.ninv_r[t].wq;
    r.last = kc.last_r[t].w;
    r.last_q = kc.last_r[t].wq;
  }
  return r;
}

// Canonical coefficient-form residues of one product limb at column c (a
// limb each thread reads once: nontemporal loads, as for the ModDown's own
// limb and its output below, so that these streams leave L2 to the special
// prime's rounding term that every data prime of a column reads).
template <class A>
__device__ __forceinline__ void column_residues(uint64_t (&x)[kE], const uint64_t* __restrict__ src,
                                                const typename A::TW* __restrict__ tab, const NttPrime& pr) {
  const A ar(pr);
  typename A::T v[kE];
#pragma unroll
  for (int k = 0; k < kE; ++k) v[k] = load_form<A>(__builtin_nontemporal_load(&src[unsigned(k) << kRowLog]));
  top_inv<A>(v, tab, ar, pr);
#pragma unroll
  for (int k = 0; k < kE; ++k) x[k] = ar.to_u64_inv(v[k]);
}

// Special-prime limbs first: one thread per (ciphertext, component,
// column) finishes the inverse transform and leaves [P_p + floor(p/2)]_p in
// place of the limb, the rounding term every data prime's ModDown reads.
template <class AU>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) ks_cols_special_kernel(KsRows f) {
  const KsConst& kc = *f.kc;
  const unsigned K = unsigned(kc.K), L = unsigned(kc.L);
  const unsigned gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= f.cts * 2 * kCols) return;
  const unsigned c = gid & (kCols - 1), w = __builtin_amdgcn_readfirstlane(gid >> kRowLog);
  const unsigned comp = w & 1u, b = f.b0 + (w >> 1);
  uint64_t* pl = f.prod + ((size_t(b) * 2 + comp) * K + L) * kN + c;
  const uint64_t p = kc.q[L], half = p >> 1;
  uint64_t last[kE];
  column_residues<AU>(last, pl, f.tw_inv_u + (size_t(L) << kLog), product_prime<AU>(f, kc, int(L)));
#pragma unroll
  for (int k = 0; k < kE; ++k) {
    const uint64_t x = last[k] + half;
    pl[unsigned(k) << kRowLog] = x >= p ? x - p : x;
  }
}

// Then one thread per (ciphertext, component, data prime, column) finishes
// that prime's inverse transform (policy A) and applies ModDown (+ c0).
template <class A>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(std::is_same<typename A::T, double>::value ? 3 : 4)))
    ks_cols_inv_kernel(KsRows f) {
  const KsConst& kc = *f.kc;
  const unsigned K = unsigned(kc.K), L = unsigned(kc.L);
  const unsigned gid = blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= f.cts * 2 * L * kCols) return;
  const unsigned c = gid & (kCols - 1), w = __builtin_amdgcn_readfirstlane(gid >> kRowLog);
  const unsigned i = w % L, comp = (w / L) & 1u, b = f.b0 + w / (2 * L);
  const uint64_t* pc = f.prod + ((size_t(b) * 2 + comp) * K << kLog) + c;
  const uint64_t qi = kc.q[i];
  const uint64_t* c0 = f.in + ((size_t(b) * 2 * L + i) << kLog);
  uint64_t* o = f.out + (((size_t(b) * 2 + comp) * L + i) << kLog) + c;
  if constexpr (std::is_same<typename A::T, double>::value) {
    if (f.moddown_f64) {
      // exact FP64 ModDown for 2^32 < q_i < 2^50: last = hi 2^32 + lo gives
      // [last]_{q_i} = hi 2^32 + lo (mod q_i) with one product, then
      // (x - [last]_{q_i} + floor(p/2)) p^-1, all centred, canonical at the end
      const NttPrime pi = f.primes[i];
      const ArF64 ar(pi);
      // every operand is loaded before the inverse stages, so the loads of
      // the rounding term and c0 overlap the arithmetic
      double v[kE];
      uint64_t lastv[kE], c0v[kE];
#pragma unroll
      for (int k = 0; k < kE; ++k) v[k] = double_of(__builtin_nontemporal_load(&pc[(size_t(i) << kLog) + (unsigned(k) << kRowLog)]));
#pragma unroll
      for (int k = 0; k < kE; ++k) lastv[k] = pc[(size_t(L) << kLog) + (unsigned(k) << kRowLog)];
      if (comp == 0) {
        gather_column(c0v, c0, c, f.ginv, qi);
      } else {
#pragma unroll
        for (int k = 0; k < kE; ++k) c0v[k] = 0;
      }
      top_inv<ArF64>(v, f.tw_inv_f + (size_t(i) << kLog), ar, pi);
      const double c32 = 4294967296.0, c32q = c32 * pi.qinv;
      const double ip = double(kc.invp[i].w), ipq = ip * pi.qinv, half = double(kc.half_mod[i]);
#pragma unroll
      for (int k = 0; k < kE; ++k) {
        const uint64_t last = lastv[k];
        // |red| < 1.9 q, |x| <= q/2 + 1: the factor below stays under 3.4 q
        const double red = mul_f64(double(last >> 32), c32, c32q, pi.qd) + double(last & 0xffffffffull);
        double r = mul_f64(reduce_f64(v[k], pi.qd, pi.qinv) - red + half, ip, ipq, pi.qd);  // |r| < 1.8 q
        r += ArF64::from_u64(c0v[k]);
        __builtin_nontemporal_store(ar.to_u64(r), &o[unsigned(k) << kRowLog]);
      }
      return;
    }
  }
  uint64_t x[kE], c0v[kE];
  column_residues<A>(x, pc + (size_t(i) << kLog), inv_table<A>(f, int(i)), product_prime<A>(f, kc, int(i)));
  if (comp == 0) gather_column(c0v, c0, c, f.ginv, qi);
#pragma unroll
  for (int k = 0; k < kE; ++k) {
    const uint64_t last = pc[(size_t(L) << kLog) + (unsigned(k) << kRowLog)];
    const uint64_t reduced = reduce_to(last, kc, int(i), f.narrow);  // last mod q_i
    const uint64_t corr = sub_mod(reduced, kc.half_mod[i], qi);
    uint64_t val = mul_shoup(sub_mod(x[k], corr, qi), kc.invp[i].w, kc.invp[i].wq, qi);
    if (comp == 0) val = add_mod(val, c0v[k], qi);
    __builtin_nontemporal_store(val, &o[unsigned(k) << kRowLog]);
  }
}

}  // namespace

// Digit size when every digit has the same number of primes (0 otherwise).
static int uniform_digit(const KsConst& kc) {
  const int d = kc.dig_lo[1] - kc.dig_lo[0];
  for (int j = 1; j < kc.dnum; ++j)
    if (kc.dig_lo[j + 1] - kc.dig_lo[j] != d) return 0;
  return d;
}

template <int D, class AU>
static void launch_cols_fwd(const KsRows& f, unsigned dnum, unsigned t_u64, unsigned K, hipStream_t s) {
  const auto grid = [&](unsigned t_n, unsigned g) { return dim3((f.cts * dnum * ((t_n + g - 1) / g) * kCols + 255) / 256); };
  constexpr unsigned GU = kColTargets<ArU64, D>();
  if (!t_u64) {  // every prime on the integer path
    hipLaunchKernelGGL((ks_cols_fwd_kernel<D, AU, GU>), grid(K, GU), dim3(256), 0, s, f, 0u, K);
    return;
  }
  // float data primes, integer special prime (t_u64 = L, K = L + 1)
  const unsigned works = f.cts * dnum * kCols / 256;
  hipLaunchKernelGGL((ks_cols_fwd_pair<D, AU>), dim3((works + 7) / 8 * 16), dim3(256), 0, s, f, works);
}

// One chunk of ciphertexts through the four launches, the integer-path
// primes on policy AU.
template <class AU>
static void launch_chunk(const KsRows& f, const KsConst& kc, int dig, hipStream_t s, hipEvent_t* ev) {
  const auto mark = [&](int i) {
    if (ev) (void)hipEventRecord(ev[i], s);
  };
  const unsigned K = unsigned(kc.K), L = unsigned(kc.L), dnum = unsigned(kc.dnum), rows = kN >> kRowLog;
  // the integer-path primes t_u64 .. K - 1 (the special prime, or every
  // prime when a data prime has 50 bits or more), the float-path data
  // primes below t_u64
  const unsigned t_u64 = f.data_f64 ? L : 0;
  switch (dig) {
    case 1: launch_cols_fwd<1, AU>(f, dnum, t_u64, K, s); break;
    case 2: launch_cols_fwd<2, AU>(f, dnum, t_u64, K, s); break;
    default: launch_cols_fwd<3, AU>(f, dnum, t_u64, K, s); break;
  }
  mark(0);
  const unsigned items = f.cts * K * rows;
  hipLaunchKernelGGL(ks_rows2_kernel<AU>, dim3(items), dim3(kRow2Threads), 0, s, f, t_u64);
  mark(1);
  hipLaunchKernelGGL(ks_cols_special_kernel<AU>, dim3((f.cts * 2 * kCols + 255) / 256), dim3(256), 0, s, f);
  mark(2);
  const dim3 c_grid((f.cts * 2 * L * kCols + 255) / 256);
  if (f.data_f64)
    hipLaunchKernelGGL(ks_cols_inv_kernel<ArF64>, c_grid, dim3(256), 0, s, f);
  else
    hipLaunchKernelGGL(ks_cols_inv_kernel<AU>, c_grid, dim3(256), 0, s, f);
  mark(3);
}

bool keyswitch_rows_supported(const KsConst& kc) {
  const int d = uniform_digit(kc);
  return kc.log_n == kLog && d >= 1 && d <= 3;
}

hipError_t launch_keyswitch_rows(const KsArgs& a, const KsConst* kc_dev, const KsConst& kc, const NttDevice& d,
                                 hipStream_t s) {
  const int dig = uniform_digit(kc);
  if (kc.log_n != kLog || dig < 1 || dig > 3 || !a.inter || a.inter_cts == 0) return hipErrorNotSupported;
  KsRows f;
  f.in = a.in;
  f.out = a.out;
  f.key = a.key;
  f.key_stride = a.key_stride;
  f.key_group = unsigned(a.key_group ? a.key_group : 1);
  f.e = a.inter;
  f.prod = a.prod;
  f.kc = kc_dev;
  f.primes = d.primes;
  f.tw_fwd_u = d.tw_fwd_u;
  f.tw_inv_u = d.tw_inv_u;
  f.tw_fwd_f = d.tw_fwd_f;
  f.tw_inv_f = d.tw_inv_f;
  f.ginv = a.galois_inv;
  f.data_f64 = 1;
  f.moddown_f64 = 1;
  for (int i = 0; i < kc.L; ++i) {
    f.data_f64 &= kc.q[i] < (1ull << 50) ? 1 : 0;
    f.moddown_f64 &= (kc.q[i] < (1ull << 50) && kc.q[i] > (1ull << 32)) ? 1 : 0;
  }
  uint64_t q_max = 0, q_min = ~0ull;
  for (int t = 0; t < kc.K; ++t) {
    q_max = std::max(q_max, kc.q[t]);
    q_min = std::min(q_min, kc.q[t]);
  }
  f.narrow = q_max / 2 < q_min ? 1 : 0;  // q_max < 2 q_min
  for (size_t b0 = 0; b0 < a.batch; b0 += a.inter_cts) {
    f.b0 = unsigned(b0);
    f.cts = unsigned(std::min<size_t>(a.inter_cts, a.batch - b0));
    // every key prime below 2^60: the lazy integer path with Montgomery key
    // products (KsConst::lazy); else Harvey's bounds and Shoup key products
    // phase events only when the whole batch is one chunk
    hipEvent_t* ev = a.batch <= a.inter_cts ? a.phase_events : nullptr;
    if (kc.lazy)
      launch_chunk<ArU64L>(f, kc, dig, s, ev);
    else
      launch_chunk<ArU64>(f, kc, dig, s, ev);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace praghip
