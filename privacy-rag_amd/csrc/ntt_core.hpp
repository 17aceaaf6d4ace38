// Negacyclic NTT / INTT core for gfx950: one workgroup per limb of N = 2^LOGN
// coefficients, N/16 threads, 16 coefficients per thread held in registers.
//
// The transform is the reference's radix-2 stage sequence (ntt.cu:104-127,
// stage() ntt.cu:42-53): forward stage s has gap N>>(s+1) and twiddle
// fwd[(1<<s) + group]; inverse stage l has gap 1<<l and twiddle
// inv[N-(N>>l)+1+group], and the last inverse stage scales by N^-1.  Those
// stages are grouped four at a time into radix-16 register passes: a pass over
// the gap bits [LO, LO+R) gives each thread the 2^R coefficients that differ
// only in those bits.  Between passes the limb is exchanged through LDS (one
// 8-byte slot per coefficient plus one pad slot per 16, which keeps every
// pass's access pattern free of bank conflicts).
//
// Twiddles: a pass's twiddles are loaded into registers in one batch - for the
// float path halfway through the previous pass, so their L2 latency hides
// behind half a pass of arithmetic; for the integer path (16-byte pairs, too
// many registers to hold two passes) at the start of the pass, one wait per
// pass.
//
// Arithmetic policies:
//   ArU64 - any q < 2^62: Harvey's lazy butterflies (forward values in [0,4q),
//           inverse in [0,2q)) over Shoup twiddle pairs, canonical at the end;
//   ArF64 - q < 2^50: residues as exact integers in doubles, products with an
//           error-free FMA split, values re-centred every fourth forward /
//           third inverse stage.
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
  double ninv_f, last_f;      // N^-1 and w_last * N^-1 as doubles
  uint64_t one_q;             // floor(2^64 / q), the Shoup quotient of 1
  int use_f64;                // q < 2^50: the float path is exact
  int pad;
};

// lift59_residue with the prime's Shoup quotient of 1 instead of a division
// (for q <= 2^59: |v| < 2^58 reduced by one Shoup product by 1).
__host__ __device__ __forceinline__ uint64_t lift59_residue(uint64_t v, const NttPrime& p) {
  if (p.q > (1ull << 59)) return v + ((p.q - (1ull << 59)) & (0ull - (v >> 58)));
  const bool neg = (v >> 58) != 0;
  const uint64_t r = mul_shoup(neg ? (1ull << 59) - v : v, 1, p.one_q, p.q);
  return neg && r ? p.q - r : r;
}

__host__ __device__ __forceinline__ unsigned lds_pos(unsigned x) { return x + (x >> 4); }

// Load of a twiddle (or other table word) that no kernel writes while it runs,
// through the constant address space: when the address is the same for every
// lane of the wave the compiler issues it as a scalar load into SGPRs, whatever
// stores the kernel makes elsewhere.
template <class T>
__device__ __forceinline__ T load_invariant(const T* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return *(const __attribute__((address_space(4))) T*)p;
#else
  return *p;  // host pass: never executed
#endif
}

// A value that is the same in every lane (a twiddle loaded from a wave-uniform
// address), moved into scalar registers so it takes no VGPRs.
__device__ __forceinline__ uint64_t sgpr_u64(uint64_t x) {
  // readfirstlane returns int: zero-extend each half
  const unsigned hi = unsigned(__builtin_amdgcn_readfirstlane(unsigned(x >> 32)));
  const unsigned lo = unsigned(__builtin_amdgcn_readfirstlane(unsigned(x)));
  return (uint64_t(hi) << 32) | lo;
}
__device__ __forceinline__ double to_sgpr(double x) {
  return __longlong_as_double((long long)sgpr_u64((uint64_t)__double_as_longlong(x)));
}
__device__ __forceinline__ ulonglong2 to_sgpr(ulonglong2 x) {
  ulonglong2 r;
  r.x = sgpr_u64(x.x);
  r.y = sgpr_u64(x.y);
  return r;
}

constexpr int kLogE = 4;  // 16 coefficients per thread
constexpr int kE = 1 << kLogE;

// ---------------------------------------------------------------- policies
struct ArU64 {
  using T = uint64_t;
  using TW = ulonglong2;  // (w, floor(w 2^64 / q))
  static constexpr bool kAhead = false;  // 16-byte twiddles: load at the pass start
  uint64_t q, q2;
  __device__ explicit ArU64(const NttPrime& p) : q(p.q), q2(p.q2) {}
  __device__ __forceinline__ T from_u64(uint64_t x) const { return x; }
  __device__ __forceinline__ uint64_t to_u64_fwd(T x) const {  // [0,4q) -> [0,q)
    x = x >= q2 ? x - q2 : x;
    return x >= q ? x - q : x;
  }
  __device__ __forceinline__ uint64_t to_u64_inv(T x) const { return x >= q ? x - q : x; }  // [0,2q)
  // UNI: the twiddle is the same in every lane and held in scalar registers
  template <bool UNI = false>
  __device__ __forceinline__ void fwd(T& x, T& y, TW w) const {  // CT, values in [0,4q)
    T a = x >= q2 ? x - q2 : x;
    const T t = mul_shoup_lazy_t<UNI>(y, w.x, w.y, q);
    x = a + t;
    y = a - t + q2;
  }
  template <bool UNI = false>
  __device__ __forceinline__ void fwd_at(int, T& x, T& y, TW w) const { fwd<UNI>(x, y, w); }
  template <bool UNI = false>
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {  // GS, values in [0,2q)
    T s = x + y;
    s = s >= q2 ? s - q2 : s;
    const T d = x - y + q2;
    x = s;
    y = mul_shoup_lazy_t<UNI>(d, w.x, w.y, q);
  }
  __device__ __forceinline__ void inv_last(T& x, T& y, const NttPrime& p) const {
    const T s = x + y, d = x - y + q2;
    x = mul_shoup_lazy_t<false>(s, p.ninv, p.ninv_q, q);
    y = mul_shoup_lazy_t<false>(d, p.last, p.last_q, q);
  }
  __device__ __forceinline__ void settle(T&) const {}
  // Harvey's bounds hold without re-centring
  static constexpr bool settle_fwd(int) { return false; }
  static constexpr bool settle_inv(int) { return false; }
};

// The integer path for q < 2^60, where 16q < 2^64 leaves room for lazier
// bounds than Harvey's:
//   forward - a butterfly's X input is reduced by 8q (when at or above 8q)
//             only at stages s = 4, 8, 12, ...; every other stage adds at most
//             2q to the bound (X + T and X - T + 2q, Shoup product T < 2q).
//             From inputs below 8q the values after stage s are below
//             8q + 2q (1 + s mod 4) <= 16q (10q, 12q, 14q, 16q, 10q, ...);
//   inverse - values below 4q: the sum reduced by 4q, the difference offset
//             by 4q before its Shoup product; the last stage's products are
//             below 2q.
struct ArU64L : ArU64 {
  uint64_t q4, q8;
  __device__ explicit ArU64L(const NttPrime& p) : ArU64(p), q4(4 * p.q), q8(8 * p.q) {}
  __device__ __forceinline__ uint64_t to_u64_fwd(T x) const {  // [0,16q) -> [0,q)
    x = x >= q8 ? x - q8 : x;
    x = x >= q4 ? x - q4 : x;
    x = x >= q2 ? x - q2 : x;
    return x >= q ? x - q : x;
  }
  template <bool UNI = false>
  __device__ __forceinline__ void fwd_at(int s, T& x, T& y, TW w) const {
    T a = x;
    if (s > 0 && s % 4 == 0) a = a >= q8 ? a - q8 : a;
    const T t = mul_shoup_lazy_t<UNI>(y, w.x, w.y, q);
    x = a + t;
    y = a - t + q2;
  }
  template <bool UNI = false>
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {
    T s = x + y;
    s = s >= q4 ? s - q4 : s;
    const T d = x - y + q4;
    x = s;
    y = mul_shoup_lazy_t<UNI>(d, w.x, w.y, q);
  }
  __device__ __forceinline__ void inv_last(T& x, T& y, const NttPrime& p) const {
    const T s = x + y, d = x - y + q4;
    x = mul_shoup_lazy_t<false>(s, p.ninv, p.ninv_q, q);
    y = mul_shoup_lazy_t<false>(d, p.last, p.last_q, q);
  }
};

// ArU64 and ArU64L whose inverse butterfly takes the compiler's Shoup
// product: the keyswitch rows kernel's inverse passes.  With the carry-out
// product there, every twiddle product of those passes came out wrong on the
// GPU - with the lazy form and Montgomery key products (each of the two alone
// was exact), and with the per-stage form and Shoup key products (a 62-bit
// special prime) - while the same product is exact in the rows' forward
// passes and in every other transform.  The compiled code shows no wait-state
// shortfall, no write of the carry between its producer and its reader and
// no spill; the cause is not known, so these passes keep the compiler's
// product.
struct ArU64C : ArU64 {
  __device__ explicit ArU64C(const NttPrime& p) : ArU64(p) {}
  template <bool = false>
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {
    T s = x + y;
    s = s >= q2 ? s - q2 : s;
    const T d = x - y + q2;
    x = s;
    y = mul_shoup_lazy(d, w.x, w.y, q);
  }
};
struct ArU64LC : ArU64L {
  __device__ explicit ArU64LC(const NttPrime& p) : ArU64L(p) {}
  template <bool = false>
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {
    T s = x + y;
    s = s >= q4 ? s - q4 : s;
    const T d = x - y + q4;
    x = s;
    y = mul_shoup_lazy(d, w.x, w.y, q);
  }
};

// Float path bounds (q < 2^50, |x| <= M q, mul_f64 gives |t| <= (1/2 + 3A/8) q
// for a factor |a| <= A q, A <= 4; sums must stay below 2^53 = 8 * 2^50):
//   forward : inputs |x| <= q; stages 0..2 grow the bound 1 -> 1.88 -> 3.08
//             -> 4.73, every value is re-centred (|x| <= q/2 + 1) after
//             stages s = 2 mod 4, and four stages from there reach 1.19,
//             2.14, 3.44, 5.23 - factors stay below 3.5 q;
//   inverse : the sum side doubles and the difference goes through the
//             product: from |x| <= q, 2 -> 4 after stages 0, 1; re-centred after
//             stages l = 1 mod 3, then 1 -> 2 -> 4 (differences below 4 q);
//             the last stage multiplies both outputs (N^-1 folded).
struct ArF64 {
  using T = double;
  using TW = double;  // w (the quotient is estimated from the rounded product)
  static constexpr bool kAhead = true;  // load the next pass's twiddles one pass early
  double q, qinv;
  __device__ explicit ArF64(const NttPrime& p) : q(p.qd), qinv(p.qinv) {}
  // Exact conversions for integers below 2^52: the bit pattern of 2^52 + x is
  // 0x4330... with x in its 52 mantissa bits.
  __device__ __forceinline__ static T from_u64(uint64_t x) {
    return __longlong_as_double((long long)(x | 0x4330000000000000ull)) - 4503599627370496.0;
  }
  __device__ __forceinline__ uint64_t to_u64(T x) const {
    x = reduce_f64(x, q, qinv);  // |x| <= q/2 + 1
    x += x < 0.0 ? q + 4503599627370496.0 : 4503599627370496.0;
    return (uint64_t)__double_as_longlong(x) & 0x000FFFFFFFFFFFFFull;
  }
  __device__ __forceinline__ uint64_t to_u64_fwd(T x) const { return to_u64(x); }
  __device__ __forceinline__ uint64_t to_u64_inv(T x) const { return to_u64(x); }
  __device__ __forceinline__ T mul(T a, TW w) const { return mul_f64_hq(a, w, q, qinv); }
  template <bool = false>
  __device__ __forceinline__ void fwd(T& x, T& y, TW w) const {
    const T t = mul(y, w);
    const T a = x;
    x = a + t;
    y = a - t;
  }
  template <bool = false>
  __device__ __forceinline__ void fwd_at(int, T& x, T& y, TW w) const { fwd(x, y, w); }
  template <bool = false>
  __device__ __forceinline__ void inv(T& x, T& y, TW w) const {
    const T s = x + y, d = x - y;
    x = s;
    y = mul(d, w);
  }
  __device__ __forceinline__ void inv_last(T& x, T& y, const NttPrime& p) const {
    const T s = x + y, d = x - y;
    x = mul(s, p.ninv_f);
    y = mul(d, p.last_f);
  }
  __device__ __forceinline__ void settle(T& x) const { x = reduce_f64(x, q, qinv); }
  static constexpr bool settle_fwd(int s) { return s % 4 == 2; }
  static constexpr bool settle_inv(int l) { return l % 3 == 1; }
};

// The float path of the standalone transform, whose inputs and outputs are
// canonical: it re-centres only after forward stages s = 3 mod 5 and inverse
// stages l = 2 mod 4 (2 and 3 re-centrings at N = 16384 instead of 3 and 4).
// Bounds (|x| <= M q; a product by a factor |a| <= A q is within
// (1/2 + 3A/8) q for any A, so M -> 1.375 M + 1/2 per forward stage):
//   forward : canonical inputs, stages 0..3 reach 1.88, 3.08, 4.73, 7.01;
//             after a re-centring (q/2 + 1) five stages reach 1.19, 2.13,
//             3.43, 5.22, 7.68 - factors below 5.3 q, values below 7.7 q;
//   inverse : sums double from q (canonical) or q/2 + 1 (re-centred), so the
//             values and the differences that become factors stay within
//             8 q + 16;
// every value and remainder stays below 2^53 because q < 2^50 - 2 (q odd,
// prime).  The keyswitch kernels keep ArF64's schedule, whose bounds their
// phases rely on.
struct ArF64T : ArF64 {
  __device__ explicit ArF64T(const NttPrime& p) : ArF64(p) {}
  static constexpr bool settle_fwd(int s) { return s % 5 == 3; }
  static constexpr bool settle_inv(int l) { return l % 4 == 2; }
};

// The float path with each pass's twiddles loaded when the pass starts (for
// kernels that keep more than the limb in registers).
struct ArF64Lean : ArF64 {
  static constexpr bool kAhead = false;
  __device__ explicit ArF64Lean(const NttPrime& p) : ArF64(p) {}
};

// Pass geometry, for 2^LE coefficients per thread (LE = 4 unless a caller
// asks for fewer).  Forward passes take LE gap bits from the top down, the
// last one the remainder [0, RSHORT); inverse passes start with the remainder
// [0, RSHORT) and continue upwards LE bits at a time.
template <int LOGN, int LE = kLogE>
struct Passes {
  static constexpr int NP = (LOGN + LE - 1) / LE;
  static constexpr int RSHORT = LOGN - LE * (NP - 1);
  static constexpr int fwd_lo(int p) { return p < NP - 1 ? LOGN - LE * (p + 1) : 0; }
  static constexpr int fwd_r(int p) { return p < NP - 1 ? LE : RSHORT; }
  static constexpr int inv_lo(int p) { return p == 0 ? 0 : RSHORT + LE * (p - 1); }
  static constexpr int inv_r(int p) { return p == 0 ? RSHORT : LE; }
  static constexpr int lo(bool inv, int p) { return inv ? inv_lo(p) : fwd_lo(p); }
  static constexpr int r(bool inv, int p) { return inv ? inv_r(p) : fwd_r(p); }
  static constexpr int LANE_BITS = LOGN - LE < 6 ? LOGN - LE : 6;  // thread bits inside a wave
  static constexpr int WAVE_BITS = LOGN - LE - LANE_BITS;          // thread bits naming the wave
};

// Placement of a thread's 2^LE registers in a pass.  The coefficient index is
// assembled from three fields:
//   register bits - the pass's gap bits [LO, LO+R), and when R < LE (LO = 0
//                   then) LE - R bits just below the wave bits for the
//                   independent blocks;
//   wave bits     - the top WAVE_BITS bits, except in the pass whose gap bits
//                   are the top bits, where they sit just below them;
//   lane bits     - every other bit, in increasing order.
// With the wave bits fixed to the top in all but one pass, a wave owns the
// same contiguous 2^(LOGN - WAVE_BITS) coefficients in consecutive passes, so those
// exchanges stay inside the wave (its own LDS region, no workgroup barrier);
// only the exchange into or out of the top pass crosses waves.  The first
// forward pass and the last inverse pass put consecutive lanes on consecutive
// coefficients (coalesced global access); the last forward and first inverse
// pass give each lane runs of 2^R consecutive coefficients, consecutive lanes
// on consecutive runs.
template <int LOGN, bool INV, int P, int LE = kLogE>
struct PassMap {
  using S = Passes<LOGN, LE>;
  static constexpr int LO = S::lo(INV, P), R = S::r(INV, P);
  static constexpr int WAVE_LO = (LO + R == LOGN) ? LO - S::WAVE_BITS : LOGN - S::WAVE_BITS;
  // block bits (R < LE, LO = 0): just below the wave bits
  static constexpr int BLOCK_LO = WAVE_LO - (LE - R);
  static constexpr int reg_bit(int q) { return q < R ? LO + q : BLOCK_LO + (q - R); }
  static constexpr bool is_reg(int e) { return (e >= LO && e < LO + R) || (e >= BLOCK_LO && e < WAVE_LO && R < LE); }
  static constexpr bool is_wave(int e) { return e >= WAVE_LO && e < WAVE_LO + S::WAVE_BITS; }
  static constexpr int lane_bit(int q) {
    int c = 0;
    for (int e = 0; e < LOGN; ++e)
      if (!is_reg(e) && !is_wave(e)) {
        if (c == q) return e;
        ++c;
      }
    return -1;
  }
  // every lane bit lies below the gap bits: the bits above them (the twiddle
  // group) are the same for all lanes of a wave
  static constexpr bool uniform_groups() {
    for (int q = 0; q < S::LANE_BITS; ++q)
      if (lane_bit(q) >= LO + R) return false;
    return true;
  }
  __host__ __device__ static constexpr unsigned reg_field(int j) {
    unsigned x = 0;
    for (int q = 0; q < LE; ++q) x |= unsigned((j >> q) & 1) << reg_bit(q);
    return x;
  }
  __host__ __device__ static unsigned thread_field(unsigned t) {
    unsigned x = 0;
#pragma unroll
    for (int q = 0; q < S::LANE_BITS; ++q) x |= ((t >> q) & 1u) << lane_bit(q);
#pragma unroll
    for (int q = 0; q < S::WAVE_BITS; ++q) x |= ((t >> (6 + q)) & 1u) << (WAVE_LO + q);
    return x;
  }
  __host__ __device__ static unsigned elem(unsigned t, int j) { return thread_field(t) | reg_field(j); }
  // padded LDS slot of register j relative to register 0: the fields are
  // disjoint, so the sum never carries into bit 4 and lds_pos is linear
  __host__ __device__ static constexpr unsigned slot_offset(int j) {
    const unsigned d = reg_field(j);
    return d + (d >> 4);
  }
};

// ------------------------------------------------------------------ passes
// Twiddles of one pass: SUB blocks x (2^R - 1) entries, in the order the pass
// consumes them (block, stage, group).
template <int R, int LE = kLogE>
constexpr int pass_twiddles() { return ((1 << LE) >> R) * ((1 << R) - 1); }

constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

// Twiddles of pass P of a 2^LOGN transform with 2^LE coefficients per thread.
template <int LOGN, bool INV, int P, int LE>
constexpr int pass_tw_count() {
  constexpr int R = Passes<LOGN, LE>::r(INV, P);
  return pass_twiddles<R, LE>();
}

template <int LOGN, bool INV, int P, int LE, class TW>
__device__ __forceinline__ void load_pass_twiddles_e(TW (&w)[(pass_tw_count<LOGN, INV, P, LE>())], unsigned t,
                                                     const TW* __restrict__ tab) {
  using M = PassMap<LOGN, INV, P, LE>;
  constexpr int LO = M::LO, R = M::R, SUB = (1 << LE) >> R;
  constexpr unsigned N = 1u << LOGN;
  int n = 0;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
    // group index of the block: the coefficient bits above the gap bits.
    // When no lane bit lies there, all lanes of a wave share it and the
    // twiddle loads go through the scalar unit into SGPRs.
    const unsigned hi_lane = M::elem(t, b << R) >> (LO + R);
    const unsigned hi = M::uniform_groups() ? __builtin_amdgcn_readfirstlane(hi_lane) : hi_lane;
    const auto ld = [&](unsigned x) { return M::uniform_groups() ? load_invariant(tab + x) : tab[x]; };
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!INV) {
        const int s = LOGN - LO - R + i;
#pragma unroll
        for (int k = 0; k < (1 << i); ++k) w[n++] = ld((1u << s) + (hi << i) + k);
      } else {
        const int l = LO + i;
#pragma unroll
        for (int k = 0; k < (1 << (R - 1 - i)); ++k) {
          if (l != LOGN - 1) w[n] = ld(N - (N >> l) + 1 + (hi << (R - 1 - i)) + k);
          ++n;
        }
      }
    }
  }
}
template <int LOGN, bool INV, int P, class TW>
__device__ __forceinline__ void load_pass_twiddles(TW (&w)[pass_twiddles<Passes<LOGN>::r(INV, P)>()], unsigned t,
                                                   const TW* __restrict__ tab) {
  load_pass_twiddles_e<LOGN, INV, P, kLogE>(w, t, tab);
}

// Forward radix-2^R pass over gap bits [LO, LO+R): global stages
// s = LOGN-LO-R .. LOGN-LO-1.
// A pass calls `mid` once, halfway through its butterflies (after stage R/2-1
// of a single block, or after block SUB/2-1): the twiddles of the early stages
// are dead by then, which is where the next pass's twiddle loads go.
template <int R, int LE = kLogE>
__device__ __forceinline__ constexpr bool is_mid(int b, int i) {
  return ((1 << LE) >> R) == 1 ? (i == R / 2 - 1) : (b == ((1 << LE) >> R) / 2 - 1 && i == R - 1);
}

// UNI: every twiddle of the pass is wave-uniform and in scalar registers.
template <int LOGN, int LO, int R, bool UNI = false, class A, class F, int E>
__device__ __forceinline__ void fwd_pass(typename A::T (&v)[E], const typename A::TW (&w)[pass_twiddles<R, ilog2(E)>()],
                                         const A& ar, F&& mid) {
  constexpr int LE = ilog2(E), SUB = E >> R;
  int n = 0;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int s = LOGN - LO - R + i, g = R - 1 - i;
#pragma unroll
      for (int k = 0; k < (1 << i); ++k, ++n) {
#pragma unroll
        for (int m = 0; m < (1 << g); ++m) {
          const int j0 = (b << R) | (k << (g + 1)) | m, j1 = j0 | (1 << g);
          ar.template fwd_at<UNI>(s, v[j0], v[j1], w[n]);
        }
      }
      if (A::settle_fwd(s) && s != LOGN - 1) {  // the final stage is reduced on output
#pragma unroll
        for (int m = 0; m < (1 << R); ++m) ar.settle(v[(b << R) | m]);
      }
      if (is_mid<R, LE>(b, i)) mid();
    }
  }
}

// Inverse radix-2^R pass over gap bits [LO, LO+R): stages l = LO .. LO+R-1.
template <int LOGN, int LO, int R, bool UNI = false, class A, class F, int E>
__device__ __forceinline__ void inv_pass(typename A::T (&v)[E], const typename A::TW (&w)[pass_twiddles<R, ilog2(E)>()],
                                         const A& ar, const NttPrime& pr, F&& mid) {
  constexpr int LE = ilog2(E), SUB = E >> R;
  int n = 0;
#pragma unroll
  for (int b = 0; b < SUB; ++b) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int l = LO + i;
#pragma unroll
      for (int k = 0; k < (1 << (R - 1 - i)); ++k, ++n) {
#pragma unroll
        for (int m = 0; m < (1 << i); ++m) {
          const int j0 = (b << R) | (k << (i + 1)) | m, j1 = j0 | (1 << i);
          if (l == LOGN - 1)  // last stage: one group, twiddle and N^-1 folded
            ar.inv_last(v[j0], v[j1], pr);
          else
            ar.template inv<UNI>(v[j0], v[j1], w[n]);
        }
      }
      if (A::settle_inv(l) && l != LOGN - 1) {
#pragma unroll
        for (int m = 0; m < (1 << R); ++m) ar.settle(v[(b << R) | m]);
      }
      if (is_mid<R, LE>(b, i)) mid();
    }
  }
}

// Exchange between consecutive passes.  When both passes give the wave the
// same coefficients (same wave bits) the exchange stays in the wave's own LDS
// region: LDS operations of one wave execute in order, so only a compiler
// barrier is needed.  Otherwise the whole workgroup synchronises before (other
// waves may still read their regions), between, and after.
template <int LOGN, bool INV, int P, class T, int E>
__device__ __forceinline__ void exchange(T (&v)[E], T* lds, unsigned t) {
  constexpr int LE = ilog2(E);
  using A = PassMap<LOGN, INV, P, LE>;
  using B = PassMap<LOGN, INV, P + 1, LE>;
  constexpr bool in_wave = A::WAVE_LO == B::WAVE_LO || Passes<LOGN, LE>::WAVE_BITS == 0;
  if constexpr (!in_wave) __syncthreads();
  T* wbase = lds + lds_pos(A::elem(t, 0));
#pragma unroll
  for (int j = 0; j < (1 << LE); ++j) wbase[A::slot_offset(j)] = v[j];
  if constexpr (in_wave)
    __builtin_amdgcn_wave_barrier();
  else
    __syncthreads();
  const T* rbase = lds + lds_pos(B::elem(t, 0));
#pragma unroll
  for (int j = 0; j < (1 << LE); ++j) v[j] = rbase[B::slot_offset(j)];
  if constexpr (in_wave) {
    __builtin_amdgcn_wave_barrier();
  } else {
    __syncthreads();
    // The compiler does not count s_barrier as a memory access when it sinks
    // loads into a successor block: where the values read here are first used
    // after a branch, it moved these LDS reads below the barrier, where a
    // faster wave's next LDS writes can overwrite what they read.  An empty asm
    // with a memory clobber does count, and pins the reads above it.
    asm volatile("" ::: "memory");
  }
}

// Pass P with its twiddles already in registers; loads pass P+1's twiddles
// first, then computes, exchanges and recurses.
// `before_last` runs once the LDS is no longer needed by this limb (after the
// last exchange, or at once for a single-pass transform).
template <int LOGN, bool INV, int P, class A, class F>
__device__ __forceinline__ void run_passes(typename A::T (&v)[kE], typename A::T* lds, unsigned t,
                                           const typename A::TW* __restrict__ tab, const A& ar,
                                           const NttPrime& pr,
                                           const typename A::TW (&w)[pass_twiddles<Passes<LOGN>::r(INV, P)>()],
                                           F&& before_last) {
  using S = Passes<LOGN>;
  constexpr int LO = S::lo(INV, P), R = S::r(INV, P);
  // uniform groups: the pass's twiddles were loaded by scalar memory loads
  // (load_invariant at a wave-uniform index)
  constexpr bool UNI = PassMap<LOGN, INV, P>::uniform_groups();
  if constexpr (P + 1 < S::NP) {
    constexpr int R1 = S::r(INV, P + 1);
    typename A::TW wn[pass_twiddles<R1>()];
    auto prefetch = [&] {
      if constexpr (A::kAhead) load_pass_twiddles<LOGN, INV, P + 1>(wn, t, tab);
    };
    if constexpr (INV)
      inv_pass<LOGN, LO, R, UNI>(v, w, ar, pr, prefetch);
    else
      fwd_pass<LOGN, LO, R, UNI>(v, w, ar, prefetch);
    exchange<LOGN, INV, P>(v, lds, t);
    if constexpr (!A::kAhead) load_pass_twiddles<LOGN, INV, P + 1>(wn, t, tab);
    run_passes<LOGN, INV, P + 1>(v, lds, t, tab, ar, pr, wn, before_last);
  } else {
    before_last();
    if constexpr (INV)
      inv_pass<LOGN, LO, R, UNI>(v, w, ar, pr, [] {});
    else
      fwd_pass<LOGN, LO, R, UNI>(v, w, ar, [] {});
  }
}

// Whole-limb transform on register data (v holds the input layout on entry
// and the output layout on exit; values stay in the policy's lazy form).
template <int LOGN, bool INV, class A, class F>
__device__ __forceinline__ void ntt_regs(typename A::T (&v)[kE], typename A::T* lds, unsigned t,
                                         const typename A::TW* __restrict__ tab, const A& ar, const NttPrime& pr,
                                         F&& before_last) {
  using S = Passes<LOGN>;
  typename A::TW w0[pass_twiddles<S::r(INV, 0)>()];
  load_pass_twiddles<LOGN, INV, 0>(w0, t, tab);
  run_passes<LOGN, INV, 0>(v, lds, t, tab, ar, pr, w0, before_last);
}
template <int LOGN, bool INV, class A>
__device__ __forceinline__ void ntt_regs(typename A::T (&v)[kE], typename A::T* lds, unsigned t,
                                         const typename A::TW* __restrict__ tab, const A& ar, const NttPrime& pr) {
  ntt_regs<LOGN, INV>(v, lds, t, tab, ar, pr, [] {});
}

// Register layouts at the boundaries of a transform.
template <int LOGN, int LE = kLogE>
__device__ __forceinline__ unsigned fwd_in_index(unsigned t, int j) { return PassMap<LOGN, false, 0, LE>::elem(t, j); }
template <int LOGN, int LE = kLogE>
__device__ __forceinline__ unsigned fwd_out_index(unsigned t, int j) {
  return PassMap<LOGN, false, Passes<LOGN, LE>::NP - 1, LE>::elem(t, j);
}
template <int LOGN, int LE = kLogE>
__device__ __forceinline__ unsigned inv_in_index(unsigned t, int j) { return PassMap<LOGN, true, 0, LE>::elem(t, j); }
template <int LOGN, int LE = kLogE>
__device__ __forceinline__ unsigned inv_out_index(unsigned t, int j) {
  return PassMap<LOGN, true, Passes<LOGN, LE>::NP - 1, LE>::elem(t, j);
}

template <int LOGN, int LE = kLogE>
constexpr int ntt_threads() { return (1 << LOGN) >> LE; }

constexpr size_t lds_bytes(int log_n) { return (((size_t)1 << log_n) + ((size_t)1 << log_n) / 16) * 8; }

}  // namespace praghip
