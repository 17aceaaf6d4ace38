// Modular arithmetic shared by the gfx950 kernels (device) and the plan
// builders (host).  All moduli are odd primes q < 2^62.
//
// Integer path: Shoup multiplication by a precomputed constant (the operand /
// quotient pairs of SEAL's MultiplyUIntModOperand, used by the reference at
// switch.cu:13-16), in Harvey's lazy form: for any a < 2^64 and w < q,
//   a*w - mulhi(a, floor(w*2^64/q))*q  lies in [0, 2q).
// Barrett-128 for products of two runtime residues (switch.cu:30-45).
//
// Float path (q < 2^50): residues held as exact integers in IEEE doubles.  The
// product a*w is split error-free into hi + lo with one FMA, the quotient
// c = rint(a * fl(w * fl(1/q))) is within 1/2 + 3|a|/8q of a*w/q (three
// roundings of relative size 2^-53, |a*w/q| < |a| < |a|/q * 2^50), and the
// remainder hi - c*q is exact because it is an integer below 2^53.  Results
// are centred: |r| <= (1/2 + 3A/8) q for |a| <= A q, w < q; any A <= 4 keeps
// every intermediate below 2^53.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define PH_HD __host__ __device__ __forceinline__

namespace praghip {

PH_HD uint64_t mulhi64(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(a, b);
#else
  return (uint64_t)(((unsigned __int128)a * b) >> 64);
#endif
}

// ------------------------------------------------------------------ integer
struct Shoup {
  uint64_t w, wq;  // operand, floor(operand * 2^64 / q)
};

// a*w mod q in [0, 2q) for any a < 2^64.
PH_HD uint64_t mul_shoup_lazy(uint64_t a, uint64_t w, uint64_t wq, uint64_t q) {
  return a * w - mulhi64(a, wq) * q;
}

// The same products with fewer VALU instructions on gfx950, for the
// transforms' butterflies and the Montgomery key products.  The compiler's expansion of
// a 64-bit high word spends four of its nine instructions on moves that build
// zero-extended register pairs.  Here, from 32-bit halves:
//   m1 = a1 b0 + hi(a0 b0) < 2^64,
//   a0 b1 + m1 = c 2^64 + m2      (v_mad_u64_u32 reports the carry c in an
//                                  SGPR pair),
//   hi(a b) = a1 b1 + (m2 >> 32) + c 2^32,
// where a1 b1 + (m2 >> 32) < 2^64 and adding the carry to the high half cannot
// overflow: six instructions.  UNI: b is the same in every lane of the wave
// and was loaded into scalar registers by a scalar memory load (the carry
// product reads its high half from an SGPR); otherwise it is read from VGPRs,
// which is correct for any b.  The empty asm statements keep an assembled
// 64-bit result as one register pair, so that later additions do not split it
// into zero-extended halves again.
//
// gfx950 needs two wait states between a VALU write of an SGPR lane mask (the
// carry) and a VALU read of it as a carry-in.  The compiler inserts them for
// its own instructions but cannot see this dependency between two asm
// statements: the high-word product that must come between them is one, the
// s_nop 0 before the v_addc the other.  A UNI operand must not come from a
// VALU write (v_readfirstlane), whose hazard the compiler would not cover
// either.
#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ uint64_t pin_pair(uint64_t x) {
  asm("" : "+v"(x));
  return x;
}
template <bool UNI>
__device__ __forceinline__ uint64_t mad_carry(uint32_t a0, uint32_t b1, uint64_t m1, uint64_t& c) {
  uint64_t m2;
  if constexpr (UNI)
    asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(m2), "=s"(c) : "v"(a0), "s"(b1), "v"(m1));
  else
    asm("v_mad_u64_u32 %0, %1, %2, %3, %4" : "=v"(m2), "=s"(c) : "v"(a0), "v"(b1), "v"(m1));
  return m2;
}
// a1 b1 + (m2 >> 32) + c 2^32
__device__ __forceinline__ uint64_t mulhi_top(uint32_t a1, uint32_t b1, uint64_t m2, uint64_t c) {
  const uint64_t r = uint64_t(a1) * b1 + uint32_t(m2 >> 32);
  uint32_t rh;
  uint64_t c_out;
  asm("s_nop 0\n\tv_addc_co_u32_e64 %0, %1, %2, 0, %3" : "=v"(rh), "=s"(c_out) : "v"(uint32_t(r >> 32)), "s"(c));
  return pin_pair((uint64_t(rh) << 32) | uint32_t(r));
}
#endif
template <bool UNI>
PH_HD uint64_t mulhi64_t(uint64_t a, uint64_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t a0 = uint32_t(a), a1 = uint32_t(a >> 32), b0 = uint32_t(b), b1 = uint32_t(b >> 32);
  uint64_t c;
  const uint64_t m2 = mad_carry<UNI>(a0, b1, uint64_t(a1) * b0 + __umulhi(a0, b0), c);
  return mulhi_top(a1, b1, m2, c);
#else
  return mulhi64(a, b);
#endif
}

// Both words of a*b (lo returned, hi in `hi`); on the device the low word
// shares the partial products of the high one: lo = a0 b0 + (m2 mod 2^32) 2^32.
PH_HD uint64_t mul_wide(uint64_t a, uint64_t b, uint64_t& hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t a0 = uint32_t(a), a1 = uint32_t(a >> 32), b0 = uint32_t(b), b1 = uint32_t(b >> 32);
  const uint64_t p = uint64_t(a0) * b0;
  uint64_t c;
  const uint64_t m2 = mad_carry<false>(a0, b1, uint64_t(a1) * b0 + uint32_t(p >> 32), c);
  hi = mulhi_top(a1, b1, m2, c);
  return pin_pair((m2 << 32) | uint32_t(p));
#else
  const unsigned __int128 x = (unsigned __int128)a * b;
  hi = (uint64_t)(x >> 64);
  return (uint64_t)x;
#endif
}

// mul_shoup_lazy with the quotient from mulhi64_t<UNI> (UNI: w and wq are the
// same in every lane).  The low word a w - Q q = a w + Q (2^64 - q) mod 2^64
// is one sum: the two low 32x32 products in a 64-bit accumulator, the four
// cross products added to its high half.
template <bool UNI>
PH_HD uint64_t mul_shoup_lazy_t(uint64_t a, uint64_t w, uint64_t wq, uint64_t q) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint64_t Q = mulhi64_t<UNI>(a, wq), nq = 0 - q;
  const uint32_t a0 = uint32_t(a), a1 = uint32_t(a >> 32), w0 = uint32_t(w), w1 = uint32_t(w >> 32);
  const uint32_t Q0 = uint32_t(Q), Q1 = uint32_t(Q >> 32), n0 = uint32_t(nq), n1 = uint32_t(nq >> 32);
  const uint64_t x = uint64_t(Q0) * n0 + uint64_t(a0) * w0;
  const uint32_t h = uint32_t(x >> 32) + a0 * w1 + a1 * w0 + Q0 * n1 + Q1 * n0;
  return pin_pair((uint64_t(h) << 32) | uint32_t(x));
#else
  return mul_shoup_lazy(a, w, wq, q);
#endif
}
PH_HD uint64_t mul_shoup(uint64_t a, uint64_t w, uint64_t wq, uint64_t q) {
  uint64_t r = mul_shoup_lazy(a, w, wq, q);
  return r >= q ? r - q : r;
}
PH_HD uint64_t add_mod(uint64_t a, uint64_t b, uint64_t q) {
  uint64_t x = a + b;
  return x >= q ? x - q : x;
}
PH_HD uint64_t sub_mod(uint64_t a, uint64_t b, uint64_t q) {
  uint64_t x = a + q - b;
  return x >= q ? x - q : x;
}

// a*b mod q by Barrett reduction of the 128-bit product x = xh 2^64 + xl with
// the ratio R = floor((2^128-1)/q) = r1 2^64 + r0 (the reduction SEAL uses,
// which the reference's kernels call at switch.cu:30-45).  The quotient
// estimate is floor(x R / 2^128): the high word of x R's middle column
// (xl r1 + xh r0 + hi(xl r0)) carries into its top word
// (xh r1 + hi(xl r1) + hi(xh r0)); the estimate is at most one below
// floor(x / q), so x - est q lies in [0, 2q) and is exact in the low word.
struct Barrett {
  uint64_t q, r0, r1;
};
PH_HD uint64_t mul_barrett(uint64_t a, uint64_t b, const Barrett m) {
  const uint64_t xl = a * b, xh = mulhi64(a, b);
  const uint64_t t0 = xl * m.r1, t1 = xh * m.r0;
  const uint64_t mid0 = t0 + mulhi64(xl, m.r0);
  const uint64_t mid1 = mid0 + t1;
  const uint64_t carries = uint64_t(mid0 < t0) + uint64_t(mid1 < t1);
  const uint64_t est = xh * m.r1 + mulhi64(xl, m.r1) + mulhi64(xh, m.r0) + carries;
  const uint64_t r = xl - est * m.q;
  return r >= m.q ? r - m.q : r;
}

// Montgomery product with R = 2^64: x k 2^-64 mod q, in [0, 2q) whenever
// x k < q 2^64 (nq = -q^-1 mod 2^64).  m = (x k mod 2^64) nq makes x k + m q
// a multiple of 2^64; its low word cancels the low word of x k with a carry
// exactly when that low word is non-zero, and (x k + m q) / 2^64 < 2q.
PH_HD uint64_t mul_mont(uint64_t x, uint64_t k, uint64_t q, uint64_t nq) {
  uint64_t hi;
  const uint64_t lo = mul_wide(x, k, hi);
  const uint64_t m = lo * nq;
  return hi + mulhi64_t<false>(m, q) + uint64_t(lo != 0);
}

// floor(w 2^64 / q) for w < q, from the Barrett ratio R = floor((2^128-1)/q):
// t = w r1 + floor(w r0 / 2^64) = floor(w R / 2^64) fits 64 bits (w r1 < 2^64)
// and is the quotient or one less, since R > 2^128/q - 1 and w < 2^64; the
// remainder w 2^64 - t q lies in [0, 2q) and is exact mod 2^64.
PH_HD uint64_t shoup_quotient(uint64_t w, const Barrett m) {
  const uint64_t t = w * m.r1 + mulhi64(w, m.r0);
  const uint64_t rem = 0 - t * m.q;
  return rem >= m.q ? t + 1 : t;
}

// The signed value of a ring-2^59 word v (bit 58 the sign) as a canonical
// residue mod q (resident.cu:23-30, matrix.cu:23-26): v + ((q - 2^59) &
// -(v >> 58)) for the reference's primes (q > 2^59); the remainder for smaller
// primes.
PH_HD uint64_t lift59_residue(uint64_t v, uint64_t q) {
  if (q > (1ull << 59)) return v + ((q - (1ull << 59)) & (0ull - (v >> 58)));
  if (!(v >> 58)) return v % q;
  const uint64_t d = ((1ull << 59) - v) % q;
  return d ? q - d : 0;
}

// -------------------------------------------------------------------- float
struct ShoupF {
  double w, wq;  // operand (exact integer), operand / q
};

// a*w mod q, centred: |r| <= (1/2 + 3A/8) q for |a| <= A q, A <= 4 (q < 2^50,
// w < q, wq = w * (1/q)).
PH_HD double mul_f64(double a, double w, double wq, double q) {
  const double hi = a * w;
  const double lo = __builtin_fma(a, w, -hi);
  const double c = __builtin_rint(a * wq);
  return __builtin_fma(-c, q, hi) + lo;
}
// The same product with the quotient estimated from the rounded product,
// c = rint(fl(a w) fl(1/q)): fl(a w) fl(1/q) carries three roundings, as
// fl(a fl(w fl(1/q))) does, so the bound above holds unchanged, and no w/q is
// formed (one multiply fewer per twiddle, one register fewer per twiddle).
PH_HD double mul_f64_hq(double a, double w, double q, double qinv) {
  const double hi = a * w;
  const double lo = __builtin_fma(a, w, -hi);
  const double c = __builtin_rint(hi * qinv);
  return __builtin_fma(-c, q, hi) + lo;
}
// x mod q, centred to |r| <= q/2 + 1 for |x| < 2^53 (qinv = 1/q).
PH_HD double reduce_f64(double x, double q, double qinv) {
  const double c = __builtin_rint(x * qinv);
  return __builtin_fma(-c, q, x);
}
// centred residue (|x| < 2q) -> canonical [0, q)
PH_HD double canon_f64(double x, double q) {
  x = x < 0.0 ? x + q : x;
  return x >= q ? x - q : x;
}

}  // namespace praghip
