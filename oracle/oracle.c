/*
 * CPU oracle for the BFV polynomial engine and the party-local share GEMM.
 *
 * TEST INFRASTRUCTURE ONLY.  It checks results: it is linked or called
 * only by tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of
 * bench.py.  The product library (privacy-rag_amd/) never calls it and never
 * falls back to it.
 *
 * It restates, in plain C with 128-bit host integers, the arithmetic of the
 * reference's GPU backends and of the SEAL 4.1.2 routines they replace.  Each
 * function cites the reference file:line it follows (paths relative to
 * implementation_v1/).  SEAL itself is not vendored by the reference and is
 * absent here, so the SEAL conventions are restated from its published
 * algorithm (NTTTables, ntt_negacyclic_harvey, barrett_reduce_128,
 * RNSTool::divide_and_round_q_last, GaloisTool::apply_galois) and pinned by
 * closed-form tests (tests/test_oracle.py, tests/golden/closed_form.py).
 *
 * Every residue handed in or out is canonical ([0, q)).  q < 2^62 throughout.
 */
#include <stdint.h>
#include <stddef.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef unsigned __int128 u128;

/* ------------------------------------------------------------------------ */
/* Seeded counter-based generator (splitmix64 finaliser over seed+(i+1)*phi).  */
/* Residues use Lemire's mulhi(z, q); int8 weights mulhi(z,255)-127; shifts    */
/* mulhi(z,8).                                                                  */
/* ------------------------------------------------------------------------ */
uint64_t orc_splitmix64(uint64_t seed, uint64_t index) {
  uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}
static inline uint64_t mulhi64(uint64_t a, uint64_t b) { return (uint64_t)(((u128)a * b) >> 64); }

/* limb l of a [.., P, N] buffer uses prime q[l % P] */
void orc_fill_residues(uint64_t *out, size_t limbs, size_t n, const uint64_t *q, size_t primes,
                       uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (size_t l = 0; l < limbs; ++l) {
    const uint64_t qq = q[l % primes];
    for (size_t k = 0; k < n; ++k) out[l * n + k] = mulhi64(orc_splitmix64(seed, l * n + k), qq);
  }
}
void orc_fill_u64(uint64_t *out, size_t count, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < count; ++i) out[i] = orc_splitmix64(seed, i);
}
void orc_fill_i8(int8_t *out, size_t count, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < count; ++i) out[i] = (int8_t)((int64_t)mulhi64(orc_splitmix64(seed, i), 255) - 127);
}
void orc_fill_shift(int8_t *out, size_t count, uint64_t seed) {
  for (size_t i = 0; i < count; ++i) out[i] = (int8_t)mulhi64(orc_splitmix64(seed, i), 8);
}

/* ------------------------------------------------------------------------ */
/* Number theory (host).                                                     */
/* ------------------------------------------------------------------------ */
uint64_t orc_mulmod(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)(((u128)a * b) % q); }
uint64_t orc_powmod(uint64_t a, uint64_t e, uint64_t q) {
  uint64_t r = 1 % q;
  a %= q;
  while (e) {
    if (e & 1) r = orc_mulmod(r, a, q);
    a = orc_mulmod(a, a, q);
    e >>= 1;
  }
  return r;
}
uint64_t orc_invmod(uint64_t a, uint64_t q) { /* q prime */
  return orc_powmod(a % q, q - 2, q);
}
int orc_is_prime(uint64_t n) {
  static const uint64_t bases[] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
  if (n < 2) return 0;
  for (size_t i = 0; i < 12; ++i) {
    if (n == bases[i]) return 1;
    if (n % bases[i] == 0) return 0;
  }
  uint64_t d = n - 1;
  int s = 0;
  while (!(d & 1)) { d >>= 1; ++s; }
  for (size_t i = 0; i < 12; ++i) {
    uint64_t x = orc_powmod(bases[i], d, n);
    if (x == 1 || x == n - 1) continue;
    int composite = 1;
    for (int r = 1; r < s; ++r) {
      x = orc_mulmod(x, x, n);
      if (x == n - 1) { composite = 0; break; }
    }
    if (composite) return 0;
  }
  return 1;
}
/* SEAL CoeffModulus::Create rule: the largest primes below 2^bits that are
 * congruent to 1 modulo 2N, in descending order (bfv.cpp:94-95 uses it with
 * bits=60 and gets the locked primes in ascending listing order). */
size_t orc_gen_primes(int bits, uint64_t two_n, size_t count, uint64_t *out) {
  uint64_t upper = (bits >= 64) ? ~0ULL : (1ULL << bits);
  uint64_t cand = upper - (upper % two_n) + 1; /* first value == 1 mod 2N at or above upper-2N */
  if (cand >= upper) cand -= two_n;
  size_t found = 0;
  while (found < count && cand > two_n) {
    if (orc_is_prime(cand)) out[found++] = cand;
    cand -= two_n;
  }
  return found;
}
static uint64_t bitrev(uint64_t x, unsigned bits) {
  uint64_t r = 0;
  for (unsigned i = 0; i < bits; ++i) r |= ((x >> i) & 1ULL) << (bits - 1 - i);
  return r;
}
/* SEAL try_minimal_primitive_root(2N, q): any primitive 2N-th root g, then
 * the smallest of g^1, g^3, ..., g^(2N-1).  Returns 0 if q != 1 mod 2N. */
uint64_t orc_minimal_root(uint64_t q, uint64_t two_n) {
  if ((q - 1) % two_n) return 0;
  const uint64_t cofactor = (q - 1) / two_n;
  uint64_t g = 0;
  for (uint64_t x = 2; x < q; ++x) {
    uint64_t c = orc_powmod(x, cofactor, q);
    if (orc_powmod(c, two_n / 2, q) == q - 1) { g = c; break; }
  }
  if (!g) return 0;
  const uint64_t g2 = orc_mulmod(g, g, q);
  uint64_t cur = g, best = g;
  for (uint64_t i = 0; i < two_n; i += 2) {
    if (cur < best) best = cur;
    cur = orc_mulmod(cur, g2, q);
  }
  return best;
}
/* SEAL MultiplyUIntModOperand::set_quotient: floor(w * 2^64 / q). */
uint64_t orc_shoup_quotient(uint64_t w, uint64_t q) { return (uint64_t)(((u128)w << 64) / q); }

/* SEAL NTTTables (4.1.2) as exported by seal_tables.cpp:22-33:
 *   forward[bitrev(i)] = psi^i (i=1..N-1), forward[0] = 1;
 *   inverse[bitrev(i-1)+1] = psi^-i (i=1..N-1), inverse[0] = 1;
 *   invn = N^-1 mod q.
 * Each entry is an (operand, quotient) pair, layout [N][2]. */
int orc_ntt_tables(uint64_t q, unsigned log_n, uint64_t *fwd_pairs, uint64_t *inv_pairs,
                   uint64_t *invn_pair) {
  const uint64_t n = 1ULL << log_n;
  const uint64_t psi = orc_minimal_root(q, 2 * n);
  if (!psi) return -1;
  const uint64_t psi_inv = orc_invmod(psi, q);
  fwd_pairs[0] = 1; fwd_pairs[1] = orc_shoup_quotient(1, q);
  inv_pairs[0] = 1; inv_pairs[1] = orc_shoup_quotient(1, q);
  uint64_t p = psi, pi = psi_inv;
  for (uint64_t i = 1; i < n; ++i) {
    const uint64_t f = bitrev(i, log_n), r = bitrev(i - 1, log_n) + 1;
    fwd_pairs[2 * f] = p; fwd_pairs[2 * f + 1] = orc_shoup_quotient(p, q);
    inv_pairs[2 * r] = pi; inv_pairs[2 * r + 1] = orc_shoup_quotient(pi, q);
    p = orc_mulmod(p, psi, q);
    pi = orc_mulmod(pi, psi_inv, q);
  }
  const uint64_t ni = orc_invmod(n % q, q);
  invn_pair[0] = ni; invn_pair[1] = orc_shoup_quotient(ni, q);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Modular primitives of the reference kernels.                               */
/* ------------------------------------------------------------------------ */
/* Shoup multiply, canonical a (switch.cu:13-16 `mul`, ntt.cu:37-39). */
static inline uint64_t mul_shoup(uint64_t a, uint64_t w, uint64_t wq, uint64_t q) {
  uint64_t t = mulhi64(a, wq);
  uint64_t r = a * w - t * q;
  return r >= q ? r - q : r;
}
uint64_t orc_mul_shoup(uint64_t a, uint64_t w, uint64_t wq, uint64_t q) { return mul_shoup(a, w, wq, q); }
static inline uint64_t add_mod(uint64_t a, uint64_t b, uint64_t q) { uint64_t x = a + b; return x >= q ? x - q : x; }
static inline uint64_t sub_mod(uint64_t a, uint64_t b, uint64_t q) { uint64_t x = a + q - b; return x >= q ? x - q : x; }

/* Barrett-128 (switch.cu:30-45): ratio = floor((2^128-1)/q) as (r0, r1). */
void orc_barrett_ratio(uint64_t q, uint64_t *r0, uint64_t *r1) {
  u128 ratio = (~(u128)0) / q;
  *r0 = (uint64_t)ratio;
  *r1 = (uint64_t)(ratio >> 64);
}
/* a*b mod q.  The reference's kernels reduce the 128-bit product with SEAL's
 * Barrett ratio (switch.cu:30-45); the result is the exact residue, so the
 * oracle states it directly as a 128-bit remainder (the ratio arguments are
 * kept for the callers' signatures). */
static inline uint64_t mul_barrett(uint64_t a, uint64_t b, uint64_t q, uint64_t r0, uint64_t r1) {
  (void)r0;
  (void)r1;
  return (uint64_t)(((u128)a * b) % q);
}
uint64_t orc_mul_barrett(uint64_t a, uint64_t b, uint64_t q) {
  uint64_t r0, r1;
  orc_barrett_ratio(q, &r0, &r1);
  return mul_barrett(a, b, q, r0, r1);
}

/* ------------------------------------------------------------------------ */
/* Negacyclic NTT / INTT, radix-2, stage by stage as the reference launches  */
/* them (ntt.cu:111-116 driving stage() ntt.cu:42-53):                        */
/*   forward stage l: gap = N>>(l+1), root = fwd[(1<<l) + group] (CT);        */
/*   inverse stage l: gap = 1<<l, root = inv[N-(N>>l)+1+group] (GS), and the  */
/*   last stage multiplies both outputs by N^-1.                               */
/* The loops run group by group (no division per butterfly) and keep Harvey's */
/* lazy ranges - forward values in [0, 4q), inverse in [0, 2q), with the      */
/* Shoup product a*w - floor(a*w'/2^64)*q in [0, 2q) for any a < 2^64 -, then */
/* reduce to canonical once at the end: every stage is exact mod q, so the   */
/* canonical outputs are the reference's.                                     */
/* ------------------------------------------------------------------------ */
static inline uint64_t shoup_lazy(uint64_t a, uint64_t w, uint64_t wq, uint64_t q) {
  return a * w - mulhi64(a, wq) * q;
}
void orc_ntt_forward(uint64_t *a, unsigned log_n, uint64_t q, const uint64_t *fwd_pairs) {
  const size_t n = (size_t)1 << log_n;
  const uint64_t q2 = 2 * q;
  for (unsigned l = 0; l < log_n; ++l) {
    const size_t gap = n >> (l + 1), groups = (size_t)1 << l;
    for (size_t g = 0; g < groups; ++g) {
      const uint64_t w = fwd_pairs[2 * (groups + g)], wq = fwd_pairs[2 * (groups + g) + 1];
      uint64_t *x = a + 2 * g * gap, *y = x + gap;
      for (size_t j = 0; j < gap; ++j) {
        const uint64_t u = x[j] >= q2 ? x[j] - q2 : x[j];
        const uint64_t t = shoup_lazy(y[j], w, wq, q);
        x[j] = u + t;
        y[j] = u - t + q2;
      }
    }
  }
  for (size_t i = 0; i < n; ++i) {
    const uint64_t v = a[i] >= q2 ? a[i] - q2 : a[i];
    a[i] = v >= q ? v - q : v;
  }
}
void orc_ntt_inverse(uint64_t *a, unsigned log_n, uint64_t q, const uint64_t *inv_pairs,
                     const uint64_t *invn_pair) {
  const size_t n = (size_t)1 << log_n;
  const uint64_t q2 = 2 * q;
  for (unsigned l = 0; l < log_n; ++l) {
    const size_t gap = (size_t)1 << l, groups = n >> (l + 1), root_start = n - (n >> l) + 1;
    const int last = (l + 1 == log_n);
    for (size_t g = 0; g < groups; ++g) {
      const uint64_t w = inv_pairs[2 * (root_start + g)], wq = inv_pairs[2 * (root_start + g) + 1];
      uint64_t *x = a + 2 * g * gap, *y = x + gap;
      for (size_t j = 0; j < gap; ++j) {
        const uint64_t u = x[j], v = y[j];
        uint64_t s = u + v;
        s = s >= q2 ? s - q2 : s;
        uint64_t d = shoup_lazy(u - v + q2, w, wq, q);
        if (last) {
          s = shoup_lazy(s, invn_pair[0], invn_pair[1], q);
          d = shoup_lazy(d, invn_pair[0], invn_pair[1], q);
        }
        x[j] = s;
        y[j] = d;
      }
    }
  }
  for (size_t i = 0; i < n; ++i) a[i] = a[i] >= q ? a[i] - q : a[i];
}
/* NttBatch::transform (ntt.cu:104-127) over a [limbs][N] buffer whose limb l
 * uses prime index l % primes.  Tables are [primes][N][2] / [primes][2]. */
void orc_ntt_batch(uint64_t *data, size_t limbs, unsigned log_n, size_t primes, const uint64_t *q,
                   const uint64_t *fwd, const uint64_t *inv, const uint64_t *invn, int inverse,
                   int threads) {
  const size_t n = (size_t)1 << log_n;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
  for (size_t l = 0; l < limbs; ++l) {
    const size_t k = l % primes;
    if (inverse)
      orc_ntt_inverse(data + l * n, log_n, q[k], inv + 2 * k * n, invn + 2 * k);
    else
      orc_ntt_forward(data + l * n, log_n, q[k], fwd + 2 * k * n);
  }
  (void)threads;
}

/* ------------------------------------------------------------------------ */
/* Galois automorphism a(X) -> a(X^g) in coefficient form                     */
/* (SEAL GaloisTool::apply_galois, called at keyswitch/seal_adapter.cpp:50):  */
/* coefficient i moves to i*g mod 2N; it is negated when that is >= N.        */
/* ------------------------------------------------------------------------ */
void orc_galois(const uint64_t *in, uint64_t *out, unsigned log_n, uint64_t q, uint32_t g) {
  const size_t n = (size_t)1 << log_n;
  for (size_t i = 0; i < n; ++i) {
    const size_t raw = (size_t)(((u128)i * g) % (2 * n));
    const uint64_t v = in[i];
    out[raw & (n - 1)] = (raw >= n) ? (v ? q - v : 0) : v;
  }
}
/* Negacyclic monomial shift by X^e (bfv_acyclic_pack.hpp:9-22). */
void orc_monomial_shift(const uint64_t *in, uint64_t *out, unsigned log_n, uint64_t q, size_t e) {
  const size_t n = (size_t)1 << log_n;
  e %= 2 * n;
  for (size_t j = 0; j < n; ++j) {
    const size_t dest = (j + e) % (2 * n);
    out[dest % n] = dest >= n ? (in[j] ? q - in[j] : 0) : in[j];
  }
}

/* ------------------------------------------------------------------------ */
/* Keyswitch, coefficient form in and out (Switch::evaluate switch.cu:113-125  */
/* with the CPU Galois step of keyswitch/seal_adapter.cpp:44-51):             */
/*   in  [2][L][N] over q_0..q_{L-1}; key [dnum][2][L+1][N] NTT form over     */
/*   q_0..q_{L-1}, p = q_L (the special prime); out [2][L][N].                 */
/* Digit j covers data primes [s_j, s_{j+1}), s_j = j*(L/dnum) + min(j, L%dnum) */
/* (balanced: the first L%dnum digits hold one extra prime; dnum=3, L=6 gives  */
/* pairs).  With dnum = L (one prime per digit) the ModUp step is exactly the */
/* reference decompose (switch.cu:63-68: digit residue reduced into each key  */
/* prime).  For alpha > 1 it is the fast base conversion                       */
/*   [d]_t = sum_i [[c1]_i * (Q_j/q_i)^-1]_{q_i} * (Q_j/q_i)  mod t            */
/* (no correction; the result is d + u*Q_j with 0 <= u < alpha).              */
/* Then: forward NTT of every expanded limb, key inner product with Barrett-  */
/* 128 (switch.cu:69-73), inverse NTT, ModDown (switch.cu:74-82).             */
/* ------------------------------------------------------------------------ */
typedef struct {
  size_t L, dnum;
  unsigned log_n;
  const uint64_t *q; /* L+1 */
  const uint64_t *fwd, *inv, *invn; /* per prime tables, L+1 primes */
} ks_ctx;

static void ks_one(const ks_ctx *c, const uint64_t *in, uint64_t *out, const uint64_t *key,
                   uint32_t galois, uint64_t *scratch /* (dnum+2)*(L+1)*N + 2*L*N */) {
  const size_t n = (size_t)1 << c->log_n, L = c->L, K = L + 1;
  uint64_t *perm = scratch;                 /* [2][L][N] */
  uint64_t *expanded = perm + 2 * L * n;    /* [dnum][K][N] */
  uint64_t *prod = expanded + c->dnum * K * n; /* [2][K][N] */
  for (size_t comp = 0; comp < 2; ++comp)
    for (size_t i = 0; i < L; ++i) {
      const uint64_t *src = in + (comp * L + i) * n;
      uint64_t *dst = perm + (comp * L + i) * n;
      if (galois == 1) memcpy(dst, src, n * 8);
      else orc_galois(src, dst, c->log_n, c->q[i], galois);
    }
  const uint64_t *c1 = perm + L * n;
  for (size_t j = 0; j < c->dnum; ++j) {
    const size_t base = L / c->dnum, extra = L % c->dnum;
    const size_t lo = j * base + (j < extra ? j : extra), hi = lo + base + (j < extra ? 1 : 0);
    /* constants of the digit: inv_hat[i] = (Q_j/q_i)^-1 mod q_i, hat_t[i] = Q_j/q_i mod t */
    uint64_t inv_hat[64];
    for (size_t i = lo; i < hi; ++i) {
      uint64_t h = 1;
      for (size_t i2 = lo; i2 < hi; ++i2) if (i2 != i) h = orc_mulmod(h, c->q[i2] % c->q[i], c->q[i]);
      inv_hat[i - lo] = orc_invmod(h, c->q[i]);
    }
    for (size_t t = 0; t < K; ++t) {
      uint64_t *dst = expanded + (j * K + t) * n;
      const uint64_t qt = c->q[t];
      if (t >= lo && t < hi) { memcpy(dst, c1 + t * n, n * 8); continue; }
      uint64_t hat_t[64];
      for (size_t i = lo; i < hi; ++i) {
        uint64_t h = 1;
        for (size_t i2 = lo; i2 < hi; ++i2) if (i2 != i) h = orc_mulmod(h, c->q[i2] % qt, qt);
        hat_t[i - lo] = h;
      }
      for (size_t k = 0; k < n; ++k) {
        uint64_t acc = 0;
        for (size_t i = lo; i < hi; ++i) {
          const uint64_t y = orc_mulmod(c1[i * n + k], inv_hat[i - lo], c->q[i]);
          acc = add_mod(acc, orc_mulmod(y % qt, hat_t[i - lo], qt), qt);
        }
        dst[k] = acc;
      }
    }
  }
  for (size_t j = 0; j < c->dnum; ++j)
    for (size_t t = 0; t < K; ++t)
      orc_ntt_forward(expanded + (j * K + t) * n, c->log_n, c->q[t], c->fwd + 2 * t * n);
  for (size_t comp = 0; comp < 2; ++comp)
    for (size_t t = 0; t < K; ++t) {
      uint64_t r0, r1;
      orc_barrett_ratio(c->q[t], &r0, &r1);
      uint64_t *dst = prod + (comp * K + t) * n;
      for (size_t k = 0; k < n; ++k) {
        uint64_t sum = 0;
        for (size_t j = 0; j < c->dnum; ++j) {
          const uint64_t v = mul_barrett(expanded[(j * K + t) * n + k],
                                         key[((j * 2 + comp) * K + t) * n + k], c->q[t], r0, r1);
          sum = add_mod(sum, v, c->q[t]);
        }
        dst[k] = sum;
      }
      orc_ntt_inverse(dst, c->log_n, c->q[t], c->inv + 2 * t * n, c->invn + 2 * t);
    }
  /* ModDown by the special prime p = q_L (switch.cu:74-82). */
  const uint64_t p = c->q[L], half = p >> 1;
  for (size_t comp = 0; comp < 2; ++comp)
    for (size_t i = 0; i < L; ++i) {
      const uint64_t qi = c->q[i];
      const uint64_t invp = orc_invmod(p % qi, qi), invp_q = orc_shoup_quotient(invp, qi);
      const uint64_t halfmod = half % qi;
      for (size_t k = 0; k < n; ++k) {
        uint64_t last = prod[(comp * K + L) * n + k] + half;
        last = last >= p ? last - p : last;
        const uint64_t reduced = last % qi;
        const uint64_t correction = sub_mod(reduced, halfmod, qi);
        const uint64_t value = mul_shoup(sub_mod(prod[(comp * K + i) * n + k], correction, qi), invp, invp_q, qi);
        out[(comp * L + i) * n + k] = comp == 0 ? add_mod(perm[i * n + k], value, qi) : value;
      }
    }
}

/* Batched keyswitch: in/out [batch][2][L][N]; key_stride words between
 * consecutive ciphertexts' keys (0 = one shared key). */
int orc_keyswitch(const uint64_t *in, uint64_t *out, const uint64_t *key, size_t key_stride,
                  size_t batch, const uint64_t *q, size_t L, size_t dnum, unsigned log_n,
                  uint32_t galois, const uint64_t *fwd, const uint64_t *inv, const uint64_t *invn,
                  int threads) {
  if (dnum == 0 || dnum > L || L > 63) return -1;
  ks_ctx c;
  c.L = L; c.dnum = dnum; c.log_n = log_n;
  c.q = q; c.fwd = fwd; c.inv = inv; c.invn = invn;
  const size_t n = (size_t)1 << log_n, words = 2 * L * n;
  const size_t scratch_words = 2 * L * n + (dnum + 2) * (L + 1) * n;
  int status = 0;
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
#endif
  {
    uint64_t *scratch = (uint64_t *)malloc(scratch_words * 8);
    if (!scratch) status = -2;
    else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
      for (size_t b = 0; b < batch; ++b)
        ks_one(&c, in + b * words, out + b * words, key + b * key_stride, galois, scratch);
      free(scratch);
    }
  }
  (void)threads;
  return status;
}

/* ------------------------------------------------------------------------ */
/* Public-key encryption of zero at the key level, then ModDown               */
/* (PublicZero::evaluate, enc0.cu:99-114; sequence of the CPU reference        */
/* enc0/seal_adapter.cpp:56-61): samples [3][K][N] = u, e0, e1 as residues of  */
/* the K = L+1 key primes; pk [2][K][N] in NTT form;                          */
/*   P_c = INTT(NTT(u) (.) pk_c) + e_c,  out_c = ModDown_p(P_c)  [2][L][N].    */
/* ------------------------------------------------------------------------ */
int orc_enc0(const uint64_t *samples, const uint64_t *pk, uint64_t *out, const uint64_t *q, size_t L,
             unsigned log_n, const uint64_t *fwd, const uint64_t *inv, const uint64_t *invn, int threads) {
  const size_t K = L + 1, n = (size_t)1 << log_n;
  uint64_t *u = (uint64_t *)malloc(K * n * 8), *prod = (uint64_t *)malloc(2 * K * n * 8);
  if (!u || !prod) { free(u); free(prod); return -2; }
  memcpy(u, samples, K * n * 8);
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
  for (size_t t = 0; t < K; ++t) orc_ntt_forward(u + t * n, log_n, q[t], fwd + 2 * t * n);
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 1) num_threads(threads)
#endif
  for (size_t comp = 0; comp < 2; ++comp)
    for (size_t t = 0; t < K; ++t) {
      uint64_t r0, r1;
      orc_barrett_ratio(q[t], &r0, &r1);
      uint64_t *dst = prod + (comp * K + t) * n;
      for (size_t k = 0; k < n; ++k) dst[k] = mul_barrett(u[t * n + k], pk[(comp * K + t) * n + k], q[t], r0, r1);
      orc_ntt_inverse(dst, log_n, q[t], inv + 2 * t * n, invn + 2 * t);
      const uint64_t *e = samples + ((comp + 1) * K + t) * n;
      for (size_t k = 0; k < n; ++k) dst[k] = add_mod(dst[k], e[k], q[t]);
    }
  const uint64_t p = q[L], half = p >> 1;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 1) num_threads(threads)
#endif
  for (size_t comp = 0; comp < 2; ++comp)
    for (size_t i = 0; i < L; ++i) {
      const uint64_t qi = q[i];
      const uint64_t invp = orc_invmod(p % qi, qi), invp_q = orc_shoup_quotient(invp, qi);
      const uint64_t halfmod = half % qi;
      for (size_t k = 0; k < n; ++k) {
        uint64_t last = prod[(comp * K + L) * n + k] + half;
        last = last >= p ? last - p : last;
        const uint64_t correction = sub_mod(last % qi, halfmod, qi);
        out[(comp * L + i) * n + k] =
            mul_shoup(sub_mod(prod[(comp * K + i) * n + k], correction, qi), invp, invp_q, qi);
      }
    }
  free(u);
  free(prod);
  (void)threads;
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Party-local share GEMM (bfv_matrix.inc:177-182; same loop at :101-105 and   */
/* :156-160): Y[b][o] = sum_j X[b][j] * W[o][j] in wrapping uint64, then the  */
/* optional per-output left shift (exact on additive shares) and the mask to  */
/* the ring 2^mask_bits (mask_bits 59 = reference ring, 64 = no mask).         */
/* W is signed (int8 or int32, [O][K] = the reference [out][in] order); it    */
/* enters the ring as its two's-complement word, as artifacts.hpp:86-92 lifts */
/* it.                                                                          */
/* ------------------------------------------------------------------------ */
int orc_share_gemm(const uint64_t *x, const void *w, int w_bits, const int8_t *shifts, uint64_t *y,
                   size_t m, size_t k, size_t n, int mask_bits, int threads) {
  if (w_bits != 8 && w_bits != 32) return -1;
  if (mask_bits < 1 || mask_bits > 64) return -1;
  const uint64_t mask = mask_bits == 64 ? ~0ULL : ((1ULL << mask_bits) - 1);
#ifdef _OPENMP
  if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
  for (size_t b = 0; b < m; ++b) {
    const uint64_t *xr = x + b * k;
    for (size_t o = 0; o < n; ++o) {
      uint64_t acc = 0;
      if (w_bits == 8) {
        const int8_t *wr = (const int8_t *)w + o * k;
        for (size_t j = 0; j < k; ++j) acc += xr[j] * (uint64_t)(int64_t)wr[j];
      } else {
        const int32_t *wr = (const int32_t *)w + o * k;
        for (size_t j = 0; j < k; ++j) acc += xr[j] * (uint64_t)(int64_t)wr[j];
      }
      if (shifts) acc <<= (unsigned)shifts[o];
      y[b * n + o] = acc & mask;
    }
  }
  (void)threads;
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Element-wise ops of the other backends.                                    */
/* ------------------------------------------------------------------------ */
/* Centred lift of a ring-2^59 word into Z_q (resident.cu:23-30, matrix.cu:23-26):
 * the signed value of v (v - 2^59 when bit 58 is set) as a canonical residue.
 * For the reference's primes (q > 2^59) this is its branch-free
 * v + ((q - 2^59) & -(v >> 58)); smaller primes take the remainder. */
uint64_t orc_lift59(uint64_t v, uint64_t q) {
  if (q > (1ULL << 59)) return v + ((q - (1ULL << 59)) & (0ULL - (v >> 58)));
  if (!(v >> 58)) return v % q;
  const uint64_t d = ((1ULL << 59) - v) % q;
  return d ? q - d : 0;
}
/* Centred lift over blocks (matrix.cu:23-26 for width 0, resident.cu:23-30
 * for width > 0): out[b][k][z] = lift(v, q_k) with v = ring[b][z] (ring
 * [blocks][n]) or v = ring[b][width-1-z] for z < width and 0 above (ring
 * [blocks][width]). */
void orc_lift59_blocks(const uint64_t *ring, uint64_t *out, size_t blocks, size_t n, size_t width,
                       const uint64_t *q, size_t primes) {
  for (size_t b = 0; b < blocks; ++b)
    for (size_t k = 0; k < primes; ++k)
      for (size_t z = 0; z < n; ++z) {
        uint64_t v;
        if (width == 0)
          v = orc_lift59(ring[b * n + z], q[k]);
        else
          v = z < width ? orc_lift59(ring[b * width + (width - 1 - z)], q[k]) : 0;
        out[(b * primes + k) * n + z] = v;
      }
}

/* LocalShares ring ops (compute/local_shares.cu:9-12), mod 2^bits. */
static uint64_t ring_mask_bits(int bits) { return bits >= 64 ? ~0ULL : (1ULL << bits) - 1; }
void orc_ring_add(const uint64_t *a, const uint64_t *b, uint64_t *c, size_t n, int bits) {
  for (size_t i = 0; i < n; ++i) c[i] = (a[i] + b[i]) & ring_mask_bits(bits);
}
void orc_ring_scale(const uint64_t *a, uint64_t k, uint64_t *c, size_t n, int bits) {
  for (size_t i = 0; i < n; ++i) c[i] = (a[i] * k) & ring_mask_bits(bits);
}
/* layout: c[i] = a[map[i]]; an index out of range gives 0 here (the
 * reference rejects such a map before any kernel runs). */
void orc_ring_layout(const uint64_t *a, size_t n_in, const uint64_t *map, uint64_t *c, size_t n_out) {
  for (size_t i = 0; i < n_out; ++i) c[i] = map[i] < n_in ? a[map[i]] : 0;
}
void orc_ring_sum_rows(const uint64_t *a, uint64_t *out, size_t rows, size_t cols, int bits) {
  for (size_t r = 0; r < rows; ++r) {
    uint64_t x = 0;
    for (size_t i = 0; i < cols; ++i) x += a[r * cols + i];
    out[r] = x & ring_mask_bits(bits);
  }
}

/* Dyadic multiply-accumulate out = sum_b a_b (.) w_b mod q with Barrett-128
 * (resident.cu:38-45 accumulate, matrix.cu:34-38 product). a is
 * [blocks][limbs][N], w is [blocks][primes][N] broadcast over the limbs whose
 * prime index is l % primes; out [limbs][N]. */
void orc_dyadic_mac(const uint64_t *a, const uint64_t *w, uint64_t *out, size_t blocks,
                    size_t limbs, size_t n, size_t primes, const uint64_t *q, size_t w_limbs) {
  for (size_t l = 0; l < limbs; ++l) {
    const size_t k = l % primes;
    for (size_t z = 0; z < n; ++z) {
      uint64_t sum = 0;
      for (size_t b = 0; b < blocks; ++b)
        sum = add_mod(sum, orc_mul_barrett(a[(b * limbs + l) * n + z], w[(b * w_limbs + (l % w_limbs)) * n + z], q[k]), q[k]);
      out[l * n + z] = sum;
    }
  }
}
/* Party-local dot product and BFV Delta scaling (resident.cu:60-74 and
 * resident/seal_adapter.cpp:43-53):
 *   m = (sum_j s[j] * w[j] mod 2^64) & (2^59-1)
 *   scaled_k = Delta_k * m + floor((r*m + 2^58) / 2^59) mod q_k
 * where Delta_k = floor(Q/t) mod q_k and r = Q mod t (t = 2^59). */
void orc_local_dot_scale(const uint64_t *shares, const uint64_t *weights, size_t words,
                         size_t slots, const uint64_t *delta, uint64_t r, const uint64_t *q,
                         size_t primes, uint64_t *scaled) {
  for (size_t s = 0; s < slots; ++s) {
    uint64_t sum = 0;
    for (size_t j = 0; j < words; ++j) sum += shares[s * words + j] * weights[j];
    const uint64_t m = sum & ((1ULL << 59) - 1);
    const u128 num = (u128)r * m + (1ULL << 58);
    const uint64_t fix = (uint64_t)(num >> 59);
    for (size_t k = 0; k < primes; ++k) {
      const uint64_t z = orc_mulmod(m, delta[k], q[k]);
      scaled[s * primes + k] = (uint64_t)(((u128)z + fix) % q[k]);
    }
  }
}
