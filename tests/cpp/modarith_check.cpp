// CPU check of the integer helpers in modarith.hpp against 128-bit host
// arithmetic: shoup_quotient(w, m) == floor(w 2^64 / q) and mul_shoup /
// mul_barrett == a w mod q, for primes from 2^20 to 2^62 and edge operands
// (0, 1, q-1, q/2, random), mul_mont (x k 2^-64 mod q) for primes below
// 2^60, and the float product mul_f64_hq against its bound for primes below
// 2^50.  Plants a wrong ratio, a wrong -q^-1 and a wrong reciprocal to show
// the checks fail.
#include <cstdio>
#include <random>
#include <vector>

#include "modarith.hpp"
using namespace praghip;
using u128 = unsigned __int128;

static Barrett ratio(uint64_t q) {
  const u128 r = (~(u128)0) / q;
  return Barrett{q, uint64_t(r), uint64_t(r >> 64)};
}

static int check(uint64_t q, std::mt19937_64& rng, const Barrett m) {
  int bad = 0;
  std::vector<uint64_t> ws = {0, 1, q - 1, q / 2, q / 2 + 1, q - 2};
  for (int i = 0; i < 2000; ++i) ws.push_back(rng() % q);
  for (uint64_t w : ws) {
    const uint64_t want = uint64_t(((u128)w << 64) / q);
    const uint64_t wq = shoup_quotient(w, m);
    if (wq != want) ++bad;
    for (uint64_t a : {uint64_t(0), uint64_t(1), q - 1, rng() % q, rng() % q}) {
      const uint64_t prod = uint64_t((u128)a * w % q);
      if (mul_shoup(a, w, wq, q) != prod || mul_barrett(a, w, m) != prod) ++bad;
    }
  }
  return bad;
}

// mul_mont(x, k) for the lazy integer key products: x below 12q (a forward
// transform's output bound), k canonical, q < 2^60.  The result must lie in
// [0, 2q) and satisfy r 2^64 == x k (mod q).
static int check_mont(uint64_t q, uint64_t nq, std::mt19937_64& rng) {
  int bad = 0;
  const uint64_t x12 = 12 * q;
  std::vector<uint64_t> xs = {0, 1, q - 1, q, 2 * q + 1, x12 - 1, x12 / 2};
  std::vector<uint64_t> ks = {0, 1, q - 1, q / 2};
  for (int i = 0; i < 400; ++i) xs.push_back(rng() % x12), ks.push_back(rng() % q);
  for (uint64_t x : xs)
    for (size_t j = 0; j < ks.size(); j += (x < 8 ? 1 : 37)) {
      const uint64_t k = ks[j], r = mul_mont(x, k, q, nq);
      if (r >= 2 * q || (((u128)r << 64) % q) != ((u128)x * k) % q) ++bad;
    }
  return bad;
}

// mul_f64_hq (the float path's product, q < 2^50): for |a| <= A q and w < q
// the result r is an integer with r == a w (mod q) and |r| <= (1/2 + 3A/8) q
// (the bound the re-centring schedules rely on), for A up to 8.  qinv is
// `qinv` (1/q rounded, or a planted wrong value).
static int check_f64(uint64_t q, double qinv, std::mt19937_64& rng) {
  int bad = 0;
  const double qd = double(q);
  std::vector<uint64_t> ws = {0, 1, q - 1, q / 2, q - 2};
  for (int i = 0; i < 300; ++i) ws.push_back(rng() % q);
  for (double A : {1.0, 4.0, 5.3, 7.7, 8.0}) {
    const int64_t amax = int64_t(A * qd);
    std::vector<int64_t> as = {0, 1, -1, amax, -amax, amax - 1, int64_t(q) - 1};
    for (int i = 0; i < 300; ++i) as.push_back(int64_t(rng() % uint64_t(2 * amax + 1)) - amax);
    const double lim = (0.5 + 0.375 * A) * qd;
    for (int64_t a : as)
      for (uint64_t w : ws) {
        const double r = mul_f64_hq(double(a), double(w), qd, qinv);
        if (r != __builtin_rint(r) || __builtin_fabs(r) > lim) {
          ++bad;
          continue;
        }
        const __int128 d = (__int128)a * (__int128)w - (__int128)(int64_t)r;
        if (d % (__int128)q != 0) ++bad;
      }
  }
  return bad;
}

int main() {
  std::mt19937_64 rng(12345);
  const std::vector<uint64_t> primes = {
      1048583ull,             // 2^20 + 7
      1125899906826241ull,    // a prime below 2^50
      1152921504599080961ull, 1152921504606748673ull,  // locked 60-bit primes
      4611686018427322369ull, // a prime below 2^62
  };
  int bad = 0;
  for (uint64_t q : primes) bad += check(q, rng, ratio(q));
  // planted error: an off-by-one ratio must be caught
  Barrett wrong = ratio(primes[2]);
  wrong.r0 -= 1ull << 40;
  const int planted = check(primes[2], rng, wrong);
  // Montgomery products on the primes below 2^60; -q^-1 mod 2^64 by Newton
  // iteration (each step doubles the correct low bits), pinned by q nq == -1
  int mont_bad = 0, mont_planted = 0;
  for (uint64_t q : primes) {
    if (q >> 60) continue;
    uint64_t y = q;  // q q == 1 mod 8: three correct bits
    for (int i = 0; i < 6; ++i) y *= 2 - q * y;
    const uint64_t nq = 0 - y;
    if (q * nq != ~0ull) ++mont_bad;
    mont_bad += check_mont(q, nq, rng);
    mont_planted += check_mont(q, nq + 2, rng) > 0;
  }
  // the float product on primes below 2^50; a reciprocal 2^-30 too large
  // must break the bound
  int f64_bad = 0;
  for (uint64_t q : {1048583ull, 1125899906826241ull, 562949952798721ull, 1125899904679937ull})
    f64_bad += check_f64(q, 1.0 / double(q), rng);
  const int f64_planted = check_f64(1125899906826241ull, (1.0 / 1125899906826241.0) * (1.0 + 0x1p-30), rng);
  printf("bad=%d planted=%d mont_bad=%d mont_planted=%d f64_bad=%d f64_planted=%d\n", bad, planted, mont_bad,
         mont_planted, f64_bad, f64_planted);
  const bool ok = bad == 0 && planted > 0 && mont_bad == 0 && mont_planted == 4 && f64_bad == 0 && f64_planted > 0;
  printf(ok ? "ALL OK\n" : "FAIL\n");
  return !ok;
}
