// CPU check of the integer helpers in modarith.hpp against 128-bit host
// arithmetic: shoup_quotient(w, m) == floor(w 2^64 / q) and mul_shoup /
// mul_barrett == a w mod q, for primes from 2^20 to 2^62 and edge operands
// (0, 1, q-1, q/2, random).  Plants one wrong ratio to show the check fails.
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
  printf("bad=%d planted=%d\n", bad, planted);
  printf(bad == 0 && planted > 0 ? "ALL OK\n" : "FAIL\n");
  return !(bad == 0 && planted > 0);
}
