// CPU check of the NTT register/LDS layout (PassMap in ntt_core.hpp), for every
// pass of every transform size:
//   - elem(t, j) is a bijection onto [0, N);
//   - lds_pos(elem(t, j)) == lds_pos(elem(t, 0)) + slot_offset(j), inside the
//     N + N/16 padded buffer;
//   - when uniform_groups() holds, the twiddle group (bits above the gap bits)
//     is the same for all lanes of a wave;
//   - consecutive passes with equal wave bits give each wave the same
//     coefficients (their exchange stays inside the wave);
//   - the forward output registers pair up at adjacent positions.
#include <cstdio>
#include <vector>

#include "ntt_core.hpp"
using namespace praghip;

template <int LOGN, bool INV, int P>
int check_pass() {
  using M = PassMap<LOGN, INV, P>;
  constexpr unsigned N = 1u << LOGN, THREADS = N >> kLogE, LIMIT = N + N / 16;
  std::vector<int> seen(N, 0);
  int bad = 0;
  for (unsigned t = 0; t < THREADS; ++t)
    for (int j = 0; j < kE; ++j) {
      const unsigned x = M::elem(t, j);
      if (x >= N) { ++bad; continue; }
      seen[x]++;
      if (lds_pos(x) != lds_pos(M::elem(t, 0)) + M::slot_offset(j) || lds_pos(x) >= LIMIT) ++bad;
      // element bits in the gap window must come from the register index
      if (((x >> M::LO) & ((1u << M::R) - 1)) != (unsigned(j) & ((1u << M::R) - 1))) ++bad;
    }
  for (unsigned x = 0; x < N; ++x) bad += seen[x] != 1;
  if (M::uniform_groups())
    for (unsigned t = 0; t < THREADS; ++t)
      for (int b = 0; b < (kE >> M::R); ++b)
        if ((M::elem(t, b << M::R) >> (M::LO + M::R)) != (M::elem(t & ~63u, b << M::R) >> (M::LO + M::R))) ++bad;
  if constexpr (P + 1 < Passes<LOGN>::NP) {
    using B = PassMap<LOGN, INV, P + 1>;
    if (M::WAVE_LO == B::WAVE_LO)
      for (unsigned t = 0; t < THREADS; ++t) {
        const unsigned w = t >> 6;
        for (int j = 0; j < kE; ++j) {
          // the coefficient t holds after the exchange belongs to wave w before it
          const unsigned x = B::elem(t, j);
          bool found = false;
          for (unsigned l = 0; l < 64 && (w * 64 + l) < THREADS && !found; ++l)
            for (int j2 = 0; j2 < kE && !found; ++j2) found = M::elem(w * 64 + l, j2) == x;
          if (!found) ++bad;
        }
      }
    bad += check_pass<LOGN, INV, P + 1>();
  }
  if (bad) printf("LOGN=%d INV=%d pass=%d: %d violations\n", LOGN, int(INV), P, bad);
  return bad;
}

template <int LOGN>
int check_size() {
  // after the last forward pass registers 2k and 2k + 1 sit at adjacent,
  // 16-byte aligned positions (the keyswitch loads its keys in pairs)
  using Last = PassMap<LOGN, false, Passes<LOGN>::NP - 1>;
  int bad = 0;
  for (unsigned t = 0; t < (1u << LOGN) >> kLogE; ++t)
    for (int j = 0; j < kE; j += 2) bad += (Last::elem(t, j) & 1) || Last::elem(t, j + 1) != Last::elem(t, j) + 1;
  if (bad) printf("LOGN=%d: %d unpaired forward outputs\n", LOGN, bad);
  return bad + check_pass<LOGN, false, 0>() + check_pass<LOGN, true, 0>();
}

int main() {
  const int bad = check_size<4>() + check_size<5>() + check_size<6>() + check_size<7>() + check_size<8>() +
                  check_size<9>() + check_size<10>() + check_size<11>() + check_size<12>() + check_size<13>() +
                  check_size<14>();
  printf(bad ? "FAIL\n" : "ALL OK\n");
  return bad != 0;
}
