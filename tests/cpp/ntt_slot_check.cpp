// CPU check of the NTT register/LDS layout (PassMap in ntt_core.hpp), for every
// pass of every transform size with 16 coefficients per thread, and of the
// 1024-coefficient row transforms with 8 and 4 coefficients per thread:
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

template <int LOGN, bool INV, int P, int LE = kLogE>
int check_pass() {
  using M = PassMap<LOGN, INV, P, LE>;
  constexpr int kE = 1 << LE;
  constexpr unsigned N = 1u << LOGN, THREADS = N >> LE, LIMIT = N + N / 16;
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
  if constexpr (P + 1 < Passes<LOGN, LE>::NP) {
    using B = PassMap<LOGN, INV, P + 1, LE>;
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
    bad += check_pass<LOGN, INV, P + 1, LE>();
  }
  if (bad) printf("LOGN=%d LE=%d INV=%d pass=%d: %d violations\n", LOGN, LE, int(INV), P, bad);
  return bad;
}

template <int LOGN, int LE = kLogE>
int check_size() {
  // after the last forward pass registers 2k and 2k + 1 sit at adjacent,
  // 16-byte aligned positions (the keyswitch loads its keys in pairs)
  using Last = PassMap<LOGN, false, Passes<LOGN, LE>::NP - 1, LE>;
  int bad = 0;
  for (unsigned t = 0; t < (1u << LOGN) >> LE; ++t)
    for (int j = 0; j < (1 << LE); j += 2)
      bad += (Last::elem(t, j) & 1) || Last::elem(t, j + 1) != Last::elem(t, j) + 1;
  if (bad) printf("LOGN=%d LE=%d: %d unpaired forward outputs\n", LOGN, LE, bad);
  return bad + check_pass<LOGN, false, 0, LE>() + check_pass<LOGN, true, 0, LE>();
}

int main() {
  const int bad = check_size<4>() + check_size<5>() + check_size<6>() + check_size<7>() + check_size<8>() +
                  check_size<9>() + check_size<10>() + check_size<11>() + check_size<12>() + check_size<13>() +
                  check_size<14>() + check_size<10, 3>() + check_size<10, 2>();
  printf(bad ? "FAIL\n" : "ALL OK\n");
  return bad != 0;
}
