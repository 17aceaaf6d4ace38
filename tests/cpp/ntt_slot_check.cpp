// CPU check of the NTT LDS layout: for every pass of every transform size,
// lds_pos(elem_index(t, j)) == lds_pos(elem_index(t, 0)) + slot_offset(j), and
// every slot stays inside the N + N/16 padded buffer.
#include "ntt_core.hpp"
#include <cstdio>
using namespace praghip;
template <int LOGN, int LO, int R> int check() {
  constexpr unsigned THREADS = (1u << LOGN) >> kLogE;
  int bad = 0; unsigned maxpos = 0;
  for (unsigned t = 0; t < THREADS; ++t)
    for (int j = 0; j < kE; ++j) {
      unsigned a = lds_pos(elem_index<LOGN, LO, R>(t, j));
      unsigned b = lds_pos(elem_index<LOGN, LO, R>(t, 0)) + slot_offset<LOGN, LO, R>(j);
      if (a != b) ++bad;
      if (b > maxpos) maxpos = b;
    }
  printf("LOGN=%d LO=%d R=%d bad=%d maxpos=%u limit=%u\n", LOGN, LO, R, bad, maxpos, (1u << LOGN) + (1u << LOGN) / 16);
  return bad + (maxpos >= (1u << LOGN) + (1u << LOGN) / 16);
}
template <int LOGN> int all() {
  using S = Passes<LOGN>;
  int bad = 0;
  bad += check<LOGN, S::fwd_lo(0), S::fwd_r(0)>();
  if constexpr (S::NP > 1) bad += check<LOGN, S::fwd_lo(1), S::fwd_r(1)>() + check<LOGN, S::inv_lo(1), S::inv_r(1)>();
  if constexpr (S::NP > 2) bad += check<LOGN, S::fwd_lo(2), S::fwd_r(2)>() + check<LOGN, S::inv_lo(2), S::inv_r(2)>();
  if constexpr (S::NP > 3) bad += check<LOGN, S::fwd_lo(3), S::fwd_r(3)>() + check<LOGN, S::inv_lo(3), S::inv_r(3)>();
  bad += check<LOGN, S::inv_lo(0), S::inv_r(0)>();
  return bad;
}
int main() {
  int bad = all<4>() + all<5>() + all<6>() + all<7>() + all<8>() + all<9>() + all<10>() + all<11>() + all<12>() + all<13>() + all<14>();
  printf(bad ? "FAIL\n" : "ALL OK\n");
  return bad != 0;
}
