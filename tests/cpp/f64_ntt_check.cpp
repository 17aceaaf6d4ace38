// CPU check of the float-path NTT arithmetic (ArF64 in ntt_core.hpp with
// mul_f64_hq / reduce_f64 from modarith.hpp), stage by stage in the reference's
// radix-2 order (ntt.cu:42-53).  The register passes of the GPU kernel apply
// the same butterflies to the same operands and re-centre whole blocks after
// the same stages, so every intermediate value here equals the GPU's.
//
// For every butterfly output the double must be an exact integer congruent to
// the exact residue (tracked alongside in 128-bit integers) and below 2^53.
// Both re-centring schedules are replayed: ArF64's (the keyswitch kernels;
// every factor within 4q, every value below 8q) and ArF64T's (the standalone
// transform; factors and values within 8q + 16).  The final canonical outputs
// are compared with the expected transform.
//
// Input file (little-endian u64): q, log_n, cases, fwd_pairs[N][2],
// inv_pairs[N][2], invn_pair[2], then per case: input[N], forward[N] (the
// expected forward transform of input); the inverse is checked by
// transforming `forward` back to `input`.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "modarith.hpp"
#include "ntt_core.hpp"
using namespace praghip;
typedef unsigned __int128 u128;

static uint64_t mulmod(uint64_t a, uint64_t b, uint64_t q) { return (uint64_t)((u128)a * b % q); }

struct Checker {
  uint64_t q;
  double qd, qinv;
  double max_factor = 0, max_value = 0, factor_lim;
  long bad = 0;
  Checker(uint64_t q_, double lim) : q(q_), qd(double(q_)), qinv(1.0 / double(q_)), factor_lim(lim) {}
  // residue of an integer-valued double
  uint64_t res(double x) {
    if (x != std::rint(x) || std::fabs(x) >= 9007199254740992.0) { ++bad; return 0; }
    long long v = (long long)x % (long long)q;
    return uint64_t(v < 0 ? v + (long long)q : v);
  }
  double mul(double a, double w, uint64_t wi, uint64_t ai) {
    max_factor = std::fmax(max_factor, std::fabs(a) / qd);
    if (std::fabs(a) > factor_lim * qd) ++bad;
    const double r = mul_f64_hq(a, w, qd, qinv);  // ArF64::mul
    if (res(r) != mulmod(ai, wi, q)) ++bad;
    return r;
  }
  void track(double x) { max_value = std::fmax(max_value, std::fabs(x) / qd); }
};

int main(int argc, char** argv) {
  if (argc != 2) return 2;
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) return 2;
  uint64_t hdr[3];
  if (std::fread(hdr, 8, 3, f) != 3) return 2;
  const uint64_t q = hdr[0];
  const int log_n = int(hdr[1]);
  const size_t n = size_t(1) << log_n, cases = hdr[2];
  std::vector<uint64_t> fwd(2 * n), inv(2 * n), invn(2);
  if (std::fread(fwd.data(), 8, 2 * n, f) != 2 * n || std::fread(inv.data(), 8, 2 * n, f) != 2 * n ||
      std::fread(invn.data(), 8, 2, f) != 2)
    return 2;
  const uint64_t last_i = mulmod(inv[2 * (n - 1)], invn[0], q);
  std::vector<std::vector<uint64_t>> ins(cases, std::vector<uint64_t>(n)), expects(cases, std::vector<uint64_t>(n));
  for (size_t c = 0; c < cases; ++c)
    if (std::fread(ins[c].data(), 8, n, f) != n || std::fread(expects[c].data(), 8, n, f) != n) return 2;
  int fails = 0;
  for (int sparse = 0; sparse < 2; ++sparse) {
  const auto settle_fwd = [&](int s) { return sparse ? ArF64T::settle_fwd(s) : ArF64::settle_fwd(s); };
  const auto settle_inv = [&](int l) { return sparse ? ArF64T::settle_inv(l) : ArF64::settle_inv(l); };
  const double lim = sparse ? 8.0 + 16.0 / double(q) : 4.0, vlim = sparse ? 8.0 + 16.0 / double(q) : 8.0;
  Checker ck(q, lim);
  long mismatches = 0;
  for (size_t c = 0; c < cases; ++c) {
    const std::vector<uint64_t>& in = ins[c];
    const std::vector<uint64_t>& expect = expects[c];
    // forward: values and exact residues
    std::vector<double> v(n);
    std::vector<uint64_t> e(in);
    for (size_t i = 0; i < n; ++i) v[i] = double(in[i]);
    for (int s = 0; s < log_n; ++s) {
      const size_t gap = n >> (s + 1);
      for (size_t g = 0; g < (size_t(1) << s); ++g) {
        const uint64_t wi = fwd[2 * ((size_t(1) << s) + g)];
        const double w = double(wi);
        for (size_t k = 0; k < gap; ++k) {
          const size_t j0 = 2 * g * gap + k, j1 = j0 + gap;
          const double t = ck.mul(v[j1], w, wi, e[j1]);
          const double x = v[j0];
          v[j0] = x + t;
          v[j1] = x - t;
          const uint64_t tm = mulmod(e[j1], wi, q);
          const uint64_t x0 = e[j0];
          e[j0] = (x0 + tm) % q;
          e[j1] = (x0 + q - tm) % q;
          ck.track(v[j0]);
          ck.track(v[j1]);
          if (ck.res(v[j0]) != e[j0] || ck.res(v[j1]) != e[j1]) ++ck.bad;
        }
      }
      if (settle_fwd(s) && s != log_n - 1)
        for (size_t i = 0; i < n; ++i) {
          v[i] = reduce_f64(v[i], ck.qd, ck.qinv);
          if (std::fabs(v[i]) > 0.5 * ck.qd + 1.0 || ck.res(v[i]) != e[i]) ++ck.bad;
        }
    }
    for (size_t i = 0; i < n; ++i) {
      const double r = canon_f64(reduce_f64(v[i], ck.qd, ck.qinv), ck.qd);
      if (uint64_t(r) != expect[i] || e[i] != expect[i]) ++mismatches;
    }
    // inverse of the expected forward transform
    for (size_t i = 0; i < n; ++i) {
      v[i] = double(expect[i]);
      e[i] = expect[i];
    }
    for (int l = 0; l < log_n; ++l) {
      const size_t gap = size_t(1) << l;
      const size_t root_start = n - (n >> l) + 1;
      for (size_t j0 = 0; j0 < n; ++j0) {
        if (j0 & gap) continue;
        const size_t j1 = j0 + gap, g = j0 >> (l + 1);
        const double x = v[j0], y = v[j1];
        const double s = x + y, d = x - y;
        const uint64_t es = (e[j0] + e[j1]) % q, ed = (e[j0] + q - e[j1]) % q;
        if (l == log_n - 1) {
          v[j0] = ck.mul(s, double(invn[0]), invn[0], es);
          v[j1] = ck.mul(d, double(last_i), last_i, ed);
          e[j0] = mulmod(es, invn[0], q);
          e[j1] = mulmod(ed, last_i, q);
        } else {
          const uint64_t wi = inv[2 * (root_start + g)];
          v[j0] = s;
          v[j1] = ck.mul(d, double(wi), wi, ed);
          e[j0] = es;
          e[j1] = mulmod(ed, wi, q);
        }
        ck.track(v[j0]);
        ck.track(v[j1]);
        if (ck.res(v[j0]) != e[j0] || ck.res(v[j1]) != e[j1]) ++ck.bad;
      }
      if (settle_inv(l) && l != log_n - 1)
        for (size_t i = 0; i < n; ++i) {
          v[i] = reduce_f64(v[i], ck.qd, ck.qinv);
          if (std::fabs(v[i]) > 0.5 * ck.qd + 1.0 || ck.res(v[i]) != e[i]) ++ck.bad;
        }
    }
    for (size_t i = 0; i < n; ++i) {
      const double r = canon_f64(reduce_f64(v[i], ck.qd, ck.qinv), ck.qd);
      if (uint64_t(r) != in[i]) ++mismatches;
    }
  }
  std::printf("%s q=%llu log_n=%d cases=%zu max_factor=%.3f max_value=%.3f bad=%ld mismatches=%ld\n",
              sparse ? "ArF64T" : "ArF64", (unsigned long long)q, log_n, cases, ck.max_factor, ck.max_value, ck.bad,
              mismatches);
  if (ck.bad || mismatches || ck.max_factor > lim || ck.max_value > vlim) ++fails;
  }
  if (fails) return 1;
  std::printf("ALL OK\n");
  return 0;
}
