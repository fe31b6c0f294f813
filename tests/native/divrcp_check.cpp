// Host check of hi2_amd/csrc/divrcp.h (compiled by tests/test_divrcp.py with g++ -mfma
// -ffp-contract=off, the same fma and rounding semantics as the gfx950 kernels):
//   div_rcp(a, b, 1/b)      == a / b bit for bit,
//   div_rcp_fast(a, b, 1/b) == a / b wherever div_rcp_ok(a, a / b's estimate) accepts,
//   div_rcp_code(a, b, 1/b) rounds and clamps to the same code as a / b (b normal),
//   div_code(a, b, 1/b)     the same for every finite nonzero b (subnormal b included),
// over random operand pairs of every exponent and the operands the fast iteration alone
// gets wrong (subnormal and zero numerators, subnormal quotients, overflow, inf, NaN).
// Prints one line per family and exits nonzero on the first family with a mismatch.
#define HI2X_HD
#include "../../hi2_amd/csrc/divrcp.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

static uint32_t bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
static float from_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
static bool same(float x, float y) { return bits(x) == bits(y) || (x != x && y != y); }
static float clamp_code(float q, float nm) {  // torch.clamp(q, 0, nm): NaN propagates
  q = (q < 0.0f) ? 0.0f : q;
  q = (q > nm) ? nm : q;
  return q;
}
static bool same_code(float q, float r, float nm) {
  const float a = clamp_code(std::nearbyint(q), nm), b = clamp_code(std::nearbyint(r), nm);
  return a == b || (a != a && b != b);
}

struct Family {
  const char* name;
  long n = 0, bad = 0, bad_code = 0, bad_ok = 0, bad_any = 0;
  float ea = 0, eb = 0;
};

static void check(Family& f, float a, float b) {
  if (b == 0.0f) return;  // callers divide by a nonzero step or factor diagonal
  const float y = 1.0f / b, q = a / b;
  ++f.n;
  if (!same(div_rcp(a, b, y), q)) {
    if (!f.bad) f.ea = a, f.eb = b;
    ++f.bad;
  }
  // where div_rcp_ok accepts the operands, the bare iteration is the IEEE quotient
  if (div_rcp_ok(a, a * y) && !same(div_rcp_fast(a, b, y), q)) {
    if (!f.bad && !f.bad_ok) f.ea = a, f.eb = b;
    ++f.bad_ok;
  }
  // div_code: any finite divisor (the ladder fit's candidate steps can be subnormal)
  if (std::isfinite(b))
    for (float nm : {3.0f, 15.0f, 255.0f})
      if (!same_code(div_code(a, b, y), q, nm)) {
        if (!f.bad && !f.bad_any) f.ea = a, f.eb = b;
        ++f.bad_any;
        break;
      }
  // div_rcp_code's divisors are normal and finite (div_code_ok), else div_code branches
  const float ab = std::fabs(b);
  if (div_code_ok(b) != (ab >= 0x1p-126f && ab <= 0x1.fffffep127f)) {
    ++f.bad_any;
    return;
  }
  if (!div_code_ok(b)) return;
  for (float nm : {3.0f, 15.0f, 255.0f})
    if (!same_code(div_rcp_code(a, b, y), q, nm)) {
      if (!f.bad && !f.bad_code) f.ea = a, f.eb = b;
      ++f.bad_code;
      break;
    }
}

int main() {
  std::mt19937_64 g(12345);
  auto rnd_float = [&](uint32_t e_lo, uint32_t e_hi) {
    const uint32_t e = e_lo + (uint32_t)(g() % (e_hi - e_lo + 1));
    float v = from_bits((e << 23) | (uint32_t)(g() & 0x7fffff));
    return (g() & 1) ? -v : v;
  };
  Family fam[7] = {{"random pairs, every exponent"}, {"subnormal numerators"},
                   {"subnormal / tiny quotients"}, {"zero numerators"},
                   {"overflowing quotients"}, {"inf / nan operands"},
                   {"subnormal divisors (fit steps)"}};
  for (long i = 0; i < 4000000; ++i) check(fam[0], rnd_float(0, 254), rnd_float(0, 254));
  for (long i = 0; i < 2000000; ++i) check(fam[1], rnd_float(0, 0), rnd_float(1, 254));
  for (long i = 0; i < 2000000; ++i) {
    const float b = rnd_float(100, 254);
    check(fam[2], rnd_float(1, 60), b);
  }
  for (long i = 0; i < 100000; ++i) {
    const float b = rnd_float(0, 254);
    check(fam[3], 0.0f, b);
    check(fam[3], -0.0f, b);
  }
  for (long i = 0; i < 1000000; ++i) check(fam[4], rnd_float(180, 254), rnd_float(0, 80));
  const float inf = INFINITY, nan = NAN;
  for (long i = 0; i < 100000; ++i) {
    const float v = rnd_float(0, 254);
    check(fam[5], inf, v);
    check(fam[5], -inf, v);
    check(fam[5], nan, v);
    check(fam[5], v, inf);
  }
  // the ladder fit over a block whose span is tiny: numerators x - lo of the span's
  // size and below, steps span / nm subnormal
  for (long i = 0; i < 2000000; ++i) {
    const float b = rnd_float(0, 0);
    check(fam[6], rnd_float(0, 8), b);
    check(fam[6], rnd_float(0, 254), b);
  }
  int rc = 0;
  for (const Family& f : fam) {
    std::printf("%-32s %9ld pairs  div_rcp mismatches %ld  accepted fast mismatches %ld  code "
                "mismatches %ld  any-divisor code mismatches %ld", f.name, f.n, f.bad, f.bad_ok,
                f.bad_code, f.bad_any);
    if (f.bad || f.bad_code || f.bad_ok || f.bad_any) {
      std::printf("  (first: a=%a b=%a)", f.ea, f.eb);
      rc = 1;
    }
    std::printf("\n");
  }
  return rc;
}
