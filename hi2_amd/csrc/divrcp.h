// Correctly rounded fp32 division through a precomputed reciprocal.  Shared by the gfx950
// kernels and, for its exhaustive check against IEEE division, the host compiler
// (HI2X_HD defined empty).
#pragma once

#ifndef HI2X_HD
#define HI2X_HD __host__ __device__
#endif

// Markstein's iteration for a / b given y = a correctly rounded 1 / b: q0 = a y is
// within 2 ulp of a / b, the first fma correction makes it faithful and the second,
// from a faithful quotient, the correctly rounded one (the remainders a - b q are exact
// in an fma).  Five dependent operations instead of the ten of the scaled IEEE division
// sequence.  Exact only for operands that keep every intermediate normal: use div_rcp
// or div_rcp_code, which add the range test.
HI2X_HD inline float div_rcp_fast(float a, float b, float y) {
  const float q0 = a * y;
  const float r0 = __builtin_fmaf(-b, q0, a);
  const float q1 = __builtin_fmaf(r0, y, q0);
  const float r1 = __builtin_fmaf(-b, q1, a);
  return __builtin_fmaf(r1, y, q1);
}

// Whether div_rcp_fast(a, b, y) is a / b correctly rounded, given q0 = a y: |a| and |q0|
// in [2^-100, 2^100] (no subnormal numerator, quotient or remainder and no overflow), or
// a = +0 with a finite reciprocal (the iteration then yields the quotient's signed
// zero; -0 is left to the IEEE division).  Checked on 10^8 random operand pairs of every exponent.
HI2X_HD inline bool div_rcp_ok(float a, float q0) {
  const float aa = __builtin_fabsf(a), aq = __builtin_fabsf(q0);
  return (aa >= 0x1p-100f && aq >= 0x1p-100f && aq <= 0x1p100f) ||
         (__builtin_bit_cast(unsigned, a) == 0u && q0 == 0.0f);
}

// a / b correctly rounded (bit-identical to IEEE division) for every a and every b with
// y = 1 / b: the iteration where |a| and |a y| lie in [2^-100, 2^100] (no subnormal
// numerator, quotient or remainder and no overflow; checked on 10^8 random operand pairs
// of every exponent), a * b for a = +-0 (the quotient's signed zero when b is finite and
// nonzero), the IEEE division otherwise (subnormal or tiny numerators and quotients,
// infinities, NaN).  The iteration and the range test always run; the other two paths
// are a branch taken only by lanes outside the range.  With exact = false the lane
// keeps the iteration's value whatever the range (lanes whose result is discarded).
HI2X_HD inline float div_rcp(float a, float b, float y, bool exact = true) {
  const float q0 = a * y;
  const float r0 = __builtin_fmaf(-b, q0, a);
  const float q1 = __builtin_fmaf(r0, y, q0);
  const float r1 = __builtin_fmaf(-b, q1, a);
  float q = __builtin_fmaf(r1, y, q1);
  const float aa = __builtin_fabsf(a), aq = __builtin_fabsf(q0);
  const bool in_range = aa >= 0x1p-100f && aq >= 0x1p-100f && aq <= 0x1p100f;
  if (__builtin_expect(exact && !in_range, 0)) {
    const float ab = __builtin_fabsf(b);
    q = (aa == 0.0f && ab > 0.0f && ab <= 0x1.fffffep127f) ? a * b : a / b;
  }
  return q;
}

// a / b for a quotient that is only ever rounded to an integer code and clamped to
// [0, nm] (clamp_code(rint(.))): the same code as the IEEE quotient for every a and every
// normal finite b (y = 1 / b; the callers' divisors are ladder steps, 1 for a zero step,
// and factor diagonals), without a branch.  Where |a y| <= 2^100 the
// iteration is used: it is exact when |a| and |a y| are >= 2^-100, and otherwise both it
// and the IEEE quotient are below 2^-99 in magnitude, which rint takes to a zero and
// clamp to code 0 (the sign of that zero never reaches a stored value: lo + (+-0) step
// and the squared differences are the same).  Above 2^100, q0 = a y itself, within 2 ulp
// of the quotient or infinite with its sign, clamps to the same end of the ladder as the
// quotient (the iteration could turn an overflowed q0 into NaN).
HI2X_HD inline float div_rcp_code(float a, float b, float y) {
  const float q0 = a * y;
  const float r0 = __builtin_fmaf(-b, q0, a);
  const float q1 = __builtin_fmaf(r0, y, q0);
  const float r1 = __builtin_fmaf(-b, q1, a);
  const float q = __builtin_fmaf(r1, y, q1);
  return (__builtin_fabsf(q0) <= 0x1p100f) ? q : q0;
}

// Whether div_rcp_code(., b, 1 / b) gives the IEEE quotient's code: b normal and finite.
// A subnormal b (a ladder fit's candidate step over a block whose span is below about
// 2^-120) has a reciprocal that overflows or is too large for the iteration's remainders.
HI2X_HD inline bool div_code_ok(float b) {
  const float ab = __builtin_fabsf(b);
  return ab >= 0x1p-126f && ab <= 0x1.fffffep127f;
}

// div_rcp_code for every finite nonzero b: the IEEE quotient where b is subnormal (a
// branch taken only by such lanes).
HI2X_HD inline float div_code(float a, float b, float y) {
  if (__builtin_expect(!div_code_ok(b), 0)) return a / b;
  return div_rcp_code(a, b, y);
}
