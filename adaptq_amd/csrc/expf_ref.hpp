// expf_ref.hpp -- the single-precision exponential of the reference's host
// libm, for the sparse-V selection.
//
// The reference's softmax uses expf (attention.cpp:422-426); on its x86
// hosts that is glibc 2.35's expf (sysdeps/ieee754/flt-32/e_expf.c, the
// algorithm of Arm's optimized-routines, which states a bound of 0.502 ulp:
// it is not correctly rounded everywhere).  Which tokens the sparse-V cut
// keeps depends on the exact probabilities, so the selection needs the same
// bits, not merely an accurate exponential: a correctly rounded exponential
// differs from glibc's on about 0.06 % of the inputs in [-20, 0].
//
// The published algorithm, restated in double precision:
//   z  = x * 32/ln 2;  k = round(z) (by adding 1.5 * 2^52);  r = z - k
//   2^(k/32) = 2^(k div 32) * T[k mod 32]  (T held as bits minus i << 47, so
//              adding k << 47 to the bits places the exponent)
//   exp(x)  ~= 2^(k/32) * (C0 r^3 + C1 r^2 + C2 r + 1)   (r in [-1/2, 1/2])
// with the polynomial coefficients of the published implementation scaled
// by 1/32 per power of r; special cases: NaN -> NaN, x > 88.72 -> inf,
// x < -103.97 (and -inf) -> 0.  glibc's x86-64 build selects, on hosts with
// FMA (the reference's AVX2+FMA hosts), a copy compiled with FMA contraction:
// its multiply-adds are fused, and the fused r = fma(32/ln 2, x, -k) decides
// a few results (2 of the 2.24e9 floats in [-104, 89] differ from the
// unfused form), so every multiply-add here is an explicit fma.  Plain C++
// for host and device (AQ_HD): the host build equals libm's expf on every
// float in [-104, 89] and the special values (tests/cpp/expf_check.cpp).
#pragma once

#include <stdint.h>

#include "codebook.hpp"

namespace aq {

namespace expf_detail {

// bits(2^(i/32)) - (i << 47), i = 0..31 (2^(i/32) rounded to double)
constexpr uint64_t kTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

constexpr double kN = 32.0;
constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN;
constexpr double kShift = 0x1.8p+52;
constexpr double kC0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;

AQ_HD inline uint64_t dbits(double d) {
  uint64_t u;
  __builtin_memcpy(&u, &d, 8);
  return u;
}

AQ_HD inline double dfrom(uint64_t u) {
  double d;
  __builtin_memcpy(&d, &u, 8);
  return d;
}

}  // namespace expf_detail

AQ_HD inline float expf_ref(float x) {
  using namespace expf_detail;
  if (x != x) return x + x;
  if (x > 0x1.62e42ep6f) return __builtin_inff();
  if (x < -0x1.9fe368p6f) return 0.0f;  // also -inf
  const double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = dbits(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const double s = dfrom(kTab[ki & 31u] + (ki << 47));
  const double p = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(p, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace aq
