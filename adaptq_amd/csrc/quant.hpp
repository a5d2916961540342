// quant.hpp -- codebook index of one rotated, clipped value (A6).
//
// quantize<B>: the reference's branchless binary search (codebook.cpp:119-144):
// the count of thresholds t with v >= t, NaN -> the lower centre code.
// quantize4_tab: the same function for 4-bit codes from one table lookup.
// The thresholds are symmetric (thr(14-k) = -thr(k) exactly) and the centre
// one is 0, so for v >= 0 (including -0.0, as v >= 0 holds for it) the index
// is 8 + #{positive t : |v| >= t} and for v < 0 it is 7 - #{positive t : |v| > t}.
// Both conditions are one unsigned compare on key = bits(|v|) + [v >= 0]
// against bits(t) (positive floats order like their bit patterns).  The table
// has one entry per bucket of bits(|v|) >> 18 (exponent and 5 mantissa bits)
// over [2^-4, 4], where each bucket holds at most one positive threshold:
// n = thresholds below the bucket, t = the one inside it (or none).  Values
// below 2^-4 or from 4 up use the end buckets, which hold no threshold.
// Equality with quantize<4> over every float is checked on the host
// (tests/cpp/quant_exhaustive.cpp).
#pragma once

#include "codebook.hpp"

namespace aq {

AQ_HD inline uint32_t f32_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}

template <int B>
AQ_HD inline uint32_t quantize(float v) {
  if (v != v) return B == 2 ? 1u : B == 3 ? 3u : 7u;
  if constexpr (B == 2) {
    bool c1 = v >= thr<2>(1);
    bool c0 = v >= (c1 ? thr<2>(2) : thr<2>(0));
    return (c1 ? 2u : 0u) | (c0 ? 1u : 0u);
  } else if constexpr (B == 3) {
    bool c2 = v >= thr<3>(3);
    bool c1 = v >= (c2 ? thr<3>(5) : thr<3>(1));
    float t0 = c2 ? (c1 ? thr<3>(6) : thr<3>(4)) : (c1 ? thr<3>(2) : thr<3>(0));
    bool c0 = v >= t0;
    return (c2 ? 4u : 0u) | (c1 ? 2u : 0u) | (c0 ? 1u : 0u);
  } else {
    bool c3 = v >= thr<4>(7);
    bool c2 = v >= (c3 ? thr<4>(11) : thr<4>(3));
    float t1 = c3 ? (c2 ? thr<4>(13) : thr<4>(9)) : (c2 ? thr<4>(5) : thr<4>(1));
    bool c1 = v >= t1;
    float t0 = c3 ? (c2 ? (c1 ? thr<4>(14) : thr<4>(12)) : (c1 ? thr<4>(10) : thr<4>(8)))
                  : (c2 ? (c1 ? thr<4>(6) : thr<4>(4)) : (c1 ? thr<4>(2) : thr<4>(0)));
    bool c0 = v >= t0;
    return (c3 ? 8u : 0u) | (c2 ? 4u : 0u) | (c1 ? 2u : 0u) | (c0 ? 1u : 0u);
  }
}

struct Q4Entry {
  uint32_t t;  // bits of the positive threshold inside the bucket, or ~0
  uint32_t n;  // positive thresholds below the bucket
};

constexpr int kQ4Lo = 3936;  // bits(2^-4) >> 18
constexpr int kQ4Hi = 4128;  // bits(4.0f) >> 18
constexpr int kQ4Entries = kQ4Hi - kQ4Lo + 1;

AQ_HD inline Q4Entry q4_entry(int i) {
  const uint32_t lo = (uint32_t)(kQ4Lo + i) << 18, hi = lo + (1u << 18);
  Q4Entry e{~0u, 0u};
  for (int k = 8; k < 15; ++k) {
    const uint32_t t = f32_bits(thr<4>(k));
    if (t < lo) ++e.n;
    else if (t < hi && i < kQ4Entries - 1) e.t = t;
  }
  return e;
}

AQ_HD inline uint32_t quantize4_tab(float v, const Q4Entry *tab) {
  const uint32_t ab = f32_bits(v) & 0x7FFFFFFFu;
  const bool nonneg = !(v < 0.0f);
  const uint32_t key = ab + (nonneg ? 1u : 0u);
  uint32_t b = ab >> 18;
  b = b < (uint32_t)kQ4Lo ? (uint32_t)kQ4Lo : b > (uint32_t)kQ4Hi ? (uint32_t)kQ4Hi : b;
  const Q4Entry e = tab[b - kQ4Lo];
  const uint32_t m = e.n + (key > e.t ? 1u : 0u);
  const uint32_t idx = nonneg ? 8u + m : 7u - m;
  return v != v ? 7u : idx;
}

}  // namespace aq
