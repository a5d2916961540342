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
// quantize_ss2/3/4: the sign-split forms of the append kernels (below).
// quantize_bd2: 2-bit codes of a value before its scalings by 1/sqrt(p) and
// sqrt(p), against thresholds moved through both roundings (below).
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

// Sign-split quantisers of the append kernel, for finite v (a NaN vector is
// given the NaN code by the caller: a NaN in any input element reaches every
// element through the FWHT, so NaN is a property of the whole vector).
//   s   = sign of v as 0 or ~0
//   key = bits(|v|) + [sign bit clear]
//   u   = centre code 2^(B-1) + #{positive thresholds t : key > bits(t)}
//   code = u ^ (s & (2^B - 1))
// For v >= 0, key > bits(t) is v >= t; for v < 0 it is |v| > t, and the
// negative side's count 2^(B-1) - 1 - m equals (2^(B-1) + m) ^ (2^B - 1).
// -0.0 belongs to the positive side (-0.0 >= 0 holds): the 2- and 3-bit forms
// add +0.0 first (which turns -0.0 into +0.0 and changes nothing else); the
// 4-bit form reads the bucket table with n raised by 8 (q4s_entry), whose
// lowest bucket holds a threshold at key 0 over a base count of 7, so key 0
// (only -0.0 has it) gives 7 ^ 15 = 8 and every other key in it gives 8.
// Equality with quantize<B> over every finite float is checked on the host
// (tests/cpp/quant_exhaustive.cpp).
struct SignSplit {
  uint32_t s, ab, key;
};

AQ_HD inline SignSplit sign_split(float c) {
  const uint32_t bits = f32_bits(c);
  SignSplit r;
  r.s = (uint32_t)((int32_t)bits >> 31);
  r.ab = bits & 0x7FFFFFFFu;
  r.key = r.ab + 1u + r.s;
  return r;
}

AQ_HD inline Q4Entry q4s_entry(int i) {
  Q4Entry e = q4_entry(i);
  if (i == 0) return Q4Entry{0u, 7u};  // holds no threshold (checked below)
  e.n += 8u;
  return e;
}

AQ_HD inline uint32_t quantize_ss4(float v, const Q4Entry *tab8) {
  const SignSplit x = sign_split(v);
  uint32_t b = x.ab >> 18;
  b = b < (uint32_t)kQ4Lo ? (uint32_t)kQ4Lo : b > (uint32_t)kQ4Hi ? (uint32_t)kQ4Hi : b;
  const Q4Entry e = tab8[b - kQ4Lo];
  const uint32_t u = e.n + (x.key > e.t ? 1u : 0u);
  return u ^ (x.s & 15u);
}

AQ_HD inline uint32_t quantize_ss3(float v) {
  const SignSplit x = sign_split(v + 0.0f);
  const uint32_t u = 4u + (x.key > f32_bits(thr<3>(4)) ? 1u : 0u) +
                     (x.key > f32_bits(thr<3>(5)) ? 1u : 0u) +
                     (x.key > f32_bits(thr<3>(6)) ? 1u : 0u);
  return u ^ (x.s & 7u);
}

AQ_HD inline uint32_t quantize_ss2(float v) {
  const SignSplit x = sign_split(v + 0.0f);
  const uint32_t u = 2u + (x.key > f32_bits(thr<2>(2)) ? 1u : 0u);
  return u ^ (x.s & 3u);
}

// 2-bit codes from the rotated value before its two scalings.  The reference
// codes v = fl(fl(b * c) * d), c = 1/sqrt(p) and d = sqrt(p) as floats
// (fwht.cpp:60-66, quantizer.cpp:73-75), with quantize<2>: the count of
// thresholds t with v >= t.  Rounding is monotone, so v(b) is nondecreasing
// in b and v >= t holds exactly when b >= alpha_t, the least float b whose v
// reaches t (for t = 0: the most negative b whose v is -0, as -0 >= 0).
// BdThr holds alpha_t of the three 2-bit thresholds, ascending, found by
// bisection over the floats with the same two roundings.  Equality with
// quantize<2>(v(b)) over every float b is checked on the host
// (tests/cpp/quant_exhaustive.cpp).
struct BdThr {
  float q2[3];
};

AQ_HD inline uint32_t quantize_bd2(float v, float q0, float q1, float q2) {
  return (v >= q0 ? 1u : 0u) + (v >= q1 ? 1u : 0u) + (v >= q2 ? 1u : 0u);
}

// Host: the thresholds for c = 1/sqrt(p), d = sqrt(p) as the launch passes them.
namespace bd_detail {
inline float key_float(long long k) {
  const uint32_t u = k >= 0 ? (uint32_t)k : 0x80000000u | (uint32_t)(-k);
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}
inline float scaled(float b, float c, float d) {
  volatile float y = b * c;  // two roundings, as the reference
  volatile float v = y * d;
  return v;
}
// least ordered key (k >= 0: bits k; k < 0: -|bits|) whose float f has
// v(f) >= t; true at +inf since c, d > 0
inline long long least(float t, float c, float d) {
  long long lo = -0x7F800000LL, hi = 0x7F800000LL;
  while (lo < hi) {
    const long long m = lo + (hi - lo) / 2;
    if (scaled(key_float(m), c, d) >= t) hi = m;
    else lo = m + 1;
  }
  return lo;
}
}  // namespace bd_detail

inline BdThr bd_thresholds(float c, float d) {
  BdThr b{};
  for (int j = 0; j < 3; ++j) b.q2[j] = bd_detail::key_float(bd_detail::least(thr<2>(j), c, d));
  return b;
}

}  // namespace aq
