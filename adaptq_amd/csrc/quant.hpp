// quant.hpp -- codebook index of one rotated, clipped value (A6).
//
// quantize<B>: the reference's branchless binary search (codebook.cpp:119-144):
// the count of thresholds t with v >= t, NaN -> the lower centre code.
// quantize_g4: the same function for 4-bit codes from one lookup in a grid
// of quarter-unit cells: cell g = floor(4 v) covers [g/4, (g+1)/4).  The 15
// thresholds are at least 0.2527 apart, so a cell holds at most one of them:
// the code is n + [v >= t], n = thresholds below the cell, t = the one inside
// it (NaN for none, so the compare fails).  Cells below -10 and from 9 up hold
// none and are clamped to those end cells.  The compare v >= t on v itself
// decides as the binary search does, -0.0 included (cell 0, whose threshold
// is 0).  Equality with quantize<4> over every finite float is checked on the
// host (tests/cpp/quant_exhaustive.cpp).
// quantize_ss2/3: the sign-split forms of the append kernels (below).
// quantize_bd2: 2-bit codes of a value before its scalings by 1/sqrt(p) and
// sqrt(p), against thresholds moved through both roundings (below).
#pragma once

#include <math.h>

#include "codebook.hpp"

namespace aq {

AQ_HD constexpr uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

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

struct Q4Cell {
  float t;     // the threshold inside the cell, or NaN
  uint32_t n;  // thresholds below the cell
};

constexpr int kQ4CellLo = -10;  // cell of [-2.5, -2.25) and everything below
constexpr int kQ4CellHi = 9;    // cell of [2.25, 2.5) and everything above
constexpr int kQ4Cells = kQ4CellHi - kQ4CellLo + 1;

AQ_HD constexpr Q4Cell q4_cell(int i) {
  const int g = kQ4CellLo + i;
  Q4Cell c{__builtin_nanf(""), 0u};
  for (int k = 0; k < 15; ++k) {
    const float t = thr<4>(k);
    if (4.0f * t < (float)g) ++c.n;
    else if (4.0f * t < (float)(g + 1)) c.t = t;
  }
  return c;
}

// every cell, evaluated by the compiler (kernels copy it into LDS)
struct Q4Table {
  Q4Cell c[kQ4Cells];
};
AQ_HD constexpr Q4Table q4_table() {
  Q4Table t{};
  for (int i = 0; i < kQ4Cells; ++i) t.c[i] = q4_cell(i);
  return t;
}

// Table index of v's cell, for non-NaN v: floor(4 v) - kQ4CellLo clamped to
// the table, computed as the truncation of the clamped fma(v, 4, 10), which
// is nonnegative.  The fma rounds (by at most 1e-6 in w, 2.4e-7 in v), so a
// v just below a cell's upper edge can land in the next cell; that changes no
// code: 0, the lower edge of its own cell, is the only threshold within
// 0.0026 of a cell edge, so a value moved across an edge is on the same side
// of every threshold of both cells.  (Checked with quantize_g4 on every
// float.)
AQ_HD inline int q4_cell_index(float v) {
  const float w = fminf(fmaxf(fmaf(v, 4.0f, (float)-kQ4CellLo), 0.0f), (float)(kQ4Cells - 1));
  return (int)w;
}

// non-NaN v (a NaN vector is given its code as a whole by the caller)
AQ_HD inline uint32_t quantize_g4(float v, const Q4Cell *tab) {
  const Q4Cell c = tab[q4_cell_index(v)];
  return c.n + (v >= c.t ? 1u : 0u);
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
// -0.0 belongs to the positive side (-0.0 >= 0 holds): both forms add +0.0
// first (which turns -0.0 into +0.0 and changes nothing else).
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
