// seqsum_terms.hpp -- the per-term arithmetic of block_seq_sum (seqsum.hpp):
// binade prediction, rounded integer increments and stop thresholds.  Plain
// C++ with no HIP dependency, so the host test (tests/cpp/seqsum_check.cpp)
// runs the same functions the kernels do.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define AQ_SEQ_HD __host__ __device__ __forceinline__
#else
#define AQ_SEQ_HD inline
#endif

namespace aq {

namespace seqsum_detail {

constexpr uint32_t kTop = 1u << 24;  // K at the top of a binade
constexpr int kUnc = 1000;           // class of a term added by the hardware
constexpr int kNoClass = -100000;    // before the first term: no class
constexpr int kMaxSeg = 512;         // segments per chunk (more: the chunk runs term by term)
constexpr int kBlock = 1024;         // threads of the calling block
constexpr int kSerialMax = 256;      // terms up to which one lane runs the chain
constexpr int kWaves = kBlock / 64;
constexpr int kMaxT = 8;             // terms per thread and chunk at most

// Class of term j of a chunk (P: fp64 sum of s at the chunk start and the
// terms before it): the grid exponent eu = B - 23 of the binade [2^B,
// 2^(B+1)) that s lies in when the term is added, if the interval around the
// prediction and the addition with its rounding stay inside that binade;
// else kUnc.
AQ_SEQ_HD int term_class(double P, float x, int j) {
  const double sum = P + (double)x;
  const double del = (double)(j + 1) * 0x1.08p-24 * sum + 0x1p-140;
  const double lo = P - del, hi = P + del;
  if (!(lo >= 0x1p-100)) return kUnc;
  int64_t lob;
  __builtin_memcpy(&lob, &lo, sizeof lob);
  const int B = (int)((lob >> 52) & 0x7FF) - 1023;  // lo in [2^B, 2^(B+1))
  if (!(hi + (double)x + __builtin_ldexp(1.0, B - 21) < __builtin_ldexp(1.0, B + 1))) return kUnc;
  return B - 23;
}

// r = x / 2^eu rounded to the nearest integer, for a term of class eu; false
// for a tie (x / 2^eu exactly halfway) or a term too large for the binade.
AQ_SEQ_HD bool term_incr(float x, int eu, uint32_t &r) {
  uint32_t b;
  __builtin_memcpy(&b, &x, sizeof b);
  b &= 0x7FFFFFFFu;  // -0 -> +0
  const uint32_t exb = b >> 23;
  const uint32_t M = (b & 0x7FFFFFu) | (exb ? 0x800000u : 0u);
  r = 0u;
  if (M == 0u) return true;
  const int d = (exb ? (int)exb - 150 : -149) - eu;
  if (d >= 0) {
    if (d >= 7) return false;
    r = M << d;
    return true;
  }
  const int sh = -d;
  if (sh > 25) return true;  // below half an ulp: adds nothing
  const uint32_t frac = M & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (frac == half) return false;
  r = (M >> sh) + (frac > half ? 1u : 0u);
  return true;
}

// the least K with K 2^eu >= stop (2^31: never)
AQ_SEQ_HD uint32_t kstop_of(float stop, int eu) {
  if (!(stop > 0.0f)) return 0u;
  if (stop == __builtin_inff()) return 1u << 31;
  uint32_t b;
  __builtin_memcpy(&b, &stop, sizeof b);
  const uint32_t exb = b >> 23;
  const uint32_t M = (b & 0x7FFFFFu) | (exb ? 0x800000u : 0u);
  const int k = (exb ? (int)exb - 150 : -149) - eu;
  if (k >= 0) return k >= 7 ? 1u << 31 : M << k;
  if (k < -30) return 1u;
  return (M + (1u << -k) - 1u) >> -k;
}

// The error bound of a thread's run of terms (P: the fp64 prefix before its
// first term, loc: the fp64 sum of its terms, jend: the index within the
// chunk past its last term): the largest of its terms' bounds in term_class.
AQ_SEQ_HD double range_del(double P, double loc, int jend) {
  return (double)jend * 0x1.08p-24 * (P + loc) + 0x1p-140;
}

AQ_SEQ_HD int exponent_of(double v) {  // v > 0 normal: v in [2^e, 2^(e+1))
  int64_t b;
  __builtin_memcpy(&b, &v, sizeof b);
  return (int)((b >> 52) & 0x7FF) - 1023;
}

// One class for the whole run: when [P - del, P + loc + del], with room for
// the last addition's rounding, sits inside one binade, every term's own
// interval (term_class) lies inside it, and all the run's terms have that
// class; else kUnc.
AQ_SEQ_HD int range_class(double P, double loc, int jend) {
  const double del = range_del(P, loc, jend);
  const double lo = P - del, hi = P + loc + del;
  if (!(lo >= 0x1p-100)) return kUnc;
  const int B = exponent_of(lo);
  if (!(hi + __builtin_ldexp(1.0, B - 21) < __builtin_ldexp(1.0, B + 1))) return kUnc;
  return B - 23;
}

// When the run's range crosses exactly one binade edge: its exponent E (the
// range lies in [2^(E-1), 2^(E+1) - 2^(E-21))); else kUnc.
AQ_SEQ_HD int edge_of(double P, double loc, int jend) {
  const double del = range_del(P, loc, jend);
  const double lo = P - del, hi = P + loc + del;
  if (!(lo >= 0x1p-100)) return kUnc;
  const int B = exponent_of(lo);
  if (!(hi + __builtin_ldexp(1.0, B - 20) < __builtin_ldexp(1.0, B + 2))) return kUnc;
  return B + 1;
}

// Class of one term of such a run (P: the fp64 prefix before the term, del:
// the run's bound): below the edge if s and the addition stay under 2^E with
// room for its rounding, above it if s starts at or over 2^E; else kUnc.
// The run's range bounds the other side of each binade.
AQ_SEQ_HD int split_class(double P, double x, double del, int E) {
  const double lo = P - del, hi = P + x + del;
  if (hi + __builtin_ldexp(1.0, E - 22) < __builtin_ldexp(1.0, E)) return E - 1 - 23;
  if (lo >= __builtin_ldexp(1.0, E)) return E - 23;
  return kUnc;
}

// Class of a thread's run of terms predicted from fp32 sums (P: s before the
// run, within about 2^-19 P of the exact value when it comes from a scan of
// at most 2^15 fp32 partial sums; loc: the run's own sum; jend: the terms
// since the sum's start at the run's end): the grid exponent eu = B - 23
// when [P - del, P + loc + del] with del = (jend + 64) 2^-22 (P + loc) lies
// in the binade [2^B, 2^(B+1)) with room for the last rounding, else kUnc.
// del is four times the chain's own drift bound plus the prefix error; a
// prediction only chooses the path (the walk checks every class it uses).
AQ_SEQ_HD int run_class_f32(float P, float loc, int jend) {
  const float top = P + loc;
  const float del = (float)(jend + 64) * 0x1p-22f * top;
  const float lo = P - del, hi = top + del;
  if (!(lo >= 0x1p-100f) || !(hi < 0x1p127f)) return kUnc;
  uint32_t b;
  __builtin_memcpy(&b, &lo, sizeof b);
  const int B = (int)(b >> 23) - 127;  // lo in [2^B, 2^(B+1))
  if (!(hi < __builtin_ldexpf(1.0f, B + 1) - __builtin_ldexpf(1.0f, B - 20))) return kUnc;
  return B - 23;
}

// term_incr for a term known to fit its class: x / 2^eu is exact in fp32
// (below 2^24), so the increment is its nearest integer; false for a tie.
AQ_SEQ_HD bool scaled_incr(float x, int eu, uint32_t &r) {
  const float y = __builtin_ldexpf(x, -eu);
  const bool tie = y - __builtin_floorf(y) == 0.5f;
  r = tie ? 0u : (uint32_t)__builtin_rintf(y);
  return !tie;
}

}  // namespace seqsum_detail

}  // namespace aq
