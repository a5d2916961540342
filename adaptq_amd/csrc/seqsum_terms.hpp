// seqsum_terms.hpp -- the per-term arithmetic of chain_sum_block (seqsum.hpp):
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
constexpr int kNoClass = -100000;    // a segment without clean terms
constexpr int kBlock = 1024;         // threads of the calling block
constexpr int kWaves = kBlock / 64;
constexpr int kMaxT = 8;             // terms per thread and chunk at most

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

}  // namespace seqsum_detail

}  // namespace aq
