// seqsum.hpp -- a left-to-right fp32 sum of non-negative terms, bit for bit,
// by a whole block in parallel.
//
// The reference's softmax denominator (attention.cpp:422-426) and sparse-V
// mass loop (attention.cpp:454-472) are chains s = fl(s + x_i) whose exact
// bits decide which tokens sparse-V keeps.  One lane runs such a chain at
// about 4 ns a term; this computes the same bits with every thread of the
// block.
//
// While s stays in one binade [2^E, 2^(E+1)), every representable s is K u
// with u = 2^(E-23) and K an integer in [2^23, 2^24), and fl(s + x) = (K + r) u
// where r is x / u rounded to the nearest integer -- independent of s, except
// when x / u lies exactly halfway (a tie): then the sum rounds to the even one
// of K + m and K + m + 1 (m = floor(x / u)), which depends on the parity of K
// and leaves K even.  A run of terms added inside one binade is therefore an
// integer increment that depends only on the parity K starts with: a pair of
// increments and a pair of output parities, which compose associatively.
//
// The block takes 1024 T terms at a time:
//   1. an fp64 prefix sum P_i predicts the binade of s before each term (the
//      fp32 chain is within (i + 1) 2^-24 P of it); a term whose prediction is
//      not clear of a binade edge, or whose addition may leave the binade, is
//      marked to be added by the hardware;
//   2. consecutive clear terms of one binade form segments; a segmented scan
//      of the terms' parity functions gives every segment's increment pair;
//   3. one lane walks the segments with the exact s: a marked term is one
//      fp32 add; a segment checks that s lies in its binade, adds its
//      increment for s's parity, and checks that K stays below 2^24 -- if a
//      check fails (a prediction was wrong), the chunk is redone term by term
//      on one lane, so the result is the chain's in every case;
//   4. the stop test of the mass loop (stop before adding term i once s >=
//      stop) is K >= ceil(stop / u) inside a segment; the block finds the
//      first such term of the segment the walk stops in.
// Terms must be finite and not negative (-0 is fine).  Checked against the
// one-lane chain through the sparse-V weights, which the GPU tests compare
// with the oracle's bit for bit, and, for the integer model itself, against
// sequential fp32 sums of random, tie-heavy, subnormal and
// stop-at-a-reached-value sequences.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aq {

namespace seqsum_detail {

constexpr uint32_t kSat = 1u << 30;  // saturation of the integer sums (above any binade)
constexpr uint32_t kTop = 1u << 24;  // K at the top of a binade
constexpr int kUnc = 1000;           // class of a term added by the hardware
constexpr int kMaxSeg = 512;         // segments per chunk (more: the chunk runs term by term)
constexpr int kBlock = 1024;         // threads of the calling block
constexpr int kSerialMax = 256;      // terms up to which one lane runs the chain
constexpr int kWaves = kBlock / 64;

__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) {
  const uint32_t s = a + b;  // a, b <= 2^30: no wrap
  return s > kSat ? kSat : s;
}

// s >= 0 finite: s = K 2^eu on the grid of s's binade
__device__ __forceinline__ void band_of(float s, int &eu, uint32_t &K) {
  const uint32_t b = __float_as_uint(s) & 0x7FFFFFFFu;
  const uint32_t exb = b >> 23;
  eu = (int)(exb > 1u ? exb : 1u) - 150;
  K = (b & 0x7FFFFFu) | (exb ? 0x800000u : 0u);
}

// the least K with K 2^eu >= stop (2 kSat: never)
__device__ __forceinline__ uint32_t kstop_of(float stop, int eu) {
  if (!(stop > 0.0f)) return 0u;
  if (stop == __builtin_inff()) return 2u * kSat;
  const uint32_t b = __float_as_uint(stop);
  const uint32_t exb = b >> 23;
  const uint32_t M = (b & 0x7FFFFFu) | (exb ? 0x800000u : 0u);
  const int k = (exb ? (int)exb - 150 : -149) - eu;
  if (k >= 0) return k >= 7 ? 2u * kSat : M << k;
  if (k < -30) return 1u;
  return (M + (1u << -k) - 1u) >> -k;
}

// c ? a : b for c in {0, 1}, as arithmetic (a select between two members of
// a struct can otherwise become an indexed load from a stack copy)
__device__ __forceinline__ uint32_t pick(uint32_t c, uint32_t a, uint32_t b) {
  return b ^ ((a ^ b) & (0u - c));
}

// Parity function of a run of additions: increments i0 / i1 for K even / odd
// at the start, out parities in par bit 0 / bit 1.
struct Fn {
  uint32_t i0, i1, par;
};
__device__ __forceinline__ Fn fn_id() { return Fn{0u, 0u, 2u}; }
// F, then G
__device__ __forceinline__ Fn fn_then(const Fn &F, const Fn &G) {
  const uint32_t f0 = F.par & 1u, f1 = (F.par >> 1) & 1u;
  return Fn{sat_add(F.i0, pick(f0, G.i1, G.i0)), sat_add(F.i1, pick(f1, G.i1, G.i0)),
            ((G.par >> f0) & 1u) | (((G.par >> f1) & 1u) << 1)};
}
// one addition of x on the grid 2^eu (x finite, not negative; no crossing)
__device__ __forceinline__ Fn fn_term(float x, int eu) {
  const uint32_t b = __float_as_uint(x) & 0x7FFFFFFFu;  // -0 -> +0
  const uint32_t exb = b >> 23;
  const uint32_t M = (b & 0x7FFFFFu) | (exb ? 0x800000u : 0u);
  const int d = (exb ? (int)exb - 150 : -149) - eu;
  uint32_t st = 0u;
  if (M != 0u) {
    if (d >= 0) {
      st = d >= 7 ? kSat : M << d;
    } else if (-d <= 25) {
      const int sh = -d;
      const uint32_t m = M >> sh, frac = M & ((1u << sh) - 1u), half = 1u << (sh - 1);
      if (frac == half) return Fn{m + (m & 1u), m + ((m + 1u) & 1u), 0u};  // to even
      st = m + (frac > half ? 1u : 0u);
    }
  }
  return Fn{st, st, (st & 1u) ? 1u : 2u};
}
__device__ __forceinline__ uint32_t fn_inc(const Fn &F, uint32_t K) { return pick(K & 1u, F.i1, F.i0); }

// Class of term j of a chunk (P: fp64 sum of s at the chunk start and the
// terms before): the grid exponent eu of the binade s lies in when it is
// added, if that binade is clear and the addition cannot leave it; else kUnc.
__device__ __forceinline__ int term_class(double P, float x, int j) {
  const double sum = P + (double)x;
  const double del = (double)(j + 1) * 0x1.08p-24 * sum + 0x1p-140;
  const double lo = P - del, hi = P + del;
  if (!(lo >= 0x1p-100)) return kUnc;
  const int B = (int)((__double_as_longlong(lo) >> 52) & 0x7FF) - 1023;  // lo in [2^B, 2^(B+1))
  if (!(hi + (double)x + __builtin_ldexp(1.0, B - 21) < __builtin_ldexp(1.0, B + 1))) return kUnc;
  return B - 23;
}

}  // namespace seqsum_detail

// Shared memory of block_seq_sum.
struct SeqShared {
  double dsum[seqsum_detail::kWaves];
  uint32_t wflag[seqsum_detail::kWaves], wi0[seqsum_detail::kWaves], wi1[seqsum_detail::kWaves],
      wpar[seqsum_detail::kWaves], wcnt[seqsum_detail::kWaves];
  int last_cls[seqsum_detail::kBlock];
  int seg_start[seqsum_detail::kMaxSeg + 1];
  int seg_cls[seqsum_detail::kMaxSeg];
  uint32_t seg_i0[seqsum_detail::kMaxSeg], seg_i1[seqsum_detail::kMaxSeg];
  float seg_x[seqsum_detail::kMaxSeg];  // the term of a one-term (hardware) segment
  int nseg, stop_at, stop_seg, redo;
  uint32_t stop_K;
  float s;
};

// s = fl(s + load(i)) for i = 0, 1, ... while i < n and s < stop (tested
// before each addition), as one lane would run it.  Returns how many terms
// were added and the sum after them (the same in every thread).  Called by all
// kBlock threads with uniform arguments; load(i) for 0 <= i < n returns term
// i (finite, not negative).
struct SeqResult {
  int count;  // terms added
  float s;    // the sum after them
};

template <int T, class Load>
__device__ __forceinline__ SeqResult block_seq_sum(Load load, int n, float s, float stop,
                                                   SeqShared &sh) {
  using namespace seqsum_detail;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (n <= kSerialMax) {
    // short: the chain itself
    if (tid == 0) {
      int i = 0;
      for (; i < n && s < stop; ++i) s = __fadd_rn(s, load(i));
      sh.stop_at = i;
      sh.s = s;
    }
    __syncthreads();
    const SeqResult r{sh.stop_at, sh.s};
    __syncthreads();
    return r;
  }
  for (int c0 = 0;; c0 += kBlock * T) {
    if (!(s < stop) || c0 >= n) return SeqResult{c0 < n ? c0 : n, s};
    const int cn = n - c0 < kBlock * T ? n - c0 : kBlock * T;  // terms of this chunk
    const int j0 = tid * T;                                     // first term of this thread
    float x[T];
#pragma unroll
    for (int k = 0; k < T; ++k) x[k] = j0 + k < cn ? load(c0 + j0 + k) : 0.0f;

    // ---- 1. fp64 prefix: P before the thread's first term ----
    double loc = 0.0;
#pragma unroll
    for (int k = 0; k < T; ++k) loc += (double)x[k];
    double incl = loc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double y = __shfl_up(incl, off, 64);
      if (lane >= off) incl += y;
    }
    if (lane == 63) sh.dsum[wave] = incl;
    __syncthreads();
    double P = (double)s + (incl - loc);
    for (int w = 0; w < wave; ++w) P += sh.dsum[w];

    // ---- 2. classes and heads ----
    int cls[T];
#pragma unroll
    for (int k = 0; k < T; ++k) {
      cls[k] = j0 + k < cn ? term_class(P, x[k], j0 + k) : kUnc;
      P += (double)x[k];
    }
    sh.last_cls[tid] = cls[T - 1];
    __syncthreads();
    uint32_t heads = 0u;  // bit k: term k starts a segment
    {
      int pc = tid > 0 ? sh.last_cls[tid - 1] : kUnc;
#pragma unroll
      for (int k = 0; k < T; ++k) {
        if (j0 + k < cn && (cls[k] == kUnc || pc == kUnc || cls[k] != pc)) heads |= 1u << k;
        pc = cls[k];
      }
    }
    // the thread's composition since its last head (all of it if none)
    Fn acc = fn_id();
#pragma unroll
    for (int k = 0; k < T; ++k) {
      const Fn f = (j0 + k < cn && cls[k] != kUnc) ? fn_term(x[k], cls[k]) : fn_id();
      acc = ((heads >> k) & 1u) ? f : fn_then(acc, f);
    }
    // ---- segmented scan over threads of (any head, function since the last
    // head, number of heads) ----
    uint32_t fl = heads ? 1u : 0u, cnt = (uint32_t)__popc(heads);
    Fn F = acc;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t pf = __shfl_up(fl, off, 64), pn = __shfl_up(cnt, off, 64);
      const Fn pF{__shfl_up(F.i0, off, 64), __shfl_up(F.i1, off, 64), __shfl_up(F.par, off, 64)};
      if (lane >= off) {
        if (!fl) F = fn_then(pF, F);
        fl |= pf;
        cnt += pn;
      }
    }
    if (lane == 63) {
      sh.wflag[wave] = fl;
      sh.wi0[wave] = F.i0;
      sh.wi1[wave] = F.i1;
      sh.wpar[wave] = F.par;
      sh.wcnt[wave] = cnt;
    }
    __syncthreads();
    uint32_t ccnt = 0u;  // heads in earlier waves, and their carried composition
    Fn C = fn_id();
    for (int w = 0; w < wave; ++w) {
      const Fn W{sh.wi0[w], sh.wi1[w], sh.wpar[w]};
      C = sh.wflag[w] ? W : fn_then(C, W);
      ccnt += sh.wcnt[w];
    }
    uint32_t efl = __shfl_up(fl, 1, 64), ecnt = __shfl_up(cnt, 1, 64);
    Fn E{__shfl_up(F.i0, 1, 64), __shfl_up(F.i1, 1, 64), __shfl_up(F.par, 1, 64)};
    if (lane == 0) {
      efl = 0u;
      ecnt = 0u;
      E = fn_id();
    }
    const Fn X = efl ? E : fn_then(C, E);  // the current segment's part before this thread
    const uint32_t sid0 = ccnt + ecnt;      // heads before this thread
    if (tid == kBlock - 1) sh.nseg = (int)(ccnt + cnt);

    // ---- segment table: a head writes the closing segment's increments and
    // its own start and class; the chunk's last term closes the last one ----
    {
      Fn a = X;
      uint32_t sid = sid0;
#pragma unroll
      for (int k = 0; k < T; ++k) {
        if (j0 + k < cn) {
          const Fn f = cls[k] != kUnc ? fn_term(x[k], cls[k]) : fn_id();
          if ((heads >> k) & 1u) {
            if (sid >= 1u && sid <= (uint32_t)kMaxSeg) {
              sh.seg_i0[sid - 1] = a.i0;
              sh.seg_i1[sid - 1] = a.i1;
            }
            ++sid;
            if (sid <= (uint32_t)kMaxSeg) {
              sh.seg_start[sid - 1] = c0 + j0 + k;
              sh.seg_cls[sid - 1] = cls[k];
              sh.seg_x[sid - 1] = x[k];
            }
            a = f;
          } else {
            a = fn_then(a, f);
          }
          if (j0 + k == cn - 1 && sid <= (uint32_t)kMaxSeg) {
            sh.seg_i0[sid - 1] = a.i0;
            sh.seg_i1[sid - 1] = a.i1;
          }
        }
      }
    }
    __syncthreads();

    // ---- 3. the walk over the segments with the exact s.  Inside a binade
    // the fp32 sum is the bit pattern plus the integer increment, and s >=
    // stop the float comparison. ----
    if (tid == 0) {
      const int ns = sh.nseg;
      float w = s;
      int stop_at = -1, stop_seg = -1, redo = ns > kMaxSeg ? 1 : 0;
      if (!redo) sh.seg_start[ns] = c0 + cn;
      for (int k = 0; k < ns && !redo; ++k) {
        const int cl = sh.seg_cls[k];
        if (!(w < stop)) {
          stop_at = sh.seg_start[k];
          break;
        }
        if (cl == kUnc) {
          w = __fadd_rn(w, sh.seg_x[k]);
          continue;
        }
        const uint32_t wb = __float_as_uint(w), exb = (uint32_t)(cl + 150);
        const uint32_t inc = pick(wb & 1u, sh.seg_i1[k], sh.seg_i0[k]);
        const uint32_t nb = wb + inc;
        if ((wb >> 23) != exb || inc >= kTop || (nb >> 23) != exb) {
          redo = 1;
          break;
        }
        if (!(__uint_as_float(nb) < stop)) {
          stop_seg = k;
          break;
        }
        w = __uint_as_float(nb);
      }
      if (redo) {
        // a prediction failed: the chunk term by term
        w = s;
        stop_at = -1;
        stop_seg = -1;
        for (int i = c0; i < c0 + cn; ++i) {
          if (!(w < stop)) {
            stop_at = i;
            break;
          }
          w = __fadd_rn(w, load(i));
        }
      }
      sh.stop_at = stop_at;
      sh.stop_seg = stop_seg;
      sh.stop_K = (__float_as_uint(w) & 0x7FFFFFu) | 0x800000u;
      sh.s = w;
    }
    __syncthreads();
    const int stop_seg = sh.stop_seg;
    if (stop_seg >= 0) {
      // ---- 4. the first term of the segment with K >= kst before it ----
      const int lo = sh.seg_start[stop_seg], hi = sh.seg_start[stop_seg + 1];
      const int eu = sh.seg_cls[stop_seg];
      const uint32_t K0 = sh.stop_K, kst = kstop_of(stop, eu);
      if (tid == 0) sh.stop_at = hi;
      __syncthreads();
      Fn a = X;
      int first = 0x7FFFFFFF;  // this thread's first term with K >= kst before it
#pragma unroll
      for (int k = 0; k < T; ++k) {
        const int i = c0 + j0 + k;
        if (j0 + k < cn) {
          if ((heads >> k) & 1u) a = fn_id();
          if (i > lo && i < hi && sat_add(K0, fn_inc(a, K0)) >= kst && i < first) first = i;
          a = fn_then(a, cls[k] != kUnc ? fn_term(x[k], cls[k]) : fn_id());
        }
      }
      // terms are thread-major: the wave's first candidate is its lowest lane's
      const uint64_t bal = __ballot(first != 0x7FFFFFFF);
      if (bal && lane == (int)__builtin_ctzll(bal)) atomicMin(&sh.stop_at, first);
      __syncthreads();
      const int at = sh.stop_at;
      // the value before term `at` (or after the segment): recomputed by its owner
      if (at == hi) {
        if (tid == 0) sh.s = __builtin_ldexpf((float)sat_add(K0, fn_inc(Fn{sh.seg_i0[stop_seg], sh.seg_i1[stop_seg], 0u}, K0)), eu);
      } else {
        Fn b = X;
#pragma unroll
        for (int k = 0; k < T; ++k) {
          const int i = c0 + j0 + k;
          if (j0 + k < cn) {
            if ((heads >> k) & 1u) b = fn_id();
            if (i == at) sh.s = __builtin_ldexpf((float)sat_add(K0, fn_inc(b, K0)), eu);
            b = fn_then(b, cls[k] != kUnc ? fn_term(x[k], cls[k]) : fn_id());
          }
        }
      }
      __syncthreads();
    }
    const int stop_at = sh.stop_at;
    s = sh.s;
    __syncthreads();  // sh is reused by the next chunk
    if (stop_at >= 0) return SeqResult{stop_at, s};
  }
}

}  // namespace aq
