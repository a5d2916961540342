// seqsum.hpp -- a left-to-right fp32 sum of non-negative terms, bit for bit,
// by a whole block in parallel.
//
// The reference's softmax denominator (attention.cpp:422-426) and sparse-V
// mass loop (attention.cpp:454-472) are chains s = fl(s + x_i) whose exact
// bits decide which tokens sparse-V keeps.  One lane runs such a chain at
// about 4 ns a term; this computes the same bits with every thread of the
// block.
//
// While s stays in one binade [2^B, 2^(B+1)), every representable s is K u
// with u = 2^(B-23) and K an integer in [2^23, 2^24), and fl(s + x) = (K + r) u
// where r = x / u rounded to the nearest integer -- independent of s, unless
// x / u lies exactly halfway (a tie: the sum then rounds to the even one of
// two neighbours, which depends on K).  A run of non-tie terms added inside
// one binade therefore adds the plain integer sum of their r to K.
//
// The block takes kBlock T terms at a time:
//   1. an fp64 prefix sum P_j predicts s before term j (the fp32 chain is
//      within (j + 1) 2^-24 P of it); a term is clean when the whole
//      interval around P_j plus the term, with its rounding, stays inside one
//      binade, and it is not a tie; every other term is added by the
//      hardware, one add on one lane;
//   2. one integer prefix scan gives every term the sum of the r before it,
//      and the number of segments (maximal runs of clean terms of one binade,
//      and single hardware terms) before it;
//   3. one wave walks the segments with the exact s: a hardware term is an
//      fp32 add; a clean segment checks that s lies in its binade, adds the
//      difference of the prefix sums at its ends to K, and checks that K
//      stays below 2^24 -- if a check fails (a prediction was wrong), the
//      chunk is redone term by term on one lane, so the result is the
//      chain's in every case;
//   4. the stop test of the mass loop (stop before adding term i once s >=
//      stop) is K >= ceil(stop / u) inside a clean segment; the block finds
//      the first such term of the segment the walk stops in.
// Terms must be finite and not negative (-0 is fine).  The per-term
// functions are host-callable; tests/cpp/seqsum_check.cpp runs the same
// segment algorithm on the host against sequential fp32 sums of random,
// tie-heavy, subnormal, wide-range and stop-at-a-reached-value sequences,
// and the GPU tests compare the sparse-V weights that depend on these sums
// with the oracle's bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "seqsum_terms.hpp"

namespace aq {

// Shared memory of block_seq_sum.
struct SeqShared {
  double dsum[seqsum_detail::kWaves];
  uint64_t wscan[seqsum_detail::kWaves];
  uint32_t wcnt[seqsum_detail::kWaves];
  int last_cls[seqsum_detail::kBlock];
  uint64_t seg_r[seqsum_detail::kMaxSeg + 1];  // sum of r before the segment's first term
  int seg_start[seqsum_detail::kMaxSeg + 1];
  int seg_cls[seqsum_detail::kMaxSeg];
  float xs[seqsum_detail::kBlock * seqsum_detail::kMaxT];  // the chunk's terms
  int nseg, stop_at, stop_seg;
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

namespace seqsum_detail {

// Terms xs[i - c0] for i in [from, to) added one at a time while s < stop
// (s: its bit pattern wb, uniform over the wave).  Whole steps of 8 terms,
// read from LDS one step ahead, are added as one chain; the sum never
// decreases (terms are not negative), so when a step ends below the stop no
// test inside it failed.  The step that reaches the stop, and the last
// partial step, are added term by term with the test before each.  Returns
// the index whose test failed, or -1.
__device__ __forceinline__ int hw_run(const float *xs, int c0, int from, int to, float stop,
                                      uint32_t &wb) {
  float w = __uint_as_float(wb);
  int i = from;
  if (i + 8 <= to) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = xs[i + k - c0];
    for (;;) {
      const bool more = i + 16 <= to;
      float nv[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) nv[k] = more ? xs[i + 8 + k - c0] : 0.0f;
      float wn = w;
#pragma unroll
      for (int k = 0; k < 8; ++k) wn = __fadd_rn(wn, v[k]);
      if (!__builtin_amdgcn_readfirstlane((int)(wn < stop))) break;  // i: the step to test
      w = wn;
      i += 8;
      if (!more) break;
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = nv[k];
    }
  }
  for (; i < to; ++i) {
    if (!__builtin_amdgcn_readfirstlane((int)(w < stop))) {
      wb = __builtin_amdgcn_readfirstlane(__float_as_uint(w));
      return i;
    }
    w = __fadd_rn(w, xs[i - c0]);
  }
  wb = __builtin_amdgcn_readfirstlane(__float_as_uint(w));
  return -1;
}

}  // namespace seqsum_detail

namespace seqsum_detail {

// Steps 1 and 2 for one chunk of cn terms whose first term has index c0:
// the thread's terms x[T] (chunk positions j0 = tid T ..), P0 the fp64
// prediction of s before the chunk's first term, and jbase the number of
// terms between the exact start and the chunk (0 when s is exact at the
// chunk, else the chunk's index: the prediction's bound grows with it).
// Returns the thread's classes and increments and ex, the sum of r before
// its first term; sh holds the chunk's segment table (nseg, and for the
// first kMaxSeg segments their start, class and sum of r before them, plus
// the start and sum of the one after).  Ends with a barrier.
template <int T>
__device__ __forceinline__ void seq_classify(const float (&x)[T], int cn, int c0, double P0,
                                             int jbase, SeqShared &sh, int (&cls)[T],
                                             uint32_t (&r)[T], uint64_t &ex) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j0 = tid * T;
  // ---- 1. fp64 prefix before the thread's first term, classes ----
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
  double P = P0 + (incl - loc);
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) P += sh.dsum[w];
  {
    const int nv = cn - j0 < T ? cn - j0 : T;  // the thread's terms in the chunk
    const int jb = jbase + j0;                 // terms before the thread's first since the exact start
    const int u = nv > 0 ? range_class(P, loc, jb + nv) : kUnc;
    if (u != kUnc) {
#pragma unroll
      for (int k = 0; k < T; ++k) {
        uint32_t rk = 0u;
        const bool ok = j0 + k < cn && scaled_incr(x[k], u, rk);
        cls[k] = ok ? u : kUnc;
        r[k] = ok ? rk : 0u;
      }
    } else {
      const int E = nv > 0 ? edge_of(P, loc, jb + nv) : kUnc;
      if (E != kUnc) {
        // the range crosses one binade edge 2^E: each term below or above it
        const double del = range_del(P, loc, jb + nv);
#pragma unroll
        for (int k = 0; k < T; ++k) {
          const int c = j0 + k < cn ? split_class(P, (double)x[k], del, E) : kUnc;
          uint32_t rk = 0u;
          const bool ok = c != kUnc && scaled_incr(x[k], c, rk);
          cls[k] = ok ? c : kUnc;
          r[k] = ok ? rk : 0u;
          P += (double)x[k];
        }
      } else {
#pragma unroll
        for (int k = 0; k < T; ++k) {
          int c = j0 + k < cn ? term_class(P, x[k], jb + k) : kUnc;
          r[k] = 0u;
          if (c != kUnc && !term_incr(x[k], c, r[k])) {
            c = kUnc;
            r[k] = 0u;
          }
          cls[k] = c;
          P += (double)x[k];
        }
      }
    }
  }
  sh.last_cls[tid] = cls[T - 1];
  __syncthreads();

  // ---- 2. segment heads (a change of class; runs of hardware terms are
  // one segment) and the scans of the sum of r and of the heads ----
  uint32_t heads = 0u;  // bit k: term k starts a segment
  uint64_t rsum = 0u;
  {
    int pc = tid > 0 ? sh.last_cls[tid - 1] : kNoClass;
#pragma unroll
    for (int k = 0; k < T; ++k) {
      if (j0 + k < cn && cls[k] != pc) heads |= 1u << k;
      pc = cls[k];
      rsum += r[k];
    }
  }
  const uint32_t hmine = (uint32_t)__popc(heads);
  uint64_t sc = rsum;
  uint32_t hc = hmine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint64_t y = __shfl_up(sc, off, 64);
    const uint32_t yh = __shfl_up(hc, off, 64);
    if (lane >= off) {
      sc += y;
      hc += yh;
    }
  }
  if (lane == 63) {
    sh.wscan[wave] = sc;
    sh.wcnt[wave] = hc;
  }
  __syncthreads();
  ex = sc - rsum;  // exclusive prefixes of this thread
  uint32_t hex = hc - hmine;
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) {
      ex += sh.wscan[w];
      hex += sh.wcnt[w];
    }
  if (tid == kBlock - 1) {
    const int ns = (int)(hex + hmine);
    sh.nseg = ns;
    if (ns <= kMaxSeg) {
      sh.seg_r[ns] = ex + rsum;
      sh.seg_start[ns] = c0 + cn;
    }
  }

  // ---- segment table: each head records its start, class and the sum of
  // r before it (the first kMaxSeg segments, and the start of the next) ----
  {
    uint32_t hid = hex;
    uint64_t R = ex;
#pragma unroll
    for (int k = 0; k < T; ++k) {
      if ((heads >> k) & 1u) {
        if (hid <= (uint32_t)kMaxSeg) {
          sh.seg_start[hid] = c0 + j0 + k;
          sh.seg_r[hid] = R;
        }
        if (hid < (uint32_t)kMaxSeg) sh.seg_cls[hid] = cls[k];
        ++hid;
      }
      R += r[k];
    }
  }
  __syncthreads();
}

// Step 3 for one chunk [c0, c0 + cn) whose terms are at sh.xs and segment
// table in sh (seq_classify's), from the exact sum s: the walk over the
// segments by wave 0 (each lane holds one segment of a group of 64, read
// back with readlane), a redo of the chunk term by term if a prediction
// fails, the rest of the chunk term by term beyond kMaxSeg segments.  Wave
// 0 leaves in sh: stop_at (the index whose stop test failed, else -1),
// stop_seg (the clean segment inside which s reaches the stop, else -1),
// stop_K and s (the sum before that segment, or after the chunk / before
// stop_at).  The caller synchronises.
__device__ __forceinline__ void seq_walk(int c0, int cn, float s, float stop, SeqShared &sh) {
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) != 0) return;
  // beyond kMaxSeg segments, the walk takes the first kMaxSeg and adds the
  // rest of the chunk term by term
  const int ns_all = sh.nseg, ns = ns_all < kMaxSeg ? ns_all : kMaxSeg;
  const uint32_t sb = __float_as_uint(stop);  // stop > 0 here
  uint32_t wb = __builtin_amdgcn_readfirstlane(__float_as_uint(s));
  int stop_at = -1, stop_seg = -1, redo = 0;
  for (int base = 0; base < ns && !redo && stop_at < 0 && stop_seg < 0; base += 64) {
    const int k = base + lane;
    const int l_cls = k < ns ? sh.seg_cls[k] : kUnc;
    const int l_start = k < ns ? sh.seg_start[k] : 0;
    const int l_end = k < ns ? sh.seg_start[k + 1] : 0;
    const uint64_t l_inc = k < ns ? sh.seg_r[k + 1] - sh.seg_r[k] : 0u;
    const uint32_t l_inc32 = l_inc >= kTop ? kTop : (uint32_t)l_inc;
    const int m = ns - base < 64 ? ns - base : 64;
    for (int t = 0; t < m; ++t) {
      const int cl = __builtin_amdgcn_readlane(l_cls, t);
      const int st = __builtin_amdgcn_readlane(l_start, t);
      if (cl == kUnc) {
        stop_at = hw_run(sh.xs, c0, st, __builtin_amdgcn_readlane(l_end, t), stop, wb);
        if (stop_at >= 0) break;
        continue;
      }
      if ((wb & 0x7FFFFFFFu) >= sb) {
        stop_at = st;
        break;
      }
      // a clean segment: s is positive and normal, K += the segment's r
      const uint32_t inc = (uint32_t)__builtin_amdgcn_readlane((int)l_inc32, t);
      const uint32_t exb = (uint32_t)(cl + 150), nb = wb + inc;
      if ((wb >> 23) != exb || inc >= kTop || (nb >> 23) != exb) {
        redo = 1;
        break;
      }
      if (nb >= sb) {
        stop_seg = base + t;
        break;
      }
      wb = nb;
    }
  }
  if (redo) {
    // a prediction failed: the chunk term by term
    wb = __builtin_amdgcn_readfirstlane(__float_as_uint(s));
    stop_at = hw_run(sh.xs, c0, c0, c0 + cn, stop, wb);
    stop_seg = -1;
  } else if (ns_all > kMaxSeg && stop_at < 0 && stop_seg < 0) {
    stop_at = hw_run(sh.xs, c0, sh.seg_start[kMaxSeg], c0 + cn, stop, wb);
  }
  if (lane == 0) {
    sh.stop_at = stop_at;
    sh.stop_seg = stop_seg;
    sh.stop_K = (wb & 0x7FFFFFu) | 0x800000u;
    sh.s = __uint_as_float(wb);
  }
}

// A segment list flattened for a sum without a stop: segment k covers terms
// [start[k], start[k + 1]) (start[m] is the end) of class cls[k] (kUnc: added
// by the hardware); inc[k] is a clean segment's sum of r (kTop when it
// reaches 2^24), x0[k] / x1[k] a hardware segment's first two terms.  The
// terms [c0, c0 + cn) are at xs.  From the exact sum s, wave 0 walks the list
// (a failed check redoes the whole range term by term) and returns the sum;
// other waves return s.  Each lane holds one segment of a group of 64, read
// back with readlane, so a segment costs no memory access except the terms
// of a hardware segment past its second (seq_add_run).
__device__ __forceinline__ float rl_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// w + xs[from - c0] + ... + xs[to - 1 - c0], left to right (w >= +0 and
// terms not negative; xs holds kBlock kMaxT terms): steps of 8 terms in
// registers, the next 8 read from LDS while these are added; past `to` a step
// adds +0, which leaves the sum as it is (the reads stay inside xs and are
// not branched around).
__device__ __forceinline__ float seq_add_run(const float *xs, int c0, int from, int to, float w) {
  constexpr int kLast = kBlock * kMaxT - 1;
  auto term = [&](int i) {
    const float v = xs[i - c0 < kLast ? i - c0 : kLast];
    return i < to ? v : 0.0f;
  };
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = term(from + k);
  for (int i = from; i < to; i += 8) {
    float nv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) nv[k] = term(i + 8 + k);
#pragma unroll
    for (int k = 0; k < 8; ++k) w = __fadd_rn(w, v[k]);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = nv[k];
  }
  return w;
}

__device__ __forceinline__ float seq_walk_flat(const float *xs, int c0, int cn, const int *start,
                                               const int *cls, const uint32_t *inc,
                                               const float *x0, const float *x1, int m, float s) {
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) != 0) return s;
  // the sum's bits stay scalar through clean segments
  uint32_t wb = __builtin_amdgcn_readfirstlane(__float_as_uint(s));
  int redo = 0;
  for (int base = 0; base < m && !redo; base += 64) {
    const int k = base + lane;
    const int l_cls = k < m ? cls[k] : kUnc;
    const int l_start = k < m ? start[k] : 0;
    const int l_end = k < m ? start[k + 1] : 0;
    const uint32_t l_inc = k < m ? inc[k] : 0u;
    const float l_x0 = k < m ? x0[k] : 0.0f;
    const float l_x1 = k < m ? x1[k] : 0.0f;
    const int g = m - base < 64 ? m - base : 64;
    for (int t = 0; t < g; ++t) {
      const int cl = __builtin_amdgcn_readlane(l_cls, t);
      if (cl == kUnc) {
        const int st = __builtin_amdgcn_readlane(l_start, t);
        const int len = __builtin_amdgcn_readlane(l_end, t) - st;
        float w = __fadd_rn(__uint_as_float(wb), rl_f(l_x0, t));
        if (len > 1) w = __fadd_rn(w, rl_f(l_x1, t));
        if (len > 2) w = seq_add_run(xs, c0, st + 2, st + len, w);
        wb = __builtin_amdgcn_readfirstlane(__float_as_uint(w));
        continue;
      }
      // a clean segment: s in the class's binade and K + inc below 2^24 (a
      // failure is recorded and the walk runs on without adding: no branch
      // out of the loop, so the compiler keeps the bits in scalar registers)
      const uint32_t in = (uint32_t)__builtin_amdgcn_readlane((int)l_inc, t);
      const bool ok = ((wb >> 23) == (uint32_t)(cl + 150)) & ((wb & 0x7FFFFFu) + in < 0x800000u);
      redo |= ok ? 0 : 1;
      wb = __builtin_amdgcn_readfirstlane(ok ? wb + in : wb);
    }
  }
  if (redo) return seq_add_run(xs, c0, c0, c0 + cn, s);  // a prediction failed
  return __uint_as_float(wb);
}

}  // namespace seqsum_detail

template <int T, class Load>
__device__ __forceinline__ SeqResult block_seq_sum(Load load, int n, float s, float stop,
                                                   SeqShared &sh) {
  using namespace seqsum_detail;
  static_assert(T >= 1 && T <= kMaxT, "terms per thread");
  const int tid = threadIdx.x, lane = tid & 63;
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
  const int j0 = tid * T;  // first term of this thread within a chunk
  float x[T];
#pragma unroll
  for (int k = 0; k < T; ++k) x[k] = j0 + k < n ? load(j0 + k) : 0.0f;
  for (int c0 = 0;; c0 += kBlock * T) {
    if (!(s < stop) || c0 >= n) return SeqResult{c0 < n ? c0 : n, s};
    const int cn = n - c0 < kBlock * T ? n - c0 : kBlock * T;  // terms of this chunk
#pragma unroll
    for (int k = 0; k < T; ++k) sh.xs[j0 + k] = x[k];
    int cls[T];
    uint32_t r[T];
    uint64_t ex;
    seq_classify<T>(x, cn, c0, (double)s, 0, sh, cls, r, ex);

    // the next chunk's terms are requested before the walk
    const int c1 = c0 + kBlock * T;
#pragma unroll
    for (int k = 0; k < T; ++k) x[k] = c1 + j0 + k < n ? load(c1 + j0 + k) : 0.0f;

    seq_walk(c0, cn, s, stop, sh);
    __syncthreads();
    const int stop_seg = sh.stop_seg;
    if (stop_seg >= 0) {
      // ---- 4. the first term of the segment with K >= kst before it ----
      const int lo = sh.seg_start[stop_seg], hi = sh.seg_start[stop_seg + 1];
      const int eu = sh.seg_cls[stop_seg];
      const uint64_t r_lo = sh.seg_r[stop_seg], r_hi = sh.seg_r[stop_seg + 1];
      const uint32_t K0 = sh.stop_K, kst = kstop_of(stop, eu);
      __syncthreads();
      if (tid == 0) sh.stop_at = hi;
      __syncthreads();
      uint64_t R = ex;
      int first = 0x7FFFFFFF;  // this thread's first term with K >= kst before it
#pragma unroll
      for (int k = 0; k < T; ++k) {
        const int i = c0 + j0 + k;
        if (i > lo && i < hi && (uint64_t)K0 + (R - r_lo) >= (uint64_t)kst && i < first) first = i;
        R += r[k];
      }
      // terms are thread-major: the wave's first candidate is its lowest lane's
      const uint64_t bal = __ballot(first != 0x7FFFFFFF);
      if (bal && lane == (int)__builtin_ctzll(bal)) atomicMin(&sh.stop_at, first);
      __syncthreads();
      const int at = sh.stop_at;
      // the sum before term `at` (or after the segment)
      if (at == hi) {
        if (tid == 0) sh.s = __builtin_ldexpf((float)(K0 + (uint32_t)(r_hi - r_lo)), eu);
      } else {
        uint64_t Rb = ex;
#pragma unroll
        for (int k = 0; k < T; ++k) {
          if (c0 + j0 + k == at) sh.s = __builtin_ldexpf((float)(K0 + (uint32_t)(Rb - r_lo)), eu);
          Rb += r[k];
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
