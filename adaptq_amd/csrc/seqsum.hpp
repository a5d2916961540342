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
// one binade therefore adds the plain integer sum of their r to K, and only
// the terms where s crosses a binade edge, and ties, need the hardware's
// own adds in order.  chain_sum_block (below) predicts each thread's binade
// from an fp32 prefix sum, sums the increments of its clean terms in
// parallel, and walks the few segments on one wave, checking every
// prediction it uses against the exact s.  Terms must be finite and not
// negative (-0 is fine).  The per-term functions are host-callable;
// tests/cpp/seqsum_check.cpp runs the same segment algorithm on the host
// against sequential fp32 sums of random, tie-heavy, subnormal, wide-range
// and stop-at-a-reached-value sequences, with planted mispredictions, and
// the GPU tests compare the sparse-V weights that depend on these sums with
// the oracle's bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "seqsum_terms.hpp"

namespace aq {

// The result of s = fl(s + x_i) for i = 0, 1, ... while i < n and s < stop
// (tested before each addition), as one lane would run it: how many terms
// were added and the sum after them (the same in every thread).
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


__device__ __forceinline__ float rl_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

}  // namespace seqsum_detail

// ---- every thread classifies its own terms, one wave walks ----
//
// chain_sum_block: the same chain for at most kBlock E terms that the block
// already holds in registers, thread t owning terms t E .. t E + E - 1 (and
// an LDS copy xs of all m terms).
//   1. each thread predicts one class for its E terms from an fp32 prefix
//      (run_class_f32) and sums their increments r (fast_incr); a thread
//      whose prediction fails or that holds a tie is a hardware thread;
//   2. a segment ends at a hardware thread, at the last clean thread before
//      a different class, or at the last thread; its record holds the class
//      of its clean threads (or none), the block's inclusive sum of r at its
//      end and its last thread;
//   3. wave 0 walks the records in order without branches: K += the
//      segment's increment, then the hardware thread's terms by fp32 adds
//      (lane k adds record k's terms; the walk keeps lane i's sum),
//      recording the value each segment starts from; then every record
//      checks its own start in parallel (s in the class's binade, K below
//      2^24 after the clean threads); a failed check redoes the whole chain
//      on one lane, so the result is the chain's in every case;
//   4. STOP (the stop tested before each term): it lies in the first segment
//      whose end reaches it: in its hardware terms the walk tests them one by
//      one, in its clean part the block finds the thread whose K range holds
//      kstop_of(stop) and that thread steps through its terms.
// Non-finite or negative terms send the whole sum to one lane.

// A record's last thread, with kRecHw when it is a hardware thread.
constexpr int kRecHw = 0x8000, kRecThr = 0x7FFF;

// LDS of chain_sum_block.
struct ChainShared {
  int cls[seqsum_detail::kBlock];  // the thread's class, or kUnc
  int rec_cls[seqsum_detail::kBlock];
  uint32_t rec_R[seqsum_detail::kBlock];
  int rec_end[seqsum_detail::kBlock];  // last thread, | kRecHw when it is a hardware thread
  float wtot[seqsum_detail::kWaves];   // sum of the wave's terms
  uint32_t wr[seqsum_detail::kWaves];  // sum of the wave's r
  int wcnt[seqsum_detail::kWaves];     // segments ending in the wave
  int wbad[seqsum_detail::kWaves];     // a term that is not finite and >= 0
  int q_search, q_start, q_end, q_cls;
  uint32_t q_K0, q_Rp, q_exp;
  int count;
  float s;
};

namespace seqsum_detail {

// A block barrier that orders LDS only: global loads issued before it stay in
// flight (the sums share nothing through global memory, and chain_sum_long's
// next chunk is requested before a chunk is walked).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int CTRL, int ROW_MASK, int BANK_MASK, bool BOUND>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, BANK_MASK, BOUND);
}
// Inclusive scan over the wave by DPP: row shifts by 1, 2, 3 (zero fill),
// 4 (lanes 4..15 of each row) and 8 (lanes 8..15), then lane 15's total into
// rows 1 and 3 and lane 31's into rows 2 and 3.  Exact for integers; for
// floats the rounding of this order differs from a left-to-right sum, which
// the prediction's margin covers (run_class_f32).
template <class T>
__device__ __forceinline__ T wave_scan_dpp(T v) {
  auto bits = [](T a) -> uint32_t {
    if constexpr (sizeof(T) == 4 && !__is_same(T, uint32_t)) return __float_as_uint(a);
    else return a;
  };
  auto val = [](uint32_t b) -> T {
    if constexpr (sizeof(T) == 4 && !__is_same(T, uint32_t)) return __uint_as_float(b);
    else return b;
  };
  const uint32_t vb = bits(v);
  T s = v + val(dpp_u<0x111, 0xF, 0xF, true>(vb));  // row_shr:1
  s += val(dpp_u<0x112, 0xF, 0xF, true>(vb));      // row_shr:2
  s += val(dpp_u<0x113, 0xF, 0xF, true>(vb));      // row_shr:3
  s += val(dpp_u<0x114, 0xF, 0xE, false>(bits(s)));  // row_shr:4
  s += val(dpp_u<0x118, 0xF, 0xC, false>(bits(s)));  // row_shr:8
  s += val(dpp_u<0x142, 0xA, 0xF, false>(bits(s)));  // row_bcast:15
  s += val(dpp_u<0x143, 0xC, 0xF, false>(bits(s)));  // row_bcast:31
  return s;
}

// r = x / 2^eu rounded to the nearest integer for a term of class eu (x >= 0
// or -0): false for a tie or for r >= 2^23.  x / 2^eu is exact in fp32 (a
// result that underflows is below 1/2).
__device__ __forceinline__ bool fast_incr(float x, int eu, uint32_t &r) {
  const float y = __builtin_ldexpf(x, -eu);
  r = (uint32_t)__builtin_rintf(y);
  return y < 8388608.0f && y - __builtin_floorf(y) != 0.5f;
}

}  // namespace seqsum_detail

// Steps 1 and 2 of chain_sum_block: every thread's class and increments,
// predicted from s0 (the exact sum before the terms, or a prediction of it:
// the walk checks every class it uses), and the segment records in cs (with
// cs.wbad, a term not finite and >= 0, per wave).  Returns the thread's class,
// the sum of its r, the block's inclusive sum of r at it, and the number of
// records.  Ends with a barrier.
struct ChainThread {
  int c;
  uint32_t rs, Rb;
  int nseg;
};

template <int E>
__device__ __forceinline__ ChainThread chain_records(const float (&x)[E], int m, float s0,
                                                     ChainShared &cs) {
  using namespace seqsum_detail;
  static_assert(E >= 1 && E <= 8, "terms per thread");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j0 = tid * E;
  const int nt = (m + E - 1) / E;  // threads with terms
  const bool has = tid < nt;
  float loc = 0.0f;
  bool bad = false;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (j0 + e < m) {
      loc += x[e];
      bad |= !(x[e] >= 0.0f && x[e] <= 3.402823466e38f);
    }
  // ---- 1. prefix prediction, class, increments ----
  const float inc = wave_scan_dpp(loc);
  const uint64_t bad_w = __ballot(bad);
  if (lane == 63) cs.wtot[wave] = inc;
  if (lane == 0) cs.wbad[wave] = bad_w != 0;
  lds_barrier();
  float P = s0 + (inc - loc);
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) P += cs.wtot[w];
  int c = kUnc;
  uint32_t rs = 0;
  if (has) {
    c = run_class_f32(P, loc, j0 + E);
    if (c != kUnc) {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        uint32_t r = 0;
        if (j0 + e < m && !fast_incr(x[e], c, r)) c = kUnc;
        rs += j0 + e < m ? r : 0u;
      }
    }
    // a thread whose run alone reaches 2^23 ulps never passes the walk's check
    if (c == kUnc || rs >= (kTop >> 1)) {
      c = kUnc;
      rs = 0;
    }
  }
  const uint32_t rin = wave_scan_dpp(rs);  // below 64 x 2^23: no wrap
  cs.cls[tid] = c;
  if (lane == 63) cs.wr[wave] = rin;
  lds_barrier();
  // ---- 2. segment records ----
  uint32_t Rb = rin;  // the block's inclusive sum of r
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w < wave) Rb += cs.wr[w];
  const int cn = tid + 1 < nt ? cs.cls[tid + 1] : kNoClass;
  const int cp = tid > 0 ? cs.cls[tid - 1] : kUnc;
  const bool end = has && (c == kUnc || tid == nt - 1 || (cn != kUnc && cn != c));
  const uint64_t em = __ballot(end);
  if (lane == 0) cs.wcnt[wave] = __popcll(em);
  lds_barrier();
  int kidx = __popcll(em & ((1ull << lane) - 1ull)), nseg = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int cw = cs.wcnt[w];
    if (w < wave) kidx += cw;
    nseg += cw;
  }
  if (end) {
    cs.rec_cls[kidx] = c != kUnc ? c : (cp != kUnc ? cp : kNoClass);
    cs.rec_R[kidx] = Rb;
    cs.rec_end[kidx] = tid | (c == kUnc ? kRecHw : 0);
  }
  lds_barrier();

  return ChainThread{c, rs, Rb, nseg};
}

template <int E, bool STOP>
__device__ __forceinline__ SeqResult chain_sum_block(const float (&x)[E], int m, float s0, float stop,
                                                     const float *xs, ChainShared &cs) {
  using namespace seqsum_detail;
  if constexpr (!STOP) stop = __builtin_inff();
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j0 = tid * E;
  const ChainThread ct = chain_records<E>(x, m, s0, cs);
  const int c = ct.c, nseg = ct.nseg;
  const uint32_t rs = ct.rs, Rb = ct.Rb;

  // ---- 3. the walk, on wave 0 ----
  if (wave == 0) {
    bool fail = __ballot(lane < kWaves && cs.wbad[lane < kWaves ? lane : 0] != 0) != 0;
    uint32_t wb = __builtin_amdgcn_readfirstlane(__float_as_uint(s0));
    int count = m, search = 0;
    if (!(s0 < stop)) {
      count = 0;
    } else if (!fail) {
      for (int base = 0; base < nseg; base += 64) {
        const int k = base + lane;
        const bool v = k < nseg;
        const int lc = v ? cs.rec_cls[k] : kNoClass;
        const uint32_t lrp = v && k > 0 ? cs.rec_R[k - 1] : 0u;
        const uint32_t linc = v ? cs.rec_R[k] - lrp : 0u;
        const int le = v ? cs.rec_end[k] : 0;
        const int lt = le & kRecThr;
        float lx[E];
#pragma unroll
        for (int e = 0; e < E; ++e) lx[e] = (le & kRecHw) && lt * E + e < m ? xs[lt * E + e] : 0.0f;
        const int cnt = nseg - base < 64 ? nseg - base : 64;
        // the walk: the running sum's bits stay in a vector register (the
        // same in every lane); every lane adds its own record's hardware
        // terms to it and the one of record i is kept
        uint32_t wv = wb, sst = 0u, smid = 0u;
        for (int i = 0; i < cnt; ++i) {
          asm volatile("" : "+v"(wv));
          const uint32_t in = (uint32_t)__builtin_amdgcn_readlane((int)linc, i);
          sst = lane == i ? wv : sst;
          wv += in;
          if constexpr (STOP) smid = lane == i ? wv : smid;
          float sv = __uint_as_float(wv);
#pragma unroll
          for (int e = 0; e < E; ++e) sv = __fadd_rn(sv, lx[e]);
          wv = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(sv), i);
        }
        wb = __builtin_amdgcn_readfirstlane(wv);
        // every record checks the value its clean threads started from
        const bool bad_k = lane < cnt && lc != kNoClass &&
                           (((sst >> 23) != (uint32_t)(lc + 150)) | ((sst & 0x7FFFFFu) + linc >= 0x800000u));
        if (__ballot(bad_k) != 0) {
          fail = true;
          break;
        }
        if constexpr (STOP) {
          if (!(__uint_as_float(wb) < stop)) {
            // the first segment of this batch whose end reaches the stop
            const uint32_t nxt = (uint32_t)__shfl_down((int)sst, 1, 64);
            const uint32_t send = lane == cnt - 1 ? wb : nxt;
            const int ks = (int)__builtin_ctzll(__ballot(lane < cnt && !(__uint_as_float(send) < stop)));
            const uint32_t s_mid = (uint32_t)__builtin_amdgcn_readlane((int)smid, ks);
            const int t = __builtin_amdgcn_readlane(lt, ks);
            if (!(__uint_as_float(s_mid) < stop)) {
              // in its clean part: the block finds the thread (below)
              const uint32_t s_st = (uint32_t)__builtin_amdgcn_readlane((int)sst, ks);
              if (lane == 0) {
                cs.q_cls = __builtin_amdgcn_readlane(lc, ks);
                cs.q_K0 = 0x800000u | (s_st & 0x7FFFFFu);
                cs.q_exp = s_st & 0xFF800000u;
                cs.q_Rp = (uint32_t)__builtin_amdgcn_readlane((int)lrp, ks);
                cs.q_start = base + ks > 0 ? (cs.rec_end[base + ks - 1] & kRecThr) + 1 : 0;
                cs.q_end = t;
              }
              search = 1;
            } else {
              // in its hardware thread's terms, one by one
              float sv = __uint_as_float(s_mid);
              count = t * E + E;
#pragma unroll
              for (int e = 0; e < E; ++e) {
                const int i = t * E + e;
                if (count == t * E + E && i < m) {
                  if (!(sv < stop)) count = i;
                  else sv = __fadd_rn(sv, rl_f(lx[e], ks));
                }
              }
              wb = __builtin_amdgcn_readfirstlane(__float_as_uint(sv));
            }
            break;
          }
        }
      }
    }
    if (fail) {  // a prediction failed, or a term is not finite and >= 0
      wb = __builtin_amdgcn_readfirstlane(__float_as_uint(s0));
      const int at = hw_run(xs, 0, 0, m, stop, wb);
      count = at >= 0 ? at : m;
      search = 0;
    }
    if (lane == 0) {
      cs.count = count < m ? count : m;
      cs.s = __uint_as_float(wb);
      cs.q_search = search;
    }
  }
  lds_barrier();
  if constexpr (STOP) {
    if (cs.q_search) {
      if (tid >= cs.q_start && tid <= cs.q_end && c != kUnc) {
        const uint32_t ks = kstop_of(stop, cs.q_cls);
        uint32_t Kb = cs.q_K0 + (Rb - rs - cs.q_Rp);
        if (Kb < ks && Kb + rs >= ks) {
          int e = 0;
#pragma unroll
          for (int q = 0; q < E; ++q) {
            if (e == q && Kb < ks) {
              uint32_t r = 0;
              fast_incr(x[q], c, r);
              Kb += r;
              e = q + 1;
            }
          }
          cs.count = j0 + e < m ? j0 + e : m;
          cs.s = __uint_as_float(cs.q_exp | (Kb - 0x800000u));
        }
      }
      lds_barrier();
    }
  }
  const SeqResult res{cs.count, cs.s};
  lds_barrier();
  return res;
}

// The chain over any number of terms, chunks of kBlock kMaxT through
// chain_sum_block, each from the exact sum the one before ended with (the
// next chunk's terms are requested before a chunk is walked).  load(i) for
// 0 <= i < n returns term i; xs: kBlock kMaxT floats of LDS.  Called by all
// kBlock threads with uniform arguments.
template <bool STOP, class Load>
__device__ __forceinline__ SeqResult chain_sum_long(Load load, int n, float s, float stop, float *xs,
                                                    ChainShared &cs) {
  using namespace seqsum_detail;
  constexpr int E = kMaxT, C = kBlock * kMaxT;
  const int j0 = threadIdx.x * E;
  float x[E];
#pragma unroll
  for (int k = 0; k < E; ++k) x[k] = j0 + k < n ? load(j0 + k) : 0.0f;
  for (int c0 = 0; c0 < n; c0 += C) {
    const int cn = n - c0 < C ? n - c0 : C;
#pragma unroll
    for (int k = 0; k < E; ++k) xs[j0 + k] = x[k];
    lds_barrier();
    float y[E];
#pragma unroll
    for (int k = 0; k < E; ++k) y[k] = c0 + C + j0 + k < n ? load(c0 + C + j0 + k) : 0.0f;
    const SeqResult r = chain_sum_block<E, STOP>(x, cn, s, stop, xs, cs);
    s = r.s;
    if (STOP && r.count < cn) return SeqResult{c0 + r.count, s};
#pragma unroll
    for (int k = 0; k < E; ++k) x[k] = y[k];
  }
  return SeqResult{n, s};
}

}  // namespace aq
