// The segment algorithm of chain_sum_block (adaptq_amd/csrc/seqsum.hpp) run
// on the host, as the block runs it (threads of E terms classified by
// run_class_f32 from a prefix, integer increments from seqsum_terms.hpp,
// segment records, the walk with its checks and full redo, the stop found in
// a segment's clean part or hardware terms), against the plain left-to-right
// fp32 chain with its stop test.  Sequences: softmax-like exponentials,
// sorted probabilities and their quad sums with mass stops (also stops equal
// to a value the chain reaches), tie-heavy terms (exact small integers and
// dyadic fractions over large sums), subnormals, wide exponent ranges, zeros
// and -0, and non-zero start values; 1 to 8 terms per thread (up to 8,192
// terms a call), with exact and with planted wrong prefixes.  Prints the
// mismatch count and how many sums the planted errors sent to the redo;
// exits 0 when nothing mismatches.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../adaptq_amd/csrc/seqsum_terms.hpp"

using namespace aq::seqsum_detail;

static uint32_t fbits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
static float bfloat(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

struct Res {
  int count;
  float s;
};

// The one-lane chain: add while s < stop.
static Res chain(const std::vector<float> &x, float s, float stop) {
  int i = 0;
  const int n = (int)x.size();
  for (; i < n && s < stop; ++i) s = s + x[i];
  return {i, s};
}

// the value after segment k: the next segment's start, or the final sum
static uint32_t k_end_of(int k, int nseg, const std::vector<uint32_t> &sst, uint32_t fin) {
  return k + 1 < nseg ? sst[k + 1] : fin;
}

static long long g_wcases = 0, g_wsegs = 0, g_wredo = 0, g_wclean_stop = 0;

// chain_sum_block (seqsum.hpp) serially.  Threads of E consecutive terms,
// each classified as one (run_class_f32) from the prefix (times `bias`,
// to plant mispredictions).  A segment ends at a hardware thread, at the
// last clean thread before a different class, or at the last thread; its
// record: the class of its clean threads (or none), the block's inclusive
// sum of r at its end, its last thread.  The walk adds each segment's
// increment to K (checked: s in the class's binade, K below 2^24) and then
// its hardware thread's terms; a failed check redoes the whole chain.  The
// stop: the first segment whose end reaches it; inside its clean part the
// thread whose K range holds the threshold steps through its terms.
static Res model_wave(const std::vector<float> &x, float s0, float stop, int E, double bias) {
  const int m = (int)x.size(), nt = (m + E - 1) / E;
  ++g_wcases;
  for (float v : x)
    if (!(v >= 0.0f && v <= 3.402823466e38f)) return chain(x, s0, stop);
  if (!(s0 < stop) || m == 0) return {0, s0};
  std::vector<int> cls(nt, kUnc);
  std::vector<uint32_t> rs(nt, 0), Rb(nt, 0);
  double P = (double)s0;
  uint32_t run = 0;
  for (int t = 0; t < nt; ++t) {
    const int j0 = t * E;
    float loc = 0.0f;
    for (int e = 0; e < E && j0 + e < m; ++e) loc += x[j0 + e];
    int c = run_class_f32((float)(P * bias), loc, j0 + E);
    uint32_t r_sum = 0;
    if (c != kUnc)
      for (int e = 0; e < E && j0 + e < m; ++e) {
        uint32_t r = 0;
        if (!term_incr(x[j0 + e], c, r) || r >= (kTop >> 1)) c = kUnc;  // fast_incr's limits
        r_sum += r;
      }
    if (c == kUnc || r_sum >= (kTop >> 1)) {
      c = kUnc;
      r_sum = 0;
    }
    cls[t] = c;
    rs[t] = r_sum;
    run += r_sum;
    Rb[t] = run;
    P += (double)loc;
  }
  struct Rec {
    int cls;
    uint32_t R;
    int end;
  };
  std::vector<Rec> rec;
  for (int t = 0; t < nt; ++t) {
    const int c = cls[t], cn = t + 1 < nt ? cls[t + 1] : kNoClass;
    if (c == kUnc || t == nt - 1 || (cn != kUnc && cn != c)) {
      const int cp = t > 0 ? cls[t - 1] : kUnc;
      rec.push_back({c != kUnc ? c : (cp != kUnc ? cp : kNoClass), Rb[t], t});
    }
  }
  const int nseg = (int)rec.size();
  g_wsegs += nseg;
  // the walk, every segment, with the start and after-clean-part values
  std::vector<uint32_t> sst(nseg), smid(nseg);
  uint32_t wb = fbits(s0);
  bool fail = false;
  for (int k = 0; k < nseg; ++k) {
    const uint32_t in = rec[k].R - (k ? rec[k - 1].R : 0u), mant = wb & 0x7FFFFFu;
    sst[k] = wb;
    if (rec[k].cls != kNoClass && !(((wb >> 23) == (uint32_t)(rec[k].cls + 150)) && mant + in < 0x800000u))
      fail = true;
    wb += in;
    smid[k] = wb;
    if (cls[rec[k].end] == kUnc) {
      float sv = bfloat(wb);
      for (int e = 0; e < E; ++e) {
        const int i = rec[k].end * E + e;
        sv = sv + (i < m ? x[i] : 0.0f);
      }
      wb = fbits(sv);
    }
  }
  if (fail) {
    ++g_wredo;
    return chain(x, s0, stop);
  }
  if (!(bfloat(wb) >= stop)) return {m, bfloat(wb)};
  int ks_seg = 0;
  while (!(bfloat(k_end_of(ks_seg, nseg, sst, wb)) >= stop)) ++ks_seg;
  const int k = ks_seg;
  const int start = k ? rec[k - 1].end + 1 : 0;
  if (bfloat(smid[k]) >= stop) {
    // inside the clean part: the thread whose K range holds the threshold
    ++g_wclean_stop;
    const int c = rec[k].cls;
    const uint32_t K0 = 0x800000u | (sst[k] & 0x7FFFFFu), ks = kstop_of(stop, c);
    const uint32_t Rp = k ? rec[k - 1].R : 0u;
    for (int t = start; t <= rec[k].end; ++t) {
      if (cls[t] == kUnc) continue;
      uint32_t Kb = K0 + (Rb[t] - rs[t] - Rp);
      const uint32_t Ka = Kb + rs[t];
      if (!(Kb < ks && Ka >= ks)) continue;
      int e = 0;
      for (; e < E; ++e) {
        if (Kb >= ks) break;
        uint32_t r = 0;
        term_incr(t * E + e < m ? x[t * E + e] : 0.0f, c, r);
        Kb += r;
      }
      const int cnt = t * E + e;
      return {cnt < m ? cnt : m, bfloat((sst[k] & 0xFF800000u) | (Kb - 0x800000u))};
    }
    return {-1, 0.0f};  // unreachable
  }
  // inside the hardware thread's terms
  const int t = rec[k].end;
  float sv = bfloat(smid[k]);
  for (int e = 0; e < E; ++e) {
    const int i = t * E + e;
    if (i >= m) return {m, sv};
    if (!(sv < stop)) return {i, sv};
    sv = sv + x[i];
  }
  const int cnt = t * E + E;
  return {cnt < m ? cnt : m, sv};
}

// chain_sum_long: chunks of 8,192 terms (8 a thread), each from the exact sum
// the one before ended with.
static Res model_long(const std::vector<float> &x, float s0, float stop, double bias) {
  const int n = (int)x.size(), C = 1024 * 8;
  float s = s0;
  for (int c0 = 0; c0 < n; c0 += C) {
    const int cn = n - c0 < C ? n - c0 : C;
    const std::vector<float> chunk(x.begin() + c0, x.begin() + c0 + cn);
    const Res r = model_wave(chunk, s, stop, 8, bias);
    s = r.s;
    if (r.count < cn) return {c0 + r.count, s};
  }
  return {n, s};
}

static long long g_cases = 0, g_bad = 0;

static void check(const std::vector<float> &x, float s0, float stop, const char *what) {
  const Res a = chain(x, s0, stop);
  for (double bias : {1.0, 1.05, 0.97}) {
    const Res b = model_long(x, s0, stop, bias);
    ++g_cases;
    if (a.count != b.count || fbits(a.s) != fbits(b.s)) {
      if (g_bad < 10)
        std::printf("MISMATCH (chunks) %s n=%zu bias=%g stop=%a: chain (%d, %a) model (%d, %a)\n", what,
                    x.size(), bias, (double)stop, a.count, (double)a.s, b.count, (double)b.s);
      ++g_bad;
    }
  }
  for (int E : {1, 2, 4, 8}) {
    if ((int)x.size() > 1024 * E) continue;
    for (double bias : {1.0, 1.05, 0.97}) {
      const Res b = model_wave(x, s0, stop, E, bias);
      ++g_cases;
      if (a.count != b.count || fbits(a.s) != fbits(b.s)) {
        if (g_bad < 10)
          std::printf("MISMATCH (per thread) %s n=%zu E=%d bias=%g stop=%a: chain (%d, %a) model (%d, %a)\n",
                      what, x.size(), E, bias, (double)stop, a.count, (double)a.s, b.count, (double)b.s);
        ++g_bad;
      }
    }
  }
}

int main() {
  std::mt19937_64 rng(12345);
  std::normal_distribution<double> nd(0.0, 1.0);
  std::uniform_real_distribution<double> ud(0.0, 1.0);
  const float inf = INFINITY;
  for (int rep = 0; rep < 6; ++rep) {
    for (int n : {5, 65, 257, 1000, 2048, 5000, 8192, 33000}) {
      for (double sig : {0.05, 1.0, 4.0}) {
        // softmax exponentials, their sum, the probabilities sorted
        // descending, their quad sums and mass stops
        std::vector<float> l(n), e(n);
        float mx = -1e30f;
        for (int i = 0; i < n; ++i) {
          l[i] = (float)(sig * nd(rng));
          if (l[i] > mx) mx = l[i];
        }
        for (int i = 0; i < n; ++i) e[i] = std::exp(l[i] - mx);
        check(e, 0.0f, inf, "softmax sum");
        const float sv = chain(e, 0.0f, inf).s, inv = 1.0f / sv;
        std::vector<float> p(n);
        for (int i = 0; i < n; ++i) p[i] = e[i] * inv;
        std::sort(p.begin(), p.end(), [](float a, float b) { return a > b; });
        std::vector<float> q(n / 4);
        for (int k = 0; k < n / 4; ++k) q[k] = ((p[4 * k] + p[4 * k + 1]) + p[4 * k + 2]) + p[4 * k + 3];
        for (float vm : {0.5f, 0.95f, 0.999f, 0.9999f, 1.0f, 2.0f}) check(q, 0.0f, vm, "mass quads");
        // stops at values the chain reaches exactly
        std::vector<float> reach;
        float m = 0.0f;
        for (float t : q) {
          m = m + t;
          reach.push_back(m);
        }
        for (int k = 0; k < 4 && !reach.empty(); ++k)
          check(q, 0.0f, reach[(size_t)(ud(rng) * reach.size()) % reach.size()], "mass at a reached value");
        check(p, 0.0f, 0.95f, "mass singles");
      }
    }
    // tie-heavy: exact small integers and dyadic fractions over large sums
    for (int n : {300, 4000, 40000}) {
      std::vector<float> t(n);
      for (int i = 0; i < n; ++i) t[i] = (float)(1 + (rng() % 3));
      check(t, 16777216.0f, inf, "integers over 2^24");
      check(t, 8388608.0f, inf, "integers over 2^23");
      for (int i = 0; i < n; ++i) t[i] = std::ldexp(1.0f, -(int)(rng() % 4));
      check(t, 4194304.0f, inf, "dyadic over 2^22");
      check(t, 0.0f, inf, "dyadic from 0");
      for (int i = 0; i < n; ++i) t[i] = 0.5f + (float)(rng() % 4) * 0.25f;
      check(t, 0.0f, (float)n * 0.6f, "dyadic with a stop");
      // subnormals and zeros
      for (int i = 0; i < n; ++i) t[i] = bfloat((uint32_t)(rng() % 0x800000u));
      check(t, 0.0f, inf, "subnormals");
      for (int i = 0; i < n; ++i) t[i] = (rng() % 3 == 0) ? -0.0f : (rng() % 2 ? 0.0f : 1e-38f);
      check(t, 0.0f, inf, "zeros and -0");
      // wide exponent range
      for (int i = 0; i < n; ++i) t[i] = std::ldexp((float)(0.5 + 0.5 * ud(rng)), (int)(rng() % 120) - 60);
      check(t, 0.0f, inf, "wide range");
      check(t, 1.0f, 3.0e17f, "wide range with a stop");
      // uniform terms with a non-zero start
      for (int i = 0; i < n; ++i) t[i] = (float)ud(rng);
      check(t, 123.456f, inf, "uniform from 123.456");
      check(t, 0.0f, (float)n * 0.25f, "uniform with a stop");
    }
  }
  std::printf("%lld cases, %lld mismatches\n", g_cases, g_bad);
  std::printf("per thread: %lld sums, %lld segments, %lld redone, %lld stops inside a clean part\n",
              g_wcases, g_wsegs, g_wredo, g_wclean_stop);
  return g_bad == 0 ? 0 : 1;
}
