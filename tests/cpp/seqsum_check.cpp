// The segment algorithm of block_seq_sum (adaptq_amd/csrc/seqsum.hpp) run on
// the host, one chunk at a time exactly as the block runs it (fp64 prefix,
// per-thread, one-edge and per-term classes and integer increments from
// seqsum_terms.hpp, segment heads, the walk with its runs of hardware terms,
// checks, serial redo and serial tail beyond the segment table, the stop
// search inside a clean segment), against the plain left-to-right fp32
// chain with its stop test.  Sequences: softmax-like exponentials, sorted
// probabilities and their quad sums with mass stops (also stops equal to a
// value the chain reaches), tie-heavy terms (exact small integers and dyadic
// fractions over large sums), subnormals, wide exponent ranges, zeros and
// -0, and non-zero start values; 1 to 8 terms per thread (chunks of 1,024 to
// 8,192 terms).  Prints the mismatch count and the share of chunks redone;
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

static long long g_chunks = 0, g_redo = 0, g_tail = 0;

// The block algorithm, serially: chunks of kBlock threads x T terms (C =
// kBlock T), each thread's run classified as one (range_class) or term by
// term, runs of hardware terms as one segment.
static Res model(const std::vector<float> &x, float s, float stop, int T) {
  const int n = (int)x.size(), C = kBlock * T;
  if (n <= kSerialMax) return chain(x, s, stop);
  for (int c0 = 0;; c0 += C) {
    if (!(s < stop) || c0 >= n) return {c0 < n ? c0 : n, s};
    const int cn = n - c0 < C ? n - c0 : C;
    ++g_chunks;
    std::vector<int> cls(cn);
    std::vector<uint32_t> r(cn);
    double P = (double)s;  // the prefix before each thread's run (the block's
                           // scan associates differently; the bounds cover it)
    for (int j0 = 0; j0 < cn; j0 += T) {
      const int nv = cn - j0 < T ? cn - j0 : T;
      double loc = 0.0;
      for (int k = 0; k < nv; ++k) loc += (double)x[c0 + j0 + k];
      const int u = range_class(P, loc, j0 + nv);
      const int E = u == kUnc ? edge_of(P, loc, j0 + nv) : kUnc;
      const double del = range_del(P, loc, j0 + nv);
      double Pj = P;
      for (int k = 0; k < nv; ++k) {
        const float xj = x[c0 + j0 + k];
        int c;
        uint32_t rj = 0u;
        if (u != kUnc) {
          c = scaled_incr(xj, u, rj) ? u : kUnc;
        } else if (E != kUnc) {
          c = split_class(Pj, (double)xj, del, E);
          if (c != kUnc && !scaled_incr(xj, c, rj)) c = kUnc;
        } else {
          c = term_class(Pj, xj, j0 + k);
          if (c != kUnc && !term_incr(xj, c, rj)) c = kUnc;
        }
        cls[j0 + k] = c;
        r[j0 + k] = c == kUnc ? 0u : rj;
        Pj += (double)xj;
      }
      P += loc;
    }
    // segments: a head wherever the class changes
    std::vector<int> seg_start, seg_cls;
    std::vector<uint64_t> seg_r;
    uint64_t R = 0;
    int pc = kNoClass;
    for (int j = 0; j < cn; ++j) {
      if (cls[j] != pc) {
        seg_start.push_back(c0 + j);
        seg_cls.push_back(cls[j]);
        seg_r.push_back(R);
      }
      pc = cls[j];
      R += r[j];
    }
    const int ns_all = (int)seg_start.size(), ns = ns_all < kMaxSeg ? ns_all : kMaxSeg;
    seg_start.push_back(c0 + cn);
    seg_r.push_back(R);
    auto hw_run = [&](int from, int to, float &w) {
      int i = from;
      while (i + 8 <= to) {
        float wn = w;
        for (int k = 0; k < 8; ++k) wn = wn + x[i + k];
        if (!(wn < stop)) break;
        w = wn;
        i += 8;
      }
      for (; i < to; ++i) {
        if (!(w < stop)) return i;
        w = w + x[i];
      }
      return -1;
    };
    // walk: the first kMaxSeg segments, then the rest of the chunk term by term
    float w = s;
    int stop_at = -1, stop_seg = -1, redo = 0;
    for (int k = 0; k < ns && !redo; ++k) {
      const int cl = seg_cls[k];
      if (cl == kUnc) {
        stop_at = hw_run(seg_start[k], seg_start[k + 1], w);
        if (stop_at >= 0) break;
        continue;
      }
      if (!(w < stop)) {
        stop_at = seg_start[k];
        break;
      }
      const uint64_t inc64 = seg_r[k + 1] - seg_r[k];
      const uint32_t inc = inc64 >= kTop ? kTop : (uint32_t)inc64;
      const uint32_t wb = fbits(w), exb = (uint32_t)(cl + 150), nb = wb + inc;
      if ((wb >> 23) != exb || inc >= kTop || (nb >> 23) != exb) {
        redo = 1;
        break;
      }
      if (!(bfloat(nb) < stop)) {
        stop_seg = k;
        break;
      }
      w = bfloat(nb);
    }
    if (redo) {
      ++g_redo;
      w = s;
      stop_seg = -1;
      stop_at = hw_run(c0, c0 + cn, w);
    } else if (ns_all > kMaxSeg && stop_at < 0 && stop_seg < 0) {
      ++g_tail;
      stop_at = hw_run(seg_start[kMaxSeg], c0 + cn, w);
    }
    if (stop_seg >= 0) {
      const int lo = seg_start[stop_seg], hi = seg_start[stop_seg + 1];
      const int eu = seg_cls[stop_seg];
      const uint64_t r_lo = seg_r[stop_seg];
      const uint32_t K0 = (fbits(w) & 0x7FFFFFu) | 0x800000u, kst = kstop_of(stop, eu);
      int at = hi;
      uint64_t Rb = r_lo;
      for (int i = lo; i < hi; ++i) {
        if (i > lo && (uint64_t)K0 + (Rb - r_lo) >= (uint64_t)kst) {
          at = i;
          break;
        }
        Rb += r[i - c0];
      }
      if (at == hi) Rb = seg_r[stop_seg + 1];
      w = std::ldexp((float)(K0 + (uint32_t)(Rb - r_lo)), eu);
      stop_at = at;
    }
    s = w;
    if (stop_at >= 0) return {stop_at, s};
  }
}

static long long g_gchunks = 0, g_gredo = 0, g_gtail = 0;

// The pre-classified path of the sparse-V softmax sum (sparse.hip:
// sparse_sum_classify_kernel, then seq_walk_flat in the select kernel), with
// no stop: chunks of kBlock T terms classified from the fp64 prefix of every
// term before them (not the exact sum at the chunk) with the bound counting
// the terms since the sum's start; each chunk's flat list holds its first
// kMaxSeg segments and then the rest of the chunk as one hardware segment;
// windows of W chunks are walked together, a failed check redoing the whole
// window term by term.  bias != 1 scales the prefix, a planted misprediction
// that the walk's checks must catch (the redo then gives the chain's sum).
static float model_global(const std::vector<float> &x, int T, int W, double bias = 1.0) {
  const int n = (int)x.size(), C = kBlock * T;
  struct Ent {
    int start, cls;
    uint32_t inc;
  };
  std::vector<std::vector<Ent>> lists;
  double Pc = 0.0;  // fp64 prefix before the chunk
  for (int c0 = 0; c0 < n; c0 += C) {
    const int cn = n - c0 < C ? n - c0 : C;
    ++g_gchunks;
    std::vector<int> cls(cn);
    std::vector<uint32_t> r(cn);
    double P = Pc * bias;
    for (int j0 = 0; j0 < cn; j0 += T) {
      const int nv = cn - j0 < T ? cn - j0 : T;
      const int jb = c0 + j0;  // terms since the sum's start
      double loc = 0.0;
      for (int k = 0; k < nv; ++k) loc += (double)x[c0 + j0 + k];
      const int u = range_class(P, loc, jb + nv);
      const int E = u == kUnc ? edge_of(P, loc, jb + nv) : kUnc;
      const double del = range_del(P, loc, jb + nv);
      double Pj = P;
      for (int k = 0; k < nv; ++k) {
        const float xj = x[c0 + j0 + k];
        int c;
        uint32_t rj = 0u;
        if (u != kUnc) {
          c = scaled_incr(xj, u, rj) ? u : kUnc;
        } else if (E != kUnc) {
          c = split_class(Pj, (double)xj, del, E);
          if (c != kUnc && !scaled_incr(xj, c, rj)) c = kUnc;
        } else {
          c = term_class(Pj, xj, jb + k);
          if (c != kUnc && !term_incr(xj, c, rj)) c = kUnc;
        }
        cls[j0 + k] = c;
        r[j0 + k] = c == kUnc ? 0u : rj;
        Pj += (double)xj;
      }
      P += loc;
    }
    for (int j = 0; j < cn; ++j) Pc += (double)x[c0 + j];  // the true prefix
    std::vector<Ent> L;
    int pc = kNoClass;
    uint64_t R = 0, Rseg = 0;
    for (int j = 0; j < cn; ++j) {
      if (cls[j] != pc) {
        if (!L.empty()) {
          const uint64_t d = R - Rseg;
          L.back().inc = d >= kTop ? kTop : (uint32_t)d;
        }
        L.push_back({c0 + j, cls[j], 0u});
        Rseg = R;
      }
      pc = cls[j];
      R += r[j];
    }
    {
      const uint64_t d = R - Rseg;
      L.back().inc = d >= kTop ? kTop : (uint32_t)d;
    }
    if ((int)L.size() > kMaxSeg) {
      ++g_gtail;
      const int st = L[kMaxSeg].start;
      L.resize(kMaxSeg);
      L.push_back({st, kUnc, 0u});
    }
    lists.push_back(L);
  }
  float s = 0.0f;
  for (size_t c = 0; c < lists.size(); c += (size_t)W) {
    const int w0 = (int)c * C, w1 = std::min(n, (int)(c + W) * C);
    std::vector<Ent> L;
    for (size_t h = c; h < c + W && h < lists.size(); ++h) L.insert(L.end(), lists[h].begin(), lists[h].end());
    uint32_t wb = fbits(s);
    bool redo = false;
    for (size_t k = 0; k < L.size(); ++k) {
      const int end = k + 1 < L.size() ? L[k + 1].start : w1;
      if (L[k].cls == kUnc) {
        float w = bfloat(wb);
        for (int i = L[k].start; i < end; ++i) w = w + x[i];
        wb = fbits(w);
        continue;
      }
      const bool ok = (wb >> 23) == (uint32_t)(L[k].cls + 150) && (wb & 0x7FFFFFu) + L[k].inc < 0x800000u;
      if (!ok) redo = true;
      else wb += L[k].inc;
    }
    if (redo) {
      ++g_gredo;
      float w = s;
      for (int i = w0; i < w1; ++i) w = w + x[i];
      wb = fbits(w);
    }
    s = bfloat(wb);
  }
  return s;
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

static long long g_cases = 0, g_bad = 0;

// No stop: the pre-classified path of the softmax sum against the chain.
static void check_global(const std::vector<float> &x, const char *what) {
  const Res a = chain(x, 0.0f, INFINITY);
  for (int T : {2, 8})
    for (double bias : {1.0, 1.05}) {
      const float b = model_global(x, T, T == 2 ? 4 : 1, bias);
      ++g_cases;
      if (fbits(a.s) != fbits(b)) {
        if (g_bad < 10)
          std::printf("MISMATCH (pre-classified) %s n=%zu T=%d bias=%g: chain %a model %a\n", what,
                      x.size(), T, bias, (double)a.s, (double)b);
        ++g_bad;
      }
    }
}

static void check(const std::vector<float> &x, float s0, float stop, const char *what) {
  const Res a = chain(x, s0, stop);
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
  for (int T : {8, 4, 2, 1}) {
    const Res b = model(x, s0, stop, T);
    ++g_cases;
    if (a.count != b.count || fbits(a.s) != fbits(b.s)) {
      if (g_bad < 10)
        std::printf("MISMATCH %s n=%zu T=%d stop=%a: chain (%d, %a) model (%d, %a)\n", what,
                    x.size(), T, (double)stop, a.count, (double)a.s, b.count, (double)b.s);
      ++g_bad;
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
        check_global(e, "softmax sum");
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
      check_global(t, "small integers");
      check(t, 8388608.0f, inf, "integers over 2^23");
      for (int i = 0; i < n; ++i) t[i] = std::ldexp(1.0f, -(int)(rng() % 4));
      check(t, 4194304.0f, inf, "dyadic over 2^22");
      check(t, 0.0f, inf, "dyadic from 0");
      check_global(t, "dyadic");
      for (int i = 0; i < n; ++i) t[i] = 0.5f + (float)(rng() % 4) * 0.25f;
      check(t, 0.0f, (float)n * 0.6f, "dyadic with a stop");
      // subnormals and zeros
      for (int i = 0; i < n; ++i) t[i] = bfloat((uint32_t)(rng() % 0x800000u));
      check(t, 0.0f, inf, "subnormals");
      check_global(t, "subnormals");
      for (int i = 0; i < n; ++i) t[i] = (rng() % 3 == 0) ? -0.0f : (rng() % 2 ? 0.0f : 1e-38f);
      check(t, 0.0f, inf, "zeros and -0");
      check_global(t, "zeros and -0");
      // wide exponent range
      for (int i = 0; i < n; ++i) t[i] = std::ldexp((float)(0.5 + 0.5 * ud(rng)), (int)(rng() % 120) - 60);
      check(t, 0.0f, inf, "wide range");
      check_global(t, "wide range");
      check(t, 1.0f, 3.0e17f, "wide range with a stop");
      // uniform terms with a non-zero start
      for (int i = 0; i < n; ++i) t[i] = (float)ud(rng);
      check(t, 123.456f, inf, "uniform from 123.456");
      check_global(t, "uniform");
      check(t, 0.0f, (float)n * 0.25f, "uniform with a stop");
    }
  }
  std::printf("%lld cases, %lld mismatches, %lld of %lld chunks redone, %lld with a serial tail; "
              "pre-classified: %lld windows redone, %lld of %lld chunks past %d segments\n",
              g_cases, g_bad, g_redo, g_chunks, g_tail, g_gredo, g_gtail, g_gchunks, kMaxSeg);
  std::printf("per thread: %lld sums, %lld segments, %lld redone, %lld stops inside a clean part\n",
              g_wcases, g_wsegs, g_wredo, g_wclean_stop);
  return g_bad == 0 ? 0 : 1;
}
