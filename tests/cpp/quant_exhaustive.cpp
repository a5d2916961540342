// Every float bit pattern: the 4-bit cell quantiser quantize_g4 (with the NaN
// code put in front, as the wide append kernel does) and the sign-split
// quantisers quantize_ss2/3 (adaptq_amd/csrc/quant.hpp, the append kernels') against
// quantize<B> (the reference's binary search restated) and, on a stride,
// against the oracle's quantize_fast; then quantize_bd2 against quantize<2>
// of the twice-rounded scaled value for every padded size up to 128.  The sign-split forms are defined for
// finite inputs (the kernel gives NaN vectors their code as a whole), so NaN
// patterns are skipped for them.  Prints the mismatch count; exits 0 when it
// is 0.
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../adaptq_amd/csrc/quant.hpp"

extern "C" int orc_quantize_fast(float v, int bits);

int main() {
  constexpr aq::Q4Table tab = aq::q4_table();
  // the end cells, which take every value beyond them, hold no threshold
  if (tab.c[0].n != 0 || tab.c[0].t == tab.c[0].t || tab.c[aq::kQ4Cells - 1].n != 15 ||
      tab.c[aq::kQ4Cells - 1].t == tab.c[aq::kQ4Cells - 1].t) {
    std::printf("end cells hold a threshold\n");
    return 1;
  }
  std::atomic<unsigned long long> bad{0};
  const int T = 8;
  std::vector<std::thread> pool;
  for (int w = 0; w < T; ++w)
    pool.emplace_back([&, w] {
      const uint64_t lo = ((uint64_t)w << 32) / T, hi = ((uint64_t)(w + 1) << 32) / T;
      for (uint64_t x = lo; x < hi; ++x) {
        const uint32_t u = (uint32_t)x;
        float v;
        std::memcpy(&v, &u, 4);
        const uint32_t a = v != v ? 7u : aq::quantize_g4(v, tab.c), b = aq::quantize<4>(v);
        bool wrong = a != b;
        if ((u & 0xFFF) == 0x5A5) wrong = wrong || (int)b != orc_quantize_fast(v, 4);
        if (v == v) {
          wrong = wrong || aq::quantize_ss3(v) != aq::quantize<3>(v);
          wrong = wrong || aq::quantize_ss2(v) != aq::quantize<2>(v);
        }
        if (wrong && bad.fetch_add(1) < 10)
          std::printf("mismatch bits=%08x v=%g g4=%u search=%u ss3=%u/%u ss2=%u/%u\n", u, v,
                      a, b, aq::quantize_ss3(v), aq::quantize<3>(v),
                      aq::quantize_ss2(v), aq::quantize<2>(v));
      }
    });
  for (auto &t : pool) t.join();
  std::printf("checked 4294967296 mismatches %llu\n", bad.load());
  if (bad.load() != 0) return 1;

  // The 2-bit b-domain quantiser of the lane-per-vector append kernel
  // (quantize_bd2) against quantize<2> of the value the reference codes,
  // v = fl(fl(b * c) * d), for every finite float b and every padded size that
  // kernel serves (c, d as its launch computes them).
  for (int p = 1; p <= 128; p *= 2) {
    const float d = sqrtf((float)p), c = 1.0f / d;
    const aq::BdThr bt = aq::bd_thresholds(c, d);
    std::atomic<unsigned long long> bad_p{0};
    std::vector<std::thread> pp;
    for (int w = 0; w < T; ++w)
      pp.emplace_back([&, w] {
        const uint64_t lo = ((uint64_t)w << 32) / T, hi = ((uint64_t)(w + 1) << 32) / T;
        for (uint64_t x = lo; x < hi; ++x) {
          const uint32_t u = (uint32_t)x;
          float b;
          std::memcpy(&b, &u, 4);
          if (b != b) continue;
          const float y = b * c;
          const float v = y * d;
          const uint32_t r2 = aq::quantize<2>(v);
          const uint32_t g2 = aq::quantize_bd2(b, bt.q2[0], bt.q2[1], bt.q2[2]);
          if (g2 != r2 && bad_p.fetch_add(1) < 10)
            std::printf("p=%d mismatch bits=%08x b=%g v=%g bd2=%u/%u\n", p, u, b, v, g2, r2);
        }
      });
    for (auto &t : pp) t.join();
    std::printf("p=%d b-domain checked mismatches %llu\n", p, bad_p.load());
    if (bad_p.load() != 0) return 1;
  }
  return 0;
}
