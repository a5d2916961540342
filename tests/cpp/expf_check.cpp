// Every float in [-104, 89] (and the specials): aq::expf_ref
// (adaptq_amd/csrc/expf_ref.hpp, the sparse-V kernels' exponential, built
// here for the host) against the host libm's expf, bit for bit.  Prints the
// mismatch count; exits 0 when it is 0.
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../adaptq_amd/csrc/expf_ref.hpp"

static uint32_t bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

int main() {
  std::atomic<unsigned long long> bad{0}, n{0};
  const uint32_t neg_end = bits(-104.0f), pos_end = bits(89.0f);
  const int T = 8;
  std::vector<std::thread> pool;
  for (int w = 0; w < T; ++w)
    pool.emplace_back([&, w] {
      unsigned long long b = 0, c = 0;
      auto one = [&](uint32_t u) {
        float x;
        std::memcpy(&x, &u, 4);
        const float a = std::exp(x), r = aq::expf_ref(x);
        ++c;
        if (bits(a) != bits(r) && !(a != a && r != r)) {
          if (b < 4) std::printf("x=%a libm=%a expf_ref=%a\n", x, a, r);
          ++b;
        }
      };
      for (uint64_t u = 0x80000000u + w; u <= neg_end; u += T) one((uint32_t)u);
      for (uint64_t u = w; u <= pos_end; u += T) one((uint32_t)u);
      bad += b;
      n += c;
    });
  for (auto &t : pool) t.join();
  const float specials[] = {-INFINITY, INFINITY, NAN, -200.0f, 200.0f, -103.97f, 88.73f};
  for (float x : specials) {
    const float a = std::exp(x), r = aq::expf_ref(x);
    if (bits(a) != bits(r) && !(a != a && r != r)) {
      std::printf("special x=%a libm=%a expf_ref=%a\n", x, a, r);
      ++bad;
    }
  }
  std::printf("checked %llu floats, %llu mismatches\n", (unsigned long long)n.load(),
              (unsigned long long)bad.load());
  return bad == 0 ? 0 : 1;
}
