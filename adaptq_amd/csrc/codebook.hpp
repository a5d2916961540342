// codebook.hpp -- the quantisation codebooks and decision thresholds.
//
// Plain C++ usable by the gfx950 kernels and by host code (a host compiler
// sees AQ_HD as nothing), so host-side tests can check the quantisers
// exhaustively.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define AQ_HD __host__ __device__
#else
#define AQ_HD
#endif

namespace aq {

// Lloyd-Max N(0,1) codebooks (core/codebook.cpp:32-62).  These literal
// tables are the quantisation format, so they equal the reference's.
struct CB {
  static constexpr float b2[4] = {-1.5104f, -0.4528f, 0.4528f, 1.5104f};
  static constexpr float b3[8] = {-2.1529f, -1.3439f, -0.7560f, -0.2451f,
                                  0.2451f,  0.7560f,  1.3439f,  2.1529f};
  static constexpr float b4[16] = {-2.4008f, -1.8944f, -1.5105f, -1.2016f,
                                   -0.9138f, -0.6402f, -0.3795f, -0.1258f,
                                   0.1258f,  0.3795f,  0.6402f,  0.9138f,
                                   1.2016f,  1.5105f,  1.8944f,  2.4008f};
};

template <int B>
AQ_HD constexpr float cb(int i) {
  return B == 2 ? CB::b2[i] : B == 3 ? CB::b3[i] : CB::b4[i];
}

// Decision threshold k (between centroids k and k+1): the float expression
// (c[k] + c[k+1]) * 0.5f, exactly 0 at the centre (codebook.cpp:67-100).
// Evaluated at compile time with IEEE round-to-nearest, as the reference's
// static initialisers are.
template <int B>
AQ_HD constexpr float thr(int k) {
  return k == (1 << B) / 2 - 1 ? 0.0f : (cb<B>(k) + cb<B>(k + 1)) * 0.5f;
}

}  // namespace aq
