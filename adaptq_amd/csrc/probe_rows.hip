// probe_rows.hip -- the bulk append's memory traffic without its codec, for
// the measurement of what bounds that kernel (a separate timing library,
// `python -m adaptq_amd.build --probes`; never part of libadaptq.so).
//
// Each kernel reads n_rows input rows of 128 floats (512 B, one config-5 K or
// V vector each) and, unless it reads only, writes NB bytes per row (64: a
// 4-bit row at padded 128, 32: a 2-bit row), with the codec replaced by an
// XOR fold of the row's words, so the time is that of the traffic alone.
//   mode 0: the append kernel's own pattern: load_wave_rows (16-byte chunks
//           by 4-lane groups, two permlane exchange stages), then one row per
//           lane left as 16-byte stores at NB-byte stride
//   mode 1: the same bytes read and written linearly: load j of a wave covers
//           1 KB of consecutive input bytes, store j 1 KB of consecutive
//           output bytes (no exchange; the fold is of other rows' bytes)
//   mode 2: mode 1's reads only (a store that never happens keeps them)
// Launch shape as the append kernel's: 128-thread blocks, 3 waves per SIMD.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rows.hpp"

namespace aq {
namespace {

constexpr int kP = 128;
constexpr int kRB = 4 * kP;

template <int MODE, int NB>
__global__ __launch_bounds__(128, 3) void probe_rows_kernel(const float *__restrict__ src,
                                                            uint8_t *__restrict__ dst,
                                                            long long n_rows) {
  const int lane = threadIdx.x & 63;
  const long long t0 = (long long)blockIdx.x * 128 + (threadIdx.x & ~63);
  if (t0 + 64 > n_rows) return;  // whole waves only (the host passes a multiple of 128)
  const char *rows = reinterpret_cast<const char *>(src + t0 * kP);
  float buf[kP];
  if constexpr (MODE == 0) {
    load_wave_rows<kP>(src + t0 * kP, lane, buf);
  } else {
#pragma unroll
    for (int j = 0; j < kP / 4; ++j) {
      const uint4 x = *reinterpret_cast<const uint4 *>(rows + (uint32_t)(j * 1024 + lane * 16));
      buf[4 * j] = __uint_as_float(x.x);
      buf[4 * j + 1] = __uint_as_float(x.y);
      buf[4 * j + 2] = __uint_as_float(x.z);
      buf[4 * j + 3] = __uint_as_float(x.w);
    }
  }
  constexpr int NW = NB / 4, PER = kP / NW;
  uint32_t o[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    uint32_t a = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) a ^= __float_as_uint(buf[PER * j + q]) >> (q & 3);
    o[j] = a;
  }
  if constexpr (MODE == 2) {
    uint32_t a = 0;
#pragma unroll
    for (int j = 0; j < NW; ++j) a ^= o[j];
    if (a == 0x9E3779B9u) reinterpret_cast<uint32_t *>(dst)[t0 + lane] = a;
  } else if constexpr (MODE == 0) {
    uint4 *d = reinterpret_cast<uint4 *>(dst + (t0 + lane) * NB);
#pragma unroll
    for (int j = 0; j < NB / 16; ++j) d[j] = make_uint4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
  } else {
    uint8_t *d = dst + t0 * NB;
#pragma unroll
    for (int j = 0; j < NB / 16; ++j)
      *reinterpret_cast<uint4 *>(d + (uint32_t)(j * 1024 + lane * 16)) =
          make_uint4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
  }
}

template <int MODE, int NB>
hipError_t launch(const float *src, uint8_t *dst, long long n_rows, hipStream_t s) {
  probe_rows_kernel<MODE, NB><<<dim3((unsigned)(n_rows / 128)), 128, 0, s>>>(src, dst, n_rows);
  return hipGetLastError();
}

}  // namespace
}  // namespace aq

// mode 0-2 as above; nb 64 or 32; n_rows a positive multiple of 128 below
// 2^31 * 128; src holds n_rows * 512 bytes, dst n_rows * nb.  Returns 0, or
// -1 for arguments outside these (nothing launched), or the HIP error.
extern "C" int adaptq_probe_rows(int mode, int nb, const float *src, void *dst, long long n_rows,
                                 void *stream) {
  if (n_rows <= 0 || n_rows % 128 != 0 || n_rows / 128 > 0x7FFFFFFFLL || !src || !dst) return -1;
  hipStream_t s = (hipStream_t)stream;
  uint8_t *d = (uint8_t *)dst;
  hipError_t e;
  if (nb == 64) {
    e = mode == 0 ? aq::launch<0, 64>(src, d, n_rows, s)
        : mode == 1 ? aq::launch<1, 64>(src, d, n_rows, s)
        : mode == 2 ? aq::launch<2, 64>(src, d, n_rows, s)
                    : hipErrorInvalidValue;
  } else if (nb == 32) {
    e = mode == 0 ? aq::launch<0, 32>(src, d, n_rows, s)
        : mode == 1 ? aq::launch<1, 32>(src, d, n_rows, s)
        : mode == 2 ? aq::launch<2, 32>(src, d, n_rows, s)
                    : hipErrorInvalidValue;
  } else {
    return -1;
  }
  if (e == hipErrorInvalidValue && (mode < 0 || mode > 2)) return -1;
  return (int)e;
}
