// rows.hpp -- the bulk append's load of a wave's 64 input rows (shared by
// the append kernel and the load-pattern probe).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aq {

// The 64 consecutive rows of a wave (P floats each), loaded 64 bytes of a row
// per group of lanes.  Lanes form 16 groups of 4 members: lane bits 4 and 5
// are the member index i, bits 0-3 the group, and member i owns row lane.  For
// each 64-byte block of the rows, load r has every member of a group read its
// 16-byte chunk i of member r's row, so a group reads half a line per load
// instead of each lane touching a line of its own.  Two exchange stages then
// give every lane its own row's chunks in order (a 4 x 4 transpose of 16-byte
// chunks): at the stage over member bit m, slot s of member i trades with
// slot s ^ m of member i ^ m when bit m of s differs from bit m of i; member
// bit 0 is lane ^ 16 and bit 1 lane ^ 32, one permlane16/permlane32 swap per
// slot pair and word (the odd rows of a swap's first operand trade with the
// even rows of its second).  Measured on config 5's rows: 4 % faster than one
// row per lane; 8-member groups (whole lines, a third stage by DPP) cost more
// VALU than they save.  Every lane of the wave must be active.
template <int P>
__device__ __forceinline__ void load_wave_rows(const float *wave_rows, int lane, float (&buf)[P]) {
  constexpr int RB = P * 4;
  const int i = (lane >> 4) & 3;
  const uint32_t base = (uint32_t)(lane & 15) * RB + (uint32_t)i * 16;
  const char *src = reinterpret_cast<const char *>(wave_rows);
#pragma unroll
  for (int blk = 0; blk < P / 16; ++blk) {
    uint32_t v[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint4 x =
          *reinterpret_cast<const uint4 *>(src + base + (uint32_t)(16 * r * RB + blk * 64));
      v[r][0] = x.x;
      v[r][1] = x.y;
      v[r][2] = x.z;
      v[r][3] = x.w;
    }
#pragma unroll
    for (int s = 0; s < 4; s += 2)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const auto r = __builtin_amdgcn_permlane16_swap(v[s][w], v[s + 1][w], false, false);
        v[s][w] = r[0];
        v[s + 1][w] = r[1];
      }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const auto r = __builtin_amdgcn_permlane32_swap(v[s][w], v[s + 2][w], false, false);
        v[s][w] = r[0];
        v[s + 2][w] = r[1];
      }
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int w = 0; w < 4; ++w) buf[16 * blk + 4 * k + w] = __uint_as_float(v[k][w]);
  }
}

}  // namespace aq
