// device.hpp -- data layout shared by the host C ABI and the gfx950 kernels.
//
// One attention head ("context") owns, in device HBM:
//   k_codes [cap][k_pb] u8   packed K codes, reference bytes; for 2/4-bit K at
//                            padded 64/128 the bytes of slot s are stored in
//                            XOR order (kperm_mask below)
//   v_codes [cap][v_pb] u8   packed V codes       (cache/ring_buffer.cpp:47-84)
//   k_scale [cap] f32, v_scale [cap] f32          L2 norms (1.0 for bits=16)
//   raw_k/raw_v [hyb][dim] f32                    hybrid mirror (attention.cpp:356-365)
//   signs   [padded/32] u32                       Rademacher D as a bit mask
//   desc    HeadDesc                              pointers + config + ring state
// With bits = 16 a "code row" is padded fp32 (k_pb = 4 * padded).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "codebook.hpp"

namespace aq {

constexpr int kMaxPadded = 1024;
constexpr int kMaxSignWords = kMaxPadded / 32;

// Mutable ring state.  The host keeps its own copy for API return values; the
// device copy is what kernels read, advanced by commit kernels in stream order.
struct RingState {
  int head;       // next slot to write
  int size;       // valid tokens
  int raw_count;  // tokens in the hybrid mirror
  int pad_;
};

struct HeadDesc {
  uint8_t *k_codes;
  uint8_t *v_codes;
  float *k_scale;
  float *v_scale;
  float *raw_k;
  float *raw_v;
  uint32_t *signs;  // bit i set <=> D[i] = +1
  int dim, padded, k_bits, v_bits, k_pb, v_pb, cap, hyb;
  float v_mass;
  int pad_[3];
  RingState st;
};

__host__ __device__ inline int packed_bytes(int padded, int bits) {
  return bits == 16 ? padded * 4 : (padded * bits + 7) / 8;
}

// K rows of 2/4-bit codes at padded 64 or 128 are stored with their bytes
// permuted per slot: stored[j ^ (slot & mask)] = reference[j], with mask =
// min(row bytes, 32) - 1 (0 = unpermuted).  Decode gives lane l the token of
// slot l mod 64, so at any static byte position the 32 lanes of a half-wave
// read 32 different byte positions of their rows; the K lookup table keeps
// position jj in LDS bank jj, and its reads are conflict-free.  The byte
// values are the reference's; adaptq_read_slots returns them in reference
// order.
__host__ __device__ constexpr int kperm_mask(int padded, int bits) {
  return (bits == 2 || bits == 4) && (padded == 64 || padded == 128)
             ? ((padded * bits / 8) < 32 ? (padded * bits / 8) : 32) - 1
             : 0;
}

// State after appending n tokens starting from s, restating
// cache/ring_buffer.cpp:105-119 (insert) and attention.cpp:354-365 (mirror):
// the mirror takes tokens while the ring has not evicted and holds fewer than
// hyb vectors, and is emptied for good by the first eviction.
__host__ __device__ inline RingState ring_after(RingState s, int n, int cap, int hyb) {
  RingState r = s;
  if (n <= 0) return r;
  if (cap > 0) {
    r.head = (int)(((long long)s.head + n) % cap);
    long long sz = (long long)s.size + n;
    r.size = sz > cap ? cap : (int)sz;
  }
  if (hyb > 0) {
    bool evicts = (long long)s.size + n > cap;
    if (evicts) {
      r.raw_count = 0;
    } else {
      int room = hyb - s.raw_count;
      int m = n < room ? n : room;
      r.raw_count = s.raw_count + (m > 0 ? m : 0);
    }
  }
  return r;
}

// Number of leading tokens of an n-token append that enter the mirror
// (0 when the batch evicts, since the mirror then ends empty).
__host__ __device__ inline int mirror_count(RingState s, int n, int cap, int hyb) {
  if (hyb <= 0 || (long long)s.size + n > cap) return 0;
  int room = hyb - s.raw_count;
  int m = n < room ? n : room;
  return m > 0 ? m : 0;
}

}  // namespace aq
