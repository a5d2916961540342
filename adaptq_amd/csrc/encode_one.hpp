// encode_one.hpp -- the one-row codec shared by append_one_kernel (append.hip)
// and the decode step that appends its token first (decode.hip).
//
// One wave encodes one K or V row of one token, lane l holding entries l and
// l + 64, with the float steps of the reference's codec in its order
// (quantizer.cpp:53-101, fwht.cpp:33-66, codebook.cpp:119-144, packing
// quantizer.cpp:156-209): the sum of squares left to right (every lane runs
// the chain over the squares in LDS), the butterflies of span 1, 2, ...
// between lanes (shfl_xor) and, at padded 128, inside the lane; codes are
// gathered in LDS and lane k packs word k of the row; the ring insert and
// the hybrid mirror follow ring_buffer.cpp:105-119 and attention.cpp:338-366.
#pragma once

#include "device.hpp"
#include "quant.hpp"

namespace aq {

// The packed word k of a row whose codes are all the NaN code (1 / 3 / 7 for
// 2 / 3 / 4 bits; codebook.cpp:119-144): 0x55 and 0x77 bytes; 3-bit rows
// repeat the 24-bit group 011 x 8 = bytes 6D B6 DB.
template <int B>
__device__ __forceinline__ uint32_t nan_word(int k) {
  if constexpr (B == 2) return 0x55555555u;
  else if constexpr (B == 4) return 0x77777777u;
  else return k % 3 == 0 ? 0x6DDBB66Du : k % 3 == 1 ? 0xB66DDBB6u : 0xDBB66DDBu;
}

// Token t (of n_tok appended at once, ring state st before them) of head d,
// side 0 (key, KB bits) or 1 (value, VB bits), from the dim floats at x.
// s_sq (P floats) and s_code (P bytes): this wave's LDS scratch; s_q4: the
// 4-bit cell table (q4_table) when KB or VB is 4.  lds_row /
// lds_scale, when not null, receive a copy of the stored row (in its stored
// word order) and scale, for quantised rows.
template <int P, int KB, int VB>
__device__ __forceinline__ void encode_one_row(HeadDesc *d, const RingState st, int n_tok, int t,
                                               const float *__restrict__ x, int dim, int side,
                                               int lane, float inv_sqrt_p, float sqrt_p,
                                               const Q4Cell *s_q4, float *s_sq, uint8_t *s_code,
                                               uint32_t *lds_row, float *lds_scale) {
  constexpr int E = P / 64;
  const int cap = d->cap;
  if (t < mirror_count(st, n_tok, cap, d->hyb)) {
    float *m = (side == 0 ? d->raw_k : d->raw_v) + (size_t)(st.raw_count + t) * dim;
    for (int i = lane; i < dim; i += 64) m[i] = x[i];
  }
  if (cap <= 0 || t < n_tok - cap) return;  // overwritten within this append
  const int slot = (int)(((long long)st.head + t) % cap);
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = lane + 64 * e < dim ? x[lane + 64 * e] : 0.0f;
  const int B = side == 0 ? KB : VB;
  uint8_t *codes = side == 0 ? d->k_codes : d->v_codes;
  float *scales = side == 0 ? d->k_scale : d->v_scale;
  auto seq_sumsq = [&](const float (&u)[E]) {
    // left to right over the P squares (every lane runs the same chain)
#pragma unroll
    for (int e = 0; e < E; ++e) s_sq[lane + 64 * e] = __fmul_rn(u[e], u[e]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float4 *q4 = reinterpret_cast<const float4 *>(s_sq);
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < P / 16; ++b) {
      float4 r[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) r[k] = q4[4 * b + k];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        acc = __fadd_rn(acc, r[k].x);
        acc = __fadd_rn(acc, r[k].y);
        acc = __fadd_rn(acc, r[k].z);
        acc = __fadd_rn(acc, r[k].w);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // s_sq is read by every lane before it is rewritten
    return acc;
  };
  if (B == 16) {
    float *row = reinterpret_cast<float *>(codes + (size_t)slot * 4 * P);
#pragma unroll
    for (int e = 0; e < E; ++e) row[lane + 64 * e] = v[e];
    if (lane == 0) scales[slot] = 1.0f;
    return;  // (no row copy: callers that want one take quantised rows only)
  }
  const float s = seq_sumsq(v);
  const float norm = sqrtf(__fadd_rn(s, 1e-12f));
  const float inv = 1.0f / norm;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int i = lane + 64 * e;
    const uint32_t flip = (~d->signs[i >> 5] >> (i & 31)) << 31;
    v[e] = __uint_as_float(__float_as_uint(__fmul_rn(v[e], inv)) ^ flip);
  }
#pragma unroll
  for (int len = 1; len < 64 && len < P; len <<= 1) {
    const bool upper = (lane & len) != 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float o = __shfl_xor(v[e], len, 64);
      v[e] = upper ? __fsub_rn(o, v[e]) : __fadd_rn(v[e], o);
    }
  }
  if constexpr (E == 2) {
    const float lo = v[0], hi = v[1];
    v[0] = __fadd_rn(lo, hi);
    v[1] = __fsub_rn(lo, hi);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = __fmul_rn(__fmul_rn(v[e], inv_sqrt_p), sqrt_p);
  // the clamp (see encode_vec): inert when s >= 1e-10
  bool nan_row;
  if (s >= 1e-10f) {
    nan_row = __shfl(v[0], 0, 64) != __shfl(v[0], 0, 64);
  } else {
    const float s2 = seq_sumsq(v);
    const float sigma = sqrtf(__fadd_rn(s2 / (float)P, 1e-12f));
    const float clip = __fmul_rn(3.0f, sigma);
#pragma unroll
    for (int e = 0; e < E; ++e) v[e] = __builtin_amdgcn_fmed3f(v[e], -clip, clip);
    nan_row = s2 != s2;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const uint32_t q = B == 4 ? quantize_g4(v[e], s_q4) : B == 3 ? quantize_ss3(v[e]) : quantize_ss2(v[e]);
    s_code[lane + 64 * e] = (uint8_t)q;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int nw = P * B / 32;  // words of the row
  if (lane < nw) {
    const uint8_t *cd = s_code;
    uint32_t w = 0u;
    if (nan_row) {
      w = B == 2 ? nan_word<2>(lane) : B == 4 ? nan_word<4>(lane) : nan_word<3>(lane);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;  // byte b of the row, MSB-first codes
        uint32_t byte;
        if (B == 4) {
          byte = ((uint32_t)cd[2 * b] << 4) | cd[2 * b + 1];
        } else if (B == 2) {
          byte = ((uint32_t)cd[4 * b] << 6) | ((uint32_t)cd[4 * b + 1] << 4) |
                 ((uint32_t)cd[4 * b + 2] << 2) | cd[4 * b + 3];
        } else {
          const int g = b / 3;  // 24-bit big-endian group of 8 codes
          uint32_t grp = 0u;
#pragma unroll
          for (int k = 0; k < 8; ++k) grp |= (uint32_t)cd[8 * g + k] << (21 - 3 * k);
          byte = (grp >> (16 - 8 * (b % 3))) & 255u;
        }
        w |= byte << (8 * j);
      }
    }
    uint32_t *row = reinterpret_cast<uint32_t *>(codes + (size_t)slot * (P * B / 8));
    const uint32_t xm = side == 0 ? (uint32_t)kperm_mask(P, B) : 0u;
    uint32_t at = (uint32_t)lane;
    if (xm != 0u) {
      // the K row's XOR byte order (kperm_mask): word i, bytes permuted by x & 3, at i ^ (x >> 2)
      const uint32_t xx = (uint32_t)slot & xm;
      at ^= xx >> 2;
      w = __builtin_amdgcn_perm(0u, w, 0x03020100u ^ ((xx & 3u) * 0x01010101u));
    }
    row[at] = w;
    if (lds_row) lds_row[at] = w;
  }
  if (lane == 0) {
    scales[slot] = norm;
    if (lds_row) *lds_scale = norm;
  }
}

}  // namespace aq
