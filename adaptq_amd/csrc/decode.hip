// decode.hip -- attention over the packed ring for gfx950 (dense softmax).
//
// What is computed, per (head, query), restating attention.cpp:480-660 with
// v_mass <= 0:
//   quantised K:  qr = H (D . q)  (the reference's rotation, fwht.cpp:33-66,
//                 scaled back by sqrt(p)*||q||, attention.cpp:537-550, is
//                 exactly the unnormalised Hadamard transform of D.q),
//                 logit_t = (sum_i qr_i CB_K[c_ti]) / (sqrt(dim) p) * kscale_t
//   fp32 K (16):  logit_t = (q . k_t) / sqrt(dim)            (:565-580)
//   weights:      softmax over the ring
//   quantised V:  acc = sum_t p_t vscale_t / sqrt(p) CB_V[c_t]  (rotated domain)
//                 out = (H acc / sqrt(p)) . D, first dim entries   (fwht.cpp:106-134)
//   fp32 V (16):  out = sum_t p_t v_t
// Hybrid branch (:491-523) = fp32 K and V read from the raw mirror.
//
// Work split ("flash decoding"): grid = (splits, items).  A block of 4 waves
// takes one contiguous token range of one item; each wave streams 64-token
// tiles with an online softmax; a block writes (max, sum, acc[p]) and the
// finalize kernel merges splits and applies the inverse FWHT.
//
// LUT kernel (padded 64, 128 and 256): one lane per
// token.
//   K: byte lookup table in LDS, LUT[j][b] = the contribution of code byte j
//      with value b (2 codes at 4 bits, 4 at 2 bits, a 6-bit code pair at 3
//      bits), so a token costs one LDS read per code byte; at padded 256 the
//      2- and 4-bit table holds nibbles instead (one read per 4 bits of
//      codes), the byte table being 128 KB there.
//   V: per-lane accumulators acc[p] in VGPRs, fed from a codebook-only table
//      (byte -> 4 floats at 2 bits, byte -> 2 floats at 4 bits, 6-bit pair ->
//      2 floats at 3 bits); reduced across lanes once per block.
// Wide kernel (padded 512 and 1024, quantised K and V): a wave per token, the
// row's dimensions over the lanes, a fixed-point K table per (code,
// dimension).
// Generic kernel (any padded up to 1024): one block-wide reduction per token
// group; used for shapes the other kernels do not cover.
#include <algorithm>

#include "encode_one.hpp"
#include "launch.hpp"

namespace aq {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <int B>
__device__ __forceinline__ float cbv(int i) {
  return cb<B>(i);
}

// Bytes of one ring row.
template <int P, int B>
struct RowBytes {
  static constexpr int value = B == 16 ? 4 * P : (P * B) / 8;
};

// Load NB bytes (NB % 8 == 0) of row `t` into 32-bit words.
template <int NB>
__device__ __forceinline__ void load_row(const uint8_t *base, long long t, uint32_t (&w)[NB / 4]) {
  const uint8_t *p = base + (size_t)t * NB;
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const uint4 v = reinterpret_cast<const uint4 *>(p)[i];
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) {
      const uint2 v = reinterpret_cast<const uint2 *>(p)[i];
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  }
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t *w, int j) {
  return (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
}

// 3-bit rows: code pair m (0..3) of group g as a 6-bit value s_{2m}<<3|s_{2m+1}.
__device__ __forceinline__ uint32_t pair3(const uint32_t *w, int g, int m) {
  const uint32_t w24 = (byte_of(w, 3 * g) << 16) | (byte_of(w, 3 * g + 1) << 8) | byte_of(w, 3 * g + 2);
  return (w24 >> (18 - 6 * m)) & 63u;
}

// K lookup table entries.  2 and 4 bits: byte value b, byte position jj at
// word b * 64 + jj (position jj in LDS bank jj; see kperm_mask); 3 bits:
// code pair m of group g, 6-bit value v at word (4g + m) * 64 + v.
template <int P, int KB>
struct KLut {
  static constexpr int size = (KB == 4 || KB == 2) ? (P <= 128 ? 256 * 64 : (KB == 4 ? P : P / 2) * 16)
                              : KB == 3 ? (P / 2) * 64 : 1;
};
template <int VB>
struct VLut {
  static constexpr int size = VB == 2 ? 32 : VB == 4 ? 16 : VB == 3 ? 8 : 4;
};

// Rotate the query into shared memory.  Quantised K: qr = H (D . q) (butterfly
// stages in place); fp32 K: qr = q.  Padded entries are zero.
template <int P>
__device__ void load_query(float *s_q, const float *q, int dim, bool rotate, const uint32_t *signs) {
  if constexpr (P == 64 || P == 128) {
    // one wave: lane l holds entries l and l + 64, butterflies of span < 64
    // between lanes, span 64 inside the lane (the same additions, no barriers)
    constexpr int E = P / 64;
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      float v[E];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int i = lane + 64 * e;
        v[e] = i < dim ? q[i] : 0.0f;
        if (rotate && !((signs[i >> 5] >> (i & 31)) & 1u)) v[e] = -v[e];
      }
      if (rotate) {
#pragma unroll
        for (int len = 1; len < 64; len <<= 1) {
          const bool upper = (lane & len) != 0;
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const float o = __shfl_xor(v[e], len, 64);
            v[e] = upper ? o - v[e] : v[e] + o;
          }
        }
        if constexpr (E == 2) {
          const float lo = v[0], hi = v[1];
          v[0] = lo + hi;
          v[1] = lo - hi;
        }
      }
#pragma unroll
      for (int e = 0; e < E; ++e) s_q[lane + 64 * e] = v[e];
    }
    __syncthreads();
    return;
  }
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    float v = i < dim ? q[i] : 0.0f;
    if (rotate && !((signs[i >> 5] >> (i & 31)) & 1u)) v = -v;
    s_q[i] = v;
  }
  __syncthreads();
  if (!rotate) return;
  for (int len = 1; len < P; len <<= 1) {
    for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
      const int j = (k / len) * 2 * len + (k % len);
      const float lo = s_q[j], hi = s_q[j + len];
      s_q[j] = lo + hi;
      s_q[j + len] = lo - hi;
    }
    __syncthreads();
  }
}

template <int P, int KB>
__device__ void build_klut(float *lut, const float *qr) {
  if constexpr (KB == 4) {
    constexpr int NB = P / 2;
    for (int e = threadIdx.x; e < NB * 256; e += blockDim.x) {
      const int b = e / NB, j = e % NB;
      lut[b * 64 + j] = qr[2 * j] * cbv<4>(b >> 4) + qr[2 * j + 1] * cbv<4>(b & 15);
    }
  } else if constexpr (KB == 2) {
    constexpr int NB = P / 4;
    for (int e = threadIdx.x; e < NB * 256; e += blockDim.x) {
      const int b = e / NB, j = e % NB;
      lut[b * 64 + j] = (qr[4 * j] * cbv<2>(b >> 6) + qr[4 * j + 1] * cbv<2>((b >> 4) & 3)) +
                        (qr[4 * j + 2] * cbv<2>((b >> 2) & 3) + qr[4 * j + 3] * cbv<2>(b & 3));
    }
  } else if constexpr (KB == 3) {
    for (int e = threadIdx.x; e < (P / 2) * 64; e += blockDim.x) {
      const int j = e >> 6, b = e & 63;
      lut[e] = qr[2 * j] * cbv<3>(b >> 3) + qr[2 * j + 1] * cbv<3>(b & 7);
    }
  }
}

// Fixed-point K table for 2- and 4-bit codes: entry[b][jj] = trunc(f * the
// byte's contribution qr . CB[codes]), f the largest power of two with
// f * max|CB| * sum_i |qr_i| <= 2^29, so every partial sum of a row's lookups
// stays below 2^29 + 64 in magnitude and a row's lookups add in int32, two per
// v_add3_u32.  f being a power of two, an entry is the float table's entry
// scaled exactly, truncated by less than one unit (2^-28 of the bound); the
// 64-term sum is then exact, where a float sum would round at every step.  A
// byte splits into a high half (code pair or code) taken per wave, so its
// codebook index is wave-uniform, and a low half unrolled over compile-time
// codebook entries.
template <int KB>
struct KMaxCode {
  static constexpr float value = KB == 4 ? 2.4008f : 1.5104f;  // max |CB|
};

template <int P, int KB>
__device__ void build_klut_fixed(int32_t *lut, const float *qr, float f) {
  constexpr int NB = P * KB / 8;  // byte positions
  const int j = threadIdx.x & 63;
  const int nw = blockDim.x >> 6;
  if (j >= NB) return;
  float b[16];
  float qa0, qa1 = 0.0f;
  if constexpr (KB == 4) {
    qa0 = qr[2 * j] * f;
    const float qb = qr[2 * j + 1] * f;
#pragma unroll
    for (int lo = 0; lo < 16; ++lo) b[lo] = qb * cbv<4>(lo);
  } else {
    qa0 = qr[4 * j] * f;
    qa1 = qr[4 * j + 1] * f;
    const float qb0 = qr[4 * j + 2] * f, qb1 = qr[4 * j + 3] * f;
#pragma unroll
    for (int lo = 0; lo < 16; ++lo) b[lo] = qb0 * cbv<2>(lo >> 2) + qb1 * cbv<2>(lo & 3);
  }
  for (int hi = threadIdx.x >> 6; hi < 16; hi += nw) {
    const int h = __builtin_amdgcn_readfirstlane(hi);
    const float a = KB == 4 ? qa0 * CB::b4[h] : qa0 * CB::b2[h >> 2] + qa1 * CB::b2[h & 3];
#pragma unroll
    for (int lo = 0; lo < 16; ++lo) lut[(h * 16 + lo) * 64 + j] = (int32_t)(a + b[lo]);
  }
}

// Fixed-point K table of padded 256 and up (2- and 4-bit codes), one entry
// per code unit and nibble value: a unit is a 4-bit code, or a pair of 2-bit
// codes (2u, 2u + 1); byte j of a row holds units 2j (high nibble) and 2j + 1
// (low nibble).  Entry (u, v) = trunc(f * the unit's contribution qr . CB[v])
// with f as in build_klut_fixed, at byte (u >> 2) * 256 + v * 16 + (u & 3) * 4:
// the nibble's own bits, masked with 0xF0, give the register part of the
// address (v * 16, distinct banks for distinct values), and the unit the
// instruction's immediate offset.  All lanes look up the same unit at once.
template <int P, int KB>
__device__ void build_klut_nib(int32_t *lut, const float *qr, float f) {
  constexpr int U = KB == 4 ? P : P / 2;
  for (int e = threadIdx.x; e < U * 16; e += blockDim.x) {
    const int u = e >> 4, v = e & 15;
    float c;
    if constexpr (KB == 4) c = (qr[u] * f) * cbv<4>(v);
    else c = (qr[2 * u] * f) * cbv<2>(v >> 2) + (qr[2 * u + 1] * f) * cbv<2>(v & 3);
    lut[((u >> 2) * 16 + v) * 4 + (u & 3)] = (int32_t)c;
  }
}

// Byte offset of unit u's row in build_klut_nib's table.
__host__ __device__ constexpr int nib_off(int u) { return (u >> 2) * 256 + (u & 3) * 4; }

// Codebook tables for V; distinct entries never share an LDS bank.
// 2-bit: nibble n (two codes) -> float2 at byte 16n; 4-bit: nibble n -> float
// at byte 16n (with a 16-byte stride the high nibble's table offset is its
// own bits, byte & 0xF0); 3-bit: code -> float.
template <int VB>
__device__ void build_vlut(float *lut) {
  if constexpr (VB == 2) {
    for (int b = threadIdx.x; b < 16; b += blockDim.x) {
      lut[4 * b] = cbv<2>(b >> 2);
      lut[4 * b + 1] = cbv<2>(b & 3);
    }
  } else if constexpr (VB == 4) {
    for (int b = threadIdx.x; b < 16; b += blockDim.x) lut[4 * b] = cbv<4>(b);
  } else if constexpr (VB == 3) {
    for (int b = threadIdx.x; b < 8; b += blockDim.x) lut[b] = cbv<3>(b);
  }
}

// Sum over the lanes of a wave of v[0..P) (P >= 64): butterfly reduce-scatter;
// on return lane L holds the totals of entries [L*P/64, (L+1)*P/64) in
// v[0..P/64).
// The halves are chosen with a bit mask rather than a select so the compiler
// cannot turn the choice into a lane-dependent array index (which would move
// v[] to scratch memory).
template <int P>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[P], int lane) {
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const int m = 32 >> step;
    const int half = P >> (step + 1);
    const uint32_t up = (lane & m) ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const uint32_t a = __float_as_uint(v[j]), b = __float_as_uint(v[j + half]);
      const float send = __uint_as_float((a & up) | (b & ~up));
      const float keep = __uint_as_float((b & up) | (a & ~up));
      v[j] = keep + __shfl_xor(send, m, 64);
    }
  }
}

struct ItemView {
  const uint8_t *k_rows;
  const uint8_t *v_rows;
  const float *k_scale;
  const float *v_scale;
  int n;
};

template <bool RAW>
__device__ __forceinline__ ItemView item_view(const HeadDesc *d) {
  ItemView r;
  if constexpr (RAW) {
    r.k_rows = reinterpret_cast<const uint8_t *>(d->raw_k);
    r.v_rows = reinterpret_cast<const uint8_t *>(d->raw_v);
  } else {
    r.k_rows = d->k_codes;
    r.v_rows = d->v_codes;
  }
  r.k_scale = d->k_scale;
  r.v_scale = d->v_scale;
  r.n = d->st.size;
  return r;
}

// Writes the block's partial (max, sum, acc[P]) for (item, split).
template <int P>
__device__ void write_partial(float *part, float m, float l, const float *acc_lds) {
  if (threadIdx.x == 0) {
    part[0] = m;
    part[1] = l;
  }
  for (int i = threadIdx.x; i < P; i += blockDim.x) part[4 + i] = acc_lds[i];
}

// Headroom (base 2) of the quantised-K decode's lazy reference maximum: the
// weights exp2(logit - m) stay below 2^16, far from fp32 overflow for any
// ring (2^31 tokens x 2^16 x the V scales).
constexpr float kLazyMax = 16.0f;

// The reference seeds the running maximum of every softmax at -1e30
// (attention.cpp:496, :566, and compute_avx2): logits at or below it get
// weight expf(l - (-1e30)) = 0.  In base-2 units (quantised K) the seed is
// -1e30 * log2 e.
constexpr float kMaxSeed = -1e30f;
constexpr float kMaxSeed2 = -1.44269504e30f;

// Normalise acc (in LDS, P entries) by 1/L, undo the rotation (inverse FWHT
// and signs, fwht.cpp:106-134) when V is quantised, and write dim outputs.
// guard (the hybrid branch, attention.cpp:513): a zero or non-finite L
// normalises by 1/n instead; elsewhere the reference divides by L as is.
template <bool INVERSE_FWHT>
__device__ void finish_item(float *s_acc, int P, int dim, float L, const uint32_t *signs,
                            float *out, bool guard = false, int n = 1) {
  const float invL = guard && !(L > 0.0f && isfinite(L)) ? 1.0f / (float)n : 1.0f / L;
  if (P == 64 || P == 128) {
    // one wave, the same operations in the same order without barriers (every
    // caller ends here): lane l holds entries l and l + 64
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const bool two = P == 128;
    float v0 = s_acc[lane] * invL, v1 = two ? s_acc[lane + 64] * invL : 0.0f;
    if (INVERSE_FWHT) {
#pragma unroll
      for (int len = 1; len < 64; len <<= 1) {
        const bool upper = (lane & len) != 0;
        const float o0 = __shfl_xor(v0, len, 64), o1 = __shfl_xor(v1, len, 64);
        v0 = upper ? o0 - v0 : v0 + o0;
        v1 = upper ? o1 - v1 : v1 + o1;
      }
      if (two) {
        const float lo = v0, hi = v1;
        v0 = lo + hi;
        v1 = lo - hi;
      }
      const float scale = 1.0f / sqrtf((float)P);
      v0 = v0 * scale;
      v1 = v1 * scale;
      if (lane < dim) out[lane] = ((signs[lane >> 5] >> (lane & 31)) & 1u) ? v0 : -v0;
      if (two && lane + 64 < dim)
        out[lane + 64] = ((signs[(lane + 64) >> 5] >> (lane & 31)) & 1u) ? v1 : -v1;
    } else {
      if (lane < dim) out[lane] = v0;
      if (two && lane + 64 < dim) out[lane + 64] = v1;
    }
    return;
  }
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_acc[i] *= invL;
  __syncthreads();
  if (INVERSE_FWHT) {
    for (int len = 1; len < P; len <<= 1) {
      for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
        const int j = (k / len) * 2 * len + (k % len);
        const float lo = s_acc[j], hi = s_acc[j + len];
        s_acc[j] = lo + hi;
        s_acc[j + len] = lo - hi;
      }
      __syncthreads();
    }
    const float scale = 1.0f / sqrtf((float)P);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
      const float v = s_acc[i] * scale;
      out[i] = ((signs[i >> 5] >> (i & 31)) & 1u) ? v : -v;
    }
  } else {
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = s_acc[i];
  }
}

#define AQ_AS1 __attribute__((address_space(1)))
#define AQ_AS4 __attribute__((address_space(4)))

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Wave-wide reductions with DPP inside 16-lane rows and readlane across rows
// (no LDS traffic; the result is wave-uniform).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = op(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = op(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = op(v, dpp<0x124>(v));  // row_ror:4
  v = op(v, dpp<0x128>(v));  // row_ror:8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return op(op(r0, r1), op(r2, r3));
}

// Wave maximum with a wave-uniform result: four DPP-modified maxes inside
// each 16-lane row (one instruction per step; the compiler's own DPP moves
// come with canonicalising maxes around them), then the four row results.
// A DPP read of a VGPR written by the previous VALU instruction needs two wait
// states, made explicit because the compiler does not see inside the asm.
__device__ __forceinline__ float wave_max_dpp(float v) {
  float t;
  asm("s_nop 1\n\t"
      "v_max_f32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf"
      : "=&v"(t)
      : "v"(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Load NB bytes at byte offset off (32-bit) of a row array in global memory.
template <int NB>
__device__ __forceinline__ void load_row_o(const uint8_t *base, uint32_t off, uint32_t (&w)[NB / 4]) {
  const AQ_AS1 uint8_t *p = (const AQ_AS1 uint8_t *)base + off;
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const u32x4 v = *reinterpret_cast<const AQ_AS1 u32x4 *>(p + 16 * i);
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) {
      const u32x2 v = *reinterpret_cast<const AQ_AS1 u32x2 *>(p + 8 * i);
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  }
}

// Load NB bytes of row t through the global address space into words.
template <int NB>
__device__ __forceinline__ void load_row_g(const uint8_t *base, long long t, uint32_t (&w)[NB / 4]) {
  const AQ_AS1 uint8_t *p = (const AQ_AS1 uint8_t *)base + (size_t)t * NB;
  if constexpr (NB % 16 == 0) {
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) {
      const u32x4 v = reinterpret_cast<const AQ_AS1 u32x4 *>(p)[i];
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) {
      const u32x2 v = reinterpret_cast<const AQ_AS1 u32x2 *>(p)[i];
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  }
}

// byte K of x, ANDed with m, in one instruction (SDWA source select).  The
// compiler splits (x >> 8K) & m into a shift or bit-field extract plus an
// AND, because SDWA takes no literal operands.
template <int K>
__device__ __forceinline__ uint32_t and_byte(uint32_t x, uint32_t m) {
  uint32_t r;
  if constexpr (K == 0)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
        : "=v"(r) : "v"(x), "v"(m));
  else if constexpr (K == 1)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1 src1_sel:DWORD"
        : "=v"(r) : "v"(x), "v"(m));
  else if constexpr (K == 2)
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2 src1_sel:DWORD"
        : "=v"(r) : "v"(x), "v"(m));
  else
    asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3 src1_sel:DWORD"
        : "=v"(r) : "v"(x), "v"(m));
  return r;
}

template <int K>
__device__ __forceinline__ void vq_addr(uint32_t xh, uint32_t xl, uint32_t m, uint32_t &ah,
                                        uint32_t &al) {
  ah = and_byte<K>(xh, m);
  al = and_byte<K>(xl, m);
}

// Bytes of LDS reserved in front of the K lookup table for the V codebook
// table, so that both are addressed with the 16-bit immediate offset of
// ds_read (the K table of padded 128 fills 64 KB by itself).
constexpr int kVlutBytes = 256;

// LUT kernel geometry: 8 waves per block share one K table; a wave streams
// 64-token tiles.
constexpr int kLutWaves = 8;
constexpr int kLutThreads = 64 * kLutWaves;

// V accumulation of one row segment of one token: acc[0..D) += wgt *
// CB_V[codes] over the D dimensions held in vw (D * VB / 8 bytes, a whole
// number of 32-bit words).  Table addresses come from the code word (high
// nibbles) or the word shifted left by 4 (low nibbles), so each nibble costs
// one masked byte select (SDWA) and one LDS read.
template <int D, int VB>
__device__ __forceinline__ void vseg_accumulate(float (&acc)[D], const uint32_t *vw, float wgt,
                                                const uint8_t *lds, uint32_t mask) {
  constexpr int HB = D * VB / 8;  // bytes in the segment
  if constexpr (VB == 2) {
    // nibble n of byte j -> float2 at 16n: codes (dims) 4j,4j+1 | 4j+2,4j+3
#pragma unroll
    for (int q = 0; q < HB / 4; ++q) {
      const uint32_t xh = vw[q], xl = vw[q] << 4;
      uint32_t ahs[4], als[4];
      vq_addr<0>(xh, xl, mask, ahs[0], als[0]);
      vq_addr<1>(xh, xl, mask, ahs[1], als[1]);
      vq_addr<2>(xh, xl, mask, ahs[2], als[2]);
      vq_addr<3>(xh, xl, mask, ahs[3], als[3]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = 4 * q + k;
        const f32x2 hi = *reinterpret_cast<const f32x2 *>(lds + ahs[k]);
        const f32x2 lo = *reinterpret_cast<const f32x2 *>(lds + als[k]);
        acc[4 * j] = fmaf(hi.x, wgt, acc[4 * j]);
        acc[4 * j + 1] = fmaf(hi.y, wgt, acc[4 * j + 1]);
        acc[4 * j + 2] = fmaf(lo.x, wgt, acc[4 * j + 2]);
        acc[4 * j + 3] = fmaf(lo.y, wgt, acc[4 * j + 3]);
      }
    }
  } else if constexpr (VB == 4) {
    // nibble -> float at 16n: dims 2j (high nibble), 2j+1 (low nibble)
#pragma unroll
    for (int q = 0; q < HB / 4; ++q) {
      const uint32_t xh = vw[q], xl = vw[q] << 4;
      uint32_t ahs[4], als[4];
      vq_addr<0>(xh, xl, mask, ahs[0], als[0]);
      vq_addr<1>(xh, xl, mask, ahs[1], als[1]);
      vq_addr<2>(xh, xl, mask, ahs[2], als[2]);
      vq_addr<3>(xh, xl, mask, ahs[3], als[3]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = 4 * q + k;
        acc[2 * j] = fmaf(*reinterpret_cast<const float *>(lds + ahs[k]), wgt, acc[2 * j]);
        acc[2 * j + 1] = fmaf(*reinterpret_cast<const float *>(lds + als[k]), wgt, acc[2 * j + 1]);
      }
    }
  } else {
    // 3-bit: 8 codes per 24-bit big-endian group -> float at c*4
#pragma unroll
    for (int g = 0; g < D / 8; ++g) {
      const uint32_t w24 = (byte_of(vw, 3 * g) << 16) | (byte_of(vw, 3 * g + 1) << 8) |
                           byte_of(vw, 3 * g + 2);
      const uint32_t w26 = w24 << 2;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t a = (w26 >> (21 - 3 * k)) & 0x1Cu;
        acc[8 * g + k] = fmaf(*reinterpret_cast<const float *>(lds + a), wgt, acc[8 * g + k]);
      }
    }
  }
}

// V rows are split into SPLIT segments of P/SPLIT dimensions: quarters when
// a quarter row is a whole number of 16-byte units, halves otherwise
// (3-bit codes at padded 64).
template <int P, int VB>
struct VSplit {
  static constexpr int row_bytes = VB == 16 ? 4 * P : P * VB / 8;
  static constexpr int value = (row_bytes % 16 == 0) ? 4 : 2;
};

// Segment transpose across lanes.  Lane l = G*r + c (G = 64/SPLIT lanes per
// row group r, column c) holds segment q of its own row in
// x[q*SW .. q*SW+SW); afterwards it holds segment r of the row of lane
// G*s + c in x[s*SW ..], s < SPLIT.  permlane32_swap exchanges lanes 32-63 of
// its first operand with lanes 0-31 of its second; permlane16_swap exchanges
// the odd 16-lane rows of its first operand with the even rows of its second.
template <int SPLIT, int SW>
__device__ __forceinline__ void transpose_segments(uint32_t *x) {
  if constexpr (SPLIT == 2) {
#pragma unroll
    for (int i = 0; i < SW; ++i) {
      const auto r = __builtin_amdgcn_permlane32_swap(x[i], x[SW + i], false, false);
      x[i] = r[0];
      x[SW + i] = r[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < SW; ++i) {
      const auto r0 = __builtin_amdgcn_permlane32_swap(x[i], x[2 * SW + i], false, false);
      const auto r1 = __builtin_amdgcn_permlane32_swap(x[SW + i], x[3 * SW + i], false, false);
      x[i] = r0[0];
      x[2 * SW + i] = r0[1];
      x[SW + i] = r1[0];
      x[3 * SW + i] = r1[1];
    }
#pragma unroll
    for (int i = 0; i < SW; ++i) {
      const auto r0 = __builtin_amdgcn_permlane16_swap(x[i], x[SW + i], false, false);
      const auto r1 = __builtin_amdgcn_permlane16_swap(x[2 * SW + i], x[3 * SW + i], false, false);
      x[i] = r0[0];
      x[SW + i] = r0[1];
      x[2 * SW + i] = r1[0];
      x[3 * SW + i] = r1[1];
    }
  }
}

// Clock stamps, compiled only into the timing library (AQ_CLOCK_STAMPS,
// `python -m adaptq_amd.build --clock-stamps`): thread 0 of every block of
// decode_lut_kernel records s_memtime (shader clock cycles) and
// s_memrealtime (the constant 100 MHz clock) at its start and end, into slot
// [launch][block] of g_clk; the launch index is set beforehand by
// adaptq_clock_stamp_set.  The clock a launch ran at is the ratio of the two
// deltas summed over its blocks.
#ifdef AQ_CLOCK_STAMPS
constexpr int kClkLaunches = 32, kClkBlocks = 16384;
__device__ unsigned long long g_clk[kClkLaunches * kClkBlocks * 4];
__device__ int g_clk_launch;
__global__ void clk_set_kernel(int i) { g_clk_launch = i; }
#define AQ_CLK_BEGIN()                                     \
  unsigned long long clk_c0 = 0, clk_r0 = 0;               \
  int clk_l = 0;                                           \
  if (!FUSE && threadIdx.x == 0) {                         \
    clk_c0 = __builtin_amdgcn_s_memtime();                 \
    clk_r0 = __builtin_amdgcn_s_memrealtime();             \
    clk_l = g_clk_launch;                                  \
  }
#define AQ_CLK_END()                                                                             \
  if (!FUSE && threadIdx.x == 0) {                                                               \
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();                                 \
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();                             \
    const size_t b = ((size_t)(clk_l & (kClkLaunches - 1)) * kClkBlocks +                       \
                      ((blockIdx.y * gridDim.x + blockIdx.x) & (kClkBlocks - 1))) * 4;          \
    g_clk[b] = clk_c0;                                                                           \
    g_clk[b + 1] = clk_r0;                                                                       \
    g_clk[b + 2] = c1;                                                                           \
    g_clk[b + 3] = r1;                                                                           \
  }
#else
#define AQ_CLK_BEGIN()
#define AQ_CLK_END()
#endif

// With n_splits == 1 the block owns its item and writes the final output
// (outs) directly; otherwise it writes a partial for finalize_kernel.
//
// One lane per token for K: a byte lookup table in LDS gives one read per
// code byte.  For V, the SPLIT lanes of a column exchange row segments
// (transpose_segments) so that each lane accumulates one segment of
// P/SPLIT dimensions for SPLIT tokens: the same FMAs as one token per lane,
// with 1/SPLIT of the accumulator registers (hence the occupancy).  V
// codebook tables are small enough that distinct entries sit in distinct LDS
// banks:
//   2-bit: nibble (2 codes) -> float2, 16 entries
//   4-bit: nibble (1 code)  -> float, 16 entries
//   3-bit: code             -> float, 8 entries
//
// FUSE (a decode step, launch_decode_step): the launch first appends one token
// per item, app.k/app.v [item][dim]: waves 1 and 2 encode its key and value
// rows with the one-row codec (encode_one.hpp) into the ring, and into LDS,
// while wave 0 rotates the query; the decode covers the ring after the
// append.  Row loads issued before the new rows are written may return the
// slot's old bytes, so the lanes whose token is the new slot take its rows
// and scales from the LDS copies (one tile per kernel, a wave-uniform
// branch).  One block per item (n_splits == 1), quantised K and V at padded
// 64, no raw mirror decode.
template <int P, int KB, int VB, bool RAW, bool FUSE = false>
__global__ __launch_bounds__(kLutThreads, P <= 128 && (KB == 2 || KB == 4) ? 4 : 2) void decode_lut_kernel(
    HeadDesc *const *item_desc, const float *__restrict__ queries, int chunk, int n_splits,
    float *__restrict__ partials, float *__restrict__ outs, StepAppend app, int qdim) {
  constexpr bool KQ = KB != 16;
  constexpr bool VQ = VB != 16;
  constexpr int KNB = RAW ? 4 * P : RowBytes<P, KB>::value;
  constexpr int VNB = RAW ? 4 * P : RowBytes<P, VB>::value;
  constexpr int KW = KQ ? KNB / 4 : 1;
  constexpr int VW = VQ ? VNB / 4 : 1;
  constexpr int SPLIT = VSplit<P, VB>::value;
  constexpr int G = 64 / SPLIT;  // lanes per row group
  constexpr int D = P / SPLIT;   // dimensions per lane
  constexpr int SW = VQ ? VW / SPLIT : 1;
  // LDS: [V table | K table | query | per-wave partials]
  __shared__ __align__(16) uint8_t s_mem[kVlutBytes + 4 * KLut<P, KB>::size];
  __shared__ float s_q[P];
  __shared__ float s_red[kLutWaves][P];
  __shared__ float s_ml[kLutWaves][2];
  float *s_vlut = reinterpret_cast<float *>(s_mem);
  float *s_klut = reinterpret_cast<float *>(s_mem + kVlutBytes);

  const int item = blockIdx.y, split = blockIdx.x;
  // Descriptor fields are read through the constant address space so they
  // load as scalars (a generic-pointer load is assumed divergent).
  const AQ_AS4 HeadDesc *d =
      (const AQ_AS4 HeadDesc *)((const AQ_AS4 uint64_t *)item_desc)[item];
  // every item of a launch has this dim (it is also d->dim): the query's
  // address does not wait for the descriptor
  const int dim = qdim;
  static_assert(!FUSE || (KB != 16 && VB != 16 && !RAW && P == 64), "fused step: quantised K and V");
  RingState st0{};  // FUSE: the ring state before the step's append
  int new_slot = -1;
  if constexpr (FUSE) {
    st0.head = d->st.head;
    st0.size = d->st.size;
    st0.raw_count = d->st.raw_count;
    new_slot = st0.head;
  }
  const int n = FUSE ? ring_after(st0, 1, d->cap, d->hyb).size : d->st.size;
  const int t_begin = split * chunk;
  const int t_end = min(n, t_begin + chunk);
  float *part = partials + ((size_t)item * n_splits + split) * (P + 4);
  const int lane = threadIdx.x & 63;
  const int grow = lane / G, gcol = lane % G;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t *signs = (const uint32_t *)d->signs;
  AQ_CLK_BEGIN();
  if (t_begin >= t_end) {
    if (n_splits == 1) {
      for (int i = threadIdx.x; i < dim; i += blockDim.x) outs[(size_t)item * dim + i] = 0.0f;
      return;
    }
    for (int i = threadIdx.x; i < P; i += blockDim.x) part[4 + i] = 0.0f;
    if (threadIdx.x == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    return;
  }

  const uint8_t *k_rows = RAW ? (const uint8_t *)d->raw_k : (const uint8_t *)d->k_codes;
  const uint8_t *v_rows = RAW ? (const uint8_t *)d->raw_v : (const uint8_t *)d->v_codes;
  const AQ_AS1 float *k_scale = (const AQ_AS1 float *)d->k_scale;
  const AQ_AS1 float *v_scale = (const AQ_AS1 float *)d->v_scale;

  // Software pipeline: the first tile is requested before the tables are
  // built; afterwards the K row of the next tile is requested as soon as
  // this tile's logits are done and the V row as soon as its segments have
  // been exchanged, so each load has a compute phase to hide behind without
  // extra registers.  The wave raises its priority while it issues those
  // loads, so that the VALU-bound phases of the other waves on the SIMD do
  // not delay the requests (measured: 3-8% shorter decode at config 5).
  constexpr int kStride = kLutWaves * kTile;
  int base = t_begin + wave * kTile;
  uint32_t kc[KW], vw[VW];

  // K rows in XOR byte order (kperm_mask): this lane's tokens all sit in
  // slots = lane (mod 64), so stored byte 4i+k of its rows is byte position
  // jj = (4i+k) ^ x.  A word xr[i] holds 4*jj for k = 0..3 in its bytes
  // (lx0 = 4x in every byte, XORed with the static part); v_perm joins a code
  // byte b and 4*jj into the table offset b*256 + 4*jj.
  constexpr bool KPERM = KQ && (KB == 2 || KB == 4) && P <= 128;
  constexpr bool NIB = KQ && (KB == 2 || KB == 4) && P >= 256;  // build_klut_nib's table
  constexpr uint32_t kXMask = (uint32_t)kperm_mask(P, KB);
  const uint32_t lx0 = (4u * ((uint32_t)lane & kXMask)) * 0x01010101u;
  // Row offsets are 32-bit (the host routes rings of 4 GiB and more to the
  // generic kernel) so loads take a scalar base plus one VGPR offset.
  float ksc = 1.0f, vsc = 1.0f;
  {
    const uint32_t tt = (uint32_t)min(base + lane, t_end - 1);  // t_begin < t_end here
    if constexpr (KQ) load_row_o<KNB>(k_rows, tt * KNB, kc);
    if constexpr (VQ) load_row_o<VNB>(v_rows, tt * VNB, vw);
    if constexpr (KQ) ksc = k_scale[tt];
    if constexpr (VQ) vsc = v_scale[tt];
  }

  // FUSE: waves 1 and 2 encode the step's key and value rows (LDS scratch of
  // the codec, its 4-bit cell table per wave, the stored rows' copies)
  // while wave 0 rotates the query; load_query's closing barrier publishes
  // both
  constexpr bool kQ4 = FUSE && (KB == 4 || VB == 4);
  __shared__ Q4Cell s_app_q4[kQ4 ? 2 : 1][kQ4 ? kQ4Cells : 1];
  __shared__ __align__(16) float s_app_sq[FUSE ? 2 : 1][FUSE ? P : 1];
  __shared__ uint8_t s_app_code[FUSE ? 2 : 1][FUSE ? P : 1];
  __shared__ uint32_t s_app_row[FUSE ? 2 : 1][FUSE ? (KW > VW ? KW : VW) : 1];
  __shared__ float s_app_scale[2];
  if constexpr (FUSE) {
    if (wave == 1 || wave == 2) {
      const int side = wave - 1;
      if constexpr (kQ4) {
        static constexpr Q4Table kTab = q4_table();
        if (lane < kQ4Cells) s_app_q4[side][lane] = kTab.c[lane];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      const float *x = (side == 0 ? app.k : app.v) + (size_t)item * dim;
      encode_one_row<P, KB, VB>(item_desc[item], st0, 1, 0, x, dim, side, lane, app.inv_sqrt_p,
                                app.sqrt_p, s_app_q4[kQ4 ? side : 0], s_app_sq[side],
                                s_app_code[side], s_app_row[side], &s_app_scale[side]);
    }
  }
  load_query<P>(s_q, queries + (size_t)item * dim, dim, KQ, signs);
  // fixed-point scale of the K table (2/4-bit keys): f and 1/f
  __shared__ float s_fix[2];
  if constexpr (KPERM || NIB) {
    if (threadIdx.x < 64) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < P / 64; ++i) a += fabsf(s_q[threadIdx.x + 64 * i]);
      a = wave_sum(a) * KMaxCode<KB>::value;
      if (threadIdx.x == 0) {
        // the largest power of two f with f * max|CB| * sum|qr| <= 2^29
        const float f = a > 0.0f ? ldexpf(1.0f, min(ilogbf(536870912.0f / a), 100)) : 1.0f;
        s_fix[0] = f;
        s_fix[1] = 1.0f / f;
      }
    }
    __syncthreads();
    if constexpr (NIB) build_klut_nib<P, KB>(reinterpret_cast<int32_t *>(s_klut), s_q, s_fix[0]);
    else build_klut_fixed<P, KB>(reinterpret_cast<int32_t *>(s_klut), s_q, s_fix[0]);
  } else if constexpr (KQ) {
    build_klut<P, KB>(s_klut, s_q);
  }
  if constexpr (VQ) build_vlut<VB>(s_vlut);
  __syncthreads();

  // Quantised K: logits are kept in base-2 units (log2 e folded into the
  // scale) and weighted with exp2, one instruction; fp32 K keeps the
  // reference's natural-unit logits and expf, bit for bit.
  constexpr float kLog2e = 1.44269504088896340736f;
  const float attn_s = KQ ? kLog2e / (sqrtf((float)dim) * (float)P) : 1.0f / sqrtf((float)dim);
  const float attn_fix = KPERM || NIB ? attn_s * s_fix[1] : attn_s;  // undoes the table's fixed point
  const float isp = VQ ? 1.0f / sqrtf((float)P) : 1.0f;
  const uint32_t vmask = 0xF0u;
  auto wexp = [](float z) -> float {
    if constexpr (KQ) return __builtin_amdgcn_exp2f(z);
    else return expf(z);
  };

  // Logit of the token of this lane in the tile at tile_base (K row kc).
  auto tile_logit = [&](const uint32_t *kc_in, float kscale, int tile_base) -> float {
    const int tt = tile_base + lane;
    uint32_t kcw[KW];
#pragma unroll
    for (int i = 0; i < KW; ++i) kcw[i] = kc_in[i];
    if constexpr (FUSE) {
      // the lanes whose (clamped) row is the step's new slot: its LDS copy
      if (tile_base <= new_slot && new_slot < tile_base + kTile) {
        const bool mine = min(tt, t_end - 1) == new_slot;
#pragma unroll
        for (int i = 0; i < KW; ++i) kcw[i] = mine ? s_app_row[0][i] : kcw[i];
        kscale = mine ? s_app_scale[0] : kscale;
      }
    }
    float dot;
    if constexpr (KQ && KB == 3) {
      float p4[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) p4[m] = s_klut[m * 64 + pair3(kcw, 0, m)];
#pragma unroll
      for (int g = 1; g < P / 8; ++g)
#pragma unroll
        for (int m = 0; m < 4; ++m) p4[m] += s_klut[(4 * g + m) * 64 + pair3(kcw, g, m)];
      dot = ((p4[0] + p4[1]) + (p4[2] + p4[3])) * attn_s * kscale;
    } else if constexpr (NIB) {
      // two lookups per code byte: the high nibble's offset is the byte
      // masked with 0xF0, the low nibble's the byte of the word shifted left
      // by 4, masked the same way (one SDWA and each)
      const uint8_t *lb = reinterpret_cast<const uint8_t *>(s_klut);
      int32_t p4[4] = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < KW; ++i) {
        const uint32_t wh = kcw[i], wl = kcw[i] << 4;
        uint32_t ah[4], al[4];
        vq_addr<0>(wh, wl, 0xF0u, ah[0], al[0]);
        vq_addr<1>(wh, wl, 0xF0u, ah[1], al[1]);
        vq_addr<2>(wh, wl, 0xF0u, ah[2], al[2]);
        vq_addr<3>(wh, wl, 0xF0u, ah[3], al[3]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int u = 8 * i + 2 * k;
          p4[k] = p4[k] + *reinterpret_cast<const int32_t *>(lb + nib_off(u) + ah[k]) +
                  *reinterpret_cast<const int32_t *>(lb + nib_off(u + 1) + al[k]);
        }
      }
      dot = (float)((p4[0] + p4[1]) + (p4[2] + p4[3])) * (attn_fix * kscale);
    } else if constexpr (KQ) {
      // selector k: byte 0 <- byte k of xr[i], byte 1 <- code byte k, bytes 2-3 <- 0.
      // xr[i] is rebuilt per tile (one XOR each) rather than held in 16
      // registers; the empty asm keeps the compiler from hoisting it.
      const uint8_t *lb = reinterpret_cast<const uint8_t *>(s_klut);
      uint32_t lx = lx0;
      asm volatile("" : "+v"(lx));
      uint32_t xr[KW];
#pragma unroll
      for (int i = 0; i < KW; ++i) xr[i] = ((uint32_t)(16 * i) * 0x01010101u + 0x0C080400u) ^ lx;
      auto look = [&](int i, int k) -> int32_t {
        return *reinterpret_cast<const int32_t *>(
            lb + __builtin_amdgcn_perm(kcw[i], xr[i], 0x0C0C0000u | ((4u + k) << 8) | (uint32_t)k));
      };
      int32_t p4[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) p4[k] = look(0, k) + look(1, k);
#pragma unroll
      for (int i = 2; i < KW; i += 2)
#pragma unroll
        for (int k = 0; k < 4; ++k) p4[k] = p4[k] + look(i, k) + look(i + 1, k);
      dot = (float)((p4[0] + p4[1]) + (p4[2] + p4[3])) * (attn_fix * kscale);
    } else {
      // fp32 keys: the reference's sequential, unfused dot product
      // (attention.cpp:212-219 and :497-502), so that peaked softmaxes see
      // the same logits to the last bit.
      const AQ_AS1 float *kr =
          (const AQ_AS1 float *)k_rows + (uint32_t)min(tt, t_end - 1) * (uint32_t)(RAW ? dim : P);
      float acc_d = 0.0f;
#pragma unroll
      for (int i = 0; i < P; i += 4) {
        const f32x4 k4 = *reinterpret_cast<const AQ_AS1 f32x4 *>(kr + i);
        acc_d = __fadd_rn(acc_d, __fmul_rn(s_q[i], k4.x));
        acc_d = __fadd_rn(acc_d, __fmul_rn(s_q[i + 1], k4.y));
        acc_d = __fadd_rn(acc_d, __fmul_rn(s_q[i + 2], k4.z));
        acc_d = __fadd_rn(acc_d, __fmul_rn(s_q[i + 3], k4.w));
      }
      dot = __fmul_rn(acc_d, attn_s);
    }
    return tt < t_end ? dot : -INFINITY;
  };

  float acc[D];
#pragma unroll
  for (int i = 0; i < D; ++i) acc[i] = 0.0f;
  float m_run = KQ ? kMaxSeed2 : kMaxSeed, l_run = 0.0f;

  // The loop body holds the V phase of tile i and the K phase of tile i+1.
  float logit = tile_logit(kc, ksc, base);
  if constexpr (KQ) {
    const uint32_t tn = (uint32_t)min(base + kStride + lane, t_end - 1);
    load_row_o<KNB>(k_rows, tn * KNB, kc);
    ksc = k_scale[tn];
  }
  // the last tile has no next tile: its V phase runs without the next
  // tile's loads and K phase (a separate copy keeps the loop branch-free)
  auto step = [&](auto last_tag) {
    constexpr bool LAST = decltype(last_tag)::value;
    const bool valid = base + lane < t_end;
    if constexpr (FUSE) {
      // this tile's V rows: the new slot's from its LDS copy (see tile_logit)
      if (base <= new_slot && new_slot < base + kTile) {
        const bool mine = min(base + lane, t_end - 1) == new_slot;
#pragma unroll
        for (int i = 0; i < VW; ++i) vw[i] = mine ? s_app_row[1][i] : vw[i];
        vsc = mine ? s_app_scale[1] : vsc;
      }
    }

    // ---- online softmax (wave-uniform reference maximum) ----
    // Quantised K: the reference maximum moves only when a logit exceeds it
    // by more than kLazyMax (base 2), so weights stay below 2^kLazyMax and
    // most tiles need one compare instead of the wave maximum; the softmax
    // is the same up to rounding, as the maximum only scales every weight.
    const bool bump = KQ ? __ballot(logit > m_run + kLazyMax) != 0ull : true;
    if (bump) {
      const float tmax = wave_max_dpp(logit);
      if (tmax > m_run) {
        const float alpha = m_run == -INFINITY ? 0.0f : wexp(m_run - tmax);
#pragma unroll
        for (int i = 0; i < D; ++i) acc[i] *= alpha;
        l_run *= alpha;
        m_run = tmax;
      }
    }
    const float e = valid ? wexp(logit - m_run) : 0.0f;
    l_run += e;
    const float wgt = VQ ? e * vsc * isp : e;

    // ---- V: exchange row segments within each column ----
    // After the transposes, wv[s] and segment s of x belong to the token of
    // lane G*s + gcol; x holds segment grow of its row.  Invalid tokens
    // carry weight 0 and valid (clamped) codes.
    uint32_t wv[SPLIT];
#pragma unroll
    for (int s2 = 0; s2 < SPLIT; ++s2) wv[s2] = __float_as_uint(wgt);
    transpose_segments<SPLIT, 1>(wv);
    uint32_t x[VW];
    if constexpr (VQ) {
#pragma unroll
      for (int i = 0; i < VW; ++i) x[i] = vw[i];
      transpose_segments<SPLIT, SW>(x);
      if constexpr (!LAST) {
      // past the end every lane reads the last row (one line)
      const uint32_t tn = (uint32_t)min(base + kStride + lane, t_end - 1);
      __builtin_amdgcn_s_setprio(2);
      load_row_o<VNB>(v_rows, tn * VNB, vw);
      vsc = v_scale[tn];
      __builtin_amdgcn_s_setprio(0);
      }
    }

    // ---- V phase of this tile, then the K phase of the next ----
    if constexpr (VQ) {
#pragma unroll
      for (int s2 = 0; s2 < SPLIT; ++s2)
        vseg_accumulate<D, VB>(acc, x + s2 * SW, __uint_as_float(wv[s2]), s_mem, vmask);
    } else {
      const AQ_AS1 float *vr = (const AQ_AS1 float *)v_rows;
      const int stride = RAW ? dim : P;
#pragma unroll
      for (int s2 = 0; s2 < SPLIT; ++s2) {
        const uint32_t tok = (uint32_t)min(base + G * s2 + gcol, t_end - 1);
        const AQ_AS1 float *row = vr + (tok * (uint32_t)stride + (uint32_t)(grow * D));
        const float ws = __uint_as_float(wv[s2]);
#pragma unroll
        for (int i = 0; i < D; i += 4) {
          const f32x4 v4 = *reinterpret_cast<const AQ_AS1 f32x4 *>(row + i);
          acc[i] = fmaf(v4.x, ws, acc[i]);
          acc[i + 1] = fmaf(v4.y, ws, acc[i + 1]);
          acc[i + 2] = fmaf(v4.z, ws, acc[i + 2]);
          acc[i + 3] = fmaf(v4.w, ws, acc[i + 3]);
        }
      }
    }
    if constexpr (!LAST) {
    logit = tile_logit(kc, ksc, base + kStride);
    if constexpr (KQ) {
      const uint32_t tn2 = (uint32_t)min(base + 2 * kStride + lane, t_end - 1);
      __builtin_amdgcn_s_setprio(2);
      load_row_o<KNB>(k_rows, tn2 * KNB, kc);
      ksc = k_scale[tn2];
      __builtin_amdgcn_s_setprio(0);
    }
      }
  };
  for (; base + kStride < t_end; base += kStride) step(std::false_type{});
  if (base < t_end) step(std::true_type{});

  // ---- block merge: waves -> one (m, l, acc) ----
  // l_run: every token's e is held by its own lane once.
  const float l_w = wave_reduce<false>(l_run);
  // reduce acc[D] over the G lanes of each row group: lane (grow, gcol) ends
  // with the totals of dimensions grow*D + (D/G)*gcol + k, k < D/G
#pragma unroll
  for (int step = 0; (G >> step) > 1; ++step) {
    const int m = (G / 2) >> step;
    const int half = D >> (step + 1);
    const uint32_t up = (lane & m) ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int j = 0; j < half; ++j) {
      const uint32_t a = __float_as_uint(acc[j]), bb = __float_as_uint(acc[j + half]);
      const float send = __uint_as_float((a & up) | (bb & ~up));
      const float keep = __uint_as_float((bb & up) | (a & ~up));
      acc[j] = keep + __shfl_xor(send, m, 64);
    }
  }
  {
    const int d0 = grow * D + (D / G) * gcol;
#pragma unroll
    for (int k = 0; k < D / G; ++k) s_red[wave][d0 + k] = acc[k];
  }
  if (lane == 0) {
    s_ml[wave][0] = m_run;
    s_ml[wave][1] = l_w;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kLutWaves; ++w) M = fmaxf(M, s_ml[w][0]);
  float f[kLutWaves], L = 0.0f;
#pragma unroll
  for (int w = 0; w < kLutWaves; ++w) {
    f[w] = s_ml[w][0] == -INFINITY ? 0.0f : wexp(s_ml[w][0] - M);
    L += f[w] * s_ml[w][1];
  }
  if (n_splits == 1) {
    // s_q is free now: merge the waves into it and finish the item here.
    for (int i = threadIdx.x; i < P; i += blockDim.x) {
      float a = 0.0f;
#pragma unroll
      for (int w = 0; w < kLutWaves; ++w) a += f[w] * s_red[w][i];
      s_q[i] = a;
    }
    __syncthreads();
    if constexpr (FUSE) {
      // the step's ring state, once every wave has read the old one
      if (threadIdx.x == 0) item_desc[item]->st = ring_after(st0, 1, d->cap, d->hyb);
    }
    finish_item<VQ && !RAW>(s_q, P, dim, L, signs, outs + (size_t)item * dim, RAW, n);
    AQ_CLK_END();
    return;
  }
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < kLutWaves; ++w) a += f[w] * s_red[w][i];
    part[4 + i] = a;
  }
  if (threadIdx.x == 0) {
    // the finalize kernel merges splits in natural units
    part[0] = KQ ? M * 0.69314718055994530942f : M;
    part[1] = L;
  }
  AQ_CLK_END();
}

// Code c of a packed row (generic unpack; restates quantizer.cpp:161-209).
template <int B>
__device__ __forceinline__ int code_at(const uint8_t *row, int i) {
  if constexpr (B == 4) {
    const uint32_t b = row[i >> 1];
    return (i & 1) ? (b & 15) : (b >> 4);
  } else if constexpr (B == 2) {
    return (row[i >> 2] >> (6 - 2 * (i & 3))) & 3;
  } else {
    const uint8_t *p = row + 3 * (i >> 3);
    const uint32_t w24 = ((uint32_t)p[0] << 16) | ((uint32_t)p[1] << 8) | p[2];
    return (w24 >> (21 - 3 * (i & 7))) & 7;
  }
}

// Code i of a K row stored in the slot's XOR byte order (x = slot & mask).
template <int B>
__device__ __forceinline__ int kcode_at(const uint8_t *row, int i, int x) {
  if constexpr (B == 4) {
    const uint32_t b = row[(i >> 1) ^ x];
    return (i & 1) ? (b & 15) : (b >> 4);
  } else if constexpr (B == 2) {
    return (row[(i >> 2) ^ x] >> (6 - 2 * (i & 3))) & 3;
  } else {
    return code_at<B>(row, i);
  }
}

// Generic kernel: any padded up to 1024.  Thread j owns dims j, j+256, ...;
// tokens are processed in groups of 8 with one block reduction per group.
template <int KB, int VB, bool RAW>
__global__ __launch_bounds__(kThreads) void decode_generic_kernel(
    HeadDesc *const *item_desc, const float *__restrict__ queries, int chunk, int n_splits,
    float *__restrict__ partials) {
  constexpr bool KQ = KB != 16;
  constexpr bool VQ = VB != 16;
  constexpr int G = 8;
  __shared__ float s_q[kMaxPadded];
  __shared__ float s_part[kWaves][G];
  // codebooks in LDS: a run-time index into the constant tables would be a
  // memory load per code
  __shared__ float s_cbk[16], s_cbv[16];
  const int item = blockIdx.y, split = blockIdx.x;
  const HeadDesc *d = item_desc[item];
  const ItemView iv = item_view<RAW>(d);
  const int dim = d->dim, P = d->padded;
  const int n = iv.n;
  const int t_begin = split * chunk;
  const int t_end = min(n, t_begin + chunk);
  float *part = partials + ((size_t)item * n_splits + split) * (P + 4);
  if (t_begin >= t_end) {
    for (int i = threadIdx.x; i < P; i += blockDim.x) part[4 + i] = 0.0f;
    if (threadIdx.x == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    return;
  }
  const float *q = queries + (size_t)item * dim;
  if constexpr (KQ) {
    if (threadIdx.x < (1 << KB)) s_cbk[threadIdx.x] = cbv<KB>(threadIdx.x);
  }
  if constexpr (VQ) {
    if (threadIdx.x < (1 << VB)) s_cbv[threadIdx.x] = cbv<VB>(threadIdx.x);
  }
  for (int i = threadIdx.x; i < P; i += blockDim.x) {
    float v = i < dim ? q[i] : 0.0f;
    if (KQ && !((d->signs[i >> 5] >> (i & 31)) & 1u)) v = -v;
    s_q[i] = v;
  }
  __syncthreads();
  if (KQ) {
    for (int len = 1; len < P; len <<= 1) {
      for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
        const int j = (k / len) * 2 * len + (k % len);
        const float lo = s_q[j], hi = s_q[j + len];
        s_q[j] = lo + hi;
        s_q[j + len] = lo - hi;
      }
      __syncthreads();
    }
  }
  const float attn_s = KQ ? 1.0f / (sqrtf((float)dim) * (float)P) : 1.0f / sqrtf((float)dim);
  const float isp = VQ ? 1.0f / sqrtf((float)P) : 1.0f;
  const int kstride = RAW ? dim * 4 : packed_bytes(P, KB);
  const int vstride = RAW ? dim * 4 : packed_bytes(P, VB);
  const int own = RAW ? dim : P;  // dims that carry data
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  float acc[kMaxPadded / kThreads];
#pragma unroll
  for (int r = 0; r < kMaxPadded / kThreads; ++r) acc[r] = 0.0f;
  float m_run = kMaxSeed, l_run = 0.0f;

  for (int t0 = t_begin; t0 < t_end; t0 += G) {
    if constexpr (KQ) {
      float pd[G];
      const int xmask = kperm_mask(P, KB);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        pd[g] = 0.0f;
        const int t = t0 + g;
        if (t >= t_end) continue;
        const uint8_t *row = iv.k_rows + (size_t)t * kstride;
        const int x = t & xmask;
        for (int i = threadIdx.x; i < own; i += kThreads)
          pd[g] = fmaf(s_q[i], s_cbk[kcode_at<KB>(row, i, x)], pd[g]);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float s = wave_sum(pd[g]);
        if (lane == 0) s_part[wave][g] = s;
      }
    } else if (threadIdx.x < G) {
      // fp32 keys: one thread per token, the reference's sequential unfused
      // dot product (attention.cpp:212-219 and :497-502)
      const int t = t0 + threadIdx.x;
      float dsum = 0.0f;
      if (t < t_end) {
        const float *row = reinterpret_cast<const float *>(iv.k_rows + (size_t)t * kstride);
        for (int i = 0; i < dim; ++i) dsum = __fadd_rn(dsum, __fmul_rn(s_q[i], row[i]));
      }
      s_part[0][threadIdx.x] = dsum;
    }
    __syncthreads();
    float lg[G];
    float gmax = -INFINITY;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float s = 0.0f;
      if constexpr (KQ) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += s_part[w][g];
      } else {
        s = s_part[0][g];
      }
      const int t = t0 + g;
      lg[g] = t < t_end ? (KQ ? s * attn_s * iv.k_scale[t] : __fmul_rn(s, attn_s)) : -INFINITY;
      gmax = fmaxf(gmax, lg[g]);
    }
    __syncthreads();
    if (gmax > m_run) {
      const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - gmax);
#pragma unroll
      for (int r = 0; r < kMaxPadded / kThreads; ++r) acc[r] *= alpha;
      l_run *= alpha;
      m_run = gmax;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int t = t0 + g;
      if (t >= t_end) continue;
      const float e = expf(lg[g] - m_run);
      l_run += e;
      const float wgt = VQ ? e * iv.v_scale[t] * isp : e;
      const uint8_t *row = iv.v_rows + (size_t)t * vstride;
#pragma unroll
      for (int r = 0; r < kMaxPadded / kThreads; ++r) {
        const int i = threadIdx.x + r * kThreads;
        if (i >= own) break;
        float vv;
        if constexpr (VQ) vv = s_cbv[code_at<VB>(row, i)];
        else vv = reinterpret_cast<const float *>(row)[i];
        acc[r] = fmaf(vv, wgt, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kMaxPadded / kThreads; ++r) {
    const int i = threadIdx.x + r * kThreads;
    if (i < P) part[4 + i] = i < own ? acc[r] : 0.0f;
  }
  if (threadIdx.x == 0) {
    part[0] = m_run;
    part[1] = l_run;
  }
}

// Wide kernel (padded 512 and 1024, quantised K and V): one wave per token at
// a time, the row's dimensions spread over the lanes.  Lane l owns dimensions
// [C l, C l + C), C = P / 64, so a row's codes arrive in one coalesced load
// per wave (C KB / 8 bytes per lane).
//   K: fixed-point table in LDS, entry (code c, dimension i) = f qr_i
//      CB_K[c] rounded to the nearest integer, f the largest power of two
//      with f max|CB| sum_i |qr_i| <= 2^30 (so every partial sum of a row's
//      entries stays below 2^30 + P / 2 in magnitude); a lane adds its C
//      entries in int32 and the wave adds the lanes' sums by DPP, exactly.
//      The one-lane-per-token LUT kernel's byte entries cover two or four
//      codes each; here a row adds P entries, so rounding (rather than
//      truncating) and the larger scale keep the sum's error near the fp32
//      dot product's.
//      Plane c holds lane group g's C entries at words g (C + 1) .. (C + 1)
//      g + C - 1: with the odd stride C + 1 the 64 lanes' reads of their k-th
//      entry fall in 64 distinct banks whatever their codes.
//   V: per-lane accumulators of the lane's C dimensions, codebook in LDS.
// Each wave runs an online softmax (base 2) over its tokens, GT at a time;
// the block merges its waves and writes (max, sum, acc[P]) for the finalize
// kernel.  The LUT kernel's one lane per token needs a row's codes (and a
// V accumulator per dimension segment) in one lane's registers, which at
// these sizes do not fit.
template <int NB>
__device__ __forceinline__ void load_lane_bytes(const uint8_t *p, uint32_t (&w)[(NB + 3) / 4]) {
  const AQ_AS1 uint8_t *g = (const AQ_AS1 uint8_t *)p;
  if constexpr (NB == 2) {
    w[0] = *reinterpret_cast<const AQ_AS1 uint16_t *>(g);
  } else if constexpr (NB == 3) {
    w[0] = (uint32_t)g[0] | ((uint32_t)g[1] << 8) | ((uint32_t)g[2] << 16);
  } else if constexpr (NB == 4) {
    w[0] = *reinterpret_cast<const AQ_AS1 uint32_t *>(g);
  } else if constexpr (NB == 6) {
    const AQ_AS1 uint16_t *h = reinterpret_cast<const AQ_AS1 uint16_t *>(g);
    w[0] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
    w[1] = h[2];
  } else {
    static_assert(NB == 8, "2, 3, 4, 6 or 8 bytes a lane");
    const u32x2 v = *reinterpret_cast<const AQ_AS1 u32x2 *>(g);
    w[0] = v.x;
    w[1] = v.y;
  }
}

// Code k of a lane's bytes (the row's bytes from the lane's first, as loaded
// by load_lane_bytes): MSB-first in each byte at 2 and 4 bits, big-endian
// 24-bit groups of 8 codes at 3 bits (quantizer.cpp:156-209).
template <int B>
__device__ __forceinline__ uint32_t lane_code(const uint32_t *w, int k) {
  if constexpr (B == 4) {
    return (byte_of(w, k >> 1) >> ((k & 1) ? 0 : 4)) & 15u;
  } else if constexpr (B == 2) {
    return (byte_of(w, k >> 2) >> (6 - 2 * (k & 3))) & 3u;
  } else {
    const int g = 3 * (k >> 3);
    const uint32_t w24 = (byte_of(w, g) << 16) | (byte_of(w, g + 1) << 8) | byte_of(w, g + 2);
    return (w24 >> (21 - 3 * (k & 7))) & 7u;
  }
}

__device__ __forceinline__ int wave_isum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, true);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, true);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, true);  // row_ror:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, true);  // row_ror:8
  return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
         (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

constexpr int kWideTokens = 4;  // tokens a wave takes per step

template <int P, int KB, int VB>
__global__ __launch_bounds__(kThreads) void decode_wide_kernel(HeadDesc *const *item_desc,
                                                               const float *__restrict__ queries,
                                                               int chunk, int n_splits,
                                                               float *__restrict__ partials) {
  static_assert(P == 512 || P == 1024, "padded 512 or 1024");
  static_assert(KB >= 2 && KB <= 4 && VB >= 2 && VB <= 4, "quantised K and V");
  constexpr int C = P / 64;             // dimensions a lane
  constexpr int KBY = C * KB / 8, VBY = C * VB / 8;
  constexpr int KRB = P * KB / 8, VRB = P * VB / 8;
  constexpr int NC = 1 << KB;
  constexpr int LS = C + 1;             // words of a lane group in a code plane
  constexpr int PS = 64 * LS;           // words of a code plane
  constexpr int GT = kWideTokens;
  static_assert(NC * PS >= kWaves * P, "the waves' accumulators fit in the table's space");
  __shared__ int32_t s_k[NC * PS];      // K table; after the tokens, the waves' acc[P]
  __shared__ float s_q[P];
  __shared__ float s_cbv[16];
  __shared__ float2 s_cbv2[16];  // 2-bit V: nibble -> its two codes' centres
  __shared__ float s_ml[kWaves][2];
  __shared__ float s_fix[2];
  const int item = blockIdx.y, split = blockIdx.x;
  const HeadDesc *d = item_desc[item];
  const int dim = d->dim, n = d->st.size;
  const int t_begin = split * chunk, t_end = min(n, t_begin + chunk);
  float *part = partials + ((size_t)item * n_splits + split) * (P + 4);
  if (t_begin >= t_end) {
    for (int i = threadIdx.x; i < P; i += blockDim.x) part[4 + i] = 0.0f;
    if (threadIdx.x == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (threadIdx.x < (1 << VB)) s_cbv[threadIdx.x] = cbv<VB>(threadIdx.x);
  if (VB == 2 && threadIdx.x < 16)
    s_cbv2[threadIdx.x] = make_float2(cbv<2>(threadIdx.x >> 2), cbv<2>(threadIdx.x & 3));
  load_query<P>(s_q, queries + (size_t)item * dim, dim, true, d->signs);  // ends with a barrier
  if (wave == 0) {
    float a = 0.0f;
    for (int i = lane; i < P; i += 64) a += fabsf(s_q[i]);
    a = wave_sum(a) * fabsf(cbv<KB>(0));  // the outermost centre has the largest magnitude
    if (lane == 0) {
      // the largest power of two f with f * max|CB| * sum|qr| <= 2^30
      const float f = a > 0.0f ? ldexpf(1.0f, min(ilogbf(1073741824.0f / a), 100)) : 1.0f;
      s_fix[0] = f;
      s_fix[1] = 1.0f / f;
    }
  }
  __syncthreads();
  {
    const float f = s_fix[0];
    // P is a multiple of the block size, so the code plane c is uniform per pass
    for (int e = threadIdx.x; e < NC * P; e += kThreads) {
      const int c = e / P, i = e - c * P;
      s_k[c * PS + (i / C) * LS + i % C] = (int32_t)rintf((s_q[i] * f) * cbv<KB>(c));
    }
  }
  __syncthreads();

  constexpr float kLog2e = 1.44269504088896340736f;
  const float attn = kLog2e / (sqrtf((float)dim) * (float)P) * s_fix[1];
  const float isp = 1.0f / sqrtf((float)P);
  const uint8_t *krow = d->k_codes + lane * KBY;
  const uint8_t *vrow = d->v_codes + lane * VBY;
  const AQ_AS1 float *k_scale = (const AQ_AS1 float *)d->k_scale;
  const AQ_AS1 float *v_scale = (const AQ_AS1 float *)d->v_scale;
  const int32_t *tk = s_k + lane * LS;
  float acc[C];
#pragma unroll
  for (int k = 0; k < C; ++k) acc[k] = 0.0f;
  float m_run = kMaxSeed2, l_run = 0.0f;
  // A step takes GT tokens; the next step's rows are requested before this
  // step's are used, into the other of two register sets (the loop runs two
  // steps an iteration, so no set is copied).
  struct Rows {
    uint32_t k[GT][(KBY + 3) / 4], v[GT][(VBY + 3) / 4];
    float ks[GT], vs[GT];
  };
  auto fetch = [&](int t0, Rows &r) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const size_t t = (size_t)min(t0 + g, t_end - 1);
      load_lane_bytes<KBY>(krow + t * KRB, r.k[g]);
      load_lane_bytes<VBY>(vrow + t * VRB, r.v[g]);
      r.ks[g] = k_scale[t];
      r.vs[g] = v_scale[t];
    }
  };
  constexpr int kStep = kWaves * GT;
  auto step = [&](int t0, const Rows &r, Rows &next) {
    if (t0 + kStep < t_end) fetch(t0 + kStep, next);
    float lg[GT];
    float gmax = -INFINITY;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      int sum = 0;
#pragma unroll
      for (int k = 0; k < C; ++k) sum += tk[lane_code<KB>(r.k[g], k) * PS + k];
      sum = wave_isum(sum);
      lg[g] = t0 + g < t_end ? (float)sum * attn * r.ks[g] : -INFINITY;
      gmax = fmaxf(gmax, lg[g]);
    }
    if (gmax > m_run) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - gmax);
#pragma unroll
      for (int k = 0; k < C; ++k) acc[k] *= alpha;
      l_run *= alpha;
      m_run = gmax;
    }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (t0 + g >= t_end) break;
      const float e = __builtin_amdgcn_exp2f(lg[g] - m_run);
      l_run += e;
      const float w = e * r.vs[g] * isp;
      if constexpr (VB == 2) {
        // two codes a read: the nibble's pair of centres (s_cbv2)
#pragma unroll
        for (int k = 0; k < C; k += 2) {
          const float2 cv = s_cbv2[(byte_of(r.v[g], k >> 2) >> (4 - 2 * (k & 3))) & 15u];
          acc[k] = fmaf(cv.x, w, acc[k]);
          acc[k + 1] = fmaf(cv.y, w, acc[k + 1]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < C; ++k) acc[k] = fmaf(s_cbv[lane_code<VB>(r.v[g], k)], w, acc[k]);
      }
    }
  };
  Rows ra, rb;
  int t0 = t_begin + wave * GT;
  if (t0 < t_end) fetch(t0, ra);
  for (; t0 < t_end; t0 += 2 * kStep) {
    step(t0, ra, rb);
    if (t0 + kStep >= t_end) break;
    step(t0 + kStep, rb, ra);
  }

  // ---- block merge: waves -> one (m, l, acc) ----
  __syncthreads();  // every wave is done with the K table
  float *s_acc = reinterpret_cast<float *>(s_k);  // [kWaves][P]
#pragma unroll
  for (int k = 0; k < C; ++k) s_acc[wave * P + lane * C + k] = acc[k];
  if (lane == 0) {
    s_ml[wave][0] = m_run;
    s_ml[wave][1] = l_run;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][0]);
  float fw[kWaves], L = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    fw[w] = s_ml[w][0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_ml[w][0] - M);
    L += fw[w] * s_ml[w][1];
  }
  for (int i = threadIdx.x; i < P; i += kThreads) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) a += fw[w] * s_acc[w * P + i];
    part[4 + i] = a;
  }
  if (threadIdx.x == 0) {
    // the finalize kernel merges splits in natural units
    part[0] = M * 0.69314718055994530942f;
    part[1] = L;
  }
}

// Row-dot kernel (padded 512 and 1024 with fp32 keys: K16 rings and the
// hybrid branch's mirror).  A block takes kThreads tokens of one item.
//   1. logits: one thread per token, the reference's sequential unfused dot
//      product over the dim entries (attention.cpp:212-219, :497-502),
//      times 1/sqrt(dim); the query is in LDS (read broadcast), the row
//      streams in 16-byte loads;
//   2. the block's maximum (seeded at -1e30 like the reference) and
//      e = expf(l - max) into LDS;
//   3. the V sum with the dimensions over the lanes, as the wide kernel's:
//      wave w takes tokens w, w + 4, ..., lane l dimensions [C l, C l + C),
//      C = P / 64, one coalesced load per wave and token (fp32 rows, or
//      codes and their scale);
//   4. (max, sum, acc[P]) for the finalize kernel.
// The generic kernel ran the same per-token dot with 8 threads of 256 at a
// time.
template <int P, int VB, bool RAW>
__global__ __launch_bounds__(kThreads) void decode_rowdot_kernel(HeadDesc *const *item_desc,
                                                                 const float *__restrict__ queries,
                                                                 int chunk, int n_splits,
                                                                 float *__restrict__ partials) {
  static_assert(P == 512 || P == 1024, "padded 512 or 1024");
  static_assert(!RAW || VB == 16, "the mirror holds fp32 values");
  constexpr bool VQ = VB != 16;
  constexpr int C = P / 64;
  constexpr int VBY = VQ ? C * VB / 8 : 0;
  constexpr int VRB = VQ ? P * VB / 8 : 0;
  __shared__ float s_q[P];
  __shared__ float s_e[kThreads];
  __shared__ float s_red[kWaves];
  __shared__ float s_cbv[16];
  __shared__ float s_acc[kWaves][P];
  const int item = blockIdx.y, split = blockIdx.x;
  const HeadDesc *d = item_desc[item];
  const ItemView iv = item_view<RAW>(d);
  const int dim = d->dim, n = iv.n;
  const int t_begin = split * chunk, t_end = min(n, t_begin + chunk);
  float *part = partials + ((size_t)item * n_splits + split) * (P + 4);
  if (t_begin >= t_end) {
    for (int i = threadIdx.x; i < P; i += blockDim.x) part[4 + i] = 0.0f;
    if (threadIdx.x == 0) {
      part[0] = -INFINITY;
      part[1] = 0.0f;
    }
    return;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if constexpr (VQ) {
    if (threadIdx.x < (1 << VB)) s_cbv[threadIdx.x] = cbv<VB>(threadIdx.x);
  }
  const float *q = queries + (size_t)item * dim;
  for (int i = threadIdx.x; i < P; i += kThreads) s_q[i] = i < dim ? q[i] : 0.0f;
  __syncthreads();

  // 1. this thread's token's logit
  const int kstride = RAW ? dim : P;  // floats per key row
  const float attn_s = 1.0f / sqrtf((float)dim);
  const int t = t_begin + threadIdx.x;
  float lg = -INFINITY;
  if (t < t_end) {
    const float *row = reinterpret_cast<const float *>(iv.k_rows) + (size_t)t * kstride;
    float dsum = 0.0f;
    int i = 0;
    if ((kstride & 3) == 0) {
      // 16-byte loads, 8 in flight ahead of their products
      for (; i + 32 <= dim; i += 32) {
        float4 r[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) r[k] = reinterpret_cast<const float4 *>(row + i)[k];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          dsum = __fadd_rn(dsum, __fmul_rn(s_q[i + 4 * k], r[k].x));
          dsum = __fadd_rn(dsum, __fmul_rn(s_q[i + 4 * k + 1], r[k].y));
          dsum = __fadd_rn(dsum, __fmul_rn(s_q[i + 4 * k + 2], r[k].z));
          dsum = __fadd_rn(dsum, __fmul_rn(s_q[i + 4 * k + 3], r[k].w));
        }
      }
    }
    for (; i < dim; ++i) dsum = __fadd_rn(dsum, __fmul_rn(s_q[i], row[i]));
    lg = __fmul_rn(dsum, attn_s);
  }

  // 2. the block maximum (the reference's compare from -1e30) and the weights
  float m = t < t_end && lg > kMaxSeed ? lg : kMaxSeed;
  m = wave_max(m);
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  float M = s_red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_red[w]);
  const float e = t < t_end ? expf(lg - M) : 0.0f;
  s_e[threadIdx.x] = e;
  __syncthreads();
  float l = wave_sum(e);
  if (lane == 0) s_red[wave] = l;

  // 3. the V sum, dimensions over the lanes
  float acc[C];
#pragma unroll
  for (int k = 0; k < C; ++k) acc[k] = 0.0f;
  const float isp = VQ ? 1.0f / sqrtf((float)P) : 1.0f;
  for (int tt = t_begin + wave; tt < t_end; tt += kWaves) {
    const float et = s_e[tt - t_begin];
    if constexpr (VQ) {
      uint32_t vw[(VBY + 3) / 4];
      load_lane_bytes<VBY>(iv.v_rows + (size_t)tt * VRB + lane * VBY, vw);
      const float w = et * iv.v_scale[tt] * isp;
#pragma unroll
      for (int k = 0; k < C; ++k) acc[k] = fmaf(s_cbv[lane_code<VB>(vw, k)], w, acc[k]);
    } else {
      const int vstride = RAW ? dim : P;
      const float *vr = reinterpret_cast<const float *>(iv.v_rows) + (size_t)tt * vstride;
      if (!RAW || (dim & 3) == 0) {
        // C = 8 or 16 floats a lane: whole 16-byte loads within the row
#pragma unroll
        for (int k = 0; k < C; k += 4) {
          const int i0 = lane * C + k;
          float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          if (i0 + 4 <= (RAW ? dim : P)) v = *reinterpret_cast<const float4 *>(vr + i0);
          else {
            if (i0 < dim) v.x = vr[i0];
            if (i0 + 1 < dim) v.y = vr[i0 + 1];
            if (i0 + 2 < dim) v.z = vr[i0 + 2];
          }
          acc[k] = fmaf(v.x, et, acc[k]);
          acc[k + 1] = fmaf(v.y, et, acc[k + 1]);
          acc[k + 2] = fmaf(v.z, et, acc[k + 2]);
          acc[k + 3] = fmaf(v.w, et, acc[k + 3]);
        }
      } else {
#pragma unroll
        for (int k = 0; k < C; ++k) {
          const int i = lane * C + k;
          acc[k] = fmaf(i < dim ? vr[i] : 0.0f, et, acc[k]);
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < C; ++k) s_acc[wave][lane * C + k] = acc[k];
  __syncthreads();
  // 4. the block's partial (natural units)
  for (int i = threadIdx.x; i < P; i += kThreads) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) a += s_acc[w][i];
    part[4 + i] = a;
  }
  if (threadIdx.x == 0) {
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) L += s_red[w];
    part[0] = M;
    part[1] = L;
  }
}

// Merge the splits of each item, normalise, undo the rotation.  The split
// maxima, weights and sums are spread over the block (split s on thread
// s mod kThreads); each dimension's weighted sum over the splits is shared by
// kThreads / P thread groups, group g taking splits s = g (mod groups).
constexpr int kMaxSplitWeights = 1024;  // plan_splits never makes more splits

template <bool INVERSE_FWHT>
__global__ __launch_bounds__(kThreads) void finalize_kernel(HeadDesc *const *item_desc, int P,
                                                            int n_splits,
                                                            const float *__restrict__ partials,
                                                            float *__restrict__ outs, int guard) {
  // Latency-bound (a few KB per item): every partial the block reads is
  // requested before any is used, and the descriptor (dim, signs, ring size)
  // only at the end.  An empty ring is one whose splits are all empty (the
  // decode kernels write -inf as an empty split's maximum and seed a
  // non-empty one's at -1e30 or above).
  constexpr int kPre = 16;  // partial sums a thread requests before the weights are known
  __shared__ float s_acc[kMaxPadded];
  __shared__ float s_f[kMaxSplitWeights];
  __shared__ float s_red[kWaves];
  __shared__ float s_grp[kThreads];
  const int item = blockIdx.x;
  const size_t stride = (size_t)P + 4;
  const float *part = partials + (size_t)item * n_splits * stride;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int groups = P < kThreads ? kThreads / P : 1;
  const int gi = threadIdx.x % P, grp = threadIdx.x / P;  // used when groups > 1
  float pre[kPre];
  if (groups > 1) {
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
      const int sp = grp + k * groups;
      pre[k] = sp < n_splits ? part[sp * stride + 4 + gi] : 0.0f;
    }
  }
  float m = -INFINITY;
  for (int sp = threadIdx.x; sp < n_splits; sp += kThreads) m = fmaxf(m, part[sp * stride]);
  m = wave_max(m);
  if (lane == 0) s_red[wave] = m;
  __syncthreads();
  float M = s_red[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  const HeadDesc *d = item_desc[item];
  if (M == -INFINITY) {  // an empty ring: zeros (attention.cpp:482-485)
    const int dim = d->dim;
    float *out = outs + (size_t)item * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = 0.0f;
    return;
  }
  float l = 0.0f;
  for (int sp = threadIdx.x; sp < n_splits; sp += kThreads) {
    const float ms = part[sp * stride];
    const float f = ms == -INFINITY ? 0.0f : expf(ms - M);
    if (sp < kMaxSplitWeights) s_f[sp] = f;
    l += f * part[sp * stride + 1];
  }
  l = wave_sum(l);
  if (lane == 0) s_red[wave] = l;
  __syncthreads();
  float L = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) L += s_red[w];
  auto weight = [&](int sp) -> float {
    if (sp < kMaxSplitWeights) return s_f[sp];
    const float ms = part[sp * stride];
    return ms == -INFINITY ? 0.0f : expf(ms - M);
  };
  if (groups > 1) {
    // P divides kThreads (P is a power of two below it); the splits of this
    // thread's group in order: the requested ones, then the rest
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
      const int sp = grp + k * groups;
      if (sp < n_splits) a += weight(sp) * pre[k];
    }
#pragma unroll 4
    for (int sp = grp + kPre * groups; sp < n_splits; sp += groups)
      a += weight(sp) * part[sp * stride + 4 + gi];
    s_grp[threadIdx.x] = a;
    __syncthreads();
    if (threadIdx.x < P) {
      float t = 0.0f;
      for (int q = 0; q < groups; ++q) t += s_grp[q * P + threadIdx.x];
      s_acc[threadIdx.x] = t;
    }
  } else {
    for (int i = threadIdx.x; i < P; i += kThreads) {
      float a = 0.0f;
#pragma unroll 4
      for (int sp = 0; sp < n_splits; ++sp) a += weight(sp) * part[sp * stride + 4 + i];
      s_acc[i] = a;
    }
  }
  __syncthreads();
  const int dim = d->dim;
  finish_item<INVERSE_FWHT>(s_acc, P, dim, L, d->signs, outs + (size_t)item * dim, guard != 0,
                            d->st.size);
}

struct SplitPlan {
  int splits, chunk;
};

SplitPlan plan_splits(int n_items, int max_n, int min_chunk, int target_blocks) {
  SplitPlan sp;
  int by_work = (max_n + min_chunk - 1) / min_chunk;
  if (by_work < 1) by_work = 1;
  int want = (target_blocks + n_items - 1) / n_items;
  sp.splits = want < by_work ? want : by_work;
  if (sp.splits < 1) sp.splits = 1;
  int chunk = (max_n + sp.splits - 1) / sp.splits;
  chunk = ((chunk + kTile - 1) / kTile) * kTile;
  if (chunk < kTile) chunk = kTile;
  sp.chunk = chunk;
  sp.splits = (max_n + chunk - 1) / chunk;
  if (sp.splits < 1) sp.splits = 1;
  return sp;
}

template <int P, bool RAW>
hipError_t dispatch_lut(const DecodeShape &sh, dim3 grid, HeadDesc *const *descs, const float *q,
                        int chunk, int splits, float *part, float *out, hipStream_t s) {
#define AQ_LUT(KB_, VB_)                                                                         \
  if (sh.k_bits == KB_ && sh.v_bits == VB_) {                                                     \
    decode_lut_kernel<P, KB_, VB_, RAW><<<grid, kLutThreads, 0, s>>>(descs, q, chunk, splits, part, out, \
                                                                   StepAppend{}, sh.dim);            \
    return hipGetLastError();                                                                     \
  }
  if constexpr (RAW) {
    AQ_LUT(16, 16)
  } else {
    AQ_LUT(4, 2) AQ_LUT(4, 3) AQ_LUT(4, 4) AQ_LUT(4, 16)
    AQ_LUT(3, 2) AQ_LUT(3, 3) AQ_LUT(3, 4) AQ_LUT(3, 16)
    AQ_LUT(2, 2) AQ_LUT(2, 3) AQ_LUT(2, 4) AQ_LUT(2, 16)
    AQ_LUT(16, 2) AQ_LUT(16, 3) AQ_LUT(16, 4) AQ_LUT(16, 16)
  }
#undef AQ_LUT
  return hipErrorInvalidValue;
}

template <bool RAW>
hipError_t dispatch_generic(const DecodeShape &sh, dim3 grid, HeadDesc *const *descs,
                            const float *q, int chunk, int splits, float *part, hipStream_t s) {
#define AQ_GEN(KB_, VB_)                                                                           \
  if (sh.k_bits == KB_ && sh.v_bits == VB_) {                                                       \
    decode_generic_kernel<KB_, VB_, RAW><<<grid, kThreads, 0, s>>>(descs, q, chunk, splits, part); \
    return hipGetLastError();                                                                       \
  }
  if constexpr (RAW) {
    AQ_GEN(16, 16)
  } else {
    AQ_GEN(4, 2) AQ_GEN(4, 3) AQ_GEN(4, 4) AQ_GEN(4, 16)
    AQ_GEN(3, 2) AQ_GEN(3, 3) AQ_GEN(3, 4) AQ_GEN(3, 16)
    AQ_GEN(2, 2) AQ_GEN(2, 3) AQ_GEN(2, 4) AQ_GEN(2, 16)
    AQ_GEN(16, 2) AQ_GEN(16, 3) AQ_GEN(16, 4) AQ_GEN(16, 16)
  }
#undef AQ_GEN
  return hipErrorInvalidValue;
}

template <int P>
hipError_t dispatch_wide(const DecodeShape &sh, dim3 grid, HeadDesc *const *descs, const float *q,
                         int chunk, int splits, float *part, hipStream_t s) {
#define AQ_WIDE(KB_, VB_)                                                                        \
  if (sh.k_bits == KB_ && sh.v_bits == VB_) {                                                    \
    decode_wide_kernel<P, KB_, VB_><<<grid, kThreads, 0, s>>>(descs, q, chunk, splits, part);     \
    return hipGetLastError();                                                                    \
  }
  AQ_WIDE(4, 2) AQ_WIDE(4, 3) AQ_WIDE(4, 4)
  AQ_WIDE(3, 2) AQ_WIDE(3, 3) AQ_WIDE(3, 4)
  AQ_WIDE(2, 2) AQ_WIDE(2, 3) AQ_WIDE(2, 4)
#undef AQ_WIDE
  return hipErrorInvalidValue;
}

template <int P>
hipError_t dispatch_rowdot(const DecodeShape &sh, dim3 grid, HeadDesc *const *descs,
                           const float *q, int chunk, int splits, float *part, hipStream_t s) {
  if (chunk > kThreads) return hipErrorInvalidValue;  // one token a thread
  if (sh.raw) {
    decode_rowdot_kernel<P, 16, true><<<grid, kThreads, 0, s>>>(descs, q, chunk, splits, part);
    return hipGetLastError();
  }
#define AQ_ROWDOT(VB_)                                                                              \
  if (sh.v_bits == VB_) {                                                                           \
    decode_rowdot_kernel<P, VB_, false><<<grid, kThreads, 0, s>>>(descs, q, chunk, splits, part);    \
    return hipGetLastError();                                                                       \
  }
  AQ_ROWDOT(2) AQ_ROWDOT(3) AQ_ROWDOT(4) AQ_ROWDOT(16)
#undef AQ_ROWDOT
  return hipErrorInvalidValue;
}

// The row-dot kernel serves padded 512 and 1024 with fp32 keys: K16 rings
// and the hybrid branch's mirror (a block takes kThreads tokens).
bool rowdot_eligible(const DecodeShape &sh) {
  return (sh.padded == 512 || sh.padded == 1024) && (sh.raw || sh.k_bits == 16) &&
         (sh.raw || sh.v_bits == 2 || sh.v_bits == 3 || sh.v_bits == 4 || sh.v_bits == 16);
}

// The wide kernel serves padded 512 and 1024 with quantised K and V.
bool wide_eligible(const DecodeShape &sh) {
  return !sh.raw && (sh.padded == 512 || sh.padded == 1024) && sh.k_bits >= 2 && sh.k_bits <= 4 &&
         sh.v_bits >= 2 && sh.v_bits <= 4;
}

// The LUT kernel serves padded 64, 128 and 256 (raw mirrors only when
// unpadded), the wide kernel padded 512 and 1024 with quantised K and V;
// everything else takes the generic kernel.
bool lut_eligible(const DecodeShape &sh) {
  if (!((sh.padded == 64 || sh.padded == 128 || sh.padded == 256) &&
        (!sh.raw || sh.dim == sh.padded)))
    return false;
  // the LUT kernel addresses rows with 32-bit byte offsets
  const long long row = sh.raw ? 4LL * sh.padded
                               : std::max(packed_bytes(sh.padded, sh.k_bits), packed_bytes(sh.padded, sh.v_bits));
  return (long long)(sh.max_n > 0 ? sh.max_n : 1) * row < (1LL << 32);
}

SplitPlan decode_plan(int n_items, const DecodeShape &sh) {
  const int max_n = sh.max_n > 0 ? sh.max_n : 1;
  const bool lut = lut_eligible(sh);
  // Short rings at padded 64: one block per item streams up to four tiles per
  // wave, cheaper than a finalize launch (measured: 4 heads x 1,100 tokens
  // 13.8 -> 11.2 us; at padded 128 the extra tiles cost more than it saves)
  // fp32 mirrors at padded 64 carry 512 bytes a token: chunks down to one
  // tile, about one block a CU, merged by the finalize launch (measured:
  // config 2's hybrid step, 24 calls of 14 heads x 512 tokens, 268 -> 252 us
  // with 128-token chunks, 241-248 us with 64; one block per head before)
  if (lut && sh.raw && sh.padded == 64) return plan_splits(n_items, max_n, kTile, 256);
  if (lut && sh.padded == 64 && max_n <= 4 * kLutWaves * kTile) {
    SplitPlan sp;
    sp.splits = 1;
    sp.chunk = ((max_n + kTile - 1) / kTile) * kTile;
    return sp;
  }
  // LUT kernel: about one 512-thread block per CU (256 CUs): each extra block
  // repeats the query rotation and the K table build, and the splits add
  // finalize work (measured: 4 heads x 131,072 tokens 48 -> 27 us, 64 heads x
  // 8,192 tokens 35 -> 25 us, 8 heads x 32,768 tokens 28 -> 25 us against a
  // target of 1,024 blocks; none of the sampled shapes slower).
  if (lut) return plan_splits(n_items, max_n, kLutWaves * kTile, 256);
  // wide kernel: each block builds a table of 2^KB x P entries, so a block
  // takes at least 512 tokens; 4 blocks a CU at padded 512 (a 4-bit table
  // takes 36 KB of LDS), 2 at padded 1024 (68 KB)
  if (wide_eligible(sh)) return plan_splits(n_items, max_n, 512, sh.padded == 512 ? 1024 : 512);
  // row-dot kernel: one token a thread, so chunks of exactly kThreads tokens
  if (rowdot_eligible(sh)) {
    SplitPlan sp;
    sp.chunk = kThreads;
    sp.splits = (max_n + kThreads - 1) / kThreads;
    if (sp.splits < 1) sp.splits = 1;
    return sp;
  }
  return plan_splits(n_items, max_n, 256, 1024);
}

}  // namespace

hipError_t launch_finalize(HeadDesc *const *descs, int n_items, int padded, int n_splits,
                           const float *partials, float *outs, bool inverse_fwht, hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  if (inverse_fwht)
    finalize_kernel<true><<<n_items, kThreads, 0, s>>>(descs, padded, n_splits, partials, outs, 0);
  else
    finalize_kernel<false><<<n_items, kThreads, 0, s>>>(descs, padded, n_splits, partials, outs, 0);
  return hipGetLastError();
}

size_t decode_workspace_floats(int n_items, const DecodeShape &shape) {
  DecodeShape sh = shape;
  if (sh.raw) sh.k_bits = sh.v_bits = 16;  // as launch_decode plans it
  const SplitPlan sp = decode_plan(n_items, sh);
  // one split through the LUT kernel: the kernel finishes its items itself
  if (sp.splits == 1 && lut_eligible(sh)) return 0;
  return (size_t)n_items * sp.splits * (sh.padded + 4);
}

// Items per launch: the grid's y dimension holds items (at most 65,535).
constexpr int kMaxItemsPerLaunch = 65535;

hipError_t launch_decode_items(HeadDesc *const *descs, int n_items, const DecodeShape &sh,
                               const SplitPlan &sp, const float *d_q, float *d_out, float *d_ws,
                               hipStream_t s);

hipError_t launch_decode(HeadDesc *const *descs, int n_items, const DecodeShape &shape,
                         const float *d_q, float *d_out, float *d_ws, hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  DecodeShape sh = shape;
  if (sh.raw) sh.k_bits = sh.v_bits = 16;  // the mirror holds fp32 keys and values
  const SplitPlan sp = decode_plan(n_items, sh);
  // one split plan for all items; chunks of items take consecutive
  // queries, outputs and workspace
  for (int c0 = 0; c0 < n_items; c0 += kMaxItemsPerLaunch) {
    const int cnt = n_items - c0 < kMaxItemsPerLaunch ? n_items - c0 : kMaxItemsPerLaunch;
    float *ws = d_ws ? d_ws + (size_t)c0 * sp.splits * (sh.padded + 4) : nullptr;
    const hipError_t e = launch_decode_items(descs + c0, cnt, sh, sp, d_q + (size_t)c0 * sh.dim,
                                             d_out + (size_t)c0 * sh.dim, ws, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <int P>
hipError_t dispatch_lut_step(const DecodeShape &sh, dim3 grid, HeadDesc *const *descs,
                             const float *q, int chunk, float *out, const StepAppend &app,
                             hipStream_t s) {
#define AQ_STEP(KB_, VB_)                                                                        \
  if (sh.k_bits == KB_ && sh.v_bits == VB_) {                                                     \
    decode_lut_kernel<P, KB_, VB_, false, true><<<grid, kLutThreads, 0, s>>>(descs, q, chunk, 1,  \
                                                                            nullptr, out, app,    \
                                                                            sh.dim);              \
    return hipGetLastError();                                                                     \
  }
  AQ_STEP(4, 2) AQ_STEP(4, 3) AQ_STEP(4, 4)
  AQ_STEP(3, 2) AQ_STEP(3, 3) AQ_STEP(3, 4)
  AQ_STEP(2, 2) AQ_STEP(2, 3) AQ_STEP(2, 4)
#undef AQ_STEP
  return hipErrorNotSupported;
}

bool decode_step_supported(int n_items, const DecodeShape &sh) {
  // padded 64 only: at 128 the fused kernels spill (the key rows of 16
  // words and the codec's registers), and rings there rarely plan one block
  // per item
  return n_items > 0 && n_items <= kMaxItemsPerLaunch && !sh.raw && sh.k_bits != 16 &&
         sh.v_bits != 16 && sh.padded == 64 && lut_eligible(sh) &&
         decode_plan(n_items, sh).splits == 1;
}

hipError_t launch_decode_step(HeadDesc *const *descs, int n_items, const DecodeShape &sh,
                              const StepAppend &app, const float *d_q, float *d_out,
                              hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  if (!decode_step_supported(n_items, sh)) return hipErrorNotSupported;
  const SplitPlan sp = decode_plan(n_items, sh);
  const dim3 grid(1, n_items);
  return dispatch_lut_step<64>(sh, grid, descs, d_q, sp.chunk, d_out, app, s);
}

hipError_t launch_decode_items(HeadDesc *const *descs, int n_items, const DecodeShape &sh,
                               const SplitPlan &sp, const float *d_q, float *d_out, float *d_ws,
                               hipStream_t s) {
  const bool raw = sh.raw;
  const bool lut_ok = lut_eligible(sh);
  const dim3 grid(sp.splits, n_items);
  hipError_t e;
  if (lut_ok) {
    if (sh.padded == 64)
      e = raw ? dispatch_lut<64, true>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, d_out, s)
              : dispatch_lut<64, false>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, d_out, s);
    else if (sh.padded == 256)
      e = raw ? dispatch_lut<256, true>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, d_out, s)
              : dispatch_lut<256, false>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, d_out, s);
    else
      e = raw ? dispatch_lut<128, true>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, d_out, s)
              : dispatch_lut<128, false>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, d_out, s);
    if (e != hipSuccess || sp.splits == 1) return e;  // one split: the kernel finished the items
  } else if (wide_eligible(sh)) {
    e = sh.padded == 512 ? dispatch_wide<512>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, s)
                         : dispatch_wide<1024>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, s);
  } else if (rowdot_eligible(sh)) {
    e = sh.padded == 512 ? dispatch_rowdot<512>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, s)
                         : dispatch_rowdot<1024>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, s);
  } else {
    e = raw ? dispatch_generic<true>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, s)
            : dispatch_generic<false>(sh, grid, descs, d_q, sp.chunk, sp.splits, d_ws, s);
  }
  if (e != hipSuccess) return e;
  const bool fwht = !raw && sh.v_bits != 16;
  if (fwht)
    finalize_kernel<true><<<n_items, kThreads, 0, s>>>(descs, sh.padded, sp.splits, d_ws, d_out, 0);
  else
    finalize_kernel<false><<<n_items, kThreads, 0, s>>>(descs, sh.padded, sp.splits, d_ws, d_out,
                                                        raw ? 1 : 0);
  return hipGetLastError();
}

}  // namespace aq

#ifdef AQ_CLOCK_STAMPS
// The timing library's reader of the clock stamps (no counterpart in the
// reference; declared nowhere else): set the launch index the next decode
// launches record under, and copy the stamps out (n = kClkLaunches x
// kClkBlocks x 4 words).
extern "C" int adaptq_clock_stamp_set(int launch, void *stream) {
  aq::clk_set_kernel<<<1, 1, 0, (hipStream_t)stream>>>(launch);
  return (int)hipGetLastError();
}
extern "C" int adaptq_clock_stamp_read(unsigned long long *host, size_t n) {
  const size_t cap = (size_t)aq::kClkLaunches * aq::kClkBlocks * 4;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(aq::g_clk), (n < cap ? n : cap) * 8, 0,
                                  hipMemcpyDeviceToHost);
}
#endif
