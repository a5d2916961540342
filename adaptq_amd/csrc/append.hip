// append.hip -- bit-exact quantise-and-insert kernel for gfx950.
//
// One lane encodes one vector end to end in VGPRs: the reference's codec is
// order-sensitive only in its two left-to-right float sums (||x||^2 and the
// clip sigma, core/quantizer.cpp:59-63 and :81-84), which a lane computes in
// the same order; the FWHT butterflies are element-wise and so give the same
// bits however they are scheduled.  Lanes map to consecutive tokens of one
// head, so a wave reads 64 consecutive input rows and writes 64 consecutive
// ring slots.
//
// Restated reference steps (file:line under /root/reference):
//   s = sum x_i*x_i left to right         quantizer.cpp:59-63
//   norm = sqrtf(s + 1e-12f); x *= 1/norm quantizer.cpp:66-69
//   signs + butterflies, * RN(1/RN(sqrtp)) fwht.cpp:33-66
//   * sqrtf(p)                            quantizer.cpp:73-75
//   sigma, +-3 sigma clamp                quantizer.cpp:81-89
//   binary-search index, NaN -> 1/3/7     codebook.cpp:119-144 (quant.hpp;
//                                         4-bit codes by one table lookup)
//   MSB-first pack                        quantizer.cpp:156-209
//   ring insert, mirror                   ring_buffer.cpp:105-119, attention.cpp:338-366
#include <algorithm>

#include "encode_one.hpp"
#include "launch.hpp"
#include "quant.hpp"
#include "rows.hpp"

namespace aq {

namespace {

// Store nbytes (a compile-time count) from w[] to dst with the widest stores
// the row alignment allows.
template <int NB>
__device__ __forceinline__ void store_row(uint8_t *dst, const uint32_t (&w)[(NB + 3) / 4],
                                          int slot) {
  if constexpr (NB % 16 == 0) {
    uint4 *p = reinterpret_cast<uint4 *>(dst + (size_t)slot * NB);
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) p[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  } else if constexpr (NB % 8 == 0) {
    uint2 *p = reinterpret_cast<uint2 *>(dst + (size_t)slot * NB);
#pragma unroll
    for (int i = 0; i < NB / 8; ++i) p[i] = make_uint2(w[2 * i], w[2 * i + 1]);
  } else if constexpr (NB % 4 == 0) {
    uint32_t *p = reinterpret_cast<uint32_t *>(dst + (size_t)slot * NB);
#pragma unroll
    for (int i = 0; i < NB / 4; ++i) p[i] = w[i];
  } else {
    uint8_t *p = dst + (size_t)slot * NB;
#pragma unroll
    for (int i = 0; i < NB; ++i) p[i] = (uint8_t)(w[i / 4] >> (8 * (i % 4)));
  }
}

// Store a K row with its bytes in the slot's XOR order (kperm_mask): word i,
// bytes permuted within the word by x & 3, goes to word position i ^ (x >> 2).
// The words are put in stored order in registers (a conditional swap per bit
// of x >> 2), so the row leaves as whole 16-byte stores.
template <int NB>
__device__ __forceinline__ void store_row_perm(uint8_t *dst, const uint32_t (&w)[NB / 4], int slot,
                                               uint32_t x) {
  constexpr int NW = NB / 4;
  const uint32_t sel = 0x03020100u ^ ((x & 3u) * 0x01010101u);
  const uint32_t xw = x >> 2;
  uint32_t o[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) o[i] = __builtin_amdgcn_perm(0u, w[i], sel);
  // o[i] <- o[i ^ xw]: one conditional swap level per bit of xw
#pragma unroll
  for (int b = 0; (1 << b) < NW; ++b) {
    const bool f = (xw >> b) & 1u;
#pragma unroll
    for (int i = 0; i < NW; ++i)
      if ((i & (1 << b)) == 0) {
        const uint32_t a = o[i], c = o[i | (1 << b)];
        o[i] = f ? c : a;
        o[i | (1 << b)] = f ? a : c;
      }
  }
  if constexpr (NB % 16 == 0) {
    uint4 *p = reinterpret_cast<uint4 *>(dst + (size_t)slot * NB);
#pragma unroll
    for (int i = 0; i < NB / 16; ++i) p[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
  } else {
    uint32_t *p = reinterpret_cast<uint32_t *>(dst + (size_t)slot * NB);
#pragma unroll
    for (int i = 0; i < NW; ++i) p[i] = o[i];
  }
}

template <int P, int B>
struct Row {
  static constexpr int bytes = B == 16 ? 4 * P : (P * B + 7) / 8;
  static constexpr int words = (bytes + 3) / 4;
};

// A pointer the caller knows to be equal across the wave, as scalar registers.
template <class T>
__device__ __forceinline__ T *wave_uniform(T *p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<T *>(((uint64_t)hi << 32) | lo);
}

// Codebook indices of the P values in buf (finite), clamped to [nclip, clip]
// when CLAMP, packed MSB-first into little-endian words
// (quantizer.cpp:156-209): 4 bits = two codes per byte, high nibble first;
// 2 bits = four per byte; 3 bits = eight per 24-bit big-endian group.
// BD (2 bits): buf holds the values before the two scalings and the codes
// come from quantize_bd2 (thresholds q0 < q1 < q2); the clamp, when CLAMP, is
// then applied to the codes: a code is a nondecreasing function of the value,
// so the code of the clamped value is the code clamped to
// [code(nclip), code(clip)] (passed as cl, ch).
// s_q4: the 4-bit cell table (quantize_g4).
template <int P, int B, bool CLAMP, bool BD = false>
__device__ __forceinline__ void pack_codes(const float (&buf)[P], uint32_t (&w)[Row<P, B>::words],
                                           const Q4Cell *s_q4, float nclip, float clip,
                                           float q0 = 0.0f, float q1 = 0.0f, float q2 = 0.0f,
                                           uint32_t cl = 0u, uint32_t ch = 0u) {
  static_assert(!BD || B == 2, "b-domain codes for 2 bits");
#pragma unroll
  for (int i = 0; i < P; ++i) {
    uint32_t q;
    if constexpr (BD) {
      q = quantize_bd2(buf[i], q0, q1, q2);
      if constexpr (CLAMP) q = q < cl ? cl : q > ch ? ch : q;
    } else {
      // the reference's two-sided clamp is the median for finite values
      const float v = CLAMP ? __builtin_amdgcn_fmed3f(buf[i], nclip, clip) : buf[i];
      q = B == 4 ? quantize_g4(v, s_q4) : B == 3 ? quantize_ss3(v) : quantize_ss2(v);
    }
    // Bit position of code i inside the little-endian word stream.
    int byte, shift;
    if constexpr (B == 4) {
      byte = i / 2;
      shift = (i % 2) ? 0 : 4;
    } else if constexpr (B == 2) {
      byte = i / 4;
      shift = 6 - 2 * (i % 4);
    } else {
      // 3-bit: group g = i/8 is the 24-bit big-endian word s0<<21|...|s7.
      const int g = i / 8, k = i % 8;
      const int bit = 21 - 3 * k;  // position inside the 24-bit word
      // byte 0 of the group holds bits 23..16, byte 1 bits 15..8, byte 2 7..0
      const int lo_byte = 2 - bit / 8, lo_shift = bit % 8;
      if (lo_shift + 3 <= 8) {
        byte = 3 * g + lo_byte;
        shift = lo_shift;
      } else {
        // the code straddles two bytes: low part here, high part in byte-1
        const int b0 = 3 * g + lo_byte;
        const int nlow = 8 - lo_shift;
        w[b0 / 4] |= (q & ((1u << nlow) - 1u)) << (8 * (b0 % 4) + lo_shift);
        const int b1 = b0 - 1;
        w[b1 / 4] |= (q >> nlow) << (8 * (b1 % 4));
        continue;
      }
    }
    w[byte / 4] |= q << (8 * (byte % 4) + shift);
  }
}

// Encode one vector (P values in buf, zero-padded) of side `side` into ring
// slot `slot`: the reference's quantize_into (quantizer.cpp:53-137) on the
// lane's own registers, then the row and its scale leave as whole stores.
// BD (2 bits): q0..q2 are the thresholds of the values before the two
// scalings (quant.hpp, BdThr); a wave whose clamp is inert codes those values
// and skips the scalings.
// U: the wave's rows are all of one head, so the ring's base pointers are
// held in scalar registers across the codec (not in four VGPRs, which the
// three-wave register budget would spill).
template <int P, int B, bool BD = false, bool U = false>
__device__ __forceinline__ void encode_vec(float (&buf)[P], const HeadDesc *d, int side, int slot,
                                           float inv_sqrt_p, float sqrt_p, const Q4Cell *s_q4,
                                           float q0 = 0.0f, float q1 = 0.0f, float q2 = 0.0f) {
  uint8_t *codes = side == 0 ? d->k_codes : d->v_codes;
  float *scales = side == 0 ? d->k_scale : d->v_scale;
  if constexpr (U) {
    codes = wave_uniform(codes);
    scales = wave_uniform(scales);
  }

  if constexpr (B == 16) {
    uint32_t w[Row<P, 16>::words];
#pragma unroll
    for (int i = 0; i < P; ++i) w[i] = __float_as_uint(buf[i]);
    store_row<Row<P, 16>::bytes>(codes, w, slot);
    scales[slot] = 1.0f;
    return;
  } else {
    // ||x||^2 left to right; padded zeros add +0 and change nothing.
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < P; ++i) s = __fadd_rn(s, __fmul_rn(buf[i], buf[i]));
    const float norm = sqrtf(__fadd_rn(s, 1e-12f));
    const float inv = 1.0f / norm;

    // Normalise; the sign D[i] = -1 is an exact flip of the sign bit.
    uint32_t sg[(P + 31) / 32];
#pragma unroll
    for (int k = 0; k < (P + 31) / 32; ++k) sg[k] = d->signs[k];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const uint32_t flip = (~sg[i / 32] >> (i % 32)) << 31;
      buf[i] = __uint_as_float(__float_as_uint(__fmul_rn(buf[i], inv)) ^ flip);
    }
#pragma unroll
    for (int len = 1; len < P; len <<= 1) {
#pragma unroll
      for (int base = 0; base < P; base += 2 * len) {
#pragma unroll
        for (int j = base; j < base + len; ++j) {
          const float lo = buf[j], hi = buf[j + len];
          buf[j] = __fadd_rn(lo, hi);
          buf[j + len] = __fsub_rn(lo, hi);
        }
      }
    }
    // The clamp to +-3 sigma (quantizer.cpp:81-89) can change a code only if
    // clip = 3 sigma is not above the largest threshold (0.9816 / 1.7484 /
    // 2.1476 for 2 / 3 / 4 bits): then every |v| > clip codes as clip does.
    // sigma is bounded without summing: for s >= 1e-10, ||x/norm||^2 >=
    // s / (s + 1e-12) less the roundings of s, norm, inv and the products
    // (< 150 u) >= 0.9899; the butterflies move the norm of H D x/norm by
    // less than 7 u relative (log2 p stages of u each, a stage scaling norms
    // by sqrt 2), the two scalings and the sequential sum of squares by less
    // than (p + 3) u; so sigma^2 = s2 / p + 1e-12 >= 0.9898 and clip >= 2.98.
    // A wave whose rows all have s >= 1e-10 skips sigma and the clamp; any
    // other wave (tiny or NaN rows) takes the reference's steps as written.
    // Either way the codes are the reference's.
    const bool clamp_inert = __all(s >= 1e-10f);
    uint32_t w[Row<P, B>::words];
#pragma unroll
    for (int k = 0; k < Row<P, B>::words; ++k) w[k] = 0u;
    bool nan_row;
    // A NaN anywhere in the input reaches every element through the FWHT.
    if constexpr (BD) {
      // codes of the values before the scalings by 1/sqrt(p) and sqrt(p)
      if (clamp_inert) {
        nan_row = buf[0] != buf[0];
        pack_codes<P, B, false, true>(buf, w, s_q4, 0.0f, 0.0f, q0, q1, q2);
      } else {
        float s2 = 0.0f;
#pragma unroll
        for (int i = 0; i < P; ++i) {
          const float v = __fmul_rn(__fmul_rn(buf[i], inv_sqrt_p), sqrt_p);
          s2 = __fadd_rn(s2, __fmul_rn(v, v));
        }
        const float sigma = sqrtf(__fadd_rn(s2 / (float)P, 1e-12f));
        const float clip = __fmul_rn(3.0f, sigma);
        nan_row = s2 != s2;
        pack_codes<P, B, true, true>(buf, w, s_q4, 0.0f, 0.0f, q0, q1, q2, quantize<B>(-clip),
                                     quantize<B>(clip));
      }
    } else {
#pragma unroll
      for (int i = 0; i < P; ++i) buf[i] = __fmul_rn(__fmul_rn(buf[i], inv_sqrt_p), sqrt_p);
      if (clamp_inert) {
        nan_row = buf[0] != buf[0];
        pack_codes<P, B, false>(buf, w, s_q4, 0.0f, 0.0f);
      } else {
        float s2 = 0.0f;
#pragma unroll
        for (int i = 0; i < P; ++i) s2 = __fadd_rn(s2, __fmul_rn(buf[i], buf[i]));
        const float sigma = sqrtf(__fadd_rn(s2 / (float)P, 1e-12f));
        const float clip = __fmul_rn(3.0f, sigma);
        nan_row = s2 != s2;
        pack_codes<P, B, true>(buf, w, s_q4, -clip, clip);
      }
    }
    // A NaN row: every code is the NaN code.
    if (nan_row) {
#pragma unroll
      for (int k = 0; k < Row<P, B>::words; ++k) w[k] = nan_word<B>(k);
    }
    constexpr int xmask = kperm_mask(P, B);
    bool stored = false;
    if constexpr (xmask != 0) {
      if (side == 0) {
        store_row_perm<Row<P, B>::bytes>(codes, w, slot, (uint32_t)slot & (uint32_t)xmask);
        stored = true;
      }
    }
    if (!stored) store_row<Row<P, B>::bytes>(codes, w, slot);
    scales[slot] = norm;
  }
}

// Encode n_tok tokens of one side (K or V) for n_ctx heads.
// UNIFORM: block (x, y) holds tokens x * 128 .. of head y, so a wave never
// mixes heads: the descriptor and sign words are scalar loads and a sign flip
// is one XOR with a scalar mask.  Otherwise lanes run over (head, token)
// pairs in order (for few tokens per head).
//
// commit != 0 (the caller's guarantee: each head's tokens are all in one block,
// i.e. UNIFORM with n_tok <= 128, or one token per head): this launch also
// advances each head's ring state, once every thread of the head has read the
// old one, and no commit_kernel follows.
// Encode token t of context c (ring state st as read before any commit) for
// one side; the caller has placed the thread on (c, t).
template <int P, int B, bool UNIFORM, bool BD = false>
__device__ __forceinline__ void encode_row(const HeadDesc *d, const RingState st, int c, int t,
                                           int side, const float *__restrict__ src, int n_tok,
                                           int dim, float inv_sqrt_p, float sqrt_p,
                                           const Q4Cell *s_q4, float q0 = 0.0f, float q1 = 0.0f,
                                           float q2 = 0.0f) {
  const int cap = d->cap;
  const float *x = src + ((size_t)c * n_tok + t) * dim;

  // Token t survives the batch only if fewer than cap tokens follow it.
  const bool write_ring = cap > 0 && t >= n_tok - cap;
  const int slot = cap > 0 ? (int)(((long long)st.head + t) % cap) : 0;
  const bool write_mirror = t < mirror_count(st, n_tok, cap, d->hyb);
  if constexpr (UNIFORM) {
    // a wave whose tokens the same call evicts and the mirror does not take
    // reads nothing (the lanes of a wave all return or none do)
    if (!__any(write_ring || write_mirror)) return;
  }

  float buf[P];
  // a wave whose 64 rows are all in the batch loads them by row segments
  bool by_groups = false;
  if constexpr (UNIFORM && (P == 64 || P == 128)) {
    const int t0 = blockIdx.x * blockDim.x + (threadIdx.x & ~63);
    if (dim == P && t0 + 64 <= n_tok) {
      load_wave_rows<P>(src + ((size_t)c * n_tok + t0) * P, threadIdx.x & 63, buf);
      by_groups = true;
    }
  }
  if (by_groups) {
  } else if (dim == P && (P % 4) == 0) {
#pragma unroll
    for (int i = 0; i < P; i += 4) {
      float4 v = *reinterpret_cast<const float4 *>(x + i);
      buf[i] = v.x;
      buf[i + 1] = v.y;
      buf[i + 2] = v.z;
      buf[i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < P; ++i) buf[i] = i < dim ? x[i] : 0.0f;
  }

  if (write_mirror) {
    float *m = (side == 0 ? d->raw_k : d->raw_v) + (size_t)(st.raw_count + t) * dim;
    for (int i = 0; i < dim; ++i) m[i] = x[i];
  }
  if (!write_ring) return;

  // scalar base pointers where the codec would otherwise spill them (4-bit
  // codes: K side 1,035 -> 1,011 us on config 5; the 2-bit codec fits without)
  encode_vec<P, B, BD, UNIFORM && B == 4>(buf, d, side, slot, inv_sqrt_p, sqrt_p, s_q4, q0, q1,
                                           q2);
}

// Three waves per SIMD instead of two at the compiler's own 192-200 VGPRs:
// measured on config 5's bulk append, K side 1,101 -> 1,030 us, V side 996 ->
// 988 us.  Within the 168-VGPR budget the 4-bit codec fits without scratch
// (with its ring pointers in scalar registers) and the 2-bit codec needs 158
// VGPRs.
//
// 4-bit codes come from the quarter-unit cell table (quantize_g4: an fma, a
// clamp, a conversion and one 8-byte LDS read per value, instead of the
// sign-split key and a bucket table over the exponent and mantissa bits):
// measured on config 5's bulk append, K side 1,003 -> 993 us.
//
// 2-bit codes come from the values before the two scalings (bd: the
// thresholds for this launch's inv_sqrt_p and sqrt_p, quant.hpp): two
// multiplies and the sign-split key fewer per element; measured on config 5's
// bulk append, V side 988 -> 874 us.
template <int P, int B, bool UNIFORM>
__global__ __launch_bounds__(128, 3) void append_kernel(HeadDesc *const *descs, int n_ctx,
                                                     int side, const float *__restrict__ src,
                                                     int n_tok, int dim, float inv_sqrt_p,
                                                     float sqrt_p, int commit, BdThr bd) {
  constexpr bool BD = B == 2;
  // 4-bit codes: the cell table of quantize_g4, in LDS before any lane leaves
  __shared__ Q4Cell s_q4[B == 4 ? kQ4Cells : 1];
  if constexpr (B == 4) {
    static constexpr Q4Table kTab = q4_table();
    if (threadIdx.x < kQ4Cells) s_q4[threadIdx.x] = kTab.c[threadIdx.x];
    __syncthreads();
  }
  int c, t;
  if constexpr (UNIFORM) {
    c = blockIdx.y;
    t = blockIdx.x * blockDim.x + threadIdx.x;
  } else {
    const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= (long long)n_ctx * n_tok) return;
    c = (int)(g / n_tok);
    t = (int)(g - (long long)c * n_tok);
  }
  const HeadDesc *d = descs[c];
  const RingState st = d->st;
  const int cap = d->cap;
  if (commit) {
    if constexpr (UNIFORM) {
      __syncthreads();  // the block's threads all hold the old state
      if (threadIdx.x == 0) descs[c]->st = ring_after(st, n_tok, cap, d->hyb);
    } else {
      descs[c]->st = ring_after(st, n_tok, cap, d->hyb);  // one token: this lane's head only
    }
  }
  if constexpr (UNIFORM) {
    if (t >= n_tok) return;
  }
  encode_row<P, B, UNIFORM, BD>(d, st, c, t, side, src, n_tok, dim, inv_sqrt_p, sqrt_p, s_q4,
                                bd.q2[0], bd.q2[1], bd.q2[2]);
}

// Both sides of a head-per-block append in one launch: blockIdx.z 0 codes
// the K rows (KB bits), 1 the V rows, each block as append_kernel's UNIFORM
// blocks do (one head, 128 tokens).  No block advances the ring states (a V
// block could run before a K block of the same head has read them):
// commit_kernel follows.  One launch instead of two lets the second side's
// blocks fill the CUs while the first side's last blocks drain.
template <int P, int KB, int VB>
__global__ __launch_bounds__(128, 3) void append_pair_kernel(HeadDesc *const *descs,
                                                          const float *__restrict__ keys,
                                                          const float *__restrict__ vals,
                                                          int n_tok, int dim, float inv_sqrt_p,
                                                          float sqrt_p, BdThr bd) {
  __shared__ Q4Cell s_q4[(KB == 4 || VB == 4) ? kQ4Cells : 1];
  if constexpr (KB == 4 || VB == 4) {
    static constexpr Q4Table kTab = q4_table();
    if (threadIdx.x < kQ4Cells) s_q4[threadIdx.x] = kTab.c[threadIdx.x];
    __syncthreads();
  }
  const int c = blockIdx.y;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const HeadDesc *d = descs[c];
  const RingState st = d->st;
  if (t >= n_tok) return;
  if (blockIdx.z == 0)
    encode_row<P, KB, true, KB == 2>(d, st, c, t, 0, keys, n_tok, dim, inv_sqrt_p, sqrt_p, s_q4,
                                     bd.q2[0], bd.q2[1], bd.q2[2]);
  else
    encode_row<P, VB, true, VB == 2>(d, st, c, t, 1, vals, n_tok, dim, inv_sqrt_p, sqrt_p, s_q4,
                                     bd.q2[0], bd.q2[1], bd.q2[2]);
}

// Both sides of one token per head in one launch (n_tok == 1, lanes over
// heads): each lane encodes its head's K row, then its V row, and advances the
// head's ring state, which no other lane reads.  Halves the launches of a
// decode step's append.
template <int P, int KB, int VB>
__global__ __launch_bounds__(128) void append_kv_kernel(HeadDesc *const *descs, int n_ctx,
                                                        const float *__restrict__ keys,
                                                        const float *__restrict__ vals,
                                                        int dim, float inv_sqrt_p, float sqrt_p) {
  __shared__ Q4Cell s_q4[(KB == 4 || VB == 4) ? kQ4Cells : 1];
  if constexpr (KB == 4 || VB == 4) {
    static constexpr Q4Table kTab = q4_table();
    if (threadIdx.x < kQ4Cells) s_q4[threadIdx.x] = kTab.c[threadIdx.x];
    __syncthreads();
  }
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n_ctx) return;
  const HeadDesc *d = descs[c];
  const RingState st = d->st;
  descs[c]->st = ring_after(st, 1, d->cap, d->hyb);
  encode_row<P, KB, false>(d, st, c, 0, 0, keys, 1, dim, inv_sqrt_p, sqrt_p, s_q4);
  encode_row<P, VB, false>(d, st, c, 0, 1, vals, 1, dim, inv_sqrt_p, sqrt_p, s_q4);
}

// Few vectors: a wave per vector (wave 0 the key, wave 1 the value of token
// blockIdx.y of head blockIdx.x), lane l holding entries l and l + 64.  The
// same float steps as encode_vec in the same order: the sums of squares left
// to right (every lane runs the chain over the squares in LDS), the
// butterflies of span 1, 2, ... between lanes (shfl_xor) and, at padded 128,
// inside the lane; codes are gathered in LDS and lane k packs word k of the
// row.  A lane per vector (append_kv_kernel, append_kernel) leaves each wave
// with the whole codec's dependency chain for 64 vectors, which few vectors
// cannot hide (about 10 us for one token of 4 heads, 36 us for 2,048 tokens
// of 4 heads).  With one token the kernel advances the ring states itself;
// with more, commit_kernel follows.
template <int P, int KB, int VB>
__global__ __launch_bounds__(128) void append_one_kernel(HeadDesc *const *descs,
                                                         const float *__restrict__ keys,
                                                         const float *__restrict__ vals, int dim,
                                                         int n_tok, float inv_sqrt_p,
                                                         float sqrt_p) {
  __shared__ Q4Cell s_q4[(KB == 4 || VB == 4) ? kQ4Cells : 1];
  __shared__ __align__(16) float s_sq[2][P];
  __shared__ uint8_t s_code[2][P];
  const int c = blockIdx.x, t = blockIdx.y;
  const int lane = threadIdx.x & 63, side = threadIdx.x >> 6;
  if constexpr (KB == 4 || VB == 4) {
    static constexpr Q4Table kTab = q4_table();
    if (threadIdx.x < kQ4Cells) s_q4[threadIdx.x] = kTab.c[threadIdx.x];
  }
  HeadDesc *d = descs[c];
  const RingState st = d->st;
  __syncthreads();  // both waves have the old state and the table
  const int cap = d->cap;
  if (n_tok == 1 && threadIdx.x == 0) d->st = ring_after(st, 1, cap, d->hyb);
  const float *x = (side == 0 ? keys : vals) + ((size_t)c * n_tok + t) * dim;
  encode_one_row<P, KB, VB>(d, st, n_tok, t, x, dim, side, lane, inv_sqrt_p, sqrt_p, s_q4,
                            s_sq[side], s_code[side], nullptr, nullptr);
}

// Same codec for padded dimensions above 128: identical float steps in the
// same order, with the vector in per-lane scratch instead of VGPRs (wide heads
// are rare; the unrolled register kernel would cost minutes of compile time).
template <int B>
__global__ __launch_bounds__(128) void append_kernel_wide(HeadDesc *const *descs, int n_ctx,
                                                          int side, const float *__restrict__ src,
                                                          int n_tok, int dim, int P,
                                                          float inv_sqrt_p, float sqrt_p) {
  __shared__ Q4Cell s_q4[B == 4 ? kQ4Cells : 1];
  if constexpr (B == 4) {
    static constexpr Q4Table kTab = q4_table();
    if (threadIdx.x < kQ4Cells) s_q4[threadIdx.x] = kTab.c[threadIdx.x];
    __syncthreads();
  }
  const long long g = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long long)n_ctx * n_tok) return;
  const int c = (int)(g / n_tok);
  const int t = (int)(g - (long long)c * n_tok);
  const HeadDesc *d = descs[c];
  const RingState st = d->st;
  const int cap = d->cap;
  const float *x = src + ((size_t)c * n_tok + t) * dim;
  const bool write_ring = cap > 0 && t >= n_tok - cap;
  const int slot = cap > 0 ? (int)(((long long)st.head + t) % cap) : 0;
  if (t < mirror_count(st, n_tok, cap, d->hyb)) {
    float *m = (side == 0 ? d->raw_k : d->raw_v) + (size_t)(st.raw_count + t) * dim;
    for (int i = 0; i < dim; ++i) m[i] = x[i];
  }
  if (!write_ring) return;
  uint8_t *codes = side == 0 ? d->k_codes : d->v_codes;
  float *scales = side == 0 ? d->k_scale : d->v_scale;
  const int pb = packed_bytes(P, B);
  uint8_t *row = codes + (size_t)slot * pb;
  if constexpr (B == 16) {
    float *r = reinterpret_cast<float *>(row);
    for (int i = 0; i < P; ++i) r[i] = i < dim ? x[i] : 0.0f;
    scales[slot] = 1.0f;
    return;
  } else {
    float buf[kMaxPadded];
    float s = 0.0f;
    for (int i = 0; i < P; ++i) {
      buf[i] = i < dim ? x[i] : 0.0f;
      s = __fadd_rn(s, __fmul_rn(buf[i], buf[i]));
    }
    const float norm = sqrtf(__fadd_rn(s, 1e-12f));
    const float inv = 1.0f / norm;
    for (int i = 0; i < P; ++i) buf[i] = __fmul_rn(buf[i], inv);
    for (int i = 0; i < P; i += 2) {
      const uint32_t f0 = ((d->signs[i >> 5] >> (i & 31)) & 1u) ^ 1u;
      const uint32_t f1 = ((d->signs[(i + 1) >> 5] >> ((i + 1) & 31)) & 1u) ^ 1u;
      const float a = __uint_as_float(__float_as_uint(buf[i]) ^ (f0 << 31));
      const float b = __uint_as_float(__float_as_uint(buf[i + 1]) ^ (f1 << 31));
      buf[i] = __fadd_rn(a, b);
      buf[i + 1] = __fsub_rn(a, b);
    }
    for (int len = 2; len < P; len <<= 1)
      for (int base = 0; base < P; base += 2 * len)
        for (int j = base; j < base + len; ++j) {
          const float lo = buf[j], hi = buf[j + len];
          buf[j] = __fadd_rn(lo, hi);
          buf[j + len] = __fsub_rn(lo, hi);
        }
    float s2 = 0.0f;
    for (int i = 0; i < P; ++i) {
      buf[i] = __fmul_rn(__fmul_rn(buf[i], inv_sqrt_p), sqrt_p);
      s2 = __fadd_rn(s2, __fmul_rn(buf[i], buf[i]));
    }
    const float sigma = sqrtf(__fadd_rn(s2 / (float)P, 1e-12f));
    const float clip = __fmul_rn(3.0f, sigma);
    for (int i = 0; i < pb; ++i) row[i] = 0;
    for (int i = 0; i < P; ++i) {
      float v = buf[i];
      if (v > clip) v = clip;
      if (v < -clip) v = -clip;
      const uint32_t q = B == 4 ? (v != v ? 7u : quantize_g4(v, s_q4)) : quantize<B>(v);
      if constexpr (B == 4) {
        row[i / 2] |= (uint8_t)(q << ((i % 2) ? 0 : 4));
      } else if constexpr (B == 2) {
        row[i / 4] |= (uint8_t)(q << (6 - 2 * (i % 4)));
      } else {
        const int g8 = i / 8, k = i % 8, bit = 21 - 3 * k;
        const uint32_t w = q << bit;  // inside the 24-bit big-endian group
        row[3 * g8] |= (uint8_t)(w >> 16);
        row[3 * g8 + 1] |= (uint8_t)(w >> 8);
        row[3 * g8 + 2] |= (uint8_t)w;
      }
    }
    scales[slot] = norm;
  }
}

__global__ void commit_kernel(HeadDesc *const *descs, int n_ctx, int n_tok) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n_ctx) return;
  HeadDesc *d = descs[c];
  d->st = ring_after(d->st, n_tok, d->cap, d->hyb);
}

__global__ void reset_kernel(HeadDesc *const *descs, int n_ctx) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n_ctx) return;
  RingState z = {0, 0, 0, 0};
  descs[c]->st = z;
}

hipError_t launch_wide(HeadDesc *const *descs, int n_ctx, int side, int bits, const float *src,
                       int n_tok, int dim, int P, hipStream_t s) {
  const float sp = sqrtf((float)P);
  const float isp = 1.0f / sp;
  const long long total = (long long)n_ctx * n_tok;
  const dim3 grid((unsigned)((total + 127) / 128));
  switch (bits) {
    case 2: append_kernel_wide<2><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, P, isp, sp); break;
    case 3: append_kernel_wide<3><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, P, isp, sp); break;
    case 4: append_kernel_wide<4><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, P, isp, sp); break;
    case 16: append_kernel_wide<16><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, P, isp, sp); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int P, bool U>
hipError_t launch_side_as(HeadDesc *const *descs, int n_ctx, int side, int bits, const float *src,
                          int n_tok, int dim, int commit, hipStream_t s) {
  const float sp = sqrtf((float)P);
  const float isp = 1.0f / sp;
  // the 2-bit thresholds of the values before the scalings, found once
  static const BdThr bd = bd_thresholds(isp, sp);
  dim3 grid;
  if (U) {
    grid = dim3((unsigned)((n_tok + 127) / 128), (unsigned)n_ctx);
  } else {
    const long long total = (long long)n_ctx * n_tok;
    grid = dim3((unsigned)((total + 127) / 128));
  }
  switch (bits) {
    case 2: append_kernel<P, 2, U><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, isp, sp, commit, bd); break;
    case 3: append_kernel<P, 3, U><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, isp, sp, commit, bd); break;
    case 4: append_kernel<P, 4, U><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, isp, sp, commit, bd); break;
    case 16: append_kernel<P, 16, U><<<grid, 128, 0, s>>>(descs, n_ctx, side, src, n_tok, dim, isp, sp, commit, bd); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Head-per-block launches once a head has at least a wave of tokens.
bool head_per_block(int n_ctx, int n_tok) { return n_tok >= 64 && n_ctx <= 65535; }

// The V-side launch can advance the ring states itself (see append_kernel)
// when each head's tokens fall in one block.
bool commit_in_kernel(int n_ctx, int n_tok) {
  return n_tok == 1 || (head_per_block(n_ctx, n_tok) && n_tok <= 128);
}

template <int P>
hipError_t launch_side(HeadDesc *const *descs, int n_ctx, int side, int bits, const float *src,
                       int n_tok, int dim, int commit, hipStream_t s) {
  if (head_per_block(n_ctx, n_tok))
    return launch_side_as<P, true>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s);
  return launch_side_as<P, false>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s);
}

}  // namespace

// Blocks per side up to which a head-per-block append runs both sides in one
// launch (append_pair_kernel): a few rounds of blocks per CU, whose last round
// leaves CUs idle in a launch of one side (measured: config 4's 40,000-token
// append, 2,504 blocks a side, 96 -> 78 us).  Above, one launch per side (a
// config-5 chunk, 65,536 blocks a side: 30.0 ms for 16 chunks against 31.3
// paired, whose 4-bit/2-bit codec pair keeps 20 bytes in scratch).
constexpr long long kPairMaxBlocks = 8192;

// Token-heads up to which an append takes a wave per vector (above, a lane
// per vector keeps the launch to a few waves' worth of work per CU).  Without
// mirror rows to copy, a lane per vector with both sides in one launch is
// faster from a few thousand up (measured: config 1's 2,048 tokens x 4 heads
// 14.5 -> 11.5 us, config 2's 24 appends of 512 tokens x 14 heads 272 -> 228
// us); with them it is slower (config 1 hybrid 15-17 -> 23-27 us, config 2
// hybrid 305-309 -> 556-558 us).
constexpr int kOneWaveMaxVectors = 16384;
constexpr int kOneWaveMaxPacked = 4096;

hipError_t launch_append(HeadDesc *const *descs, int n_ctx, int dim, int padded, int k_bits,
                         int v_bits, const float *keys, const float *vals, int n_tok,
                         hipStream_t s, bool mirror) {
  if (n_ctx <= 0 || n_tok <= 0) return hipSuccess;
  // a lane per vector copies a mirror row by itself, a wave per vector with
  // its 64 lanes: appends that copy rows stay a wave per vector up to
  // kOneWaveMaxVectors, the others only up to kOneWaveMaxPacked
  const long long one_wave_max = mirror ? kOneWaveMaxVectors : kOneWaveMaxPacked;
  if ((padded == 64 || padded == 128) && n_tok <= 65535 &&
      (long long)n_ctx * n_tok <= one_wave_max) {
    // few vectors: a wave per vector, a block per token and head (both sides;
    // the ring states in the kernel for one token, by commit_kernel for more)
    const float sp = sqrtf((float)padded), isp = 1.0f / sp;
    const dim3 grid((unsigned)n_ctx, (unsigned)n_tok);
#define AQ_ONE(P_, KB_, VB_)                                                                   \
  if (padded == P_ && k_bits == KB_ && v_bits == VB_) {                                       \
    append_one_kernel<P_, KB_, VB_><<<grid, 128, 0, s>>>(descs, keys, vals, dim, n_tok, isp, sp); \
    if (n_tok == 1) return hipGetLastError();                                                 \
    if (const hipError_t e1 = hipGetLastError(); e1 != hipSuccess) return e1;                \
    commit_kernel<<<(n_ctx + 255) / 256, 256, 0, s>>>(descs, n_ctx, n_tok);                   \
    return hipGetLastError();                                                                 \
  }
#define AQ_ONE_V(P_, KB_) AQ_ONE(P_, KB_, 2) AQ_ONE(P_, KB_, 3) AQ_ONE(P_, KB_, 4) AQ_ONE(P_, KB_, 16)
    AQ_ONE_V(64, 2) AQ_ONE_V(64, 3) AQ_ONE_V(64, 4) AQ_ONE_V(64, 16)
    AQ_ONE_V(128, 2) AQ_ONE_V(128, 3) AQ_ONE_V(128, 4) AQ_ONE_V(128, 16)
#undef AQ_ONE_V
#undef AQ_ONE
    return hipErrorInvalidValue;
  }
  if (n_tok == 1 && (padded == 64 || padded == 128)) {
    // one launch for both sides and the ring states
    const float sp = sqrtf((float)padded), isp = 1.0f / sp;
    const dim3 grid((unsigned)((n_ctx + 127) / 128));
#define AQ_KV(P_, KB_, VB_)                                                                       \
  if (padded == P_ && k_bits == KB_ && v_bits == VB_) {                                          \
    append_kv_kernel<P_, KB_, VB_><<<grid, 128, 0, s>>>(descs, n_ctx, keys, vals, dim, isp, sp); \
    return hipGetLastError();                                                                    \
  }
#define AQ_KV_V(P_, KB_) AQ_KV(P_, KB_, 2) AQ_KV(P_, KB_, 3) AQ_KV(P_, KB_, 4) AQ_KV(P_, KB_, 16)
    AQ_KV_V(64, 2) AQ_KV_V(64, 3) AQ_KV_V(64, 4) AQ_KV_V(64, 16)
    AQ_KV_V(128, 2) AQ_KV_V(128, 3) AQ_KV_V(128, 4) AQ_KV_V(128, 16)
#undef AQ_KV_V
#undef AQ_KV
    return hipErrorInvalidValue;
  }
  if ((padded == 64 || padded == 128) && head_per_block(n_ctx, n_tok) &&
      !commit_in_kernel(n_ctx, n_tok) && k_bits >= 2 && k_bits <= 4 && v_bits >= 2 &&
      v_bits <= 4 && (long long)n_ctx * ((n_tok + 127) / 128) <= kPairMaxBlocks) {
    // both sides in one launch, then the ring states
    const float sp = sqrtf((float)padded), isp = 1.0f / sp;
    const dim3 grid((unsigned)((n_tok + 127) / 128), (unsigned)n_ctx, 2u);
    static const BdThr bd64 = bd_thresholds(1.0f / sqrtf(64.0f), sqrtf(64.0f));
    static const BdThr bd128 = bd_thresholds(1.0f / sqrtf(128.0f), sqrtf(128.0f));
    const BdThr bd = padded == 64 ? bd64 : bd128;
    bool launched = false;
#define AQ_PAIR(P_, KB_, VB_)                                                                    \
  if (!launched && padded == P_ && k_bits == KB_ && v_bits == VB_) {                             \
    append_pair_kernel<P_, KB_, VB_><<<grid, 128, 0, s>>>(descs, keys, vals, n_tok, dim, isp, sp, \
                                                          bd);                                    \
    launched = true;                                                                              \
  }
#define AQ_PAIR_V(P_, KB_) AQ_PAIR(P_, KB_, 2) AQ_PAIR(P_, KB_, 3) AQ_PAIR(P_, KB_, 4)
    AQ_PAIR_V(64, 2) AQ_PAIR_V(64, 3) AQ_PAIR_V(64, 4)
    AQ_PAIR_V(128, 2) AQ_PAIR_V(128, 3) AQ_PAIR_V(128, 4)
#undef AQ_PAIR_V
#undef AQ_PAIR
    if (!launched) return hipErrorInvalidValue;
    if (const hipError_t e1 = hipGetLastError(); e1 != hipSuccess) return e1;
    commit_kernel<<<(n_ctx + 255) / 256, 256, 0, s>>>(descs, n_ctx, n_tok);
    return hipGetLastError();
  }
  hipError_t e = hipSuccess;
  const bool fold = padded <= 128 && commit_in_kernel(n_ctx, n_tok);
  for (int side = 0; side < 2 && e == hipSuccess; ++side) {
    const int bits = side == 0 ? k_bits : v_bits;
    const float *src = side == 0 ? keys : vals;
    const int commit = fold && side == 1 ? 1 : 0;  // after the K side has read the state
    switch (padded) {
      case 1: e = launch_side<1>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 2: e = launch_side<2>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 4: e = launch_side<4>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 8: e = launch_side<8>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 16: e = launch_side<16>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 32: e = launch_side<32>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 64: e = launch_side<64>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 128: e = launch_side<128>(descs, n_ctx, side, bits, src, n_tok, dim, commit, s); break;
      case 256:
      case 512:
      case 1024: e = launch_wide(descs, n_ctx, side, bits, src, n_tok, dim, padded, s); break;
      default: return hipErrorInvalidValue;
    }
  }
  if (e != hipSuccess || fold) return e;
  commit_kernel<<<(n_ctx + 255) / 256, 256, 0, s>>>(descs, n_ctx, n_tok);
  return hipGetLastError();
}

hipError_t launch_reset_state(HeadDesc *const *descs, int n_ctx, hipStream_t s) {
  if (n_ctx <= 0) return hipSuccess;
  reset_kernel<<<(n_ctx + 255) / 256, 256, 0, s>>>(descs, n_ctx);
  return hipGetLastError();
}

}  // namespace aq
