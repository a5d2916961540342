// sparse.hip -- sparse-V decode (v_mass > 0, quantised K and V) for gfx950.
//
// Restates attention.cpp:373-474 with v_mass > 0 (line 469 read as the
// V-codebook call it evidently means):
//   logits_t  = (dot(qr, CB_K[codes_t]) * attn_s) * kscale_t, t oldest->newest
//   p_t       = expf(logit_t - max) / sum (sum accumulated left to right)
//   order     = tokens by p descending
//   selection = whole quads of that order while the running mass
//               mass += ((p0 + p1) + p2) + p3 is below v_mass, then single
//               tokens while it is still below
//   acc       = sum over the selection, in that order, of
//               fma(CB_V[code], (p_t * vscale_t) / sqrt(p), acc)
//   out       = inverse FWHT of acc (fwht.cpp:106-134)
// The selected set decides the output to within the weight of the tokens at
// the cut, so this path reproduces the reference's arithmetic order where it
// matters: the query rotation (attention.cpp:537-550), the 8-lane FMA dot
// with its pairwise lane sum (attention.cpp:83-136), and the left-to-right
// softmax sum.  Exactly equal probabilities are ordered by age here; the
// reference's std::sort leaves their order unspecified.
//
// Kernels: one grid over (token blocks, items) computes the logits and the
// blocks' maxima.  Up to 8,192 tokens, one block per item then does softmax,
// the sort (a stable radix sort in LDS) and the cut, and turns the selection
// into per-token weights.  Above, a grid computes the exponentials, one block
// per item their left-to-right sum and the sort keys, a per-item radix sort
// over many blocks orders them, and one block per item takes the cut.  A grid over
// (token chunks, items) sums the weighted V rows (deriving the weights from
// the cut above 8,192 tokens); one block per item adds the chunks and
// applies the inverse FWHT.  Short rings (up to 3,072 tokens) run the last
// three steps in one block per item, at padded 64 the logits too
// (sparse_fused_kernel).
#include <type_traits>

#include "expf_ref.hpp"
#include "launch.hpp"
#include "seqsum.hpp"

namespace aq {

namespace {

constexpr int kThreads = 256;
constexpr int kSelThreads = 1024;
// Rings up to kSelectInBlock tokens are selected inside the select kernel
// (radix sort in LDS); longer ones sort over many blocks between two kernels
// (measured, 8 heads d128: 12,000 tokens 242 -> 198 us and 16,384 tokens
// 264 -> 237 us sorted outside the select kernel; at 8,192 tokens and below
// the in-block sort is as fast or faster).
constexpr int kSelectInBlock = 8192;
constexpr int kLdsSort = kSelectInBlock;  // keys the select kernel sorts in LDS
constexpr int kStage = 4096;    // floats per LDS staging chunk

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

// Code i of a K row stored in the slot's XOR byte order (x = slot & mask,
// kperm_mask in device.hpp; x = 0 for unpermuted rows).
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

template <int B>
__device__ __forceinline__ float cbv(int i) {
  return cb<B>(i);
}

__device__ __forceinline__ bool sign_plus(const uint32_t *signs, int i) {
  return (signs[i >> 5] >> (i & 31)) & 1u;
}

// Query rotation with the reference's exact float steps: sequential ||q||^2,
// normalise, sign+butterflies, * RN(1/RN(sqrt p)), * (sqrt p * ||q||).
// The query entries lane l of wave 0 holds in rotate_query_exact's one-wave
// path (P = 64 or 128): l and l + 64.  Loaded apart from the rotation so a
// caller can issue them before other loads.
__device__ __forceinline__ float2 query_lanes(const float *q, int dim, int P) {
  const int lane = threadIdx.x;
  float2 v = make_float2(0.0f, 0.0f);
  if (lane < 64) {
    if (lane < dim) v.x = q[lane];
    if (P == 128 && lane + 64 < dim) v.y = q[lane + 64];
  }
  return v;
}

__device__ __forceinline__ void rotate_query_exact(float *s_q, const float *q, int dim, int P,
                                   const uint32_t *signs, float inv_sqrt_p, float sqrt_p,
                                   const float2 *preloaded = nullptr) {
  if (P == 64 || P == 128) {
    // one wave, lane l holding entries l and l + 64, the same operations in
    // the same order: the squares' sum left to right (every lane runs the
    // chain over the squares in LDS), the butterflies of span < 64 between
    // lanes, span 64 inside the lane; no block barriers until the result
    const float2 qv = preloaded ? *preloaded : query_lanes(q, dim, P);
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      const bool two = P == 128;
      float v0 = qv.x;
      float v1 = qv.y;
      s_q[lane] = __fmul_rn(v0, v0);
      if (two) s_q[lane + 64] = __fmul_rn(v1, v1);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float sq = 0.0f;
      {
        const float4 *q4 = reinterpret_cast<const float4 *>(s_q);
        const int nb = dim / 16;
        for (int b = 0; b < nb; ++b) {
          float4 r[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) r[k] = q4[4 * b + k];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            sq = __fadd_rn(sq, r[k].x);
            sq = __fadd_rn(sq, r[k].y);
            sq = __fadd_rn(sq, r[k].z);
            sq = __fadd_rn(sq, r[k].w);
          }
        }
        for (int i = 16 * nb; i < dim; ++i) sq = __fadd_rn(sq, s_q[i]);
      }
      const float qn = sqrtf(__fadd_rn(sq, 1e-12f));
      const float inv = 1.0f / qn;
      v0 = __fmul_rn(v0, inv);
      v1 = __fmul_rn(v1, inv);
      if (!sign_plus(signs, lane)) v0 = -v0;
      if (two && !sign_plus(signs, lane + 64)) v1 = -v1;
#pragma unroll
      for (int len = 1; len < 64; len <<= 1) {
        const bool upper = (lane & len) != 0;
        const float o0 = __shfl_xor(v0, len, 64), o1 = __shfl_xor(v1, len, 64);
        v0 = upper ? __fsub_rn(o0, v0) : __fadd_rn(v0, o0);
        v1 = upper ? __fsub_rn(o1, v1) : __fadd_rn(v1, o1);
      }
      if (two) {
        const float lo = v0, hi = v1;
        v0 = __fadd_rn(lo, hi);
        v1 = __fsub_rn(lo, hi);
      }
      const float m = __fmul_rn(sqrt_p, qn);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();  // every lane has read the squares
      s_q[lane] = __fmul_rn(__fmul_rn(v0, inv_sqrt_p), m);
      if (two) s_q[lane + 64] = __fmul_rn(__fmul_rn(v1, inv_sqrt_p), m);
    }
    __syncthreads();
    return;
  }
  __shared__ float s_qn;
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_q[i] = i < dim ? q[i] : 0.0f;
  __syncthreads();
  if (threadIdx.x == 0) {
    // left to right; 16 entries' loads in flight ahead of their squares
    float s = 0.0f;
    const float4 *q4 = reinterpret_cast<const float4 *>(s_q);
    const int nb = dim / 16;
    for (int b = 0; b < nb; ++b) {
      float4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = q4[4 * b + k];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s = __fadd_rn(s, __fmul_rn(v[k].x, v[k].x));
        s = __fadd_rn(s, __fmul_rn(v[k].y, v[k].y));
        s = __fadd_rn(s, __fmul_rn(v[k].z, v[k].z));
        s = __fadd_rn(s, __fmul_rn(v[k].w, v[k].w));
      }
    }
    for (int i = 16 * nb; i < dim; ++i) s = __fadd_rn(s, __fmul_rn(s_q[i], s_q[i]));
    s_qn = sqrtf(__fadd_rn(s, 1e-12f));
  }
  __syncthreads();
  const float qn = s_qn;
  const float inv = 1.0f / qn;
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_q[i] = __fmul_rn(s_q[i], inv);
  __syncthreads();
  for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
    const int i = 2 * k;
    const float a = sign_plus(signs, i) ? s_q[i] : -s_q[i];
    const float b = sign_plus(signs, i + 1) ? s_q[i + 1] : -s_q[i + 1];
    s_q[i] = __fadd_rn(a, b);
    s_q[i + 1] = __fsub_rn(a, b);
  }
  __syncthreads();
  for (int len = 2; len < P; len <<= 1) {
    for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
      const int j = (k / len) * 2 * len + (k % len);
      const float lo = s_q[j], hi = s_q[j + len];
      s_q[j] = __fadd_rn(lo, hi);
      s_q[j + len] = __fsub_rn(lo, hi);
    }
    __syncthreads();
  }
  const float m = __fmul_rn(sqrt_p, qn);
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_q[i] = __fmul_rn(__fmul_rn(s_q[i], inv_sqrt_p), m);
  __syncthreads();
}

// The inverse FWHT of s_acc[0..P) (the block's LDS, complete) with the
// signs, to out[0..dim): butterflies of span 1 .. P/2 as lo + hi, lo - hi,
// then x * (1/sqrt(P)) and the sign D_i (fwht.cpp:106-134).  At padded 64
// and 128 one wave does it with shuffles (the same operations in the same
// order, lane l holding entries l and l + 64); the other waves return at
// once, so no block barrier may follow a call.
__device__ void inverse_fwht_out(float *s_acc, int P, int dim, const uint32_t *signs, float *out) {
  if (P == 64 || P == 128) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const bool two = P == 128;
    float v0 = s_acc[lane], v1 = two ? s_acc[lane + 64] : 0.0f;
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
    const float w0 = __fmul_rn(v0, scale), w1 = __fmul_rn(v1, scale);
    if (lane < dim) out[lane] = sign_plus(signs, lane) ? w0 : -w0;
    if (two && lane + 64 < dim) out[lane + 64] = sign_plus(signs, lane + 64) ? w1 : -w1;
    return;
  }
  for (int len = 1; len < P; len <<= 1) {
    for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
      const int jj = (k / len) * 2 * len + (k % len);
      const float lo = s_acc[jj], hi = s_acc[jj + len];
      s_acc[jj] = lo + hi;
      s_acc[jj + len] = lo - hi;
    }
    __syncthreads();
  }
  const float scale = 1.0f / sqrtf((float)P);
  for (int i = threadIdx.x; i < dim; i += blockDim.x) {
    const float v = __fmul_rn(s_acc[i], scale);
    out[i] = sign_plus(signs, i) ? v : -v;
  }
}

template <int PT, int KB>
struct KRow {
  static constexpr int words = PT * KB / 32;  // PT = 64 or 128
};

// The row's words in reference byte order (PT = 64/128): 3-bit rows are
// stored so; 2/4-bit rows are XOR-permuted by x = slot & mask.  Two steps,
// so the loads can be issued well before the words are used: kload_raw
// reads the words in word order (x >> 2 undone), kperm_raw then undoes the
// byte order inside each word (x & 3).
template <int PT, int KB>
__device__ __forceinline__ void kload_raw(const uint8_t *row, int x, uint32_t *w) {
  constexpr int W = KRow<PT, KB>::words;
  if constexpr (KB == 3) {
    // 24 or 48 bytes a row: 8-byte loads
    const uint2 *r = reinterpret_cast<const uint2 *>(row);
#pragma unroll
    for (int i = 0; i < W / 2; ++i) {
      const uint2 v = r[i];
      w[2 * i] = v.x;
      w[2 * i + 1] = v.y;
    }
  } else {
    // 16 to 64 bytes a row: 16-byte loads in stored order, then word i of
    // the reference order is stored word i ^ (x >> 2), by one conditional
    // swap per bit of x >> 2 (below XS)
    constexpr int XS = (kperm_mask(PT, KB) + 1) / 4;
    static_assert(W % 4 == 0 && XS <= W, "whole 16-byte groups");
    const uint4 *r = reinterpret_cast<const uint4 *>(row);
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const uint4 v = r[i];
      w[4 * i] = v.x;
      w[4 * i + 1] = v.y;
      w[4 * i + 2] = v.z;
      w[4 * i + 3] = v.w;
    }
    // (the swaps are byte permutes: written as selects, the compiler turns
    // the stages back into one run-time index and a compare chain per word)
    const uint32_t xw = (uint32_t)x >> 2;
    constexpr int NB = XS >= 8 ? 3 : XS >= 4 ? 2 : XS >= 2 ? 1 : 0;  // log2(XS)
    static_assert((1 << NB) == XS || XS == 0, "XS is a power of two");
#pragma unroll
    for (int sb = 0; sb < NB; ++sb) {
      const int b = 1 << sb;
      // all bytes from the first operand (the partner word) or the second
      const uint32_t sel = (xw & (uint32_t)b) ? 0x07060504u : 0x03020100u;
#pragma unroll
      for (int i = 0; i < W; ++i) {
        if (i & b) continue;
        const uint32_t lo = w[i], hi = w[i | b];
        w[i] = __builtin_amdgcn_perm(hi, lo, sel);
        w[i | b] = __builtin_amdgcn_perm(lo, hi, sel);
      }
    }
  }
}
template <int PT, int KB>
__device__ __forceinline__ void kperm_raw(int x, uint32_t *w) {
  if constexpr (KB != 3) {
    const uint32_t sel = 0x03020100u ^ (((uint32_t)x & 3u) * 0x01010101u);
#pragma unroll
    for (int i = 0; i < KRow<PT, KB>::words; ++i) w[i] = __builtin_amdgcn_perm(0u, w[i], sel);
  }
}
template <int PT, int KB>
__device__ __forceinline__ void kload_row(const uint8_t *row, int x, uint32_t *w) {
  kload_raw<PT, KB>(row, x, w);
  kperm_raw<PT, KB>(x, w);
}

// dot(s_q, CB[codes]) of a row given as words in reference order, with the
// reference's 8 FMA lanes summed pairwise (attention.cpp:83-136)
template <int PT, int KB>
__device__ __forceinline__ float kdot_words(const uint32_t *w, const float *s_q, const float *cbk) {
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if constexpr (KB == 3) {
    // 24-bit big-endian groups of 8 codes
#pragma unroll
    for (int g = 0; g < PT / 8; ++g) {
      const int b0 = 3 * g;
      const uint32_t w24 = (((w[b0 >> 2] >> (8 * (b0 & 3))) & 255u) << 16) |
                           (((w[(b0 + 1) >> 2] >> (8 * ((b0 + 1) & 3))) & 255u) << 8) |
                           ((w[(b0 + 2) >> 2] >> (8 * ((b0 + 2) & 3))) & 255u);
#pragma unroll
      for (int k = 0; k < 8; ++k)
        s[k] = fmaf(cbk[(w24 >> (21 - 3 * k)) & 7u], s_q[8 * g + k], s[k]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      int c;
      if constexpr (KB == 4) {
        const int byte = j >> 1;
        c = (int)((w[byte >> 2] >> (8 * (byte & 3) + ((j & 1) ? 0 : 4))) & 15u);
      } else {
        const int byte = j >> 2;
        c = (int)((w[byte >> 2] >> (8 * (byte & 3) + 6 - 2 * (j & 3))) & 3u);
      }
      s[j & 7] = fmaf(cbk[c], s_q[j], s[j & 7]);
    }
  }
  const float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];
  return (t0 + t1) + (t2 + t3);
}

// dot(s_q, CB[codes of row]) with the reference's 8 FMA lanes (lane L takes
// codes L, L+8, ...) summed pairwise (attention.cpp:83-136).  cbk is the K
// codebook in LDS (a run-time index into a constant array is a memory load
// per code).  PT = 0: any padded size, codes read byte by byte.  PT = 64/128:
// the row is read as words (kload_row).
template <int PT, int KB>
__device__ __forceinline__ float kdot_row(const uint8_t *row, int x, const float *s_q, int P,
                                          const float *cbk) {
  if constexpr (PT != 0 && KB >= 2 && KB <= 4) {
    uint32_t w[KRow<PT, KB>::words];
    kload_row<PT, KB>(row, x, w);
    return kdot_words<PT, KB>(w, s_q, cbk);
  } else {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if constexpr (KB >= 2 && KB <= 4) {
      // unpermuted rows (padded 256 and up) in 16-byte loads: CB bytes hold CC
      // codes, a multiple of 8, so code jj still goes to s[jj % 8] in order
      constexpr int CB = KB == 3 ? 48 : 16;
      constexpr int CC = CB * 8 / KB;
      if (x == 0 && P % CC == 0) {
        const uint4 *r4 = reinterpret_cast<const uint4 *>(row);
        for (int c = 0; c < P / CC; ++c) {
          uint32_t w[CB / 4];
#pragma unroll
          for (int u = 0; u < CB / 16; ++u) {
            const uint4 v = r4[c * (CB / 16) + u];
            w[4 * u] = v.x;
            w[4 * u + 1] = v.y;
            w[4 * u + 2] = v.z;
            w[4 * u + 3] = v.w;
          }
          auto byte = [&](int b) -> uint32_t { return (w[b >> 2] >> ((b & 3) * 8)) & 0xFFu; };
#pragma unroll
          for (int j = 0; j < CC; ++j) {
            uint32_t code;
            if constexpr (KB == 4) {
              const uint32_t bb = byte(j >> 1);
              code = (j & 1) ? (bb & 15u) : (bb >> 4);
            } else if constexpr (KB == 2) {
              code = (byte(j >> 2) >> (6 - 2 * (j & 3))) & 3u;
            } else {
              const int g = j >> 3;
              const uint32_t w24 = (byte(3 * g) << 16) | (byte(3 * g + 1) << 8) | byte(3 * g + 2);
              code = (w24 >> (21 - 3 * (j & 7))) & 7u;
            }
            s[j & 7] = fmaf(cbk[code], s_q[c * CC + j], s[j & 7]);
          }
        }
        const float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];
        return (t0 + t1) + (t2 + t3);
      }
    }
    for (int j = 0; j < P; j += 8)
#pragma unroll
      for (int L = 0; L < 8; ++L)
        if (j + L < P) s[L] = fmaf(cbk[kcode_at<KB>(row, j + L, x)], s_q[j + L], s[L]);
    const float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];
    return (t0 + t1) + (t2 + t3);
  }
}

// Logical token t of an n-token ring lives in slot s0 + t (mod cap), with
// s0 = (head - n) mod cap (attention.cpp:562-563).
__device__ __forceinline__ int ring_slot(int s0, int t, int cap) {
  const int s = s0 + t;
  return s >= cap ? s - cap : s;
}

// Logits blocks: kThreads threads of kLgPer tokens (token k kThreads + t of
// the block is thread t's k-th).  Per item the workspace holds the n logits
// (later the exponentials, then the weights), 1/sum at [n], and from [n + 4]
// four floats per logits block: the block's maximum logit, then (from the
// exp kernel) its smallest and largest exponential and a NaN flag.
constexpr int kLgPer = 1;
constexpr int kLgTokens = kThreads * kLgPer;
__host__ __device__ constexpr int lg_blocks(int n) { return (n + kLgTokens - 1) / kLgTokens; }

// The per-item workspace (floats, from lg): the n logits / exponentials /
// weights and four scalars at [n] (1/sum, then the cut's selection), padded
// to 16 bytes; then kStat floats per logits block (its maximum logit,
// smallest and largest exponential, NaN flag).  Rings above kSelectInBlock
// use all of it.
constexpr int kStat = 4;
__host__ __device__ constexpr size_t lg_words(int n) { return ((size_t)n + 4 + 3) & ~(size_t)3; }
__device__ __forceinline__ float *lg_stats(float *lg, int n) { return lg + lg_words(n); }

template <int PT, int KB>
__global__ __launch_bounds__(kThreads) void sparse_logits_kernel(HeadDesc *const *item_desc,
                                                                 const float *__restrict__ queries,
                                                                 int max_n, float inv_sqrt_p,
                                                                 float sqrt_p, float *ws,
                                                                 size_t ws_stride) {
  __shared__ float s_q[kMaxPadded];
  __shared__ float s_cbk[16];
  __shared__ float s_m[kThreads / 64];
  const int item = blockIdx.y;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, cap = d->cap, dim = d->dim, P = d->padded;
  const int i0 = blockIdx.x * kLgTokens;
  if (i0 >= n) return;
  const int tid = threadIdx.x;
  if (tid < (1 << KB)) s_cbk[tid] = cbv<KB>(tid);
  const int s0 = (int)(((long long)d->st.head - n + cap) % cap);
  const float attn_s = 1.0f / (sqrtf((float)dim) * (float)P);
  float *lg = ws + (size_t)item * ws_stride;
  rotate_query_exact(s_q, queries + (size_t)item * dim, dim, P, d->signs, inv_sqrt_p, sqrt_p);
  // one token at a time (unrolled, the dots would share the query's
  // registers and spill); the block's maximum with the reference's start
  // value and NaN-skipping compare (attention.cpp:566), which maxima of
  // blocks combine the same way
  float m = -1e30f;
#pragma unroll 1
  for (int k = 0; k < kLgPer; ++k) {
    const int i = i0 + k * kThreads + tid;
    if (i < n) {
      const int slot = ring_slot(s0, i, cap);
      const float dot = kdot_row<PT, KB>(d->k_codes + (size_t)slot * d->k_pb,
                                         slot & kperm_mask(P, KB), s_q, P, s_cbk);
      const float l = __fmul_rn(__fmul_rn(dot, attn_s), d->k_scale[slot]);
      lg[i] = l;
      if (l > m) m = l;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    const float y = __shfl_xor(m, off);
    if (y > m) m = y;
  }
  if ((tid & 63) == 0) s_m[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    for (int w2 = 1; w2 < kThreads / 64; ++w2)
      if (s_m[w2] > m) m = s_m[w2];
    lg_stats(lg, n)[kStat * blockIdx.x] = m;
  }
}

// Exponentials of rings the select kernel does not sort itself (n >
// kSelectInBlock): grid (logits blocks, items).  The item's maximum is the
// maximum of its blocks' maxima; e = expf(l - max) (the reference's libm
// expf, bit for bit) over the logits; each block records its smallest and
// largest e and whether any is NaN.
__global__ __launch_bounds__(kThreads) void sparse_exp_kernel(HeadDesc *const *item_desc, float *ws,
                                                              size_t ws_stride) {
  __shared__ float s_r[3][kThreads / 64];
  const int item = blockIdx.y;
  const int n = item_desc[item]->st.size;
  if (n <= kSelectInBlock) return;  // select_small takes the logits
  const int nb = lg_blocks(n);
  if ((int)blockIdx.x >= nb) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float *lg = ws + (size_t)item * ws_stride;
  float *st = lg_stats(lg, n);
  const int i0 = blockIdx.x * kLgTokens;
  float lv[kLgPer];
#pragma unroll
  for (int k = 0; k < kLgPer; ++k) {
    const int i = i0 + k * kThreads + tid;
    lv[k] = i < n ? lg[i] : 0.0f;
  }
  float mx = -1e30f;
  for (int b = tid; b < nb; b += kThreads)
    if (st[kStat * b] > mx) mx = st[kStat * b];
  for (int off = 32; off > 0; off >>= 1) {
    const float y = __shfl_xor(mx, off);
    if (y > mx) mx = y;
  }
  if (lane == 0) s_r[0][wave] = mx;
  __syncthreads();
  for (int w2 = 0; w2 < kThreads / 64; ++w2)
    if (s_r[0][w2] > mx) mx = s_r[0][w2];
  float e_lo = __builtin_inff(), e_hi = 0.0f;
  int nan_e = 0;
#pragma unroll
  for (int k = 0; k < kLgPer; ++k) {
    const int i = i0 + k * kThreads + tid;
    if (i < n) {
      const float e = expf_ref(lv[k] - mx);
      lg[i] = e;
      nan_e |= e != e;
      e_lo = fminf(e_lo, e);
      e_hi = fmaxf(e_hi, e);
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    e_lo = fminf(e_lo, __shfl_xor(e_lo, off));
    e_hi = fmaxf(e_hi, __shfl_xor(e_hi, off));
  }
  nan_e = __syncthreads_or(nan_e);  // also orders s_r[0]'s reads before the writes below
  if (lane == 0) {
    s_r[1][wave] = e_lo;
    s_r[2][wave] = e_hi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w2 = 0; w2 < kThreads / 64; ++w2) {
      e_lo = fminf(e_lo, s_r[1][w2]);
      e_hi = fmaxf(e_hi, s_r[2][w2]);
    }
    float *sb = st + kStat * blockIdx.x;
    sb[1] = e_lo;
    sb[2] = e_hi;
    sb[3] = nan_e ? 1.0f : 0.0f;
  }
}

// Sort key of token i with probability p: unsigned order of the key is the
// selection order -- larger p first, equal p older first, NaN after every
// number, padding (i >= n) after everything.  hi = 0x7F800000 - |p| bits for
// numbers (p >= 0 here), 0xFFFFFFFF for NaN; lo = i.
__device__ __forceinline__ uint32_t key_hi(float p) {
  const uint32_t b = __float_as_uint(p) & 0x7FFFFFFFu;
  return b > 0x7F800000u ? 0xFFFFFFFFu : 0x7F800000u - b;
}
__device__ __forceinline__ uint64_t make_key(float p, int i) {
  return ((uint64_t)key_hi(p) << 32) | (uint32_t)i;
}
constexpr uint64_t kPadKey = ~(uint64_t)0;

__device__ __forceinline__ float hi_p(uint32_t hi) {
  return __uint_as_float(hi == 0xFFFFFFFFu ? 0x7FC00000u : 0x7F800000u - hi);
}
__device__ __forceinline__ float key_p(uint64_t k) { return hi_p((uint32_t)(k >> 32)); }
__device__ __forceinline__ int key_i(uint64_t k) { return (int)(uint32_t)k; }


// The reference's mass loop over quad sums q[0..m): while mass < v_mass, add
// the next one.  Returns how many it takes; *mass is updated.  The sums are
// >= 0, so the running mass never decreases (and stays NaN once NaN): the
// number taken is the number of positions whose mass before them is still
// below v_mass, counted beside a plain chain of adds.  Past the stop the
// chain runs on to the end of its batch of 32, which leaves *mass at or above
// v_mass (or NaN) as the reference's is, so the single-token loop that
// follows runs exactly when the reference's does.
__device__ int mass_scan(const float *q, int m, float v_mass, float *mass) {
  const float4 *q4 = reinterpret_cast<const float4 *>(q);
  float ms = *mass;
  int taken = 0;
  for (int b = 0; b < m / 32 && ms < v_mass; ++b) {
    float4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = q4[8 * b + k];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        taken += ms < v_mass ? 1 : 0;
        ms = __fadd_rn(ms, e[c]);
      }
    }
  }
  for (int i = (m / 32) * 32; i < m && ms < v_mass; ++i) {
    ms = __fadd_rn(ms, q[i]);
    ++taken;
  }
  *mass = ms;
  return taken;
}

// Sum of the totals of the waves before `wave` (NW of them in LDS, 16-byte
// aligned): NW / 4 broadcast 16-byte reads rather than a chain of dependent
// ones.
template <int NW>
__device__ __forceinline__ uint32_t waves_before(const uint32_t *wsum, int wave) {
  static_assert(NW % 4 == 0, "whole 16-byte groups");
  const uint4 *w4 = reinterpret_cast<const uint4 *>(wsum);
  uint32_t b = 0u;
#pragma unroll
  for (int q = 0; q < NW / 4; ++q) {
    const uint4 v = w4[q];
    b += (4 * q < wave ? v.x : 0u) + (4 * q + 1 < wave ? v.y : 0u) +
         (4 * q + 2 < wave ? v.z : 0u) + (4 * q + 3 < wave ? v.w : 0u);
  }
  return b;
}

// Shared memory of the select kernel.  The small path (n <= kLdsSort) keeps
// 32-bit keys, 16-bit token indices and 16 x kSelThreads 16-bit radix counts
// (cnt also holds chain_sum_block's LDS); the large path keeps its sort keys
// in the workspace and stages its sums' terms over the keys.
struct SelectShared {
  union {
    uint32_t key[kLdsSort];  // also the exponentials, as floats
    float xs[seqsum_detail::kBlock * seqsum_detail::kMaxT];  // chain_sum_long's terms
  };
  uint16_t idx[kLdsSort];
  uint16_t cnt[16 * kSelThreads];  // cnt[digit * kSelThreads + thread]
  __align__(16) float stage[kStage];
  float red[kSelThreads];
  __align__(16) uint32_t wsum[kSelThreads / 64];
  float bcast[2];
  int cut;
  uint64_t last;
};
static_assert(kLdsSort == seqsum_detail::kBlock * seqsum_detail::kMaxT, "the sums' terms fit over the keys");

// Block maximum with the reference's NaN-skipping compare (x > m ? x : m;
// every partial maximum is a number, so the tree gives the sequential value).
__device__ __forceinline__ float block_max(float m, SelectShared &sh) {
  for (int off = 32; off > 0; off >>= 1) {
    const float y = __shfl_xor(m, off);
    if (y > m) m = y;
  }
  if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = m;
  __syncthreads();
  float r = sh.red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
    if (sh.red[w] > r) r = sh.red[w];
  __syncthreads();
  return r;
}

// Exclusive scan of cnt[] (16 x kSelThreads 16-bit counts, digit-major) in
// place: thread t scans entries 16t .. 16t+15, waves scan the thread totals,
// the wave totals are added in order.  Counts stay packed two to a word: every
// prefix is below 2^16 (at most 65,535 keys), so adding base * 0x10001 to a
// word carries nothing from the low half into the high one.
__device__ __forceinline__ void scan_counts(SelectShared &sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint4 *c4 = reinterpret_cast<uint4 *>(sh.cnt) + 2 * tid;
  const uint4 a = c4[0], b = c4[1];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t run = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = w[i] & 0xFFFFu, hi = w[i] >> 16;
    w[i] = run | ((run + lo) << 16);
    run += lo + hi;
  }
  uint32_t incl = run;
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sh.wsum[wave] = incl;
  __syncthreads();
  const uint32_t base = incl - run + waves_before<kSelThreads / 64>(sh.wsum, wave);
  const uint32_t b2 = base * 0x10001u;
  c4[0] = make_uint4(w[0] + b2, w[1] + b2, w[2] + b2, w[3] + b2);
  c4[1] = make_uint4(w[4] + b2, w[5] + b2, w[6] + b2, w[7] + b2);
  __syncthreads();
}

// Stable sort of up to 2 kSelThreads 32-bit keys by comparison: the pairs
// (key, position) are distinct, so sorting them gives the stable order.
// (An LSD radix sort in LDS with 8- or 9-bit digits, ranked by wave ballots,
// took 11.6-12.8 us of config 1 and 3's decodes; this one 9.1-9.4 us.)  Thread t holds positions E t .. E t + E - 1 (E = 1 or 2) as
// 64-bit values key << 32 | position; its slots without a token (positions
// from n on, and the second slot when E = 1) hold key 0xFFFFFFFF with a
// position of 2,048 or more, distinct and after every token.  Each wave sorts
// its 128 values in registers (a bitonic network, partners by DPP moves up to
// lane ^ 8 and lane shuffles beyond); four
// rounds of pairwise merges in LDS (sh.cnt as two 2,048-value buffers) then
// give one run: a value's place in the merged run is its place in its own
// run plus the count of smaller values in the other, found by binary search.
// Leaves the order in sh.key[0, n) and sh.idx[0, n); touches no other key.
template <int E>
__device__ __forceinline__ void sort_small_merge(SelectShared &sh, int n, const uint32_t (&k)[E]) {
  static_assert(E == 1 || E == 2, "one or two keys a thread");
  constexpr int NV = 2 * kSelThreads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint64_t a[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int pos = tid * E + e;
    a[e] = (e < E && pos < n) ? ((uint64_t)k[e < E ? e : 0] << 32) | (uint32_t)pos
                              : (0xFFFFFFFFull << 32) | (uint32_t)(NV + 2 * tid + e);
  }
  // the value of lane ^ m: DPP within a row of 16 lanes (quad permutes for
  // 1 and 2, row shifts by 4 either way, a row rotation by 8), lane shuffles
  // for 16 and 32
  auto xch = [&](uint32_t x, int m) -> uint32_t {
    if (m == 1) return __builtin_amdgcn_update_dpp(0u, x, 0xB1, 0xF, 0xF, false);
    if (m == 2) return __builtin_amdgcn_update_dpp(0u, x, 0x4E, 0xF, 0xF, false);
    if (m == 4) {
      const uint32_t up = __builtin_amdgcn_update_dpp(0u, x, 0x104, 0xF, 0xF, false);  // lane + 4
      const uint32_t dn = __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xF, 0xF, false);  // lane - 4
      return (lane & 4) ? dn : up;
    }
    if (m == 8) return __builtin_amdgcn_update_dpp(0u, x, 0x128, 0xF, 0xF, false);
    return (uint32_t)__shfl_xor((int)x, m, 64);
  };
  auto shfl64 = [&](uint64_t x, int m) -> uint64_t {
    return ((uint64_t)xch((uint32_t)(x >> 32), m) << 32) | xch((uint32_t)x, m);
  };
  // bitonic sort of the wave's 128 values: value i = 2 lane + e
#pragma unroll
  for (int kk = 2; kk <= 128; kk <<= 1) {
    const bool asc = ((2 * lane) & kk) == 0;
#pragma unroll
    for (int j = kk >> 1; j > 1; j >>= 1) {
      const int m = j >> 1;
      const bool lower = (lane & m) == 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint64_t b = shfl64(a[e], m);
        const uint64_t lo = a[e] < b ? a[e] : b, hi = a[e] < b ? b : a[e];
        a[e] = lower == asc ? lo : hi;
      }
    }
    const uint64_t lo = a[0] < a[1] ? a[0] : a[1], hi = a[0] < a[1] ? a[1] : a[0];
    a[0] = asc ? lo : hi;
    a[1] = asc ? hi : lo;
  }
  uint64_t *X = reinterpret_cast<uint64_t *>(sh.cnt), *Y = X + NV;
  X[128 * wave + 2 * lane] = a[0];
  X[128 * wave + 2 * lane + 1] = a[1];
  __syncthreads();
#pragma unroll
  for (int L = 128; L < NV; L <<= 1) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int p = 2 * tid + e;
      const uint64_t x = X[p];
      const int r = p / L;
      const uint64_t *other = X + (size_t)(r ^ 1) * L;
      int c = 0;  // values of the other run below x
#pragma unroll
      for (int step = L; step >= 1; step >>= 1) {
        const int q = c + step;
        if (q <= L && other[q - 1] < x) c = q;
      }
      Y[(r & ~1) * L + (p - r * L) + c] = x;
    }
    __syncthreads();
    uint64_t *t = X;
    X = Y;
    Y = t;
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int p = 2 * tid + e;
    if (p < n) {
      const uint64_t x = X[p];
      sh.key[p] = (uint32_t)(x >> 32);
      sh.idx[p] = (uint16_t)(x & 0xFFFFu);
    }
  }
  __syncthreads();
}

// Selection for n <= kLdsSort tokens.  Thread t owns tokens E t .. E t + E - 1
// in registers.  Steps:
//   1. max of the logits (the reference's start value -1e30 and compare)
//   2. e = expf(l - max) into LDS (expf_ref: the reference's libm expf, bit
//      for bit); thread 0 adds them left to right
//      (attention.cpp:422-426); p = e * (1/sum)
//   3. stable sort of the 32-bit keys less the smallest one: order p
//      descending, ties older first.  Up to 2 kSelThreads tokens:
//      sort_small_merge (bitonic within waves, merges in LDS); above: an LSD
//      radix sort, 4 bits a pass, in registers, skipping digits every key
//      shares
//   4. quad sums ((p0+p1)+p2)+p3 of the sorted order in parallel; thread 0
//      runs the mass loop over them, then the single tokens
//      (attention.cpp:454-472)
//   5. per-token weights (p * vscale) * isp for the selected tokens, else 0,
//      written over the logits in token order
//   The logits come from lg, or, with lin != null, from the caller's
//   registers (the same tokens); the weights go to lg and, if given, to wout.
template <int E>
__device__ __forceinline__ void select_small(const HeadDesc *d, float v_mass, float *lg, int n, int s0,
                             SelectShared &sh, const float *lin = nullptr,
                             float *wout = nullptr) {
  static_assert(E == 1 || E == 2 || E == 4 || E == 8, "tokens per thread");
  const int tid = threadIdx.x, p0 = tid * E;
  const int cap = d->cap, P = d->padded;
  float ev[E];
#pragma unroll
  for (int e = 0; e < E; ++e) ev[e] = p0 + e < n ? (lin ? lin[e] : lg[p0 + e]) : 0.0f;
  if (!wout) wout = lg;
  float mx = -1e30f;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (p0 + e < n && ev[e] > mx) mx = ev[e];
  mx = block_max(mx, sh);

  // the exponentials' left-to-right sum (attention.cpp:422-426), bit for
  // bit, by chain_sum_block: each thread classifies its own E terms, one
  // wave walks (4 heads x 2,048 tokens: 3.9 us; one lane's chain took 8.9).
  // The exponentials also go to LDS (the walk's hardware terms read them
  // there).  Up to 4 tokens a thread they stay
  // there for the weights (step 5), above the keys the sort writes:
  // sort_small_merge's sh.key[0, n) with n <= 2048 (its buffers are sh.cnt),
  // the 4-bit sort's sh.key[0, 4096).  At 8 a thread the weights recompute
  // them from the logits in lg.
  static_assert(sizeof(ChainShared) <= sizeof(sh.cnt), "chain_sum_block's LDS in sh.cnt");
  ChainShared &cs = *reinterpret_cast<ChainShared *>(sh.cnt);
  float *ef = reinterpret_cast<float *>(sh.key) + (E <= 2 ? 2048 : E == 4 ? 4096 : 0);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    ev[e] = p0 + e < n ? expf_ref(ev[e] - mx) : 0.0f;
    if (p0 + e < n) ef[p0 + e] = ev[e];
  }
  __syncthreads();
  const float inv = 1.0f / chain_sum_block<E, false>(ev, n, 0.0f, __builtin_inff(), ef, cs).s;

  // Keys are sorted less the smallest one, key_hi(inv): every e is at most
  // 1 (or NaN), so every p = e inv is at most inv (or NaN, whose key is the
  // largest), and the subtraction keeps the order.  The digits then cover
  // only the key range.
  const uint32_t kmin = key_hi(inv);
  uint32_t k[E], ix[E];
  uint32_t kor = 0, kand = 0xFFFFFFFFu;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const bool valid = p0 + e < n;
    k[e] = valid ? key_hi(__fmul_rn(ev[e], inv)) - kmin : 0u;
    ix[e] = (uint32_t)(p0 + e);
    if (valid) {
      kor |= k[e];
      kand &= k[e];
    }
  }
  uint32_t diff = 0;
  if constexpr (E > 2) {
    // digits every key shares do not move anything: skip their passes
    for (int off = 32; off > 0; off >>= 1) {
      kor |= __shfl_xor(kor, off);
      kand &= __shfl_xor(kand, off);
    }
    if ((tid & 63) == 0) {
      sh.wsum[tid >> 6] = kor;
      reinterpret_cast<uint32_t *>(sh.red)[tid >> 6] = kand;
    }
    __syncthreads();
    uint32_t o = 0, a = 0xFFFFFFFFu;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
      o |= sh.wsum[w];
      a &= reinterpret_cast<uint32_t *>(sh.red)[w];
    }
    diff = o ^ a;
    kor = o;
    __syncthreads();
  }

  if constexpr (E <= 2) {
    sort_small_merge<E>(sh, n, k);
  } else {
  // positions from n on sort after every token: the OR of the keys is at
  // least each of them, shares their common digits, and stable order puts
  // the later positions last among equal keys
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (p0 + e >= n) k[e] = kor;
  for (int sft = 0; sft < 32; sft += 4) {
    if (((diff >> sft) & 15u) == 0) continue;
    // counts of each digit among this thread's tokens (8-bit fields) and the
    // rank of each token among its thread's tokens of the same digit
    // (the rank goes into bits 16.. of ix, below the token index's 16 bits)
    uint64_t c_lo = 0, c_hi = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t dg = (k[e] >> sft) & 15u;
      const uint32_t f = (dg & 7u) * 8u;
      const uint64_t cw = dg < 8u ? c_lo : c_hi;
      ix[e] = (ix[e] & 0xFFFFu) | ((uint32_t)(cw >> f) & 255u) << 16;
      if (dg < 8u) c_lo += (uint64_t)1 << f;
      else c_hi += (uint64_t)1 << f;
    }
#pragma unroll
    for (int dd = 0; dd < 16; ++dd)
      sh.cnt[dd * kSelThreads + tid] =
          (uint16_t)(((dd < 8 ? c_lo : c_hi) >> ((dd & 7) * 8)) & 255u);
    __syncthreads();
    scan_counts(sh);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const uint32_t dg = (k[e] >> sft) & 15u;
      const uint32_t dst = (uint32_t)sh.cnt[dg * kSelThreads + tid] + (ix[e] >> 16);
      sh.key[dst] = k[e];
      sh.idx[dst] = (uint16_t)ix[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e) {
      k[e] = sh.key[p0 + e];
      ix[e] = sh.idx[p0 + e];
    }
    __syncthreads();
  }
  // sorted order into LDS (the passes may all have been skipped)
#pragma unroll
  for (int e = 0; e < E; ++e) {
    sh.key[p0 + e] = k[e];
    sh.idx[p0 + e] = (uint16_t)ix[e];
  }
  __syncthreads();
  }

  // the mass loop (attention.cpp:454-472): quad sums ((p0+p1)+p2)+p3 of the
  // sorted order, EQ consecutive ones a thread, added while the mass is below
  // v_mass by chain_sum_block; then, if every quad went in, the single tokens
  // on one lane
  constexpr int EQ = E >= 4 ? E / 4 : 1;
  const int n_quads = n / 4;
  float qv[EQ];
#pragma unroll
  for (int e = 0; e < EQ; ++e) {
    const int q = tid * EQ + e;
    qv[e] = 0.0f;
    if (q < n_quads) {
      qv[e] = __fadd_rn(__fadd_rn(__fadd_rn(hi_p(sh.key[4 * q] + kmin), hi_p(sh.key[4 * q + 1] + kmin)),
                                  hi_p(sh.key[4 * q + 2] + kmin)),
                        hi_p(sh.key[4 * q + 3] + kmin));
      sh.stage[q] = qv[e];
    }
  }
  __syncthreads();
  const SeqResult mq = chain_sum_block<EQ, true>(qv, n_quads, 0.0f, v_mass, sh.stage, cs);
  if (tid == 0) {
    float mass = mq.s;
    int ii = 4 * mq.count;
    for (; ii < n && mass < v_mass; ++ii) mass = __fadd_rn(mass, hi_p(sh.key[ii] + kmin));
    sh.cut = ii;
  }
  __syncthreads();
  if (tid == 0) {
    const int ii = sh.cut;
    sh.last = ii > 0 ? ((uint64_t)(sh.key[ii - 1] + kmin) << 32) | sh.idx[ii - 1] : 0;
  }
  __syncthreads();
  // The selection is the first cut keys of the sorted order, i.e. every key
  // up to the last one taken (keys are distinct).  Each thread forms its own
  // tokens' p again (e from LDS, or at 8 tokens a thread from the logits
  // still in lg: the same bits as before) and writes their weights in token
  // order.
  const int cut = sh.cut;
  const uint64_t last = sh.last;
  const float isp = 1.0f / sqrtf((float)P);
  float vs[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int t = p0 + e;
    vs[e] = t < n ? d->v_scale[ring_slot(s0, t, cap)] : 0.0f;
  }
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int t = p0 + e;
    if (t < n) {
      // with 8 tokens a thread there are no logits in registers (lin is
      // null: only sparse_select_kernel runs this width)
      const float ee = E <= 4 ? ef[t] : expf_ref(lg[t] - mx);
      const float p = __fmul_rn(ee, inv);
      const float w = cut > 0 && make_key(p, t) <= last ? __fmul_rn(__fmul_rn(p, vs[e]), isp) : 0.0f;
      wout[t] = w;
      if (wout != lg) lg[t] = w;  // the workspace keeps every launch's weights
    }
  }
}

// Sort of rings above kSelectInBlock tokens: a stable LSD radix sort of each
// item's 32-bit keys key_hi(p) with the tokens as payload.  The keys are
// stored less the item's smallest key (which the select kernel finds with
// 1/sum), so the digits cover only the bits of the key range: kRsBits a
// pass, at most 3 passes (keys of probabilities in [0, 1] span less than
// 2^30; NaN keys are all equal).  Ties keep token order, which is the order
// make_key gives them.  Pass k runs over (blocks of kRsKeys positions) x
// items.  The count kernel (at pass 0 it first writes the keys and tokens in
// token order): a block counts the pass's digits among its positions and
// stores them at count[block][digit].  Above kRsSuper blocks the super kernel
// adds them per superblock of kRsSuper blocks.  The scatter kernel: a block
// takes its offsets from the item's counts (digits below, then the same digit
// in blocks before it: whole superblocks' sums, then the blocks of its own
// superblock), ranks its keys stably in LDS (a ballot per digit bit and
// running per-wave digit counts) and writes each key to offset[digit] + its
// rank among the block's keys of that digit.  Nothing crosses blocks inside a
// launch (device-wide atomics on the counts, and a last-block scan behind
// device-scope fences, each measured 3-5x slower than the separate launches).
constexpr int kRsThreads = 512;
constexpr int kRsRounds = 4;
constexpr int kRsWaves = kRsThreads / 64;
constexpr int kRsKeys = kRsThreads * kRsRounds;  // positions per block and pass
constexpr int kRsBits = 10;
constexpr int kRsPasses = 3;
constexpr int kRsDigits = 1 << kRsBits;
constexpr int kRsDPT = kRsDigits / kRsThreads;  // digits per thread
constexpr int kRsSuper = 32;                    // blocks per superblock
static_assert(kRsDigits % kRsThreads == 0, "whole digits per thread");

__host__ __device__ constexpr int rs_blocks(int S) { return (S + kRsKeys - 1) / kRsKeys; }
// superblocks of a ring of S tokens (0 when the scatter sums every block)
__host__ __device__ constexpr int rs_supers(int S) {
  return rs_blocks(S) > kRsSuper ? (rs_blocks(S) + kRsSuper - 1) / kRsSuper : 0;
}

// Word offsets inside an item's sort region (uint32), for rings of at most S
// tokens: a header (0: passes, 5: the smallest key, 6: tokens; pass k takes
// bits kRsBits k and up), the counts ((block, digit), block-major), the
// superblock sums ((superblock, digit)), then keys A, keys B, tokens A,
// tokens B of Sa = align64(S) words.
struct ItemSort {
  static constexpr size_t cnt = 16;
  __host__ __device__ static constexpr size_t sup(int S) {
    return cnt + (size_t)kRsDigits * rs_blocks(S);
  }
  __host__ __device__ static constexpr size_t keys(int S) {
    return sup(S) + (size_t)kRsDigits * rs_supers(S);
  }
  __host__ __device__ static constexpr size_t sa(int S) { return ((size_t)S + 63) & ~(size_t)63; }
  __host__ __device__ static constexpr size_t words(int S) { return keys(S) + 4 * sa(S); }
};

// The item sort's state for one (item, pass): false when the item does not
// take this pass (sorted in the select kernel, or its key range is shorter).
struct RsPass {
  uint32_t *reg;
  int n, G, sft;
  const uint32_t *sk, *stk;  // input keys and tokens
  uint32_t *dk, *dtk;        // output keys and tokens
};

// np: the item's passes; kmin: its smallest key.
__device__ __forceinline__ bool rs_pass(int pass, uint32_t *sort_ws, size_t item_words, int S,
                                        RsPass &r, int &np, uint32_t &kmin) {
  // one read of the header (the select kernel's): no tokens for items it
  // sorted itself
  r.reg = sort_ws + (size_t)blockIdx.y * item_words;
  const uint4 h = *reinterpret_cast<const uint4 *>(r.reg);
  const uint4 h1 = *reinterpret_cast<const uint4 *>(r.reg + 4);
  np = (int)h.x;
  kmin = h1.y;
  r.n = (int)h1.z;
  r.G = (r.n + kRsKeys - 1) / kRsKeys;
  if ((int)blockIdx.x >= r.G) return false;
  r.sft = pass * kRsBits;
  const size_t Sa = ItemSort::sa(S);
  const int in = pass & 1, out = in ^ 1;
  const size_t k0 = ItemSort::keys(S);
  r.sk = r.reg + k0 + in * Sa;
  r.stk = r.reg + k0 + (2 + in) * Sa;
  r.dk = r.reg + k0 + out * Sa;
  r.dtk = r.reg + k0 + (2 + out) * Sa;
  return true;
}

// Count kernel of one pass of the item sort (see above): grid (blocks, items).
// Pass 0 also writes the sort's input: keys key_hi(e inv) less the smallest
// key and tokens, in token order, from the exponentials and inv at lg[n] of
// the item's workspace (ws) -- also for an item that takes no pass (every
// key equal), whose cut reads them as they are.
__global__ __launch_bounds__(kRsThreads) void sparse_rsort_count_kernel(int pass, uint32_t *sort_ws,
                                                                        size_t item_words, int S,
                                                                        const float *ws,
                                                                        size_t ws_stride) {
  __shared__ uint32_t s_hist[kRsDigits];
  RsPass r;
  int np;
  uint32_t kmin;
  if (!rs_pass(pass, sort_ws, item_words, S, r, np, kmin)) return;
  const int b = blockIdx.x, tid = threadIdx.x;
  uint32_t k[kRsRounds];
  if (pass == 0) {
    const float *lg = ws + (size_t)blockIdx.y * ws_stride;
    const float inv = lg[r.n];
    uint32_t *ka = r.reg + ItemSort::keys(S), *ta = ka + 2 * ItemSort::sa(S);
#pragma unroll
    for (int j = 0; j < kRsRounds; ++j) {
      const int pos = b * kRsKeys + j * kRsThreads + tid;
      k[j] = pos < r.n ? key_hi(__fmul_rn(lg[pos], inv)) - kmin : 0u;
      if (pos < r.n) {
        ka[pos] = k[j];
        ta[pos] = (uint32_t)pos;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kRsRounds; ++j) {
      const int pos = b * kRsKeys + j * kRsThreads + tid;
      k[j] = pos < r.n ? r.sk[pos] : 0u;
    }
  }
  if (pass >= np) return;
#pragma unroll
  for (int j = 0; j < kRsDPT; ++j) s_hist[j * kRsThreads + tid] = 0u;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kRsRounds; ++j)
    if (b * kRsKeys + j * kRsThreads + tid < r.n)
      atomicAdd(&s_hist[(k[j] >> r.sft) & (kRsDigits - 1u)], 1u);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kRsDPT; ++j)
    r.reg[ItemSort::cnt + (size_t)b * kRsDigits + j * kRsThreads + tid] = s_hist[j * kRsThreads + tid];
}

// Superblock sums of one pass of the item sort (see above): grid
// (superblocks, items), for items of more than kRsSuper blocks; thread t adds
// digits 2t, 2t + 1 over the superblock's blocks.
__global__ __launch_bounds__(kRsThreads) void sparse_rsort_super_kernel(int pass, uint32_t *sort_ws,
                                                                        size_t item_words, int S) {
  uint32_t *reg = sort_ws + (size_t)blockIdx.y * item_words;
  const int np = (int)reg[0], n = (int)reg[6];
  const int G = rs_blocks(n), B = blockIdx.x;
  if (pass >= np || G <= kRsSuper || B * kRsSuper >= G) return;
  static_assert(kRsDPT == 2, "two digits (one uint2) per thread");
  const uint2 *c = reinterpret_cast<const uint2 *>(reg + ItemSort::cnt) + threadIdx.x;
  const int b0 = B * kRsSuper, b1 = min(G, b0 + kRsSuper);
  uint32_t a0 = 0u, a1 = 0u;
#pragma unroll 8
  for (int b = b0; b < b1; ++b) {
    const uint2 v = c[(size_t)b * (kRsDigits / 2)];
    a0 += v.x;
    a1 += v.y;
  }
  reinterpret_cast<uint2 *>(reg + ItemSort::sup(S))[(size_t)B * (kRsDigits / 2) + threadIdx.x] =
      make_uint2(a0, a1);
}

// Scatter kernel of one pass of the item sort (see above): grid (blocks, items).
// Wave w of the block owns positions w 64 R .. w 64 R + 64 R - 1 of its
// range, 64 a round: a key's rank among the block's keys of its digit is the
// count of that digit in earlier waves (a prefix over the waves' totals),
// plus in this wave's earlier rounds (the wave's running count), plus in
// lanes below it (a ballot per digit bit).
__global__ __launch_bounds__(kRsThreads) void sparse_rsort_pass_kernel(int pass, uint32_t *sort_ws,
                                                                       size_t item_words, int S) {
  constexpr int R = kRsRounds, NW = kRsWaves;
  __shared__ __align__(16) uint16_t s_wc[NW][kRsDigits];  // per-wave digit counts
  __shared__ uint32_t s_off[kRsDigits];
  __shared__ __align__(16) uint32_t s_wsum[NW];
  RsPass rp;
  int np;
  uint32_t kmin;
  if (!rs_pass(pass, sort_ws, item_words, S, rp, np, kmin) || pass >= np) return;
  const int b = blockIdx.x, n = rp.n, sft = rp.sft;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int p0 = b * kRsKeys + wave * 64 * R + lane;  // this lane's position in round 0
  uint32_t kk[R], tk[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool valid = p0 + 64 * r < n;
    kk[r] = valid ? rp.sk[p0 + 64 * r] : 0u;
    tk[r] = valid ? rp.stk[p0 + 64 * r] : 0u;
  }
  // this block's offsets: thread t takes digits 2t, 2t + 1, adds each one's
  // counts over every block (total) and over the blocks before this one (up
  // to kRsSuper blocks one by one; beyond, whole superblocks' sums and then
  // the blocks of this block's superblock); an exclusive scan of the totals
  // over the digits gives each digit's start
  static_assert(kRsDPT == 2, "two digits (one uint2) per thread");
  {
    const uint2 *c = reinterpret_cast<const uint2 *>(rp.reg + ItemSort::cnt) + tid;
    uint32_t tot[2] = {0u, 0u}, pre[2] = {0u, 0u};
    // sums of n_part rows of uint2 (stride kRsDigits / 2) from src: all into
    // tot, the first n_pre also into pre
    auto add_rows = [&](const uint2 *src, int n_part, int n_pre, bool into_tot) {
      for (int j0 = 0; j0 < n_part; j0 += 8) {
        uint2 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          v[j] = j0 + j < n_part ? src[(size_t)(j0 + j) * (kRsDigits / 2)] : make_uint2(0u, 0u);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const bool before = j0 + j < n_pre;
          pre[0] += before ? v[j].x : 0u;
          pre[1] += before ? v[j].y : 0u;
          if (into_tot) {
            tot[0] += v[j].x;
            tot[1] += v[j].y;
          }
        }
      }
    };
    if (rp.G <= kRsSuper) {
      add_rows(c, rp.G, b, true);
    } else {
      const uint2 *sc = reinterpret_cast<const uint2 *>(rp.reg + ItemSort::sup(S)) + tid;
      const int Bb = b / kRsSuper;
      add_rows(sc, (rp.G + kRsSuper - 1) / kRsSuper, Bb, true);
      add_rows(c + (size_t)Bb * kRsSuper * (kRsDigits / 2), b - Bb * kRsSuper, b - Bb * kRsSuper,
               false);
    }
    const uint32_t mine = tot[0] + tot[1];
    uint32_t incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(incl, o, 64);
      if (lane >= o) incl += y;
    }
    if (lane == 63) s_wsum[wave] = incl;
    uint4 *z4 = reinterpret_cast<uint4 *>(&s_wc[0][0]);
    for (int i = tid; i < NW * kRsDigits / 8; i += kRsThreads) z4[i] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    const uint32_t base = incl - mine + waves_before<NW>(s_wsum, wave);
    s_off[2 * tid] = base + pre[0];
    s_off[2 * tid + 1] = base + tot[0] + pre[1];
  }
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t dg[R], rk[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool valid = p0 + 64 * r < n;
    dg[r] = (kk[r] >> sft) & (kRsDigits - 1u);
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < kRsBits; ++bit) {
      const uint64_t m = __ballot((dg[r] >> bit) & 1u);
      same &= ((dg[r] >> bit) & 1u) ? m : ~m;
    }
    const uint32_t lower = (uint32_t)__popcll(same & below);
    const uint32_t earlier = s_wc[wave][dg[r]];  // this wave's earlier rounds
    rk[r] = earlier + lower;
    if (valid && lower == 0u) s_wc[wave][dg[r]] = (uint16_t)(earlier + (uint32_t)__popcll(same));
  }
  __syncthreads();
  // per digit, the counts of the waves before (exclusive prefix, in place)
  for (int d = tid; d < kRsDigits; d += kRsThreads) {
    uint32_t run = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t c = s_wc[w][d];
      s_wc[w][d] = (uint16_t)run;
      run += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (p0 + 64 * r < n) {
      const uint32_t dst = s_off[dg[r]] + s_wc[wave][dg[r]] + rk[r];
      rp.dk[dst] = kk[r];
      rp.dtk[dst] = tk[r];
    }
  }
}

// One block of kSelThreads per item: the sparse-V selection.  n <=
// kSelectInBlock: select_small, all of it, as per-token weights.  Larger n:
// the exponentials (sparse_exp_kernel's) are added left to right (inv =
// 1/sum is kept at lg[n]) and the item sort's header written (its keys,
// key_hi(p) less the smallest key with the tokens in token order, come from
// its first count kernel); the sort orders p descending, ties older first;
// sparse_cut_kernel then takes the cut, sparse_vsum_kernel derives the
// weights and sums the weighted V rows over many blocks, and
// sparse_finish_kernel applies the inverse FWHT.  The V sum runs in token
// order instead of the reference's sorted order, which changes only its
// rounding; the selected set is the reference's.
__global__ __launch_bounds__(kSelThreads) void sparse_select_kernel(HeadDesc *const *item_desc,
                                                                    float v_mass, float *ws,
                                                                    size_t ws_stride,
                                                                    uint32_t *sort_ws,
                                                                    size_t item_words) {
  __shared__ SelectShared sh;
  const int item = blockIdx.x;
  const int tid = threadIdx.x;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, cap = d->cap;
  // items this kernel sorts itself take no item-sort pass
  if (sort_ws && n <= kSelectInBlock && tid == 0) {
    sort_ws[(size_t)item * item_words] = 0u;
    sort_ws[(size_t)item * item_words + 6] = 0u;
  }
  if (n == 0) return;
  float *lg = ws + (size_t)item * ws_stride;
  const int s0 = (int)(((long long)d->st.head - n + cap) % cap);
  if (n <= kSelectInBlock) {
    if (n <= kSelThreads) select_small<1>(d, v_mass, lg, n, s0, sh);
    else if (n <= 2 * kSelThreads) select_small<2>(d, v_mass, lg, n, s0, sh);
    else if (n <= 4 * kSelThreads) select_small<4>(d, v_mass, lg, n, s0, sh);
    else select_small<8>(d, v_mass, lg, n, s0, sh);
    return;
  }
  float *s_red = sh.red, *s_bcast = sh.bcast;

  // 1-2. the maximum and the exponentials come from the logits and exp
  // kernels (lg holds the e), each block's NaN flag and e range at st; then
  // the exponentials' left-to-right sum (a NaN term makes it NaN)
  const float *st = lg_stats(lg, n);
  const int nb = lg_blocks(n);
  int nan_e = 0;
  float e_lo = __builtin_inff(), e_hi = 0.0f;
  for (int b = tid; b < nb; b += kSelThreads) {
    nan_e |= st[kStat * b + 3] != 0.0f;
    e_lo = fminf(e_lo, st[kStat * b + 1]);
    e_hi = fmaxf(e_hi, st[kStat * b + 2]);
  }
  if (__syncthreads_or(nan_e)) {
    if (tid == 0) s_bcast[0] = __builtin_nanf("");
  } else {
    // the left-to-right sum of the exponentials in lg, 8,192 terms at a time
    static_assert(sizeof(ChainShared) <= sizeof(sh.cnt), "chain_sum_block's LDS in sh.cnt");
    ChainShared &cs = *reinterpret_cast<ChainShared *>(sh.cnt);
    const float sv =
        chain_sum_long<false>([lg](int i) { return lg[i]; }, n, 0.0f, __builtin_inff(), sh.xs, cs).s;
    if (tid == 0) s_bcast[0] = 1.0f / sv;
  }
  __syncthreads();
  const float inv = s_bcast[0];
  if (tid == 0) lg[n] = inv;

  // 3. the item sort's header: the passes the key range needs, the smallest
  // key (the first count kernel writes the keys less it, from lg and inv).
  // p = e * inv is monotone in e, so the largest e gives the smallest key and
  // the smallest e the largest (a NaN inv makes every key 0xFFFFFFFF).
  uint32_t *reg = sort_ws + (size_t)item * item_words;
  for (int off = 32; off > 0; off >>= 1) {
    e_lo = fminf(e_lo, __shfl_xor(e_lo, off));
    e_hi = fmaxf(e_hi, __shfl_xor(e_hi, off));
  }
  if ((tid & 63) == 0) {
    s_red[tid >> 6] = e_lo;
    s_red[32 + (tid >> 6)] = e_hi;
  }
  __syncthreads();
  for (int w = 0; w < kSelThreads / 64; ++w) {
    e_lo = fminf(e_lo, s_red[w]);
    e_hi = fmaxf(e_hi, s_red[32 + w]);
  }
  const uint32_t kmin = key_hi(__fmul_rn(e_hi, inv)), kmax = key_hi(__fmul_rn(e_lo, inv));
  if (tid == 0) {
    const uint32_t range = kmax - kmin;
    const int bits = range ? 32 - __clz((int)range) : 0;
    const int np = (bits + kRsBits - 1) / kRsBits;  // 0: every key equal, token order is sorted
    reg[0] = (uint32_t)np;
    reg[5] = kmin;
    reg[6] = (uint32_t)n;
  }
}

// The cut of an item above kSelectInBlock tokens, over its sorted keys (the
// item sort's final buffers: key_hi less the smallest key, and tokens).
// sparse_vsum_kernel derives the weights from it.
__global__ __launch_bounds__(kSelThreads) void sparse_cut_kernel(HeadDesc *const *item_desc,
                                                                 float v_mass, float *ws,
                                                                 size_t ws_stride, int S,
                                                                 const uint32_t *sort_ws,
                                                                 size_t item_words) {
  __shared__ float s_stage[kStage];
  __shared__ float s_bcast[2];
  __shared__ int s_cut;
  __shared__ uint64_t s_last;
  __shared__ float s_xs[seqsum_detail::kBlock * seqsum_detail::kMaxT];
  __shared__ ChainShared s_cs;
  const int item = blockIdx.x;
  const int tid = threadIdx.x;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size;
  if (n <= kSelectInBlock) return;  // select_small wrote its weights
  float *lg = ws + (size_t)item * ws_stride;
  // sorted key i (the last pass's output)
  const uint32_t *reg = sort_ws + (size_t)item * item_words;
  const size_t fin = reg[0] & 1u, Sa = ItemSort::sa(S);
  const uint32_t *kk = reg + ItemSort::keys(S) + fin * Sa;
  const uint32_t *tt = reg + ItemSort::keys(S) + (2 + fin) * Sa;
  const uint32_t kmin = reg[5];
  auto skey = [kk, tt, kmin](int i) -> uint64_t {
    return ((uint64_t)(kk[i] + kmin) << 32) | tt[i];
  };

  // 4. the cut: whole quads while mass < v_mass, then single tokens; NaN
  // probabilities (sorted last) keep the one-lane chain
  const int n_quads = n / 4;  // quads with ii + 3 < n
  auto quad = [kk, kmin](int k) {
    // the quad's four keys are adjacent and 16-byte aligned: one load
    const uint4 h = *reinterpret_cast<const uint4 *>(kk + 4 * k);
    return __fadd_rn(__fadd_rn(__fadd_rn(hi_p(h.x + kmin), hi_p(h.y + kmin)), hi_p(h.z + kmin)),
                     hi_p(h.w + kmin));
  };
  if (kk[n - 1] + kmin == 0xFFFFFFFFu) {
    float mass = 0.0f;
    int ii = 0;
    bool open = true;  // thread 0: the quad loop has not stopped
    for (int base = 0; base < n_quads; base += kStage) {
      const int m = n_quads - base < kStage ? n_quads - base : kStage;
      for (int k = tid; k < m; k += blockDim.x) s_stage[k] = quad(base + k);
      __syncthreads();
      if (tid == 0 && open) {
        const int k = mass_scan(s_stage, m, v_mass, &mass);
        ii = 4 * (base + k);
        open = k == m;
        s_bcast[1] = open ? 1.0f : 0.0f;
      }
      __syncthreads();
      if (s_bcast[1] == 0.0f) break;
      __syncthreads();
    }
    if (tid == 0) {
      for (; ii < n && mass < v_mass; ++ii) mass = __fadd_rn(mass, key_p(skey(ii)));
      s_cut = ii;
    }
  } else {
    const SeqResult rq = chain_sum_long<true>(quad, n_quads, 0.0f, v_mass, s_xs, s_cs);
    // the single tokens run only after every whole quad, i.e. over the last
    // n % 4 tokens at most (once the mass reaches v_mass they add nothing)
    if (tid == 0) {
      int ii = 4 * rq.count;
      float mass = rq.s;
      for (; ii < n && mass < v_mass; ++ii) mass = __fadd_rn(mass, key_p(skey(ii)));
      s_cut = ii;
    }
  }
  __syncthreads();
  if (tid == 0) s_last = s_cut > 0 ? skey(s_cut - 1) : 0;
  __syncthreads();
  const int cut = s_cut;
  const uint64_t last = s_last;

  // 5. the selection for sparse_vsum_kernel, which turns it into per-token
  // weights: the cut first keys of the sorted order, i.e. every key up to
  // the last one taken (keys are distinct)
  if (tid == 0) {
    lg[n + 1] = __uint_as_float(cut > 0 ? 1u : 0u);
    lg[n + 2] = __uint_as_float((uint32_t)last);
    lg[n + 3] = __uint_as_float((uint32_t)(last >> 32));
  }
}

// Short rings (n <= kFusedMax): one block of kSelThreads per item does the
// selection, the weighted V sum and the inverse FWHT, and at padded 64 the
// logits too.  The logits are sparse_logits_kernel's (same kdot_row and
// roundings), the selection is select_small's, so the selected set and the
// per-token weights are the multi-kernel path's bit for bit; the V sum's
// rounding order differs from the multi-kernel path's chunked sums, as both
// differ from the reference's sorted order.  Measured against the four
// launches at padded 64: 4 heads x 2,048 tokens 56 -> 52 us, 256 heads x
// 2,048 tokens 75 -> 58 us, even at 4,096 tokens.  At padded 128 one block
// per item computing every logit is slower than the logits kernel's many
// blocks (8 heads x 2,048 tokens 62 -> 80 us), so there the logits kernel
// runs first (LOGITS_IN) and the fused kernel takes over from the selection.
constexpr int kFusedMax = 3 * kSelThreads;

// V row unit read by one lane of the fused kernel: a 32-bit word of 2- or
// 4-bit codes (16 or 8 codes), or a 3-byte group of 8 3-bit codes.
template <int VB>
struct VWord {
  static constexpr int bytes = VB == 3 ? 3 : 4;
  static constexpr int codes = VB == 3 ? 8 : 32 / VB;
};

// Bit position of code c (0 = first) inside a unit as loaded: words are
// little-endian with codes MSB-first in each byte; a 3-byte group is the
// big-endian 24-bit value.
template <int VB>
__device__ __forceinline__ int vcode_shift(int c) {
  if constexpr (VB == 2) return 8 * (c >> 2) + 6 - 2 * (c & 3);
  else if constexpr (VB == 4) return 8 * (c >> 1) + 4 - 4 * (c & 1);
  else return 21 - 3 * c;
}


template <int PT, int KB, int VB, bool LOGITS_IN>
__global__ __launch_bounds__(kSelThreads) void sparse_fused_kernel(
    HeadDesc *const *item_desc, const float *__restrict__ queries, float v_mass, float inv_sqrt_p,
    float sqrt_p, float *ws, size_t ws_stride, float *__restrict__ outs) {
  // one LDS object with the codebooks and the query first: their addresses
  // stay below the 64 KB of a ds_read's immediate offset, so a codebook
  // lookup is one read of the code's byte offset (a separate variable may be
  // placed after the ~100 KB of SelectShared and cost an add per lookup)
  // V pair table (2-bit codes): a nibble of a row, two adjacent codes, to
  // their two centres in one read (16 entries: no bank conflicts; a 256-entry
  // byte table for 4-bit codes conflicts and is slower)
  constexpr int kPairs = VB == 2 ? 16 : 1;
  struct FusedShared {
    float cbk[16];
    float cb[16];
    float2 cb2[kPairs];
    float q[PT];
    SelectShared sel;
  };
  __shared__ FusedShared fs;
  SelectShared &sh = fs.sel;
  float *const s_q = fs.q;
  float *const s_cb = fs.cb;
  float *const s_cbk = fs.cbk;
  constexpr int UB = VWord<VB>::bytes, CPU = VWord<VB>::codes;
  constexpr int U = PT * VB / 8 / UB;  // units per V row (4..16)
  constexpr int TPI = 64 / U;          // tokens per wave step
  constexpr int NW = kSelThreads / 64;
  constexpr int UNR = 4;               // row loads in flight per lane
  const int item = blockIdx.x, tid = threadIdx.x;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, cap = d->cap, dim = d->dim;
  float *out = outs + (size_t)item * dim;
  if (n == 0) {
    for (int i = tid; i < dim; i += blockDim.x) out[i] = 0.0f;
    return;
  }
  if (tid < (1 << VB)) s_cb[tid] = cbv<VB>(tid);
  if constexpr (VB == 2) {
    if (tid < kPairs) fs.cb2[tid] = make_float2(cbv<2>(tid >> 2), cbv<2>(tid & 3));
  }
  if (tid < (1 << KB)) s_cbk[tid] = cbv<KB>(tid);
  float *lg = ws + (size_t)item * ws_stride;
  const int s0 = (int)(((long long)d->st.head - n + cap) % cap);
  const int E = n <= kSelThreads ? 1 : n <= 2 * kSelThreads ? 2 : 4;
  float lreg[4];  // the thread's logits when computed here
  if constexpr (!LOGITS_IN) {
    // logits of the tokens select_small gives this thread (E per thread),
    // handed over in registers; the query, then their K rows and scales
    // are requested before the query rotation, which hides the rows'
    // latency
    constexpr int KW = KRow<PT, KB>::words;
    const float2 qv = query_lanes(queries + (size_t)item * dim, dim, PT);
    uint32_t kw[4][KW];
    float ks[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = tid * E + e;
      if (e < E && t < n) {
        const int slot = ring_slot(s0, t, cap);
        ks[e] = d->k_scale[slot];
        kload_raw<PT, KB>(d->k_codes + (size_t)slot * d->k_pb, slot & kperm_mask(PT, KB), kw[e]);
      }
    }
    rotate_query_exact(s_q, nullptr, dim, PT, d->signs, inv_sqrt_p, sqrt_p, &qv);
    const float attn_s = 1.0f / (sqrtf((float)dim) * (float)PT);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = tid * E + e;
      if (e < E && t < n) {
        kperm_raw<PT, KB>(ring_slot(s0, t, cap) & kperm_mask(PT, KB), kw[e]);
        const float dot = kdot_words<PT, KB>(kw[e], s_q, s_cbk);
        lreg[e] = __fmul_rn(__fmul_rn(dot, attn_s), ks[e]);
      }
    }
  }
  // the weights go to LDS over the sort keys (select_small reads no key
  // after its cut)
  float *w_lds = reinterpret_cast<float *>(sh.key);
  const float *lin = LOGITS_IN ? nullptr : lreg;
  if (E == 1) select_small<1>(d, v_mass, lg, n, s0, sh, lin, w_lds);
  else if (E == 2) select_small<2>(d, v_mass, lg, n, s0, sh, lin, w_lds);
  else select_small<4>(d, v_mass, lg, n, s0, sh, lin, w_lds);
  __syncthreads();

  // weighted V rows: lane (sub, u) takes unit u of token wave * TPI + sub,
  // then every NW * TPI tokens; UNR rows are requested before any is used
  const int lane = tid & 63, wave = tid >> 6, sub = lane / U, u = lane % U;
  const uint8_t *vsrc = d->v_codes;
  const int vpb = d->v_pb;
  float acc[CPU];
#pragma unroll
  for (int c = 0; c < CPU; ++c) acc[c] = 0.0f;
  for (int t = wave * TPI + sub; t < n; t += NW * TPI * UNR) {
    uint32_t bits[UNR];
    float wt[UNR];
#pragma unroll
    for (int j = 0; j < UNR; ++j) {
      const int tj = t + j * NW * TPI;
      wt[j] = tj < n ? w_lds[tj] : 0.0f;
      const uint8_t *row = vsrc + (size_t)ring_slot(s0, tj < n ? tj : n - 1, cap) * vpb;
      if constexpr (UB == 4) {
        bits[j] = reinterpret_cast<const uint32_t *>(row)[u];
      } else {
        const uint8_t *g = row + 3 * u;
        bits[j] = ((uint32_t)g[0] << 16) | ((uint32_t)g[1] << 8) | (uint32_t)g[2];
      }
    }
#pragma unroll
    for (int j = 0; j < UNR; ++j) {
      if constexpr (VB == 2) {
        // codes 2k and 2k + 1 share a nibble, the first in its high bits; the
        // same products in the same order as one code at a time
#pragma unroll
        for (int k = 0; k < CPU / 2; ++k) {
          const float2 cv = fs.cb2[(bits[j] >> (vcode_shift<VB>(2 * k + 1))) & (uint32_t)(kPairs - 1)];
          acc[2 * k] = fmaf(cv.x, wt[j], acc[2 * k]);
          acc[2 * k + 1] = fmaf(cv.y, wt[j], acc[2 * k + 1]);
        }
      } else {
#pragma unroll
        for (int c = 0; c < CPU; ++c)
          acc[c] = fmaf(s_cb[(bits[j] >> vcode_shift<VB>(c)) & ((1u << VB) - 1u)], wt[j], acc[c]);
      }
    }
  }
  // the TPI token groups of a wave (lanes u + U * sub), then the waves in order
#pragma unroll
  for (int off = U; off < 64; off <<= 1)
#pragma unroll
    for (int c = 0; c < CPU; ++c) acc[c] += __shfl_xor(acc[c], off);
  float *s_red = reinterpret_cast<float *>(sh.cnt);  // NW x PT floats
  if (sub == 0) {
#pragma unroll
    for (int c = 0; c < CPU; ++c) s_red[wave * PT + u * CPU + c] = acc[c];
  }
  __syncthreads();
  float *s_acc = sh.stage;
  for (int j = tid; j < PT; j += blockDim.x) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) a += s_red[w * PT + j];
    s_acc[j] = a;
  }
  __syncthreads();
  inverse_fwht_out(s_acc, PT, dim, d->signs, out);
}

// Codes per byte-aligned unit of a packed row and the unit's size in bytes:
// 2-bit: 1 byte = 4 codes, 4-bit: 1 byte = 2 codes, 3-bit: 3 bytes = 8 codes.
template <int VB>
struct VUnit {
  static constexpr int codes = VB == 3 ? 8 : 8 / VB;
  static constexpr int bytes = VB == 3 ? 3 : 1;
};

// Tokens per sparse_vsum_kernel block (at most).
constexpr int kVChunkMax = 256;

// Weighted V sum of one block's chunk of tokens:
//   part[item][split][j] = sum over t in the chunk of fma(CB_V[code_tj], w_t, .)
// with w_t the selection weight (0 for tokens left out).  A row of P codes is
// U = P / VUnit::codes units; a wave takes TPI = max(1, 64 / U) tokens per
// step, lane (sub, u) the units u, u + 64, ... of token sub, so every lane
// reads whole bytes of a row in one coalesced cache line.  PT: the padded
// size when it is 64 or 128 (one unit per lane: 16 tokens' loads in flight
// per lane), else 0 (any size, 4 tokens in flight).
template <int VB, int PT>
__global__ __launch_bounds__(kThreads) void sparse_vsum_kernel(HeadDesc *const *item_desc,
                                                               float *ws, size_t ws_stride,
                                                               int chunk, int n_splits,
                                                               float *partials) {
  constexpr int CPU = VUnit<VB>::codes, UB = VUnit<VB>::bytes;
  // codes per lane: at most 16 (P = 1024: 4 x 4, 8 x 2 or 2 x 8), one unit at PT
  constexpr int kMaxAcc = PT ? CPU : 16;
  __shared__ float s_cb[16];
  __shared__ float s_red[kThreads / 64][kMaxPadded];
  __shared__ float s_w[kVChunkMax];  // the chunk's weights
  const int item = blockIdx.y, split = blockIdx.x;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, cap = d->cap, P = d->padded, vpb = d->v_pb;
  const int t0 = split * chunk;
  if (t0 >= n) return;
  if (threadIdx.x < (1 << VB)) s_cb[threadIdx.x] = cbv<VB>(threadIdx.x);
  float *w = ws + (size_t)item * ws_stride;
  const int s0 = (int)(((long long)d->st.head - n + cap) % cap);
  // rings above kSelectInBlock: w holds the exponentials, and the cut
  // kernel's selection sits at [n]: 1/sum, whether any token is taken, and
  // the last sort key taken; the weight (p_t * vscale_t) / sqrt(p) of a
  // selected token (p_t recomputed exactly as its key was made) is derived
  // here and written back over its exponential
  const bool derive = n > kSelectInBlock;
  const float inv = derive ? w[n] : 1.0f;
  const bool any = derive && __float_as_uint(w[n + 1]) != 0u;
  const uint64_t last =
      derive ? ((uint64_t)__float_as_uint(w[n + 3]) << 32) | __float_as_uint(w[n + 2]) : 0u;
  const float isp = 1.0f / sqrtf((float)P);
  const int U = (P + CPU - 1) / CPU;
  const int TPI = U < 64 ? 64 / U : 1;
  const int R = U > 64 ? U / 64 : 1;  // units per lane (R * CPU <= kMaxAcc)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / (U < 64 ? U : 64), u0 = lane % (U < 64 ? U : 64);
  const bool active = sub < TPI;
  float acc[kMaxAcc];
#pragma unroll
  for (int k = 0; k < kMaxAcc; ++k) acc[k] = 0.0f;
  const int t_end = t0 + chunk < n ? t0 + chunk : n;
  const uint8_t *vsrc = d->v_codes;
  // the chunk's weights into LDS, a token a thread (derived once, not by
  // every lane that reads a unit of the token's row)
  for (int i = threadIdx.x; i < t_end - t0; i += kThreads) {
    const int t = t0 + i;
    float wt = w[t];
    if (derive) {
      const float p = __fmul_rn(wt, inv);
      wt = any && make_key(p, t) <= last
               ? __fmul_rn(__fmul_rn(p, d->v_scale[ring_slot(s0, t, cap)]), isp)
               : 0.0f;
      w[t] = wt;
    }
    s_w[i] = wt;
  }
  __syncthreads();
  // UNR tokens per step, their weights and code units requested before any
  // is used (rows of weight 0 still load: the step's loads stay in flight
  // together)
  constexpr int UNR = PT ? 16 : 4;
  const int step = (kThreads / 64) * TPI;
  if (active) {
    for (int t = t0 + wave * TPI + sub; t < t_end; t += UNR * step) {
      float wt[UNR];
      uint32_t bits[UNR][kMaxAcc / CPU];
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        const int tj = t + j * step;
        wt[j] = tj < t_end ? s_w[tj - t0] : 0.0f;
        const uint8_t *row = vsrc + (size_t)ring_slot(s0, tj < t_end ? tj : t_end - 1, cap) * vpb;
#pragma unroll
        for (int r = 0; r < kMaxAcc / CPU; ++r) {
          bits[j][r] = 0u;
          if (r >= R) continue;
          const int u = u0 + 64 * r;
          if constexpr (UB == 1) {
            bits[j][r] = row[u];
          } else {
            // a row of fewer than 8 codes holds a partial group
            const int b0 = 3 * u;
            bits[j][r] = ((uint32_t)row[b0] << 16) |
                         ((b0 + 1 < vpb ? (uint32_t)row[b0 + 1] : 0u) << 8) |
                         (b0 + 2 < vpb ? (uint32_t)row[b0 + 2] : 0u);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < UNR; ++j)
#pragma unroll
        for (int r = 0; r < kMaxAcc / CPU; ++r) {
          if (r >= R) break;
#pragma unroll
          for (int c = 0; c < CPU; ++c) {
            const int code = (int)((bits[j][r] >> (VB * (CPU - 1 - c))) & ((1u << VB) - 1u));
            acc[r * CPU + c] = fmaf(s_cb[code], wt[j], acc[r * CPU + c]);
          }
        }
    }
  }
  // sum the TPI token groups of each wave (lanes u0 + U * sub), then the waves
  for (int off = U; off < 64; off <<= 1)
#pragma unroll
    for (int k = 0; k < kMaxAcc; ++k) acc[k] += __shfl_xor(acc[k], off);
  if (active && sub == 0) {
    for (int r = 0; r < R; ++r)
      for (int c = 0; c < CPU; ++c) {
        const int j = (u0 + 64 * r) * CPU + c;
        if (j < P) s_red[wave][j] = acc[r * CPU + c];
      }
  }
  __syncthreads();
  float *part = partials + ((size_t)item * n_splits + split) * P;
  for (int j = threadIdx.x; j < P; j += kThreads) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < kThreads / 64; ++k) a += s_red[k][j];
    part[j] = a;
  }
}

// Sum of the splits of each item, inverse FWHT (fwht.cpp:106-134), signs.
__global__ __launch_bounds__(kThreads) void sparse_finish_kernel(HeadDesc *const *item_desc,
                                                                 int chunk, int n_splits,
                                                                 const float *partials,
                                                                 float *__restrict__ outs) {
  __shared__ float s_acc[kMaxPadded];
  const int item = blockIdx.x;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, dim = d->dim, P = d->padded;
  float *out = outs + (size_t)item * dim;
  if (n == 0) {
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = 0.0f;
    return;
  }
  const int used = (n + chunk - 1) / chunk;
  const float *part = partials + (size_t)item * n_splits * P;
  // the chunks' partial sums: kThreads / P thread groups (P < kThreads) take
  // every groups-th chunk with several loads in flight, then add up in order
  __shared__ float s_grp[kThreads];
  const int groups = P < kThreads ? kThreads / P : 1;
  if (groups > 1) {
    const int j = threadIdx.x % P, grp = threadIdx.x / P;
    float a = 0.0f;
#pragma unroll 8
    for (int sp = grp; sp < used; sp += groups) a += part[(size_t)sp * P + j];
    s_grp[threadIdx.x] = a;
    __syncthreads();
    if (threadIdx.x < P) {
      float t = 0.0f;
      for (int g = 0; g < groups; ++g) t += s_grp[g * P + threadIdx.x];
      s_acc[threadIdx.x] = t;
    }
  } else {
    for (int j = threadIdx.x; j < P; j += blockDim.x) {
      float a = 0.0f;
#pragma unroll 8
      for (int sp = 0; sp < used; ++sp) a += part[(size_t)sp * P + j];
      s_acc[j] = a;
    }
  }
  __syncthreads();
  inverse_fwht_out(s_acc, P, dim, d->signs, out);
}

// Per item: the logits, then the exponentials, then the weights (n floats),
// 1/sum at [n] for rings that sort outside the select kernel, and the
// logits blocks' statistics from [n + 4].
size_t item_stride(int n) { return lg_words(n) + (size_t)kStat * lg_blocks(n); }

// Items per launch: the grid holds items in one dimension (at most 65,535).
constexpr int kMaxItems = 65535;

size_t align64(size_t x) { return (x + 63) & ~(size_t)63; }

}  // namespace

// Tokens per sparse_vsum_kernel block.
constexpr int kVChunk = kVChunkMax;

int vsum_splits(int n) { return (n + kVChunk - 1) / kVChunk; }

size_t sparse_workspace_floats(int n_items, const DecodeShape &sh) {
  const int n = sh.max_n > 0 ? sh.max_n : 1;
  size_t f = align64((size_t)n_items * item_stride(n) + (size_t)n_items * vsum_splits(n) * sh.padded);
  const int cnt = n_items < kMaxItems ? n_items : kMaxItems;
  if (n > kSelectInBlock) f += align64((size_t)cnt * ItemSort::words(n));
  return f;
}

hipError_t launch_decode_sparse(HeadDesc *const *descs, int n_items, const DecodeShape &sh,
                                float v_mass, const float *d_q, float *d_out, float *ws,
                                hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  const int n = sh.max_n > 0 ? sh.max_n : 1;
  const size_t stride = item_stride(n);
  const float sp = sqrtf((float)sh.padded);
  const float isp = 1.0f / sp;
  const int splits = vsum_splits(n);
  float *parts_all = ws + (size_t)n_items * stride;
  float *sort_base = ws + align64((size_t)n_items * stride + (size_t)n_items * splits * sh.padded);
  // items go in the grid's y dimension (at most 65,535 per launch); chunks of
  // items take consecutive queries, outputs and workspace
  for (int c0 = 0; c0 < n_items; c0 += kMaxItems) {
    const int cnt = n_items - c0 < kMaxItems ? n_items - c0 : kMaxItems;
    HeadDesc *const *dsc = descs + c0;
    const float *q = d_q + (size_t)c0 * sh.dim;
    float *out = d_out + (size_t)c0 * sh.dim;
    float *w = ws + (size_t)c0 * stride;
    float *parts = parts_all + (size_t)c0 * splits * sh.padded;
    const dim3 g1(lg_blocks(n), cnt);
    if (n <= kFusedMax && (sh.padded == 64 || sh.padded == 128)) {
      // padded 128: the logits kernel's many blocks first, then the rest in
      // one block per item
#define AQ_FUSED(PT, KB_, VB_)                                                                    \
  if (sh.padded == PT && sh.k_bits == KB_ && sh.v_bits == VB_) {                                  \
    if (PT == 128)                                                                                \
      sparse_logits_kernel<PT, KB_><<<g1, kThreads, 0, s>>>(dsc, q, n, isp, sp, w, stride);        \
    sparse_fused_kernel<PT, KB_, VB_, PT == 128><<<cnt, kSelThreads, 0, s>>>(dsc, q, v_mass, isp,  \
                                                                              sp, w, stride, out); \
    const hipError_t fe = hipGetLastError();                                                      \
    if (fe != hipSuccess) return fe;                                                              \
    continue;                                                                                     \
  }
      AQ_FUSED(64, 2, 2) AQ_FUSED(64, 2, 3) AQ_FUSED(64, 2, 4)
      AQ_FUSED(64, 3, 2) AQ_FUSED(64, 3, 3) AQ_FUSED(64, 3, 4)
      AQ_FUSED(64, 4, 2) AQ_FUSED(64, 4, 3) AQ_FUSED(64, 4, 4)
      AQ_FUSED(128, 2, 2) AQ_FUSED(128, 2, 3) AQ_FUSED(128, 2, 4)
      AQ_FUSED(128, 3, 2) AQ_FUSED(128, 3, 3) AQ_FUSED(128, 3, 4)
      AQ_FUSED(128, 4, 2) AQ_FUSED(128, 4, 3) AQ_FUSED(128, 4, 4)
#undef AQ_FUSED
    }
#define AQ_LOGITS(PT, KB_) \
  sparse_logits_kernel<PT, KB_><<<g1, kThreads, 0, s>>>(dsc, q, n, isp, sp, w, stride)
    switch (sh.k_bits) {
      case 2:
        if (sh.padded == 64) AQ_LOGITS(64, 2);
        else if (sh.padded == 128) AQ_LOGITS(128, 2);
        else AQ_LOGITS(0, 2);
        break;
      case 3:
        if (sh.padded == 64) AQ_LOGITS(64, 3);
        else if (sh.padded == 128) AQ_LOGITS(128, 3);
        else AQ_LOGITS(0, 3);
        break;
      case 4:
        if (sh.padded == 64) AQ_LOGITS(64, 4);
        else if (sh.padded == 128) AQ_LOGITS(128, 4);
        else AQ_LOGITS(0, 4);
        break;
      default: return hipErrorInvalidValue;
    }
#undef AQ_LOGITS
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (n > kSelectInBlock) {
      sparse_exp_kernel<<<g1, kThreads, 0, s>>>(dsc, w, stride);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    if (n <= kSelectInBlock) {
      sparse_select_kernel<<<cnt, kSelThreads, 0, s>>>(dsc, v_mass, w, stride, nullptr, 0);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    } else {
      // the item sort: keys, up to kRsPasses passes (each returns at once
      // for items whose key range is shorter), the cut
      uint32_t *rs = reinterpret_cast<uint32_t *>(sort_base);
      const size_t iw = ItemSort::words(n);
      sparse_select_kernel<<<cnt, kSelThreads, 0, s>>>(dsc, v_mass, w, stride, rs, iw);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
      const dim3 gp(rs_blocks(n), cnt);
      const int ns = rs_supers(n);
      for (int pass = 0; pass < kRsPasses; ++pass) {
        sparse_rsort_count_kernel<<<gp, kRsThreads, 0, s>>>(pass, rs, iw, n, w, stride);
        if (ns > 0)
          sparse_rsort_super_kernel<<<dim3(ns, cnt), kRsThreads, 0, s>>>(pass, rs, iw, n);
        sparse_rsort_pass_kernel<<<gp, kRsThreads, 0, s>>>(pass, rs, iw, n);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
      sparse_cut_kernel<<<cnt, kSelThreads, 0, s>>>(dsc, v_mass, w, stride, n, rs, iw);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    const dim3 g3(splits, cnt);
    switch (sh.v_bits) {
      case 2:
        if (sh.padded == 64) sparse_vsum_kernel<2, 64><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        else if (sh.padded == 128) sparse_vsum_kernel<2, 128><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        else sparse_vsum_kernel<2, 0><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        break;
      case 3:
        if (sh.padded == 64) sparse_vsum_kernel<3, 64><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        else if (sh.padded == 128) sparse_vsum_kernel<3, 128><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        else sparse_vsum_kernel<3, 0><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        break;
      case 4:
        if (sh.padded == 64) sparse_vsum_kernel<4, 64><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        else if (sh.padded == 128) sparse_vsum_kernel<4, 128><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        else sparse_vsum_kernel<4, 0><<<g3, kThreads, 0, s>>>(dsc, w, stride, kVChunk, splits, parts);
        break;
      default: return hipErrorInvalidValue;
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    sparse_finish_kernel<<<cnt, kThreads, 0, s>>>(dsc, kVChunk, splits, parts, out);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace aq
