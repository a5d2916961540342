// mquery.hip -- decode of many queries per head (gfx950).
//
// With nq queries per head, the dense decode (attention.cpp:373-474 with
// v_mass <= 0) is two products per head over the ring:
//   logits   S[q][t] = sum_i qr[q][i] * CB_K[c_ti]        (qr = H (D . q))
//   output   O[q][d] = sum_t p[q][t] * vscale_t / sqrt(p) * CB_V[c_td]
// so each K/V tile can be read once for all the queries of its head instead
// of once per query (decode.hip's LUT kernel, one query per item).
//
// Logits are the reference's own floats.  On peaked softmaxes (outlier
// channels: logits of +-300, where one fp32 unit is 3e-5) the reference's
// rounding of the dot moves outputs by about 1e-4, so a more accurate dot
// (a double-precision matrix product was tried) lands as far from it on the
// other side.  Each logit is computed as attention.cpp:93-136 and :83-88
// compute it: eight fused multiply-add chains (chain L takes dims L, L + 8,
// ... in order), combined ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7)), times
// 1/(sqrt(dim) p), times the key's scale; the query rotation repeats the
// reference's float steps (attention.cpp:528-550, fwht.cpp:33-66).  A lane
// owns one token of a 64-token tile with its dequantised K row in registers,
// and the rotated query entries, uniform across the wave, come from the
// scalar cache as the FMAs' SGPR operand: the FMA stream has no other
// operand traffic.  The V sum runs on v_mfma_f32_16x16x4f32, the softmax
// weight and the V scale folded into its A operand (fp32 accumulation, as the
// reference's).  The online softmax is the LUT kernel's with the reference's
// -1e30 seed, in natural units (exp2 of (logit - max) * log2 e, so the
// weights of the tokens near the maximum carry no rounding of the logit's
// magnitude); splits over tokens end in decode.hip's finalize kernel.
//
// Operand layouts (established on the device): lane l supplies A[l % 16][l /
// 16] and B[l / 16][l % 16]; result register r of lane l is D[4 (l / 16) +
// r][l % 16].  The V product takes queries as M and tokens as K, so lane l
// supplies the weight of query l % 16 and token 4 r + l / 16 of each 16-token
// subtile at k-step r; the logits (one token per lane) reach that layout
// through LDS.
//
// Block: kMqWaves (8) waves and kMqQueries (16) queries of one head over one
// token split.  Every wave handles all 16 queries; the waves split the
// tokens: wave w takes the 64-token tiles starting at t_begin + 64 w, then
// every 64 kMqWaves tokens.  Lane l owns token l of its wave's tile: the K
// row, dequantised through the codebook in LDS into registers (the next
// tile's row requested a tile ahead; rows stored in XOR byte order,
// device.hpp kperm_mask, are read back in reference order by load_k_row),
// and the V slices the MFMA's B operand takes from global memory.  A wave's
// logits reach the MFMA layout through its own LDS region (transposed, row
// stride 17); at the end the waves' (m, l, acc) records meet in LDS and are
// merged per query.
#include <algorithm>

#include "launch.hpp"

namespace aq {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMqWaves = 8;
constexpr int kMqThreads = 64 * kMqWaves;
constexpr int kMqQueries = 16;  // queries per block, shared by its waves
constexpr int kMqTile = 64;     // tokens per wave step (one per lane)
constexpr float kLog2e = 1.44269504088896340736f;

// Code k (MSB-first packing, quantizer.cpp:156-209) of a little-endian word
// stream w[] holding a row's bytes from byte 0.
template <int B>
__device__ __forceinline__ uint32_t code_in(const uint32_t *w, int k) {
  if constexpr (B == 4) {
    const int byte = k >> 1;
    return (w[byte >> 2] >> (8 * (byte & 3) + ((k & 1) ? 0 : 4))) & 15u;
  } else if constexpr (B == 2) {
    const int byte = k >> 2;
    return (w[byte >> 2] >> (8 * (byte & 3) + 6 - 2 * (k & 3))) & 3u;
  } else {
    // 3 bits: group G = k / 8 is the big-endian 24-bit value of bytes 3G..3G+2
    const int G = k >> 3, b0 = 3 * G;
    auto byte_at = [&](int b) { return (w[b >> 2] >> (8 * (b & 3))) & 0xFFu; };
    const uint32_t v = (byte_at(b0) << 16) | (byte_at(b0 + 1) << 8) | byte_at(b0 + 2);
    return (v >> (21 - 3 * (k & 7))) & 7u;
  }
}

// The K row of `slot` in reference byte order, as little-endian words.  Rows
// of 2/4-bit codes are stored XOR-permuted (device.hpp kperm_mask): reference
// word w sits at stored word w ^ (x >> 2) with its bytes permuted by x & 3,
// x = slot & mask.
template <int P, int KB>
__device__ __forceinline__ void load_k_row(const HeadDesc *d, uint32_t slot, uint32_t *kw) {
  constexpr int W = P * KB / 32;
  const uint32_t *r32 = reinterpret_cast<const uint32_t *>(d->k_codes + (size_t)slot * (P * KB / 8));
  if constexpr (KB == 3) {
#pragma unroll
    for (int i = 0; i < W; ++i) kw[i] = r32[i];
  } else {
    constexpr uint32_t xmask = (uint32_t)kperm_mask(P, KB);
    const uint32_t x = slot & xmask;
    const uint32_t sel = 0x03020100u ^ ((x & 3u) * 0x01010101u);
    if constexpr (W % 4 == 0) {
      // whole 16-byte chunks: chunk c of the reference row is stored chunk c ^ (x >> 4)
      const uint4 *r128 = reinterpret_cast<const uint4 *>(r32);
#pragma unroll
      for (int c = 0; c < W / 4; ++c) {
        const uint4 v = r128[c ^ (x >> 4)];
        const uint32_t q[4] = {v.x, v.y, v.z, v.w};
        const uint32_t xw = (x >> 2) & 3u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // reference word 4c + i is stored word (4c + i) ^ (x >> 2): in chunk c ^ (x >> 4), slot i ^ xw
          uint32_t sw = q[0];
          sw = xw == (uint32_t)(i ^ 1) ? q[1] : sw;
          sw = xw == (uint32_t)(i ^ 2) ? q[2] : sw;
          sw = xw == (uint32_t)(i ^ 3) ? q[3] : sw;
          kw[4 * c + i] = __builtin_amdgcn_perm(0u, sw, sel);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) kw[i] = __builtin_amdgcn_perm(0u, r32[i ^ (x >> 2)], sel);
    }
  }
}

// This lane's V codes: the P / 16 codes of dims [P/16 c, P/16 (c + 1)) of
// the row (V rows are unpermuted MSB-first bit streams), left-aligned in a
// word, code i in bits [32 - VB (i + 1), 32 - VB i).
template <int P, int VB>
__device__ __forceinline__ uint32_t v_slice(const uint8_t *row, int c) {
  constexpr int BITS = (P / 16) * VB, ROWW = P * VB / 32;
  const uint32_t *r32 = reinterpret_cast<const uint32_t *>(row);
  const int b0 = c * BITS;
  const int w0 = b0 >> 5;
  const uint32_t a = __builtin_bswap32(r32[w0]);
  if constexpr (32 % BITS == 0) {
    return a << (b0 & 31);  // the slice never straddles a word
  } else {
    const uint32_t b = __builtin_bswap32(r32[min(w0 + 1, ROWW - 1)]);
    const uint64_t win = ((uint64_t)a << 32) | b;
    return (uint32_t)((win << (b0 & 31)) >> 32);
  }
}

// Read-only global memory seen through the constant address space: loads at
// wave-uniform addresses become scalar loads.
typedef const __attribute__((address_space(4))) float cfloat;

// Rotated queries of query group qg of head h: rows of P floats at
// qrot[((h * qgroups + qg) * 16 + jj) * P], zero rows past nq.  One wave per
// query, lane l holding entries l and l + 64, with the reference's float steps
// (attention.cpp:528-550, fwht.cpp:33-66): qn = sqrt(sum q^2 + 1e-12) left to
// right, q / qn, signs, butterflies of span 1, 2, ..., P/2 (lo + hi, lo - hi),
// * RN(1/RN(sqrt p)), * RN(sqrt p * qn).
template <int P>
__global__ __launch_bounds__(256) void mq_rotate_kernel(HeadDesc *const *item_desc, int n_heads,
                                                        int nq, int qgroups,
                                                        const float *__restrict__ queries,
                                                        float *__restrict__ qrot) {
  constexpr int E = P / 64;  // entries per lane
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= qgroups * kMqQueries) return;
  const int j = row;  // query index: group row / 16, row % 16 within it
  const HeadDesc *d = item_desc[h];
  const int dim = d->dim;
  float *out = qrot + ((size_t)h * qgroups * kMqQueries + row) * P;
  if (j >= nq) {
#pragma unroll
    for (int i = 0; i < E; ++i) out[lane + 64 * i] = 0.0f;
    return;
  }
  const float *q = queries + (size_t)(j * n_heads + h) * dim;
  const cfloat *qs = (const cfloat *)q;
  // left to right: the row's 16-entry blocks come in as scalar loads ahead of
  // their squares
  float sq = 0.0f;
  const int nb = dim / 16;
  for (int b = 0; b < nb; ++b) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = qs[16 * b + k];
#pragma unroll
    for (int k = 0; k < 16; ++k) sq = __fadd_rn(sq, __fmul_rn(v[k], v[k]));
  }
  for (int e = 16 * nb; e < dim; ++e) sq = __fadd_rn(sq, __fmul_rn(qs[e], qs[e]));
  const float qn = sqrtf(__fadd_rn(sq, 1e-12f));
  const float inv = 1.0f / qn;
  float x[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int e = lane + 64 * i;
    float v = __fmul_rn(e < dim ? q[e] : 0.0f, inv);
    if (!((d->signs[e >> 5] >> (e & 31)) & 1u)) v = -v;
    x[i] = v;
  }
#pragma unroll
  for (int len = 1; len < 64; len <<= 1) {
    const bool upper = (lane & len) != 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float other = __shfl_xor(x[i], len, 64);
      x[i] = upper ? __fsub_rn(other, x[i]) : __fadd_rn(x[i], other);
    }
  }
  if constexpr (E == 2) {
    const float lo = x[0], hi = x[1];
    x[0] = __fadd_rn(lo, hi);
    x[1] = __fsub_rn(lo, hi);
  }
  const float sqrt_p = sqrtf((float)P);
  const float inv_sqrt_p = 1.0f / sqrt_p;
  const float post = __fmul_rn(sqrt_p, qn);
#pragma unroll
  for (int i = 0; i < E; ++i) out[lane + 64 * i] = __fmul_rn(__fmul_rn(x[i], inv_sqrt_p), post);
}


// Block (split, head h, query group qg), 1-D grid with the split fastest:
// the blocks resident together mostly share one head's 16 queries, 8 KB of
// scalar-cache working set.  Wave w of the block takes the 64-token tiles w,
// w + 4, ... of the block's token range on its own (no barriers in the token
// loop) and the four waves' (m, l, acc) merge in LDS at the end.
template <int P, int KB, int VB>
__global__ __launch_bounds__(kMqThreads, 1) void decode_mq_kernel(
    HeadDesc *const *item_desc, int n_heads, int nq, int qgroups, int chunk, int n_splits,
    const float *__restrict__ qrot, float *__restrict__ partials) {
  constexpr int NT = P / 16;       // 16-column output tiles; lane c holds dims [NT c, NT c + NT)
  constexpr int KW = P * KB / 32;  // words of a K row
  constexpr int LST = 17;          // row stride of a wave's transposed logits
  constexpr int MST = P + 4;       // row stride of a wave's merge record: m, l, pad, pad, acc
  constexpr uint32_t vmask = (1u << VB) - 1u;
  constexpr int SMEM = kMqWaves * kMqQueries * MST > kMqWaves * kMqTile * LST
                           ? kMqWaves * kMqQueries * MST
                           : kMqWaves * kMqTile * LST;
  __shared__ __align__(16) float s_buf[SMEM];  // transposed logits; then the merge records
  __shared__ float s_cbk[16];
  __shared__ float s_cbv[16];

  const int bid = blockIdx.x;
  const int split = bid % n_splits, rest = bid / n_splits;
  const int h = rest % n_heads, qg = rest / n_heads;
  const HeadDesc *d = item_desc[h];
  const int dim = d->dim, n = d->st.size;
  const int t_begin = split * chunk, t_end = min(n, t_begin + chunk);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, g = lane >> 4;
  const int j0 = qg * kMqQueries;  // first query of the block
  auto part_of = [&](int j) {
    return partials + ((size_t)(j * n_heads + h) * n_splits + split) * (P + 4);
  };

  if (t_begin >= t_end) {
    // empty split: (m, l, acc) = (-inf, 0, 0) for the block's queries
    for (int i = threadIdx.x; i < kMqQueries * (P + 4); i += kMqThreads) {
      const int jj = i / (P + 4), e = i - jj * (P + 4);
      if (j0 + jj < nq) part_of(j0 + jj)[e] = e == 0 ? -INFINITY : 0.0f;
    }
    return;
  }

  if (threadIdx.x < (1 << KB)) s_cbk[threadIdx.x] = cb<KB>(threadIdx.x);
  if (threadIdx.x < (1 << VB)) s_cbv[threadIdx.x] = cb<VB>(threadIdx.x);
  __syncthreads();

  // the block's 16 rotated queries (wave-uniform: scalar loads)
  const cfloat *qw = (const cfloat *)(qrot + (size_t)(h * qgroups + qg) * kMqQueries * P);
  const float attn_s = 1.0f / (sqrtf((float)dim) * (float)P);
  const float isp = 1.0f / sqrtf((float)P);
  const uint8_t *vbase = d->v_codes;
  constexpr int v_pb = P * VB / 8;
  float *s_lg = s_buf + wave * (kMqTile * LST);
  f32x4 acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;  // query c16; the first tile seeds it with the reference's -1e30
  float l_part = 0.0f;      // this lane's tokens' share of query c16's sum

  // K row of this lane's token in the wave's first tile (then prefetched a tile ahead)
  const int tb0 = t_begin + kMqTile * wave;
  uint32_t kw[KW];
  float ksc = 0.0f;
  if (tb0 < t_end) {
    const uint32_t slot = (uint32_t)min(tb0 + lane, t_end - 1);
    load_k_row<P, KB>(d, slot, kw);
    ksc = d->k_scale[slot];
  }
  for (int tb = tb0; tb < t_end; tb += kMqTile * kMqWaves) {
    // ---- V slices of the lane's 16 tokens (consumed after the logits) ----
    const bool tvalid = tb + lane < t_end;
    uint32_t vsl[16];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int vs = min(tb + 16 * u + 4 * r + g, t_end - 1);
        vsl[4 * u + r] = v_slice<P, VB>(vbase + (size_t)vs * v_pb, c16);
      }
    // this lane's token's V scale, passed on through the logits' pad column
    const float vsc_own = tvalid ? d->v_scale[min(tb + lane, t_end - 1)] : 0.0f;
    float kv[P];
#pragma unroll
    for (int e = 0; e < P; ++e) kv[e] = s_cbk[code_in<KB>(kw, e)];
    const float kscale = ksc;
    // prefetch the next tile's K row
    const int tn = tb + kMqTile * kMqWaves;
    if (tn < t_end) {
      const uint32_t slot = (uint32_t)min(tn + lane, t_end - 1);
      load_k_row<P, KB>(d, slot, kw);
      ksc = d->k_scale[slot];
    }

    // ---- logits (attention.cpp:93-136, :83-88), one query at a time, its
    // 64-float halves loaded into SGPRs in turn ----
#pragma unroll 1
    for (int q = 0; q < kMqQueries; ++q) {
      const cfloat *qq = qw + q * P;
      float s8[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int e = 0; e < 64; ++e) s8[e & 7] = fmaf(kv[e], qq[e], s8[e & 7]);
      if constexpr (P == 128) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int e = 64; e < 128; ++e) s8[e & 7] = fmaf(kv[e], qq[e], s8[e & 7]);
      }
      const float dot = (__fadd_rn(s8[0], s8[4]) + __fadd_rn(s8[1], s8[5])) +
                        (__fadd_rn(s8[2], s8[6]) + __fadd_rn(s8[3], s8[7]));
      s_lg[lane * LST + q] = tvalid ? __fmul_rn(__fmul_rn(dot, attn_s), kscale) : -INFINITY;
    }
    s_lg[lane * LST + 16] = vsc_own;

    // ---- to the V product's layout: lane has query c16, tokens 16u + 4r + g ----
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float lg[4][4], vsc[4][4];
    float tmax = -1e30f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        lg[u][r] = s_lg[(16 * u + 4 * r + g) * LST + c16];
        vsc[u][r] = s_lg[(16 * u + 4 * r + g) * LST + 16];
        tmax = fmaxf(tmax, lg[u][r]);
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // the next tile's logits overwrite s_lg
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = __builtin_amdgcn_exp2f(__fmul_rn(m_run - m_new, kLog2e));
    m_run = m_new;
    l_part *= alpha;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // rescale O rows (query 4 g + r of the result layout) by their query's alpha
      const float a = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) acc[nt][r] *= a;
    }

    // ---- weighted V: O[q][NT c16 + nt] += sum_t w[q][t] V[t][NT c16 + nt] ----
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = __builtin_amdgcn_exp2f(__fmul_rn(lg[u][r] - m_new, kLog2e));
        l_part += e;
        const float w = e * vsc[u][r] * isp;
        const uint32_t sl = vsl[4 * u + r];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float v = s_cbv[(sl >> (32 - VB * (nt + 1))) & vmask];
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(w, v, acc[nt], 0, 0, 0);
        }
      }
  }

  // ---- merge the waves: record (m, l) of query c16 and acc rows 4 g + r ----
  __syncthreads();  // every wave is done with its logits
  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  float *rec = s_buf + wave * (kMqQueries * MST);
  if (g == 0) {
    rec[c16 * MST] = m_run;
    rec[c16 * MST + 1] = l_tot;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) rec[(4 * g + r) * MST + 4 + NT * c16 + nt] = acc[nt][r];
  __syncthreads();
  for (int i = threadIdx.x; i < kMqQueries * (P + 4); i += kMqThreads) {
    const int jj = i / (P + 4), e = i - jj * (P + 4);
    if (j0 + jj >= nq || e == 2 || e == 3) continue;
    float mw[kMqWaves], M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kMqWaves; ++w) {
      mw[w] = s_buf[(w * kMqQueries + jj) * MST];
      M = fmaxf(M, mw[w]);
    }
    float out;
    if (e == 0) {
      out = M;
    } else {
      out = 0.0f;
#pragma unroll
      for (int w = 0; w < kMqWaves; ++w) {
        // a wave without tokens has m = -inf and contributes 0
        const float f = __builtin_amdgcn_exp2f(__fmul_rn(mw[w] - M, kLog2e));
        out += s_buf[(w * kMqQueries + jj) * MST + e] * f;
      }
    }
    part_of(j0 + jj)[e] = out;
  }
}

struct MqPlan {
  int splits, chunk, qgroups;
};

MqPlan mq_plan(int n_heads, int nq, int max_n) {
  MqPlan mp;
  mp.qgroups = (nq + kMqQueries - 1) / kMqQueries;
  const int max1 = max_n > 0 ? max_n : 1;
  // about one block per CU (256 blocks), at least one tile per wave
  constexpr int kStep = kMqTile * kMqWaves;
  const int blocks = n_heads * mp.qgroups;
  int splits = (256 + blocks - 1) / blocks;
  const int by_work = (max1 + kStep - 1) / kStep;
  splits = std::max(1, std::min(splits, by_work));
  int chunk = (max1 + splits - 1) / splits;
  chunk = ((chunk + kStep - 1) / kStep) * kStep;
  mp.chunk = chunk;
  mp.splits = (max1 + chunk - 1) / chunk;
  return mp;
}

// Queries per head from which the matrix-core kernel replaces the LUT
// kernel's one-query items.
constexpr int kMqMinQueries = 16;

bool mq_eligible(int n_items, int n_heads, const DecodeShape &sh) {
  if (n_heads <= 0 || n_items % n_heads != 0) return false;
  const int nq = n_items / n_heads;
  const bool kq = sh.k_bits >= 2 && sh.k_bits <= 4, vq = sh.v_bits >= 2 && sh.v_bits <= 4;
  return !sh.raw && kq && vq && (sh.padded == 64 || sh.padded == 128) && nq >= kMqMinQueries &&
         n_heads <= 65535 && (int64_t)n_heads * ((nq + kMqQueries - 1) / kMqQueries) *
                                      ((sh.max_n + kMqTile * kMqWaves - 1) / (kMqTile * kMqWaves)) <
                                  (int64_t)1 << 31;
}

template <int P>
hipError_t dispatch_mq(const DecodeShape &sh, dim3 grid, HeadDesc *const *descs, int n_heads,
                       int nq, const MqPlan &mp, const float *q, float *qrot, float *part,
                       hipStream_t s) {
  mq_rotate_kernel<P><<<dim3((mp.qgroups * kMqQueries + 3) / 4, n_heads), 256, 0, s>>>(
      descs, n_heads, nq, mp.qgroups, q, qrot);
  if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
#define AQ_MQ(KB_, VB_)                                                                     \
  if (sh.k_bits == KB_ && sh.v_bits == VB_) {                                               \
    decode_mq_kernel<P, KB_, VB_><<<grid, kMqThreads, 0, s>>>(descs, n_heads, nq, mp.qgroups, \
                                                              mp.chunk, mp.splits, qrot, part); \
    return hipGetLastError();                                                               \
  }
  AQ_MQ(4, 2) AQ_MQ(4, 3) AQ_MQ(4, 4)
  AQ_MQ(3, 2) AQ_MQ(3, 3) AQ_MQ(3, 4)
  AQ_MQ(2, 2) AQ_MQ(2, 3) AQ_MQ(2, 4)
#undef AQ_MQ
  return hipErrorInvalidValue;
}

// Workspace of the multi-query path: the rotated queries (n_heads * qgroups
// * 64 rows of P floats), then the split partials (item, split) of P + 4.
size_t mq_qrot_floats(int n_heads, const MqPlan &mp, int padded) {
  return (size_t)n_heads * mp.qgroups * kMqQueries * padded;
}

}  // namespace

size_t decode_multi_workspace_floats(int n_items, int n_heads, const DecodeShape &sh) {
  if (!mq_eligible(n_items, n_heads, sh)) return decode_workspace_floats(n_items, sh);
  const MqPlan mp = mq_plan(n_heads, n_items / n_heads, sh.max_n);
  return mq_qrot_floats(n_heads, mp, sh.padded) + (size_t)n_items * mp.splits * (sh.padded + 4);
}

hipError_t launch_decode_multi(HeadDesc *const *descs, int n_items, int n_heads,
                               const DecodeShape &sh, const float *d_q, float *d_out,
                               float *d_ws, hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  if (!mq_eligible(n_items, n_heads, sh))
    return launch_decode(descs, n_items, sh, d_q, d_out, d_ws, s);
  const int nq = n_items / n_heads;
  const MqPlan mp = mq_plan(n_heads, nq, sh.max_n);
  const dim3 grid(mp.splits * n_heads * mp.qgroups);
  float *qrot = d_ws, *part = d_ws + mq_qrot_floats(n_heads, mp, sh.padded);
  const hipError_t e =
      sh.padded == 64 ? dispatch_mq<64>(sh, grid, descs, n_heads, nq, mp, d_q, qrot, part, s)
                      : dispatch_mq<128>(sh, grid, descs, n_heads, nq, mp, d_q, qrot, part, s);
  if (e != hipSuccess) return e;
  return launch_finalize(descs, n_items, sh.padded, mp.splits, part, d_out, true, s);
}

}  // namespace aq
