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
// Kernels: one grid over (token blocks, items) computes the logits; one block
// per item does softmax, a bitonic sort (in LDS up to 8192 tokens, else in the
// workspace), the cut, the V gather and the inverse FWHT.
#include "launch.hpp"

namespace aq {

namespace {

constexpr int kThreads = 256;
constexpr int kLdsSort = 8192;

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
__device__ void rotate_query_exact(float *s_q, const float *q, int dim, int P,
                                   const uint32_t *signs, float inv_sqrt_p, float sqrt_p) {
  __shared__ float s_qn;
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int i = 0; i < dim; ++i) s = __fadd_rn(s, __fmul_rn(q[i], q[i]));
    s_qn = sqrtf(__fadd_rn(s, 1e-12f));
  }
  __syncthreads();
  const float qn = s_qn;
  const float inv = 1.0f / qn;
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_q[i] = __fmul_rn(i < dim ? q[i] : 0.0f, inv);
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

template <int KB>
__global__ __launch_bounds__(kThreads) void sparse_logits_kernel(HeadDesc *const *item_desc,
                                                                 const float *__restrict__ queries,
                                                                 int max_n, float inv_sqrt_p,
                                                                 float sqrt_p, float *ws,
                                                                 size_t ws_stride) {
  __shared__ float s_q[kMaxPadded];
  const int item = blockIdx.y;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, cap = d->cap, dim = d->dim, P = d->padded;
  if ((int)(blockIdx.x * blockDim.x) >= n) return;
  rotate_query_exact(s_q, queries + (size_t)item * dim, dim, P, d->signs, inv_sqrt_p, sqrt_p);
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int slot = (int)(((long long)d->st.head - n + cap + i) % cap);
  const uint8_t *row = d->k_codes + (size_t)slot * d->k_pb;
  const int x = slot & kperm_mask(P, KB);
  // 8 FMA lanes over codes L, L+8, ...; lanes summed pairwise.
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < P; j += 8)
#pragma unroll
    for (int L = 0; L < 8; ++L)
      if (j + L < P) s[L] = fmaf(cbv<KB>(kcode_at<KB>(row, j + L, x)), s_q[j + L], s[L]);
  const float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];
  const float dot = (t0 + t1) + (t2 + t3);
  const float attn_s = 1.0f / (sqrtf((float)dim) * (float)P);
  ws[(size_t)item * ws_stride + i] = __fmul_rn(__fmul_rn(dot, attn_s), d->k_scale[slot]);
}

struct Key {
  float p;
  int i;
};

// a precedes b: larger probability first, then older token; NaN last.
__device__ __forceinline__ bool before(Key a, Key b) {
  const bool an = a.p != a.p, bn = b.p != b.p;
  if (an || bn) return !an && bn;
  if (a.p != b.p) return a.p > b.p;
  return a.i < b.i;
}

__device__ void bitonic(Key *m, int N) {
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < N; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const Key a = m[i], b = m[ixj];
          const bool up = (i & k) == 0;
          if (up ? before(b, a) : before(a, b)) {
            m[i] = b;
            m[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

template <int VB>
__global__ __launch_bounds__(kThreads) void sparse_select_kernel(HeadDesc *const *item_desc,
                                                                 float v_mass, float *ws,
                                                                 size_t ws_stride, int sort_cap,
                                                                 float *__restrict__ outs) {
  __shared__ Key s_keys[kLdsSort];
  __shared__ float s_acc[kMaxPadded];
  __shared__ float s_red[kThreads];
  __shared__ float s_inv;
  __shared__ int s_cut;
  const int item = blockIdx.x;
  const HeadDesc *d = item_desc[item];
  const int n = d->st.size, cap = d->cap, dim = d->dim, P = d->padded;
  float *out = outs + (size_t)item * dim;
  if (n == 0) {
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = 0.0f;
    return;
  }
  float *lg = ws + (size_t)item * ws_stride;
  int N = 1;
  while (N < n) N <<= 1;
  Key *keys = N <= kLdsSort ? s_keys : reinterpret_cast<Key *>(lg + sort_cap);

  // max with the reference's starting value and NaN-skipping compare
  float mx = -1e30f;
  for (int i = threadIdx.x; i < n; i += blockDim.x)
    if (lg[i] > mx) mx = lg[i];
  s_red[threadIdx.x] = mx;
  __syncthreads();
  for (int w = blockDim.x / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w && s_red[threadIdx.x + w] > s_red[threadIdx.x])
      s_red[threadIdx.x] = s_red[threadIdx.x + w];
    __syncthreads();
  }
  mx = s_red[0];
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) lg[i] = expf(lg[i] - mx);
  __syncthreads();
  if (threadIdx.x == 0) {
    float sv = 0.0f;
    for (int i = 0; i < n; ++i) sv = __fadd_rn(sv, lg[i]);
    s_inv = 1.0f / sv;
  }
  __syncthreads();
  const float inv = s_inv;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    Key k;
    if (i < n) {
      lg[i] = __fmul_rn(lg[i], inv);
      k.p = lg[i];
      k.i = i;
    } else {
      k.p = -1.0f;
      k.i = 0x7fffffff;
    }
    keys[i] = k;
  }
  __syncthreads();
  bitonic(keys, N);

  if (threadIdx.x == 0) {
    float mass = 0.0f;
    int ii = 0;
    for (; ii + 3 < n && mass < v_mass; ii += 4) {
      const float q4 = __fadd_rn(__fadd_rn(__fadd_rn(keys[ii].p, keys[ii + 1].p), keys[ii + 2].p),
                                 keys[ii + 3].p);
      mass = __fadd_rn(mass, q4);
    }
    for (; ii < n && mass < v_mass; ++ii) mass = __fadd_rn(mass, keys[ii].p);
    s_cut = ii;
  }
  __syncthreads();
  const int cut = s_cut;
  const float isp = 1.0f / sqrtf((float)P);
  for (int j = threadIdx.x; j < P; j += blockDim.x) {
    float a = 0.0f;
    for (int k = 0; k < cut; ++k) {
      const int t = keys[k].i;
      const int slot = (int)(((long long)d->st.head - n + cap + t) % cap);
      const float w = __fmul_rn(__fmul_rn(keys[k].p, d->v_scale[slot]), isp);
      a = fmaf(cbv<VB>(code_at<VB>(d->v_codes + (size_t)slot * d->v_pb, j)), w, a);
    }
    s_acc[j] = a;
  }
  __syncthreads();
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
    const float v = __fmul_rn(s_acc[i], scale);
    out[i] = sign_plus(d->signs, i) ? v : -v;
  }
}

int pow2_at_least(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// Per item: logits/probabilities (keys_at floats, even so the 8-byte sort keys
// that follow are aligned), then 2 floats per sort key.
int keys_at(int n) { return ((n + 32 + 1) / 2) * 2; }

size_t item_stride(int n) { return (size_t)keys_at(n) + 2 * (size_t)pow2_at_least(n); }

}  // namespace

size_t sparse_workspace_floats(int n_items, const DecodeShape &sh) {
  const int n = sh.max_n > 0 ? sh.max_n : 1;
  return (size_t)n_items * item_stride(n);
}

hipError_t launch_decode_sparse(HeadDesc *const *descs, int n_items, const DecodeShape &sh,
                                float v_mass, const float *d_q, float *d_out, float *ws,
                                hipStream_t s) {
  if (n_items <= 0) return hipSuccess;
  const int n = sh.max_n > 0 ? sh.max_n : 1;
  const size_t stride = item_stride(n);
  const int sort_cap = keys_at(n);
  const float sp = sqrtf((float)sh.padded);
  const float isp = 1.0f / sp;
  const dim3 g1((n + kThreads - 1) / kThreads, n_items);
  switch (sh.k_bits) {
    case 2: sparse_logits_kernel<2><<<g1, kThreads, 0, s>>>(descs, d_q, n, isp, sp, ws, stride); break;
    case 3: sparse_logits_kernel<3><<<g1, kThreads, 0, s>>>(descs, d_q, n, isp, sp, ws, stride); break;
    case 4: sparse_logits_kernel<4><<<g1, kThreads, 0, s>>>(descs, d_q, n, isp, sp, ws, stride); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  switch (sh.v_bits) {
    case 2: sparse_select_kernel<2><<<n_items, kThreads, 0, s>>>(descs, v_mass, ws, stride, sort_cap, d_out); break;
    case 3: sparse_select_kernel<3><<<n_items, kThreads, 0, s>>>(descs, v_mass, ws, stride, sort_cap, d_out); break;
    case 4: sparse_select_kernel<4><<<n_items, kThreads, 0, s>>>(descs, v_mass, ws, stride, sort_cap, d_out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace aq
