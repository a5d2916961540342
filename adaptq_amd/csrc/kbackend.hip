// kbackend.hip -- IKernelBackend (include/adaptq/kernel.h) on gfx950.
//
// The reference's V2 runtime takes its compute primitives from an
// IKernelBackend (kernels/scalar/kdot_scalar.cpp is its portable reference:
// fwht_forward/inverse, kdot_batch, vaccum_batch over host CompressResult
// arrays).  This backend packs the rows the CompressResults point to into
// pinned staging, copies them to the device on its own stream and runs:
//   kb_kdot_kernel        one lane per token: (q_rot . CB[codes]) * scale / p,
//                         the reference's left-to-right sum (unfused)
//   kb_vaccum_kernel      blocks of 256 tokens, one thread per dimension:
//                         partial sums of w * scale * CB[code]; kb_sum_kernel
//                         adds the block partials in block order
//   kb_fwht_*_kernel      one block per vector: the reference's stage
//                         structure and scale roundings (core/fwht.cpp:33-66,
//                         :106-134), so results are bit-exact
// Rows are the reference's packed layout (quantizer.cpp:156-225), read as they
// come from the runtime's storage; the library's own XOR-ordered rings are
// not involved.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>

#include "../../include/adaptq/kernel.h"
#include "device.hpp"

namespace aq {
namespace {

constexpr int kKbChunk = 256;  // tokens per vaccum block

template <int B>
__device__ __forceinline__ int kb_code(const uint8_t *row, int i) {
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

template <int B>
__global__ __launch_bounds__(256) void kb_kdot_kernel(const float *__restrict__ q,
                                                      const uint8_t *__restrict__ rows,
                                                      const float *__restrict__ scales, int N,
                                                      int P, int rb, float inv,
                                                      float *__restrict__ out) {
  __shared__ float s_q[kMaxPadded];
  __shared__ float s_cb[16];
  for (int i = threadIdx.x; i < P; i += blockDim.x) s_q[i] = q[i];
  for (int i = threadIdx.x; i < (1 << B); i += blockDim.x) s_cb[i] = cb<B>(i);
  __syncthreads();
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const uint8_t *row = rows + (size_t)t * rb;
  float dot = 0.0f;
  for (int i = 0; i < P; ++i) dot = __fadd_rn(dot, __fmul_rn(s_q[i], s_cb[kb_code<B>(row, i)]));
  out[t] = __fmul_rn(__fmul_rn(dot, scales[t]), inv);
}

template <int B>
__global__ void kb_vaccum_kernel(const uint8_t *__restrict__ rows, const float *__restrict__ w,
                                 const float *__restrict__ scales, int N, int P, int rb,
                                 float *__restrict__ part) {
  __shared__ float s_cb[16];
  for (int i = threadIdx.x; i < (1 << B); i += blockDim.x) s_cb[i] = cb<B>(i);  // blockDim may be < 16
  __syncthreads();
  const int d = threadIdx.x;  // blockDim.x == P
  const int t0 = blockIdx.x * kKbChunk, t1 = min(N, t0 + kKbChunk);
  float a = 0.0f;
  for (int t = t0; t < t1; ++t) {
    const float wt = w[t];
    if (wt == 0.0f) continue;
    const float ws = __fmul_rn(wt, scales[t]);
    a = __fadd_rn(a, __fmul_rn(ws, s_cb[kb_code<B>(rows + (size_t)t * rb, d)]));
  }
  part[(size_t)blockIdx.x * P + d] = a;
}

__global__ void kb_sum_kernel(const float *__restrict__ part, int n_parts, int P,
                              float *__restrict__ acc) {
  const int d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= P) return;
  float a = 0.0f;
  for (int c = 0; c < n_parts; ++c) a = __fadd_rn(a, part[(size_t)c * P + d]);
  acc[d] = a;
}

// Butterfly stages len = first .. P/2 on s[P] (one block, blockDim >= P/2).
__device__ void kb_stages(float *s, int P, int first) {
  for (int len = first; len < P; len <<= 1) {
    for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
      const int j = (k / len) * 2 * len + (k % len);
      const float lo = s[j], hi = s[j + len];
      s[j] = __fadd_rn(lo, hi);
      s[j + len] = __fsub_rn(lo, hi);
    }
    __syncthreads();
  }
}

// fwht.cpp:33-66: signs fused into the len-1 stage, remaining stages, then
// x *= RN(1 / RN(sqrt(p))).
__global__ void kb_fwht_forward_kernel(float *x, const int8_t *D, int P) {
  __shared__ float s[kMaxPadded];
  if (P == 1) {
    if (threadIdx.x == 0) x[0] = __fmul_rn(x[0], (float)D[0]);
    return;
  }
  for (int k = threadIdx.x; k < P / 2; k += blockDim.x) {
    const float a = __fmul_rn(x[2 * k], (float)D[2 * k]);
    const float b = __fmul_rn(x[2 * k + 1], (float)D[2 * k + 1]);
    s[2 * k] = __fadd_rn(a, b);
    s[2 * k + 1] = __fsub_rn(a, b);
  }
  __syncthreads();
  kb_stages(s, P, 2);
  const float inv = 1.0f / sqrtf((float)P);
  for (int i = threadIdx.x; i < P; i += blockDim.x) x[i] = __fmul_rn(s[i], inv);
}

// fwht.cpp:106-134: every stage, then x = (x * RN(1 / RN(sqrt(p)))) * D.
__global__ void kb_fwht_inverse_kernel(float *x, const int8_t *D, int P) {
  __shared__ float s[kMaxPadded];
  for (int i = threadIdx.x; i < P; i += blockDim.x) s[i] = x[i];
  __syncthreads();
  kb_stages(s, P, 1);
  const float scale = 1.0f / sqrtf((float)P);
  for (int i = threadIdx.x; i < P; i += blockDim.x)
    x[i] = __fmul_rn(__fmul_rn(s[i], scale), (float)D[i]);
}

void kb_check(hipError_t e, const char *what) {
  if (e != hipSuccess)
    throw std::runtime_error(std::string("adaptq hip kernel backend: ") + what + ": " +
                             hipGetErrorString(e));
}

struct KbBuf {
  void *p = nullptr;
  size_t bytes = 0;
  bool pinned = false;
  void ensure(size_t n, const char *what) {
    if (n <= bytes) return;
    release();
    const size_t want = std::max<size_t>(n, 4096);
    kb_check(pinned ? hipHostMalloc(&p, want, hipHostMallocDefault) : hipMalloc(&p, want), what);
    bytes = want;
  }
  void release() {
    if (p) (void)(pinned ? hipHostFree(p) : hipFree(p));
    p = nullptr;
    bytes = 0;
  }
};

class HipKernelBackend final : public adaptq::IKernelBackend {
 public:
  void fwht_forward(float *x, const int8_t *D, int padded) override { fwht(x, D, padded, true); }
  void fwht_inverse(float *x, const int8_t *D, int padded) override { fwht(x, D, padded, false); }

  void kdot_batch(const float *q_rot, const adaptq::CompressResult *k_results, int N, int padded,
                  int bits, float *logits_out) override {
    if (N <= 0) return;
    check_shape(padded, bits);
    std::lock_guard<std::mutex> g(mu_);
    init();
    const int rb = packed_bytes(padded, bits);
    stage_rows(k_results, N, rb);
    hq_.ensure((size_t)padded * 4, "pinned query");
    std::memcpy(hq_.p, q_rot, (size_t)padded * 4);
    dq_.ensure((size_t)padded * 4, "device query");
    dout_.ensure((size_t)N * 4, "device logits");
    kb_check(hipMemcpyAsync(dq_.p, hq_.p, (size_t)padded * 4, hipMemcpyHostToDevice, s_), "copy");
    const float inv = 1.0f / (float)padded;
    const dim3 grid((unsigned)((N + 255) / 256));
    const float *q = static_cast<const float *>(dq_.p);
    const auto *rows = static_cast<const uint8_t *>(drows_.p);
    const auto *sc = static_cast<const float *>(dscale_.p);
    float *out = static_cast<float *>(dout_.p);
    if (bits == 2) kb_kdot_kernel<2><<<grid, 256, 0, s_>>>(q, rows, sc, N, padded, rb, inv, out);
    else if (bits == 3) kb_kdot_kernel<3><<<grid, 256, 0, s_>>>(q, rows, sc, N, padded, rb, inv, out);
    else kb_kdot_kernel<4><<<grid, 256, 0, s_>>>(q, rows, sc, N, padded, rb, inv, out);
    kb_check(hipGetLastError(), "kdot launch");
    hout_.ensure((size_t)N * 4, "pinned logits");
    kb_check(hipMemcpyAsync(hout_.p, out, (size_t)N * 4, hipMemcpyDeviceToHost, s_), "copy");
    kb_check(hipStreamSynchronize(s_), "kdot");
    std::memcpy(logits_out, hout_.p, (size_t)N * 4);
  }

  void vaccum_batch(float *acc, const adaptq::CompressResult *v_results, const float *weights,
                    int N, int padded, int bits) override {
    check_shape(padded, bits);
    if (N <= 0) {
      std::memset(acc, 0, (size_t)padded * 4);
      return;
    }
    std::lock_guard<std::mutex> g(mu_);
    init();
    const int rb = packed_bytes(padded, bits);
    stage_rows(v_results, N, rb);
    hw_.ensure((size_t)N * 4, "pinned weights");
    std::memcpy(hw_.p, weights, (size_t)N * 4);
    dw_.ensure((size_t)N * 4, "device weights");
    kb_check(hipMemcpyAsync(dw_.p, hw_.p, (size_t)N * 4, hipMemcpyHostToDevice, s_), "copy");
    const int parts = (N + kKbChunk - 1) / kKbChunk;
    dpart_.ensure((size_t)parts * padded * 4, "device partials");
    dout_.ensure((size_t)padded * 4, "device acc");
    const auto *rows = static_cast<const uint8_t *>(drows_.p);
    const auto *w = static_cast<const float *>(dw_.p);
    const auto *sc = static_cast<const float *>(dscale_.p);
    float *part = static_cast<float *>(dpart_.p);
    if (bits == 2) kb_vaccum_kernel<2><<<parts, padded, 0, s_>>>(rows, w, sc, N, padded, rb, part);
    else if (bits == 3) kb_vaccum_kernel<3><<<parts, padded, 0, s_>>>(rows, w, sc, N, padded, rb, part);
    else kb_vaccum_kernel<4><<<parts, padded, 0, s_>>>(rows, w, sc, N, padded, rb, part);
    kb_check(hipGetLastError(), "vaccum launch");
    kb_sum_kernel<<<(padded + 255) / 256, 256, 0, s_>>>(part, parts, padded,
                                                        static_cast<float *>(dout_.p));
    kb_check(hipGetLastError(), "vaccum sum launch");
    hout_.ensure((size_t)padded * 4, "pinned acc");
    kb_check(hipMemcpyAsync(hout_.p, dout_.p, (size_t)padded * 4, hipMemcpyDeviceToHost, s_), "copy");
    kb_check(hipStreamSynchronize(s_), "vaccum");
    std::memcpy(acc, hout_.p, (size_t)padded * 4);
  }

  bool is_available() const override {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess && n > 0;
  }
  const char *name() const override { return "hip-gfx950"; }

 private:
  static void check_shape(int padded, int bits) {
    if (padded < 1 || padded > kMaxPadded || (padded & (padded - 1)) != 0)
      throw std::invalid_argument("adaptq hip kernel backend: padded must be a power of two <= 1024");
    if (bits < 2 || bits > 4)
      throw std::invalid_argument("adaptq hip kernel backend: bits must be 2, 3 or 4");
  }

  void init() {
    if (ready_) return;
    kb_check(hipStreamCreateWithFlags(&s_, hipStreamNonBlocking), "stream");
    for (KbBuf *b : {&hrows_, &hscale_, &hq_, &hw_, &hout_, &hx_}) b->pinned = true;
    ready_ = true;
  }

  // rows[i] = the first rb bytes of results[i].data, scales[i] = results[i].scale
  void stage_rows(const adaptq::CompressResult *r, int N, int rb) {
    hrows_.ensure((size_t)N * rb, "pinned rows");
    hscale_.ensure((size_t)N * 4, "pinned scales");
    auto *hr = static_cast<uint8_t *>(hrows_.p);
    auto *hs = static_cast<float *>(hscale_.p);
    for (int i = 0; i < N; ++i) {
      if (!r[i].data || r[i].data_bytes < rb)
        throw std::invalid_argument("adaptq hip kernel backend: a CompressResult holds fewer "
                                    "bytes than a packed row");
      std::memcpy(hr + (size_t)i * rb, r[i].data, (size_t)rb);
      hs[i] = r[i].scale;
    }
    drows_.ensure((size_t)N * rb, "device rows");
    dscale_.ensure((size_t)N * 4, "device scales");
    kb_check(hipMemcpyAsync(drows_.p, hr, (size_t)N * rb, hipMemcpyHostToDevice, s_), "copy");
    kb_check(hipMemcpyAsync(dscale_.p, hs, (size_t)N * 4, hipMemcpyHostToDevice, s_), "copy");
  }

  void fwht(float *x, const int8_t *D, int padded, bool forward) {
    if (padded < 1 || padded > kMaxPadded || (padded & (padded - 1)) != 0)
      throw std::invalid_argument("adaptq hip kernel backend: padded must be a power of two <= 1024");
    std::lock_guard<std::mutex> g(mu_);
    init();
    hx_.ensure((size_t)padded * 5, "pinned vector");
    auto *hx = static_cast<uint8_t *>(hx_.p);
    std::memcpy(hx, x, (size_t)padded * 4);
    std::memcpy(hx + (size_t)padded * 4, D, (size_t)padded);
    dx_.ensure((size_t)padded * 5, "device vector");
    kb_check(hipMemcpyAsync(dx_.p, hx, (size_t)padded * 5, hipMemcpyHostToDevice, s_), "copy");
    float *dx = static_cast<float *>(dx_.p);
    const auto *dD = reinterpret_cast<const int8_t *>(static_cast<uint8_t *>(dx_.p) + (size_t)padded * 4);
    const int threads = std::max(1, std::min(padded / 2, 512));
    if (forward) kb_fwht_forward_kernel<<<1, threads, 0, s_>>>(dx, dD, padded);
    else kb_fwht_inverse_kernel<<<1, threads, 0, s_>>>(dx, dD, padded);
    kb_check(hipGetLastError(), "fwht launch");
    kb_check(hipMemcpyAsync(hx, dx, (size_t)padded * 4, hipMemcpyDeviceToHost, s_), "copy");
    kb_check(hipStreamSynchronize(s_), "fwht");
    std::memcpy(x, hx, (size_t)padded * 4);
  }

  std::mutex mu_;
  bool ready_ = false;
  hipStream_t s_ = nullptr;
  KbBuf hrows_, hscale_, hq_, hw_, hout_, hx_;            // pinned host staging
  KbBuf drows_, dscale_, dq_, dw_, dout_, dpart_, dx_;    // device
};

}  // namespace
}  // namespace aq

namespace adaptq {

IKernelBackend *create_hip_backend() {
  static aq::HipKernelBackend backend;
  return &backend;
}

IKernelBackend *select_kernel_backend() { return create_hip_backend(); }

}  // namespace adaptq
