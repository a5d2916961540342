// layout.hip -- strided row gather/scatter between a caller's tensor layout
// (ggml's [dim, n_heads, n_tokens] f32 tensors with byte strides nb1, nb2)
// and the contiguous [n][dim] rows the append and decode launches take.
#include "launch.hpp"

namespace aq {

namespace {

// Contiguous row r = a * B + b  <->  strided row at byte offset a*sa + b*sb.
__global__ void gather_rows_kernel(float *__restrict__ dst, const uint8_t *__restrict__ src,
                                   int A, int B, int dim, size_t sa, size_t sb) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)A * B * dim;
  if (i >= total) return;
  const size_t r = i / dim;
  const int d = (int)(i - r * dim);
  const size_t a = r / B, b = r - a * B;
  dst[i] = reinterpret_cast<const float *>(src + a * sa + b * sb)[d];
}

__global__ void scatter_rows_kernel(uint8_t *__restrict__ dst, const float *__restrict__ src,
                                    int A, int B, int dim, size_t sa, size_t sb) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)A * B * dim;
  if (i >= total) return;
  const size_t r = i / dim;
  const int d = (int)(i - r * dim);
  const size_t a = r / B, b = r - a * B;
  reinterpret_cast<float *>(dst + a * sa + b * sb)[d] = src[i];
}

}  // namespace

hipError_t launch_gather_rows(float *d_dst, const void *d_src, int A, int B, int dim, size_t sa,
                              size_t sb, hipStream_t s) {
  const size_t total = (size_t)A * B * dim;
  if (total == 0) return hipSuccess;
  gather_rows_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
      d_dst, static_cast<const uint8_t *>(d_src), A, B, dim, sa, sb);
  return hipGetLastError();
}

hipError_t launch_scatter_rows(void *d_dst, const float *d_src, int A, int B, int dim, size_t sa,
                               size_t sb, hipStream_t s) {
  const size_t total = (size_t)A * B * dim;
  if (total == 0) return hipSuccess;
  scatter_rows_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(
      static_cast<uint8_t *>(d_dst), d_src, A, B, dim, sa, sb);
  return hipGetLastError();
}

}  // namespace aq
