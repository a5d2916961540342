// kernel_shim.cpp -- test harness around the reference's scalar IKernelBackend.
//
// TEST INFRASTRUCTURE ONLY.  Compiled with the reference's
// kernels/scalar/kdot_scalar.cpp, core/fwht.cpp and core/codebook.cpp, read in
// place from /root/reference (see oracle/Makefile), into
// oracle/_ref/libkernel_ref.so.  Exposes the reference's portable backend
// (its correctness reference for every other backend) through plain C entry
// points with the same arguments as the kernel check program's cases.
#include "adaptq/kernel.h"

#include <vector>

namespace adaptq {
IKernelBackend *create_scalar_backend();
}

extern "C" {

void kref_kdot(const float *q, const unsigned char *rows, const float *scales, int N, int P,
               int bits, float *out) {
  const int rb = (P * bits + 7) / 8;
  std::vector<adaptq::CompressResult> r((size_t)N);
  for (int i = 0; i < N; ++i)
    r[(size_t)i] = adaptq::CompressResult{rows + (size_t)i * rb, rb, scales[i], (uint8_t)bits,
                                          (adaptq::StorageSlot)i};
  adaptq::create_scalar_backend()->kdot_batch(q, r.data(), N, P, bits, out);
}

void kref_vaccum(const unsigned char *rows, const float *scales, const float *w, int N, int P,
                 int bits, float *acc) {
  const int rb = (P * bits + 7) / 8;
  std::vector<adaptq::CompressResult> r((size_t)N);
  for (int i = 0; i < N; ++i)
    r[(size_t)i] = adaptq::CompressResult{rows + (size_t)i * rb, rb, scales[i], (uint8_t)bits,
                                          (adaptq::StorageSlot)i};
  adaptq::create_scalar_backend()->vaccum_batch(acc, r.data(), w, N, P, bits);
}

void kref_fwht(float *x, const signed char *D, int P, int forward) {
  if (forward) adaptq::create_scalar_backend()->fwht_forward(x, D, P);
  else adaptq::create_scalar_backend()->fwht_inverse(x, D, P);
}

}  // extern "C"
