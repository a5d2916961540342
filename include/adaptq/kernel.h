/*
 * adaptq/kernel.h -- kernel-backend interface, with a gfx950 HIP backend.
 *
 * IKernelBackend is the reference's include/adaptq/kernel.h:24-93 interface
 * (same class, same virtual functions in the same order, same argument
 * meaning), the seam its V2 RuntimeContext takes its compute primitives from
 * (runtime/runtime_context.cpp:142 calls select_kernel_backend()).  This
 * library's backend runs them on the GPU:
 *
 *   fwht_forward / fwht_inverse   the codec's transforms on x[padded], in
 *                                 place, bit-exact with the reference's
 *                                 core/fwht.cpp (same stage structure and
 *                                 scale roundings)
 *   kdot_batch                    logits[i] = (q_rot . CB[codes_i]) * scale_i
 *                                 / padded, as kernels/scalar/kdot_scalar.cpp
 *   vaccum_batch                  acc = sum_i weights[i] * scale_i * CB[codes_i]
 *                                 (acc zeroed first, zero weights skipped)
 *
 * Arguments are host memory, as in the interface: each call packs the rows
 * the CompressResults point to into pinned staging, runs on the backend's
 * stream and returns when the outputs are back.  bits is 2, 3 or 4 (the
 * reference's backends read packed codes only).  Calls are serialised by a
 * lock; HIP failures throw std::runtime_error.
 */
#pragma once

#include <cstdint>

#include "storage.h"

namespace adaptq {

class IKernelBackend {
 public:
  virtual ~IKernelBackend() = default;
  virtual void fwht_forward(float *x, const int8_t *D, int padded) = 0;
  virtual void fwht_inverse(float *x, const int8_t *D, int padded) = 0;
  virtual void kdot_batch(const float *q_rot, const CompressResult *k_results, int N,
                          int padded, int bits, float *logits_out) = 0;
  virtual void vaccum_batch(float *acc, const CompressResult *v_results, const float *weights,
                            int N, int padded, int bits) = 0;
  virtual bool is_available() const = 0;
  virtual const char *name() const = 0;
};

/* The gfx950 HIP backend (process-global; do not delete).  Creating it
 * touches no GPU; the first call does. */
IKernelBackend *create_hip_backend();

/* The reference's selector (kernel.h:80-86) returns the best CPU backend;
 * this library has one backend, the HIP one, and no CPU fallback. */
IKernelBackend *select_kernel_backend();

} /* namespace adaptq */
