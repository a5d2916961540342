/*
 * adaptq_mha_backend.h -- IAdaptQBackend over an adaptq_mha_t.
 *
 * Same class as the reference's include/adaptq_mha_backend.h:11-48
 * (AdaptQMHABackend, constructor argument order, forwarding to the
 * adaptq_mha_* functions), so its callers build unchanged.
 */
#pragma once

#include <cstdint>

#include "adaptq.h"
#include "adaptq_backend.h"

class AdaptQMHABackend final : public IAdaptQBackend {
 public:
  AdaptQMHABackend(int n_h, int h_dim, int k_bits, int v_bits, int capacity, uint64_t seed,
                   float v_mass, int hybrid_thresh)
      : mha_(adaptq_mha_create(n_h, h_dim, k_bits, v_bits, capacity, seed, v_mass,
                               hybrid_thresh)),
        n_heads_(n_h),
        head_dim_(h_dim) {}
  ~AdaptQMHABackend() override { adaptq_mha_destroy(mha_); }
  AdaptQMHABackend(const AdaptQMHABackend &) = delete;
  AdaptQMHABackend &operator=(const AdaptQMHABackend &) = delete;

  /* False when creation failed; adaptq_last_error() says why. */
  bool ok() const { return mha_ != nullptr; }
  adaptq_mha_t handle() const { return mha_; }

  void append_kv(int head, const float *k, const float *v, int pos) override {
    adaptq_mha_append(mha_, head, k, v, pos);
  }
  int compute(int head, const float *q, float *out) override {
    return adaptq_mha_compute(mha_, head, q, out);
  }
  int compute_batch(int head, const float *qs, int n, float *outs) override {
    return adaptq_mha_compute_batch(mha_, head, qs, n, outs);
  }
  void reset() override { adaptq_mha_reset(mha_); }
  size_t kv_bytes() const override { return adaptq_mha_total_kv_bytes(mha_); }
  int n_heads() const override { return n_heads_; }
  int head_dim() const override { return head_dim_; }

 private:
  adaptq_mha_t mha_ = nullptr;
  int n_heads_ = 0;
  int head_dim_ = 0;
};
