// ref_shim.cpp -- test harness around the reference build (oracle/_ref).
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's own
// hot-path sources, read in place from /root/reference (see oracle/Makefile);
// it includes the reference's headers from there and exposes plain C entry
// points for the pieces below the reference's C ABI (codec functions and the
// ring contents of one AttentionHead), so tests can compare our restatement
// with the reference bit for bit.  Nothing here restates any algorithm.
#include "adaptq.h"
#include "attention.h"
#include "codebook.h"
#include "fwht.h"
#include "quantizer.h"

#include <cstring>
#include <new>

extern "C" {

int refx_next_pow2(int n) { return next_pow2(n); }

void refx_rademacher(int8_t *D, int n, uint64_t seed) { gen_rademacher(D, n, seed); }

void refx_fwht_forward(float *x, const int8_t *D, int d) { fwht_forward(x, D, d); }

void refx_fwht_inverse(float *x, const int8_t *D, int d) { fwht_inverse(x, D, d); }

int refx_quantize_fast(float v, int bits) { return quantize_fast(v, bits); }

void refx_pack(const uint8_t *idx, int d, int bits, uint8_t *dst) {
  pack_indices(idx, d, bits, dst);
}

float refx_quantize_into(int dim, uint64_t seed, int bits, const float *x,
                         uint8_t *packed) {
  Quantizer q;
  q.init(dim, seed);
  return q.quantize_into(x, bits, packed);
}

void *refx_head_create(int dim, int k_bits, int v_bits, int cap, uint64_t seed,
                       float v_mass, int hyb) {
  AttentionHead *h = new (std::nothrow) AttentionHead();
  if (!h) return nullptr;
  h->init(dim, k_bits, v_bits, cap, seed, v_mass, hyb);
  return h;
}

void refx_head_destroy(void *h) { delete static_cast<AttentionHead *>(h); }

void refx_head_append(void *h, const float *k, const float *v, int pos) {
  static_cast<AttentionHead *>(h)->append_kv(k, v, pos);
}

int refx_head_compute(void *h, const float *q, float *out) {
  return static_cast<AttentionHead *>(h)->compute(q, out);
}

void refx_head_reset(void *h) {
  // Same three steps as adaptq_reset (core/adaptq_c_api.cpp:128-137).
  AttentionHead *a = static_cast<AttentionHead *>(h);
  a->kv_buf.size = 0;
  a->kv_buf.head = 0;
  a->raw_kv.clear();
}

void refx_head_info(void *h, int *head, int *size, int *k_pb, int *v_pb,
                    int *raw_floats) {
  AttentionHead *a = static_cast<AttentionHead *>(h);
  *head = a->kv_buf.head;
  *size = a->kv_buf.size;
  *k_pb = a->kv_buf.k_packed_bytes;
  *v_pb = a->kv_buf.v_packed_bytes;
  *raw_floats = (int)a->raw_kv.size();
}

void refx_head_read_slots(void *h, int first, int count, uint8_t *kc,
                          uint8_t *vc, float *ks, float *vs) {
  AttentionHead *a = static_cast<AttentionHead *>(h);
  const KVFlatBuffer &b = a->kv_buf;
  for (int i = 0; i < count; ++i) {
    int s = first + i;
    std::memcpy(kc + (size_t)i * b.k_packed_bytes, b.k_ptr(s), b.k_packed_bytes);
    std::memcpy(vc + (size_t)i * b.v_packed_bytes, b.v_ptr(s), b.v_packed_bytes);
    ks[i] = b.k_scale[s];
    vs[i] = b.v_scale[s];
  }
}

// Timing loops over the reference's own C ABI (include/adaptq.h), so a CPU
// baseline measures the reference's append and compute, not one foreign call
// per token: rows t = 0..n-1 of keys/vals ([n][dim]) at positions t, and one
// query decoded `reps` times.
void refx_append_rows(void *ctx, const float *keys, const float *vals, int n, int dim) {
  for (int t = 0; t < n; ++t)
    adaptq_append(static_cast<adaptq_ctx_t>(ctx), keys + (size_t)t * dim, vals + (size_t)t * dim, t);
}

int refx_compute_reps(void *ctx, const float *q, float *out, int reps) {
  int r = 0;
  for (int i = 0; i < reps; ++i) r = adaptq_compute(static_cast<adaptq_ctx_t>(ctx), q, out);
  return r;
}

}  // extern "C"
