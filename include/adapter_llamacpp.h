/*
 * adapter_llamacpp.h -- llama.cpp adapter over the MI355X build.
 *
 * Same class as the reference's adapters/adapter_llamacpp.h:11-38 and .cpp:27-63
 * (LlamaCppAdaptQAdapter: constructor, feed_kv, attention, attention_batch,
 * reset, kv_bytes, log_memory), so llama.cpp code written against the
 * reference builds unchanged.  Header-only; no ggml types cross it, only
 * float pointers and byte strides.  The reference's constructor passes one
 * `bits` argument to the 8-argument AdaptQMHABackend constructor
 * (adapter_llamacpp.cpp:33-37, which does not compile); here `bits` is used
 * for K and V, its evident intent, and with_bits() takes them separately.
 *
 * Additions for a GPU-resident llama.cpp: whole-layer calls (every head in
 * one launch) and the forward functions of the ggml operator nodes
 * (GGML_OP_ADAPTQ_APPEND / GGML_OP_ADAPTQ_ATTN) in host and device forms.
 */
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "adaptq.h"
#include "adaptq_mha_backend.h"

class LlamaCppAdaptQAdapter {
 public:
  LlamaCppAdaptQAdapter(int n_heads, int head_dim, int bits, int capacity, uint64_t seed = 0,
                        float v_mass = 0.95f, int hybrid_thresh = 512)
      : backend_(n_heads, head_dim, bits, bits, capacity, seed, v_mass, hybrid_thresh) {}

  /* Separate K and V bit widths (2, 3, 4 or 16). */
  static LlamaCppAdaptQAdapter with_bits(int n_heads, int head_dim, int k_bits, int v_bits,
                                         int capacity, uint64_t seed = 0, float v_mass = 0.95f,
                                         int hybrid_thresh = 512) {
    return LlamaCppAdaptQAdapter(n_heads, head_dim, k_bits, v_bits, capacity, seed, v_mass,
                                 hybrid_thresh);
  }

  LlamaCppAdaptQAdapter(const LlamaCppAdaptQAdapter &) = delete;
  LlamaCppAdaptQAdapter &operator=(const LlamaCppAdaptQAdapter &) = delete;

  /* False when creation failed; adaptq_last_error() says why. */
  bool ok() const { return backend_.ok(); }
  adaptq_mha_t handle() const { return backend_.handle(); }

  /* Call once per incoming token, once per head, after graph compute. */
  void feed_kv(int head, const float *key, const float *val, int token_pos) {
    backend_.append_kv(head, key, val, token_pos);
  }

  /* Single-query attention forward (decode step). */
  int attention(int head, const float *query, float *out) {
    return backend_.compute(head, query, out);
  }

  /* Multi-query batch attention (prefill step). */
  int attention_batch(int head, const float *queries, int n_queries, float *outs) {
    return backend_.compute_batch(head, queries, n_queries, outs);
  }

  /* Clear all cached KV (e.g. on context reset). */
  void reset() { backend_.reset(); }

  /* Compressed bytes in the KV cache. */
  size_t kv_bytes() const { return backend_.kv_bytes(); }

  /* Logs "KV: X MB vs FP16: Y MB" to stderr (reference message format). */
  void log_memory(int capacity) const {
    const double used_mb = (double)backend_.kv_bytes() / 1e6;
    const double fp16_mb =
        (double)backend_.n_heads() * capacity * backend_.head_dim() * 2 * 2 / 1e6;
    std::fprintf(stderr,
                 "[AdapTQ/llama.cpp] KV: %.2f MB  (FP16 would be %.2f MB, "
                 "%.1fx smaller)\n",
                 used_mb, fp16_mb, fp16_mb / (used_mb + 1e-9));
  }

  /* ---- additions ---- */

  /* One token for every head: keys, vals [n_heads][head_dim] host. */
  int feed_kv_all(const float *keys, const float *vals, int token_pos) {
    return adaptq_mha_append_all(handle(), keys, vals, token_pos);
  }

  /* Attention for every head: queries, outs [n_heads][head_dim] host. */
  int attention_all(const float *queries, float *outs) {
    return adaptq_mha_compute_all(handle(), queries, outs);
  }

  /* ggml operator forwards on f32 tensors [head_dim, n_heads, n] with byte
   * strides nb1, nb2 (ggml_tensor::nb[1], nb[2]).  Host data: */
  int ggml_append(const float *k, size_t k_nb1, size_t k_nb2, const float *v, size_t v_nb1,
                  size_t v_nb2, int n_tokens, int first_pos) {
    return adaptq_ggml_append_f32(handle(), k, v, backend_.head_dim(), backend_.n_heads(),
                                  n_tokens, k_nb1, k_nb2, v_nb1, v_nb2, first_pos);
  }
  int ggml_attn(const float *q, size_t q_nb1, size_t q_nb2, int n_queries, float *dst,
                size_t dst_nb1, size_t dst_nb2) {
    return adaptq_ggml_attn_f32(handle(), q, backend_.head_dim(), backend_.n_heads(), n_queries,
                                q_nb1, q_nb2, dst, dst_nb1, dst_nb2);
  }

  /* Device data (a ggml HIP backend), asynchronous on `stream` (hipStream_t). */
  int ggml_append_device(const float *d_k, size_t k_nb1, size_t k_nb2, const float *d_v,
                         size_t v_nb1, size_t v_nb2, int n_tokens, int first_pos, void *stream) {
    return adaptq_ggml_append_f32_device(handle(), d_k, d_v, backend_.head_dim(),
                                         backend_.n_heads(), n_tokens, k_nb1, k_nb2, v_nb1,
                                         v_nb2, first_pos, stream);
  }
  int ggml_attn_device(const float *d_q, size_t q_nb1, size_t q_nb2, int n_queries, float *d_dst,
                       size_t dst_nb1, size_t dst_nb2, void *stream) {
    return adaptq_ggml_attn_f32_device(handle(), d_q, backend_.head_dim(), backend_.n_heads(),
                                       n_queries, q_nb1, q_nb2, d_dst, dst_nb1, dst_nb2, stream);
  }

 private:
  LlamaCppAdaptQAdapter(int n_heads, int head_dim, int k_bits, int v_bits, int capacity,
                        uint64_t seed, float v_mass, int hybrid_thresh)
      : backend_(n_heads, head_dim, k_bits, v_bits, capacity, seed, v_mass, hybrid_thresh) {}

  AdaptQMHABackend backend_;
};
