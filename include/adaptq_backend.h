/*
 * adaptq_backend.h -- C++ backend interface over the C ABI.
 *
 * Same interface as the reference's include/adaptq_backend.h:13-83 (class and
 * method names, argument meaning, the C function-pointer table), so framework
 * adapters written against the reference (its pybind11 and llama.cpp
 * adapters) compile unchanged against this build.  All buffers are host
 * float* arrays; no tensor types.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
/* Abstract KV-cache attention backend over n_heads heads. */
struct IAdaptQBackend {
  virtual ~IAdaptQBackend() = default;
  /* Append one token's key and value (head_dim floats each) to head_idx. */
  virtual void append_kv(int head_idx, const float *key, const float *val, int token_pos) = 0;
  /* Attention for one query; returns the number of cached tokens used. */
  virtual int compute(int head_idx, const float *query, float *out) = 0;
  /* Attention for num_queries queries against the same cache. */
  virtual int compute_batch(int head_idx, const float *queries, int num_queries,
                            float *outs) = 0;
  /* Empty every head, keep the configuration. */
  virtual void reset() = 0;
  /* Bytes of packed K/V codes held (scales not counted). */
  virtual size_t kv_bytes() const = 0;
  virtual int n_heads() const = 0;
  virtual int head_dim() const = 0;
};
#endif

/* Function-pointer table for pure-C callers (reference adaptq_backend.h:64-74). */
typedef struct AdaptQBackendVTable {
  void (*append_kv)(void *ctx, int head, const float *k, const float *v, int pos);
  int (*compute)(void *ctx, int head, const float *q, float *out);
  int (*compute_batch)(void *ctx, int head, const float *qs, int n, float *outs);
  void (*reset)(void *ctx);
  size_t (*kv_bytes)(void *ctx);
  int (*n_heads)(void *ctx);
  int (*head_dim)(void *ctx);
  void (*destroy)(void *ctx);
  void *impl; /* the IAdaptQBackend, passed back as ctx */
} AdaptQBackendVTable;

#ifdef __cplusplus
/* Wrap a backend into a C table; the table does not own `backend` until
 * destroy is called through it (reference adaptq_backend_vtable.cpp:25-28). */
AdaptQBackendVTable adaptq_make_vtable(IAdaptQBackend *backend);
#endif
