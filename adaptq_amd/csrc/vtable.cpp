// vtable.cpp -- C function-pointer table over any IAdaptQBackend
// (interface of the reference's core/adaptq_backend_vtable.cpp:1-28).
#include "../../include/adaptq_backend.h"

namespace {

IAdaptQBackend *as_backend(void *c) { return static_cast<IAdaptQBackend *>(c); }

void vt_append(void *c, int h, const float *k, const float *v, int p) {
  as_backend(c)->append_kv(h, k, v, p);
}
int vt_compute(void *c, int h, const float *q, float *o) { return as_backend(c)->compute(h, q, o); }
int vt_compute_batch(void *c, int h, const float *qs, int n, float *os) {
  return as_backend(c)->compute_batch(h, qs, n, os);
}
void vt_reset(void *c) { as_backend(c)->reset(); }
size_t vt_kv_bytes(void *c) { return as_backend(c)->kv_bytes(); }
int vt_n_heads(void *c) { return as_backend(c)->n_heads(); }
int vt_head_dim(void *c) { return as_backend(c)->head_dim(); }
void vt_destroy(void *c) { delete as_backend(c); }

}  // namespace

AdaptQBackendVTable adaptq_make_vtable(IAdaptQBackend *backend) {
  AdaptQBackendVTable t;
  t.append_kv = vt_append;
  t.compute = vt_compute;
  t.compute_batch = vt_compute_batch;
  t.reset = vt_reset;
  t.kv_bytes = vt_kv_bytes;
  t.n_heads = vt_n_heads;
  t.head_dim = vt_head_dim;
  t.destroy = vt_destroy;
  t.impl = backend;
  return t;
}
