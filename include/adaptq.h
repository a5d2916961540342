/*
 * adaptq.h -- C ABI of the MI355X (gfx950 HIP) AdapTQ KV-cache hot path.
 *
 * Part 1 is a drop-in for the reference's include/adaptq.h:17-126: the same
 * 17 symbols with the same signatures, argument meaning, return codes and
 * error strings.  Behind them, the ring buffer lives in device HBM, appends
 * are quantised by a HIP kernel and attention is computed by HIP kernels.
 *
 * Part 2 lists extensions that have no counterpart in the reference; each
 * says which callers it is for.
 *
 * Threading: each handle is independent (reference adaptq.h:12).  Calls on
 * one handle are serialised by a per-handle lock.  The last-error string is
 * thread-local.  No function throws.
 */
#pragma once
#ifdef __cplusplus
extern "C" {
#endif

#include <stddef.h>
#include <stdint.h>

/* ---- Error codes (reference include/adaptq.h:17-23) ---- */
typedef enum {
  ADAPTQ_OK = 0,
  ADAPTQ_ERR_ALLOC = 1,         /* host or device allocation failed        */
  ADAPTQ_ERR_INVALID_ARG = 2,   /* NULL handle, out-of-range bits/dim      */
  ADAPTQ_ERR_OUT_OF_BOUNDS = 3, /* head_idx >= n_heads                     */
  ADAPTQ_ERR_UNSUPPORTED = 4    /* requested mode not available            */
} adaptq_error_t;

/* Message of the last error on this thread, "" if none
 * (reference include/adaptq.h:30, core/adaptq_c_api.cpp:15-21). */
const char *adaptq_last_error(void);

typedef void *adaptq_ctx_t; /* one head: ring buffer + codec state */
typedef void *adaptq_mha_t; /* n_heads contexts                     */

/* ================= Part 1: the reference's C ABI ================= */

/* Replaces reference adaptq_create (core/adaptq_c_api.cpp:63-74).
 * dim > 0 with next_pow2(dim) <= 1024; k_bits, v_bits in {2,3,4,16}
 * (16 = fp32 passthrough); capacity >= 0; hybrid_thresh >= 0.  The context
 * lives on the HIP device current at the call.  Returns NULL and sets the
 * last error on invalid arguments or failed allocation. */
adaptq_ctx_t adaptq_create(int dim, int k_bits, int v_bits, int capacity,
                           uint64_t seed, float v_mass, int hybrid_thresh);

/* Replaces reference adaptq_destroy (c_api.cpp:76-80).  NULL is a no-op. */
void adaptq_destroy(adaptq_ctx_t ctx);

/* Replaces reference adaptq_append (c_api.cpp:82-94).  Copies key and val
 * (dim floats each) before returning; quantisation runs on the device when
 * the staged tokens are flushed (by compute, kv_bytes, reset, adaptq_flush or
 * a full staging area).  token_pos is accepted and unused, as in the
 * reference. */
void adaptq_append(adaptq_ctx_t ctx, const float *key, const float *val,
                   int token_pos);

/* Replaces reference adaptq_compute (c_api.cpp:96-107).  Synchronous: out
 * (dim floats, host memory) is filled on return.  Returns the number of
 * cached tokens, 0 when empty (out zeroed), -1 on error. */
int adaptq_compute(adaptq_ctx_t ctx, const float *query, float *out);

/* Replaces reference adaptq_compute_batch (c_api.cpp:109-126): num_queries
 * queries against the same cache in one launch.  Returns the number of
 * cached tokens, 0 when empty (outs zeroed), -1 on error; num_queries == 0
 * accepts NULL buffers. */
int adaptq_compute_batch(adaptq_ctx_t ctx, const float *queries,
                         int num_queries, float *outs);

/* Replaces reference adaptq_reset (c_api.cpp:128-137): empties the ring and
 * the hybrid mirror, keeps the configuration, clears the last error. */
void adaptq_reset(adaptq_ctx_t ctx);

/* Replaces reference adaptq_kv_bytes (c_api.cpp:139-143):
 * size * (k_packed_bytes + v_packed_bytes); scales are not counted. */
size_t adaptq_kv_bytes(adaptq_ctx_t ctx);

/* Replaces reference adaptq_mha_create (c_api.cpp:149-165).  Head i uses
 * seed base_seed ^ (i * 0xDEADBEEFCAFE).  Unlike the reference, a head that
 * fails to allocate fails the whole call (NULL + last error). */
adaptq_mha_t adaptq_mha_create(int n_heads, int dim, int k_bits, int v_bits,
                               int capacity, uint64_t base_seed, float v_mass,
                               int hybrid_thresh);

/* Replaces reference adaptq_mha_destroy (c_api.cpp:167-175). */
void adaptq_mha_destroy(adaptq_mha_t mha);

/* Replaces reference adaptq_mha_append (c_api.cpp:177-195). */
void adaptq_mha_append(adaptq_mha_t mha, int head_idx, const float *key,
                       const float *val, int token_pos);

/* Replaces reference adaptq_mha_compute (c_api.cpp:197-215). */
int adaptq_mha_compute(adaptq_mha_t mha, int head_idx, const float *query,
                       float *out);

/* Replaces reference adaptq_mha_compute_batch (c_api.cpp:217-241). */
int adaptq_mha_compute_batch(adaptq_mha_t mha, int head_idx,
                             const float *queries, int num_queries,
                             float *outs);

/* Replaces reference adaptq_mha_reset (c_api.cpp:243-250). */
void adaptq_mha_reset(adaptq_mha_t mha);

/* Replaces reference adaptq_mha_total_kv_bytes (c_api.cpp:252-261). */
size_t adaptq_mha_total_kv_bytes(adaptq_mha_t mha);

/* ---- Feature flags (reference include/adaptq.h:118-120) ---- */
#define ADAPTQ_FEAT_AVX2 (1u << 0)     /* never set by this build          */
#define ADAPTQ_FEAT_HYBRID (1u << 1)
#define ADAPTQ_FEAT_SPARSE_V (1u << 2)
#define ADAPTQ_FEAT_HIP (1u << 3)      /* extension: HIP device path       */

/* Replaces reference adaptq_features (c_api.cpp:267-273). */
unsigned int adaptq_features(void);

/* Replaces reference adaptq_version (c_api.cpp:275-281), e.g.
 * "3.2.0-hip-gfx950". */
const char *adaptq_version(void);

/* ================= Part 2: extensions ================= */

/* Extension, no counterpart in the reference.  For callers that need the
 * device state settled (timing, snapshots): quantises every staged token of
 * ctx now.  Returns 0, or -1 with the last error set. */
int adaptq_flush(adaptq_ctx_t ctx);

/* Extension, no counterpart in the reference.  For parity checks and ring
 * snapshots: reports the ring geometry and state. Any pointer may be NULL. */
int adaptq_ring_info(adaptq_ctx_t ctx, int *head, int *size, int *capacity,
                     int *padded_dim, int *k_packed_bytes,
                     int *v_packed_bytes);

/* Extension, no counterpart in the reference.  For parity checks and ring
 * snapshots: copies `count` physical slots starting at first_slot to host
 * memory, codes in the reference's byte layout (k_packed_bytes per slot),
 * scales as stored.  Any output pointer may be NULL. Returns 0 or -1. */
int adaptq_read_slots(adaptq_ctx_t ctx, int first_slot, int count,
                      uint8_t *k_codes, uint8_t *v_codes, float *k_scale,
                      float *v_scale);

/* Extension, no counterpart in the reference.  For parity checks of the
 * sparse-V selection (attention.cpp:448-473): decodes `query` like
 * adaptq_compute and writes, for each cached token in ring order (oldest
 * first), the weight (p_t * vscale_t) / sqrt(padded) its V row is summed
 * with, 0 for tokens outside the selection.  weights: host [ring size].
 * Returns the ring size (0 when empty), -1 when the context does not take
 * the sparse-V branch or on error. */
int adaptq_sparse_weights(adaptq_ctx_t ctx, const float *query, float *weights);

/* Extension, no counterpart in the reference.  For callers that batch over
 * heads: the context of head head_idx of an MHA (NULL if out of range). */
adaptq_ctx_t adaptq_mha_head(adaptq_mha_t mha, int head_idx);

/* ---- Whole-MHA batches ----
 * Extension, no counterpart in the reference.  For callers that step all
 * heads of an MHA together (the Python Engine, framework adapters): one call
 * instead of one per head (reference adaptq/core.py:45-74 loops over heads),
 * one append launch and one decode launch for all heads. */

/* Append one token to every head: keys, vals host [n_heads][dim].
 * Returns 0, or -1 with the last error set. */
int adaptq_mha_append_all(adaptq_mha_t mha, const float *keys, const float *vals,
                          int token_pos);

/* Attention for every head: queries host [n_heads][dim] -> outs host
 * [n_heads][dim], synchronous.  Same results as adaptq_mha_compute per head
 * (every branch: dense, hybrid, sparse-V).  Returns the number of cached
 * tokens (of head 0), 0 when empty (outs zeroed), -1 on error. */
int adaptq_mha_compute_all(adaptq_mha_t mha, const float *queries, float *outs);

/* Device-pointer forms for torch-ROCm callers, asynchronous on `stream`
 * (a hipStream_t; NULL = the HIP null stream).  append: d_keys, d_vals
 * [n_heads][n_tokens][dim].  compute: d_queries, d_outs [n_heads][dim];
 * returns the ring size, or -1 (also when the heads differ in ring size or
 * branch, e.g. after per-head appends: use adaptq_mha_compute_all then).
 * Host inspection calls (read_slots, ring_info) see device-path appends once
 * the caller's stream has been synchronised. */
int adaptq_mha_append_all_device(adaptq_mha_t mha, const float *d_keys,
                                 const float *d_vals, int n_tokens,
                                 int first_pos, void *stream);
int adaptq_mha_compute_all_device(adaptq_mha_t mha, const float *d_queries,
                                  float *d_outs, void *stream);

/* Extension, no counterpart in the reference.  One decode step for every
 * head: append one token (d_keys, d_vals: device [n_heads][dim]) as
 * adaptq_mha_append_all_device with one token, then attention as
 * adaptq_mha_compute_all_device (d_queries -> d_outs, device [n_heads][dim]),
 * asynchronous on `stream`.  Same ring bytes and outputs as those two calls
 * (attention.cpp:338-366 then :480-660); where the step is a dense decode at
 * padded 64 with quantised K and V and one block per head, the append runs
 * inside the decode launch (one launch instead of two).  Returns the ring
 * size after the append, or -1 (the token is appended when only the decode
 * fails, e.g. heads that differ in ring size or branch). */
int adaptq_mha_append_compute_all_device(adaptq_mha_t mha, const float *d_keys,
                                         const float *d_vals, int token_pos,
                                         const float *d_queries, float *d_outs,
                                         void *stream);

/* ---- ggml operator forms ----
 * Replace the forward functions of the reference's ggml integration
 * (integration/ggml_operator_patch.md:6-117: GGML_OP_ADAPTQ_APPEND and
 * GGML_OP_ADAPTQ_ATTN nodes carrying an adaptq_mha_t in op_params), with
 * ggml's tensor layout: f32 tensors [head_dim, n_heads, n] with byte strides
 * nb1 (between heads) and nb2 (between tokens or queries), multiples of 4.
 * The reference's CPU forward passes q + h*head_dim as if a head's queries
 * were contiguous, which holds only for n_queries == 1; these honour nb2.
 *
 * append: tokens t = 0..n_tokens-1 of k and v go to every head at position
 * first_pos + t.  attn: every query attends over its head's whole current
 * cache (the reference's compute_batch semantics; no causal mask), dst gets
 * the outputs in q's layout.  Returns 0 (append) or the number of cached
 * tokens (attn), -1 on error.  The host forms are synchronous; the _device
 * forms take device pointers and run asynchronously on `stream` (a
 * hipStream_t, for a ggml HIP backend), sharing the MHA's scratch memory:
 * calls on one MHA from different streams must be ordered by the caller. */
int adaptq_ggml_append_f32(adaptq_mha_t mha, const float *k, const float *v,
                           int head_dim, int n_heads, int n_tokens,
                           size_t k_nb1, size_t k_nb2, size_t v_nb1,
                           size_t v_nb2, int first_pos);
int adaptq_ggml_attn_f32(adaptq_mha_t mha, const float *q, int head_dim,
                         int n_heads, int n_queries, size_t q_nb1,
                         size_t q_nb2, float *dst, size_t dst_nb1,
                         size_t dst_nb2);
int adaptq_ggml_append_f32_device(adaptq_mha_t mha, const float *d_k,
                                  const float *d_v, int head_dim, int n_heads,
                                  int n_tokens, size_t k_nb1, size_t k_nb2,
                                  size_t v_nb1, size_t v_nb2, int first_pos,
                                  void *stream);
int adaptq_ggml_attn_f32_device(adaptq_mha_t mha, const float *d_q,
                                int head_dim, int n_heads, int n_queries,
                                size_t q_nb1, size_t q_nb2, float *d_dst,
                                size_t dst_nb1, size_t dst_nb2, void *stream);

/* ---- Packed-ring snapshots (AQSS v2) ----
 * Replace reference replay/session_snapshot.{h,cpp} (SessionSnapshot
 * capture/save/load, session_snapshot.h:16-40 for the format) for the rings
 * of this library: layers[l] is the MHA of layer l; all share n_heads, dim
 * and bit widths.  Each head block holds its cache_size cached tokens in
 * logical order (oldest first): K rows then V rows in the reference's packed
 * byte layout, each zero-padded to slot_bytes = max(K row, V row) bytes, the
 * scales (K then V) and one format tag per slot (0x02/0x03/0x04 for 2/3/4-bit
 * codes, 0xFF for fp32 rows).  `bits` in the header is the K bit width and
 * n_tokens the largest cache_size; no token log and no strategy state are
 * written (flags 0), and both are skipped on load.
 *
 * load: validates the whole file against the MHAs first (magic, version <= 2,
 * layer/head counts, dim, slot bytes, cache sizes <= capacity, format tags),
 * then replaces every head's ring: tokens in slots 0..n-1, staged appends
 * discarded, hybrid mirror empty (a loaded ring decodes from its packed
 * codes).  Device-form appends must be synchronised by the caller first.
 * Both return 0, or -1 with the last error set (nothing changed on a failed
 * load). */
int adaptq_snapshot_save(const adaptq_mha_t *layers, int n_layers, const char *path);
int adaptq_snapshot_load(const adaptq_mha_t *layers, int n_layers, const char *path);

/* ---- Batched device-pointer path ----
 * Extension, no counterpart in the reference.  For callers whose data is
 * already in device memory (torch-ROCm tensors, serving loops) and for the
 * "all engines in one launch" decode: a plan binds n_ctx distinct contexts
 * that share dim, k_bits, v_bits, capacity, v_mass and hybrid_thresh
 * (NULL with a message otherwise). */
typedef void *adaptq_plan_t;

adaptq_plan_t adaptq_plan_create(const adaptq_ctx_t *ctxs, int n_ctx);
void adaptq_plan_destroy(adaptq_plan_t plan);

/* Append n_tokens tokens to every context of the plan in one launch.
 * d_keys, d_vals: device memory, layout [n_ctx][n_tokens][dim] fp32.
 * Asynchronous on `stream` (a hipStream_t; NULL = the HIP null stream).
 * Staged host appends of those contexts are flushed first. Returns 0/-1. */
int adaptq_plan_append_device(adaptq_plan_t plan, const float *d_keys,
                              const float *d_vals, int n_tokens,
                              int first_pos, void *stream);

/* One decode step for every context of the plan in one launch.
 * d_queries [n_ctx][dim] -> d_outs [n_ctx][dim], device memory, async on
 * `stream`.  Same results as adaptq_compute per context; contexts with an
 * empty ring get zeros.  Every non-empty context must take the same branch
 * (dense, sparse-V or hybrid; attention.cpp:480-660), which then runs as one
 * batched launch sequence.  Returns 0/-1 (-1 with a message when the
 * branches differ). */
int adaptq_plan_compute_device(adaptq_plan_t plan, const float *d_queries,
                               float *d_outs, void *stream);

/* Extension, no counterpart in the reference.  For callers that cannot
 * allocate memory during a call (tight serving loops, harnesses that forbid
 * hipMalloc): adaptq_plan_compute_device with its workspace in a static
 * device array of the library (8 MiB per GPU, held until the process ends)
 * instead of memory the plan allocates.  The call makes no hipMalloc/hipFree
 * or other allocation.  Same results as adaptq_plan_compute_device.  Returns
 * -1 with a message when the decode needs more than 8 MiB of workspace
 * (adaptq_plan_workspace_bytes tells), when a context holds staged host
 * appends (flush them first), or on a stream under HIP graph capture (not
 * supported).  Every call on a GPU shares that GPU's array; calls from
 * different streams or threads are ordered on the device, each call's work
 * waiting for the previous call's (an event per GPU), so they never overlap
 * on the GPU and give the same results as the allocating form. */
int adaptq_plan_compute_device_static(adaptq_plan_t plan, const float *d_queries,
                                      float *d_outs, void *stream);

/* Extension, no counterpart in the reference.  The bytes of device workspace
 * the plan's next decode needs in its current state (0 when it needs none or
 * when its contexts take different branches): what
 * adaptq_plan_compute_device allocates and adaptq_plan_compute_device_static
 * takes from its 8 MiB array.  Dense plans need none when each context's ring
 * fits one block per item (about 512 contexts or more at padded 64/128), else
 * (padded + 4) * 4 bytes per context and split; sparse-V plans need about
 * 4 + 4 * padded / 256 bytes per token of the longest ring per context up to
 * 8,192 tokens, and about 22 + 4 * padded / 256 bytes per token above.
 * Returns -1 on error (a null handle, or a context with staged host
 * appends). */
long long adaptq_plan_workspace_bytes(adaptq_plan_t plan);

#ifdef __cplusplus
}
#endif
