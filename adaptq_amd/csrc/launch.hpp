// launch.hpp -- host-side launchers of the gfx950 kernels (append.hip,
// decode.hip).  All are asynchronous on the given stream and return the HIP
// launch status.
#pragma once

#include "device.hpp"

namespace aq {

// Quantise and insert n_tok tokens into each of n_ctx heads.
// keys, vals: device [n_ctx][n_tok][dim] fp32.  All heads share padded,
// k_bits, v_bits and dim.  Advances every head's device ring state.
// mirror: whether any head may copy tokens to its hybrid mirror in this call
// (from the host's view of the ring states); it only picks between launch
// shapes, the result is the same either way.
hipError_t launch_append(HeadDesc *const *d_descs, int n_ctx, int dim, int padded,
                         int k_bits, int v_bits, const float *keys, const float *vals,
                         int n_tok, hipStream_t stream, bool mirror);

// Zero a head's device ring state (reset).
hipError_t launch_reset_state(HeadDesc *const *d_descs, int n_ctx, hipStream_t stream);

// The token a decode step appends before it decodes (launch_decode_step):
// key and value rows [n_items][dim] fp32 (device or pinned host memory) and
// the codec's two scalings 1/sqrt(padded), sqrt(padded) as floats.
struct StepAppend {
  const float *k, *v;
  float inv_sqrt_p, sqrt_p;
};

struct DecodeShape {
  int dim, padded, k_bits, v_bits;
  bool raw;   // hybrid branch: exact fp32 attention over the raw mirror
  int max_n;  // largest ring size among the items (host view)
};

// Floats of workspace the decode of n_items items needs.
size_t decode_workspace_floats(int n_items, const DecodeShape &shape);

// One decode per item: item i attends with query d_queries[i*dim..] over the
// ring of d_item_desc[i] and writes d_outs[i*dim..].  Dense softmax over all
// cached tokens (the v_mass <= 0 branch); items with an empty ring get zeros.
hipError_t launch_decode(HeadDesc *const *d_item_desc, int n_items, const DecodeShape &shape,
                         const float *d_queries, float *d_outs, float *d_workspace,
                         hipStream_t stream);

// One decode step in one launch where the shape allows it: append the token
// app.k/app.v[i] to item i's ring (as launch_append with one token), then
// decode as launch_decode.  shape.max_n is the largest ring size after the
// append.  Returns hipErrorNotSupported, having launched nothing, unless the
// shape takes the LUT kernel with quantised K and V at padded 64, one block
// per item, no hybrid branch; the caller then appends and decodes with two
// launches.  Items must name distinct contexts of capacity > 0.
hipError_t launch_decode_step(HeadDesc *const *d_item_desc, int n_items, const DecodeShape &shape,
                              const StepAppend &app, const float *d_queries, float *d_outs,
                              hipStream_t stream);
// Whether launch_decode_step takes n_items items of this shape.
bool decode_step_supported(int n_items, const DecodeShape &shape);

// Merge of split partials (m, l, acc[padded]) per item, laid out
// [item][split][padded + 4], into outputs [item][dim]: log-sum-exp weights,
// normalisation, inverse FWHT and signs when V is quantised.
hipError_t launch_finalize(HeadDesc *const *descs, int n_items, int padded, int n_splits,
                           const float *partials, float *outs, bool inverse_fwht, hipStream_t s);

// Decode of many queries per head: items [n_items] = n_items / n_heads
// queries of each of the n_heads heads, item j * n_heads + h being query j of
// head d_item_desc[h] (the first n_heads items name the heads); queries and
// outputs [n_items][dim] in item order.  Same results as launch_decode on
// the same items: with enough queries per head on shapes the MFMA kernel
// covers (dense branch, quantised K and V, padded 64/128) every K/V tile is
// read once for all the queries of its head (mquery.hip); otherwise
// launch_decode runs.
size_t decode_multi_workspace_floats(int n_items, int n_heads, const DecodeShape &shape);
hipError_t launch_decode_multi(HeadDesc *const *d_item_desc, int n_items, int n_heads,
                               const DecodeShape &shape, const float *d_queries, float *d_outs,
                               float *d_workspace, hipStream_t stream);

// Sparse-V decode (v_mass > 0 on quantised K and V), restating
// attention.cpp:448-473.  d_workspace must hold sparse_workspace_floats().
size_t sparse_workspace_floats(int n_items, const DecodeShape &shape);
hipError_t launch_decode_sparse(HeadDesc *const *d_item_desc, int n_items,
                                const DecodeShape &shape, float v_mass,
                                const float *d_queries, float *d_outs, float *d_workspace,
                                hipStream_t stream);

// Strided rows <-> contiguous rows (layout.hip): contiguous row r = a * B + b
// of dim floats is the row at byte offset a * sa + b * sb of the strided side.
hipError_t launch_gather_rows(float *d_dst, const void *d_src, int A, int B, int dim, size_t sa,
                              size_t sb, hipStream_t stream);
hipError_t launch_scatter_rows(void *d_dst, const float *d_src, int A, int B, int dim, size_t sa,
                               size_t sb, hipStream_t stream);

}  // namespace aq
