/*
 * oracle.h -- CPU restatement of AdapTQ's KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (adaptq_amd/, include/)
 * may include, link or call this; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker.
 *
 * Every function restates one reference function (cited file:line under
 * /root/reference) in plain C, built with -ffp-contract=off so each float
 * operation rounds exactly where the reference's does.  The attention path
 * follows the reference's AVX2 branch (the one taken on x86 hosts with
 * AVX2+FMA), whose per-lane FMA chains are reproduced with fmaf().
 *
 * Parity status per function (how each is pinned) is listed in oracle.c.
 */
#ifndef ADAPTQ_ORACLE_H
#define ADAPTQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int   orc_next_pow2(int n);
void  orc_rademacher(int8_t *D, int n, uint64_t seed);
void  orc_fwht_forward(float *x, const int8_t *D, int p);
void  orc_fwht_inverse(float *x, const int8_t *D, int p);
int   orc_quantize_fast(float v, int bits);
void  orc_codebook(int bits, float *out);  /* 2^bits centroids */
void  orc_pack(const uint8_t *idx, int p, int bits, uint8_t *dst);
void  orc_unpack(const uint8_t *src, int p, int bits, uint8_t *idx);
int   orc_packed_bytes(int p, int bits);
/* Full codec for one vector: returns the stored scale (||x||), writes packed
 * codes (orc_packed_bytes(p, bits) bytes) and, if idx != NULL, the indices. */
float orc_quantize_vec(const float *x, int dim, int p, const int8_t *D,
                       int bits, uint8_t *packed, uint8_t *idx);

typedef struct orc_head orc_head;

orc_head *orc_head_create(int dim, int k_bits, int v_bits, int capacity,
                          uint64_t seed, float v_mass, int hybrid_thresh);
void   orc_head_destroy(orc_head *h);
void   orc_head_append(orc_head *h, const float *key, const float *val,
                       int pos);
int    orc_head_compute(const orc_head *h, const float *q, float *out);
/* The same, and on the sparse-V branch each token's selection weight in ring
 * order (0 = left out) into sel_w[n]. */
int    orc_head_compute_sel(const orc_head *h, const float *q, float *out,
                            float *sel_w);
int    orc_head_compute_batch(const orc_head *h, const float *qs, int nq,
                              float *outs);
void   orc_head_reset(orc_head *h);
size_t orc_head_kv_bytes(const orc_head *h);
/* Ring introspection: head, size, capacity, padded dim, packed bytes. */
void   orc_head_info(const orc_head *h, int *head, int *size, int *cap,
                     int *padded, int *k_pb, int *v_pb, int *raw_count);
/* Copy `count` physical slots starting at `first` out of the ring. */
void   orc_head_read_slots(const orc_head *h, int first, int count,
                           uint8_t *k_codes, uint8_t *v_codes,
                           float *k_scale, float *v_scale);
const int8_t *orc_head_signs(const orc_head *h);

/* Per-head seed used by the multi-head API. */
uint64_t orc_mha_seed(uint64_t base, int head_idx);

#ifdef __cplusplus
}
#endif
#endif
