/*
 * oracle.c -- CPU restatement of AdapTQ's KV-cache hot path (test
 * infrastructure only; see oracle.h).
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off -std=c11 oracle.c -lm
 * (the recipe is oracle/Makefile).  -ffp-contract=off matters: the
 * reference's golden build contracts nothing outside its explicit FMA
 * intrinsics, so every a*b+c below must round twice unless written fmaf().
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *   orc_next_pow2, orc_rademacher   golden vectors from the reference build,
 *                                   xorshift closed form.
 *   orc_fwht_forward/_inverse       golden vectors; brute-force integer
 *                                   Hadamard on small-integer inputs (every
 *                                   stage exact); round trip; linearity.
 *   orc_quantize_fast               golden sweep; brute-force threshold count;
 *                                   the reference's own boundary tests.
 *   orc_pack/orc_unpack             closed-form bit layouts; round trip.
 *   orc_quantize_vec                golden codes+scales (bit-exact) from the
 *                                   reference build over N(0,1), Student-t,
 *                                   outliers, zeros, +-1e38, NaN, 1e-38, -0.
 *   orc_head_* (append/ring)        golden ring dumps (bit-exact); closed-form
 *                                   kv_bytes (README.md:152-158).
 *   orc_head_compute (all branches) golden outputs from the reference build
 *                                   (bit-exact on the dense and K16 paths);
 *                                   float64 brute-force attention over the
 *                                   closed-form dequantised ring.
 *   sparse-V selection              golden outputs; ties between exactly
 *                                   equal probabilities are ordered by slot
 *                                   here, while the reference's std::sort
 *                                   leaves them unspecified.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* A1  core/fwht.cpp:13-19                                             */
int orc_next_pow2(int n) {
  if (n <= 1) return 1;
  if (n > (1 << 30)) return 1 << 30;
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

/* A2  core/fwht.cpp:21-27: xorshift64 (13, 7, 17); odd -> +1, even -> -1;
 * a zero seed is replaced by a fixed non-zero constant. */
void orc_rademacher(int8_t *D, int n, uint64_t seed) {
  uint64_t s = seed ? seed : 0xdeadbeefcafe1234ULL;
  for (int i = 0; i < n; ++i) {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    D[i] = (s & 1u) ? (int8_t)1 : (int8_t)-1;
  }
}

/* Radix-2 butterflies over stride lengths 1, 2, ..., p/2; the lower element
 * of each pair becomes lo+hi and the upper lo-hi (core/fwht.cpp:43-58). */
static void butterflies(float *x, int p, int first_len) {
  for (int len = first_len; len < p; len <<= 1)
    for (int base = 0; base < p; base += 2 * len)
      for (int j = base; j < base + len; ++j) {
        float lo = x[j], hi = x[j + len];
        x[j] = lo + hi;
        x[j + len] = lo - hi;
      }
}

/* A4  core/fwht.cpp:33-66 (fwht_fused, reached through fwht_forward with a
 * power-of-two length): the first stage multiplies both inputs by their
 * signs, the later stages are plain butterflies, and the result is scaled by
 * RN(1 / RN(sqrt(p))). */
void orc_fwht_forward(float *x, const int8_t *D, int p) {
  if (p < 2) {
    if (p == 1) x[0] = x[0] * (float)D[0] * (1.0f / sqrtf(1.0f));
    return;
  }
  for (int i = 0; i < p; i += 2) {
    float a = x[i] * (float)D[i];
    float b = x[i + 1] * (float)D[i + 1];
    x[i] = a + b;
    x[i + 1] = a - b;
  }
  butterflies(x, p, 2);
  float inv = 1.0f / sqrtf((float)p);
  for (int i = 0; i < p; ++i) x[i] *= inv;
}

/* C6  core/fwht.cpp:106-134: all butterfly stages without signs, then
 * x[i] = (x[i] * scale) * D[i] with scale = RN(1 / RN(sqrt(p))). */
void orc_fwht_inverse(float *x, const int8_t *D, int p) {
  butterflies(x, p, 1);
  float scale = 1.0f / sqrtf((float)p);
  for (int i = 0; i < p; ++i) x[i] = x[i] * scale * (float)D[i];
}

/* ------------------------------------------------------------------ */
/* A7  core/codebook.cpp:32-62 -- Lloyd-Max N(0,1) centroids (the symmetric
 * post-#229 CB4).  These literal tables are the format itself. */
static const float CB2[4] = {-1.5104f, -0.4528f, 0.4528f, 1.5104f};
static const float CB3[8] = {-2.1529f, -1.3439f, -0.7560f, -0.2451f,
                             0.2451f,  0.7560f,  1.3439f,  2.1529f};
static const float CB4[16] = {-2.4008f, -1.8944f, -1.5105f, -1.2016f,
                              -0.9138f, -0.6402f, -0.3795f, -0.1258f,
                              0.1258f,  0.3795f,  0.6402f,  0.9138f,
                              1.2016f,  1.5105f,  1.8944f,  2.4008f};

static const float *codebook(int bits) {
  return bits == 2 ? CB2 : bits == 3 ? CB3 : CB4;
}

void orc_codebook(int bits, float *out) {
  const float *cb = codebook(bits);
  for (int i = 0; i < (1 << bits); ++i) out[i] = cb[i];
}

/* Decision thresholds: midpoints (c[k] + c[k+1]) * 0.5f evaluated in float,
 * with the centre threshold exactly 0 (core/codebook.cpp:67-100). */
static float thresholds[3][15];
static int thresholds_ready;

static void init_thresholds(void) {
  if (thresholds_ready) return;
  for (int b = 2; b <= 4; ++b) {
    const float *cb = codebook(b);
    int n = 1 << b;
    for (int k = 0; k < n - 1; ++k)
      thresholds[b - 2][k] = (k == n / 2 - 1) ? 0.0f : (cb[k] + cb[k + 1]) * 0.5f;
  }
  thresholds_ready = 1;
}

/* A6  core/codebook.cpp:119-144: NaN maps to the centroid just below zero
 * (1, 3, 7); otherwise the branchless binary search returns how many
 * thresholds t satisfy v >= t (the thresholds are strictly increasing). */
int orc_quantize_fast(float v, int bits) {
  init_thresholds();
  if (isnan(v)) return bits <= 2 ? 1 : bits == 3 ? 3 : 7;
  int b = bits <= 2 ? 2 : bits >= 4 ? 4 : 3;
  const float *t = thresholds[b - 2];
  int i = 0;
  for (int step = 1 << (b - 1); step >= 1; step >>= 1)
    if (v >= t[i + step - 1]) i += step;
  return i;
}

/* A8  core/quantizer.cpp:156-225: most-significant code first.
 *   4 bits: byte i = idx[2i] << 4 | idx[2i+1]
 *   2 bits: byte i = idx[4i] << 6 | idx[4i+1] << 4 | idx[4i+2] << 2 | idx[4i+3]
 *   3 bits: 8 codes -> one 24-bit big-endian word s0<<21 | ... | s7 */
int orc_packed_bytes(int p, int bits) {
  return bits == 16 ? p * 4 : (p * bits + 7) / 8;
}

void orc_pack(const uint8_t *idx, int p, int bits, uint8_t *dst) {
  if (bits == 4) {
    for (int i = 0; i < p / 2; ++i)
      dst[i] = (uint8_t)((idx[2 * i] << 4) | (idx[2 * i + 1] & 0xF));
  } else if (bits == 2) {
    for (int i = 0; i < p / 4; ++i)
      dst[i] = (uint8_t)((idx[4 * i] << 6) | (idx[4 * i + 1] << 4) |
                         (idx[4 * i + 2] << 2) | idx[4 * i + 3]);
  } else if (bits == 3) {
    for (int g = 0; g < p / 8; ++g) {
      uint32_t w = 0;
      for (int k = 0; k < 8; ++k) w |= (uint32_t)(idx[8 * g + k] & 7) << (21 - 3 * k);
      dst[3 * g] = (uint8_t)(w >> 16);
      dst[3 * g + 1] = (uint8_t)(w >> 8);
      dst[3 * g + 2] = (uint8_t)w;
    }
  }
}

void orc_unpack(const uint8_t *src, int p, int bits, uint8_t *idx) {
  if (bits == 4) {
    for (int i = 0; i < p / 2; ++i) {
      idx[2 * i] = src[i] >> 4;
      idx[2 * i + 1] = src[i] & 0xF;
    }
  } else if (bits == 2) {
    for (int i = 0; i < p / 4; ++i)
      for (int k = 0; k < 4; ++k) idx[4 * i + k] = (src[i] >> (6 - 2 * k)) & 3;
  } else if (bits == 3) {
    for (int g = 0; g < p / 8; ++g) {
      uint32_t w = ((uint32_t)src[3 * g] << 16) | ((uint32_t)src[3 * g + 1] << 8) |
                   (uint32_t)src[3 * g + 2];
      for (int k = 0; k < 8; ++k) idx[8 * g + k] = (w >> (21 - 3 * k)) & 7;
    }
  }
}

/* A5 + A9  core/quantizer.cpp:53-101, :131-137.
 * 1. s = sum_{i<dim} x_i*x_i, accumulated left to right in float;
 *    norm = sqrtf(s + 1e-12f); inv = 1.f / norm; buf = x * inv, zero-padded.
 * 2. forward FWHT with signs D; then buf *= sqrtf(p).
 * 3. sigma = sqrtf(sum(buf^2) / p + 1e-12f) (left to right); clamp to
 *    +-3*sigma with the reference's two compares (NaN passes through).
 * 4. index every coordinate, pack, return norm (the stored scale). */
float orc_quantize_vec(const float *x, int dim, int p, const int8_t *D,
                       int bits, uint8_t *packed, uint8_t *idx_out) {
  float *buf = (float *)malloc(sizeof(float) * (size_t)p);
  uint8_t *idx = (uint8_t *)malloc((size_t)p);
  float norm = 0.0f;
  for (int i = 0; i < dim; ++i) {
    buf[i] = x[i];
    float sq = x[i] * x[i];
    norm = norm + sq;
  }
  for (int i = dim; i < p; ++i) buf[i] = 0.0f;
  norm = sqrtf(norm + 1e-12f);
  float inv = 1.0f / norm;
  for (int i = 0; i < p; ++i) buf[i] *= inv;
  orc_fwht_forward(buf, D, p);
  float sp = sqrtf((float)p);
  for (int i = 0; i < p; ++i) buf[i] *= sp;
  float sum2 = 0.0f;
  for (int i = 0; i < p; ++i) {
    float sq = buf[i] * buf[i];
    sum2 = sum2 + sq;
  }
  float sigma = sqrtf(sum2 / (float)p + 1e-12f);
  float clip = 3.0f * sigma;
  for (int i = 0; i < p; ++i) {
    if (buf[i] > clip) buf[i] = clip;
    if (buf[i] < -clip) buf[i] = -clip;
  }
  for (int i = 0; i < p; ++i) idx[i] = (uint8_t)orc_quantize_fast(buf[i], bits);
  orc_pack(idx, p, bits, packed);
  if (idx_out) memcpy(idx_out, idx, (size_t)p);
  free(idx);
  free(buf);
  return norm;
}

/* ------------------------------------------------------------------ */
/* A10 + A11 + C1..C7: one attention head (attention/attention.cpp:324-677,
 * cache/ring_buffer.cpp:47-119). */
struct orc_head {
  int dim, padded, k_bits, v_bits, cap;
  float v_mass;
  int hyb;
  int8_t *D;
  int k_pb, v_pb;
  uint8_t *k_data, *v_data;
  float *k_scale, *v_scale;
  int *positions;
  int head, size;
  float *raw;      /* hybrid mirror: [raw_count][2*dim], key then value */
  int raw_count;
};

uint64_t orc_mha_seed(uint64_t base, int i) {
  /* core/adaptq_c_api.cpp:160 */
  return base ^ ((uint64_t)i * 0xDEADBEEFCAFEULL);
}

orc_head *orc_head_create(int dim, int k_bits, int v_bits, int cap,
                          uint64_t seed, float v_mass, int hyb) {
  orc_head *h = (orc_head *)calloc(1, sizeof(orc_head));
  h->dim = dim;
  h->padded = orc_next_pow2(dim);
  h->k_bits = k_bits;
  h->v_bits = v_bits;
  h->cap = cap;
  h->v_mass = v_mass;
  h->hyb = hyb;
  h->D = (int8_t *)malloc((size_t)h->padded);
  orc_rademacher(h->D, h->padded, seed);
  h->k_pb = orc_packed_bytes(h->padded, k_bits);
  h->v_pb = orc_packed_bytes(h->padded, v_bits);
  size_t c = cap > 0 ? (size_t)cap : 1;
  h->k_data = (uint8_t *)calloc(c, (size_t)h->k_pb);
  h->v_data = (uint8_t *)calloc(c, (size_t)h->v_pb);
  h->k_scale = (float *)malloc(sizeof(float) * c);
  h->v_scale = (float *)malloc(sizeof(float) * c);
  h->positions = (int *)calloc(c, sizeof(int));
  for (size_t i = 0; i < c; ++i) h->k_scale[i] = h->v_scale[i] = 1.0f;
  h->raw = hyb > 0 ? (float *)malloc(sizeof(float) * (size_t)hyb * 2 * dim) : NULL;
  return h;
}

void orc_head_destroy(orc_head *h) {
  if (!h) return;
  free(h->D);
  free(h->k_data);
  free(h->v_data);
  free(h->k_scale);
  free(h->v_scale);
  free(h->positions);
  free(h->raw);
  free(h);
}

/* Encode one vector into a slot buffer: bits==16 stores raw floats zero
 * padded to p with scale 1 (attention.cpp:341-353). */
static float encode(const orc_head *h, const float *x, int bits, uint8_t *dst) {
  if (bits == 16) {
    memset(dst, 0, (size_t)h->padded * 4);
    memcpy(dst, x, (size_t)h->dim * 4);
    return 1.0f;
  }
  return orc_quantize_vec(x, h->dim, h->padded, h->D, bits, dst, NULL);
}

void orc_head_append(orc_head *h, const float *key, const float *val, int pos) {
  uint8_t *tk = (uint8_t *)malloc((size_t)h->k_pb);
  uint8_t *tv = (uint8_t *)malloc((size_t)h->v_pb);
  float ks = encode(h, key, h->k_bits, tk);
  float vs = encode(h, val, h->v_bits, tv);
  int will_evict = h->size >= h->cap;
  if (h->cap > 0) { /* ring_buffer.cpp:105-119 */
    int s = h->head;
    memcpy(h->k_data + (size_t)s * h->k_pb, tk, (size_t)h->k_pb);
    memcpy(h->v_data + (size_t)s * h->v_pb, tv, (size_t)h->v_pb);
    h->k_scale[s] = ks;
    h->v_scale[s] = vs;
    h->positions[s] = pos;
    h->head = (h->head + 1) % h->cap;
    if (h->size < h->cap) ++h->size;
  }
  /* attention.cpp:356-365: mirror raw vectors until the threshold; forget
   * the mirror for good at the first eviction. */
  if (h->hyb > 0) {
    if (!will_evict && h->raw_count < h->hyb) {
      memcpy(h->raw + (size_t)h->raw_count * 2 * h->dim, key, (size_t)h->dim * 4);
      memcpy(h->raw + (size_t)h->raw_count * 2 * h->dim + h->dim, val, (size_t)h->dim * 4);
      ++h->raw_count;
    } else if (will_evict && h->raw_count > 0) {
      h->raw_count = 0;
    }
  }
  free(tk);
  free(tv);
}

void orc_head_reset(orc_head *h) {
  /* core/adaptq_c_api.cpp:128-137 */
  h->size = 0;
  h->head = 0;
  h->raw_count = 0;
}

size_t orc_head_kv_bytes(const orc_head *h) {
  return (size_t)h->size * (size_t)(h->k_pb + h->v_pb);
}

void orc_head_info(const orc_head *h, int *head, int *size, int *cap,
                   int *padded, int *k_pb, int *v_pb, int *raw_count) {
  if (head) *head = h->head;
  if (size) *size = h->size;
  if (cap) *cap = h->cap;
  if (padded) *padded = h->padded;
  if (k_pb) *k_pb = h->k_pb;
  if (v_pb) *v_pb = h->v_pb;
  if (raw_count) *raw_count = h->raw_count;
}

void orc_head_read_slots(const orc_head *h, int first, int count,
                         uint8_t *kc, uint8_t *vc, float *ks, float *vs) {
  for (int i = 0; i < count; ++i) {
    int s = first + i;
    if (kc) memcpy(kc + (size_t)i * h->k_pb, h->k_data + (size_t)s * h->k_pb, (size_t)h->k_pb);
    if (vc) memcpy(vc + (size_t)i * h->v_pb, h->v_data + (size_t)s * h->v_pb, (size_t)h->v_pb);
    if (ks) ks[i] = h->k_scale[s];
    if (vs) vs[i] = h->v_scale[s];
  }
}

const int8_t *orc_head_signs(const orc_head *h) { return h->D; }

/* Unpack one ring row into code indices. */
static void row_codes(const uint8_t *row, int p, int bits, uint8_t *idx) {
  orc_unpack(row, p, bits, idx);
}

/* C2 logits, attention.cpp:93-136 + :83-88: lane L of an 8-wide vector
 * accumulates codes L, L+8, L+16, ... with one FMA each, and the lanes are
 * combined as ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7)). */
static float kdot(const float *qr, const uint8_t *idx, const float *cb, int p) {
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < p; j += 8)
    for (int L = 0; L < 8 && j + L < p; ++L) s[L] = fmaf(cb[idx[j + L]], qr[j + L], s[L]);
  float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];
  return (t0 + t1) + (t2 + t3);
}

typedef struct {
  float p;
  int i;
} pidx;

static int cmp_desc(const void *a, const void *b) {
  const pidx *x = (const pidx *)a, *y = (const pidx *)b;
  if (x->p > y->p) return -1;
  if (x->p < y->p) return 1;
  return x->i - y->i;
}

/* acc[j] = fma(CB[code_j], w, acc[j]) for one ring row (vaccum1/vaccum4). */
static void vaccum(float *acc, const uint8_t *row, const float *cb, float w,
                   int p, int bits, uint8_t *idx) {
  row_codes(row, p, bits, idx);
  for (int j = 0; j < p; ++j) acc[j] = fmaf(cb[idx[j]], w, acc[j]);
}

int orc_head_compute(const orc_head *h, const float *q, float *out) {
  return orc_head_compute_sel(h, q, out, NULL);
}

/* orc_head_compute, and on the sparse-V branch the selection: sel_w[t] (t in
 * ring order, oldest first) = the weight (p_t * vscale_t) * isp the token's V
 * row is accumulated with, 0 for tokens left out.  sel_w is untouched on the
 * other branches. */
int orc_head_compute_sel(const orc_head *h, const float *q, float *out, float *sel_w) {
  const int n = h->size, cap = h->cap, dim = h->dim, p = h->padded;
  if (!n) {
    memset(out, 0, sizeof(float) * (size_t)dim);
    return 0;
  }
  float *logits = (float *)malloc(sizeof(float) * (size_t)n);

  /* C4 hybrid branch, attention.cpp:491-523 */
  if (h->hyb > 0 && n <= h->hyb && h->raw_count == n) {
    const float scale = 1.0f / sqrtf((float)dim);
    float mx = -1e30f;
    for (int i = 0; i < n; ++i) {
      const float *k = h->raw + (size_t)i * 2 * dim;
      float d = 0.0f;
      for (int j = 0; j < dim; ++j) {
        float pr = q[j] * k[j];
        d = d + pr;
      }
      logits[i] = d * scale;
      if (logits[i] > mx) mx = logits[i];
    }
    float sv = 0.0f;
    for (int i = 0; i < n; ++i) {
      logits[i] = expf(logits[i] - mx);
      sv += logits[i];
    }
    float inv = (sv > 0.0f && isfinite(sv)) ? (1.0f / sv) : (1.0f / (float)n);
    memset(out, 0, sizeof(float) * (size_t)dim);
    for (int i = 0; i < n; ++i) {
      float w = logits[i] * inv;
      const float *v = h->raw + (size_t)i * 2 * dim + dim;
      for (int j = 0; j < dim; ++j) {
        float pr = w * v[j];
        out[j] = out[j] + pr;
      }
    }
    free(logits);
    return n;
  }

  float *qr = (float *)calloc((size_t)p, sizeof(float));
  float *acc = (float *)calloc((size_t)p, sizeof(float));
  int *slots = (int *)malloc(sizeof(int) * (size_t)n);
  uint8_t *idx = (uint8_t *)malloc((size_t)p);
  memcpy(qr, q, sizeof(float) * (size_t)dim);
  float attn_s = 1.0f / sqrtf((float)dim);
  float isp = 1.0f / sqrtf((float)p);
  /* Query rotation, attention.cpp:528-550 */
  if (h->k_bits != 16) {
    float qn = 0.0f;
    for (int i = 0; i < dim; ++i) {
      float sq = q[i] * q[i];
      qn = qn + sq;
    }
    qn = sqrtf(qn + 1e-12f);
    float inv = 1.0f / qn;
    for (int i = 0; i < p; ++i) qr[i] *= inv;
    orc_fwht_forward(qr, h->D, p);
    float sp = sqrtf((float)p);
    float m = sp * qn;
    for (int i = 0; i < p; ++i) qr[i] *= m;
    attn_s = 1.0f / (sqrtf((float)dim) * (float)p);
  }
  /* Oldest to newest, attention.cpp:562-563 */
  for (int i = 0; i < n; ++i) slots[i] = (h->head - n + cap + i) % cap;

  if (h->k_bits == 16) {
    /* C3, attention.cpp:565-600: unrotated fp32 dot over dim; softmax
     * without the finite guard; fp32 V or LUT V plus inverse FWHT. */
    float mx = -1e30f;
    for (int i = 0; i < n; ++i) {
      const float *k = (const float *)(h->k_data + (size_t)slots[i] * h->k_pb);
      float d = 0.0f;
      for (int j = 0; j < dim; ++j) {
        float pr = qr[j] * k[j];
        d = d + pr;
      }
      logits[i] = d * attn_s;
      if (logits[i] > mx) mx = logits[i];
    }
    float sv = 0.0f;
    for (int i = 0; i < n; ++i) {
      logits[i] = expf(logits[i] - mx);
      sv += logits[i];
    }
    float inv = 1.0f / sv;
    for (int i = 0; i < n; ++i) logits[i] *= inv;
    const float *vcb = codebook(h->v_bits);
    for (int i = 0; i < n; ++i) {
      int s = slots[i];
      if (h->v_bits == 16) {
        const float *v = (const float *)(h->v_data + (size_t)s * h->v_pb);
        float w = logits[i];
        for (int j = 0; j < dim; ++j) {
          float pr = w * v[j];
          acc[j] = acc[j] + pr;
        }
      } else {
        float ew = logits[i] * h->v_scale[s] * isp;
        float ecb[16];
        for (int c = 0; c < (1 << h->v_bits); ++c) ecb[c] = ew * vcb[c];
        row_codes(h->v_data + (size_t)s * h->v_pb, p, h->v_bits, idx);
        for (int j = 0; j < p; ++j) acc[j] = acc[j] + ecb[idx[j]];
      }
    }
    if (h->v_bits != 16) orc_fwht_inverse(acc, h->D, p);
    memcpy(out, acc, sizeof(float) * (size_t)dim);
    goto done;
  }

  {
    /* C2, attention.cpp:373-474 (AVX2 branch, dispatched at :606-633). */
    const float *kcb = codebook(h->k_bits);
    float mx = -1e30f;
    for (int i = 0; i < n; ++i) {
      int s = slots[i];
      row_codes(h->k_data + (size_t)s * h->k_pb, p, h->k_bits, idx);
      float d = kdot(qr, idx, kcb, p);
      logits[i] = d * attn_s * h->k_scale[s];
      if (logits[i] > mx) mx = logits[i];
    }
    float sv = 0.0f;
    for (int j = 0; j < n; ++j) {
      logits[j] = expf(logits[j] - mx);
      sv += logits[j];
    }
    float inv = 1.0f / sv;
    for (int j = 0; j < n; ++j) logits[j] *= inv;

    if (h->v_bits == 16) {
      /* The reference dereferences a null codebook here (attention.cpp:553,
       * :648-655); this restates the evident intent: fp32 V, no inverse
       * FWHT. */
      for (int i = 0; i < n; ++i) {
        const float *v = (const float *)(h->v_data + (size_t)slots[i] * h->v_pb);
        for (int j = 0; j < dim; ++j) {
          float pr = logits[i] * v[j];
          acc[j] = acc[j] + pr;
        }
      }
      memcpy(out, acc, sizeof(float) * (size_t)dim);
      goto done;
    }

    const float *vcb = codebook(h->v_bits);
    if (h->v_mass <= 0.0f) {
      for (int i = 0; i < n; ++i) {
        int s = slots[i];
        vaccum(acc, h->v_data + (size_t)s * h->v_pb, vcb,
               logits[i] * h->v_scale[s] * isp, p, h->v_bits, idx);
      }
    } else {
      /* attention.cpp:448-473 (with :469 read as the V-codebook call it
       * evidently means): descending probability order, whole quads while
       * the running mass is below v_mass, then single tokens. */
      pidx *ord = (pidx *)malloc(sizeof(pidx) * (size_t)n);
      for (int i = 0; i < n; ++i) {
        ord[i].p = logits[i];
        ord[i].i = i;
      }
      qsort(ord, (size_t)n, sizeof(pidx), cmp_desc);
      if (sel_w) memset(sel_w, 0, sizeof(float) * (size_t)n);
      float mass = 0.0f;
      int ii = 0;
      for (; ii + 3 < n && mass < h->v_mass; ii += 4) {
        for (int k = 0; k < 4; ++k) {
          int t = ord[ii + k].i, s = slots[t];
          float w = logits[t] * h->v_scale[s] * isp;
          if (sel_w) sel_w[t] = w;
          vaccum(acc, h->v_data + (size_t)s * h->v_pb, vcb, w, p, h->v_bits, idx);
        }
        float q4 = ((logits[ord[ii].i] + logits[ord[ii + 1].i]) + logits[ord[ii + 2].i]) +
                   logits[ord[ii + 3].i];
        mass += q4;
      }
      for (; ii < n && mass < h->v_mass; ++ii) {
        int t = ord[ii].i, s = slots[t];
        float w = logits[t];
        float ws = w * h->v_scale[s] * isp;
        if (sel_w) sel_w[t] = ws;
        vaccum(acc, h->v_data + (size_t)s * h->v_pb, vcb, ws, p, h->v_bits, idx);
        mass += w;
      }
      free(ord);
    }
    orc_fwht_inverse(acc, h->D, p);
    memcpy(out, acc, sizeof(float) * (size_t)dim);
  }

done:
  free(qr);
  free(acc);
  free(slots);
  free(idx);
  free(logits);
  return n;
}

/* C7, attention.cpp:662-677 */
int orc_head_compute_batch(const orc_head *h, const float *qs, int nq, float *outs) {
  if (h->size == 0) {
    memset(outs, 0, sizeof(float) * (size_t)nq * (size_t)h->dim);
    return 0;
  }
  for (int i = 0; i < nq; ++i)
    orc_head_compute(h, qs + (size_t)i * h->dim, outs + (size_t)i * h->dim);
  return h->size;
}
