// Drives LlamaCppAdaptQAdapter (include/adapter_llamacpp.h) the way llama.cpp
// would: per-head feed_kv/attention against a second adapter fed through the
// ggml operator forms with padded strides.  Prints OK and exits 0 when every
// output agrees within 1e-4 (relative, norm-wise) and kv_bytes match.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "adapter_llamacpp.h"

static float rnd(unsigned &s) {  // deterministic, about N(0,1)-ish
  float a = 0.f;
  for (int i = 0; i < 4; ++i) {
    s = s * 1664525u + 1013904223u;
    a += (float)(s >> 8) / 16777216.0f - 0.5f;
  }
  return a * 1.7f;
}

static double rel(const float *a, const float *b, int n) {
  double d = 0, r = 0;
  for (int i = 0; i < n; ++i) {
    d += (double)(a[i] - b[i]) * (a[i] - b[i]);
    r += (double)b[i] * b[i];
  }
  return std::sqrt(d / (r + 1e-30));
}

int main() {
  const int H = 4, D = 64, T = 300, CAP = 512, NQ = 2;
  LlamaCppAdaptQAdapter a(H, D, 4, CAP, 7, 0.0f, 0);
  LlamaCppAdaptQAdapter b = LlamaCppAdaptQAdapter::with_bits(H, D, 4, 4, CAP, 7, 0.0f, 0);
  if (!a.ok() || !b.ok()) {
    std::printf("create failed: %s\n", adaptq_last_error());
    return 1;
  }
  // ggml layout: row (head h, token t) at byte h*nb1 + t*nb2, with padding
  const size_t nb1 = (D + 8) * 4, nb2 = nb1 * H + 64;
  std::vector<float> kb(nb2 / 4 * T), vb(nb2 / 4 * T);
  unsigned s = 12345;
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h)
      for (int d = 0; d < D; ++d) {
        kb[(t * nb2 + h * nb1) / 4 + d] = rnd(s);
        vb[(t * nb2 + h * nb1) / 4 + d] = rnd(s);
      }
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h)
      a.feed_kv(h, &kb[(t * nb2 + h * nb1) / 4], &vb[(t * nb2 + h * nb1) / 4], t);
  if (b.ggml_append(kb.data(), nb1, nb2, vb.data(), nb1, nb2, T, 0) != 0) {
    std::printf("ggml_append failed: %s\n", adaptq_last_error());
    return 1;
  }
  std::vector<float> q((size_t)NQ * H * D);
  for (auto &x : q) x = rnd(s);
  // q contiguous [NQ][H][D] -> nb1 = D*4, nb2 = H*D*4; dst padded
  const size_t dn1 = (D + 4) * 4, dn2 = dn1 * H + 32;
  std::vector<float> dst(dn2 / 4 * NQ, 123.0f);
  const int n = b.ggml_attn(q.data(), D * 4, (size_t)H * D * 4, NQ, dst.data(), dn1, dn2);
  if (n != T) {
    std::printf("ggml_attn returned %d: %s\n", n, adaptq_last_error());
    return 1;
  }
  double worst = 0;
  for (int h = 0; h < H; ++h) {
    std::vector<float> qs((size_t)NQ * D), outs((size_t)NQ * D), one(D);
    for (int j = 0; j < NQ; ++j) std::memcpy(&qs[j * D], &q[((size_t)j * H + h) * D], D * 4);
    if (a.attention_batch(h, qs.data(), NQ, outs.data()) != T) return 1;
    if (a.attention(h, qs.data(), one.data()) != T) return 1;
    worst = std::fmax(worst, rel(one.data(), outs.data(), D));
    for (int j = 0; j < NQ; ++j)
      worst = std::fmax(worst, rel(&dst[(j * dn2 + h * dn1) / 4], &outs[j * D], D));
  }
  // padding of dst untouched
  for (size_t i = 0; i < dst.size(); ++i) {
    const size_t byte = i * 4, j = byte / dn2, rem = byte % dn2, h = rem / dn1, d = (rem % dn1) / 4;
    const bool pad = h >= (size_t)H || d >= (size_t)D || j >= (size_t)NQ;
    if (pad && dst[i] != 123.0f) {
      std::printf("padding overwritten at %zu\n", i);
      return 1;
    }
  }
  if (a.kv_bytes() != b.kv_bytes()) return 1;
  a.log_memory(CAP);
  std::printf("max rel err %.3g\n", worst);
  if (!(worst <= 1e-4)) return 1;
  std::printf("OK\n");
  return 0;
}
