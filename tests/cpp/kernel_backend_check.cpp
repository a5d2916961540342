// Drives adaptq::select_kernel_backend() (include/adaptq/kernel.h) through the
// IKernelBackend interface, as the reference's V2 runtime would.
//   kernel_backend_check IN OUT
// IN holds cases written by tests/test_gpu_kernel_backend.py: per case
//   i32 bits, i32 padded, i32 N, f32 q[padded], u8 rows[N][row bytes],
//   f32 scales[N], f32 weights[N], i8 D[padded], f32 x[padded]
// OUT gets per case: f32 logits[N], f32 acc[padded], f32 fwd[padded], f32 inv[padded]
// (fwd = fwht_forward(x), inv = fwht_inverse(x)).  Prints the backend name.
#include <cstdio>
#include <cstring>
#include <vector>

#include "adaptq/kernel.h"

static int row_bytes(int padded, int bits) { return (padded * bits + 7) / 8; }

template <class T>
static bool rd(FILE *f, T *p, size_t n) {
  return std::fread(p, sizeof(T), n, f) == n;
}

int main(int argc, char **argv) {
  if (argc != 3) return 2;
  adaptq::IKernelBackend *kb = adaptq::select_kernel_backend();
  if (!kb->is_available()) {
    std::printf("backend %s not available\n", kb->name());
    return 1;
  }
  std::printf("backend %s\n", kb->name());
  FILE *in = std::fopen(argv[1], "rb");
  FILE *out = std::fopen(argv[2], "wb");
  if (!in || !out) return 2;
  int hdr[3];
  int cases = 0;
  while (rd(in, hdr, 3)) {
    const int bits = hdr[0], P = hdr[1], N = hdr[2], rb = row_bytes(P, bits);
    std::vector<float> q(P), scales(N), w(N), x(P), logits(N), acc(P);
    std::vector<uint8_t> rows((size_t)N * rb);
    std::vector<int8_t> D(P);
    if (!rd(in, q.data(), P) || !rd(in, rows.data(), rows.size()) || !rd(in, scales.data(), N) ||
        !rd(in, w.data(), N) || !rd(in, D.data(), P) || !rd(in, x.data(), P))
      return 3;
    std::vector<adaptq::CompressResult> res(N);
    for (int i = 0; i < N; ++i)
      res[i] = adaptq::CompressResult{rows.data() + (size_t)i * rb, rb, scales[i],
                                      (uint8_t)bits, (adaptq::StorageSlot)i};
    kb->kdot_batch(q.data(), res.data(), N, P, bits, logits.data());
    for (auto &a : acc) a = 12345.0f;  // vaccum_batch zeroes acc itself
    kb->vaccum_batch(acc.data(), res.data(), w.data(), N, P, bits);
    std::vector<float> fwd = x, inv = x;
    kb->fwht_forward(fwd.data(), D.data(), P);
    kb->fwht_inverse(inv.data(), D.data(), P);
    std::fwrite(logits.data(), 4, N, out);
    std::fwrite(acc.data(), 4, P, out);
    std::fwrite(fwd.data(), 4, P, out);
    std::fwrite(inv.data(), 4, P, out);
    ++cases;
  }
  std::fclose(in);
  std::fclose(out);
  std::printf("cases %d\n", cases);
  return 0;
}
