// CPU mirror of the streaming routing kernel's one-pass algorithm (test
// infrastructure, like the rest of oracle/; nothing in the library links it).
//
// The row-per-wave kernel (stream_body in kotodama_amd/csrc/attnres_kernels.hip)
// visits a token's sources once, in order, and keeps an online depth softmax:
//   first source / new maximum:  c = exp(m - logit), l = l*c + 1, m = logit,
//                                acc = acc*c + x
//   otherwise:                   p = exp(logit - m), l = l + p, acc = acc + p*x
//   out = acc * (1/l),  lse = m + log(l)
// with logit = (x . qw) * rsqrt(mean(x^2) + eps) (llama.py:640-641).  This file
// restates that recurrence in fp32 so tests can check it against the float64
// two-pass softmax of attnres_oracle.route (llama.py:642-644) on the CPU, under
// AddressSanitizer and UndefinedBehaviorSanitizer, and on adversarial orders
// of the logits (rising, falling, equal, -inf free) that exercise both branches.
//
// I/O (little-endian binary, paths on the command line):
//   in : int32 S, N, D; float32 eps; float32 src[S][N][D]; float32 qw[D]
//   out: float32 out[N][D]; float32 lse[N]
// S == 0 writes NaN everywhere (softmax over an empty set).

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <vector>

namespace {

bool read_all(FILE* f, void* p, size_t bytes) { return std::fread(p, 1, bytes, f) == bytes; }

void route_online(int S, int N, int D, float eps, const std::vector<float>& src, const std::vector<float>& qw,
                  std::vector<float>& out, std::vector<float>& lse) {
  const float nan = std::numeric_limits<float>::quiet_NaN();
  std::vector<float> acc(D);
  for (int t = 0; t < N; ++t) {
    float* o = &out[(size_t)t * D];
    if (S == 0) {
      for (int e = 0; e < D; ++e) o[e] = nan;
      lse[t] = nan;
      continue;
    }
    float m = -std::numeric_limits<float>::infinity(), l = 0.f;
    for (int e = 0; e < D; ++e) acc[e] = 0.f;
    for (int s = 0; s < S; ++s) {
      const float* x = &src[((size_t)s * N + t) * D];
      // two accumulation chains per quantity, even and odd elements, as the kernel's fp32 path
      float ss0 = 0.f, ss1 = 0.f, dt0 = 0.f, dt1 = 0.f;
      for (int e = 0; e < D; ++e) {
        if (e & 1) {
          ss1 = std::fma(x[e], x[e], ss1);
          dt1 = std::fma(x[e], qw[e], dt1);
        } else {
          ss0 = std::fma(x[e], x[e], ss0);
          dt0 = std::fma(x[e], qw[e], dt0);
        }
      }
      const float inv = 1.0f / std::sqrt((ss0 + ss1) * (1.0f / (float)D) + eps);
      const float logit = (dt0 + dt1) * inv;
      if (logit > m) {
        const float c = std::exp(m - logit);  // exp(-inf) = 0 at the first source
        l = std::fma(l, c, 1.f);
        m = logit;
        for (int e = 0; e < D; ++e) acc[e] = std::fma(acc[e], c, x[e]);
      } else {
        const float p = std::exp(logit - m);
        l += p;
        for (int e = 0; e < D; ++e) acc[e] = std::fma(x[e], p, acc[e]);
      }
    }
    const float rl = 1.0f / l;
    for (int e = 0; e < D; ++e) o[e] = acc[e] * rl;
    lse[t] = m + std::log(l);
  }
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: %s <in.bin> <out.bin>\n", argv[0]);
    return 2;
  }
  FILE* fi = std::fopen(argv[1], "rb");
  if (!fi) return 3;
  int32_t hdr[3];
  float eps = 0.f;
  if (!read_all(fi, hdr, sizeof(hdr)) || !read_all(fi, &eps, sizeof(eps))) return 4;
  const int S = hdr[0], N = hdr[1], D = hdr[2];
  if (S < 0 || N <= 0 || D <= 0 || S > 64) return 5;
  std::vector<float> src((size_t)S * N * D), qw(D);
  if (!read_all(fi, src.data(), src.size() * sizeof(float)) || !read_all(fi, qw.data(), qw.size() * sizeof(float)))
    return 6;
  std::fclose(fi);
  std::vector<float> out((size_t)N * D), lse(N);
  route_online(S, N, D, eps, src, qw, out, lse);
  FILE* fo = std::fopen(argv[2], "wb");
  if (!fo) return 7;
  const bool ok = std::fwrite(out.data(), sizeof(float), out.size(), fo) == out.size() &&
                  std::fwrite(lse.data(), sizeof(float), lse.size(), fo) == lse.size();
  std::fclose(fo);
  return ok ? 0 : 8;
}
