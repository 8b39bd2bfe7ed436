// Self-test of librbf.a: random X, Y, G; the GPU results of rbf_forward_hip /
// rbf_backward_hip against a float64 CPU evaluation of the definitions
//   K[i,j]  = exp(-gamma |x_i - y_j|^2)
//   dX[i,:] = -2 gamma sum_j G[i,j] K[i,j] (x_i - y_j)
//   dY[j,:] = -2 gamma sum_i G[i,j] K[i,j] (y_j - x_i)
// at atol = rtol = 1e-3.  Usage: rbf_test [N M D [gamma]]  (default
// 128 128 64, gamma = 1/64).  Exit status 0 when every check passes.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "rbf_delivery.h"

namespace {

// Deterministic uniform(-1, 1) stream (64-bit LCG, top 24 bits).
struct Uniform {
  uint64_t s;
  explicit Uniform(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  float next() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return (float)((double)(s >> 40) / (double)(1ull << 24) * 2.0 - 1.0);
  }
};

struct Ref {
  std::vector<double> K, dX, dY;
};

Ref reference(const std::vector<float>& X, const std::vector<float>& Y, const std::vector<float>& G,
              int N, int M, int D, double gamma) {
  Ref r;
  r.K.assign((size_t)N * M, 0.0);
  r.dX.assign((size_t)N * D, 0.0);
  r.dY.assign((size_t)M * D, 0.0);
  for (int i = 0; i < N; ++i)
    for (int j = 0; j < M; ++j) {
      double s = 0.0;
      for (int d = 0; d < D; ++d) {
        const double t = (double)X[(size_t)i * D + d] - (double)Y[(size_t)j * D + d];
        s += t * t;
      }
      const double k = std::exp(-gamma * s);
      r.K[(size_t)i * M + j] = k;
      const double w = -2.0 * gamma * (double)G[(size_t)i * M + j] * k;
      for (int d = 0; d < D; ++d) {
        const double t = (double)X[(size_t)i * D + d] - (double)Y[(size_t)j * D + d];
        r.dX[(size_t)i * D + d] += w * t;
        r.dY[(size_t)j * D + d] -= w * t;
      }
    }
  return r;
}

bool close(const char* name, const std::vector<float>& got, const std::vector<double>& want) {
  double max_abs = 0.0, max_rel = 0.0;
  bool ok = true;
  for (size_t i = 0; i < got.size(); ++i) {
    const double e = std::fabs((double)got[i] - want[i]);
    max_abs = e > max_abs ? e : max_abs;
    const double rel = e / (std::fabs(want[i]) > 1e-30 ? std::fabs(want[i]) : 1e-30);
    max_rel = rel > max_rel ? rel : max_rel;
    if (!(e <= 1e-3 + 1e-3 * std::fabs(want[i]))) ok = false;
  }
  std::printf("[%-3s] %s  max_abs_err=%.3e  max_rel_err=%.3e\n", name, ok ? "PASS" : "FAIL",
              max_abs, max_rel);
  return ok;
}

}  // namespace

int main(int argc, char** argv) {
  int N = 128, M = 128, D = 64;
  float gamma = 1.0f / 64.0f;
  if (argc >= 4) {
    N = std::atoi(argv[1]);
    M = std::atoi(argv[2]);
    D = std::atoi(argv[3]);
  }
  if (argc >= 5) gamma = (float)std::atof(argv[4]);
  if (N < 1 || M < 1 || D < 1) {
    std::fprintf(stderr, "usage: %s [N M D [gamma]] with N, M, D >= 1\n", argv[0]);
    return 2;
  }
  Uniform u(1234);
  std::vector<float> X((size_t)N * D), Y((size_t)M * D), G((size_t)N * M);
  for (auto& v : X) v = u.next();
  for (auto& v : Y) v = u.next();
  for (auto& v : G) v = u.next();

  std::vector<float> K((size_t)N * M), dX((size_t)N * D), dY((size_t)M * D);
  std::printf("=== librbf.a self-test  N=%d M=%d D=%d gamma=%.6g ===\n", N, M, D, gamma);
  if (rbf_forward_hip(X.data(), Y.data(), K.data(), N, M, D, gamma) != NL2K_SUCCESS) {
    std::printf("rbf_forward_hip failed: %s\n", rbf_last_error());
    return 1;
  }
  if (rbf_backward_hip(X.data(), Y.data(), G.data(), K.data(), dX.data(), dY.data(), N, M, D,
                       gamma) != NL2K_SUCCESS) {
    std::printf("rbf_backward_hip failed: %s\n", rbf_last_error());
    return 1;
  }
  const Ref r = reference(X, Y, G, N, M, D, gamma);
  const bool ok = close("K", K, r.K) & close("dX", dX, r.dX) & close("dY", dY, r.dY);
  // Argument checks are reported, not fatal.
  const bool rejects = rbf_forward_hip(X.data(), Y.data(), K.data(), -1, M, D, gamma) ==
                       NL2K_ERR_SHAPE;
  std::printf("[arg] %s  negative N rejected\n", rejects ? "PASS" : "FAIL");
  std::printf("=== overall: %s (atol = rtol = 1e-3) ===\n", ok && rejects ? "PASS" : "FAIL");
  return ok && rejects ? 0 : 1;
}
