// Exposes the reference's own CPU restatement of the RBF math -- the static
// functions cpu_forward / cpu_backward of cases/rbf/delivery/rbf_test.cu:24-52
// -- as C symbols, by compiling that file in place (its path comes from
// -DRBF_TEST_CU; nothing is copied).  Its main() is renamed into an unnamed
// namespace so it is dropped, together with its calls to the CUDA host
// functions, which this build does not need.  Test infrastructure only.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {
#define main rbf_test_main_unused
#include RBF_TEST_CU
#undef main
}  // namespace

extern "C" void ref_rbf_cpu_forward(const float* X, const float* Y, float* K,
                                    int N, int M, int D, float gamma) {
  std::vector<float> x(X, X + (size_t)N * D), y(Y, Y + (size_t)M * D);
  std::vector<float> k((size_t)N * M);
  cpu_forward(x, y, k, N, M, D, gamma);
  std::copy(k.begin(), k.end(), K);
}

extern "C" void ref_rbf_cpu_backward(const float* X, const float* Y,
                                     const float* G, const float* K, float* dX,
                                     float* dY, int N, int M, int D,
                                     float gamma) {
  std::vector<float> x(X, X + (size_t)N * D), y(Y, Y + (size_t)M * D);
  std::vector<float> g(G, G + (size_t)N * M), k(K, K + (size_t)N * M);
  std::vector<float> dx((size_t)N * D), dy((size_t)M * D);
  cpu_backward(x, y, g, k, dx, dy, N, M, D, gamma);
  std::copy(dx.begin(), dx.end(), dX);
  std::copy(dy.begin(), dy.end(), dY);
}
