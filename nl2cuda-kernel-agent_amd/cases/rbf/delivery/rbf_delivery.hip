// Host-pointer RBF entry points (include/rbf_delivery.h): stage the host
// arrays in device memory, run the C-ABI device entry points of
// ../kernels/rbf.hip on the default stream, copy the results back.
#include <cstddef>
#include <cstdint>

#include "../../../csrc/common.h"
#include "rbf.h"
#include "rbf_delivery.h"

namespace {

// Device allocation released on scope exit.
class DeviceArray {
 public:
  DeviceArray() = default;
  DeviceArray(const DeviceArray&) = delete;
  DeviceArray& operator=(const DeviceArray&) = delete;
  ~DeviceArray() {
    if (p_) (void)hipFree(p_);
  }
  int allocate(size_t bytes, const char* what) {
    if (bytes == 0) return NL2K_SUCCESS;
    return nl2k::check_hip(hipMalloc(&p_, bytes), what);
  }
  float* get() const { return static_cast<float*>(p_); }

 private:
  void* p_ = nullptr;
};

int upload(DeviceArray& d, const float* h, size_t count, const char* what) {
  int st = d.allocate(count * sizeof(float), what);
  if (st || count == 0) return st;
  return nl2k::check_hip(hipMemcpy(d.get(), h, count * sizeof(float), hipMemcpyHostToDevice),
                         what);
}

int download(float* h, const DeviceArray& d, size_t count, const char* what) {
  if (count == 0) return NL2K_SUCCESS;
  return nl2k::check_hip(hipMemcpy(h, d.get(), count * sizeof(float), hipMemcpyDeviceToHost),
                         what);
}

int check_sizes(int N, int M, int D, const char* who) {
  if (N < 0 || M < 0 || D < 1)
    return nl2k::fail(NL2K_ERR_SHAPE, "%s: need N >= 0, M >= 0, D >= 1 (got N=%d M=%d D=%d)",
                      who, N, M, D);
  return NL2K_SUCCESS;
}

}  // namespace

extern "C" {

int rbf_forward_hip(const float* X, const float* Y, float* K, int N, int M, int D,
                    float gamma) {
  const char* who = "rbf_forward_hip";
  int st = check_sizes(N, M, D, who);
  if (st) return st;
  if ((N > 0 && !X) || (M > 0 && !Y) || ((size_t)N * M > 0 && !K))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null host pointer", who);
  DeviceArray dX, dY, dK;
  const size_t nx = (size_t)N * D, ny = (size_t)M * D, nk = (size_t)N * M;
  if ((st = upload(dX, X, nx, who)) || (st = upload(dY, Y, ny, who)) ||
      (st = dK.allocate(nk * sizeof(float), who)))
    return st;
  st = rbf_forward_f32(dX.get(), dY.get(), dK.get(), N, M, D, gamma, nullptr);
  if (st) return st;
  if ((st = nl2k::check_hip(hipDeviceSynchronize(), who))) return st;
  if ((st = download(K, dK, nk, who))) return st;
  return nl2k::succeed();
}

int rbf_backward_hip(const float* X, const float* Y, const float* G, const float* K,
                     float* dX, float* dY, int N, int M, int D, float gamma) {
  const char* who = "rbf_backward_hip";
  int st = check_sizes(N, M, D, who);
  if (st) return st;
  const size_t nx = (size_t)N * D, ny = (size_t)M * D, nk = (size_t)N * M;
  if ((nx > 0 && (!X || !dX)) || (ny > 0 && (!Y || !dY)) || (nk > 0 && (!G || !K)))
    return nl2k::fail(NL2K_ERR_NULL, "%s: null host pointer", who);
  DeviceArray gX, gY, gG, gK, gdX, gdY, ws;
  if ((st = upload(gX, X, nx, who)) || (st = upload(gY, Y, ny, who)) ||
      (st = upload(gG, G, nk, who)) || (st = upload(gK, K, nk, who)) ||
      (st = gdX.allocate(nx * sizeof(float), who)) || (st = gdY.allocate(ny * sizeof(float), who)))
    return st;
  const size_t ws_bytes = rbf_backward_workspace_bytes(N, M, D);
  if ((st = ws.allocate(ws_bytes, who))) return st;
  st = rbf_backward_f32(gX.get(), gY.get(), gG.get(), gK.get(), gdX.get(), gdY.get(), N, M, D,
                        gamma, ws.get(), ws_bytes, nullptr);
  if (st) return st;
  if ((st = nl2k::check_hip(hipDeviceSynchronize(), who))) return st;
  if ((st = download(dX, gdX, nx, who)) || (st = download(dY, gdY, ny, who))) return st;
  return nl2k::succeed();
}

}  // extern "C"
