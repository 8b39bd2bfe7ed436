// LayerNorm over the last dimension, fp32, for MI355X (gfx950).  C-ABI in
// include/layernorm.h.
//
// Reference semantics: cases/layernorm/reference.py:14-21 (two-pass mean and
// biased variance, eps inside the square root), backward by autograd; the
// reference kernels return (y, mean, inv_std) from forward and
// (dx, dgamma, dbeta) from backward (layernorm_forward.cu:302-379,
// layernorm_backward.cu:176-219).
//
// Design: the row-normalisation kernels of csrc/rownorm.h (row-cached
// two-pass statistics in registers, prefetching backward with per-block
// dw / dbias partials summed deterministically, generic kernels for other
// shapes) with the centered, biased policy below.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "../../../csrc/common.h"
#include "../../../csrc/rownorm.h"
#include "layernorm.h"

namespace {

// mean-subtracted statistics over D, a bias, stat0 = mean, stat1 = rstd.
struct LayerNormRows {
  static constexpr bool kCentered = true, kBias = true;
  __device__ static float stat1(float rs, float) { return rs; }
  __device__ static float rs(float stat1) { return stat1; }
};

int validate(int64_t B, int64_t D, const char* who) {
  if (B < 0 || D < 1)
    return nl2k::fail(NL2K_ERR_SHAPE, "%s: need B >= 0 and D >= 1 (got B=%lld D=%lld)", who,
                      (long long)B, (long long)D);
  if (B > INT32_MAX || D > INT32_MAX || B > INT64_MAX / D)
    return nl2k::fail(NL2K_ERR_OVERFLOW, "%s: sizes too large (B=%lld D=%lld)", who,
                      (long long)B, (long long)D);
  return NL2K_SUCCESS;
}

}  // namespace

extern "C" {

const char* layernorm_last_error(void) { return nl2k::error_slot().text; }

int layernorm_forward_f32(const float* x, const float* w, const float* bias,
                          float* y, float* mean, float* rstd, int64_t B,
                          int64_t D, float eps, hipStream_t stream) {
  int st = validate(B, D, "layernorm_forward_f32");
  if (st) return st;
  if (!(eps >= 0.f))
    return nl2k::fail(NL2K_ERR_VALUE, "layernorm_forward_f32: eps must be >= 0");
  if (B == 0) return nl2k::succeed();
  if (!x || !w || !bias || !y || !mean || !rstd)
    return nl2k::fail(NL2K_ERR_NULL, "layernorm_forward_f32: null pointer argument");
  return nl2k::rownorm::run_forward<LayerNormRows>(x, w, bias, y, mean, rstd, B, D, eps, stream,
                                                   "layernorm_forward_f32");
}

size_t layernorm_backward_workspace_bytes(int64_t B, int64_t D) {
  if (validate(B, D, "layernorm_backward_workspace_bytes")) return 0;
  return nl2k::rownorm::backward_workspace_bytes<LayerNormRows>(B, D);
}

int layernorm_backward_f32(const float* dy, const float* x, const float* w,
                           const float* mean, const float* rstd, float* dx,
                           float* dw, float* dbias, int64_t B, int64_t D,
                           void* workspace, size_t workspace_bytes,
                           hipStream_t stream) {
  const char* who = "layernorm_backward_f32";
  int st = validate(B, D, who);
  if (st) return st;
  if (!dw || !dbias || (B > 0 && (!dy || !x || !w || !mean || !rstd || !dx)))
    return nl2k::fail(NL2K_ERR_NULL, "layernorm_backward_f32: null pointer argument");
  if (B == 0)  // empty batch: the parameter gradients are zero
    return nl2k::rownorm::fill_zero(dw, dbias, D, stream, "layernorm_backward_f32 (zero)");
  const bool aligned = nl2k::aligned16(dy) && nl2k::aligned16(x) && nl2k::aligned16(w) &&
                       nl2k::aligned16(dx);
  const size_t need = nl2k::rownorm::workspace_floats<LayerNormRows>(
                          D, nl2k::rownorm::plan(B, D, aligned)) * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return nl2k::fail(NL2K_ERR_WORKSPACE,
                      "layernorm_backward_f32: workspace of %zu bytes required, got %zu", need,
                      workspace ? workspace_bytes : (size_t)0);
  if (!nl2k::aligned16(workspace))
    return nl2k::fail(NL2K_ERR_ALIGN, "layernorm_backward_f32: workspace must be 16-byte aligned");
  return nl2k::rownorm::run_backward<LayerNormRows>(dy, x, w, mean, rstd, dx, dw, dbias, B, D,
                                                    static_cast<float*>(workspace), stream, who);
}

}  // extern "C"
