/*
 * liblayernorm_hip.so -- LayerNorm over the last dimension, fp32, MI355X.
 *
 *   mean[b] = sum_d x[b,d] / D
 *   var[b]  = sum_d (x[b,d] - mean[b])^2 / D          (biased)
 *   rstd[b] = 1 / sqrt(var[b] + eps)
 *   y[b,d]  = (x[b,d] - mean[b]) * rstd[b] * w[d] + bias[d]
 *
 * Backward, with g = dy o w and xhat = (x - mean) * rstd:
 *   dx[b,:] = rstd[b] * (g - mean_d(g) - xhat * mean_d(g o xhat))
 *   dw[d]   = sum_b dy[b,d] * xhat[b,d]
 *   dbias[d]= sum_b dy[b,d]
 *
 * Dense row-major fp32 device arrays owned by the caller; kernels run on
 * `stream`; nothing is allocated and no state is kept.  Sizes are validated
 * before any HIP call (NL2K_* codes, message from layernorm_last_error()).
 */
#ifndef NL2K_LAYERNORM_H
#define NL2K_LAYERNORM_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Forward.  Replaces the pybind entry `layernorm_forward(x, gamma, beta,
 * eps) -> [y, mean, inv_std]` of the reference
 * (cases/layernorm/kernels/layernorm_forward.cu:302-379), called from
 * cases/layernorm/op.py:35.  x, y: [B, D]; w, bias: [D]; mean, rstd: [B].
 * B >= 0, D >= 1, eps >= 0.
 */
int layernorm_forward_f32(const float* x, const float* w, const float* bias,
                          float* y, float* mean, float* rstd, int64_t B,
                          int64_t D, float eps, hipStream_t stream);

/* Workspace bytes layernorm_backward_f32 needs for these sizes (per-block
 * partial sums of dw and dbias). */
size_t layernorm_backward_workspace_bytes(int64_t B, int64_t D);

/*
 * Backward.  Replaces `layernorm_backward(grad_y, x, gamma, mean, inv_std)
 * -> [grad_x, grad_gamma, grad_beta]`
 * (cases/layernorm/kernels/layernorm_backward.cu:176-219), called from
 * cases/layernorm/op.py:45.  dx: [B, D]; dw, dbias: [D] (fully written).
 */
int layernorm_backward_f32(const float* dy, const float* x, const float* w,
                           const float* mean, const float* rstd, float* dx,
                           float* dw, float* dbias, int64_t B, int64_t D,
                           void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

const char* layernorm_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_LAYERNORM_H */
