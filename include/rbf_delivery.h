/*
 * librbf.a (cases/rbf/delivery) -- host-pointer RBF entry points for callers
 * without a device-memory runtime of their own (no PyTorch needed).
 *
 * Each call copies the host arrays to the GPU, runs the same kernels as
 * rbf_forward_f32 / rbf_backward_f32 (include/rbf.h), copies the results
 * back and frees its device memory before returning (synchronous).
 * Returns NL2K_SUCCESS (0) or an NL2K_* code; the message is available from
 * rbf_last_error().  X: [N, D], Y: [M, D], K, G: [N, M], dX: [N, D],
 * dY: [M, D], row-major fp32 host arrays.
 *
 * Reference interface replaced: `extern "C" void rbf_forward_cuda(...)` and
 * `rbf_backward_cuda(...)` of cases/rbf/delivery/rbf_kernels.cu:168-220
 * (same argument order; the reference aborts the process on any error,
 * these return a status instead).
 */
#ifndef NL2K_RBF_DELIVERY_H
#define NL2K_RBF_DELIVERY_H

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

int rbf_forward_hip(const float* X, const float* Y, float* K, int N, int M, int D,
                    float gamma);

int rbf_backward_hip(const float* X, const float* Y, const float* G, const float* K,
                     float* dX, float* dY, int N, int M, int D, float gamma);

const char* rbf_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_RBF_DELIVERY_H */
