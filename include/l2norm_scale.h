/*
 * libl2norm_scale_hip.so -- L2 normalisation of rows with a per-dimension
 * scale, forward and backward, fp32, for MI355X (gfx950).
 *
 *   norm[i] = sqrt(sum_j X[i,j]^2 + eps)        X, Y, dY, dX: [N, D]; g, dg: [D]
 *   Y[i,j]  = X[i,j] / norm[i] * g[j]
 *   dX[i,:] = (g dY[i,:] - xh[i,:] (xh[i,:] . (g dY[i,:]))) / norm[i],  xh = X / norm
 *   dg[j]   = sum_i dY[i,j] xh[i,j]
 *
 * Dense row-major fp32 device arrays owned by the caller; the library
 * allocates nothing, keeps no state, never synchronises and launches on
 * `stream`.  Arguments are validated before any HIP call (NL2K_* codes,
 * message from l2norm_scale_last_error()).  dg is deterministic (fixed
 * summation order).
 *
 * Reference interface replaced: the pybind entries `l2n_forward(X, g, eps)
 * -> [Y, norm]` and `l2n_backward(X, g, G, norm) -> [dX, dg]` of
 * cases/l2norm_scale/kernels/l2norm_scale.cu:140-167, called from
 * cases/l2norm_scale/op.py:22-35.
 */
#ifndef NL2K_L2NORM_SCALE_H
#define NL2K_L2NORM_SCALE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Y [N, D] and norm [N] (l2norm_scale.cu:140-150, `l2n_forward`).  The
 * row-cached path runs for D % 4 == 0, D <= 16384 and 16-byte aligned X, g,
 * Y; other shapes use generic kernels.  eps >= 0 (NL2K_ERR_VALUE). */
int l2norm_scale_forward_f32(const float* X, const float* g, float* Y, float* norm, int64_t N,
                             int64_t D, float eps, hipStream_t stream);

/* Workspace bytes l2norm_scale_backward_f32 needs (scratch, 16-byte
 * aligned). */
size_t l2norm_scale_backward_workspace_bytes(int64_t N, int64_t D);

/* dX [N, D] and dg [D] from dY, given X, g and the forward's norm
 * (l2norm_scale.cu:152-163, `l2n_backward`).  N == 0 gives dg = 0. */
int l2norm_scale_backward_f32(const float* dY, const float* X, const float* g, const float* norm,
                              float* dX, float* dg, int64_t N, int64_t D, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

const char* l2norm_scale_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_L2NORM_SCALE_H */
