/*
 * librbf_hip.so -- RBF (Gaussian) kernel matrix, forward and backward, fp32,
 * for MI355X (gfx950).
 *
 *   K[i,j] = exp(-gamma * ||X[i,:] - Y[j,:]||^2)          X:[N,D]  Y:[M,D]
 *   W      = dK o K (elementwise)
 *   dX     = -2*gamma * (rowsum(W) o X - W  . Y)            dX:[N,D]
 *   dY     = -2*gamma * (colsum(W) o Y - W^T . X)           dY:[M,D]
 *
 * All arrays are dense row-major fp32 in device memory.  The caller owns
 * every buffer (outputs and workspace); the library allocates nothing, keeps
 * no state between calls, never synchronises, and enqueues its kernels on
 * `stream` (NULL = the null stream).  Calls with invalid arguments return a
 * negative NL2K_* code before any HIP call is made.
 *
 * The Python binding (cases/rbf/op.py) calls these through ctypes with
 * tensor.data_ptr() and torch.cuda.current_stream().cuda_stream.
 */
#ifndef NL2K_RBF_H
#define NL2K_RBF_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Forward: K = exp(-gamma * sqdist(X, Y)).
 * Replaces the pybind entry `rbf_forward(Tensor X, Tensor Y, double gamma)
 * -> Tensor` of the reference (cases/rbf/kernels/rbf_forward.cu:94-120),
 * which cases/rbf/op.py:30 calls.  N, M >= 0, D >= 1.  The fp32 MFMA path
 * runs for D == 64 with 16-byte aligned X, Y, K and M % 4 == 0; every other
 * shape uses a generic HIP kernel.
 */
int rbf_forward_f32(const float* X, const float* Y, float* K, int64_t N,
                    int64_t M, int64_t D, float gamma, hipStream_t stream);

/*
 * Bytes of device workspace rbf_backward_f32 needs for these sizes: the
 * per-region partial sums of dX and dY of the tile kernels, or, for shapes
 * only the generic kernels take (D != 64, N or M past the tile limit), the
 * partial sums of the slices their walks are cut into.  0 means no
 * workspace is needed.
 */
size_t rbf_backward_workspace_bytes(int64_t N, int64_t M, int64_t D);

/*
 * Backward: dX, dY from the upstream gradient dK and the saved forward output
 * K.  Replaces the pybind entry `rbf_backward(Tensor X, Tensor Y, Tensor G,
 * Tensor K, double gamma) -> [dX, dY]` of the reference
 * (cases/rbf/kernels/rbf_backward.cu:59-88), which cases/rbf/op.py:38 calls.
 * `workspace` must hold rbf_backward_workspace_bytes(N, M, D) bytes (it may
 * be NULL when that is 0).  A call that takes the generic kernels also runs
 * with a shorter or NULL workspace, its walks then unsliced (slower, and
 * rounded differently).  dX and dY are fully overwritten.
 */
int rbf_backward_f32(const float* X, const float* Y, const float* dK,
                     const float* K, float* dX, float* dY, int64_t N,
                     int64_t M, int64_t D, float gamma, void* workspace,
                     size_t workspace_bytes, hipStream_t stream);

/*
 * Backward without a caller workspace and without any allocation: for the
 * tile kernels the same kernels and results as rbf_backward_f32 (bit for
 * bit), with the region
 * partials kept in a scratch array compiled into the library (64 MiB per
 * GPU, held from the first call on that GPU until the process ends).  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Calls that take the tile kernels
 * (D = 64, 16-byte aligned X, Y, dX, dY) and whose
 * rbf_backward_workspace_bytes(N, M, D) exceeds
 * rbf_backward_noalloc_max_bytes() are rejected with NL2K_ERR_WORKSPACE
 * before any HIP call (N = M = 4096, D = 64 needs 34 MB and fits; 8192 does
 * not); calls that take the generic kernels use no scratch (their walks
 * unsliced) and run at any size.  Every call on one GPU shares that GPU's scratch, so calls that
 * overlap in time on one GPU (different streams, or threads) race and must
 * be serialised by the caller; a call needs no initial scratch contents.
 */
int rbf_backward_f32_noalloc(const float* X, const float* Y, const float* dK,
                             const float* K, float* dX, float* dY, int64_t N,
                             int64_t M, int64_t D, float gamma, hipStream_t stream);

/* Size in bytes of that scratch array (the largest workspace the no-alloc
 * entry point serves). */
size_t rbf_backward_noalloc_max_bytes(void);

/* Message of the most recent failure on the calling thread ("" if none). */
const char* rbf_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_RBF_H */
