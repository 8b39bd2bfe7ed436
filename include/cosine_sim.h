/*
 * libcosine_sim_hip.so -- pairwise cosine similarity, forward and backward,
 * fp32, for MI355X (gfx950).
 *
 *   s_a[i]  = 1 / (|A[i,:]| + eps)     s_b[j] = 1 / (|B[j,:]| + eps)
 *   S[i,j]  = s_a[i] s_b[j] (A[i,:] . B[j,:])          A:[N,D] B:[M,D] S:[N,M]
 *   backward (autograd of the expression above, upstream dS [N,M]):
 *   dah_i   = sum_j dS[i,j] s_b[j] B[j,:]
 *   dA[i,:] = s_a[i] dah_i - ((s_a[i] A[i,:]) . dah_i) / |A[i,:]| s_a[i] A[i,:]
 *             (second term 0 when |A[i,:]| = 0); dB symmetrically with dS^T.
 *
 * All arrays are dense row-major fp32 in device memory owned by the caller;
 * the library allocates nothing, keeps no state, never synchronises and
 * enqueues its kernels on `stream`.  Arguments are validated before any HIP
 * call (NL2K_* codes, message from cosine_sim_last_error()).
 *
 * Reference interface replaced: the pybind entries `cos_forward(A, B, eps)
 * -> [S, Ah, Bh, invA, invB]` and `cos_backward(Ah, Bh, invA, invB, dS, N,
 * M, D) -> [dA, dB]` of cases/cosine_sim/kernels/cosine_sim.cu:104-130,
 * called from cases/cosine_sim/op.py:19-36.  Here the backward takes A, B
 * and the inverse norms instead of the normalised copies Ah, Bh (it scales
 * rows as it stages them), so the forward writes no [N,D] / [M,D] copies.
 */
#ifndef NL2K_COSINE_SIM_H
#define NL2K_COSINE_SIM_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* S [N, M] and the inverse norms inv_a [N], inv_b [M] (cosine_sim.cu:104-115,
 * `cos_forward`).  The fp32 MFMA path runs for D == 64 with 16-byte aligned
 * A, B; other shapes use generic kernels.  eps >= 0 (NL2K_ERR_VALUE
 * otherwise).  With N == 0 or M == 0 only the inverse norms are written. */
int cosine_sim_forward_f32(const float* A, const float* B, float* S, float* inv_a,
                           float* inv_b, int64_t N, int64_t M, int64_t D, float eps,
                           hipStream_t stream);

/* Workspace bytes cosine_sim_backward_f32 needs (scratch: no initial
 * contents, nothing kept; 16-byte aligned). */
size_t cosine_sim_backward_workspace_bytes(int64_t N, int64_t M, int64_t D);

/* dA [N, D], dB [M, D] from dS [N, M], given A, B and the forward's inverse
 * norms (cosine_sim.cu:117-126, `cos_backward`). */
int cosine_sim_backward_f32(const float* A, const float* B, const float* inv_a,
                            const float* inv_b, const float* dS, float* dA, float* dB,
                            int64_t N, int64_t M, int64_t D, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

const char* cosine_sim_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_COSINE_SIM_H */
