/*
 * libsoftmax_ce_hip.so -- softmax cross-entropy loss, forward and backward,
 * fp32 logits and int64 labels, for MI355X (gfx950).
 *
 *   lse[b]        = log sum_c exp(logits[b, c])       logits, dlogits: [B, C]
 *   loss          = (1/B) sum_b (lse[b] - logits[b, labels[b]])   labels, lse: [B]
 *   dlogits[b, c] = gout[0] / B * (exp(logits[b, c] - lse[b]) - [c == labels[b]])
 *
 * Dense row-major device arrays owned by the caller; the library
 * allocates nothing, keeps no state, never synchronises and launches on
 * `stream`.  Arguments are validated before any HIP call (NL2K_* codes,
 * message from softmax_ce_last_error()).  The loss is deterministic: one
 * partial sum per workgroup, published in the caller's scratch workspace
 * and added in a fixed order by workgroup 0 of the same launch (no float
 * atomics, one launch).  A
 * label outside [0, C) is not checked on the host (labels live on the
 * device); it makes the loss and that row's gradient NaN.  B == 0 gives
 * loss = NaN (the mean of no terms).
 *
 * Reference interface replaced: the pybind entries
 * `softmax_ce_forward(logits, labels) -> loss` of
 * cases/softmax_ce/kernels/softmax_ce_forward.cu:52-65 and
 * `softmax_ce_backward(logits, labels, gout) -> dlogits` of
 * cases/softmax_ce/kernels/softmax_ce_backward.cu:57-70, called from
 * cases/softmax_ce/op.py:28-41.
 */
#ifndef NL2K_SOFTMAX_CE_H
#define NL2K_SOFTMAX_CE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Scratch bytes softmax_ce_forward_f32 needs (8-byte aligned; a constant
 * 16392: a 16-byte slot pair for each of at most 1024 workgroups, tagged
 * with a fresh nonce per call, so no initial contents are needed, then the
 * 8-byte status word below); 0 for invalid sizes.  While `stream` is being
 * captured into a HIP graph the forward enqueues a small fill kernel over
 * the slots first (replays reuse the captured nonce); otherwise it is one
 * launch. */
size_t softmax_ce_forward_workspace_bytes(int64_t B, int64_t C);

/* Byte offset in that workspace of the uint32 trip counter: workgroup 0's
 * wait for the other workgroups' partial losses has a spin cap (never
 * expected to fire); a trip makes the loss NaN and adds 1 here.  The
 * library never clears it: a caller that wants to tell a trip from a NaN
 * caused by an invalid label zeroes it before the call and reads it after. */
size_t softmax_ce_status_offset(void);

/* loss [1] and lse [B] (softmax_ce_forward.cu:52-65, `softmax_ce_forward`;
 * lse is extra: the backward reuses it instead of recomputing each row's
 * max and sum).  The row-cached path runs for C % 4 == 0, C <= 8192 and a
 * 16-byte aligned `logits`; other shapes use a generic kernel. */
int softmax_ce_forward_f32(const float* logits, const int64_t* labels, float* loss, float* lse,
                           int64_t B, int64_t C, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* dlogits [B, C] from the forward's lse and the upstream gradient gout [1]
 * (a device pointer, read by the kernel; softmax_ce_backward.cu:57-70). */
int softmax_ce_backward_f32(const float* logits, const int64_t* labels, const float* lse,
                            const float* gout, float* dlogits, int64_t B, int64_t C,
                            hipStream_t stream);

const char* softmax_ce_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_SOFTMAX_CE_H */
