/*
 * libspmv_hip.so -- CSR sparse x dense products (SpMV at D = 1, SpMM at D > 1),
 * fp32 values, int32 or int64 indices, MI355X.
 *
 *   A: [M, K] in CSR (row_ptr[M + 1], col_idx[nnz], vals[nnz]); X: [K, D];
 *   forward   Y[m, :]  = sum_{p in row m} vals[p] * X[col_idx[p], :]
 *   backward  dvals[p] = dY[row(p), :] . X[col_idx[p], :]
 *             dX       = A^T dY  (dX[col_idx[p], :] += vals[p] * dY[row(p), :])
 *
 * Dense arrays are row-major fp32 device arrays owned by the caller; kernels
 * run on `stream`; nothing is allocated and no state is kept.  Preconditions
 * on the structure (row_ptr[0] = 0, non-decreasing, row_ptr[M] = nnz,
 * 0 <= col_idx < K) are not checked by the product entry points, which
 * would need a read-back of device memory; their kernels clamp every index
 * they load into range, so a malformed structure gives wrong numbers, never
 * an out-of-bounds access.  spmv_check_structure_* below checks them on the
 * device for a caller that wants the reference's error (op.py runs it when
 * NL2K_CHECK=1 and raises IndexError for a column out of range, as the
 * reference's index_select does, RuntimeError for a bad row_ptr).  The forward and
 * dvals are deterministic; the D == 1 forward's order of additions does not
 * depend on how rows are split between waves (which follows the device's CU
 * count), so it gives the same bits on any device.  At D > 1 with K <= 16384 (the reference's
 * default SpMM: M = K = 4096, D = 64) dX is deterministic too: each dX row
 * is summed over its column's entries in position order, from entries
 * ordered by column in the workspace (sorted by block of 16 or 64 columns
 * per 1024-position chunk when D % 4 == 0, D <= 64, K <= 4096 (D > 16) or
 * 16384 (D <= 16) and X, dY, dX are 16-byte aligned; else a column-major
 * copy of A).  At D == 1, and at D > 1 beyond 16384 columns, the order of
 * the additions into each dX element varies between runs (as with the
 * reference's atomics).
 *
 * Reference interface replaced: the pybind entries `spmv_forward(row_ptr,
 * col_idx, vals, X) -> Y` and `spmv_backward(row_ptr, col_idx, vals, X,
 * grad_Y) -> [grad_vals, grad_X]` of cases/spmv/kernels/spmv.cu:199-288,
 * called from cases/spmv/op.py:24-57 (there: int64 indices only).
 */
#ifndef NL2K_SPMV_H
#define NL2K_SPMV_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Y [M, D] = A X (spmv.cu:199-239, `spmv_forward`). */
int spmv_forward_f32_i32(const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                         const float* X, float* Y, int64_t M, int64_t K, int64_t D,
                         int64_t nnz, hipStream_t stream);
int spmv_forward_f32_i64(const int64_t* row_ptr, const int64_t* col_idx, const float* vals,
                         const float* X, float* Y, int64_t M, int64_t K, int64_t D,
                         int64_t nnz, hipStream_t stream);

/* Forward that also writes Xg [nnz] = X[col_idx[p]] (D == 1 only, the
 * column clamped into [0, K) as the forward reads it), the gathered copy
 * spmv_backward_gathered_f32_* reads for dvals instead of gathering X again.
 * No counterpart in the reference (spmv.cu:199-239 is the plain forward):
 * it trades nnz * 4 bytes kept from forward to backward for the backward's
 * random reads of X, which bound the D == 1 walk.  D != 1 returns
 * NL2K_ERR_SHAPE before any HIP call. */
int spmv_forward_gather_f32_i32(const int32_t* row_ptr, const int32_t* col_idx,
                                const float* vals, const float* X, float* Y, float* Xg,
                                int64_t M, int64_t K, int64_t D, int64_t nnz,
                                hipStream_t stream);
int spmv_forward_gather_f32_i64(const int64_t* row_ptr, const int64_t* col_idx,
                                const float* vals, const float* X, float* Y, float* Xg,
                                int64_t M, int64_t K, int64_t D, int64_t nnz,
                                hipStream_t stream);

/* Workspace bytes spmv_backward_f32_* needs when dX is requested (0 when
 * none is needed: nnz == 0, D == 1 with more than 16.7M columns, or D > 1
 * with more than 16384 columns or more than 2^31 - 1 nonzeros; dX is then
 * accumulated with fp32 atomics).  The workspace is scratch: no initial
 * contents, nothing kept; 256-byte aligned.  The size serves int32 and
 * int64 indices alike.  At D > 1 the size covers both dX routes (which one
 * a call takes depends on the alignment of its arrays); the build of the
 * column-major copy passes column totals between workgroups through
 * nonce-tagged slots (one launch, no clearing); while `stream` is being
 * captured into a HIP graph a small fill kernel clears those slots first. */
size_t spmv_backward_workspace_bytes(int64_t M, int64_t K, int64_t D, int64_t nnz);

/* Byte offset in that workspace of a uint32 trip counter for shapes that
 * take the D > 1 column-major route (SIZE_MAX otherwise): a workgroup's wait
 * for the column totals of the workgroups before it has a spin cap, never
 * expected to fire; a trip adds 1 here and leaves dX wrong (the
 * column-block route has no such wait and leaves the counter alone).  The library
 * never clears it: a caller that wants to detect a trip zeroes it before
 * the call and reads it after. */
size_t spmv_status_offset(int64_t M, int64_t K, int64_t D, int64_t nnz);

/* dvals [nnz] and dX [K, D] from dY [M, D] (spmv.cu:241-288,
 * `spmv_backward`).  Either output may be NULL to skip it; dX is fully
 * written.  When dX is requested, the workspace must hold
 * spmv_backward_workspace_bytes() bytes: at D == 1 dX = A^T dY is summed by
 * column bucket there, at D > 1 it holds the entries ordered by column
 * (per chunk by column block, or the column-major copy of A). */
int spmv_backward_f32_i32(const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                          const float* X, const float* dY, float* dvals, float* dX,
                          int64_t M, int64_t K, int64_t D, int64_t nnz, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);
int spmv_backward_f32_i64(const int64_t* row_ptr, const int64_t* col_idx, const float* vals,
                          const float* X, const float* dY, float* dvals, float* dX,
                          int64_t M, int64_t K, int64_t D, int64_t nnz, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* spmv_backward_f32_* with dvals taken from Xg, the copy
 * spmv_forward_gather_f32_* wrote for the same X and structure (D == 1
 * only): the walk then streams vals and Xg and reads no col_idx (dX is still
 * summed by column from col_idx).  Results are bit-identical to
 * spmv_backward_f32_*.  Same workspace; X is still required (the fp32-atomic
 * dX route, beyond 16.7M columns, gathers as before).  No counterpart in
 * the reference (spmv.cu:241-288 gathers X). */
int spmv_backward_gathered_f32_i32(const int32_t* row_ptr, const int32_t* col_idx,
                                   const float* vals, const float* X, const float* Xg,
                                   const float* dY, float* dvals, float* dX, int64_t M,
                                   int64_t K, int64_t D, int64_t nnz, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);
int spmv_backward_gathered_f32_i64(const int64_t* row_ptr, const int64_t* col_idx,
                                   const float* vals, const float* X, const float* Xg,
                                   const float* dY, float* dvals, float* dX, int64_t M,
                                   int64_t K, int64_t D, int64_t nnz, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* Structure check: report[4] (uint64, 16-byte aligned, device memory) gets
 * report[0] = OR of 1 (row_ptr[0] != 0), 2 (row_ptr decreasing or outside
 * [0, nnz]), 4 (row_ptr[M] != nnz), 8 (a column outside [0, K)); report[1] =
 * the first position p with col_idx[p] out of range (UINT64_MAX if none);
 * report[2] = the first r whose row_ptr[r] is bad (UINT64_MAX if none);
 * report[3] = 0.  Two kernels on `stream`, no read-back: the caller reads
 * the report after the stream.  No counterpart in the reference kernels
 * (spmv.cu:199-288 read the structure unchecked); it stands in for the
 * IndexError of the reference path's X.index_select(0, col_idx)
 * (cases/spmv/reference.py:19). */
int spmv_check_structure_i32(const int32_t* row_ptr, const int32_t* col_idx, int64_t M,
                             int64_t K, int64_t nnz, uint64_t* report, hipStream_t stream);
int spmv_check_structure_i64(const int64_t* row_ptr, const int64_t* col_idx, int64_t M,
                             int64_t K, int64_t nnz, uint64_t* report, hipStream_t stream);

const char* spmv_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_SPMV_H */
