/*
 * libscan_hip.so -- inclusive prefix sums along the last dimension, MI355X.
 *
 *   forward   y[r, i]  = sum_{j <= i} x[r, j]
 *   backward  dx[r, j] = sum_{i >= j} dy[r, i]       (reverse inclusive scan)
 *
 * x, y: dense row-major [rows, D] device arrays owned by the caller.  fp32
 * sums are accumulated in fp64 and rounded once per output, as torch's CPU
 * cumsum does; integer sums are exact in int64.  Long rows are split into
 * chunks scanned in one pass: every chunk publishes its total to the
 * workspace and adds the totals of the chunks before it in a fixed order,
 * so results are deterministic.  Kernels run on `stream`; nothing is
 * allocated and no state is kept.  Sizes are validated before any HIP call
 * (NL2K_* codes, message from scan_last_error()).
 *
 * Reference interface replaced: the pybind entries `scan_forward(Tensor)`
 * and `scan_backward(Tensor)` of cases/scan/kernels/scan.cu:83-110, called
 * from cases/scan/op.py:22-33 (there: float32 only, D == 4096 only).
 */
#ifndef NL2K_SCAN_H
#define NL2K_SCAN_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "nl2k_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Workspace bytes any scan_* call below needs for [rows, D] (0 when every
 * row fits one chunk).  The workspace needs no initial contents and no
 * clearing: each call tags what it writes with a fresh 64-bit nonce and
 * reads back only its own words (a word pair left by an earlier call, or a
 * zero-filled one, is never taken; other contents pass the check only by
 * chance, with probability 2^-64 per read), so a call is a single kernel
 * launch.  Calls that share a workspace must not overlap in time; calls on
 * different streams need different workspaces.  A larger workspace serves
 * smaller shapes too.  While `stream` is being captured into a HIP graph a
 * call enqueues a small fill kernel over the slots before the scan (replays
 * reuse the captured nonce, so each replay must start from cleared slots);
 * outside capture it stays one launch. */
size_t scan_workspace_bytes(int64_t rows, int64_t D);

/* Byte offset, inside the workspace of a [rows, D] call, of the uint32 trip
 * counter (in an 8-byte word after the slots); SIZE_MAX when the shape needs
 * no workspace or is invalid.  A chunk whose wait for its predecessors'
 * totals exceeds a spin cap (never expected: the grid is capped at the
 * device's resident workgroup count, but a CU-masked queue may hold fewer)
 * adds 1 and scans with a zero carry.  The library never clears the
 * counter: a caller that wants to detect such a trip zeroes it before the
 * call and reads it after. */
size_t scan_status_offset(int64_t rows, int64_t D);

/* Workgroups a [rows, D] launch uses when `resident_workgroups` can be on
 * the device at once (the library passes CU count x the occupancy the
 * runtime reports for the kernel); -1 for invalid arguments.  Host-only
 * planning query, no HIP call. */
int64_t scan_launch_grid(int64_t rows, int64_t D, int64_t resident_workgroups);

/* float32 -> float32 inclusive scan (scan.cu:83-95, `scan_forward`). */
int scan_forward_f32(const float* x, float* y, int64_t rows, int64_t D,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* float32 reverse inclusive scan, the gradient of the forward
 * (scan.cu:97-105, `scan_backward`). */
int scan_backward_f32(const float* dy, float* dx, int64_t rows, int64_t D,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* int32 -> int64 inclusive scan: torch.cumsum's result type for int32
 * input (cases/scan/reference.py:8-9); exact. */
int scan_forward_i32_i64(const int32_t* x, int64_t* y, int64_t rows, int64_t D,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* int32 -> int32 inclusive scan with two's-complement wrap-around (the
 * exact int64 sum truncated to 32 bits). */
int scan_forward_i32(const int32_t* x, int32_t* y, int64_t rows, int64_t D,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

const char* scan_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NL2K_SCAN_H */
