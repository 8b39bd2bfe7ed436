/*
 * Status codes shared by every C-ABI library of this package
 * (librbf_hip.so, liblayernorm_hip.so, libscan_hip.so, libspmv_hip.so,
 * libcosine_sim_hip.so, libl2norm_scale_hip.so, libsoftmax_ce_hip.so).
 *
 * Every entry point returns 0 on success or one of the negative codes below.
 * Argument validation runs before any HIP call, so a rejected call never
 * touches the device.  The text of the most recent failure on the calling
 * thread is returned by the library's <case>_last_error() function.
 *
 * The reference reports the same conditions as TORCH_CHECK failures
 * (e.g. cases/rbf/kernels/rbf_forward.cu:95-99) that surface in Python as
 * RuntimeError; the Python layer of this package maps a non-zero code to a
 * RuntimeError carrying the library's message.
 */
#ifndef NL2K_STATUS_H
#define NL2K_STATUS_H

#define NL2K_SUCCESS 0
#define NL2K_ERR_NULL (-1)      /* a required pointer is NULL               */
#define NL2K_ERR_SHAPE (-2)     /* negative or inconsistent sizes           */
#define NL2K_ERR_ALIGN (-3)     /* pointer alignment not usable             */
#define NL2K_ERR_WORKSPACE (-4) /* workspace missing or too small           */
#define NL2K_ERR_OVERFLOW (-5)  /* sizes overflow the kernels' index math   */
#define NL2K_ERR_VALUE (-6)     /* invalid scalar argument (e.g. NaN eps)   */
#define NL2K_ERR_HIP (-100)     /* a HIP runtime call or launch failed      */

#endif /* NL2K_STATUS_H */
