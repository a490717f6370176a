/*
 * Allocation-free entry point (libdataflow_noalloc.so).
 *
 * No counterpart in the reference. It is for callers that cannot allocate
 * device memory or create a Dataflow_Handle at the point of the call: code
 * under HIP graph capture, tight serving or training loops, and harnesses
 * that forbid hipMalloc. It computes exactly what submit_rms_norm_bwd
 * computes (same kernels, same launch shape, so bit-identical dX and dW),
 * without a handle and without allocating: the dW partial rows live in a
 * fixed device array of the library, one per GPU, held until the process
 * ends.
 */
#ifndef DATAFLOW_NOALLOC_H
#define DATAFLOW_NOALLOC_H

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#include "dataflow_datatype.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the library's per-GPU dW scratch: one fp32 partial row of n_cols
 * per workgroup, at most one workgroup per CU (16 MiB). */
#define DATAFLOW_NOALLOC_SCRATCH_BYTES (16u << 20)

/* Exact RMSNorm backward, as submit_rms_norm_bwd (dataflow_ops.h):
 * dX += rstd * dY * w - X * rstd^3 / n_cols * sum_j(dY * w * X) per row and
 * dW (fp32) += sum over rows of dY * X * rstd, on `stream`, which must belong
 * to the calling thread's current device. fwd_dt and bwd_dt must be equal:
 * DATAFLOW_FP32, DATAFLOW_FP16 or DATAFLOW_BF16. Returns 0 (also for zero
 * rows or columns, with nothing launched), or -1 with a message for an
 * unsupported type, a negative size, rows too long for the LDS, a partial
 * row larger than the scratch (n_cols > 4M), a stream of another device
 * than the current one (hipStreamGetDevice), or a failed launch.
 * Calls no hipMalloc, hipFree or other allocating routine. The first call on
 * a device resolves that device's scratch address once (hipGetSymbolAddress).
 * All calls on one GPU share its scratch: calls that overlap in time on one
 * GPU (different streams, or several threads) race and give wrong dW. The
 * scratch keeps the last call's partial rows; every call writes each partial
 * row it reads, so nothing needs clearing between calls. */
int dataflow_rms_norm_bwd_noalloc(hipStream_t stream, DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								  int n_rows, int n_cols, float eps,
								  const float * fwd_rms_vals, const void * rms_weight, const void * X_inp,
								  const void * upstream_dX, void * dX, float * dW);

#ifdef __cplusplus
}
#endif

#endif
