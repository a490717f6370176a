/*
 * RMSNorm kernels of the gfx950 code object (reference ABI: parameter lists
 * of src/ops/nvidia/include/nvidia_ops.h; device code in rms_norm_impl.h).
 * The dW ops keep their partial rows in this module's scratch
 * (g_rms_dw_partials, 16 MiB) and pass the grid size to their finish kernel
 * through g_rms_dw_nparts, since the finish kernel is launched with the same
 * reference argument list as the main one.
 */
#include "rms_norm_impl.h"

__device__ float g_rms_dw_partials[RMS_DW_SCRATCH_FLOATS];
/* number of partial rows written by the last main pass (its grid size) */
__device__ int g_rms_dw_nparts;

#define RMS_KERNELS(FSUF, PSUF, T)                                                                                       \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_##FSUF##_kernel(int n_rows, int n_cols, float eps,       \
			T * rms_weight, T * X, T * out, float * weighted_sums, float * rms_vals) {                                  \
		RmsArgs a = {n_rows, n_cols, eps, nullptr, nullptr, weighted_sums, rms_vals, rms_weight, X, nullptr, out, nullptr}; \
		rms_run<T, T, RMS_FWD>(a);                                                                                       \
	}                                                                                                                    \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_bwd_x_##PSUF##_kernel(int n_rows, int n_cols, float eps, \
			float * fwd_weighted_sums, float * fwd_rms_vals, T * rms_weight, T * X_inp, T * upstream_dX, T * dX) {       \
		RmsArgs a = {n_rows, n_cols, eps, fwd_weighted_sums, fwd_rms_vals, nullptr, nullptr, rms_weight, X_inp, upstream_dX, dX, nullptr}; \
		rms_run<T, T, RMS_BWD_X>(a);                                                                                     \
	}                                                                                                                    \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_bwd_w_##PSUF##_kernel(int n_rows, int n_cols, float eps, \
			float * fwd_rms_vals, T * X_inp, T * upstream_dX, T * dW) {                                                 \
		RmsArgs a = {n_rows, n_cols, eps, nullptr, fwd_rms_vals, nullptr, nullptr, nullptr, X_inp, upstream_dX, nullptr, dW, \
					 g_rms_dw_partials, &g_rms_dw_nparts};                                                                 \
		rms_run<T, T, RMS_BWD_W>(a);                                                                                     \
	}                                                                                                                    \
	extern "C" __global__ void __launch_bounds__(RMS_FINISH_THREADS) rms_norm_bwd_w_##PSUF##_kernel_finish(int n_rows, int n_cols,      \
			float eps, float * fwd_rms_vals, T * X_inp, T * upstream_dX, T * dW) {                                      \
		rms_dw_finish<T>(n_cols, dW, g_rms_dw_partials, g_rms_dw_nparts);                                                                                    \
	}                                                                                                                    \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_bwd_##PSUF##_kernel(int n_rows, int n_cols, float eps,   \
			float * fwd_rms_vals, T * rms_weight, T * X_inp, T * upstream_dX, T * dX, float * dW) {                     \
		RmsArgs a = {n_rows, n_cols, eps, nullptr, fwd_rms_vals, nullptr, nullptr, rms_weight, X_inp, upstream_dX, dX, dW, \
					 g_rms_dw_partials, &g_rms_dw_nparts};                                                                 \
		rms_run<T, float, RMS_BWD>(a);                                                                                   \
	}                                                                                                                    \
	extern "C" __global__ void __launch_bounds__(RMS_FINISH_THREADS) rms_norm_bwd_##PSUF##_kernel_finish(int n_rows, int n_cols,        \
			float eps, float * fwd_rms_vals, T * rms_weight, T * X_inp, T * upstream_dX, T * dX, float * dW) {          \
		rms_dw_finish<float>(n_cols, dW, g_rms_dw_partials, g_rms_dw_nparts);                                                                                \
	}

RMS_KERNELS(fp32, fp32_fp32, float)
RMS_KERNELS(fp16, fp16_fp16, f16_t)
RMS_KERNELS(bf16, bf16_bf16, bf16_t)

/* fp8 forward (reference: rms_norm.cu:415-659): out = fp8((x * rstd) * w);
 * the statistic slot receives sum_j x^2 instead of rstd and weighted_sums is
 * not written, as in the reference's fp8 kernels */
#define RMS_FP8_FWD_KERNEL(FSUF, T)                                                                                     \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_##FSUF##_kernel(int n_rows, int n_cols, float eps,       \
			T * rms_weight, T * X, T * out, float * weighted_sums, float * sq_sums) {                                   \
		RmsArgs a = {n_rows, n_cols, eps, nullptr, nullptr, nullptr, sq_sums, rms_weight, X, nullptr, out, nullptr,      \
					 nullptr, nullptr, true};                                                                            \
		rms_run<T, T, RMS_FWD>(a);                                                                                       \
	}

RMS_FP8_FWD_KERNEL(fp8e4m3, fp8e4m3_t)
RMS_FP8_FWD_KERNEL(fp8e5m2, fp8e5m2_t)
