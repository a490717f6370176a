/*
 * Mixed-precision variants with fp8 forward tensors and fp16 / bf16 backward
 * tensors (the reference's "<op>_fp8e4m3_fp16" ... "<op>_fp8e5m2_bf16"
 * kernels), restated in the oracle's *2 functions:
 *   rms_norm_bwd_x   W, X fp8; dY, dX 16-bit    (rms_norm_bwd_x.cu:259-590)
 *   rms_norm_bwd_w   X fp8; dY, dW 16-bit       (rms_norm_bwd_w.cu:310-700)
 *   swiglu_bwd_x     g, u fp8; dO, dG, dU 16-bit (swiglu_bwd_x.cu:82-187)
 *   softmax          X fp8, out 16-bit; x - max rounded in the output type
 *                    (softmax.cu:409-960)
 * Each lane takes eight consecutive elements at a time: eight bytes of each
 * fp8 operand and sixteen of each 16-bit one, so both stay coalesced with one
 * load per operand. Rows or tensors that are not multiples of eight elements,
 * or not aligned to 8 / 16 bytes, take element loops. The arithmetic is the
 * same-type kernels' (bwd_x_elem, swiglu_bwd_elem); the dW partial rows and
 * their finish pass are rms_norm.hip's.
 */
#include "dtypes.h"
#include "reduce.h"
#include "kernel_geometry.h"

__device__ __forceinline__ R8 ld8(const void * p) {
	typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_v;
	const u32x2_v v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_v *>(p));
	R8 r;
	r.w[0] = v.x;
	r.w[1] = v.y;
	return r;
}

__device__ __forceinline__ bool aligned8(const void * p) { return (((uintptr_t) p) & 7u) == 0; }

/* ---------------- rms_norm_bwd_x ---------------- */

template <typename TF, typename TB>
__device__ __forceinline__ void rms_bwd_x_fp8(int n_rows, int n_cols, const float * ws_in, const float * rs_in,
												const TF * W, const TF * X, const TB * dY, TB * dX) {
	const bool vec = (n_cols % 8) == 0 && aligned8(W) && aligned8(X) && aligned16(dY) && aligned16(dX);
	const int nv = n_cols / 8;
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		const long off = (long) row * n_cols;
		const float r = rs_in[row], ws = ws_in[row];
		const float r3 = r * r * r;
		if (vec) {
			for (int c = threadIdx.x; c < nv; c += blockDim.x) {
				float wf[8], xf[8], gf[8], df[8];
				unpack8_fp8<TF>(*reinterpret_cast<const R8 *>(W + 8 * c), wf);
				unpack8_fp8<TF>(ld8(X + off + 8 * c), xf);
				unpack16<TB>(ld16_nt(dY + off + 8 * c), gf);
				unpack16<TB>(ld16_nt(dX + off + 8 * c), df);
#pragma unroll
				for (int e = 0; e < 8; e++) df[e] = bwd_x_elem<TB>(wf[e], xf[e], gf[e], df[e], r, r3, ws, n_cols);
				st16_nt(dX + off + 8 * c, pack16<TB>(df));
			}
		}
		else {
			for (int j = threadIdx.x; j < n_cols; j += blockDim.x)
				dX[off + j] = from_f<TB>(bwd_x_elem<TB>(to_f(W[j]), to_f(X[off + j]), to_f(dY[off + j]), to_f(dX[off + j]), r, r3, ws, n_cols));
		}
	}
}

/* ---------------- rms_norm_bwd_w ---------------- */

/* Workgroup w sums dY * X * rstd over rows w, w + grid, ... into an LDS row of
 * n_cols floats (each thread owns its columns, so no two threads touch one
 * cell), then writes it as partial row w; the op's finish kernel adds the
 * partial rows in a fixed order (rms_dw_finish), as for the other types. */
template <typename TF, typename TB>
__device__ __forceinline__ void rms_bwd_w_fp8(int n_rows, int n_cols, const float * rs_in, const TF * X, const TB * dY) {
	extern __shared__ float colbuf[];
	if (blockIdx.x == 0 && threadIdx.x == 0) g_rms_dw_nparts = (int) gridDim.x;
	const bool vec = (n_cols % 8) == 0 && aligned8(X) && aligned16(dY);
	const int nv = n_cols / 8;
	for (int j = threadIdx.x; j < n_cols; j += blockDim.x) colbuf[j] = 0.0f;
	/* the vector loop below maps 8 columns to a thread, the zeroing one */
	__syncthreads();
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		const long off = (long) row * n_cols;
		const float r = rs_in[row];
		if (vec) {
			for (int c = threadIdx.x; c < nv; c += blockDim.x) {
				float xf[8], gf[8];
				unpack8_fp8<TF>(ld8(X + off + 8 * c), xf);
				unpack16<TB>(ld16_nt(dY + off + 8 * c), gf);
#pragma unroll
				for (int e = 0; e < 8; e++) colbuf[8 * c + e] = fmaf(gf[e] * xf[e], r, colbuf[8 * c + e]);
			}
		}
		else {
			for (int j = threadIdx.x; j < n_cols; j += blockDim.x) colbuf[j] = fmaf(to_f(dY[off + j]) * to_f(X[off + j]), r, colbuf[j]);
		}
	}
	write_partial_from_lds(colbuf, n_cols, g_rms_dw_partials);
}

/* ---------------- swiglu_bwd_x ---------------- */

template <typename TF, typename TB>
__device__ __forceinline__ void swiglu_bwd_fp8(long n, const TF * g, const TF * u, const TB * dO, TB * dG, TB * dU) {
	const long nth = (long) gridDim.x * blockDim.x;
	const long tid = (long) blockIdx.x * blockDim.x + threadIdx.x;
	const bool vec = aligned8(g) && aligned8(u) && aligned16(dO) && aligned16(dG) && aligned16(dU);
	const long nvec = vec ? n / 8 : 0;
	for (long v = tid; v < nvec; v += nth) {
		float gf[8], uf[8], df[8], ogf[8], ouf[8];
		unpack8_fp8<TF>(ld8(g + 8 * v), gf);
		unpack8_fp8<TF>(ld8(u + 8 * v), uf);
		unpack16<TB>(ld16_nt(dO + 8 * v), df);
#pragma unroll
		for (int e = 0; e < 8; e++) swiglu_bwd_elem<TB>(gf[e], uf[e], df[e], ogf[e], ouf[e]);
		st16_nt(dG + 8 * v, pack16<TB>(ogf));
		st16_nt(dU + 8 * v, pack16<TB>(ouf));
	}
	for (long i = nvec * 8 + tid; i < n; i += nth) {
		float dg, du;
		swiglu_bwd_elem<TB>(to_f(g[i]), to_f(u[i]), to_f(dO[i]), dg, du);
		dG[i] = from_f<TB>(dg);
		dU[i] = from_f<TB>(du);
	}
}

/* ---------------- softmax ---------------- */

/* Three passes per row, the later ones re-reading the row (a row of fp8 is
 * n_cols bytes, so they find it in cache): max, sum exp(d), outputs, with
 * d = rnd_out(x - max) since the reference converts x to the output type and
 * subtracts there. */
template <typename TF, typename TO>
__device__ __forceinline__ void softmax_fp8(int n_rows, int n_cols, const TF * X, TO * out) {
	__shared__ float slots[32];
	const bool vec = (n_cols % 8) == 0 && aligned8(X) && aligned16(out);
	const int nv = n_cols / 8;
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		const TF * x = X + (long) row * n_cols;
		TO * o = out + (long) row * n_cols;
		float m = -__builtin_inff();
		if (vec) {
			for (int c = threadIdx.x; c < nv; c += blockDim.x) {
				float f[8];
				unpack8_fp8<TF>(*reinterpret_cast<const R8 *>(x + 8 * c), f);
#pragma unroll
				for (int e = 0; e < 8; e++) m = __builtin_elementwise_maximum(m, f[e]);
			}
		}
		else {
			for (int j = threadIdx.x; j < n_cols; j += blockDim.x) m = __builtin_elementwise_maximum(m, to_f(x[j]));
		}
		m = block_max(m, slots);
		float sd = 0.0f;
		if (vec) {
			for (int c = threadIdx.x; c < nv; c += blockDim.x) {
				float f[8];
				unpack8_fp8<TF>(*reinterpret_cast<const R8 *>(x + 8 * c), f);
#pragma unroll
				for (int e = 0; e < 8; e++) sd += exp_fast(rnd_in<TO>(f[e] - m));
			}
		}
		else {
			for (int j = threadIdx.x; j < n_cols; j += blockDim.x) sd += exp_fast(rnd_in<TO>(to_f(x[j]) - m));
		}
		float unused = 0.0f;
		__syncthreads();   /* every wave has read the max cells */
		block_sum2(sd, unused, slots);
		const float nlog2s = -__builtin_amdgcn_logf(sd);
		if (vec) {
			for (int c = threadIdx.x; c < nv; c += blockDim.x) {
				float f[8];
				unpack8_fp8<TF>(ld8(x + 8 * c), f);
#pragma unroll
				for (int e = 0; e < 8; e++) f[e] = __builtin_amdgcn_exp2f(fmaf(rnd_in<TO>(f[e] - m), SMX_LOG2E, nlog2s));
				st16_nt(o + 8 * c, pack16<TO>(f));
			}
		}
		else {
			for (int j = threadIdx.x; j < n_cols; j += blockDim.x)
				o[j] = from_f<TO>(__builtin_amdgcn_exp2f(fmaf(rnd_in<TO>(to_f(x[j]) - m), SMX_LOG2E, nlog2s)));
		}
		__syncthreads();   /* the cells are rewritten for the next row */
	}
}

#define FP8_MIXED_KERNELS(FSUF, BSUF, TF, TB)                                                                          \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_bwd_x_##FSUF##_##BSUF##_kernel(int n_rows, int n_cols,  \
			float eps, float * fwd_weighted_sums, float * fwd_rms_vals, TF * rms_weight, TF * X_inp, TB * upstream_dX,  \
			TB * dX) {                                                                                                  \
		rms_bwd_x_fp8<TF, TB>(n_rows, n_cols, fwd_weighted_sums, fwd_rms_vals, rms_weight, X_inp, upstream_dX, dX);     \
	}                                                                                                                   \
	extern "C" __global__ void __launch_bounds__(1024) rms_norm_bwd_w_##FSUF##_##BSUF##_kernel(int n_rows, int n_cols,  \
			float eps, float * fwd_rms_vals, TF * X_inp, TB * upstream_dX, TB * dW) {                                   \
		rms_bwd_w_fp8<TF, TB>(n_rows, n_cols, fwd_rms_vals, X_inp, upstream_dX);                                       \
	}                                                                                                                   \
	extern "C" __global__ void __launch_bounds__(RMS_FINISH_THREADS) rms_norm_bwd_w_##FSUF##_##BSUF##_kernel_finish(    \
			int n_rows, int n_cols, float eps, float * fwd_rms_vals, TF * X_inp, TB * upstream_dX, TB * dW) {           \
		rms_dw_finish<TB>(n_cols, dW, g_rms_dw_partials, g_rms_dw_nparts);                                             \
	}                                                                                                                   \
	extern "C" __global__ void __launch_bounds__(512) swiglu_bwd_x_##FSUF##_##BSUF##_kernel(int num_rows, int num_cols, \
			TF * x_w1, TF * x_w3, TB * upstream_dX, TB * dX_w1, TB * dX_w3) {                                          \
		swiglu_bwd_fp8<TF, TB>((long) num_rows * (long) num_cols, x_w1, x_w3, upstream_dX, dX_w1, dX_w3);              \
	}                                                                                                                   \
	extern "C" __global__ void __launch_bounds__(SMX_THREADS) softmax_##FSUF##_##BSUF##_kernel(int n_rows, int n_cols,   \
			TF * X, TB * out) {                                                                                         \
		softmax_fp8<TF, TB>(n_rows, n_cols, X, out);                                                                   \
	}

FP8_MIXED_KERNELS(fp8e4m3, fp16, fp8e4m3_t, f16_t)
FP8_MIXED_KERNELS(fp8e4m3, bf16, fp8e4m3_t, bf16_t)
FP8_MIXED_KERNELS(fp8e5m2, fp16, fp8e5m2_t, f16_t)
FP8_MIXED_KERNELS(fp8e5m2, bf16, fp8e5m2_t, bf16_t)
