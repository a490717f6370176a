/*
 * SwiGLU forward and backward (semantics of the reference's
 * src/ops/nvidia/activations/swiglu.cu:4-68 and swiglu_bwd_x.cu:4-80;
 * restated in the oracle's swiglu_* functions).
 *
 *   fwd: out = silu(g) * u,  silu(g) = g * sigmoid(g)
 *   bwd: dU = dO * silu(g);  dG = dO * u * s * (1 + g * (1 - s)),  s = sigmoid(g)
 *
 * The backward uses the sigmoid form of the reference's closed form
 * u*(1+e+g*e)/(1+e)^2 (e = exp(-g)); it is the same function, and it stays
 * finite where the reference's form gives inf - inf = NaN (g < -88.7).
 *
 * Pure streaming: the [rows x cols] tensors are treated as flat arrays,
 * grid-stride over 16-byte chunks, U chunks per thread and stream per step
 * (U = SWIGLU_FWD_UNROLL / SWIGLU_BWD_UNROLL), software-pipelined: the next step's loads are issued
 * before this step's chunks are computed and stored, so every wave keeps
 * loads in flight through its arithmetic. Loads and stores are
 * non-temporal. The launch uses one large workgroup per CU so that at any
 * moment the whole GPU sweeps one compact window of memory, which is where
 * gfx950's HBM sustains its highest mixed read/write rate.
 */
#include "dtypes.h"
#include "kernel_geometry.h"

#define LOG2E_F 1.4426950408889634f

/* 1 / (1 + exp(-g)) with the hardware exp2 and reciprocal */
__device__ __forceinline__ float sigmoidf_fast(float g) {
	return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * LOG2E_F));
}

/* Below this gate value sigmoid(g) is under 2^-92 and the products are formed
 * from exp(g) * 2^64 (a normal number down to g = -131) and scaled back at the
 * end, so results that are normal fp32 numbers do not pass through an fp32
 * subnormal (which the hardware reciprocal and exp2 flush to zero). */
#define SWIGLU_DEEP_NEG (-64.0f)
#define TWO_POW_M64 5.421010862427522e-20f

__device__ __forceinline__ float exp_scaled64(float g) {   /* exp(g) * 2^64 */
	return __builtin_amdgcn_exp2f(fmaf(g, LOG2E_F, 64.0f));
}

/* DEEP = false drops the deep-negative branch: for fp8 outputs and finite
 * inputs every result it would produce (|silu(g) u| < 64 e^-64 57344 < 2^-70)
 * rounds to a zero of the same sign as the fast form's */
template <bool DEEP = true>
__device__ __forceinline__ float swiglu_fwd_elem(float g, float u) {
	if (DEEP && g < SWIGLU_DEEP_NEG) return ((g * u) * exp_scaled64(g)) * TWO_POW_M64;
	return (g * sigmoidf_fast(g)) * u;
}

template <typename T>
__device__ __forceinline__ void swiglu_fwd(long n, const T * g, const T * u, T * out) {
	constexpr int VEC = VecOf<T>::N;
	const long nth = (long) gridDim.x * blockDim.x;
	const long tid = (long) blockIdx.x * blockDim.x + threadIdx.x;
	const bool vec_ok = aligned16(g) && aligned16(u) && aligned16(out);
	const long nvec = vec_ok ? n / VEC : 0;
	const R16 * gv = reinterpret_cast<const R16 *>(g);
	const R16 * uv = reinterpret_cast<const R16 *>(u);
	R16 * ov = reinterpret_cast<R16 *>(out);

	R16 gr[SWIGLU_FWD_UNROLL], ur[SWIGLU_FWD_UNROLL];
#pragma unroll
	for (int k = 0; k < SWIGLU_FWD_UNROLL; k++) {
		const long v = tid + k * nth;
		if (v < nvec) { gr[k] = ld16_nt(gv + v); ur[k] = ld16_nt(uv + v); }
	}
	for (long v0 = tid; v0 < nvec; v0 += nth * SWIGLU_FWD_UNROLL) {
		vmem_wait_all();
		R16 gn[SWIGLU_FWD_UNROLL], un[SWIGLU_FWD_UNROLL];
#pragma unroll
		for (int k = 0; k < SWIGLU_FWD_UNROLL; k++) {
			const long v = v0 + (SWIGLU_FWD_UNROLL + k) * nth;
			if (v < nvec) { gn[k] = ld16_nt(gv + v); un[k] = ld16_nt(uv + v); }
		}
#pragma unroll
		for (int k = 0; k < SWIGLU_FWD_UNROLL; k++) {
			const long v = v0 + k * nth;
			if (v < nvec) {
				float gf[VEC], uf[VEC], of[VEC];
				unpack16<T>(gr[k], gf);
				unpack16<T>(ur[k], uf);
#pragma unroll
				for (int e = 0; e < VEC; e++) of[e] = swiglu_fwd_elem<!IsFp8<T>::value>(gf[e], uf[e]);
				st16_nt(ov + v, pack16<T>(of));
			}
		}
#pragma unroll
		for (int k = 0; k < SWIGLU_FWD_UNROLL; k++) { gr[k] = gn[k]; ur[k] = un[k]; }
	}
	for (long i = nvec * VEC + tid; i < n; i += nth) {
		out[i] = from_f<T>(swiglu_fwd_elem<!IsFp8<T>::value>(to_f(g[i]), to_f(u[i])));
	}
}

template <typename T>
__device__ __forceinline__ void swiglu_bwd_elem(float g, float u, float d, float & dg, float & du) {
	if (g < SWIGLU_DEEP_NEG) {
		/* sigmoid(g) = exp(g) to fp32 precision and 1 - sigmoid(g) = 1 */
		const float e = exp_scaled64(g);
		du = ((d * g) * e) * TWO_POW_M64;
		dg = ((d * u) * (1.0f + g) * e) * TWO_POW_M64;
		return;
	}
	const float s = sigmoidf_fast(g);
	du = d * (g * s);
	dg = d * (u * s * fmaf(g, 1.0f - s, 1.0f));
}

template <typename T>
__device__ __forceinline__ void swiglu_bwd(long n, const T * g, const T * u, const T * dO, T * dG, T * dU) {
	constexpr int VEC = VecOf<T>::N;
	const long nth = (long) gridDim.x * blockDim.x;
	const long tid = (long) blockIdx.x * blockDim.x + threadIdx.x;
	const bool vec_ok = aligned16(g) && aligned16(u) && aligned16(dO) && aligned16(dG) && aligned16(dU);
	const long nvec = vec_ok ? n / VEC : 0;
	const R16 * gv = reinterpret_cast<const R16 *>(g);
	const R16 * uv = reinterpret_cast<const R16 *>(u);
	const R16 * dv = reinterpret_cast<const R16 *>(dO);
	R16 * dgv = reinterpret_cast<R16 *>(dG);
	R16 * duv = reinterpret_cast<R16 *>(dU);

	R16 gr[SWIGLU_BWD_UNROLL], ur[SWIGLU_BWD_UNROLL], dr[SWIGLU_BWD_UNROLL];
#pragma unroll
	for (int k = 0; k < SWIGLU_BWD_UNROLL; k++) {
		const long v = tid + k * nth;
		if (v < nvec) { gr[k] = ld16_nt(gv + v); ur[k] = ld16_nt(uv + v); dr[k] = ld16_nt(dv + v); }
	}
	for (long v0 = tid; v0 < nvec; v0 += nth * SWIGLU_BWD_UNROLL) {
		vmem_wait_all();
		R16 gn[SWIGLU_BWD_UNROLL], un[SWIGLU_BWD_UNROLL], dn[SWIGLU_BWD_UNROLL];
#pragma unroll
		for (int k = 0; k < SWIGLU_BWD_UNROLL; k++) {
			const long v = v0 + (SWIGLU_BWD_UNROLL + k) * nth;
			if (v < nvec) { gn[k] = ld16_nt(gv + v); un[k] = ld16_nt(uv + v); dn[k] = ld16_nt(dv + v); }
		}
#pragma unroll
		for (int k = 0; k < SWIGLU_BWD_UNROLL; k++) {
			const long v = v0 + k * nth;
			if (v < nvec) {
				float gf[VEC], uf[VEC], df[VEC], ogf[VEC], ouf[VEC];
				unpack16<T>(gr[k], gf);
				unpack16<T>(ur[k], uf);
				unpack16<T>(dr[k], df);
#pragma unroll
				for (int e = 0; e < VEC; e++) swiglu_bwd_elem<T>(gf[e], uf[e], df[e], ogf[e], ouf[e]);
				st16_nt(dgv + v, pack16<T>(ogf));
				st16_nt(duv + v, pack16<T>(ouf));
			}
		}
#pragma unroll
		for (int k = 0; k < SWIGLU_BWD_UNROLL; k++) { gr[k] = gn[k]; ur[k] = un[k]; dr[k] = dn[k]; }
	}
	for (long i = nvec * VEC + tid; i < n; i += nth) {
		float dg, du;
		swiglu_bwd_elem<T>(to_f(g[i]), to_f(u[i]), to_f(dO[i]), dg, du);
		dG[i] = from_f<T>(dg);
		dU[i] = from_f<T>(du);
	}
}

#define SWIGLU_KERNELS(SUFFIX, BSUFFIX, T)                                                                           \
	extern "C" __global__ void __launch_bounds__(512) swiglu_##SUFFIX##_kernel(int num_rows, int num_cols,          \
			T * x_w1, T * x_w3, T * out) {                                                                           \
		swiglu_fwd<T>((long) num_rows * (long) num_cols, x_w1, x_w3, out);                                           \
	}                                                                                                                \
	extern "C" __global__ void __launch_bounds__(512) swiglu_bwd_x_##BSUFFIX##_kernel(int num_rows, int num_cols,  \
			T * x_w1, T * x_w3, T * upstream_dX, T * dX_w1, T * dX_w3) {                                             \
		swiglu_bwd<T>((long) num_rows * (long) num_cols, x_w1, x_w3, upstream_dX, dX_w1, dX_w3);                    \
	}

SWIGLU_KERNELS(fp32, fp32_fp32, float)
SWIGLU_KERNELS(fp16, fp16_fp16, f16_t)
SWIGLU_KERNELS(bf16, bf16_bf16, bf16_t)

/* fp8 forward (reference: swiglu.cu:70-114); the fp8 x fp16/bf16 backward
 * is in fp8_ops.hip */
#define SWIGLU_FP8_KERNEL(SUFFIX, T)                                                                                 \
	extern "C" __global__ void __launch_bounds__(512) swiglu_##SUFFIX##_kernel(int num_rows, int num_cols,          \
			T * x_w1, T * x_w3, T * out) {                                                                           \
		swiglu_fwd<T>((long) num_rows * (long) num_cols, x_w1, x_w3, out);                                           \
	}

SWIGLU_FP8_KERNEL(fp8e4m3, fp8e4m3_t)
SWIGLU_FP8_KERNEL(fp8e5m2, fp8e5m2_t)
