/*
 * Softmax, cross-entropy and the fused softmax + cross-entropy
 * (semantics of the reference's src/ops/nvidia/loss/softmax.cu:3-140,273-407
 * and the intended semantics of cross_entropy.cu:4-44; restated in the
 * oracle's softmax / cross_entropy_loss / softmax_cross_entropy_loss).
 *
 * Per row, exactly as the reference orders the arithmetic:
 *   m   = max_j x_j                          (exact)
 *   d_j = rnd(x_j - m)                       (rounded to the input type; fp32: plain fp32 difference)
 *   s   = sum_j exp(d_j)
 *   y_j = rnd_out(exp(d_j) / s)
 * cross-entropy subtracts 1 at the label in the output type:
 *   y_l = rnd_out(y_l - 1)
 * and the fused op also writes loss_r = log(sum_j exp(x_j - m)) + m - x_l
 * (from the unrounded differences) and mean_loss = sum_r loss_r / n_rows.
 *
 * gfx950 design: one 1024-thread workgroup per row; the whole row
 * (up to 16 x 16 B per thread = 128K bf16 logits) is held in VGPRs, so each
 * element is read from HBM once and written once. After the max pass the
 * registers are overwritten with d_j (exact in the storage type), so the
 * output pass needs no recomputation of x - m. exp uses the hardware exp2.
 * mean_loss is summed by a second kernel launched right after on the same
 * stream (fixed order, fp64), so it is deterministic and needs no atomics or
 * device-wide fences.
 */
#include "dtypes.h"
#include "reduce.h"
#include "kernel_geometry.h"

#define SMX_LOG2E 1.4426950408889634f

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * SMX_LOG2E); }

template <typename T> __device__ __forceinline__ float rnd_in(float f) { return to_f(from_f<T>(f)); }

/* Block reductions: each wave's partial goes to its LDS cell, one barrier,
 * then every thread reads all cells (in wave order, so the result does not
 * depend on timing). A caller reusing the same cells must make sure every
 * wave has finished reading them first. */
__device__ __forceinline__ float block_max(float v, float * slots) {
	v = wave_max(v);
	const int nw = blockDim.x >> 6;
	if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
	__syncthreads();
	float m = slots[0];
	for (int w = 1; w < nw; w++) m = fmaxf(m, slots[w]);
	return m;
}

__device__ __forceinline__ void block_sum2(float & a, float & b, float * slots) {
	a = wave_sum(a);
	b = wave_sum(b);
	const int nw = blockDim.x >> 6;
	if ((threadIdx.x & 63) == 0) { slots[threadIdx.x >> 6] = a; slots[16 + (threadIdx.x >> 6)] = b; }
	__syncthreads();
	float sa = 0.0f, sb = 0.0f;
	for (int w = 0; w < nw; w++) { sa += slots[w]; sb += slots[16 + w]; }
	a = sa;
	b = sb;
}

/* mean_loss = sum_r loss[r] / n_rows, summed in fp64 in a fixed order
 * (thread t takes rows t, t + blockDim, ...; then the waves in order). Runs as
 * the op's second kernel, after every row's loss is written. */
__device__ __forceinline__ void mean_loss_finish(int n_rows, const float * loss, float * mean_loss) {
	__shared__ double dslots[16];
	if (blockIdx.x != 0 || !loss || !mean_loss) return;
	double s = 0.0;
	for (int r = threadIdx.x; r < n_rows; r += blockDim.x) s += (double) loss[r];
	for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
	if ((threadIdx.x & 63) == 0) dslots[threadIdx.x >> 6] = s;
	__syncthreads();
	if (threadIdx.x == 0) {
		double t = 0.0;
		for (int w = 0; w < (int) (blockDim.x >> 6); w++) t += dslots[w];
		*mean_loss = (float) (t / (double) n_rows);
	}
}

/* One 32-bit word of a row in storage type T: N elements. `diff` rounds
 * x - m to T (packed, exactly as the reference's in-type subtraction) and also
 * returns the unrounded differences and the rounded values as floats; the
 * packed word is kept, so the output pass needs no repacking. */
template <typename T> struct SmxWord;
template <> struct SmxWord<bf16_t> {
	static constexpr int N = 2;
	__device__ static __forceinline__ void unpack(uint32_t w, float * f) { f[0] = bf16_lo(w); f[1] = bf16_hi(w); }
	__device__ static __forceinline__ uint32_t pack(const float * f) { return pack_bf16x2(f[0], f[1]); }
	__device__ static __forceinline__ uint32_t diff(uint32_t w, float m, float * x_m, float * d) {
		x_m[0] = bf16_lo(w) - m;
		x_m[1] = bf16_hi(w) - m;
		uint32_t dw = pack_bf16x2(x_m[0], x_m[1]);
		/* opaque, so both halves come from the one packed convert (the
		 * compiler would otherwise convert the low half a second time) */
		__asm__ volatile("" : "+v"(dw));
		unpack(dw, d);
		return dw;
	}
};
template <> struct SmxWord<f16_t> {
	static constexpr int N = 2;
	__device__ static __forceinline__ void unpack(uint32_t w, float * f) {
		const f16x2_v h = __builtin_bit_cast(f16x2_v, w);
		f[0] = (float) h.x;
		f[1] = (float) h.y;
	}
	__device__ static __forceinline__ uint32_t pack(const float * f) { return pack_f16x2(f[0], f[1]); }
	__device__ static __forceinline__ uint32_t diff(uint32_t w, float m, float * x_m, float * d) {
		float f[2];
		unpack(w, f);
		x_m[0] = f[0] - m;
		x_m[1] = f[1] - m;
		const uint32_t dw = pack_f16x2(x_m[0], x_m[1]);
		unpack(dw, d);
		return dw;
	}
};
template <> struct SmxWord<float> {
	static constexpr int N = 1;
	__device__ static __forceinline__ void unpack(uint32_t w, float * f) { f[0] = __uint_as_float(w); }
	__device__ static __forceinline__ uint32_t pack(const float * f) { return __float_as_uint(f[0]); }
	__device__ static __forceinline__ uint32_t diff(uint32_t w, float m, float * x_m, float * d) {
		x_m[0] = __uint_as_float(w) - m;
		d[0] = x_m[0];
		return __float_as_uint(d[0]);
	}
};

/* Row max over one chunk. maximum() propagates NaN, so it needs no operand
 * canonicalisation and folds into 3-input max instructions; a NaN anywhere in
 * a row makes the row's sum, and so every output and the loss, NaN either way. */
template <typename T>
__device__ __forceinline__ float chunk_max(const R16 & r, float m) {
	float f[VecOf<T>::N];
	unpack16<T>(r, f);
#pragma unroll
	for (int e = 0; e < VecOf<T>::N; e++) m = __builtin_elementwise_maximum(m, f[e]);
	return m;
}

/* waits for every outstanding vector-memory access of this wave
 * (s_waitcnt vmcnt(0); expcnt and lgkmcnt left at their maxima) */
#define WAIT_VMEM_ALL() __builtin_amdgcn_s_waitcnt(0x0F70)
/* waits for every outstanding LDS access of this wave (lgkmcnt(0)) */
#define WAIT_LDS_ALL() __builtin_amdgcn_s_waitcnt(0xC07F)

typedef __attribute__((address_space(3))) void * lds_ptr_t;

/* Register-resident row path, persistent over rows (row = block, block +
 * grid, ...). Chunk c of thread t is row chunk c * blockDim + t, addressed
 * through a per-row buffer resource (one VGPR offset for all chunks); the
 * whole row sits in VGPRs. The next row is fetched while this one computes:
 * its first SMX_PF chunks go straight into LDS (16-byte buffer loads with the
 * LDS bit) during the max and sum passes, and each of its other chunks is
 * loaded into chunk c's registers as soon as the output pass has stored this
 * row's chunk c. Each wave prefetches into and reads from its own LDS slice
 * only, so no workgroup barrier guards the buffer. */
template <typename T, typename TO, bool FUSED>
__device__ __forceinline__ void smx_regs(int n_rows, int n_cols, const T * X, TO * out, const uint32_t * labels, float * loss) {
	constexpr int VEC = VecOf<T>::N;
	using W = SmxWord<T>;
	using WO = SmxWord<TO>;
	static_assert(sizeof(T) == sizeof(TO), "in-register output packing needs equal widths");
	/* fp32 differences are not rounded, so sum exp(d) is already sum exp(x - m) */
	constexpr bool CORR = FUSED && sizeof(T) < 4;
	/* separate LDS cells for the max and the sum: each is rewritten only after
	 * every wave has passed the other reduction's barrier, so reuse needs no
	 * barrier of its own (two barriers per row) */
	__shared__ float mslots[16];
	__shared__ float sslots[32];
	__shared__ __attribute__((aligned(16))) R16 pf[SMX_PF * SMX_THREADS];
	const int tid = threadIdx.x;
	constexpr int nt = SMX_THREADS;          /* the launch guarantees blockDim.x == SMX_THREADS */
	constexpr uint32_t cstride = nt * 16u;   /* chunk stride: an immediate, rematerialised per use */
	const int wave_base = tid & ~63;
	const int nv = n_cols / VEC;
	const int nch = (nv + nt - 1) / nt;
	const uint32_t row_bytes = (uint32_t) n_cols * (uint32_t) sizeof(T);
	const uint32_t voff = (uint32_t) tid * 16u;

	/* chunks SMX_PF .. SMX_PF + RP - 1 of the next row are loaded a row ahead
	 * into VGPRs; fp32 rows keep those registers for temporaries and load the
	 * chunks past SMX_PF + RP at the top of their own row */
	constexpr int RP = sizeof(T) < 4 ? SMX_MAXCH - SMX_PF : 0;
	int row = blockIdx.x;
	R16 xr[SMX_MAXCH];
	R16 nx[RP > 0 ? RP : 1];
	/* prologue: this workgroup's first row, LDS part and register part */
	if (row < n_rows) {
		const __amdgpu_buffer_rsrc_t r0 = make_rsrc(X + (long) row * n_cols, row_bytes);
#pragma unroll
		for (int c = 0; c < SMX_PF; c++)
			if (c < nch) __builtin_amdgcn_raw_ptr_buffer_load_lds(r0, (lds_ptr_t) &pf[c * nt + wave_base], 16, voff, c * cstride, 0, BUF_AUX_NT);
#pragma unroll
		for (int c = SMX_PF; c < SMX_PF + RP; c++)
			if (c < nch) nx[c - SMX_PF] = buf_load16_nt(r0, voff, c * cstride);
	}
	WAIT_VMEM_ALL();
	for (; row < n_rows; row += gridDim.x) {
		const __amdgpu_buffer_rsrc_t rout = make_rsrc(out + (long) row * n_cols, row_bytes);
		uint32_t lab = 0xffffffffu;
		float x_lab = 0.0f;
		if (FUSED) {
			lab = labels[row];
			if (tid == 0 && lab < (uint32_t) n_cols) x_lab = to_f(X[(long) row * n_cols + lab]);
		}
		/* this row: the LDS part (landed: checked before the last output pass)
		 * and the register part loaded during the last row */
#pragma unroll
		for (int c = 0; c < SMX_PF; c++)
			if (c < nch) xr[c] = pf[c * nt + tid];
		WAIT_LDS_ALL();
#pragma unroll
		for (int c = SMX_PF; c < SMX_PF + RP; c++)
			if (c < nch) xr[c] = nx[c - SMX_PF];
		if (RP < SMX_MAXCH - SMX_PF) {
			const __amdgpu_buffer_rsrc_t rin = make_rsrc(X + (long) row * n_cols, row_bytes);
#pragma unroll
			for (int c = SMX_PF + RP; c < SMX_MAXCH; c++)
				if (c < nch) xr[c] = buf_load16_nt(rin, voff, c * cstride);
		}
		/* the whole next row is requested now and lands while this row computes */
		const int next = row + gridDim.x;
		const bool has_next = next < n_rows;
		if (has_next) {
			const __amdgpu_buffer_rsrc_t rn = make_rsrc(X + (long) next * n_cols, row_bytes);
#pragma unroll
			for (int c = 0; c < SMX_PF; c++)
				if (c < nch) __builtin_amdgcn_raw_ptr_buffer_load_lds(rn, (lds_ptr_t) &pf[c * nt + wave_base], 16, voff, c * cstride, 0, BUF_AUX_NT);
#pragma unroll
			for (int c = SMX_PF; c < SMX_PF + RP; c++)
				if (c < nch) nx[c - SMX_PF] = buf_load16_nt(rn, voff, c * cstride);
		}

		float m = -__builtin_inff();
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			/* chunks past the row end hold zeros: keep them out of the max */
			if (c < nch && c * nt + tid < nv) m = chunk_max<T>(xr[c], m);
		}
		m = block_max(m, mslots);
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) reg_barrier(xr[c]);

		/* sd = sum exp(d) with d = rnd(x - m); the fused op also needs
		 * sx = sum exp(x - m) = sum exp(d) * exp(delta), delta = (x - m) - d
		 * (exact in fp32, |delta| <= half an ulp of d), taken to first order:
		 * the neglected e^d delta^2 / 2 terms change log(sx) by < 2e-6. */
		float sd0 = 0.0f, sd1 = 0.0f, corr = 0.0f;
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			if (c < nch && c * nt + tid < nv) {
				R16 o;
#pragma unroll
				for (int i = 0; i < 4; i++) {
					float x_m[W::N], d[W::N];
					o.w[i] = W::diff(xr[c].w[i], m, x_m, d);
#pragma unroll
					for (int e = 0; e < W::N; e++) {
						const float ex = exp_fast(d[e]);
						if ((i * W::N + e) & 1) sd1 += ex; else sd0 += ex;
						/* fmaxf drops the NaN of -inf - (-inf) (where ex is 0 anyway) */
						if (CORR) corr = fmaf(ex, fmaxf(x_m[e] - d[e], -1.0f), corr);
					}
				}
				xr[c] = o;   /* d, exact in T */
			}
		}
		float sd = sd0 + sd1;
		float sx = sd + corr;
		block_sum2(sd, sx, sslots);
		/* y = exp(d) / sd as one exp2: exp2(d * log2(e) - log2(sd)) */
		const float nlog2s = -__builtin_amdgcn_logf(sd);
		/* the next row's loads are the only vector-memory traffic in flight
		 * here (issued a whole max and sum pass ago; this row's own loads were
		 * consumed by the max pass); its LDS part must have landed before the
		 * next row reads it */
		WAIT_VMEM_ALL();

		/* chunk and element holding the label (if any) */
		const int lab_chunk = (lab < (uint32_t) n_cols) ? (int) (lab / VEC) : -1;
		const int le = (int) (lab % VEC);
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			if (c < nch) {
				R16 o;
#pragma unroll
				for (int i = 0; i < 4; i++) {
					float f[W::N];
					W::unpack(xr[c].w[i], f);
#pragma unroll
					for (int e = 0; e < W::N; e++) f[e] = __builtin_amdgcn_exp2f(fmaf(f[e], SMX_LOG2E, nlog2s));
					o.w[i] = WO::pack(f);
				}
				/* the label's chunk: a wave-uniform branch taken by one wave per
				 * row, so the other chunks carry no per-element label test */
				const bool at_label = FUSED && (c * nt + tid) == lab_chunk;
				if (FUSED && __builtin_amdgcn_ballot_w64(at_label) != 0ull) {
#pragma unroll
					for (int i = 0; i < 4; i++) {
						float f[W::N];
						WO::unpack(o.w[i], f);
#pragma unroll
						for (int e = 0; e < W::N; e++)
							if (at_label && i * W::N + e == le) f[e] -= 1.0f;
						o.w[i] = WO::pack(f);
					}
				}
				buf_store16_nt(rout, voff, c * cstride, o);
			}
		}
		if (FUSED && tid == 0 && loss) {
			loss[row] = (lab < (uint32_t) n_cols) ? (logf(sx) + m - x_lab) : __builtin_nanf("");
		}
	}
	WAIT_VMEM_ALL();
}

/* any row length / alignment: three passes over global memory per row */
template <typename T, typename TO, bool FUSED>
__device__ __forceinline__ void smx_stream(int n_rows, int n_cols, const T * X, TO * out, const uint32_t * labels, float * loss) {
	__shared__ float slots[32];
	const int tid = threadIdx.x;
	const int nt = blockDim.x;
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		const T * xrow = X + (long) row * n_cols;
		TO * orow = out + (long) row * n_cols;
		uint32_t lab = 0xffffffffu;
		float x_lab = 0.0f;
		if (FUSED) {
			lab = labels[row];
			if (tid == 0 && lab < (uint32_t) n_cols) x_lab = to_f(xrow[lab]);
		}
		float m = -__builtin_inff();
		for (int j = tid; j < n_cols; j += nt) m = fmaxf(m, to_f(xrow[j]));
		m = block_max(m, slots);
		float sd = 0.0f, sx = 0.0f;
		for (int j = tid; j < n_cols; j += nt) {
			const float diff = to_f(xrow[j]) - m;
			sd += exp_fast(rnd_in<T>(diff));
			if (FUSED) sx += exp_fast(diff);
		}
		__syncthreads();
		block_sum2(sd, sx, slots);
		const float inv = 1.0f / sd;
		for (int j = tid; j < n_cols; j += nt) {
			float y = exp_fast(rnd_in<T>(to_f(xrow[j]) - m)) * inv;
			if (FUSED && (uint32_t) j == lab) y = rnd_in<TO>(y) - 1.0f;
			orow[j] = from_f<TO>(y);
		}
		if (FUSED && tid == 0 && loss) {
			loss[row] = (lab < (uint32_t) n_cols) ? (logf(sx) + m - x_lab) : __builtin_nanf("");
		}
		__syncthreads();
	}
}

template <typename T, typename TO, bool FUSED>
__device__ __forceinline__ void smx(int n_rows, int n_cols, const T * X, TO * out, const uint32_t * labels, float * loss, float * mean_loss) {
	constexpr int VEC = VecOf<T>::N;
	const bool vec_ok = (n_cols % VEC == 0) && aligned16(X) && aligned16(out) && blockDim.x == SMX_THREADS
						&& ((n_cols / VEC + SMX_THREADS - 1) / SMX_THREADS) <= SMX_MAXCH;
	if (vec_ok) smx_regs<T, TO, FUSED>(n_rows, n_cols, X, out, labels, loss);
	else smx_stream<T, TO, FUSED>(n_rows, n_cols, X, out, labels, loss);
}

#define SMX_KERNELS(SUFFIX, PSUFFIX, T)                                                                                \
	extern "C" __global__ void __launch_bounds__(SMX_THREADS) softmax_##PSUFFIX##_kernel(int n_rows, int n_cols,       \
			T * X, T * out) {                                                                                          \
		smx<T, T, false>(n_rows, n_cols, X, out, nullptr, nullptr, nullptr);                                           \
	}                                                                                                                  \
	extern "C" __global__ void __launch_bounds__(SMX_THREADS) softmax_cross_entropy_loss_##SUFFIX##_kernel(int n_rows, \
			int n_cols, T * logits, uint32_t * labels, float * loss, float * mean_loss) {                              \
		smx<T, T, true>(n_rows, n_cols, logits, logits, labels, loss, mean_loss);                                      \
	}                                                                                                                  \
	extern "C" __global__ void __launch_bounds__(SMX_THREADS) softmax_cross_entropy_loss_##SUFFIX##_kernel_finish(      \
			int n_rows, int n_cols, T * logits, uint32_t * labels, float * loss, float * mean_loss) {                  \
		mean_loss_finish(n_rows, loss, mean_loss);                                                                     \
	}                                                                                                                  \
	extern "C" __global__ void __launch_bounds__(256) cross_entropy_loss_##SUFFIX##_kernel(int n_rows, int n_cols,     \
			T * pred_logits, uint32_t * labels) {                                                                      \
		const long r = (long) blockIdx.x * blockDim.x + threadIdx.x;                                                   \
		if (r >= n_rows) return;                                                                                       \
		const uint32_t lab = labels[r];                                                                                \
		if (lab >= (uint32_t) n_cols) return;                                                                          \
		T * p = pred_logits + r * (long) n_cols + lab;                                                                 \
		*p = from_f<T>(to_f(*p) - 1.0f);                                                                               \
	}

SMX_KERNELS(fp32, fp32_fp32, float)
SMX_KERNELS(fp16, fp16_fp16, f16_t)
SMX_KERNELS(bf16, bf16_bf16, bf16_t)
