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
 * Rows are handed to the workgroups as they free up (a row counter in the
 * code object), so every workgroup keeps working until the rows run out
 * instead of the slowest CU's fixed share setting the kernel's end.
 * mean_loss is summed by the last workgroup to finish (fixed order, fp64, so
 * it is deterministic), from per-row losses stored at device scope.
 */
#include "dtypes.h"
#include "reduce.h"
#include "kernel_geometry.h"

#define SMX_LOG2E 1.4426950408889634f

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * SMX_LOG2E); }

/* Factor that moves an online sum of exp(x - ref) from reference `from` to
 * reference `to` (to >= from once a finite max has been seen). Until then the
 * reference is a placeholder 0 and the sum is 0: the exponent is clamped at 0
 * so that moving it to a max below -88 multiplies 0 by 1, not by an
 * overflowed exp (0 * inf would make the sum NaN). */
__device__ __forceinline__ float online_rescale(float from, float to) {
	return __builtin_amdgcn_exp2f(fminf((from - to) * SMX_LOG2E, 0.0f));
}

#define SMX_LN2 0.6931471805599453f

/* log(1 + y) for y >= 0 in about fifteen instructions. One lane forms each
 * row's loss on the way to the next row's first barrier, so every wave waits
 * for it: with the library's log1pf and a correctly rounded divide (about
 * 135 dependent instructions) the fused kernel took 383.0-388.6 us at
 * 4096 x 128256 bf16, with this 382.0-383.3 us (five interleaved batches on
 * one MI355X), the losses as close to an fp64 loss (6.1e-7 relative at most).
 * Below 1/32 it is the Taylor series to y^6, whose remainder is below
 * y^7 / 7 (relative 2^-30 / 7). From 1/32 up it is log(u) * (y / (u - 1))
 * with u = 1 + y rounded, which cancels the rounding of u (Goldberg, "What
 * every computer scientist should know about floating-point arithmetic",
 * 1991, theorem 4); the log comes from the hardware log2 and the quotient
 * from the hardware reciprocal, 1 ulp each, so a few ulps in all. */
__device__ __forceinline__ float log1p_pos(float y) {
	float p = fmaf(y, -1.0f / 6.0f, 0.2f);
	p = fmaf(y, p, -0.25f);
	p = fmaf(y, p, 1.0f / 3.0f);
	p = fmaf(y, p, -0.5f);
	p = fmaf(y, p, 1.0f);
	const float u = 1.0f + y;
	const float big = __builtin_amdgcn_logf(u) * SMX_LN2 * (y * __builtin_amdgcn_rcpf(u - 1.0f));
	return (y < 0.03125f) ? y * p : big;
}

/* The fused loss -log p_label = log(sum_j exp(x_j - m)) + m - x_label, from
 * `others` = the sum of exp(x_j - m) over every column but the label's, the
 * row max m and the labelled logit xl. While the label is within 16 of the
 * max it is log1p(others * exp(m - xl)): a row the label wins by far has a
 * loss of about `others`, which log(1 + others) in fp32 would round away
 * below 2^-24 (and lose relative precision well above that). Further down
 * it is log(others + exp(xl - m)) + (m - xl), where others >= 1 (the max's
 * own column is among them), so the hardware log2 is accurate there; NaN
 * and infinite inputs take that form too. */
__device__ __forceinline__ float fused_loss(float others, float m, float xl) {
	const float gap = m - xl;
	const float near = log1p_pos(others * __builtin_amdgcn_exp2f(gap * SMX_LOG2E));
	const float far = fmaf(__builtin_amdgcn_logf(others + __builtin_amdgcn_exp2f(-gap * SMX_LOG2E)), SMX_LN2, gap);
	return (gap < 16.0f) ? near : far;
}

template <typename T> __device__ __forceinline__ float rnd_in(float f) { return to_f(from_f<T>(f)); }

/* Block reductions: each wave's partial goes to its LDS cell, one barrier,
 * then every thread reads all cells (in wave order, so the result does not
 * depend on timing). A caller reusing the same cells must make sure every
 * wave has finished reading them first. */
__device__ __forceinline__ float block_max(float v, float * slots) {
	v = wave_max(v);
	const int nw = blockDim.x >> 6;
	if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
	lds_barrier();
	float m = slots[0];
	for (int w = 1; w < nw; w++) m = fmaxf(m, slots[w]);
	return m;
}

__device__ __forceinline__ void block_sum2(float & a, float & b, float * slots) {
	a = wave_sum(a);
	b = wave_sum(b);
	const int nw = blockDim.x >> 6;
	if ((threadIdx.x & 63) == 0) { slots[threadIdx.x >> 6] = a; slots[16 + (threadIdx.x >> 6)] = b; }
	lds_barrier();
	float sa = 0.0f, sb = 0.0f;
	for (int w = 0; w < nw; w++) { sa += slots[w]; sb += slots[16 + w]; }
	a = sa;
	b = sb;
}

/* Reductions of the register-row path, which keeps direct-to-LDS loads of
 * the next row in flight across them. The compiler cannot tell that those
 * loads write other LDS cells than the reduction's, so a fenced barrier or a
 * plain LDS read after it would first wait for every outstanding vector-memory
 * access (vmcnt 0), stalling on the prefetch. Here each wave's partial is
 * published with an explicit LDS wait + s_barrier and the cells are read back
 * with ds_read_b128 issued from inline assembly (each followed by its own
 * lgkmcnt wait), so only LDS traffic is waited for. The cells (16-byte
 * aligned, one per wave of SMX_THREADS) never overlap the prefetch buffer. */
typedef float f32x4_v __attribute__((ext_vector_type(4)));
constexpr int SMX_WAVES = SMX_THREADS / 64;
static_assert(SMX_WAVES % 4 == 0, "cells are read four at a time");

__device__ __forceinline__ void cells_barrier() {
	__asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ f32x4_v cells_read4(const float * cell) {
	const uint32_t a = (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) float *) cell;
	f32x4_v v;
	__asm__ volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
	return v;
}
/* same results, combined in the same wave order, as block_max / block_sum2 */
__device__ __forceinline__ float cells_max(float v, float * cells) {
	v = wave_max(v);
	if ((threadIdx.x & 63) == 0) cells[threadIdx.x >> 6] = v;
	cells_barrier();
	float m = -__builtin_inff();
#pragma unroll
	for (int w = 0; w < SMX_WAVES; w += 4) {
		const f32x4_v c = cells_read4(cells + w);
		m = fmaxf(fmaxf(m, c.x), fmaxf(c.y, c.z));
		m = fmaxf(m, c.w);
	}
	return m;
}
__device__ __forceinline__ void cells_sum2(float & a, float & b, float * cells) {
	a = wave_sum(a);
	b = wave_sum(b);
	if ((threadIdx.x & 63) == 0) { cells[threadIdx.x >> 6] = a; cells[SMX_WAVES + (threadIdx.x >> 6)] = b; }
	cells_barrier();
	float sa = 0.0f, sb = 0.0f;
#pragma unroll
	for (int w = 0; w < SMX_WAVES; w += 4) {
		const f32x4_v ca = cells_read4(cells + w);
		const f32x4_v cb = cells_read4(cells + SMX_WAVES + w);
		sa += ca.x; sa += ca.y; sa += ca.z; sa += ca.w;
		sb += cb.x; sb += cb.y; sb += cb.z; sb += cb.w;
	}
	a = sa;
	b = sb;
}

/* Launch-wide state of the softmax kernels, one copy per loaded code object
 * (per handle): SMX_TICKETS counts the rows handed out beyond each
 * workgroup's first two, SMX_DONE the workgroups that have finished. Both
 * are zero between launches: the last workgroup to finish resets them. The
 * handle orders these ops across its streams, so two launches never share
 * them. The two counters sit in different 128-byte lines. */
#define SMX_TICKETS 0
#define SMX_DONE 32
__device__ unsigned int g_smx_sched[64];

/* a row's loss, stored at device scope: the workgroup that sums the mean
 * loss may run on another XCD, whose L2 does not see this one's lines */
__device__ __forceinline__ void store_loss(float * loss, int row, float v) {
	__hip_atomic_store(loss + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* End of every softmax launch. Each workgroup counts itself done once its
 * loss stores have completed (thread 0 made them and waits for them); the
 * last one sums mean_loss = sum_r loss[r] / n_rows in fp64 in a fixed order
 * (thread t takes rows t, t + blockDim, ...; then the waves in order), reading
 * the losses at device scope, and resets the counters for the next launch.
 * No workgroup waits for another. */
template <bool FUSED>
__device__ __forceinline__ void smx_launch_end(int n_rows, const float * loss, float * mean_loss) {
	__shared__ int is_last;
	__shared__ double dslots[SMX_THREADS / 64];
	if (threadIdx.x == 0) {
		__asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
		const unsigned d = __hip_atomic_fetch_add(&g_smx_sched[SMX_DONE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		is_last = (d == gridDim.x - 1u);
	}
	__syncthreads();
	if (!is_last) return;
	if (FUSED && loss && mean_loss) {
		__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
		double s = 0.0;
		for (int r = threadIdx.x; r < n_rows; r += blockDim.x) s += (double) __hip_atomic_load(loss + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
		if ((threadIdx.x & 63) == 0) dslots[threadIdx.x >> 6] = s;
		__syncthreads();
		if (threadIdx.x == 0) {
			double t = 0.0;
			for (int w = 0; w < (int) (blockDim.x >> 6); w++) t += dslots[w];
			*mean_loss = (float) (t / (double) n_rows);
		}
	}
	if (threadIdx.x == 0) {
		__hip_atomic_store(&g_smx_sched[SMX_TICKETS], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		__hip_atomic_store(&g_smx_sched[SMX_DONE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
	}
}

/* One 32-bit word of a row in storage type T: N elements. `diff` rounds
 * x - m to T (packed, exactly as the reference's in-type subtraction) and also
 * returns the unrounded differences and the rounded values as floats; the
 * packed word is kept, so the output pass needs no repacking. */
template <typename T> struct SmxWord;
template <> struct SmxWord<bf16_t> {
	static constexpr int N = 2;
	static constexpr uint32_t NEG_INF = 0xff80ff80u;
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
	static constexpr uint32_t NEG_INF = 0xfc00fc00u;
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
	/* the same rnd(x - m) in one packed fp16 subtraction: m is an fp16
	 * value, and rounding the exact difference once to fp16 equals rounding
	 * it to fp32 first (24 >= 2 * 11 + 2 bits) */
	__device__ static __forceinline__ uint32_t diff_pk(uint32_t w, float m, float * d) {
		const _Float16 mh = (_Float16) m;
		const f16x2_v dv = __builtin_bit_cast(f16x2_v, w) - (f16x2_v){mh, mh};
		d[0] = (float) dv.x;
		d[1] = (float) dv.y;
		return __builtin_bit_cast(uint32_t, dv);
	}
};
template <> struct SmxWord<float> {
	static constexpr int N = 1;
	static constexpr uint32_t NEG_INF = 0xff800000u;
	__device__ static __forceinline__ void unpack(uint32_t w, float * f) { f[0] = __uint_as_float(w); }
	__device__ static __forceinline__ uint32_t pack(const float * f) { return __float_as_uint(f[0]); }
	__device__ static __forceinline__ uint32_t diff(uint32_t w, float m, float * x_m, float * d) {
		x_m[0] = __uint_as_float(w) - m;
		d[0] = x_m[0];
		return __float_as_uint(d[0]);
	}
};

template <typename T> struct IsF16 { static constexpr bool value = false; };
template <> struct IsF16<f16_t> { static constexpr bool value = true; };

/* fp16 chunks in the max pass: the chunk's max from packed 3-input maxima
 * (NaN-propagating like the fp32 one), and x - c in one rounding straight
 * from the packed word's low or high half (the mixed-precision fma x * 1 - c;
 * written out because the compiler turns fma(x, 1, c) into a conversion and
 * a subtraction) */
__device__ __forceinline__ float f16_chunk_max(const R16 & r, float m) {
	const f16x2_v a = __builtin_bit_cast(f16x2_v, r.w[0]), b = __builtin_bit_cast(f16x2_v, r.w[1]);
	const f16x2_v c = __builtin_bit_cast(f16x2_v, r.w[2]), d = __builtin_bit_cast(f16x2_v, r.w[3]);
	const f16x2_v mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), __builtin_elementwise_maximum(c, d));
	return __builtin_elementwise_maximum(m, __builtin_elementwise_maximum((float) mx.x, (float) mx.y));
}
__device__ __forceinline__ float f16_lo_minus(uint32_t w, float negc) {
	float r;
	__asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(negc));
	return r;
}
__device__ __forceinline__ float f16_hi_minus(uint32_t w, float negc) {
	float r;
	__asm__("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(negc));
	return r;
}

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
 * whole row sits in VGPRs. The next row is requested chunk by chunk during
 * this row's max pass and lands while it computes: its first SMX_PF chunks go
 * straight into LDS (16-byte buffer loads with the LDS bit), the others into
 * registers, and the fused op's next label into an LDS cell (a 4-byte LDS
 * load per wave). The labelled logit is copied out of the registers of the
 * thread holding it during the max pass, before the row is overwritten in
 * place, and reaches thread 0 (which writes the loss) through an LDS cell.
 * Each wave prefetches into and reads from its own LDS slice only, so no
 * workgroup barrier guards the buffer, and the reductions' barriers wait for
 * LDS only: the one wait for memory in a row comes after its output
 * stores. */
template <typename T, typename TO, bool FUSED>
__device__ __forceinline__ void smx_regs(int n_rows, int n_cols, const T * X, TO * out, const uint32_t * labels, float * loss) {
	constexpr int VEC = VecOf<T>::N;
	using W = SmxWord<T>;
	using WO = SmxWord<TO>;
	static_assert(sizeof(T) == sizeof(TO), "in-register output packing needs equal widths");
	/* the fused fp16 kernel works on the packed halves where it can (fewer
	 * conversions: fused 4096 x 128256 400.4 -> 370.0 us, outputs
	 * bit-identical); the plain softmax, which is not held up by its
	 * arithmetic, measured 363.2 -> 365.2 us that way and keeps the
	 * conversions */
	constexpr bool F16 = IsF16<T>::value && FUSED;
	/* the loss needs sx = sum exp(x - m) over the unrounded differences and
	 * without the label's column (fused_loss); that is not the softmax's sum,
	 * so it is accumulated separately, for every storage type */
	constexpr bool SX = FUSED;
	/* separate LDS cells for the max and the sum: each is rewritten only after
	 * every wave has passed the other reduction's barrier, so reuse needs no
	 * barrier of its own (two barriers per row) */
	__shared__ __attribute__((aligned(16))) float mslots[SMX_WAVES];
	__shared__ __attribute__((aligned(16))) float sslots[2 * SMX_WAVES];
	__shared__ __attribute__((aligned(16))) R16 pf[SMX_PF * SMX_THREADS];
	/* a row's label, one cell per wave: each wave loads its own copy, so its
	 * own wait for memory covers it (a load issued by one wave is not waited
	 * for by the others) */
	__shared__ uint32_t labcell[SMX_WAVES];
	/* the labelled logit, written by the thread holding it during the max
	 * pass and read by thread 0 after the sum reduction's barrier; two cells
	 * by row parity, since the next row's writer can run ahead of thread 0's
	 * read by up to one row (never two: the next row's sum barrier comes first) */
	__shared__ float xlab_cell[2];
	const int tid = threadIdx.x;
	constexpr int nt = SMX_THREADS;          /* the launch guarantees blockDim.x == SMX_THREADS */
	static_assert((nt & (nt - 1)) == 0, "power-of-two workgroup");
	constexpr uint32_t cstride = nt * 16u;   /* chunk stride: an immediate, rematerialised per use */
	const int wave_base = tid & ~63;
	const int lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int nv = n_cols / VEC;
	const int nch = (nv + nt - 1) / nt;
	const uint32_t row_bytes = (uint32_t) n_cols * (uint32_t) sizeof(T);
	const uint32_t voff = (uint32_t) tid * 16u;
	const uint64_t lab_bytes = FUSED ? (uint64_t) n_rows * 4u : 0u;
	const __amdgpu_buffer_rsrc_t rlab = make_rsrc(labels, (uint32_t) (lab_bytes < 0xffffffffull ? lab_bytes : 0xffffffffull));
	/* 4-byte loads straight into LDS from lane 0 only (lane l would write
	 * the cell at 4 l) */
	auto fetch_label = [&](int r) {
		if (FUSED && lane == 0)
			__builtin_amdgcn_raw_ptr_buffer_load_lds(rlab, (lds_ptr_t) &labcell[wave], 4, 0u, (uint32_t) r * 4u, 0, 0);
	};

	/* chunks SMX_PF .. SMX_PF + RP - 1 of the next row are loaded a row ahead
	 * into VGPRs; fp32 rows keep those registers for temporaries and load the
	 * chunks past SMX_PF + RP at the top of their own row */
	constexpr int RP = sizeof(T) < 4 ? SMX_MAXCH - SMX_PF : 0;
	int row = blockIdx.x;
	int par = 0;
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
		fetch_label(row);
	}
	WAIT_VMEM_ALL();
	/* Rows: each workgroup's first two are block and block + grid; every later
	 * one is a ticket t of the launch's row counter, row 2 * grid + t. The
	 * ticket for the row after next is taken at the top of each row by thread
	 * 0, which writes that row's index to an LDS cell at once; the other waves
	 * read it after the sum reduction's barrier, so the next row's index is
	 * known when its prefetch starts in the max pass. The cell by row parity
	 * was last read two rows back. Writing it at once keeps the ticket out of
	 * the registers for the rest of the row: kept until the sum pass, it made
	 * the fp16 fused kernel spill a prefetched chunk, whose spill waits for
	 * every outstanding load (4096 x 128256: 412.6 -> 400.4 us; bf16 and the
	 * softmax unchanged, outputs bit-identical). */
	__shared__ int nextcell[2];
	int next = row + (int) gridDim.x;
	while (row < n_rows) {
		if (tid == 0) {
			int r2 = n_rows;
			if (next < n_rows) {
				const uint32_t t = __hip_atomic_fetch_add(&g_smx_sched[SMX_TICKETS], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
				const uint32_t r = 2u * gridDim.x + t;
				r2 = r < (uint32_t) n_rows ? (int) r : n_rows;
			}
			nextcell[par] = r2;
		}
		const __amdgpu_buffer_rsrc_t rout = make_rsrc(out + (long) row * n_cols, row_bytes);
		/* this row: its label and the LDS part (landed: checked before the last
		 * output pass) and the register part loaded during the last row */
		const uint32_t lab = FUSED ? labcell[wave] : 0xffffffffu;
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
		/* the next row (requested during the max pass) and its label */
		const bool has_next = next < n_rows;
		const bool lab_ok = FUSED && lab < (uint32_t) n_cols;
		const __amdgpu_buffer_rsrc_t rn = make_rsrc(X + (long) next * n_cols, has_next ? row_bytes : 0u);
		auto issue_next = [&](int c) {
			if (has_next && c < nch) {
				if (c < SMX_PF) __builtin_amdgcn_raw_ptr_buffer_load_lds(rn, (lds_ptr_t) &pf[c * nt + wave_base], 16, voff, c * cstride, 0, BUF_AUX_NT);
				else if (c < SMX_PF + RP) nx[c - SMX_PF] = buf_load16_nt(rn, voff, c * cstride);
			}
		};
		if (has_next) fetch_label(next);

		/* the last chunk's lanes past the row end (zeros from the range check)
		 * become -inf, which leaves the max and both sums unchanged, so the
		 * passes below need no per-lane mask */
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			if (c == nch - 1 && c * nt + tid >= nv) {
#pragma unroll
				for (int i = 0; i < 4; i++) xr[c].w[i] = W::NEG_INF;
			}
		}

		/* the label sits in chunk c_lab (workgroup-uniform) of thread t_lab,
		 * element le */
		const int lab_chunk = lab_ok ? (int) (lab / VEC) : 0;
		const int c_lab = lab_ok ? lab_chunk / nt : -1;
		const int t_lab = lab_chunk & (nt - 1);
		const int le = (int) (lab % VEC);

		/* max pass. The next row is requested in two parts: its register part
		 * here, its LDS part during the sum pass. Requests made here queue
		 * behind the previous row's stores, which are still draining; the sum
		 * pass is arithmetic that would otherwise leave this CU's memory
		 * pipeline idle once the register part has landed (measured on
		 * MI355X: 4096 x 128256 bf16, fused 397 -> 385 us, softmax 393 ->
		 * 386 us, against every other split of the two parts over the two
		 * passes). Each request sits just before this row's chunk c is used
		 * (the scheduling barrier keeps that order), so the waves compute
		 * while the memory pipeline accepts them. For the loss, sx is summed
		 * in the same pass online: so = sum exp(x - mref) against a reference
		 * that trails the running max by at most 64, rescaled when it moves.
		 * (Summing it in the sum pass instead, from exp(d) corrected
		 * for the rounding of x - m, measured 7 us faster to first order but
		 * misses the 1e-4 loss bound on confident rows, and 28 us slower to
		 * second order: that pass is already the kernel's busiest.) */
		float m = -__builtin_inff();
		/* mref: the online sum's reference, a placeholder 0 until the lane
		 * has seen a finite value; mref64 = mref + 64, -inf until then */
		float mref = 0.0f, mref64 = -__builtin_inff(), so = 0.0f;
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			if (c >= SMX_PF) issue_next(c);
			__builtin_amdgcn_sched_barrier(0);
			if (c < nch) {
				/* the chunk as floats (fp16: only where the label is read;
				 * its max and terms come from the packed words) */
				float f[VEC];
				float cm = m;
				if constexpr (F16) cm = f16_chunk_max(xr[c], m);
				else {
					unpack16<T>(xr[c], f);
#pragma unroll
					for (int e = 0; e < VEC; e++) cm = __builtin_elementwise_maximum(cm, f[e]);
				}
				/* the raw labelled logit, for the loss (a workgroup-uniform
				 * chunk test, then one thread) */
				const bool lab_here = FUSED && c == c_lab && tid == t_lab;
				if (lab_here) {
					if constexpr (F16) unpack16<T>(xr[c], f);
					float xl = f[0];
#pragma unroll
					for (int e = 1; e < VEC; e++)
						if (e == le) xl = f[e];
					xlab_cell[par] = xl;
				}
				if (SX) {
					/* the reference moves only when this lane's max passes it
					 * by more than 64 (rare after the first chunk: a
					 * wave-uniform branch), so the terms stay below e^64 and
					 * 128 of them cannot overflow; measured 382.2 -> 380.8 us
					 * against moving it every chunk */
					const bool move = cm > mref64;
					if (__builtin_amdgcn_ballot_w64(move)) {
						so = move ? so * online_rescale(mref, cm) : so;
						mref = move ? cm : mref;
						mref64 = move ? cm + 64.0f : mref64;
					}
					float t[VEC];
#pragma unroll
					for (int e = 0; e < VEC; e++) {
						float x_mref;
						if constexpr (F16) x_mref = (e & 1) ? f16_hi_minus(xr[c].w[e >> 1], -mref) : f16_lo_minus(xr[c].w[e >> 1], -mref);
						else x_mref = f[e] - mref;
						t[e] = __builtin_amdgcn_exp2f(x_mref * SMX_LOG2E);
					}
					/* the loss sum leaves the label's column out (the max has
					 * it); the terms are cleared, not f, which for fp32 is the
					 * row itself and must stay as loaded */
					if (lab_here) {
#pragma unroll
						for (int e = 0; e < VEC; e++)
							if (e == le) t[e] = 0.0f;
					}
#pragma unroll
					for (int e = 0; e < VEC; e++) so += t[e];
				}
				m = cm;
			}
		}
		m = cells_max(m, mslots);
		if (SX) so *= online_rescale(mref, m);   /* sx against the row max */
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) reg_barrier(xr[c]);

		/* sum pass: sd = sum exp(d) with d = rnd(x - m); the next row's LDS
		 * part is requested here, chunk c before this row's chunk c (its
		 * slots were emptied into xr at the top of this row) */
		float sd0 = 0.0f, sd1 = 0.0f;
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			if (c < SMX_PF) issue_next(c);
			__builtin_amdgcn_sched_barrier(0);
			if (c < nch) {
				R16 o;
#pragma unroll
				for (int i = 0; i < 4; i++) {
					float x_m[W::N], d[W::N];
					if constexpr (F16) o.w[i] = W::diff_pk(xr[c].w[i], m, d);
					else o.w[i] = W::diff(xr[c].w[i], m, x_m, d);
#pragma unroll
					for (int e = 0; e < W::N; e++) {
						/* fp16: d * log2(e) from the packed half (mixed fma) */
						const float ex = F16 ? __builtin_amdgcn_exp2f(fmaf(d[e], SMX_LOG2E, 0.0f)) : exp_fast(d[e]);
						if ((i * W::N + e) & 1) sd1 += ex; else sd0 += ex;
					}
				}
				xr[c] = o;   /* d, exact in T */
			}
		}
		float sd = sd0 + sd1;
		float sx = SX ? so : sd;
		cells_sum2(sd, sx, sslots);
		const int next2 = __builtin_amdgcn_readfirstlane(nextcell[par]);
		/* y = exp(d) / sd as one exp2: exp2(d * log2(e) - log2(sd)) */
		const float nlog2s = -__builtin_amdgcn_logf(sd);
#pragma unroll
		for (int c = 0; c < SMX_MAXCH; c++) {
			/* every lane issues all SMX_MAXCH stores (chunks past the row lie
			 * outside its buffer range and store nowhere), so the wait below
			 * can count them */
			{
				R16 o;
#pragma unroll
				for (int i = 0; i < 4; i++) {
					float f[W::N];
					W::unpack(xr[c].w[i], f);
#pragma unroll
					for (int e = 0; e < W::N; e++) f[e] = __builtin_amdgcn_exp2f(fmaf(f[e], SMX_LOG2E, nlog2s));
					o.w[i] = WO::pack(f);
				}
				/* the label's chunk (a workgroup-uniform branch), in one thread */
				if (FUSED && c == c_lab && tid == t_lab) {
#pragma unroll
					for (int i = 0; i < 4; i++) {
						float f[W::N];
						WO::unpack(o.w[i], f);
#pragma unroll
						for (int e = 0; e < W::N; e++)
							if (i * W::N + e == le) f[e] -= 1.0f;
						o.w[i] = WO::pack(f);
					}
				}
				buf_store16_nt(rout, voff, c * cstride, o);
			}
		}
		/* in flight here, oldest first: the rest of the previous row's stores,
		 * the next row's loads (issued during the max and sum passes) and
		 * this row's SMX_MAXCH stores. Completions are in order, so waiting
		 * until at most SMX_MAXCH remain means the next row's LDS part and
		 * label have landed before that row reads them, while this row's
		 * stores drain behind it; waiting before the output pass instead held
		 * the pass up until the LDS part requested during the sum pass had
		 * arrived. */
		static_assert(SMX_MAXCH == 16, "the wait below counts SMX_MAXCH stores");
		__builtin_amdgcn_s_waitcnt(0x4F70);   /* vmcnt(16); expcnt, lgkmcnt at their maxima */
		if (FUSED && tid == 0 && loss) store_loss(loss, row, lab_ok ? fused_loss(sx, m, xlab_cell[par]) : __builtin_nanf(""));
		par ^= 1;
		row = next;
		next = next2;
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
			if (FUSED && (uint32_t) j != lab) sx += exp_fast(diff);
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
			store_loss(loss, row, (lab < (uint32_t) n_cols) ? fused_loss(sx, m, x_lab) : __builtin_nanf(""));
		}
		__syncthreads();
	}
}

/* Rows longer than the register path holds (more than SMX_MAXCH 16-byte
 * chunks per thread), 16-byte aligned: streaming passes over the row with
 * 16-byte accesses. The first pass finds the row max and, online, the sum of
 * exp(x - m) over the unrounded differences (each thread keeps its running
 * max and its sum against it, rescaled when the max grows; mref = 0 while the
 * max is still -inf; the workgroup combines them against the row max). In
 * fp32, x - m is not rounded, so that sum is the softmax's and two passes
 * suffice; fp16/bf16 round x - m to the storage type first, so a second pass
 * sums exp(rnd(x - m)) against the final max (the first pass's sum is then
 * the fused loss's). The last pass writes the outputs with the register
 * path's expressions. Reads before the last use the default cache policy, so
 * the later passes find the row in cache where they can. The labelled logit
 * is taken from the first pass's registers by the thread holding it (the last
 * pass may overwrite the row in place). */
template <typename T, bool FUSED>
__device__ __forceinline__ void smx_stream_vec(int n_rows, int n_cols, const T * X, T * out, const uint32_t * labels, float * loss) {
	constexpr int U = 4;
	constexpr int VEC = VecOf<T>::N;
	constexpr bool ROUNDS = sizeof(T) < 4;
	/* The first HG groups of UH chunks per thread stay in registers from the
	 * first pass to the last, so only the rest of the row is read again:
	 * fp32 16 chunks (256 KB of the row per workgroup; fused 4096 x 128256
	 * 879.6 -> 787.6 us, softmax 867.9 -> 750.3 us), 16-bit rows 8 chunks in
	 * the softmax and 6 in the fused kernel, whose label and loss state leave
	 * fewer registers (8 spilled there); held groups of two chunks, so the
	 * first pass's working set stays small (4096 x 151936: bf16 fused 660.9
	 * -> 591.1 us, softmax 651.1 -> 563.5 us, fp16 665.1 -> 588.5 and 654.3
	 * -> 559.8 us). The outputs are bit-identical; the loss sum is rescaled
	 * at other chunks, so a loss can differ in its last bits. */
	constexpr int HG = sizeof(T) == 4 ? 4 : (FUSED ? 3 : 4);
	constexpr int UH = sizeof(T) == 4 ? U : 2;   /* chunks per held group */
	__shared__ float slots[32];
	__shared__ float xlab_cell;
	__shared__ int nextcell;
	const int tid = threadIdx.x;
	const int nt = blockDim.x;
	const int nv = n_cols / VEC;
	const uint32_t row_bytes = (uint32_t) n_cols * (uint32_t) sizeof(T);
	/* Rows are handed out as workgroups free up: each workgroup's first row
	 * is its block index, every later one a ticket t of the launch's row
	 * counter, row grid + t. Thread 0 requests the ticket for the next row
	 * right after the row's held chunks and writes the row's index to an LDS
	 * cell at once: the row's end waited for all memory traffic, so its wait
	 * for the atomic's return is its wait for those chunks, which the first
	 * pass uses next (holding the ticket through that pass instead spilled
	 * registers in the fused kernels). The max reduction's barrier publishes
	 * the cell. Against fixed rows (block, block + grid, ...): fp32 4096 x
	 * 128256 fused 785.2 -> 763.3 us and softmax 751.4 -> 725.9 us, bf16
	 * 4096 x 151936 softmax 566.3 -> 557.1 us, outputs identical. */
	int row = blockIdx.x;
	while (row < n_rows) {
		const __amdgpu_buffer_rsrc_t rin = make_rsrc(X + (long) row * n_cols, row_bytes);
		const __amdgpu_buffer_rsrc_t rout = make_rsrc(out + (long) row * n_cols, row_bytes);
		const uint32_t lab = FUSED ? labels[row] : 0xffffffffu;
		const bool lab_ok = FUSED && lab < (uint32_t) n_cols;
		const int c_lab = lab_ok ? (int) (lab / VEC) : -1;
		const int le = (int) (lab % VEC);
		/* pass 1: max and the online sum of exp(x - m) */
		float m = -__builtin_inff(), mref = 0.0f, s = 0.0f;
		auto pass1 = [&](auto & v, int base) {
			constexpr int U = sizeof(v) / sizeof(R16);
			float f[U][VEC];
			float cm = m;
#pragma unroll
			for (int k = 0; k < U; k++) {
				const int c = base + k * nt + tid;
				unpack16<T>(v[k], f[k]);
#pragma unroll
				for (int e = 0; e < VEC; e++) {
					if (c >= nv) f[k][e] = -__builtin_inff();
					cm = fmaxf(cm, f[k][e]);
				}
			}
			/* the max is taken before the label branch rewrites f (else the
			 * original and rewritten f are both live: register copies on
			 * every thread) */
			if (FUSED) __asm__ volatile("" : "+v"(cm));
			/* the thread holding the label keeps its logit and leaves its
			 * column out of the loss sum (the max above has it); written as
			 * a select per element inside the branch, so f stays in
			 * registers */
#pragma unroll
			for (int k = 0; k < U; k++) {
				if (FUSED && base + k * nt + tid == c_lab) {
					float xl = f[k][0];
#pragma unroll
					for (int e = 1; e < VEC; e++)
						if (e == le) xl = f[k][e];
					xlab_cell = xl;
#pragma unroll
					for (int e = 0; e < VEC; e++)
						if (e == le) f[k][e] = -__builtin_inff();
				}
			}
			const float mr = (cm == -__builtin_inff()) ? 0.0f : cm;
			s *= online_rescale(mref, mr);
#pragma unroll
			for (int k = 0; k < U; k++) {
#pragma unroll
				for (int e = 0; e < VEC; e++) s += __builtin_amdgcn_exp2f((f[k][e] - mr) * SMX_LOG2E);
			}
			mref = mr;
			m = cm;
		};
		R16 hold[HG][UH];
		/* the held groups are read once (streaming hint), all requested
		 * before the first is used; the rest with the default policy, so the
		 * later passes find them in cache where they can */
#pragma unroll
		for (int g = 0; g < HG; g++)
#pragma unroll
			for (int k = 0; k < UH; k++) hold[g][k] = buf_load16_nt(rin, (uint32_t) (g * nt * UH + k * nt + tid) * 16u, 0);
		if (tid == 0) {
			const uint32_t r = gridDim.x + __hip_atomic_fetch_add(&g_smx_sched[SMX_TICKETS], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
			nextcell = r < (uint32_t) n_rows ? (int) r : n_rows;
		}
#pragma unroll
		for (int g = 0; g < HG; g++)
			if (g * nt * UH < nv) pass1(hold[g], g * nt * UH);
		for (int base = HG * nt * UH; base < nv; base += nt * U) {
			R16 v[U];
#pragma unroll
			for (int k = 0; k < U; k++) v[k] = buf_load16(rin, (uint32_t) (base + k * nt + tid) * 16u, 0);
			pass1(v, base);
		}
		const float mx = block_max(m, slots);
		const int next = __builtin_amdgcn_readfirstlane(nextcell);
		float sx = s * online_rescale(mref, mx);
		/* pass 2 (fp16/bf16): sd = sum exp(rnd(x - mx)) */
		float sd = 0.0f;
		if (ROUNDS) {
			auto pass2 = [&](auto & v, int base) {
				constexpr int U = sizeof(v) / sizeof(R16);
#pragma unroll
				for (int k = 0; k < U; k++) {
					if (base + k * nt + tid < nv) {
						float f[VEC];
						unpack16<T>(v[k], f);
#pragma unroll
						for (int e = 0; e < VEC; e++) sd += exp_fast(rnd_in<T>(f[e] - mx));
					}
				}
			};
#pragma unroll
			for (int g = 0; g < HG; g++)
				if (g * nt * UH < nv) pass2(hold[g], g * nt * UH);
			for (int base = HG * nt * UH; base < nv; base += nt * U) {
				R16 v[U];
#pragma unroll
				for (int k = 0; k < U; k++) v[k] = buf_load16(rin, (uint32_t) (base + k * nt + tid) * 16u, 0);
				pass2(v, base);
			}
		}
		__syncthreads();   /* every wave has read the max cells */
		block_sum2(sx, sd, slots);
		/* fp32: the softmax's sum is the loss sum plus the label's term */
		if (!ROUNDS) sd = sx + (lab_ok ? __builtin_amdgcn_exp2f((xlab_cell - mx) * SMX_LOG2E) : 0.0f);
		const float nlog2s = -__builtin_amdgcn_logf(sd);
		/* last pass: y = exp(rnd(x - mx)) / sd */
		auto pass3 = [&](auto & v, int base) {
			constexpr int U = sizeof(v) / sizeof(R16);
#pragma unroll
			for (int k = 0; k < U; k++) {
				const int c = base + k * nt + tid;
				float f[VEC];
				unpack16<T>(v[k], f);
#pragma unroll
				for (int e = 0; e < VEC; e++) f[e] = __builtin_amdgcn_exp2f(fmaf(rnd_in<T>(f[e] - mx), SMX_LOG2E, nlog2s));
				R16 o = pack16<T>(f);
				if (c == c_lab) {   /* the label element: rnd(y) - 1 */
					unpack16<T>(o, f);
					f[le] -= 1.0f;
					o = pack16<T>(f);
				}
				buf_store16_nt(rout, (uint32_t) c * 16u, 0, o);
			}
		};
#pragma unroll
		for (int g = 0; g < HG; g++)
			if (g * nt * UH < nv) pass3(hold[g], g * nt * UH);
		for (int base = HG * nt * UH; base < nv; base += nt * U) {
			R16 v[U];
#pragma unroll
			for (int k = 0; k < U; k++) v[k] = buf_load16_nt(rin, (uint32_t) (base + k * nt + tid) * 16u, 0);
			pass3(v, base);
		}
		if (FUSED && tid == 0 && loss) store_loss(loss, row, lab_ok ? fused_loss(sx, mx, xlab_cell) : __builtin_nanf(""));
		__syncthreads();   /* the cells are rewritten for the next row */
		row = next;
	}
}

template <typename T, typename TO, bool FUSED>
__device__ __forceinline__ void smx(int n_rows, int n_cols, const T * X, TO * out, const uint32_t * labels, float * loss, float * mean_loss) {
	constexpr int VEC = VecOf<T>::N;
	const bool vec_ok = (n_cols % VEC == 0) && aligned16(X) && aligned16(out) && blockDim.x == SMX_THREADS
						&& ((n_cols / VEC + SMX_THREADS - 1) / SMX_THREADS) <= SMX_MAXCH;
	if (vec_ok) smx_regs<T, TO, FUSED>(n_rows, n_cols, X, out, labels, loss);
	else if (sizeof(TO) == sizeof(T) && n_cols % VEC == 0 && aligned16(X) && aligned16(out) && blockDim.x == SMX_THREADS)
		smx_stream_vec<T, FUSED>(n_rows, n_cols, X, reinterpret_cast<T *>(out), labels, loss);
	else smx_stream<T, TO, FUSED>(n_rows, n_cols, X, out, labels, loss);
	smx_launch_end<FUSED>(n_rows, loss, mean_loss);
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
