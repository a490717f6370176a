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
 * same-type kernels' (swiglu_bwd_elem; bwd_x_elem's formula, with the division
 * by n taken as a multiplication by 1/n on the chunked path); the dW partial
 * rows and their finish pass are rms_norm.hip's.
 */
#include "dtypes.h"
#include "reduce.h"
#include "kernel_geometry.h"

typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_v;

__device__ __forceinline__ R8 ld8(const void * p) {
	const u32x2_v v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_v *>(p));
	R8 r;
	r.w[0] = v.x;
	r.w[1] = v.y;
	return r;
}

__device__ __forceinline__ bool aligned8(const void * p) { return (((uintptr_t) p) & 7u) == 0; }

__device__ __forceinline__ void reg_barrier8(R8 & r) { __asm__ volatile("" : "+v"(r.w[0]), "+v"(r.w[1])); }

/* ---------------- RMSNorm backward: row slots ---------------- */

/* One row's operands for a thread: its F8_CPT chunks of X (8 bytes each) and
 * dY / dX (16 bytes each), and the row's statistics. */
struct F8Row {
	R8 x[F8_CPT];
	R16 g[F8_CPT], d[F8_CPT];
	float r, ws;
};

/* Issue the loads of `row` (nothing past the last row or the row's end). */
template <bool BWD_X>
__device__ __forceinline__ void f8_load_row(int row, int n_rows, int cpr, int tr, int tpr, const uint8_t * X, const uint16_t * dY,
											const uint16_t * dX, const float * rs_in, const float * ws_in, F8Row & o) {
	if (row >= n_rows) return;
	const long base = (long) row * cpr;
#pragma unroll
	for (int k = 0; k < F8_CPT; k++) {
		const int c = tr + k * tpr;
		if (c < cpr) {
			o.x[k] = ld8(X + 8 * (base + c));
			o.g[k] = ld16_nt(dY + 8 * (base + c));
			if (BWD_X) o.d[k] = ld16_nt(dX + 8 * (base + c));
		}
	}
	o.r = rs_in[row];
	if (BWD_X) o.ws = ws_in[row];
}

/* Row slots: workgroup b runs blockDim / tpr slots, slot s taking rows
 * b * S + s, then every gridDim * S rows further, with the next row's loads
 * issued before the current row is computed. */
struct F8Slots {
	int tpr, cpr, S, slot, tr, first, step;
	__device__ __forceinline__ F8Slots(int n_cols) {
		tpr = f8_row_tpr(n_cols);
		cpr = n_cols / 8;
		S = (int) blockDim.x / tpr;
		slot = (int) threadIdx.x / tpr;
		tr = (int) threadIdx.x % tpr;
		first = (int) blockIdx.x * S + slot;
		step = (int) gridDim.x * S;
	}
};

template <typename TF, typename TB>
__device__ __forceinline__ bool f8_rows_vec(int n_cols, const void * a, const void * b, const void * c, const void * d) {
	const int tpr = f8_row_tpr(n_cols);
	return tpr > 0 && (blockDim.x % tpr) == 0 && aligned8(a) && aligned8(b) && aligned16(c) && aligned16(d);
}

/* dX += rnd(dY * rnd(deriv)) (the reference formula, bwd_x_elem); W's
 * chunks are decoded once per thread. (x * r^3) / n is formed as
 * (x * r^3) * (1 / n), within the fp32 evaluation slack the parity bound
 * allows for deriv. */
template <typename TF, typename TB>
__device__ __forceinline__ void rms_bwd_x_fp8(int n_rows, int n_cols, const float * ws_in, const float * rs_in,
												const TF * W, const TF * X, const TB * dY, TB * dX) {
	if (f8_rows_vec<TF, TB>(n_cols, W, X, dY, dX)) {
		const F8Slots sl(n_cols);
		const uint8_t * X8 = reinterpret_cast<const uint8_t *>(X);
		const uint16_t * G16 = reinterpret_cast<const uint16_t *>(dY);
		uint16_t * D16 = reinterpret_cast<uint16_t *>(dX);
		float wf[F8_CPT][8];
#pragma unroll
		for (int k = 0; k < F8_CPT; k++) {
			const int c = sl.tr + k * sl.tpr;
			if (c < sl.cpr) unpack8_fp8<TF>(*reinterpret_cast<const R8 *>(W + 8 * c), wf[k]);
		}
		const float inv_n = 1.0f / (float) n_cols;
		F8Row cur;
		f8_load_row<true>(sl.first, n_rows, sl.cpr, sl.tr, sl.tpr, X8, G16, D16, rs_in, ws_in, cur);
		for (int row = sl.first; row < n_rows; row += sl.step) {
			vmem_wait_all();
			F8Row nxt;
			f8_load_row<true>(row + sl.step, n_rows, sl.cpr, sl.tr, sl.tpr, X8, G16, D16, rs_in, ws_in, nxt);
			const float r = cur.r, r3 = r * r * r, ws = cur.ws;
			/* dX is read and written back: stored at device scope through a
			 * buffer resource over the row (a slot's tpr is a multiple of 64,
			 * so a wave's lanes share the row) */
			const int wrow = __builtin_amdgcn_readfirstlane(row);
			const __amdgpu_buffer_rsrc_t rd = make_rsrc(D16 + (long) wrow * n_cols, (uint32_t) n_cols * 2u);
#pragma unroll
			for (int k = 0; k < F8_CPT; k++) {
				const int c = sl.tr + k * sl.tpr;
				if (c < sl.cpr) {
					float xf[8], gf[8], df[8];
					unpack8_fp8<TF>(cur.x[k], xf);
					unpack16<TB>(cur.g[k], gf);
					unpack16<TB>(cur.d[k], df);
#pragma unroll
					for (int e = 0; e < 8; e++) {
#pragma clang fp contract(off)
						const float deriv = wf[k][e] * r - ((xf[e] * r3) * inv_n) * ws;
						df[e] = df[e] + rnd_to<TB>(gf[e] * rnd_to<TB>(deriv));
					}
					buf_store16_aux<BUF_AUX_DEV>(rd, (uint32_t) c * 16u, 0, pack16<TB>(df));
				}
			}
			cur = nxt;
		}
		return;
	}
	/* element path: one workgroup per row at a time */
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		const long off = (long) row * n_cols;
		const float r = rs_in[row], ws = ws_in[row];
		const float r3 = r * r * r;
		for (int j = threadIdx.x; j < n_cols; j += blockDim.x)
			dX[off + j] = from_f<TB>(bwd_x_elem<TB>(to_f(W[j]), to_f(X[off + j]), to_f(dY[off + j]), to_f(dX[off + j]), r, r3, ws, n_cols));
	}
}

/* dW partial rows: each slot sums dY * X * rstd over its rows in registers,
 * the slots add theirs in slot order through LDS, and the workgroup writes
 * one partial row; the op's finish kernel adds the partial rows in a fixed
 * order (rms_dw_finish), as for the other types. */
template <typename TF, typename TB>
__device__ __forceinline__ void rms_bwd_w_fp8(int n_rows, int n_cols, const float * rs_in, const TF * X, const TB * dY) {
	extern __shared__ float colbuf[];
	if (blockIdx.x == 0 && threadIdx.x == 0) g_rms_dw_nparts = (int) gridDim.x;
	if (f8_rows_vec<TF, TB>(n_cols, X, X, dY, dY)) {
		const F8Slots sl(n_cols);
		const uint8_t * X8 = reinterpret_cast<const uint8_t *>(X);
		const uint16_t * G16 = reinterpret_cast<const uint16_t *>(dY);
		float acc[F8_CPT][8];
#pragma unroll
		for (int k = 0; k < F8_CPT; k++) {
#pragma unroll
			for (int e = 0; e < 8; e++) acc[k][e] = 0.0f;
		}
		F8Row cur;
		f8_load_row<false>(sl.first, n_rows, sl.cpr, sl.tr, sl.tpr, X8, G16, nullptr, rs_in, nullptr, cur);
		for (int row = sl.first; row < n_rows; row += sl.step) {
			vmem_wait_all();
			F8Row nxt;
			f8_load_row<false>(row + sl.step, n_rows, sl.cpr, sl.tr, sl.tpr, X8, G16, nullptr, rs_in, nullptr, nxt);
			const float r = cur.r;
#pragma unroll
			for (int k = 0; k < F8_CPT; k++) {
				if (sl.tr + k * sl.tpr < sl.cpr) {
					float xf[8], gf[8];
					unpack8_fp8<TF>(cur.x[k], xf);
					unpack16<TB>(cur.g[k], gf);
#pragma unroll
					for (int e = 0; e < 8; e++) acc[k][e] = fmaf(gf[e] * xf[e], r, acc[k][e]);
				}
			}
			cur = nxt;
		}
		for (int s = 0; s < sl.S; s++) {
			__syncthreads();
			if (sl.slot == s) {
#pragma unroll
				for (int k = 0; k < F8_CPT; k++) {
					const int c = sl.tr + k * sl.tpr;
					if (c < sl.cpr) {
#pragma unroll
						for (int e = 0; e < 8; e++) colbuf[8 * c + e] = (s == 0) ? acc[k][e] : colbuf[8 * c + e] + acc[k][e];
					}
				}
			}
		}
		write_partial_from_lds(colbuf, n_cols, g_rms_dw_partials);
		return;
	}
	/* element path: the workgroup's rows one after another into an LDS row */
	for (int j = threadIdx.x; j < n_cols; j += blockDim.x) colbuf[j] = 0.0f;
	__syncthreads();
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		const long off = (long) row * n_cols;
		const float r = rs_in[row];
		for (int j = threadIdx.x; j < n_cols; j += blockDim.x) colbuf[j] = fmaf(to_f(dY[off + j]) * to_f(X[off + j]), r, colbuf[j]);
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
	/* grid-stride over 8-element chunks, the next chunk's loads issued before
	 * this one is computed and stored */
	R8 gr, ur;
	R16 dr;
	if (tid < nvec) { gr = ld8(g + 8 * tid); ur = ld8(u + 8 * tid); dr = ld16_nt(dO + 8 * tid); }
	for (long v = tid; v < nvec; v += nth) {
		vmem_wait_all();
		R8 gn, un;
		R16 dn;
		const long vn = v + nth;
		if (vn < nvec) { gn = ld8(g + 8 * vn); un = ld8(u + 8 * vn); dn = ld16_nt(dO + 8 * vn); }
		float gf[8], uf[8], df[8], ogf[8], ouf[8];
		unpack8_fp8<TF>(gr, gf);
		unpack8_fp8<TF>(ur, uf);
		unpack16<TB>(dr, df);
#pragma unroll
		for (int e = 0; e < 8; e++) swiglu_bwd_elem<TB>(gf[e], uf[e], df[e], ogf[e], ouf[e]);
		st16_nt(dG + 8 * v, pack16<TB>(ogf));
		st16_nt(dU + 8 * v, pack16<TB>(ouf));
		gr = gn;
		ur = un;
		dr = dn;
	}
	for (long i = nvec * 8 + tid; i < n; i += nth) {
		float dg, du;
		swiglu_bwd_elem<TB>(to_f(g[i]), to_f(u[i]), to_f(dO[i]), dg, du);
		dG[i] = from_f<TB>(dg);
		dU[i] = from_f<TB>(du);
	}
}

/* ---------------- softmax ---------------- */

/* Register rows: workgroups of F8_SMX_THREADS take rows block, block + grid,
 * ...; thread t holds the row's 8-byte pieces (8 fp8 values)
 * t + F8_SMX_THREADS j, j < F8_SMX_CH, so a row of up to
 * 8 * F8_SMX_CH * F8_SMX_THREADS columns is read from memory once, and each
 * wave's loads (8 bytes per lane) and stores (16 bytes per lane) cover
 * contiguous spans. Two workgroups share a CU, so one's loads overlap the
 * other's reductions and stores. Each pass decodes the pieces again (two
 * codes per instruction) instead of keeping the floats. */
template <typename TF, typename TO>
__device__ __forceinline__ void softmax_fp8_regs(int n_rows, int n_cols, const TF * X, TO * out, float * slots) {
	const int np = n_cols / 8;
	constexpr int nt = F8_SMX_THREADS;   /* the caller checked blockDim */
	const int tid = (int) threadIdx.x;
	const uint8_t * X8 = reinterpret_cast<const uint8_t *>(X);
	/* rows through buffer ranges (the row is uniform over the workgroup):
	 * 32-bit offsets, and pieces past the row load zero / store nowhere */
	for (int row = blockIdx.x; row < n_rows; row += gridDim.x) {
		R8 cur[F8_SMX_CH];
		const __amdgpu_buffer_rsrc_t rx = make_rsrc(X8 + (long) row * n_cols, (uint32_t) n_cols);
#pragma unroll
		for (int j = 0; j < F8_SMX_CH; j++) {
			if (nt * j < np) {
				const u32x2_v v = __builtin_amdgcn_raw_buffer_load_b64(rx, (uint32_t) (tid + nt * j) * 8u, 0, BUF_AUX_NT);
				cur[j].w[0] = v.x;
				cur[j].w[1] = v.y;
			}
		}
		float m = -__builtin_inff();
#pragma unroll
		for (int j = 0; j < F8_SMX_CH; j++) {
			if (tid + nt * j < np) {
				float f[8];
				unpack8_fp8<TF>(cur[j], f);
#pragma unroll
				for (int e = 0; e < 8; e++) m = __builtin_elementwise_maximum(m, f[e]);
			}
		}
		m = block_max(m, slots);
		/* the pieces are opaque again after each pass, so the compiler
		 * decodes them anew instead of keeping all 8 * F8_SMX_CH floats alive */
#pragma unroll
		for (int j = 0; j < F8_SMX_CH; j++) reg_barrier8(cur[j]);
		float sd = 0.0f;
#pragma unroll
		for (int j = 0; j < F8_SMX_CH; j++) {
			if (tid + nt * j < np) {
				float f[8];
				unpack8_fp8<TF>(cur[j], f);
#pragma unroll
				for (int e = 0; e < 8; e++) sd += exp_fast(rnd_in<TO>(f[e] - m));
			}
		}
		float unused = 0.0f;
		__syncthreads();   /* every wave has read the max cells */
		block_sum2(sd, unused, slots);
		const float nlog2s = -__builtin_amdgcn_logf(sd);
#pragma unroll
		for (int j = 0; j < F8_SMX_CH; j++) reg_barrier8(cur[j]);
		const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + (long) row * n_cols, (uint32_t) n_cols * 2u);
#pragma unroll
		for (int j = 0; j < F8_SMX_CH; j++) {
			if (nt * j < np) {
				float f[8];
				unpack8_fp8<TF>(cur[j], f);
#pragma unroll
				for (int e = 0; e < 8; e++) f[e] = __builtin_amdgcn_exp2f(fmaf(rnd_in<TO>(f[e] - m), SMX_LOG2E, nlog2s));
				buf_store16_nt(ro, (uint32_t) (tid + nt * j) * 16u, 0, pack16<TO>(f));
			}
		}
		__syncthreads();   /* the cells are rewritten for the next row */
	}
}

/* Long rows (f8_smx_pf_ok): one SMX_THREADS workgroup per CU; thread t holds
 * the row's 8-byte pieces t + SMX_THREADS j (j < F8_PF_PIECES) in registers
 * while the next row is requested, after this row's max reduction, so that
 * it lands during this row's sum and output passes: its first half straight
 * into LDS (16-byte buffer loads with the LDS bit, lane-contiguous; read back
 * in the 8-byte layout, which takes other waves' loads, hence a barrier
 * after every wave has waited for its own), its second half into registers
 * (8-byte loads). The reductions' barriers wait for LDS only (cells_max /
 * cells_sum2), so the prefetch stays in flight across them. The LDS buffer is
 * 64 KB, so the two-workgroup register path of shorter rows, compiled into the
 * same kernel, still fits two workgroups per CU. Pieces past the row end load
 * zeros and are left out of the max and the sum; their stores fall outside
 * the row's range and store nothing. Rows are handed out as workgroups free
 * up, as in the 16-bit softmax: each workgroup's first two rows are block and
 * block + grid, every later one a ticket of the code object's launch-wide row
 * counter (g_smx_sched), taken by thread 0 at the top of a row for the row
 * after next and written to an LDS cell at once; the max reduction's barrier
 * publishes it before the next row is requested. The caller resets the
 * counter at the end of the launch (smx_launch_end). */
template <typename TF, typename TO>
__device__ __forceinline__ void softmax_fp8_pf(int n_rows, int n_cols, const TF * X, TO * out) {
	constexpr int nt = SMX_THREADS;
	constexpr int NP = F8_PF_PIECES;
	constexpr int NH = NP / 2;    /* pieces per thread through LDS, and through registers */
	constexpr int NL = NH / 2;    /* 16-byte LDS loads per thread and row */
	static_assert(NP == 16, "the output pass's wait counts 16 stores");
	__shared__ __attribute__((aligned(16))) float mslots[SMX_WAVES];
	__shared__ __attribute__((aligned(16))) float sslots[2 * SMX_WAVES];
	__shared__ __attribute__((aligned(16))) uint8_t pf[NL * nt * 16];
	__shared__ int nextcell;
	const int np = n_cols / 8;
	const int tid = (int) threadIdx.x;
	const int wave_base = tid & ~63;
	const uint8_t * X8 = reinterpret_cast<const uint8_t *>(X);
	R8 nx[NH];
	auto request = [&](int r) {
		const __amdgpu_buffer_rsrc_t rx = make_rsrc(X8 + (long) r * n_cols, (uint32_t) n_cols);
#pragma unroll
		for (int k = 0; k < NL; k++)
			__builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t) &pf[16 * (k * nt + wave_base)], 16, (uint32_t) tid * 16u, k * nt * 16,
													 0, BUF_AUX_NT);
#pragma unroll
		for (int j = 0; j < NH; j++) {
			const u32x2_v v = __builtin_amdgcn_raw_buffer_load_b64(rx, (uint32_t) (tid + nt * (NH + j)) * 8u, 0, BUF_AUX_NT);
			nx[j].w[0] = v.x;
			nx[j].w[1] = v.y;
		}
	};
	int row = blockIdx.x;
	int next = row + (int) gridDim.x;
	if (row < n_rows) request(row);
	vmem_wait_all();
	cells_barrier();
	while (row < n_rows) {
		/* the ticket for the row after next, requested here and read after
		 * the max pass, so that thread 0 waits for its return (and, since
		 * vector-memory operations complete in order, for the previous row's
		 * stores) only there. An atomic increment with no wrap-around, which
		 * the compiler's atomic optimizer leaves alone: an atomic add gets
		 * its result broadcast, and so waited for, right where it is made. */
		unsigned tk = 0u;
		if (tid == 0 && next < n_rows)
			tk = __builtin_amdgcn_atomic_inc32(&g_smx_sched[SMX_TICKETS], 0xffffffffu, __ATOMIC_RELAXED, "agent");
		R8 cur[NP];
#pragma unroll
		for (int j = 0; j < NH; j++) cur[j] = *reinterpret_cast<const R8 *>(&pf[8 * (tid + nt * j)]);
#pragma unroll
		for (int j = 0; j < NH; j++) cur[NH + j] = nx[j];
		WAIT_LDS_ALL();
		float m = -__builtin_inff();
#pragma unroll
		for (int j = 0; j < NP; j++) {
			if (tid + nt * j < np) {
				float f[8];
				unpack8_fp8<TF>(cur[j], f);
#pragma unroll
				for (int e = 0; e < 8; e++) m = __builtin_elementwise_maximum(m, f[e]);
			}
		}
		/* the row after next (n_rows: none); every wave reads the cell after
		 * this row's max reduction, before the barrier at the row's end lets
		 * thread 0 write it again */
		if (tid == 0) {
			const unsigned r = 2u * gridDim.x + tk;
			nextcell = (next < n_rows && r < (unsigned) n_rows) ? (int) r : n_rows;
		}
		m = cells_max(m, mslots);
		const int next2 = __builtin_amdgcn_readfirstlane(nextcell);
		/* every wave has read its pieces (each waited for its LDS reads
		 * before the barrier in cells_max): the buffer takes the next row */
		if (next < n_rows) request(next);
#pragma unroll
		for (int j = 0; j < NP; j++) reg_barrier8(cur[j]);
		float sd = 0.0f, unused = 0.0f;
#pragma unroll
		for (int j = 0; j < NP; j++) {
			if (tid + nt * j < np) {
				float f[8];
				unpack8_fp8<TF>(cur[j], f);
#pragma unroll
				for (int e = 0; e < 8; e++) sd += exp_fast(rnd_in<TO>(f[e] - m));
			}
		}
		cells_sum2(sd, unused, sslots);
		const float nlog2s = -__builtin_amdgcn_logf(sd);
#pragma unroll
		for (int j = 0; j < NP; j++) reg_barrier8(cur[j]);
		const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + (long) row * n_cols, (uint32_t) n_cols * 2u);
#pragma unroll
		for (int j = 0; j < NP; j++) {
			float f[8];
			unpack8_fp8<TF>(cur[j], f);
#pragma unroll
			for (int e = 0; e < 8; e++) f[e] = __builtin_amdgcn_exp2f(fmaf(rnd_in<TO>(f[e] - m), SMX_LOG2E, nlog2s));
			buf_store16_nt(ro, (uint32_t) (tid + nt * j) * 16u, 0, pack16<TO>(f));
		}
		/* the next row's loads were issued before these 16 stores and
		 * complete first: once at most 16 remain, this wave's part of it has
		 * landed; the barrier then waits for every wave's */
		__builtin_amdgcn_s_waitcnt(0x4F70);   /* vmcnt(16) */
		cells_barrier();
		row = next;
		next = next2;
	}
	vmem_wait_all();
}

/* Other rows: three passes per row, the later ones re-reading the row (a
 * row of fp8 is n_cols bytes, so they find it in cache): max, sum exp(d),
 * outputs. In both paths d = rnd_out(x - max), since the reference converts x
 * to the output type and subtracts there. */
template <typename TF, typename TO>
__device__ __forceinline__ void softmax_fp8(int n_rows, int n_cols, const TF * X, TO * out) {
	__shared__ float slots[32];
	if (blockDim.x == SMX_THREADS && f8_smx_pf_ok(n_cols) && aligned16(X) && aligned16(out)) {
		softmax_fp8_pf<TF, TO>(n_rows, n_cols, X, out);
		smx_launch_end<false>(n_rows, nullptr, nullptr);
		return;
	}
	if (blockDim.x == F8_SMX_THREADS && f8_smx_regs_ok(n_cols) && aligned16(X) && aligned16(out)) {
		softmax_fp8_regs<TF, TO>(n_rows, n_cols, X, out, slots);
		return;
	}
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
