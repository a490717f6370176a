/*
 * RMSNorm device code for gfx950 (hand-written; semantics of the reference's
 * src/ops/nvidia/norm/rms_norm.cu:4-138,280-412, rms_norm_bwd_x.cu:4-86,175-256,
 * rms_norm_bwd_w.cu:4-101,211-308, restated in the oracle's rms_norm_*).
 * Included by rms_norm.hip (the code object's kernels, reference ABI) and by
 * the allocation-free library's kernels; the dW modes take their partial-row
 * buffer as an argument (RmsArgs.partials, rms_dw_finish).
 *
 * Layout: X, Y, dY, dX row-major [n_rows x n_cols]; W [n_cols];
 * weighted_sums, rms_vals (= rstd) [n_rows] fp32; dW [n_cols].
 *
 * All four ops run on the same row-slot engine (thread layout in
 * kernel_geometry.h): a slot of TPR threads covers one row with 16-byte accesses,
 * each thread keeps its W chunks and (bwd_w, fused bwd) its dW partial in
 * registers for the whole kernel, and row reductions are a DPP wave sum plus
 * one LDS exchange between the slot's waves.
 *
 * dW is reduced in two passes without atomics: each workgroup sums its slots
 * in slot order through LDS and writes one fp32 partial row to the partial
 * buffer; the finish kernel adds the partials in a fixed order. The result is
 * deterministic. Two dW-reducing launches must not share a partial buffer
 * concurrently.
 */
#pragma once

#include "dtypes.h"
#include "reduce.h"
#include "kernel_geometry.h"

enum RmsMode { RMS_FWD = 0, RMS_BWD_X = 1, RMS_BWD_W = 2, RMS_BWD = 3 };

template <typename T> __device__ __forceinline__ float rnd_to(float f) { return to_f(from_f<T>(f)); }

/* Reference formula of the X gradient (rms_norm_bwd_x.cu:245-252):
 *   deriv = w*r - ((x*r^3)/n)*ws;  dX + rnd(dY * rnd(deriv))
 * with rnd() the rounding to the storage type. Contraction is off here: for
 * fp16 the compiler would otherwise narrow dY*t to an f16 multiply and fuse
 * it with the add through the conversion, skipping the product's rounding. */
template <typename T>
__device__ __forceinline__ float bwd_x_elem(float w, float x, float dy, float dx, float r, float r3, float ws, int n_cols) {
#pragma clang fp contract(off)
	const float deriv = w * r - ((x * r3) / (float) n_cols) * ws;
	const float p = rnd_to<T>(dy * rnd_to<T>(deriv));
	return dx + p;
}

struct RmsArgs {
	int n_rows, n_cols;
	float eps;
	const float * ws_in;      /* bwd_x: fwd weighted sums */
	const float * rs_in;      /* bwd*: fwd rstd */
	float * ws_out;           /* fwd outputs (may be NULL) */
	float * rs_out;
	const void * W;
	const void * X;
	const void * dY;
	void * Y_or_dX;           /* fwd: Y; bwd_x / bwd: dX (read-modify-write) */
	void * dW;                /* bwd_w: T; bwd: fp32 */
	float * partials;         /* dW modes: one fp32 partial row per workgroup */
	int * nparts_out;         /* dW modes, optional: receives the grid size */
	bool sq_stat;             /* fwd: rs_out receives sum_j x^2 instead of rstd (the fp8 kernels) */
};

/* sums of (a, b) over the waves of this thread's slot, one barrier.
 * cells = LDS [2 parities][slots][32]: a at [w], b at [16 + w]. */
__device__ __forceinline__ void slot_sum2(float & a, float & b, float * cells, int parity, int slot, int wave_in_slot, int waves_per_slot, int slots) {
	a = wave_sum(a);
	b = wave_sum(b);
	float * c = cells + (parity * slots + slot) * 32;
	if ((threadIdx.x & 63) == 0) { c[wave_in_slot] = a; c[16 + wave_in_slot] = b; }
	lds_barrier();
	float ta = 0.0f, tb = 0.0f;
	for (int w = 0; w < waves_per_slot; w++) { ta += c[w]; tb += c[16 + w]; }
	a = ta;
	b = tb;
}

/* combine the slots' dW partials (slot order) and write this workgroup's row */
__device__ __forceinline__ void write_partial_from_lds(const float * colbuf, int n_cols, float * partials) {
	__syncthreads();
	float * part = partials + (long) blockIdx.x * n_cols;
	for (int j = threadIdx.x; j < n_cols; j += blockDim.x) part[j] = colbuf[j];
}

/* One row of a row-major tensor as a buffer range. A row past the end gets an
 * empty range: its loads return zero and its stores are dropped. `row` must be
 * wave-uniform (it lives in SGPRs). */
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void * base, int row, int n_rows, uint32_t row_bytes) {
	const bool live = row < n_rows;
	return make_rsrc(static_cast<const char *>(base) + (long) (live ? row : 0) * row_bytes, live ? row_bytes : 0u);
}

/* the registers one row slot holds for one row */
template <int MODE>
struct RmsRow {
	R16 x[RMS_CH], g[RMS_CH], d[RMS_CH];
	float r, ws;
};

/* Issue the loads of `row` (wave-uniform). Chunks a thread does not own lie
 * past the row's byte range, so they read as zero. */
template <typename T, int MODE>
__device__ __forceinline__ void rms_load_row(const RmsArgs & a, int row, uint32_t row_bytes, const uint32_t * voff, RmsRow<MODE> & o) {
	const __amdgpu_buffer_rsrc_t rx = row_rsrc(a.X, row, a.n_rows, row_bytes);
#pragma unroll
	for (int c = 0; c < RMS_CH; c++) o.x[c] = buf_load16_nt(rx, voff[c], 0);
	if (MODE != RMS_FWD) {
		const __amdgpu_buffer_rsrc_t rg = row_rsrc(a.dY, row, a.n_rows, row_bytes);
#pragma unroll
		for (int c = 0; c < RMS_CH; c++) o.g[c] = buf_load16_nt(rg, voff[c], 0);
	}
	if (MODE == RMS_BWD_X || MODE == RMS_BWD) {
		const __amdgpu_buffer_rsrc_t rd = row_rsrc(a.Y_or_dX, row, a.n_rows, row_bytes);
#pragma unroll
		for (int c = 0; c < RMS_CH; c++) o.d[c] = buf_load16_nt(rd, voff[c], 0);
	}
	const bool live = row < a.n_rows;
	o.r = (MODE != RMS_FWD && live) ? a.rs_in[row] : 0.0f;
	o.ws = (MODE == RMS_BWD_X && live) ? a.ws_in[row] : 0.0f;
}

/*
 * Vector path, software-pipelined: while a slot reduces and writes row i it
 * already has the loads of its next row (i + grid * slots) in flight, so the
 * memory pipe does not drain at the row reduction's barrier.
 */
template <typename T, typename TW, int MODE>
__device__ __forceinline__ void rms_vector(const RmsArgs & a, int nv, float * lds) {
	constexpr int V = VecOf<T>::N;
	const int tpr = rms_tpr_for(nv);
	const int slots = blockDim.x / tpr;
	const int slot = threadIdx.x / tpr;
	const int tr = threadIdx.x % tpr;
	const int wps = tpr >> 6;
	const int wis = tr >> 6;
	const int n_cols = a.n_cols;
	const uint32_t row_bytes = (uint32_t) n_cols * (uint32_t) sizeof(T);

	uint32_t voff[RMS_CH];
	bool own[RMS_CH];
	R16 wr[RMS_CH];
	float acc[RMS_CH][V];
	const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.W, (MODE != RMS_BWD_W) ? row_bytes : 0u);
#pragma unroll
	for (int c = 0; c < RMS_CH; c++) {
		voff[c] = (uint32_t) (c * tpr + tr) * 16u;
		own[c] = (c * tpr + tr) < nv;
		wr[c] = buf_load16(rw, voff[c], 0);
#pragma unroll
		for (int e = 0; e < V; e++) acc[c][e] = 0.0f;
	}

	float * cells = lds;                                   /* [2][slots][32] */
	float * colbuf = lds + RMS_CELLS_PER_SLOT * slots;     /* [n_cols] for the dW modes */
	int parity = 0;
	const int step = gridDim.x * slots;
	/* tpr is a multiple of 64, so the row is uniform over each wave */
	int row = __builtin_amdgcn_readfirstlane(blockIdx.x * slots + slot);
	/* forward statistics: lane k of the slot keeps the k-th row's weighted sum
	 * and statistic, and the lanes store them together every 64 rows and at
	 * the end (one-lane stores after every row sat in the wave's in-order
	 * memory queue and cost the forward ~0.6 us) */
	float st_ws = 0.0f, st_rs = 0.0f;
	int st_n = 0, st_row0 = row;
	auto flush_stats = [&]() {
		if (tr < st_n) {
			const int r0 = st_row0 + tr * step;
			if (r0 < a.n_rows) {
				if (a.ws_out) a.ws_out[r0] = st_ws;
				if (a.rs_out) a.rs_out[r0] = st_rs;
			}
		}
	};
	RmsRow<MODE> cur;
	rms_load_row<T, MODE>(a, row, row_bytes, voff, cur);

	for (int base_row = blockIdx.x * slots; base_row < a.n_rows; base_row += step) {
		const int nrow = row + step;
		RmsRow<MODE> nxt;
		rms_load_row<T, MODE>(a, nrow, row_bytes, voff, nxt);
		const bool live = row < a.n_rows;
		const __amdgpu_buffer_rsrc_t ro = row_rsrc(a.Y_or_dX, row, a.n_rows, row_bytes);

		if (MODE == RMS_FWD) {
			/* four interleaved partial sums (chunk, element parity) per thread,
			 * added pairwise: the fp32 rounding chain of a term is 4 + 2 long
			 * instead of RMS_CH * V */
			float ssp[4] = {0.0f, 0.0f, 0.0f, 0.0f}, swp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
			for (int c = 0; c < RMS_CH; c++) {
				float xf[V], wf[V];
				unpack16<T>(cur.x[c], xf);
				unpack16<T>(wr[c], wf);
#pragma unroll
				for (int e = 0; e < V; e++) {
					const int k = (c * 2 + (e & 1)) & 3;
					if (!IsFp8<T>::value) swp[k] = fmaf(xf[e], wf[e], swp[k]);   /* fp8: weighted sums are not written */
					ssp[k] = fmaf(xf[e], xf[e], ssp[k]);
				}
			}
			float ss = (ssp[0] + ssp[1]) + (ssp[2] + ssp[3]);
			float sw = (swp[0] + swp[1]) + (swp[2] + swp[3]);
			slot_sum2(ss, sw, cells, parity, slot, wis, wps, slots);
			parity ^= 1;
#pragma unroll
			for (int c = 0; c < RMS_CH; c++) { reg_barrier(cur.x[c]); reg_barrier(wr[c]); }
			const float r = 1.0f / sqrtf(ss / (float) n_cols + a.eps);
			if (tr == st_n) {
				st_ws = sw;
				st_rs = a.sq_stat ? ss : r;
			}
			if (++st_n == 64) {
				flush_stats();
				st_n = 0;
				st_row0 = row + step;
			}
#pragma unroll
			for (int c = 0; c < RMS_CH; c++) {
				float xf[V], wf[V];
				unpack16<T>(cur.x[c], xf);
				unpack16<T>(wr[c], wf);
#pragma unroll
				for (int e = 0; e < V; e++) xf[e] = (xf[e] * r) * wf[e];
				buf_store16_nt(ro, voff[c], 0, pack16<T>(xf));
			}
		}
		else if (MODE == RMS_BWD_X) {
			const float r = cur.r;
			const float r3 = r * r * r;
#pragma unroll
			for (int c = 0; c < RMS_CH; c++) {
				float wf[V], xf[V], gf[V], df[V];
				unpack16<T>(wr[c], wf);
				unpack16<T>(cur.x[c], xf);
				unpack16<T>(cur.g[c], gf);
				unpack16<T>(cur.d[c], df);
#pragma unroll
				for (int e = 0; e < V; e++) df[e] = bwd_x_elem<T>(wf[e], xf[e], gf[e], df[e], r, r3, cur.ws, n_cols);
				buf_store16_aux<BUF_AUX_DEV>(ro, voff[c], 0, pack16<T>(df));
			}
		}
		else {
			const float r = cur.r;
			if (MODE == RMS_BWD) {
				float dot = 0.0f;
#pragma unroll
				for (int c = 0; c < RMS_CH; c++) {
					float xf[V], gf[V], wf[V];
					unpack16<T>(cur.x[c], xf);
					unpack16<T>(cur.g[c], gf);
					unpack16<T>(wr[c], wf);
#pragma unroll
					for (int e = 0; e < V; e++) dot = fmaf(gf[e] * wf[e], xf[e], dot);
				}
				float unused = 0.0f;
				slot_sum2(dot, unused, cells, parity, slot, wis, wps, slots);
				parity ^= 1;
				/* re-unpack after the barrier instead of holding the floats across it */
#pragma unroll
				for (int c = 0; c < RMS_CH; c++) { reg_barrier(cur.x[c]); reg_barrier(cur.g[c]); reg_barrier(wr[c]); }
				const float coef = ((r * r * r) * dot) / (float) n_cols;
#pragma unroll
				for (int c = 0; c < RMS_CH; c++) {
					float xf[V], gf[V], wf[V], df[V];
					unpack16<T>(cur.x[c], xf);
					unpack16<T>(cur.g[c], gf);
					unpack16<T>(wr[c], wf);
					unpack16<T>(cur.d[c], df);
#pragma unroll
					for (int e = 0; e < V; e++) df[e] = df[e] + (r * (gf[e] * wf[e]) - xf[e] * coef);
					buf_store16_aux<BUF_AUX_DEV>(ro, voff[c], 0, pack16<T>(df));
				}
			}
			/* rows past the end loaded zeros and r = 0, so they add nothing */
#pragma unroll
			for (int c = 0; c < RMS_CH; c++) {
				float xf[V], gf[V];
				unpack16<T>(cur.x[c], xf);
				unpack16<T>(cur.g[c], gf);
#pragma unroll
				for (int e = 0; e < V; e++) acc[c][e] = fmaf(gf[e] * xf[e], r, acc[c][e]);
			}
		}
		cur = nxt;
		row = nrow;
	}
	if (MODE == RMS_FWD) flush_stats();

	if (MODE == RMS_BWD_W || MODE == RMS_BWD) {
		for (int s = 0; s < slots; s++) {
			__syncthreads();
			if (slot == s) {
#pragma unroll
				for (int c = 0; c < RMS_CH; c++) {
					if (own[c]) {
#pragma unroll
						for (int e = 0; e < V; e++) {
							const int j = (c * tpr + tr) * V + e;
							colbuf[j] = (s == 0) ? acc[c][e] : colbuf[j] + acc[c][e];
						}
					}
				}
			}
		}
		write_partial_from_lds(colbuf, n_cols, a.partials);
	}
}

/* element path: any alignment / row length; TPR = 256 */
template <typename T, typename TW, int MODE>
__device__ __forceinline__ void rms_stream(const RmsArgs & a, float * lds) {
	const int tpr = rms_stream_tpr(MODE == RMS_BWD_W || MODE == RMS_BWD, a.n_cols);
	const int slots = blockDim.x / tpr;
	const int slot = threadIdx.x / tpr;
	const int tr = threadIdx.x % tpr;
	const int wps = tpr >> 6;
	const int wis = tr >> 6;
	const int n_cols = a.n_cols;
	const T * W = reinterpret_cast<const T *>(a.W);
	float * cells = lds;                                   /* [2][slots][32] */
	float * colbuf = lds + RMS_CELLS_PER_SLOT * slots;     /* [slots][n_cols] for the dW modes */
	float * mycol = colbuf + (long) slot * n_cols;
	if (MODE == RMS_BWD_W || MODE == RMS_BWD) {
		for (int j = tr; j < n_cols; j += tpr) mycol[j] = 0.0f;
		/* the zeroing maps elements to threads one by one, the 16-byte update
		 * loops map 16-byte chunks: without this barrier a thread can clear an
		 * element another thread has already accumulated (RMS_BWD_W reads r
		 * from the saved statistics, so no row reduction orders them) */
		__syncthreads();
	}
	int parity = 0;
	for (int base_row = blockIdx.x * slots; base_row < a.n_rows; base_row += gridDim.x * slots) {
		const int row = base_row + slot;
		const bool live = row < a.n_rows;
		const long off = (long) row * n_cols;
		const T * x = reinterpret_cast<const T *>(a.X) + off;
		const T * g = reinterpret_cast<const T *>(a.dY) + off;
		T * yd = reinterpret_cast<T *>(a.Y_or_dX) + off;
		if (MODE == RMS_FWD) {
			/* rows too long for the vector path but 16-byte aligned: 16-byte
			 * chunks; the second loop re-reads the row (from cache where it
			 * still is) */
			constexpr int V = VecOf<T>::N;
			const bool vec = (n_cols % V) == 0 && aligned16(a.X) && aligned16(a.Y_or_dX) && aligned16(W);
			const int nv = n_cols / V;
			float ss = 0.0f, sw = 0.0f;
			if (live && vec) {
				for (int c = tr; c < nv; c += tpr) {
					float xf[V], wf[V];
					unpack16<T>(reinterpret_cast<const R16 *>(x)[c], xf);
					unpack16<T>(reinterpret_cast<const R16 *>(W)[c], wf);
#pragma unroll
					for (int e = 0; e < V; e++) {
						if (!IsFp8<T>::value) sw = fmaf(xf[e], wf[e], sw);
						ss = fmaf(xf[e], xf[e], ss);
					}
				}
			}
			else if (live) {
				for (int j = tr; j < n_cols; j += tpr) {
					const float xf = to_f(x[j]);
					if (!IsFp8<T>::value) sw = fmaf(xf, to_f(W[j]), sw);
					ss = fmaf(xf, xf, ss);
				}
			}
			slot_sum2(ss, sw, cells, parity, slot, wis, wps, slots);
			parity ^= 1;
			if (live) {
				const float r = 1.0f / sqrtf(ss / (float) n_cols + a.eps);
				if (tr == 0) {
					if (a.ws_out) a.ws_out[row] = sw;
					if (a.rs_out) a.rs_out[row] = a.sq_stat ? ss : r;
				}
				if (vec) {
					for (int c = tr; c < nv; c += tpr) {
						float xf[V], wf[V];
						unpack16<T>(ld16_nt(reinterpret_cast<const R16 *>(x) + c), xf);
						unpack16<T>(reinterpret_cast<const R16 *>(W)[c], wf);
#pragma unroll
						for (int e = 0; e < V; e++) xf[e] = (xf[e] * r) * wf[e];
						st16_nt(reinterpret_cast<R16 *>(yd) + c, pack16<T>(xf));
					}
				}
				else {
					for (int j = tr; j < n_cols; j += tpr) yd[j] = from_f<T>((to_f(x[j]) * r) * to_f(W[j]));
				}
			}
		}
		else if (MODE == RMS_BWD_X) {
			if (live) {
				const float r = a.rs_in[row];
				const float ws = a.ws_in[row];
				const float r3 = r * r * r;
				constexpr int V = VecOf<T>::N;
				if ((n_cols % V) == 0 && aligned16(a.X) && aligned16(a.dY) && aligned16(a.Y_or_dX) && aligned16(W)) {
					const R16 * wv = reinterpret_cast<const R16 *>(W);
					const R16 * xv = reinterpret_cast<const R16 *>(x);
					const R16 * gv = reinterpret_cast<const R16 *>(g);
					R16 * dv = reinterpret_cast<R16 *>(yd);
					for (int c = tr; c < n_cols / V; c += tpr) {
						float wf[V], xf[V], gf[V], df[V];
						unpack16<T>(wv[c], wf);
						unpack16<T>(xv[c], xf);
						unpack16<T>(gv[c], gf);
						unpack16<T>(dv[c], df);
#pragma unroll
						for (int e = 0; e < V; e++) df[e] = bwd_x_elem<T>(wf[e], xf[e], gf[e], df[e], r, r3, ws, n_cols);
						dv[c] = pack16<T>(df);
					}
				}
				else {
					for (int j = tr; j < n_cols; j += tpr) {
						yd[j] = from_f<T>(bwd_x_elem<T>(to_f(W[j]), to_f(x[j]), to_f(g[j]), to_f(yd[j]), r, r3, ws, n_cols));
					}
				}
			}
		}
		else {
			const float r = live ? a.rs_in[row] : 0.0f;
			/* 16-byte chunks when every row operand is aligned */
			constexpr int V = VecOf<T>::N;
			const bool vec = (n_cols % V) == 0 && aligned16(a.X) && aligned16(a.dY) &&
							 (MODE == RMS_BWD_W || (aligned16(a.Y_or_dX) && aligned16(W)));
			const int nv = n_cols / V;
			const R16 * xv = reinterpret_cast<const R16 *>(x);
			const R16 * gv = reinterpret_cast<const R16 *>(g);
			if (MODE == RMS_BWD) {
				const R16 * wv = reinterpret_cast<const R16 *>(W);
				float dot = 0.0f;
				if (live && vec) {
					for (int c = tr; c < nv; c += tpr) {
						float xf[V], gf[V], wf[V];
						unpack16<T>(xv[c], xf);
						unpack16<T>(gv[c], gf);
						unpack16<T>(wv[c], wf);
#pragma unroll
						for (int e = 0; e < V; e++) dot = fmaf(gf[e] * wf[e], xf[e], dot);
					}
				}
				else if (live) {
					for (int j = tr; j < n_cols; j += tpr) dot = fmaf(to_f(g[j]) * to_f(W[j]), to_f(x[j]), dot);
				}
				float unused = 0.0f;
				slot_sum2(dot, unused, cells, parity, slot, wis, wps, slots);
				parity ^= 1;
				if (live) {
					const float coef = ((r * r * r) * dot) / (float) n_cols;
					if (vec) {
						R16 * dv = reinterpret_cast<R16 *>(yd);
						for (int c = tr; c < nv; c += tpr) {
							float xf[V], gf[V], wf[V], df[V];
							unpack16<T>(xv[c], xf);
							unpack16<T>(gv[c], gf);
							unpack16<T>(wv[c], wf);
							unpack16<T>(dv[c], df);
#pragma unroll
							for (int e = 0; e < V; e++) {
								const float gw = gf[e] * wf[e];
								df[e] = df[e] + (r * gw - xf[e] * coef);
								mycol[c * V + e] = fmaf(gf[e] * xf[e], r, mycol[c * V + e]);
							}
							dv[c] = pack16<T>(df);
						}
					}
					else {
						for (int j = tr; j < n_cols; j += tpr) {
							const float gw = to_f(g[j]) * to_f(W[j]);
							yd[j] = from_f<T>(to_f(yd[j]) + (r * gw - to_f(x[j]) * coef));
						}
					}
				}
			}
			if (live && !(MODE == RMS_BWD && vec)) {   /* (the fused vector loop above already accumulated dW) */
				if (vec) {
					for (int c = tr; c < nv; c += tpr) {
						float xf[V], gf[V];
						unpack16<T>(xv[c], xf);
						unpack16<T>(gv[c], gf);
#pragma unroll
						for (int e = 0; e < V; e++) mycol[c * V + e] = fmaf(gf[e] * xf[e], r, mycol[c * V + e]);
					}
				}
				else {
					for (int j = tr; j < n_cols; j += tpr) mycol[j] = fmaf(to_f(g[j]) * to_f(x[j]), r, mycol[j]);
				}
			}
		}
	}
	if (MODE == RMS_BWD_W || MODE == RMS_BWD) {
		__syncthreads();
		/* slot order: slot 0 accumulates the others */
		if (slot == 0) {
			for (int s = 1; s < slots; s++)
				for (int j = tr; j < n_cols; j += tpr) mycol[j] += colbuf[(long) s * n_cols + j];
		}
		write_partial_from_lds(colbuf, n_cols, a.partials);
	}
}

template <typename T, typename TW, int MODE>
__device__ __forceinline__ void rms_run(const RmsArgs & a) {
	extern __shared__ float lds[];
	if ((MODE == RMS_BWD_W || MODE == RMS_BWD) && a.nparts_out && blockIdx.x == 0 && threadIdx.x == 0) *a.nparts_out = (int) gridDim.x;
	unsigned long long ptr_or = (unsigned long long) (uintptr_t) a.X;
	if (MODE != RMS_BWD_W) ptr_or |= (unsigned long long) (uintptr_t) a.W;
	if (MODE != RMS_FWD) ptr_or |= (unsigned long long) (uintptr_t) a.dY;
	if (MODE != RMS_BWD_W) ptr_or |= (unsigned long long) (uintptr_t) a.Y_or_dX;
	const int nv = rms_vec_chunks(a.n_cols, (int) sizeof(T), ptr_or);
	if (nv > 0) rms_vector<T, TW, MODE>(a, nv, lds);
	else rms_stream<T, TW, MODE>(a, lds);
}

/* finish: dW[j] = rnd(dW[j] + sum_g partial[g][j]). A workgroup covers
 * RMS_FIN_COLS consecutive columns, so the grid spans the whole chip even for
 * a few thousand columns: thread t takes column t % RMS_FIN_COLS and the
 * partial rows g = t / RMS_FIN_COLS + k * groups, with eight loads in flight;
 * the groups' sums are then added in group order, so the result does not
 * depend on timing. */
/* XCDs of an MI355X (gfx950) */
#define FIN_XCDS 8

template <typename TW>
__device__ __forceinline__ void rms_dw_finish(int n_cols, TW * dW, const float * partials, int n_parts) {
	constexpr int G = RMS_FINISH_THREADS / RMS_FIN_COLS;
	__shared__ float grp_part[G][RMS_FIN_COLS];
	const int col = threadIdx.x % RMS_FIN_COLS;
	const int grp = threadIdx.x / RMS_FIN_COLS;
	/* workgroups are dealt to the 8 XCDs round-robin, and a workgroup reads
	 * RMS_FIN_COLS * 4 bytes of each partial row, part of a 128-byte line:
	 * the workgroups of one XCD take adjacent column blocks so that a line's
	 * halves meet in that XCD's L2 instead of being fetched by two XCDs */
	const int nb = (int) gridDim.x;
	const int cb = (nb % FIN_XCDS == 0) ? ((int) blockIdx.x % FIN_XCDS) * (nb / FIN_XCDS) + (int) blockIdx.x / FIN_XCDS : (int) blockIdx.x;
	const int j = cb * RMS_FIN_COLS + col;
	float s = 0.0f;
	if (j < n_cols) {
		const float * p = partials + j;
		int g = grp;
		for (; g + 7 * G < n_parts; g += 8 * G) {
			float v[8];
#pragma unroll
			for (int k = 0; k < 8; k++) v[k] = p[(long) (g + k * G) * n_cols];
#pragma unroll
			for (int k = 0; k < 8; k++) s += v[k];
		}
		for (; g < n_parts; g += G) s += p[(long) g * n_cols];
	}
	grp_part[grp][col] = s;
	__syncthreads();
	if (grp == 0 && j < n_cols) {
		float t = 0.0f;
#pragma unroll
		for (int q = 0; q < G; q++) t += grp_part[q][col];
		dW[j] = from_f<TW>(to_f(dW[j]) + t);
	}
}

