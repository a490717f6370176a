/*
 * Geometry shared by the kernels and the launch-configuration library (plain
 * C on the host side), so both sides agree on paths, limits and layouts.
 *
 * RMSNorm vector path: each row is split over TPR threads ("a row slot");
 * thread t of the slot owns the 16-byte chunks t and t + TPR of the row
 * (RMS_CH = 2 chunks), so it always touches the same columns whatever row it
 * is on. TPR = 64 * ceil(ceil(chunks_per_row / 2) / 64), at most 1024.
 * RMSNorm element path (unaligned pointers, ragged rows, or rows longer than
 * 2 x 1024 chunks): TPR = 256 and a strided loop over the columns.
 * A workgroup holds `slots` row slots (blockDim.x = slots * TPR).
 */
#ifndef KERNEL_GEOMETRY_H
#define KERNEL_GEOMETRY_H

#define RMS_CH 2
#define RMS_MAX_TPR 1024
#define RMS_STREAM_TPR 256
/* element-path workgroups (one 256-thread row slot each) per CU, at most */
#define RMS_STREAM_GROUPS_PER_CU 8
/* LDS floats per row slot for the row reductions: [2 parities][32] */
#define RMS_CELLS_PER_SLOT 64
/* launch target: bytes of row loads outstanding per CU (each row slot keeps
 * its current and next row in flight) */
#define RMS_INFLIGHT_BYTES (64 * 1024)
/* dW finish kernel: RMS_FIN_COLS columns per workgroup, partial rows spread over its threads */
#define RMS_FINISH_THREADS 256
#define RMS_FIN_COLS 16   /* columns per finish workgroup */
/* fp32 partial rows for the two-pass dW reduction (16 MiB) */
#define RMS_DW_SCRATCH_FLOATS (4u << 20)

/* softmax / cross-entropy: one workgroup per row, rows of up to
 * SMX_THREADS * SMX_MAXCH 16-byte chunks held in registers */
#define SMX_THREADS 1024
#define SMX_MAXCH 16
/* chunks per thread of the next row prefetched into LDS (9 x 16 KB); the
 * other SMX_MAXCH - SMX_PF chunks of the next row are prefetched into VGPRs */
#define SMX_PF 9

/* RoPE, head_dim <= 512. Vector path: one ROPE_SLOT_THREADS workgroup per
 * token at a time (persistent over tokens, next token prefetched), thread t
 * owning Q chunks t + 256 j (j < ROPE_QJ) and K chunks t + 256 j (j < ROPE_KJ)
 * of 16 bytes. Element path (unaligned rows or head_dim not a multiple of the
 * vector): one wave per token, ROPE_WAVES waves per workgroup. */
#define ROPE_MAX_HEAD_DIM 512
#define ROPE_WAVES 4
#define ROPE_SLOT_THREADS 256
#define ROPE_QJ 4
#define ROPE_KJ 2
/* vector path workgroups per CU at most: the RoPE kernels' registers allow
 * four, the fused KV-cache variant's three, and the launch takes the smaller
 * of this and what the kernel's registers leave resident */
#define ROPE_SLOT_WG_PER_CU 4

/* fp8 x 16-bit RMSNorm backward (fp8_ops.hip): rows in 8-element chunks
 * (8 bytes of each fp8 operand, 16 of each 16-bit one); a row slot of TPR
 * threads covers a row, thread t owning chunks t + TPR k (k < F8_CPT), so
 * rows of up to 8 * F8_CPT * 1024 columns take this path. bwd_x: 256-thread
 * workgroups, F8_BWDX_WG_PER_CU per CU; bwd_w: one workgroup of up to 1024
 * threads per CU whose slots add their partial rows in LDS. */
#define F8_CPT 2
#define F8_BWDX_WG_PER_CU 4

/* fp8 -> 16-bit softmax (fp8_ops.hip): rows of up to 8 * F8_SMX_CH *
 * F8_SMX_THREADS columns held in registers, two workgroups per CU */
#define F8_SMX_THREADS 512
#define F8_SMX_CH 32

/* embedding / copy_to_seq_context: one wave per row, 4 waves per workgroup */
#define GS_WAVES 4

/* SwiGLU: grid-stride, one 512-thread workgroup per CU; per thread and
 * stream, U 16-byte chunks computed per step while the next U load. Measured
 * on MI355X at 8192 x 14336 bf16 over 1-4 workgroups of 256-1024 threads
 * per CU and U = 1, 2, 4: the forward (2 reads + 1 write) is fastest with
 * U = 2 (116 us), the backward (3 reads + 2 writes) with U = 1 (194 us
 * against 201 us with U = 2) */
#define SWIGLU_FWD_UNROLL 2
#define SWIGLU_BWD_UNROLL 1
#define SWIGLU_THREADS 512
#define SWIGLU_WG_PER_CU 1

#ifdef __HIPCC__
#define GEOM_FN __host__ __device__ __forceinline__
#else
#define GEOM_FN static inline
#endif

/* RMSNorm: 16-byte chunks per row, or 0 when the element path must be used */
GEOM_FN int rms_vec_chunks(int n_cols, int elem_bytes, unsigned long long ptr_or) {
	const int vec = 16 / elem_bytes;
	if (n_cols <= 0 || (n_cols % vec) != 0 || (ptr_or & 15ull) != 0ull) return 0;
	const int nv = n_cols / vec;
	if ((nv + RMS_CH - 1) / RMS_CH > RMS_MAX_TPR) return 0;
	return nv;
}

/* element path: threads per row slot. The dW modes (whose slots each keep an
 * n_cols-float partial row in LDS, so that only one slot fits per workgroup
 * once rows are long) use one slot of RMS_MAX_TPR threads from
 * RMS_STREAM_WIDE_COLS columns on */
#define RMS_STREAM_WIDE_COLS 4096
GEOM_FN int rms_stream_tpr(int dw_mode, int n_cols) {
	return (dw_mode && n_cols >= RMS_STREAM_WIDE_COLS) ? RMS_MAX_TPR : RMS_STREAM_TPR;
}

GEOM_FN int rms_tpr_for(int nv) {
	if (nv == 0) return RMS_STREAM_TPR;
	const int t = (nv + RMS_CH - 1) / RMS_CH;
	return ((t + 63) / 64) * 64;
}

/* Row slots per CU for the row-streaming RMSNorm ops: each slot keeps two rows
 * of `arrays` input rows in flight (the current one and the prefetched next
 * one), and about RMS_INFLIGHT_BYTES outstanding per CU measured best: more
 * concurrent row streams only add DRAM page misses. */
GEOM_FN long rms_slots_per_cu(int n_cols, long elem, int arrays) {
	const long per_slot = 2L * (long) n_cols * elem * (long) arrays;
	const long s = per_slot > 0 ? (long) RMS_INFLIGHT_BYTES / per_slot : 1;
	return s < 1 ? 1 : (s > 32 ? 32 : s);
}

/* Launch shape of the dW ops (bwd_w: arrays = 2, fused bwd: arrays = 3) for
 * n_rows >= 1 and n_cols >= 1: one workgroup per CU holding the CU's row
 * slots, so each workgroup writes one fp32 partial row. nv is
 * rms_vec_chunks(); max_lds the LDS bytes a workgroup may use; scratch_floats
 * the size of the partial-row buffer. Fills grid, block and dynamic LDS bytes
 * and returns 0, or -1 when the LDS cannot hold a row's partial sums, -2 when
 * one partial row does not fit the buffer. */
GEOM_FN int rms_dw_geometry(int n_rows, int n_cols, long elem, int nv, int arrays, long cu_count, long max_lds,
							long scratch_floats, unsigned * grid, unsigned * block, unsigned * lds) {
	const int tpr = (nv > 0) ? rms_tpr_for(nv) : rms_stream_tpr(1, n_cols);
	const long by_slots = rms_slots_per_cu(n_cols, elem, arrays);
	const long by_threads = (RMS_MAX_TPR / tpr) < 1 ? 1 : (RMS_MAX_TPR / tpr);
	int slots = (int) (by_slots < by_threads ? by_slots : by_threads);
	long bytes = 0;
	for (; slots >= 1; slots--) {
		const long colbuf = (nv > 0) ? (long) n_cols : (long) slots * n_cols;
		bytes = ((long) RMS_CELLS_PER_SLOT * slots + colbuf) * (long) sizeof(float);
		if (bytes <= max_lds) break;
	}
	if (slots < 1) return -1;
	const long max_parts = scratch_floats / (long) n_cols;
	if (max_parts < 1) return -2;
	long g = ((long) n_rows + slots - 1) / slots;
	if (g > cu_count) g = cu_count;
	if (g > max_parts) g = max_parts;
	*grid = (unsigned) g;
	*block = (unsigned) (slots * tpr);
	*lds = (unsigned) bytes;
	return 0;
}

/* fp8 x 16-bit RMSNorm backward: threads per row slot for the chunked path,
 * or 0 when rows must take the element path */
GEOM_FN int f8_row_tpr(int n_cols) {
	if (n_cols <= 0 || (n_cols % 8) != 0) return 0;
	const int t = (n_cols / 8 + F8_CPT - 1) / F8_CPT;
	const int tpr = ((t + 63) / 64) * 64;
	return tpr <= 1024 ? tpr : 0;
}

/* fp8 -> 16-bit softmax, long rows (fp8_ops.hip, softmax_fp8_pf): one
 * SMX_THREADS workgroup per CU holding the row in registers (F8_PF_PIECES
 * 8-byte pieces per thread) while the next row streams in, half into LDS and
 * half into registers; rows of a multiple of 16 columns from F8_PF_MIN_COLS
 * up to 8 * F8_PF_PIECES * SMX_THREADS */
#define F8_PF_PIECES 16
#define F8_PF_MIN_COLS 32768
GEOM_FN int f8_smx_pf_ok(int n_cols) {
	return n_cols >= F8_PF_MIN_COLS && (n_cols % 16) == 0 && n_cols / 8 <= F8_PF_PIECES * SMX_THREADS;
}

GEOM_FN int f8_smx_regs_ok(int n_cols) {
	return n_cols > 0 && (n_cols % 8) == 0 && n_cols / 8 <= F8_SMX_CH * F8_SMX_THREADS;
}

/* RoPE vector path: tokens per workgroup step. fp8 rows are half as long as
 * bf16 ones, so two tokens go together when their Q and K chunks fit the
 * slot's registers. */
#define ROPE_TG2_QJ 2   /* Q chunks per thread in a two-token step */
GEOM_FN int rope_tokens_per_group(int model_dim, int kv_dim, int elem_bytes) {
	if (elem_bytes != 1) return 1;
	return (2 * (model_dim / 16) <= ROPE_SLOT_THREADS * ROPE_TG2_QJ && 2 * (kv_dim / 16) <= ROPE_SLOT_THREADS * ROPE_KJ) ? 2 : 1;
}

/* RoPE: whether the vector (slot) path applies */
GEOM_FN int rope_slot_ok(int model_dim, int kv_dim, int head_dim, int elem_bytes, unsigned long long ptr_or) {
	const int vec = 16 / elem_bytes;
	if ((head_dim % vec) != 0 || (ptr_or & 15ull) != 0ull) return 0;
	return (model_dim / vec) <= ROPE_SLOT_THREADS * ROPE_QJ && (kv_dim / vec) <= ROPE_SLOT_THREADS * ROPE_KJ;
}

#endif
