/*
 * Launch geometry of the gfx950 kernels (dlopen'ed by the HIP backend).
 * One "<op>_set_launch_config" per op family, as the reference's
 * src/ops/nvidia/{norm/rms_norm_config.c, attention/attn_misc_config.c,
 * activations/swiglu_config.c, loss/loss_misc_config.c}; the geometry itself is
 * chosen for CDNA (wave64, CU count, LDS) and shared with the kernels through
 * kernel_geometry.h. Every function validates the arguments the kernel relies
 * on and returns -1 with a message instead of launching out of range.
 */
#include "hip_ops_config.h"
#include "kernel_geometry.h"

#define ARG(op, i, type) (*((type *) (op)->op_args[(i)]))

static void set_1d(Hip_Launch_Config * c, unsigned grid, unsigned block, unsigned lds) {
	c->gridDimX = grid;
	c->gridDimY = 1;
	c->gridDimZ = 1;
	c->blockDimX = block;
	c->blockDimY = 1;
	c->blockDimZ = 1;
	c->sharedMemBytes = lds;
}

static const Hip_Device_Info * dev(Dataflow_Handle * h) { return (const Hip_Device_Info *) h->device_info; }

static size_t arg_elem_bytes(Hip_Function * f, int i) {
	return dataflow_sizeof_element(f->op_skeleton.header.arg_dtypes[i]);
}

static unsigned long long ptr_bits(const void * p) { return (unsigned long long) (uintptr_t) p; }

/* ---------------- RMSNorm ---------------- */

int rms_norm_set_attribute_config(Dataflow_Handle * dataflow_handle, Hip_Function * hip_function) {
	/* LDS needs no opt-in on CDNA: every function may use the per-workgroup maximum */
	hip_function->function_config.func_max_smem = dev(dataflow_handle)->max_smem_per_block;
	int max_threads = 0;
	if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, hip_function->function_handle) != hipSuccess) {
		fprintf(stderr, "Error: could not get rms norm attribute for max_threads_per_block...\n");
		return -1;
	}
	hip_function->function_config.func_max_threads_per_block = max_threads;
	/* the dW ops (bwd_w and the fused bwd, not bwd_x) reduce through the
	 * module's partial-row scratch */
	const char * nick = hip_function->op_skeleton.header.op_nickname;
	hip_function->function_config.shares_module_scratch =
		strncmp(nick, "rms_norm_bwd_", 13) == 0 && strncmp(nick, "rms_norm_bwd_x_", 15) != 0;
	return 0;
}

static int rms_check(const char * what, int n_rows, int n_cols, size_t elem) {
	if (n_rows < 0 || n_cols < 0 || elem == 0) {
		fprintf(stderr, "Error: %s: invalid shape (%d x %d) or dtype...\n", what, n_rows, n_cols);
		return -1;
	}
	return 0;
}

/* workgroups of this function that are resident on the whole device at once;
 * the occupancy query is remembered per function for the last (block, LDS)
 * pair asked, so repeated submits of one shape do not repeat it */
static long resident_groups(Dataflow_Handle * h, Hip_Function * f, int block, size_t lds) {
	const uint64_t key = ((uint64_t) (unsigned) block << 40) | ((uint64_t) (lds & 0xffffffull) << 16);
	const uint64_t memo = __atomic_load_n(&f->function_config.occupancy_memo, __ATOMIC_RELAXED);
	int per_cu = 0;
	if (memo != 0 && (memo & ~0xffffull) == key) {
		per_cu = (int) (memo & 0xffffull);
	}
	else {
		if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f->function_handle, block, lds) != hipSuccess || per_cu < 1) per_cu = 1;
		if (lds <= 0xffffffull && per_cu <= 0xffff) __atomic_store_n(&f->function_config.occupancy_memo, key | (uint64_t) per_cu, __ATOMIC_RELAXED);
	}
	return (long) per_cu * (long) dev(h)->cu_count;
}

/* fwd / bwd_x: ~256-thread workgroups, as many per CU as the slot target
 * asks; the fp8 forward takes ~512-thread ones (8192 x 4096: 13.5 against
 * 14.0 us; the 16-bit forward is the same either way and bwd_x slower) */
static void rms_rowwise(Hip_Launch_Config * c, Dataflow_Handle * h, Hip_Function * f, int n_rows, int n_cols, size_t elem, int nv, int arrays) {
	const int tpr = rms_tpr_for(nv);
	const int slots = MY_MAX(1, ((arrays == 1 && elem == 1) ? 512 : 256) / tpr);
	const unsigned block = (unsigned) (slots * tpr);
	const unsigned lds = (unsigned) (RMS_CELLS_PER_SLOT * slots * sizeof(float));
	/* the element path (nv == 0) walks its rows with plain loads and keeps no
	 * row in flight ahead, so it needs many rows per CU to hide latency */
	const long groups_per_cu = (nv == 0) ? RMS_STREAM_GROUPS_PER_CU : MY_CEIL(rms_slots_per_cu(n_cols, (long) elem, arrays), (long) slots);
	long grid = MY_MIN((long) MY_CEIL(n_rows, slots), (long) dev(h)->cu_count * groups_per_cu);
	grid = MY_MIN(grid, resident_groups(h, f, (int) block, lds));
	set_1d(c, (unsigned) grid, block, lds);
}

int rms_norm_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const int n_rows = ARG(op, 0, int), n_cols = ARG(op, 1, int);
	const size_t elem = arg_elem_bytes(hip_function, 3);
	if (rms_check("rms norm", n_rows, n_cols, elem)) return -1;
	const int nv = rms_vec_chunks(n_cols, (int) elem, ptr_bits(ARG(op, 3, void *)) | ptr_bits(ARG(op, 4, void *)) | ptr_bits(ARG(op, 5, void *)));
	rms_rowwise(hip_launch_config, dataflow_handle, hip_function, (n_cols == 0) ? 0 : n_rows, n_cols, elem, nv, 1);
	return 0;
}

static int is_fp8(Hip_Function * f, int i) {
	const DataflowDatatype dt = f->op_skeleton.header.arg_dtypes[i];
	return dt == DATAFLOW_FP8E4M3 || dt == DATAFLOW_FP8E5M2;
}

/* fp8 x 16-bit variants (fp8_ops.hip): one 256-thread workgroup per row at a
 * time, eight elements per lane, four workgroups per CU */
static void rms_fp8_rowwise(Hip_Launch_Config * c, Dataflow_Handle * h, int n_rows, int n_cols) {
	const long grid = (n_cols == 0) ? 0 : MY_MIN((long) n_rows, (long) dev(h)->cu_count * 4);
	set_1d(c, (unsigned) grid, 256, 0);
}

int rms_norm_bwd_x_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const int n_rows = ARG(op, 0, int), n_cols = ARG(op, 1, int);
	const size_t elem = arg_elem_bytes(hip_function, 5);
	if (rms_check("rms norm bwd x", n_rows, n_cols, elem)) return -1;
	if (is_fp8(hip_function, 5)) {
		const int tpr = f8_row_tpr(n_cols);
		const int vec = tpr > 0 && ((ptr_bits(ARG(op, 5, void *)) | ptr_bits(ARG(op, 6, void *))) & 7ull) == 0 &&
						((ptr_bits(ARG(op, 7, void *)) | ptr_bits(ARG(op, 8, void *))) & 15ull) == 0;
		if (!vec) {
			rms_fp8_rowwise(hip_launch_config, dataflow_handle, n_rows, n_cols);
			return 0;
		}
		/* row slots of tpr threads, 256-thread workgroups */
		const int slots = MY_MAX(1, 256 / tpr);
		const long grid = MY_MIN((long) MY_CEIL(n_rows, slots), (long) dev(dataflow_handle)->cu_count * F8_BWDX_WG_PER_CU);
		set_1d(hip_launch_config, (unsigned) grid, (unsigned) (slots * tpr), 0);
		return 0;
	}
	const int nv = rms_vec_chunks(n_cols, (int) elem, ptr_bits(ARG(op, 5, void *)) | ptr_bits(ARG(op, 6, void *)) |
													ptr_bits(ARG(op, 7, void *)) | ptr_bits(ARG(op, 8, void *)));
	rms_rowwise(hip_launch_config, dataflow_handle, hip_function, (n_cols == 0) ? 0 : n_rows, n_cols, elem, nv, 3);
	return 0;
}

/* two-pass dW ops: slots and grid so LDS and the partial scratch fit
 * (rms_dw_geometry, shared with the allocation-free entry point) */
static int rms_dw_config(Hip_Launch_Config * c, Dataflow_Handle * h, Hip_Function * f, const char * what, int n_rows, int n_cols, size_t elem, int nv, int arrays) {
	if (n_rows == 0 || n_cols == 0) {
		set_1d(c, 0, 1, 0);
		return 0;
	}
	const long max_lds = f->function_config.func_max_smem > 0 ? f->function_config.func_max_smem : dev(h)->max_smem_per_block;
	unsigned grid = 0, block = 0, lds = 0;
	const int rc = rms_dw_geometry(n_rows, n_cols, (long) elem, nv, arrays, (long) dev(h)->cu_count, max_lds,
								   (long) RMS_DW_SCRATCH_FLOATS, &grid, &block, &lds);
	if (rc == -1) {
		fprintf(stderr, "Error: %s: rows of %d columns need more LDS than the %ld bytes available...\n", what, n_cols, max_lds);
		return -1;
	}
	if (rc != 0) {
		fprintf(stderr, "Error: %s: %d columns exceed the dW scratch of %u floats...\n", what, n_cols, (unsigned) RMS_DW_SCRATCH_FLOATS);
		return -1;
	}
	set_1d(c, grid, block, lds);
	return 0;
}

static int rms_dw_finish_config(Hip_Launch_Config * c, int n_rows, int n_cols) {
	if (n_rows == 0 || n_cols == 0) {
		set_1d(c, 0, 1, 0);
		return 0;
	}
	set_1d(c, (unsigned) MY_CEIL(n_cols, RMS_FIN_COLS), RMS_FINISH_THREADS, 0);
	return 0;
}

int rms_norm_bwd_w_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const int n_rows = ARG(op, 0, int), n_cols = ARG(op, 1, int);
	const size_t elem = arg_elem_bytes(hip_function, 4);
	if (rms_check("rms norm bwd w", n_rows, n_cols, elem)) return -1;
	if (is_fp8(hip_function, 4)) {
		/* fp8 X: one workgroup per CU, each adding its rows into one partial
		 * row of n_cols floats (combined in LDS) */
		if (n_rows == 0 || n_cols == 0) {
			set_1d(hip_launch_config, 0, 1, 0);
			return 0;
		}
		const long lds = (long) n_cols * (long) sizeof(float);
		const long max_lds = hip_function->function_config.func_max_smem > 0 ? hip_function->function_config.func_max_smem
																		   : dev(dataflow_handle)->max_smem_per_block;
		if (lds > max_lds || n_cols > (long) RMS_DW_SCRATCH_FLOATS) {
			fprintf(stderr, "Error: rms norm bwd w: rows of %d columns need more LDS than the %ld bytes available...\n", n_cols, max_lds);
			return -1;
		}
		/* aligned rows of up to 8 * F8_CPT * 1024 columns: row slots of tpr
		 * threads, as many as fill 1024 threads; otherwise 256 threads
		 * walking each row */
		const int tpr = f8_row_tpr(n_cols);
		const int vec = tpr > 0 && (ptr_bits(ARG(op, 4, void *)) & 7ull) == 0 && (ptr_bits(ARG(op, 5, void *)) & 15ull) == 0;
		const int slots = vec ? MY_MAX(1, 1024 / tpr) : 1;
		long grid = MY_MIN((long) MY_CEIL(n_rows, slots), (long) dev(dataflow_handle)->cu_count);
		grid = MY_MIN(grid, (long) RMS_DW_SCRATCH_FLOATS / (long) n_cols);
		set_1d(hip_launch_config, (unsigned) grid, vec ? (unsigned) (slots * tpr) : 256u, (unsigned) lds);
		return 0;
	}
	const int nv = rms_vec_chunks(n_cols, (int) elem, ptr_bits(ARG(op, 4, void *)) | ptr_bits(ARG(op, 5, void *)));
	return rms_dw_config(hip_launch_config, dataflow_handle, hip_function, "rms norm bwd w", n_rows, n_cols, elem, nv, 2);
}

int rms_norm_bwd_w_set_finish_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	(void) dataflow_handle;
	(void) hip_function;
	return rms_dw_finish_config(hip_launch_config, ARG(op, 0, int), ARG(op, 1, int));
}

int rms_norm_bwd_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const int n_rows = ARG(op, 0, int), n_cols = ARG(op, 1, int);
	const size_t elem = arg_elem_bytes(hip_function, 5);
	if (rms_check("rms norm bwd", n_rows, n_cols, elem)) return -1;
	const int nv = rms_vec_chunks(n_cols, (int) elem, ptr_bits(ARG(op, 4, void *)) | ptr_bits(ARG(op, 5, void *)) |
													ptr_bits(ARG(op, 6, void *)) | ptr_bits(ARG(op, 7, void *)));
	return rms_dw_config(hip_launch_config, dataflow_handle, hip_function, "rms norm bwd", n_rows, n_cols, elem, nv, 3);
}

int rms_norm_bwd_set_finish_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	(void) dataflow_handle;
	(void) hip_function;
	return rms_dw_finish_config(hip_launch_config, ARG(op, 0, int), ARG(op, 1, int));
}

/* ---------------- RoPE ---------------- */

static int rope_config(Hip_Launch_Config * c, Dataflow_Handle * h, Hip_Function * f, Op * op, const char * what,
					   unsigned long long extra_ptr_bits) {
	const uint64_t N = ARG(op, 0, uint64_t);
	const int model_dim = ARG(op, 1, int), head_dim = ARG(op, 2, int), num_kv_heads = ARG(op, 3, int);
	if (model_dim <= 0 || head_dim <= 0 || (head_dim & 1) || head_dim > ROPE_MAX_HEAD_DIM || (model_dim % head_dim) != 0 ||
		num_kv_heads < 0 || (N % (uint64_t) model_dim) != 0) {
		fprintf(stderr, "Error: %s: unsupported shape N=%lu model_dim=%d head_dim=%d num_kv_heads=%d "
				"(need even head_dim <= %d dividing model_dim, and N a multiple of model_dim)...\n",
				what, (unsigned long) N, model_dim, head_dim, num_kv_heads, ROPE_MAX_HEAD_DIM);
		return -1;
	}
	const uint64_t n_tokens = N / (uint64_t) model_dim;
	const size_t elem = arg_elem_bytes(f, 6);
	const unsigned long long ptr_or = ptr_bits(ARG(op, 6, void *)) | ptr_bits(ARG(op, 7, void *));
	uint64_t grid;
	if (elem != 0 && rope_slot_ok(model_dim, num_kv_heads * head_dim, head_dim, (int) elem, ptr_or | extra_ptr_bits)) {
		/* vector path: one workgroup per token at a time, persistent, as many
		 * per CU as the kernel's registers allow (at most ROPE_SLOT_WG_PER_CU) */
		grid = MY_MIN((uint64_t) dev(h)->cu_count * ROPE_SLOT_WG_PER_CU, (uint64_t) resident_groups(h, f, ROPE_SLOT_THREADS, 0));
		const uint64_t tg = (uint64_t) rope_tokens_per_group(model_dim, num_kv_heads * head_dim, (int) elem);
		grid = MY_MIN(MY_CEIL(n_tokens, tg), grid);
		set_1d(c, (unsigned) grid, ROPE_SLOT_THREADS, 0);
		return 0;
	}
	/* element path: one wave per token, looping; four workgroups per CU */
	grid = MY_CEIL(n_tokens, (uint64_t) ROPE_WAVES);
	grid = MY_MIN(grid, (uint64_t) dev(h)->cu_count * 4u);
	set_1d(c, (unsigned) grid, 64 * ROPE_WAVES, 0);
	return 0;
}

int rope_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	return rope_config(hip_launch_config, dataflow_handle, hip_function, op, "rope", 0ull);
}

int rope_bwd_x_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	return rope_config(hip_launch_config, dataflow_handle, hip_function, op, "rope bwd x", 0ull);
}

/* RoPE + KV-cache scatter: rope's shapes, and the same path choice with the
 * values pointer's alignment (the context rows are checked per token) */
int rope_copy_to_seq_context_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	if (ARG(op, 3, int) > 0 && (!ARG(op, 8, void *) || !ARG(op, 9, void *) || !ARG(op, 10, void *))) {
		fprintf(stderr, "Error: rope copy to seq context: values, context pointers and context sizes are required...\n");
		return -1;
	}
	return rope_config(hip_launch_config, dataflow_handle, hip_function, op, "rope copy to seq context", ptr_bits(ARG(op, 8, void *)));
}

/* ---------------- embedding / copy_to_seq_context ---------------- */

/* one wave per row, looping; eight workgroups of GS_WAVES waves per CU */
static void gs_config(Hip_Launch_Config * c, Dataflow_Handle * h, uint64_t n_rows) {
	uint64_t grid = MY_CEIL(n_rows, (uint64_t) GS_WAVES);
	grid = MY_MIN(grid, (uint64_t) dev(h)->cu_count * 8u);
	set_1d(c, (unsigned) grid, 64 * GS_WAVES, 0);
}

/* reference: src/ops/nvidia/preprocess/embedding_config.c:3-40 */
int embedding_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const int num_tokens = ARG(op, 0, int), embed_dim = ARG(op, 1, int);
	const size_t elem = arg_elem_bytes(hip_function, 3);
	if (elem == 0) {
		fprintf(stderr, "Error: embedding not available for dtype %s...\n",
				dataflow_datatype_as_string(hip_function->op_skeleton.header.arg_dtypes[3]));
		return -1;
	}
	if (num_tokens < 0 || embed_dim < 0 || (uint64_t) embed_dim * elem > 0xffffffffull) {
		fprintf(stderr, "Error: embedding: invalid shape (%d tokens x %d)...\n", num_tokens, embed_dim);
		return -1;
	}
	gs_config(hip_launch_config, dataflow_handle, (embed_dim == 0) ? 0 : (uint64_t) num_tokens);
	return 0;
}

/* reference: src/ops/nvidia/attention/attn_misc_config.c:56-80 */
int copy_to_seq_context_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const uint64_t N = ARG(op, 0, uint64_t);
	const int kv_dim = ARG(op, 2, int);
	const size_t elem = arg_elem_bytes(hip_function, 3);
	if (elem == 0 || kv_dim <= 0 || (N % (uint64_t) kv_dim) != 0 || (uint64_t) kv_dim * elem > 0xffffffffull) {
		fprintf(stderr, "Error: copy to seq context: unsupported N=%lu kv_dim=%d (need kv_dim > 0 dividing N)...\n",
				(unsigned long) N, kv_dim);
		return -1;
	}
	gs_config(hip_launch_config, dataflow_handle, N / (uint64_t) kv_dim);
	return 0;
}

/* ---------------- SwiGLU ---------------- */

static int swiglu_config(Hip_Launch_Config * c, Dataflow_Handle * h, Hip_Function * f, Op * op, const char * what) {
	const int rows = ARG(op, 0, int), cols = ARG(op, 1, int);
	const size_t elem = arg_elem_bytes(f, 2);
	if (rows < 0 || cols < 0 || elem == 0) {
		fprintf(stderr, "Error: %s: invalid shape (%d x %d) or dtype...\n", what, rows, cols);
		return -1;
	}
	const long n = (long) rows * (long) cols;
	const long chunks = MY_CEIL(n, (long) (16 / elem));
	/* the smaller of the two steps, so neither direction gets fewer threads than chunks per step */
	long grid = MY_CEIL(chunks, (long) SWIGLU_THREADS * MY_MIN(SWIGLU_FWD_UNROLL, SWIGLU_BWD_UNROLL));
	grid = MY_MIN(grid, (long) dev(h)->cu_count * SWIGLU_WG_PER_CU);
	set_1d(c, (unsigned) grid, SWIGLU_THREADS, 0);
	return 0;
}

int swiglu_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	return swiglu_config(hip_launch_config, dataflow_handle, hip_function, op, "swiglu");
}

int swiglu_bwd_x_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	return swiglu_config(hip_launch_config, dataflow_handle, hip_function, op, "swiglu bwd x");
}

/* ---------------- softmax / cross-entropy ---------------- */

/* The softmax kernels (softmax_xent.hip, and the fp8 softmax in fp8_ops.hip
 * on its long-row path) hand rows out from a counter in the code object and
 * count finished workgroups there, so the handle orders them across its
 * streams. */
int softmax_set_attribute_config(Dataflow_Handle * dataflow_handle, Hip_Function * hip_function) {
	(void) dataflow_handle;
	hip_function->function_config.shares_module_scratch = 1;
	return 0;
}

/* one workgroup per row; small rows get a smaller workgroup */
static int smx_config(Hip_Launch_Config * c, Dataflow_Handle * h, Hip_Function * f, int n_rows, int n_cols, const char * what) {
	const size_t elem = arg_elem_bytes(f, 2);
	if (n_rows < 0 || n_cols < 0 || elem == 0) {
		fprintf(stderr, "Error: %s: invalid shape (%d x %d) or dtype...\n", what, n_rows, n_cols);
		return -1;
	}
	if (n_rows == 0 || n_cols == 0) {
		set_1d(c, 0, 1, 0);
		return 0;
	}
	/* persistent over rows: one workgroup of SMX_THREADS per CU (a row fills
	 * its VGPRs and half its LDS) */
	const long grid = MY_MIN((long) n_rows, (long) dev(h)->cu_count);
	set_1d(c, (unsigned) grid, SMX_THREADS, 0);
	return 0;
}

int softmax_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	const int n_rows = ARG(op, 0, int), n_cols = ARG(op, 1, int);
	if (smx_config(hip_launch_config, dataflow_handle, hip_function, n_rows, n_cols, "softmax")) return -1;
	/* fp8 logits: long rows keep smx_config's one SMX_THREADS workgroup per CU
	 * (the next row prefetched into LDS); other rows that fit the registers
	 * take two smaller workgroups per CU */
	if (is_fp8(hip_function, 2) && n_rows > 0 && !f8_smx_pf_ok(n_cols) && f8_smx_regs_ok(n_cols) &&
		((ptr_bits(ARG(op, 2, void *)) | ptr_bits(ARG(op, 3, void *))) & 15ull) == 0) {
		const long grid = MY_MIN((long) n_rows, 2L * (long) dev(dataflow_handle)->cu_count);
		set_1d(hip_launch_config, (unsigned) grid, F8_SMX_THREADS, 0);
	}
	return 0;
}

int softmax_cross_entropy_loss_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	if (ARG(op, 5, float *) && !ARG(op, 4, float *)) {
		fprintf(stderr, "Error: softmax cross entropy loss: mean_loss needs the per-row loss buffer...\n");
		return -1;
	}
	return smx_config(hip_launch_config, dataflow_handle, hip_function, ARG(op, 0, int), ARG(op, 1, int), "softmax cross entropy loss");
}

int cross_entropy_loss_set_launch_config(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op) {
	(void) dataflow_handle;
	(void) hip_function;
	const int n_rows = ARG(op, 0, int);
	if (n_rows < 0) {
		fprintf(stderr, "Error: cross entropy loss: invalid n_rows %d...\n", n_rows);
		return -1;
	}
	set_1d(hip_launch_config, (unsigned) MY_CEIL(n_rows, 256), 256, 0);
	return 0;
}
