/*
 * CPU backend of Dataflow_Handle over the oracle — TEST INFRASTRUCTURE ONLY.
 *
 * Fills the COMPUTE_CPU slot of the reference's ComputeType
 * (src/dataflow_handle/include/dataflow_handle.h:19; the reference has no CPU
 * backend) so that the registry, fingerprint dispatch and argument marshalling
 * of the product library run in a GPU-less process: register_native_code
 * dlopens this library and looks up "<op>_<dt>_kernel" adapters below, each of
 * which reads op_args exactly as the GPU kernel does and runs the oracle.
 * Everything is synchronous; streams are accepted and ignored.
 */
#include "dataflow_handle.h"
#include "fingerprint.h"
#include "oracle.h"

#include <math.h>

typedef int (*Cpu_Kernel)(void ** op_args);

typedef struct cpu_function {
	Cpu_Kernel fn;
	Op_Skeleton op_skeleton;
} Cpu_Function;

static uint64_t cpu_hash(void * fp, uint64_t size) {
	return fingerprint_to_least_sig64((uint8_t *) fp, OP_IDENTIFIER_FINGERPRINT_NUM_BYTES) % size;
}

static int cpu_register_native_code(Dataflow_Handle * h, char * code_filename, char * config_filename, int num_funcs,
									Op_Skeleton * skeletons, char ** symbols, char ** launch_symbols, char ** init_symbols) {
	(void) config_filename;
	(void) launch_symbols;
	(void) init_symbols;
	void * lib = dlopen(code_filename, RTLD_LAZY | RTLD_LOCAL);
	if (!lib) {
		fprintf(stderr, "Error: cpu backend could not open %s (%s)\n", code_filename, dlerror());
		return -1;
	}
	int added = 0;
	for (int i = 0; i < num_funcs; i++) {
		if (!symbols[i]) continue;
		Cpu_Function f;
		memset(&f, 0, sizeof(f));
		f.fn = (Cpu_Kernel) dlsym(lib, symbols[i]);
		if (!f.fn) {
			fprintf(stderr, "Error: cpu backend has no function %s\n", symbols[i]);
			continue;
		}
		memcpy(&f.op_skeleton, &skeletons[i], sizeof(Op_Skeleton));
		if (insert_table(&h->op_table, f.op_skeleton.identifier.fingerprint, &f)) continue;
		added++;
	}
	if (added == 0) return -1;
	h->native_function_libs[h->num_native_function_libs++] = lib;
	h->num_ops += added;
	return added;
}

static int cpu_submit_op(Dataflow_Handle * h, Op * op, int stream_id) {
	if (stream_id < -1 || stream_id >= h->num_streams) {
		fprintf(stderr, "cpu backend: stream id %d (op %s) is out of range: %d streams, -1 for the null stream\n",
				stream_id, op->op_skeleton.header.op_nickname, h->num_streams);
		return -1;
	}
	Cpu_Function * f = NULL;
	if (find_table(&h->op_table, op->op_skeleton.identifier.fingerprint, false, (void **) &f) == -1 || !f) {
		fprintf(stderr, "Error: failed to find op with nickname %s and matching dtypes...\n", op->op_skeleton.header.op_nickname);
		return -1;
	}
	return f->fn(op->op_args) ? -1 : 0;
}

static void * cpu_alloc(Dataflow_Handle * h, uint64_t n) { (void) h; return malloc(n ? n : 1); }
static void cpu_free(Dataflow_Handle * h, void * p) { (void) h; free(p); }
static int cpu_set_mem(Dataflow_Handle * h, int s, void * p, uint8_t v, uint64_t n) { (void) h; (void) s; memset(p, v, n); return 0; }
static int cpu_copy(Dataflow_Handle * h, int s, void * dst, void * src, uint64_t n) { (void) h; (void) s; memcpy(dst, src, n); return 0; }
static int cpu_sync_stream(Dataflow_Handle * h, int s) { (void) h; (void) s; return 0; }
static int cpu_sync_handle(Dataflow_Handle * h) { (void) h; return 0; }

int init_cpu_dataflow_handle(Dataflow_Handle * h, int num_streams) {
	memset(h, 0, sizeof(*h));
	h->compute_type = COMPUTE_CPU;
	h->device_id = -1;
	h->num_streams = num_streams;
	for (int i = 0; i < MAX_STREAMS; i++) h->stream_prios[i] = -1;
	if (init_table(&h->op_table, cpu_hash, OP_IDENTIFIER_FINGERPRINT_NUM_BYTES, sizeof(Cpu_Function),
					OP_TABLE_MIN_SIZE, OP_TABLE_MAX_SIZE, 1.0f, 1.0f)) {
		return -1;
	}
	h->register_native_code = cpu_register_native_code;
	h->submit_op = cpu_submit_op;
	h->sync_stream = cpu_sync_stream;
	h->sync_handle = cpu_sync_handle;
	h->alloc_mem = cpu_alloc;
	h->free_mem = cpu_free;
	h->set_mem = cpu_set_mem;
	h->submit_inbound_transfer = cpu_copy;
	h->submit_outbound_transfer = cpu_copy;
	h->submit_peer_transfer = cpu_copy;
	return 0;
}

int destroy_cpu_dataflow_handle(Dataflow_Handle * h) {
	destroy_table(&h->op_table);
	for (int i = 0; i < h->num_native_function_libs; i++) dlclose(h->native_function_libs[i]);
	h->num_native_function_libs = 0;
	return 0;
}

/* ---------------- kernel-symbol adapters ---------------- */

#define A(i, type) (*((type *) op_args[(i)]))

static double * dbuf(long n) { return (double *) malloc(sizeof(double) * (size_t) (n > 0 ? n : 1)); }

static int rms_norm_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	float * ws = A(6, float *), * rs = A(7, float *);
	const long n = (long) n_rows * n_cols;
	double * y = dbuf(n), * w = dbuf(n_rows), * r = dbuf(n_rows);
	int ret = oracle_rms_norm(dt, n_rows, n_cols, A(2, float), A(3, void *), A(4, void *), y, w, r, NULL);
	if (!ret) {
		oracle_store(dt, y, n, A(5, void *));
		for (int i = 0; i < n_rows; i++) {
			if (ws) ws[i] = (float) w[i];
			if (rs) rs[i] = (float) r[i];
		}
	}
	free(y); free(w); free(r);
	return ret;
}

static int rms_norm_bwd_x_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	const long n = (long) n_rows * n_cols;
	double * v = dbuf(n);
	int ret = oracle_rms_norm_bwd_x_exact(dt, n_rows, n_cols, A(3, float *), A(4, float *), A(5, void *), A(6, void *),
											A(7, void *), A(8, void *), v);
	if (!ret) oracle_store(dt, v, n, A(8, void *));
	free(v);
	return ret;
}

static int rms_norm_bwd_w_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	double * v = dbuf(n_cols);
	int ret = oracle_rms_norm_bwd_w(dt, dt, n_rows, n_cols, A(3, float *), A(4, void *), A(5, void *), A(6, void *), v, NULL);
	if (!ret) oracle_store(dt, v, n_cols, A(6, void *));
	free(v);
	return ret;
}

static int rms_norm_bwd_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	const long n = (long) n_rows * n_cols;
	double * dx = dbuf(n), * dw = dbuf(n_cols);
	float * dW = A(8, float *);
	int ret = oracle_rms_norm_bwd(dt, n_rows, n_cols, A(3, float *), A(4, void *), A(5, void *), A(6, void *), A(7, void *),
									dW, dx, NULL, dw, NULL);
	if (!ret) {
		oracle_store(dt, dx, n, A(7, void *));
		for (int j = 0; j < n_cols; j++) dW[j] = (float) dw[j];
	}
	free(dx); free(dw);
	return ret;
}

static int rope_adapter(int dt, int bwd, void ** op_args) {
	const uint64_t N = A(0, uint64_t);
	const int model_dim = A(1, int), head_dim = A(2, int), nkv = A(3, int);
	if (model_dim <= 0 || head_dim <= 0) return -1;
	const long nq = (long) N, nk = (long) (N / (uint64_t) model_dim) * nkv * head_dim;
	double * q = dbuf(nq), * k = dbuf(nk);
	int ret = oracle_rope(dt, bwd, N, model_dim, head_dim, nkv, A(4, int), A(5, int *), A(6, void *), A(7, void *), q, k);
	if (!ret) {
		oracle_store(dt, q, nq, A(6, void *));
		oracle_store(dt, k, nk, A(7, void *));
	}
	free(q); free(k);
	return ret;
}

static int swiglu_adapter(int dt, void ** op_args) {
	const long n = (long) A(0, int) * A(1, int);
	double * o = dbuf(n);
	int ret = oracle_swiglu(dt, n, A(2, void *), A(3, void *), o);
	if (!ret) oracle_store(dt, o, n, A(4, void *));
	free(o);
	return ret;
}

static int swiglu_bwd_adapter(int dt, void ** op_args) {
	const long n = (long) A(0, int) * A(1, int);
	double * dg = dbuf(n), * du = dbuf(n);
	int ret = oracle_swiglu_bwd(dt, n, A(2, void *), A(3, void *), A(4, void *), dg, NULL, du);
	if (!ret) {
		oracle_store(dt, dg, n, A(5, void *));
		oracle_store(dt, du, n, A(6, void *));
	}
	free(dg); free(du);
	return ret;
}

static int softmax_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	const long n = (long) n_rows * n_cols;
	double * y = dbuf(n);
	int ret = oracle_softmax(dt, dt, n_rows, n_cols, A(2, void *), y);
	if (!ret) oracle_store(dt, y, n, A(3, void *));
	free(y);
	return ret;
}

static int cross_entropy_adapter(int dt, void ** op_args) {
	return oracle_cross_entropy_loss(dt, A(0, int), A(1, int), A(2, void *), A(3, uint32_t *));
}

static int softmax_xent_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	const long n = (long) n_rows * n_cols;
	float * loss = A(4, float *), * mean = A(5, float *);
	double * y = dbuf(n), * l = dbuf(n_rows), m = 0.0;
	int ret = oracle_softmax_cross_entropy_exact(dt, n_rows, n_cols, A(2, void *), A(3, uint32_t *), y, l, &m);
	if (!ret) {
		oracle_store(dt, y, n, A(2, void *));
		for (int r = 0; r < n_rows; r++) if (loss) loss[r] = (float) l[r];
		if (mean) *mean = (float) m;
	}
	free(y); free(l);
	return ret;
}

static int embedding_adapter(int elem_bytes, void ** op_args) {
	return oracle_embedding(elem_bytes, A(0, int), A(1, int), A(2, uint32_t *), A(3, void *), -1, A(4, void *));
}

static int copy_to_seq_context_adapter(int elem_bytes, void ** op_args) {
	return oracle_copy_to_seq_context(elem_bytes, A(0, uint64_t), A(2, int), A(3, void *), A(4, void *), A(5, int *),
										A(6, uint64_t *), A(7, int *));
}

/* rope forward, then the scatter of the rotated K rows and the V rows */
static int rope_copy_to_seq_context_adapter(int dt, int elem_bytes, void ** op_args) {
	int ret = rope_adapter(dt, 0, op_args);
	const int model_dim = A(1, int), head_dim = A(2, int), nkv = A(3, int);
	if (ret || nkv == 0) return ret;
	const uint64_t kv_dim = (uint64_t) nkv * (uint64_t) head_dim;
	const uint64_t n_kv = (A(0, uint64_t) / (uint64_t) model_dim) * kv_dim;
	return oracle_copy_to_seq_context(elem_bytes, n_kv, (int) kv_dim, A(7, void *), A(8, void *), A(5, int *),
										A(9, uint64_t *), A(10, int *));
}

#define ADAPT_MOVE(sfx, bytes)                                                                              \
	int embedding_##sfx##_kernel(void ** a) { return embedding_adapter(bytes, a); }                        \
	int copy_to_seq_context_##sfx##_kernel(void ** a) { return copy_to_seq_context_adapter(bytes, a); }

ADAPT_MOVE(fp32, 4)
ADAPT_MOVE(fp16, 2)
ADAPT_MOVE(bf16, 2)
ADAPT_MOVE(fp8e4m3, 1)
ADAPT_MOVE(fp8e5m2, 1)

#define ADAPT_DT(sfx, pair, code, elem)                                                                          \
	int rms_norm_##sfx##_kernel(void ** a) { return rms_norm_adapter(code, a); }                           \
	int rms_norm_bwd_x_##pair##_kernel(void ** a) { return rms_norm_bwd_x_adapter(code, a); }              \
	int rms_norm_bwd_w_##pair##_kernel(void ** a) { return rms_norm_bwd_w_adapter(code, a); }              \
	int rms_norm_bwd_##pair##_kernel(void ** a) { return rms_norm_bwd_adapter(code, a); }                  \
	int rope_##sfx##_kernel(void ** a) { return rope_adapter(code, 0, a); }                                \
	int rope_bwd_x_##sfx##_kernel(void ** a) { return rope_adapter(code, 1, a); }                          \
	int swiglu_##sfx##_kernel(void ** a) { return swiglu_adapter(code, a); }                               \
	int swiglu_bwd_x_##pair##_kernel(void ** a) { return swiglu_bwd_adapter(code, a); }                    \
	int softmax_##pair##_kernel(void ** a) { return softmax_adapter(code, a); }                            \
	int cross_entropy_loss_##sfx##_kernel(void ** a) { return cross_entropy_adapter(code, a); }            \
	int softmax_cross_entropy_loss_##sfx##_kernel(void ** a) { return softmax_xent_adapter(code, a); }      \
	int rope_copy_to_seq_context_##sfx##_kernel(void ** a) { return rope_copy_to_seq_context_adapter(code, elem, a); }

#define ORACLE_FP32_BYTES 4
#define ORACLE_FP16_BYTES 2
#define ORACLE_BF16_BYTES 2
ADAPT_DT(fp32, fp32_fp32, ORACLE_FP32, ORACLE_FP32_BYTES)
ADAPT_DT(fp16, fp16_fp16, ORACLE_FP16, ORACLE_FP16_BYTES)
ADAPT_DT(bf16, bf16_bf16, ORACLE_BF16, ORACLE_BF16_BYTES)

/* ---- fp8 forward types (OCP E4M3 / E5M2) ---- */

/* the fp8 forward writes sum_j x^2 into the statistic slot and leaves
 * weighted_sums alone (rms_norm.cu:415-659) */
static int rms_norm_fp8_adapter(int dt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	float * ss_out = A(7, float *);
	const long n = (long) n_rows * n_cols;
	double * y = dbuf(n), * ss = dbuf(n_rows);
	int ret = oracle_rms_norm(dt, n_rows, n_cols, A(2, float), A(3, void *), A(4, void *), y, NULL, NULL, NULL);
	if (!ret) ret = oracle_rms_norm_sq_sums(dt, n_rows, n_cols, A(4, void *), ss);
	if (!ret) {
		oracle_store(dt, y, n, A(5, void *));
		for (int i = 0; i < n_rows; i++) if (ss_out) ss_out[i] = (float) ss[i];
	}
	free(y); free(ss);
	return ret;
}

static int rms_norm_bwd_x2_adapter(int fdt, int bdt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	const long n = (long) n_rows * n_cols;
	double * v = dbuf(n);
	int ret = oracle_rms_norm_bwd_x2_exact(fdt, bdt, n_rows, n_cols, A(3, float *), A(4, float *), A(5, void *), A(6, void *),
											A(7, void *), A(8, void *), v);
	if (!ret) oracle_store(bdt, v, n, A(8, void *));
	free(v);
	return ret;
}

static int rms_norm_bwd_w2_adapter(int fdt, int bdt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	double * v = dbuf(n_cols);
	int ret = oracle_rms_norm_bwd_w2(fdt, bdt, bdt, n_rows, n_cols, A(3, float *), A(4, void *), A(5, void *), A(6, void *), v, NULL);
	if (!ret) oracle_store(bdt, v, n_cols, A(6, void *));
	free(v);
	return ret;
}

static int swiglu_bwd2_adapter(int fdt, int bdt, void ** op_args) {
	const long n = (long) A(0, int) * A(1, int);
	double * dg = dbuf(n), * du = dbuf(n);
	int ret = oracle_swiglu_bwd2(fdt, bdt, n, A(2, void *), A(3, void *), A(4, void *), dg, NULL, du);
	if (!ret) {
		oracle_store(bdt, dg, n, A(5, void *));
		oracle_store(bdt, du, n, A(6, void *));
	}
	free(dg); free(du);
	return ret;
}

static int softmax2_adapter(int fdt, int bdt, void ** op_args) {
	const int n_rows = A(0, int), n_cols = A(1, int);
	const long n = (long) n_rows * n_cols;
	double * y = dbuf(n);
	int ret = oracle_softmax(fdt, bdt, n_rows, n_cols, A(2, void *), y);
	if (!ret) oracle_store(bdt, y, n, A(3, void *));
	free(y);
	return ret;
}

#define ADAPT_FP8(sfx, code)                                                                                    \
	int rms_norm_##sfx##_kernel(void ** a) { return rms_norm_fp8_adapter(code, a); }                            \
	int rope_##sfx##_kernel(void ** a) { return rope_adapter(code, 0, a); }                                     \
	int swiglu_##sfx##_kernel(void ** a) { return swiglu_adapter(code, a); }
#define ADAPT_FP8_PAIR(pair, fcode, bcode)                                                                      \
	int rms_norm_bwd_x_##pair##_kernel(void ** a) { return rms_norm_bwd_x2_adapter(fcode, bcode, a); }          \
	int rms_norm_bwd_w_##pair##_kernel(void ** a) { return rms_norm_bwd_w2_adapter(fcode, bcode, a); }          \
	int swiglu_bwd_x_##pair##_kernel(void ** a) { return swiglu_bwd2_adapter(fcode, bcode, a); }                \
	int softmax_##pair##_kernel(void ** a) { return softmax2_adapter(fcode, bcode, a); }

ADAPT_FP8(fp8e4m3, ORACLE_FP8E4M3)
ADAPT_FP8(fp8e5m2, ORACLE_FP8E5M2)
ADAPT_FP8_PAIR(fp8e4m3_fp16, ORACLE_FP8E4M3, ORACLE_FP16)
ADAPT_FP8_PAIR(fp8e4m3_bf16, ORACLE_FP8E4M3, ORACLE_BF16)
ADAPT_FP8_PAIR(fp8e5m2_fp16, ORACLE_FP8E5M2, ORACLE_FP16)
ADAPT_FP8_PAIR(fp8e5m2_bf16, ORACLE_FP8E5M2, ORACLE_BF16)
