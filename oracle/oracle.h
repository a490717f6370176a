/*
 * CPU oracle for the native op path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's kernels with fp64 arithmetic and
 * explicit roundings. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the reported CPU
 * baseline; the product library never links or calls it.
 *
 * dtype codes are DataflowDatatype values: FP32 = 3, FP16 = 4, BF16 = 5,
 * FP8E4M3 = 6, FP8E5M2 = 7 (OCP 8-bit formats; forward-type tensors only:
 * the "2" variants take the forward tensors' type and the backward ones'
 * separately, as the reference's fp8 x {fp16, bf16} kernels do).
 * Outputs named *_pre are the exact value before the final rounding to the
 * output type ("v" of the parity criterion |o - v| <= ulp(v)). Where the
 * reference rounds intermediates, the oracle returns [lo, hi] bounds of that
 * value over the fp32 evaluation error of the quantity being rounded; any
 * correct fp32 implementation lands inside them (the rounding chain is
 * monotone). *_floor outputs are fp32 evaluation-noise bounds for
 * expressions that can cancel.
 *
 * Every function returns 0, or -1 for an unsupported dtype / shape.
 */
#ifndef ORACLE_H
#define ORACLE_H

#include <stdint.h>

#define ORACLE_FP32 3
#define ORACLE_FP16 4
#define ORACLE_BF16 5
#define ORACLE_FP8E4M3 6
#define ORACLE_FP8E5M2 7

double oracle_round(double v, int dt);
double oracle_ulp(double v, int dt);
void oracle_load(int dt, const void * src, long n, double * dst);
void oracle_store(int dt, const double * src, long n, void * dst);
int oracle_num_threads(void);

int oracle_rms_norm(int dt, int n_rows, int n_cols, float eps, const void * W, const void * X,
					double * y_pre, double * ws, double * rstd, double * ws_abs);
int oracle_rms_norm_bwd_x(int dt, int n_rows, int n_cols, const float * ws, const float * rs,
					const void * W, const void * X, const void * dY, const void * dX_in, double * v_lo, double * v_hi);
int oracle_rms_norm_bwd_w(int dt, int dt_w, int n_rows, int n_cols, const float * rs, const void * X, const void * dY,
					const void * dW_in, double * dw_pre, double * dw_abs);
int oracle_rms_norm_sq_sums(int dt, int n_rows, int n_cols, const void * X, double * sq_sums);
int oracle_rms_norm_bwd_x2(int fdt, int dt, int n_rows, int n_cols, const float * ws, const float * rs,
					const void * W, const void * X, const void * dY, const void * dX_in, double * v_lo, double * v_hi);
int oracle_rms_norm_bwd_w2(int fdt, int dt, int dt_w, int n_rows, int n_cols, const float * rs, const void * X, const void * dY,
					const void * dW_in, double * dw_pre, double * dw_abs);
int oracle_rms_norm_bwd(int dt, int n_rows, int n_cols, const float * rs, const void * W, const void * X, const void * dY,
					const void * dX_in, const float * dW_in, double * dx_pre, double * dx_floor, double * dw_pre, double * dw_abs);
int oracle_rope(int dt, int bwd, uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta, const int * seq_positions,
					const void * X_q, const void * X_k, double * q_pre, double * k_pre);
int oracle_swiglu(int dt, long n, const void * g, const void * u, double * out_pre);
int oracle_swiglu_bwd(int dt, long n, const void * g, const void * u, const void * dO, double * dg_pre, double * dg_floor, double * du_pre);
int oracle_swiglu_bwd2(int fdt, int dt, long n, const void * g, const void * u, const void * dO, double * dg_pre, double * dg_floor, double * du_pre);
int oracle_softmax(int dt_in, int dt_out, int n_rows, int n_cols, const void * X, double * y_pre);
int oracle_cross_entropy_loss(int dt, int n_rows, int n_cols, void * P, const uint32_t * labels);
int oracle_softmax_cross_entropy(int dt, int n_rows, int n_cols, const void * X, const uint32_t * labels,
					double * y_lo, double * y_hi, double * loss, double * mean_loss);

/* byte movement (elem_bytes = 1, 2 or 4; no rounding involved):
 * embedding: out[t, :] = table[ids[t], :]; vocab < 0 leaves ids unchecked,
 * else an id >= vocab returns -1.
 * copy_to_seq_context: row t of keys / values to rows p and S + p of the
 * context at ctx_ptrs[t] (host addresses). */
int oracle_embedding(int elem_bytes, int num_tokens, int embed_dim, const uint32_t * ids, const void * table, long vocab, void * out);
int oracle_copy_to_seq_context(int elem_bytes, uint64_t N, int kv_dim, const void * keys, const void * values,
					const int * seq_positions, const uint64_t * ctx_ptrs, const int * ctx_sizes);

/* exact rounding chains (no evaluation slack) */
int oracle_rms_norm_bwd_x_exact(int dt, int n_rows, int n_cols, const float * ws, const float * rs,
					const void * W, const void * X, const void * dY, const void * dX_in, double * v);
int oracle_softmax_cross_entropy_exact(int dt, int n_rows, int n_cols, const void * X, const uint32_t * labels,
					double * y, double * loss, double * mean_loss);
int oracle_rms_norm_bwd_x2_exact(int fdt, int dt, int n_rows, int n_cols, const float * ws, const float * rs,
					const void * W, const void * X, const void * dY, const void * dX_in, double * v);

#endif
