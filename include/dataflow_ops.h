/*
 * Op API: each submit_* fills an Op (skeleton + pointers to its arguments)
 * and hands it to handle->submit_op. Returns 0, or -1 with a message on
 * stderr. Argument order and meaning follow the reference's
 * src/dataflow_ops/include/dataflow_ops.h:146-215. Of the reference's
 * external-library ops, matmul is provided (through hipBLASLt); attention is
 * not part of this library.
 */
#ifndef DATAFLOW_OPS_H
#define DATAFLOW_OPS_H

#include "dataflow.h"
#include "ops.h"
#include "dataflow_handle.h"
#include "set_native_op_skeletons.h"
#include "set_external_op_skeletons.h"

#ifdef __cplusplus
extern "C" {
#endif

/* --- matmul (reference: src/dataflow_ops/src/matmul_op.c:10-65, external op) --- */

/* BLAS column-major semantics: D [M x N] = alpha * op(A) * op(B) + beta * C,
 * op(A) [M x K], op(B) [K x N]; A is stored M x K (ld M), or K x M (ld K)
 * when to_trans_a; B is stored K x N (ld K), or N x K (ld N) when to_trans_b;
 * C and D are M x N (ld M). With C == NULL, c_dt == DATAFLOW_NONE or
 * beta == 0, C is not read. A row-major Y [m x n] = X [m x k] @ W, W stored
 * column-major, is A = W, B = X, D = Y, to_trans_a = 1, M = n, K = k, N = m.
 * Needs the matmul op registered (register_external_matmul). */
int submit_matmul(Dataflow_Handle * handle, int stream_id,
					DataflowDatatype a_dt, DataflowDatatype b_dt, DataflowDatatype c_dt, DataflowDatatype d_dt,
					DataflowDatatype compute_dt,
					int to_trans_a, int to_trans_b,
					int M, int K, int N,
					float alpha, float beta,
					void * A, void * B, void * C, void * D,
					uint64_t workspaceBytes, void * workspace);

/* --- preprocess (reference: src/dataflow_ops/src/preprocess_ops.c:3-32) --- */

/* output[t, :] = embedding_table[token_ids[t], :] for t < num_tokens (rows of
 * embed_dim elements of fwd_dt; every storage type incl. fp8). Token ids must
 * index rows of the table, as in the reference. */
int submit_embedding(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						int num_tokens, int embed_dim,
						uint32_t * token_ids, void * embedding_table, void * output);

/* --- norm (reference: src/dataflow_ops/src/norm_ops.c:4-97) --- */

/* out = (X * rstd) * w per row; weighted_sums[r] = sum_j X*w, rms_vals[r] = rstd
 * = 1/sqrt(mean(X^2) + eps); each of the two may be NULL. */
int submit_rms_norm(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						int n_rows, int n_cols, float eps,
						void * rms_weight, void * X, void * out, float * weighted_sums, float * rms_vals);

/* dX += dY * bf(w*r - (x*r^3/n)*ws) with the reference's intermediate
 * roundings to bwd_dt (not the exact gradient; see submit_rms_norm_bwd). */
int submit_rms_norm_bwd_x(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								int n_rows, int n_cols, float eps,
								float * fwd_weighted_sums, float * fwd_rms_vals,
								void * rms_weight, void * X_inp, void * upstream_dX, void * dX);

/* dW += sum over rows of dY * X * rstd (deterministic order). */
int submit_rms_norm_bwd_w(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								int n_rows, int n_cols, float eps,
								float * fwd_rms_vals, void * X_inp, void * upstream_dX, void * dW);

/* Fused exact-gradient backward: dX += exact dL/dX, dW (fp32) += dL/dW, one
 * pass over X and dY. No reference counterpart. */
int submit_rms_norm_bwd(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								int n_rows, int n_cols, float eps,
								float * fwd_rms_vals, void * rms_weight, void * X_inp, void * upstream_dX, void * dX, float * dW);

/* --- attention misc (reference: src/dataflow_ops/src/attn_misc_ops.c:3-65) --- */

/* In-place rotary embedding of adjacent (even, odd) pairs of X_q
 * [N / model_dim tokens x model_dim] and X_k [tokens x num_kv_heads*head_dim];
 * angle = pos * theta^(-c/head_dim) for pair column c. */
int submit_rope(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
						int * seq_positions, void * X_q, void * X_k);

/* In-place inverse (transposed) rotation of dX_q and dX_k. */
int submit_rope_bwd_x(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype bwd_dt,
						uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
						int * seq_positions, void * dX_q, void * dX_k);

/* KV-cache scatter (reference: attn_misc_ops.c:69-100): for token t <
 * N / kv_dim, with ctx = (fwd_dt *) seq_context_ptrs[t], p = seq_positions[t]
 * and S = seq_context_sizes[t], row t of X_k goes to ctx row p and row t of X_v
 * to ctx row S + p (a context holds S key rows, then S value rows). */
int submit_copy_to_seq_context(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						uint64_t N, int total_tokens, int kv_dim,
						void * X_k, void * X_v, int * seq_positions, uint64_t * seq_context_ptrs, int * seq_context_sizes);

/* No reference counterpart (the fusion the reference notes at
 * attention/rope.cu:50-54): submit_rope on X_q and X_k, then
 * submit_copy_to_seq_context of the rotated X_k rows and the X_v rows
 * (kv_dim = num_kv_heads * head_dim, tokens = N / model_dim), in one kernel
 * that writes each rotated K row from registers to both places. X_v and the
 * context arrays may be NULL only when num_kv_heads is 0. */
int submit_rope_copy_to_seq_context(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
						int * seq_positions, void * X_q, void * X_k,
						void * X_v, uint64_t * seq_context_ptrs, int * seq_context_sizes);

/* --- mlp misc (reference: src/dataflow_ops/src/mlp_misc_ops.c:3-61) --- */

/* out = silu(x_w1) * x_w3 */
int submit_swiglu(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						int num_rows, int num_cols,
						void * x_w1, void * x_w3, void * out);

/* dX_w3 = dOut * silu(x_w1); dX_w1 = dOut * x_w3 * silu'(x_w1) */
int submit_swiglu_bwd_x(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
						int num_rows, int num_cols,
						void * x_w1, void * x_w3,
						void * upstream_dX, void * dX_w1, void * dX_w3);

/* --- loss (reference: src/dataflow_ops/src/loss_misc_ops.c:4-60) --- */

/* Row softmax of X (fwd_dt) into out (bwd_dt). */
int submit_softmax(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
						int n_rows, int n_cols,
						void * X, void * out);

/* pred_logits[r, labels[r]] -= 1 in place (labels >= n_cols are skipped). */
int submit_cross_entropy_loss(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype bwd_dt,
								int n_rows, int n_cols,
								void * pred_logits, uint32_t * labels);

/* Fused softmax + cross-entropy: per-row fp32 loss, fp32 mean loss, and the
 * logits overwritten in place by softmax - onehot. No reference counterpart. */
int submit_softmax_cross_entropy_loss(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype dt,
								int n_rows, int n_cols,
								void * logits, uint32_t * labels, float * loss, float * mean_loss);

#ifdef __cplusplus
}
#endif

#endif
