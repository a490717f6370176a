/*
 * Op API: build an Op on the stack (skeleton + pointers to each argument, in
 * skeleton order) and submit it. Argument order and meaning follow the
 * reference's src/dataflow_ops/src/{matmul_op.c:10-65, preprocess_ops.c:3-32, norm_ops.c:4-97,
 * attn_misc_ops.c:3-100, mlp_misc_ops.c:3-61, loss_misc_ops.c:4-60}.
 */
#include "dataflow_ops.h"

static int submit_built_op(Dataflow_Handle * handle, Op * op, int stream_id, const char * what) {
	if (!handle || !handle->submit_op) {
		fprintf(stderr, "Error: cannot submit %s op: handle is not initialised...\n", what);
		return -1;
	}
	if (handle->submit_op(handle, op, stream_id)) {
		fprintf(stderr, "Error: failed to submit %s op...\n", what);
		return -1;
	}
	return 0;
}

int submit_matmul(Dataflow_Handle * handle, int stream_id,
					DataflowDatatype a_dt, DataflowDatatype b_dt, DataflowDatatype c_dt, DataflowDatatype d_dt,
					DataflowDatatype compute_dt,
					int to_trans_a, int to_trans_b,
					int M, int K, int N,
					float alpha, float beta,
					void * A, void * B, void * C, void * D,
					uint64_t workspaceBytes, void * workspace) {
	Op op;
	set_external_matmul_skeleton(&op.op_skeleton);
	/* 0 = use every CU */
	int num_procs = 0;
	void ** a = op.op_args;
	a[0] = &num_procs;
	a[1] = &a_dt; a[2] = &b_dt; a[3] = &c_dt; a[4] = &d_dt; a[5] = &compute_dt;
	a[6] = &to_trans_a; a[7] = &to_trans_b;
	a[8] = &M; a[9] = &K; a[10] = &N;
	a[11] = &alpha; a[12] = &beta;
	a[13] = &A; a[14] = &B; a[15] = &C; a[16] = &D;
	a[17] = &workspaceBytes; a[18] = &workspace;
	return submit_built_op(handle, &op, stream_id, "matmul");
}

int submit_embedding(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						int num_tokens, int embed_dim,
						uint32_t * token_ids, void * embedding_table, void * output) {
	Op op;
	set_native_embedding_skeleton(&op.op_skeleton, fwd_dt);
	void ** a = op.op_args;
	a[0] = &num_tokens; a[1] = &embed_dim;
	a[2] = &token_ids; a[3] = &embedding_table; a[4] = &output;
	return submit_built_op(handle, &op, stream_id, "embedding");
}

int submit_rms_norm(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						int n_rows, int n_cols, float eps,
						void * rms_weight, void * X, void * out, float * weighted_sums, float * rms_vals) {
	Op op;
	set_native_rms_norm_skeleton(&op.op_skeleton, fwd_dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &eps;
	a[3] = &rms_weight; a[4] = &X; a[5] = &out;
	a[6] = &weighted_sums; a[7] = &rms_vals;
	return submit_built_op(handle, &op, stream_id, "rms norm");
}

int submit_rms_norm_bwd_x(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								int n_rows, int n_cols, float eps,
								float * fwd_weighted_sums, float * fwd_rms_vals,
								void * rms_weight, void * X_inp, void * upstream_dX, void * dX) {
	Op op;
	set_native_rms_norm_bwd_x_skeleton(&op.op_skeleton, fwd_dt, bwd_dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &eps;
	a[3] = &fwd_weighted_sums; a[4] = &fwd_rms_vals;
	a[5] = &rms_weight; a[6] = &X_inp; a[7] = &upstream_dX; a[8] = &dX;
	return submit_built_op(handle, &op, stream_id, "rms norm bwd x");
}

int submit_rms_norm_bwd_w(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								int n_rows, int n_cols, float eps,
								float * fwd_rms_vals, void * X_inp, void * upstream_dX, void * dW) {
	Op op;
	set_native_rms_norm_bwd_w_skeleton(&op.op_skeleton, fwd_dt, bwd_dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &eps;
	a[3] = &fwd_rms_vals; a[4] = &X_inp; a[5] = &upstream_dX; a[6] = &dW;
	/* the reference's version falls off the end without a return value
	 * (norm_ops.c:97); this one returns the submit status */
	return submit_built_op(handle, &op, stream_id, "rms norm bwd w");
}

int submit_rms_norm_bwd(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
								int n_rows, int n_cols, float eps,
								float * fwd_rms_vals, void * rms_weight, void * X_inp, void * upstream_dX, void * dX, float * dW) {
	Op op;
	set_native_rms_norm_bwd_skeleton(&op.op_skeleton, fwd_dt, bwd_dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &eps;
	a[3] = &fwd_rms_vals; a[4] = &rms_weight; a[5] = &X_inp;
	a[6] = &upstream_dX; a[7] = &dX; a[8] = &dW;
	return submit_built_op(handle, &op, stream_id, "rms norm bwd (fused)");
}

int submit_rope(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
						int * seq_positions, void * X_q, void * X_k) {
	Op op;
	set_native_rope_skeleton(&op.op_skeleton, fwd_dt);
	void ** a = op.op_args;
	a[0] = &N; a[1] = &model_dim; a[2] = &head_dim; a[3] = &num_kv_heads; a[4] = &theta;
	a[5] = &seq_positions; a[6] = &X_q; a[7] = &X_k;
	return submit_built_op(handle, &op, stream_id, "rope");
}

int submit_rope_copy_to_seq_context(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
						int * seq_positions, void * X_q, void * X_k,
						void * X_v, uint64_t * seq_context_ptrs, int * seq_context_sizes) {
	Op op;
	set_native_rope_copy_to_seq_context_skeleton(&op.op_skeleton, fwd_dt);
	void ** a = op.op_args;
	a[0] = &N; a[1] = &model_dim; a[2] = &head_dim; a[3] = &num_kv_heads; a[4] = &theta;
	a[5] = &seq_positions; a[6] = &X_q; a[7] = &X_k;
	a[8] = &X_v; a[9] = &seq_context_ptrs; a[10] = &seq_context_sizes;
	return submit_built_op(handle, &op, stream_id, "rope copy to seq context");
}

int submit_rope_bwd_x(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype bwd_dt,
						uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
						int * seq_positions, void * dX_q, void * dX_k) {
	Op op;
	set_native_rope_bwd_x_skeleton(&op.op_skeleton, bwd_dt);
	void ** a = op.op_args;
	a[0] = &N; a[1] = &model_dim; a[2] = &head_dim; a[3] = &num_kv_heads; a[4] = &theta;
	a[5] = &seq_positions; a[6] = &dX_q; a[7] = &dX_k;
	return submit_built_op(handle, &op, stream_id, "rope bwd x");
}

int submit_copy_to_seq_context(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						uint64_t N, int total_tokens, int kv_dim,
						void * X_k, void * X_v, int * seq_positions, uint64_t * seq_context_ptrs, int * seq_context_sizes) {
	Op op;
	set_native_copy_to_seq_context_skeleton(&op.op_skeleton, fwd_dt);
	void ** a = op.op_args;
	a[0] = &N; a[1] = &total_tokens; a[2] = &kv_dim;
	a[3] = &X_k; a[4] = &X_v; a[5] = &seq_positions; a[6] = &seq_context_ptrs; a[7] = &seq_context_sizes;
	return submit_built_op(handle, &op, stream_id, "copy to seq context");
}

int submit_swiglu(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt,
						int num_rows, int num_cols,
						void * x_w1, void * x_w3, void * out) {
	Op op;
	set_native_swiglu_skeleton(&op.op_skeleton, fwd_dt);
	void ** a = op.op_args;
	a[0] = &num_rows; a[1] = &num_cols; a[2] = &x_w1; a[3] = &x_w3; a[4] = &out;
	return submit_built_op(handle, &op, stream_id, "swiglu");
}

int submit_swiglu_bwd_x(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
						int num_rows, int num_cols,
						void * x_w1, void * x_w3,
						void * upstream_dX, void * dX_w1, void * dX_w3) {
	Op op;
	set_native_swiglu_bwd_x_skeleton(&op.op_skeleton, fwd_dt, bwd_dt);
	void ** a = op.op_args;
	a[0] = &num_rows; a[1] = &num_cols; a[2] = &x_w1; a[3] = &x_w3;
	a[4] = &upstream_dX; a[5] = &dX_w1; a[6] = &dX_w3;
	return submit_built_op(handle, &op, stream_id, "swiglu bwd x");
}

int submit_softmax(Dataflow_Handle * handle, int stream_id,
						DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
						int n_rows, int n_cols,
						void * X, void * out) {
	Op op;
	set_native_softmax_skeleton(&op.op_skeleton, fwd_dt, bwd_dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &X; a[3] = &out;
	return submit_built_op(handle, &op, stream_id, "softmax");
}

int submit_cross_entropy_loss(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype bwd_dt,
								int n_rows, int n_cols,
								void * pred_logits, uint32_t * labels) {
	Op op;
	set_native_cross_entropy_loss_skeleton(&op.op_skeleton, bwd_dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &pred_logits; a[3] = &labels;
	return submit_built_op(handle, &op, stream_id, "cross entropy loss");
}

int submit_softmax_cross_entropy_loss(Dataflow_Handle * handle, int stream_id,
								DataflowDatatype dt,
								int n_rows, int n_cols,
								void * logits, uint32_t * labels, float * loss, float * mean_loss) {
	Op op;
	set_native_softmax_cross_entropy_loss_skeleton(&op.op_skeleton, dt);
	void ** a = op.op_args;
	a[0] = &n_rows; a[1] = &n_cols; a[2] = &logits; a[3] = &labels; a[4] = &loss; a[5] = &mean_loss;
	return submit_built_op(handle, &op, stream_id, "softmax cross entropy loss");
}
