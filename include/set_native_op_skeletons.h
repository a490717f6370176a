/*
 * Skeletons (nickname + argument dtypes + SHA-256 identity) of the native
 * ops, and their bulk registration with a handle.
 * (reference: src/set_ops/include/set_native_op_skeletons.h:11-32,
 *  src/set_ops/src/set_native_op_skeletons.c:5-611)
 *
 * Nicknames are "<op>_<DT>" or "<op>_<FWD_DT>_<BWD_DT>" using
 * dataflow_datatype_as_string(); the fingerprint covers the whole 388-byte
 * header, so the same (op, dtypes) gives the same digest as the reference.
 */
#ifndef SET_NATIVE_OPS_H
#define SET_NATIVE_OPS_H

#include "dataflow.h"
#include "fingerprint.h"
#include "ops.h"
#include "dataflow_handle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Registers every native op variant the code object provides (kernel
 * symbols "<op>_<dt>[_<dt>]_kernel", launch-config symbols
 * "<op>_set_launch_config"). Returns the number of functions added or -1.
 * Call once per handle and code object. */
int register_native_ops(Dataflow_Handle * dataflow_handle, char * native_function_code_filename, char * native_function_config_filename);

/* Dispatch on the op base name. 0 on success, -1 for an unknown op. */
int set_native_op_skeleton(Op_Skeleton * skeleton, char * op_name, DataflowDatatype fwd_dt, DataflowDatatype bwd_dt);

void set_native_embedding_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype);

void set_native_rms_norm_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype);
void set_native_rms_norm_bwd_x_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype, DataflowDatatype bwd_datatype);
void set_native_rms_norm_bwd_w_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype, DataflowDatatype bwd_datatype);

void set_native_rope_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype);
void set_native_rope_bwd_x_skeleton(Op_Skeleton * skeleton, DataflowDatatype bwd_datatype);
void set_native_copy_to_seq_context_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype);

void set_native_swiglu_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype);
void set_native_swiglu_bwd_x_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype, DataflowDatatype bwd_datatype);

void set_native_softmax_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype, DataflowDatatype bwd_datatype);
void set_native_cross_entropy_loss_skeleton(Op_Skeleton * skeleton, DataflowDatatype bwd_datatype);

/* Fused RMSNorm backward with the exact gradient:
 *   dX += r*(dY*w) - x*r^3/n * sum_j(dY*w*x),   dW (fp32) += sum_rows dY*x*r
 * Nickname "rms_norm_bwd_<FWD>_<BWD>", 9 args:
 *   (INT_SCALAR n_rows, INT_SCALAR n_cols, FP32_SCALAR eps, FP32 rms_vals,
 *    fwd W, fwd X, bwd dY, bwd dX, FP32 dW).
 * No reference counterpart: the reference splits the backward into
 * rms_norm_bwd_x (a different formula) and rms_norm_bwd_w. */
void set_native_rms_norm_bwd_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype, DataflowDatatype bwd_datatype);

/* Fused softmax + cross-entropy, in place on the logits:
 *   loss[r] = logsumexp(x_r) - x_r[label_r],  mean_loss = sum(loss) / n_rows,
 *   logits <- softmax(x) - onehot(label)  (the reference's softmax followed by
 *   its cross_entropy_loss, as one pass).
 * Nickname "softmax_cross_entropy_loss_<DT>", 6 args:
 *   (INT_SCALAR n_rows, INT_SCALAR n_cols, dt logits, UINT32 labels,
 *    FP32 loss, FP32 mean_loss).
 * No reference counterpart (the reference never computes a loss value). */
void set_native_softmax_cross_entropy_loss_skeleton(Op_Skeleton * skeleton, DataflowDatatype datatype);

/* RoPE forward fused with the KV-cache scatter: rope on Q and K in place,
 * then the rotated K row and the V row of each token t written to rows p and
 * S + p of its context (p = seq_positions[t], S = seq_context_sizes[t], the
 * context at seq_context_ptrs[t]), as copy_to_seq_context does.
 * Nickname "rope_copy_to_seq_context_<DT>", 11 args:
 *   (UINT64_SCALAR N, INT_SCALAR model_dim, INT_SCALAR head_dim,
 *    INT_SCALAR num_kv_heads, INT_SCALAR theta, INT seq_positions, dt X_q,
 *    dt X_k, dt values, UINT64 seq_context_ptrs, INT seq_context_sizes).
 * No reference counterpart (the reference notes the fusion at
 * attention/rope.cu:50-54 and keeps two kernels). */
void set_native_rope_copy_to_seq_context_skeleton(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype);

#ifdef __cplusplus
}
#endif

#endif
