/*
 * The loss-path driver: the transformer head's forward and backward over the
 * native op path (reference: src/dataflow_models/dataflow_transformer/src/
 * dataflow_transformer.c:300-499, structs from transformer_structs.h:93-150 and
 * dataflow_models.h:33-39, laid out identically; Seq_Batch_Config is only
 * carried by pointer here).
 *
 * Forward (T = num_tokens, E = embedding_size, V = vocab_size):
 *   head_norm_out [T x E] = rms_norm(block_input->X) with w_head_norm
 *   head_out [T x V] = head_norm_out @ w_head  (w_head column-major E x V, i.e.
 *                      V rows of E contiguous; hipBLASLt, fp32 accumulate)
 * Inference (grad_transformer_head == NULL): model_output->logits = softmax(head_out).
 * Training: the fused softmax + cross-entropy turns head_out into dLogits in
 * place and writes model_output->loss[0..T) (fp32 per token) and the mean
 * loss to loss[T] (so `loss` holds T + 1 floats); model_output->logits is not
 * written and loss_avg is left to the caller (it is on the host). Then
 *   grad head_norm_out [T x E] = dLogits @ w_head^T
 *   grad w_head (column-major E x V) += head_norm_out^T @ dLogits
 *   grad_stream->X += exact dL/dX of the norm, grad w_head_norm (fp32 [E]) += dL/dw
 *   (the fused exact-gradient RMSNorm backward)
 * and, when next_grad_stream is given, grad_stream->X is copied there on
 * out_copy_stream_id after the compute stream's work (an event orders them).
 *
 * Differences from the reference's head, whose transformer layer does not
 * build: the forward GEMM uses the column-major convention its matmul
 * documents (M = V, K = E, N = T; the reference passes M = E, K = T, N = V);
 * the loss path is the fused op; the norm backward is the exact gradient with
 * the block input as X (the reference's bwd_w is handed head_out); fwd_dt and
 * bwd_dt must match (the fused loss op is single-typed); the gradient copy
 * waits for the compute stream.
 * Requires register_native_ops and register_external_matmul on the handle.
 */
#ifndef TRANSFORMER_HEAD_H
#define TRANSFORMER_HEAD_H

#include "dataflow.h"
#include "dataflow_handle.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct seq_batch_config Seq_Batch_Config;

typedef struct embedding_config {
	int vocab_size;
	int embedding_size;
} Embedding_Config;

typedef struct transformer_head {
	DataflowDatatype fwd_dt;
	DataflowDatatype bwd_dt;
	DataflowDatatype compute_dt;
	float eps;
	Embedding_Config embedding_config;
	void * buffer;
	void * w_head_norm;
	void * w_head;
} Transformer_Head;

typedef struct transformer_head_activations {
	int num_tokens;
	void * buffer;
	void * head_norm_out;
	void * head_norm_weighted_sums;
	void * head_norm_rms_vals;
	void * head_out;
	void * kernel_workspace;
	uint64_t kernel_workspaceBytes;
} Transformer_Head_Activations;

typedef struct transformer_block_transition {
	Seq_Batch_Config * batch_config;
	void * X;
} Transformer_Block_Transition;

typedef struct transformer_model_output {
	Seq_Batch_Config * batch_config;
	uint32_t * token_ids;
	uint32_t * labels;
	void * logits;
	void * loss;
	float loss_avg;
} Transformer_Model_Output;

/* dataflow_transformer.c:300-310 */
int submit_transformer_head(Dataflow_Handle * dataflow_handle, int compute_stream_id, int out_copy_stream_id,
							Transformer_Block_Transition * block_input, Transformer_Head * transformer_head,
							Transformer_Head_Activations * head_activations,
							Transformer_Model_Output * model_output,
							Transformer_Head * grad_transformer_head,
							Transformer_Head_Activations * grad_head_activations,
							Transformer_Block_Transition * grad_stream,
							Transformer_Block_Transition * next_grad_stream);

#ifdef __cplusplus
}
#endif

#endif
