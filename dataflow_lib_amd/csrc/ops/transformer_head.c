/*
 * The transformer head's forward and backward on the native op path and the
 * hipBLASLt matmul (reference: src/dataflow_models/dataflow_transformer/src/
 * dataflow_transformer.c:300-499; what differs from it is listed in
 * transformer_head.h).
 */
#include "transformer_head.h"
#include "dataflow_ops.h"

#define HEAD_CHECK(call, what)                                                    \
	do {                                                                          \
		if (call) {                                                               \
			fprintf(stderr, "Error: transformer head: failed to submit %s...\n", what); \
			return -1;                                                            \
		}                                                                         \
	} while (0)

int submit_transformer_head(Dataflow_Handle * dataflow_handle, int compute_stream_id, int out_copy_stream_id,
							Transformer_Block_Transition * block_input, Transformer_Head * transformer_head,
							Transformer_Head_Activations * head_activations,
							Transformer_Model_Output * model_output,
							Transformer_Head * grad_transformer_head,
							Transformer_Head_Activations * grad_head_activations,
							Transformer_Block_Transition * grad_stream,
							Transformer_Block_Transition * next_grad_stream) {
	if (!dataflow_handle || !block_input || !transformer_head || !head_activations || !model_output) {
		fprintf(stderr, "Error: transformer head: missing handle, input, head, activations or output...\n");
		return -1;
	}
	Transformer_Head * th = transformer_head;
	Transformer_Head_Activations * ha = head_activations;
	const int T = ha->num_tokens;
	const int V = th->embedding_config.vocab_size;
	const int E = th->embedding_config.embedding_size;
	if (T < 0 || V <= 0 || E <= 0) {
		fprintf(stderr, "Error: transformer head: invalid shape (tokens %d, vocab %d, embedding %d)...\n", T, V, E);
		return -1;
	}

	HEAD_CHECK(submit_rms_norm(dataflow_handle, compute_stream_id, th->fwd_dt, T, E, th->eps, th->w_head_norm, block_input->X,
								ha->head_norm_out, (float *) ha->head_norm_weighted_sums, (float *) ha->head_norm_rms_vals),
				"head rms norm");
	/* logits [T x V] row-major = (w_head^T as V x E) x (head_norm_out^T as E x T), column-major */
	HEAD_CHECK(submit_matmul(dataflow_handle, compute_stream_id, th->fwd_dt, th->fwd_dt, DATAFLOW_NONE, th->fwd_dt, th->compute_dt,
								1, 0, V, E, T, 1.0f, 0.0f, th->w_head, ha->head_norm_out, NULL, ha->head_out,
								ha->kernel_workspaceBytes, ha->kernel_workspace),
				"output projection");

	if (!grad_transformer_head) {
		HEAD_CHECK(submit_softmax(dataflow_handle, compute_stream_id, th->fwd_dt, th->bwd_dt, T, V, ha->head_out, model_output->logits),
					"softmax");
		return 0;
	}

	Transformer_Head * gh = grad_transformer_head;
	Transformer_Head_Activations * gha = grad_head_activations;
	if (!gha || !grad_stream || !model_output->labels || !model_output->loss) {
		fprintf(stderr, "Error: transformer head backward: missing gradient activations, gradient stream, labels or loss...\n");
		return -1;
	}
	if (th->fwd_dt != th->bwd_dt) {
		fprintf(stderr, "Error: transformer head backward: fwd and bwd dtypes must match (the fused loss op is single-typed)...\n");
		return -1;
	}
	float * loss = (float *) model_output->loss;
	HEAD_CHECK(submit_softmax_cross_entropy_loss(dataflow_handle, compute_stream_id, th->fwd_dt, T, V, ha->head_out,
													model_output->labels, loss, loss + T),
				"softmax cross entropy");
	/* grad head_norm_out [T x E] row-major = w_head (E x V) x dLogits^T (V x T), column-major */
	HEAD_CHECK(submit_matmul(dataflow_handle, compute_stream_id, th->bwd_dt, th->bwd_dt, DATAFLOW_NONE, th->bwd_dt, th->compute_dt,
								0, 0, E, V, T, 1.0f, 0.0f, th->w_head, ha->head_out, NULL, gha->head_norm_out,
								gha->kernel_workspaceBytes, gha->kernel_workspace),
				"head backward data matmul");
	/* grad w_head (E x V, column-major) += head_norm_out^T (E x T) x dLogits (T x V) */
	HEAD_CHECK(submit_matmul(dataflow_handle, compute_stream_id, gh->bwd_dt, gh->bwd_dt, gh->bwd_dt, gh->bwd_dt, gh->compute_dt,
								0, 1, E, T, V, 1.0f, 1.0f, ha->head_norm_out, ha->head_out, gh->w_head, gh->w_head,
								gha->kernel_workspaceBytes, gha->kernel_workspace),
				"head weight gradient matmul");
	HEAD_CHECK(submit_rms_norm_bwd(dataflow_handle, compute_stream_id, th->fwd_dt, th->bwd_dt, T, E, th->eps,
									(float *) ha->head_norm_rms_vals, th->w_head_norm, block_input->X, gha->head_norm_out,
									grad_stream->X, (float *) gh->w_head_norm),
				"head rms norm backward");

	if (next_grad_stream) {
		void * done = dataflow_handle->get_stream_state(dataflow_handle, compute_stream_id);
		if (!done || dataflow_handle->submit_dependency(dataflow_handle, out_copy_stream_id, done)) {
			fprintf(stderr, "Error: transformer head: could not order the gradient copy after the compute stream...\n");
			return -1;
		}
		const uint64_t bytes = (uint64_t) T * (uint64_t) E * dataflow_sizeof_element(th->bwd_dt);
		HEAD_CHECK(dataflow_handle->submit_peer_transfer(dataflow_handle, out_copy_stream_id, next_grad_stream->X, grad_stream->X, bytes),
					"gradient copy");
	}
	return 0;
}
