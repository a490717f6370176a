/*
 * External op skeletons (reference: src/set_ops/src/set_external_op_skeletons.c:4-70).
 */
#include "set_external_op_skeletons.h"

void set_external_matmul_skeleton(Op_Skeleton * skeleton) {
	static const DataflowDatatype args[] = {
		DATAFLOW_INT_SCALAR,                                                   /* num_procs (0 = all) */
		DATAFLOW_INT_SCALAR, DATAFLOW_INT_SCALAR, DATAFLOW_INT_SCALAR, DATAFLOW_INT_SCALAR,  /* a, b, c, d dtypes */
		DATAFLOW_INT_SCALAR,                                                   /* compute dtype */
		DATAFLOW_INT_SCALAR, DATAFLOW_INT_SCALAR,                              /* to_trans_a, to_trans_b */
		DATAFLOW_INT_SCALAR, DATAFLOW_INT_SCALAR, DATAFLOW_INT_SCALAR,         /* M, K, N */
		DATAFLOW_FP32_SCALAR, DATAFLOW_FP32_SCALAR,                            /* alpha, beta */
		DATAFLOW_VOID, DATAFLOW_VOID, DATAFLOW_VOID, DATAFLOW_VOID,            /* A, B, C, D */
		DATAFLOW_UINT64, DATAFLOW_VOID,                                        /* workspaceBytes, workspace */
	};
	Op_Skeleton_Header * h = &skeleton->header;
	memset(h, 0, sizeof(*h));
	strncpy(h->op_nickname, "matmul", MAX_OP_NICKNAME_SIZE);
	h->num_args = (int) (sizeof(args) / sizeof(args[0]));
	for (int i = 0; i < h->num_args; i++) h->arg_dtypes[i] = args[i];
	do_fingerprinting(h, sizeof(Op_Skeleton_Header), skeleton->identifier.fingerprint, OP_IDENTIFIER_FINGERPRINT_TYPE);
}

int register_external_matmul(Dataflow_Handle * dataflow_handle, char * lib_path) {
	if (!dataflow_handle || !dataflow_handle->register_external_code) {
		fprintf(stderr, "Error: cannot register matmul: handle is not initialised...\n");
		return -1;
	}
	Op_Skeleton sk;
	set_external_matmul_skeleton(&sk);
	char * syms[1] = {"hipblaslt_matmul"};
	char * inits[1] = {"hipblaslt_matmul_init"};
	const int added = dataflow_handle->register_external_code(dataflow_handle, lib_path, 1, &sk, syms, inits);
	if (added != 1) {
		fprintf(stderr, "Error: failed to register matmul op from %s...\n", lib_path);
		return -1;
	}
	return added;
}
