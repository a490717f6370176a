/*
 * Skeletons of the external (library-backed) ops (reference:
 * src/set_ops/include/set_external_op_skeletons.h,
 * src/set_ops/src/set_external_op_skeletons.c:4-70). The matmul skeleton is
 * byte-identical to the reference's, so its fingerprint is the same.
 */
#ifndef SET_EXTERNAL_OP_SKELETONS_H
#define SET_EXTERNAL_OP_SKELETONS_H

#include "dataflow.h"
#include "ops.h"
#include "fingerprint.h"
#include "dataflow_handle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* set_external_op_skeletons.c:4-70: nickname "matmul", 19 args
 * (num_procs, a/b/c/d dtype, compute dtype, trans_a, trans_b, M, K, N,
 *  alpha, beta, A, B, C, D, workspaceBytes, workspace) */
void set_external_matmul_skeleton(Op_Skeleton * skeleton);

/* Registers the matmul op from the hipBLASLt-backed external library at
 * lib_path (symbols "hipblaslt_matmul" / "hipblaslt_matmul_init"). Returns
 * the number of functions added (1) or -1. No counterpart in the reference,
 * whose tests make the same register_external_code call inline
 * (test_cuda_dataflow_handle_matmul.c:44-59). */
int register_external_matmul(Dataflow_Handle * dataflow_handle, char * lib_path);

#ifdef __cplusplus
}
#endif

#endif
