/*
 * Op description: skeleton header, fingerprint and argument block.
 *
 * Byte layout is part of the op identity (the fingerprint is SHA-256 over
 * the 388 header bytes): char[256] + int + 32 x enum, no padding
 * (reference: src/ops/include/ops.h:6-35).
 */
#ifndef OPS_H
#define OPS_H

#include "dataflow.h"

#define MAX_OP_ARGS 32

#define MAX_OP_NICKNAME_SIZE 255

/* SHA-256 of each op skeleton header */
#define OP_IDENTIFIER_FINGERPRINT_TYPE 0
#define OP_IDENTIFIER_FINGERPRINT_NUM_BYTES 32

typedef struct op_skeleton_header {
	char op_nickname[MAX_OP_NICKNAME_SIZE + 1];
	int num_args;
	DataflowDatatype arg_dtypes[MAX_OP_ARGS];
} Op_Skeleton_Header;

typedef struct op_identifier {
	uint8_t fingerprint[OP_IDENTIFIER_FINGERPRINT_NUM_BYTES];
} Op_Identifier;

typedef struct Op_Skeleton {
	Op_Skeleton_Header header;
	/* digest of header */
	Op_Identifier identifier;
} Op_Skeleton;

/* op_args[i] points at the value of argument i (the kernelParams convention
 * of hipModuleLaunchKernel); the storage only has to live until submit_op
 * returns. */
typedef struct op {
	Op_Skeleton op_skeleton;
	void * op_args[MAX_OP_ARGS];
} Op;

#endif
