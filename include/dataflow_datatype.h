/*
 * Datatype enum and helpers.
 *
 * The enumerator ORDER is part of the op identity: enum values are hashed
 * into every op fingerprint (reference: src/datatype/include/dataflow_datatype.h:7-36).
 * Never reorder or insert; only append.
 */
#ifndef DATAFLOW_DATATYPE_H
#define DATAFLOW_DATATYPE_H

#include "dataflow_common.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
	DATAFLOW_NONE,            /*  0 */
	DATAFLOW_VOID,            /*  1 */
	DATAFLOW_FP64,            /*  2 */
	DATAFLOW_FP32,            /*  3 */
	DATAFLOW_FP16,            /*  4 */
	DATAFLOW_BF16,            /*  5 */
	DATAFLOW_FP8E4M3,         /*  6 */
	DATAFLOW_FP8E5M2,         /*  7 */
	DATAFLOW_UINT64,          /*  8 */
	DATAFLOW_UINT32,          /*  9 */
	DATAFLOW_UINT16,          /* 10 */
	DATAFLOW_UINT8,           /* 11 */
	DATAFLOW_LONG,            /* 12 */
	DATAFLOW_INT,             /* 13 */
	DATAFLOW_BOOL,            /* 14 */
	DATAFLOW_FP64_SCALAR,     /* 15 */
	DATAFLOW_FP32_SCALAR,     /* 16 */
	DATAFLOW_FP16_SCALAR,     /* 17 */
	DATAFLOW_BF16_SCALAR,     /* 18 */
	DATAFLOW_FP8E4M3_SCALAR,  /* 19 */
	DATAFLOW_FP8E5M2_SCALAR,  /* 20 */
	DATAFLOW_UINT64_SCALAR,   /* 21 */
	DATAFLOW_UINT32_SCALAR,   /* 22 */
	DATAFLOW_UINT16_SCALAR,   /* 23 */
	DATAFLOW_UINT8_SCALAR,    /* 24 */
	DATAFLOW_LONG_SCALAR,     /* 25 */
	DATAFLOW_INT_SCALAR,      /* 26 */
	DATAFLOW_BOOL_SCALAR      /* 27 */
} DataflowDatatype;

/* Bytes per array element; 0 for scalars, NONE and unknown values
 * (reference: src/datatype/src/dataflow_datatype.c:4-40). */
size_t dataflow_sizeof_element(DataflowDatatype arr_dtype);

/* Upper-case name used inside op nicknames, so it feeds fingerprints;
 * "UNKNOWN" for NONE, scalars and out-of-range values
 * (reference: src/datatype/src/dataflow_datatype.c:43-78). */
char * dataflow_datatype_as_string(DataflowDatatype dtype);

/* Element-wise conversion between FP32, FP16 and BF16 host arrays
 * (round-to-nearest-even on narrowing), optionally multithreaded.
 * Returns 0, or -1 for an unsupported pair
 * (reference: src/datatype/src/dataflow_datatype.c, dataflow_convert_datatype). */
int dataflow_convert_datatype(void * to, void * from, DataflowDatatype to_dt, DataflowDatatype from_dt, long n, int num_threads);

#ifdef __cplusplus
}
#endif

#endif
