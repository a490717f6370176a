/*
 * The device abstraction: a vtable of backend functions plus the op table
 * that maps an op fingerprint to a backend function record.
 *
 * Field order, types and the fixed-size arrays follow the reference's
 * src/dataflow_handle/include/dataflow_handle.h:28-122 so that callers that
 * stack-allocate the struct keep the same layout.
 */
#ifndef DATAFLOW_HANDLE_H
#define DATAFLOW_HANDLE_H

#include "dataflow_common.h"
#include "table.h"
#include "ops.h"

#ifdef __cplusplus
extern "C" {
#endif

#define OP_TABLE_MIN_SIZE (1UL << 10)
#define OP_TABLE_MAX_SIZE (1UL << 20)

#define MAX_NATIVE_FUNCTION_LIBS 1024

#define MAX_STREAMS 256

#define FUNC_SYMBOL_MAX_LEN 512

typedef enum compute_type {
	COMPUTE_NONE,
	COMPUTE_CPU,
	COMPUTE_CUDA,
	/* AMD GPUs (HIP over the HSA runtime) use this slot */
	COMPUTE_HSA,
	COMPUTE_LEVEL_ZERO
} ComputeType;

typedef struct dataflow_handle Dataflow_Handle;

struct dataflow_handle {

	ComputeType compute_type;
	/* -1 for CPU */
	int device_id;
	void * device_handle;
	/* backend-specific device info (Hip_Device_Info for COMPUTE_HSA) */
	void * device_info;
	/* caller-chosen id when several handles share one device */
	int ctx_id;
	void * ctx;
	int num_streams;
	/* backend-specific stream array (hipStream_t[num_streams]) */
	void * streams;
	int stream_prios[MAX_STREAMS];
	char * stream_names[MAX_STREAMS];
	/* backend-specific per-stream events (hipEvent_t[num_streams]) */
	void * stream_states;

	int num_native_function_libs;
	void * native_function_libs[MAX_NATIVE_FUNCTION_LIBS];

	/* fingerprint (32 B) -> backend function record, stored by value */
	int num_ops;
	Table op_table;

	/* 0.) ops */

	/* Returns the number of functions added, or -1 if the code object or the
	 * launch-config library cannot be loaded or nothing was added. */
	int (*register_native_code)(Dataflow_Handle * dataflow_handle, char * native_code_filename, char * native_code_config_lib_filename,
								int num_funcs, Op_Skeleton * func_op_skeletons, char ** func_symbols, char ** func_set_launch_symbols, char ** func_init_symbols);
	int (*register_external_code)(Dataflow_Handle * dataflow_handle, char * external_code_filename, int num_funcs,
								Op_Skeleton * func_op_skeletons, char ** func_symbols, char ** func_init_symbols);

	/* 1.) compute: stream_id -1 selects the NULL stream. 0 or -1. */
	int (*submit_op)(Dataflow_Handle * dataflow_handle, Op * op, int stream_id);
	int (*submit_host_op)(Dataflow_Handle * dataflow_handle, void * host_func, void * host_func_arg, int stream_id);

	/* 2.) dependencies */

	/* Records the stream's event; the returned pointer stays valid until the
	 * next call for the same stream. */
	void * (*get_stream_state)(Dataflow_Handle * dataflow_handle, int stream_id);
	int (*submit_dependency)(Dataflow_Handle * dataflow_handle, int stream_id, void * other_stream_state);
	int (*sync_stream)(Dataflow_Handle * dataflow_handle, int stream_id);
	int (*sync_handle)(Dataflow_Handle * dataflow_handle);

	/* 3.) memory; set_mem with stream_id -1 is blocking */
	void * (*alloc_mem)(Dataflow_Handle * dataflow_handle, uint64_t size_bytes);
	void (*free_mem)(Dataflow_Handle * dataflow_handle, void * dev_ptr);
	int (*set_mem)(Dataflow_Handle * dataflow_handle, int stream_id, void * dev_ptr, uint8_t val, uint64_t size_bytes);
	int (*enable_access_to_host_mem)(Dataflow_Handle * dataflow_handle, void * host_ptr, uint64_t size_bytes, unsigned int flags);
	int (*disable_access_to_host_mem)(Dataflow_Handle * dataflow_handle, void * host_ptr);
	int (*enable_access_to_peer_mem)(Dataflow_Handle * dataflow_handle, Dataflow_Handle * peer_dataflow_handle);
	int (*disable_access_to_peer_mem)(Dataflow_Handle * dataflow_handle, Dataflow_Handle * peer_dataflow_handle);

	/* 4.) transfers; stream_id -1 is blocking */
	int (*submit_inbound_transfer)(Dataflow_Handle * dataflow_handle, int stream_id, void * dev_dest, void * host_src, uint64_t size_bytes);
	int (*submit_outbound_transfer)(Dataflow_Handle * dataflow_handle, int stream_id, void * host_dest, void * dev_src, uint64_t size_bytes);
	int (*submit_peer_transfer)(Dataflow_Handle * dataflow_handle, int stream_id, void * dev_dest, void * dev_src, uint64_t size_bytes);
};

/* Optional per-function init of an external function; op_table_value is the
 * backend's function record (e.g. Hip_Function). */
typedef int (*External_Lib_Func_Init)(Dataflow_Handle * dataflow_handle, void * op_table_value);

/* Signature of every external function. */
typedef int (*External_Lib_Func)(Dataflow_Handle * dataflow_handle, int stream_id, Op * op, void * op_extra);

/* Dispatches on compute_type (declared, never defined, in the reference's
 * dataflow_handle.h:139). COMPUTE_HSA initialises the HIP backend; other
 * types are rejected with -1. */
int init_dataflow_handle(Dataflow_Handle * dataflow_handle, ComputeType compute_type, int device_id, int ctx_id, unsigned int ctx_flags, int num_streams, int * opt_stream_prios, char ** opt_stream_names);

/* Releases what init_*_dataflow_handle allocated (streams, events, modules,
 * op table). No reference counterpart: the reference never frees a handle. */
int destroy_dataflow_handle(Dataflow_Handle * dataflow_handle);

#ifdef __cplusplus
}
#endif

#endif
