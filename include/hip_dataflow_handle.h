/*
 * HIP backend of Dataflow_Handle for AMD Instinct GPUs (gfx950).
 *
 * Mirrors the CUDA backend's records (reference:
 * src/dataflow_handle/nvidia/include/cuda_dataflow_handle.h:15-67):
 * native functions come from a gfx950 code object loaded with hipModuleLoad,
 * their launch geometry from a dlopen'ed config library, and submit_op
 * launches with hipModuleLaunchKernel(kernelParams = op->op_args).
 */
#ifndef HIP_DATAFLOW_HANDLE_H
#define HIP_DATAFLOW_HANDLE_H

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>
#include <limits.h>

#include "dataflow_common.h"
#include "dataflow_handle.h"

#ifdef __cplusplus
extern "C" {
#endif

#define HIP_DEFAULT_STREAM_PRIO 0

/* Workgroup size limit applied to every native function. */
#define HIP_DEV_UPPER_BOUND_MAX_THREADS_ALL_FUNC 1024

typedef struct hip_device_info {
	size_t total_mem;
	/* gfx arch number, e.g. 950 for gfx950 */
	int arch_num;
	/* compute units (the CUDA backend's sm_count) */
	int cu_count;
	int max_threads_per_block;
	/* LDS bytes per workgroup */
	int max_smem_per_block;
	/* same as max_smem_per_block: LDS needs no opt-in on CDNA */
	int optin_max_smem_per_block;
	int host_numa_id;
	int warp_size;
	/* accelerator complex dies; workgroups are dealt round-robin across them */
	int num_xcds;
	int l2_bytes;
	char arch_name[64];
} Hip_Device_Info;

typedef struct hip_function_config {
	int func_max_smem;
	int func_max_threads_per_block;
	/* set by the launch-config library's init for functions whose kernels keep
	 * per-launch partial results in the code object's module-scope scratch:
	 * the handle orders such functions across its streams (Hip_Context) */
	int shares_module_scratch;
	/* last occupancy query of the launch-config library, packed as
	 * block << 40 | LDS bytes << 16 | workgroups per CU (0: none yet); read and
	 * written as one 64-bit word, so concurrent submits see a whole entry */
	uint64_t occupancy_memo;
} Hip_Function_Config;

typedef struct hip_launch_config {
	unsigned int gridDimX;
	unsigned int gridDimY;
	unsigned int gridDimZ;
	unsigned int blockDimX;
	unsigned int blockDimY;
	unsigned int blockDimZ;
	unsigned int sharedMemBytes;
} Hip_Launch_Config;

typedef struct hip_function Hip_Function;

typedef int (*Hip_Set_Launch_Config)(Hip_Launch_Config * hip_launch_config, Dataflow_Handle * dataflow_handle, Hip_Function * hip_function, Op * op);

struct hip_function {
	Hip_Function_Config function_config;
	bool is_native;
	hipFunction_t function_handle;
	Hip_Set_Launch_Config set_launch_config;

	/* Optional second kernel launched right after function_handle on the same
	 * stream with the same kernelParams ("<symbol>_finish" in the code object,
	 * geometry from "<launch symbol minus _set_launch_config>_set_finish_launch_config").
	 * Used by ops whose cross-workgroup reduction is finished deterministically
	 * in a second pass. NULL when absent. */
	hipFunction_t finish_function_handle;
	Hip_Set_Launch_Config set_finish_launch_config;

	/* external functions */
	int (*hip_external_func)(Dataflow_Handle * dataflow_handle, int stream_id, Op * op, void * op_extra);
	void * op_extra;

	Op_Skeleton op_skeleton;
};

typedef int (*Hip_Set_Func_Attribute)(Dataflow_Handle * dataflow_handle, Hip_Function * hip_function);

/* What Dataflow_Handle.ctx points to (HIP has no per-handle contexts; the
 * CUDA backend keeps its CUcontext there). The device id comes first, so ctx
 * still reads as the device id. Functions flagged shares_module_scratch keep
 * per-launch state in their code object's module-scope memory (the RMSNorm
 * dW ops their partial rows; the 16-bit and fp32 softmax and fused
 * cross-entropy their row counter and finished-workgroup count), so the
 * handle orders them across its streams: such an op submitted on another
 * stream than the previous one first waits for everything then queued on
 * that stream (an event recorded only when the stream changes, so
 * single-stream use pays nothing). Other ops are not ordered. */
#define HIP_NO_STREAM INT_MIN
typedef struct hip_context {
	int device_id;
	int two_pass_stream;       /* stream id of the last scratch-sharing op, HIP_NO_STREAM before the first */
	hipEvent_t two_pass_event;
} Hip_Context;

/* ctx_flags is accepted for interface parity and ignored (HIP has no
 * per-handle contexts). Streams are non-blocking and all run at the default
 * priority; requested priorities are recorded in stream_prios only.
 * 0 on success, -1 on error. */
int init_hip_dataflow_handle(Dataflow_Handle * dataflow_handle, ComputeType compute_type, int device_id,
								int ctx_id, unsigned int ctx_flags,
								int num_streams, int * opt_stream_prios, char ** opt_stream_names);

/* Backend half of destroy_dataflow_handle. */
int destroy_hip_dataflow_handle(Dataflow_Handle * dataflow_handle);

#ifdef __cplusplus
}
#endif

#endif
