/*
 * Generic handle entry points: dispatch on the compute type to a backend.
 * (declared in the reference's src/dataflow_handle/include/dataflow_handle.h:139
 * but never defined there)
 */
#include "dataflow_handle.h"
#include "hip_dataflow_handle.h"

int init_dataflow_handle(Dataflow_Handle * dataflow_handle, ComputeType compute_type, int device_id, int ctx_id, unsigned int ctx_flags, int num_streams, int * opt_stream_prios, char ** opt_stream_names) {
	if (!dataflow_handle) {
		fprintf(stderr, "Error: init_dataflow_handle called with a NULL handle...\n");
		return -1;
	}
	switch (compute_type) {
		case COMPUTE_HSA:
			return init_hip_dataflow_handle(dataflow_handle, compute_type, device_id, ctx_id, ctx_flags,
											num_streams, opt_stream_prios, opt_stream_names);
		default:
			fprintf(stderr, "Error: compute type %d has no backend in this library (COMPUTE_HSA = %d is the AMD GPU backend)...\n",
					(int) compute_type, (int) COMPUTE_HSA);
			return -1;
	}
}

int destroy_dataflow_handle(Dataflow_Handle * dataflow_handle) {
	if (!dataflow_handle) {
		return -1;
	}
	switch (dataflow_handle->compute_type) {
		case COMPUTE_HSA:
			return destroy_hip_dataflow_handle(dataflow_handle);
		default:
			fprintf(stderr, "Error: cannot destroy a handle of compute type %d...\n", (int) dataflow_handle->compute_type);
			return -1;
	}
}
