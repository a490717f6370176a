/*
 * Allocation-free exact RMSNorm backward (declared in include/dataflow_noalloc.h;
 * no counterpart in the reference). The kernels are the code object's fused
 * backward and its finish pass (device code shared through rms_norm_impl.h),
 * launched with the same geometry (rms_dw_geometry), so dX and dW are
 * bit-identical to submit_rms_norm_bwd's. Their partial rows live in this
 * file's `scratch` array instead of the code object's module scratch; the
 * kernels take its device address as an argument.
 */
#include <atomic>
#include <stdio.h>

#include "rms_norm_impl.h"
#include "dataflow_noalloc.h"

static_assert(DATAFLOW_NOALLOC_SCRATCH_BYTES == RMS_DW_SCRATCH_FLOATS * sizeof(float), "scratch size");

/* one fp32 partial row per workgroup of the main pass; each GPU the library
 * runs on holds its own copy until the process ends */
static __device__ __align__(256) float scratch[RMS_DW_SCRATCH_FLOATS];

template <typename T>
__global__ void __launch_bounds__(1024) noalloc_rms_norm_bwd_kernel(int n_rows, int n_cols, float eps, const float * fwd_rms_vals,
		const T * rms_weight, const T * X_inp, const T * upstream_dX, T * dX, float * dW, float * partials) {
	RmsArgs a = {n_rows, n_cols, eps, nullptr, fwd_rms_vals, nullptr, nullptr, rms_weight, X_inp, upstream_dX, dX, dW, partials, nullptr};
	rms_run<T, float, RMS_BWD>(a);
}

__global__ void __launch_bounds__(RMS_FINISH_THREADS) noalloc_rms_norm_bwd_finish(int n_cols, float * dW, const float * partials, int n_parts) {
	rms_dw_finish<float>(n_cols, dW, partials, n_parts);
}

namespace {

constexpr int kMaxDevices = 64;

/* what the entry point needs per device, resolved on its first call there:
 * the device address of `scratch`, the CU count and the LDS limit.
 * state: 0 unset, 1 being written by one thread, 2 ready. */
struct DeviceState {
	std::atomic<int> state;
	float * scratch;
	int cu_count;
	int max_lds;
};
DeviceState g_devices[kMaxDevices];

const char * kWhat = "dataflow_rms_norm_bwd_noalloc";

int query_device(int dev, float ** ptr, int * cu_count, int * max_lds) {
	hipError_t e = hipGetSymbolAddress(reinterpret_cast<void **>(ptr), HIP_SYMBOL(scratch));
	if (e != hipSuccess || *ptr == nullptr) {
		fprintf(stderr, "%s: resolving the scratch address on device %d failed (%s)\n", kWhat, dev, hipGetErrorString(e));
		return -1;
	}
	e = hipDeviceGetAttribute(cu_count, hipDeviceAttributeMultiprocessorCount, dev);
	if (e == hipSuccess) e = hipDeviceGetAttribute(max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
	if (e != hipSuccess || *cu_count < 1 || *max_lds < 1) {
		fprintf(stderr, "%s: reading the properties of device %d failed (%s)\n", kWhat, dev, hipGetErrorString(e));
		return -1;
	}
	return 0;
}

/* the current device's state; queried once per device and kept (a thread
 * that finds another one writing it queries for itself). A stream of another
 * device is refused: the kernels would be handed this device's scratch
 * address. */
int device_state(hipStream_t stream, float ** ptr, int * cu_count, int * max_lds) {
	int dev = 0;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess) {
		fprintf(stderr, "%s: no current device (%s)\n", kWhat, hipGetErrorString(e));
		return -1;
	}
	if (stream != nullptr) {
		hipDevice_t sdev = 0;
		e = hipStreamGetDevice(stream, &sdev);
		if (e != hipSuccess) {
			fprintf(stderr, "%s: querying the stream's device failed (%s)\n", kWhat, hipGetErrorString(e));
			return -1;
		}
		if ((int) sdev != dev) {
			fprintf(stderr, "%s: the stream belongs to device %d, the calling thread's current device is %d\n", kWhat, (int) sdev, dev);
			return -1;
		}
	}
	DeviceState * d = (dev >= 0 && dev < kMaxDevices) ? &g_devices[dev] : nullptr;
	if (d && d->state.load(std::memory_order_acquire) == 2) {
		*ptr = d->scratch;
		*cu_count = d->cu_count;
		*max_lds = d->max_lds;
		return 0;
	}
	if (query_device(dev, ptr, cu_count, max_lds)) return -1;
	int empty = 0;
	if (d && d->state.compare_exchange_strong(empty, 1, std::memory_order_acq_rel)) {
		d->scratch = *ptr;
		d->cu_count = *cu_count;
		d->max_lds = *max_lds;
		d->state.store(2, std::memory_order_release);
	}
	return 0;
}

template <typename T>
const void * main_kernel() {
	return reinterpret_cast<const void *>(&noalloc_rms_norm_bwd_kernel<T>);
}

}  // namespace

extern "C" int dataflow_rms_norm_bwd_noalloc(hipStream_t stream, DataflowDatatype fwd_dt, DataflowDatatype bwd_dt,
											 int n_rows, int n_cols, float eps,
											 const float * fwd_rms_vals, const void * rms_weight, const void * X_inp,
											 const void * upstream_dX, void * dX, float * dW) {
	const void * kernel = nullptr;
	long elem = 0;
	if (fwd_dt == bwd_dt) {
		switch (fwd_dt) {
			case DATAFLOW_FP32: kernel = main_kernel<float>(); elem = 4; break;
			case DATAFLOW_FP16: kernel = main_kernel<f16_t>(); elem = 2; break;
			case DATAFLOW_BF16: kernel = main_kernel<bf16_t>(); elem = 2; break;
			default: break;
		}
	}
	if (!kernel) {
		fprintf(stderr, "%s: unsupported dtypes %s / %s (need equal FP32, FP16 or BF16)\n", kWhat,
				dataflow_datatype_as_string(fwd_dt), dataflow_datatype_as_string(bwd_dt));
		return -1;
	}
	if (n_rows < 0 || n_cols < 0) {
		fprintf(stderr, "%s: invalid shape (%d x %d)\n", kWhat, n_rows, n_cols);
		return -1;
	}
	if (n_rows == 0 || n_cols == 0) return 0;

	float * part = nullptr;
	int cu_count = 0, max_lds = 0;
	if (device_state(stream, &part, &cu_count, &max_lds)) return -1;

	const unsigned long long ptr_or = (unsigned long long) (uintptr_t) rms_weight | (unsigned long long) (uintptr_t) X_inp |
									  (unsigned long long) (uintptr_t) upstream_dX | (unsigned long long) (uintptr_t) dX;
	const int nv = rms_vec_chunks(n_cols, (int) elem, ptr_or);
	unsigned grid = 0, block = 0, lds = 0;
	const int rc = rms_dw_geometry(n_rows, n_cols, elem, nv, 3, cu_count, max_lds, (long) RMS_DW_SCRATCH_FLOATS, &grid, &block, &lds);
	if (rc == -1) {
		fprintf(stderr, "%s: rows of %d columns need more LDS than the %d bytes available\n", kWhat, n_cols, max_lds);
		return -1;
	}
	if (rc != 0 || (unsigned long long) grid * (unsigned long long) n_cols > RMS_DW_SCRATCH_FLOATS) {
		fprintf(stderr, "%s: a partial row of %d fp32 columns exceeds the %u-byte scratch\n", kWhat, n_cols, DATAFLOW_NOALLOC_SCRATCH_BYTES);
		return -1;
	}

	void * main_args[] = {&n_rows, &n_cols, &eps, &fwd_rms_vals, &rms_weight, &X_inp, &upstream_dX, &dX, &dW, &part};
	hipError_t e = hipLaunchKernel(kernel, dim3(grid), dim3(block), main_args, lds, stream);
	if (e != hipSuccess) {
		fprintf(stderr, "%s: launching the main pass failed (%s)\n", kWhat, hipGetErrorString(e));
		return -1;
	}
	int n_parts = (int) grid;
	const float * cpart = part;
	void * fin_args[] = {&n_cols, &dW, &cpart, &n_parts};
	const unsigned fgrid = (unsigned) ((n_cols + RMS_FIN_COLS - 1) / RMS_FIN_COLS);
	e = hipLaunchKernel(reinterpret_cast<const void *>(&noalloc_rms_norm_bwd_finish), dim3(fgrid), dim3(RMS_FINISH_THREADS),
						fin_args, 0, stream);
	if (e != hipSuccess) {
		fprintf(stderr, "%s: launching the finish pass failed (%s)\n", kWhat, hipGetErrorString(e));
		return -1;
	}
	return 0;
}
