/*
 * Streaming copy used only as a measurement reference (bench.py's
 * copy_reference; no op skeleton is registered for it): dst = src over
 * nchunks 16-byte chunks, grid-stride, U chunks per thread and step with all
 * of the step's loads issued before its stores, non-temporal 16-byte buffer
 * accesses - the access pattern of the path's kernels without their
 * arithmetic. Its time for an op's byte count is what the memory system
 * offers for that many bytes moved half read, half written.
 */
#include "dtypes.h"

template <int U>
__device__ __forceinline__ void stream_copy(const char * src, char * dst, uint64_t nchunks) {
	const uint64_t nth = (uint64_t) gridDim.x * blockDim.x;
	const uint64_t tid = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
	for (uint64_t base = 0; base < nchunks; base += nth * U) {
		/* one buffer range per step: chunks past the end read zero and store nowhere */
		const uint64_t win = (nchunks - base < nth * U) ? (nchunks - base) : nth * U;
		const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + base * 16, (uint32_t) (win * 16));
		const __amdgpu_buffer_rsrc_t rd = make_rsrc(dst + base * 16, (uint32_t) (win * 16));
		R16 r[U];
#pragma unroll
		for (int k = 0; k < U; k++) r[k] = buf_load16_nt(rs, (uint32_t) ((tid + k * nth) * 16), 0);
#pragma unroll
		for (int k = 0; k < U; k++) buf_store16_nt(rd, (uint32_t) ((tid + k * nth) * 16), 0, r[k]);
	}
}

/* the launch keeps nth * U * 16 bytes (one step's window) below 4 GiB */
extern "C" __global__ void __launch_bounds__(1024) dataflow_stream_copy_u2_kernel(const char * src, char * dst, uint64_t nchunks) {
	stream_copy<2>(src, dst, nchunks);
}
extern "C" __global__ void __launch_bounds__(1024) dataflow_stream_copy_u4_kernel(const char * src, char * dst, uint64_t nchunks) {
	stream_copy<4>(src, dst, nchunks);
}
