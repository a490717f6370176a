/*
 * Streaming copies used only as a measurement reference (bench.py's
 * copy_reference). Built into a code object of their own
 * (lib/bench_stream_copy_gfx950.hsaco) that bench.py loads itself; the
 * product code object does not contain them. dst = src over
 * nchunks 16-byte chunks with non-temporal 16-byte buffer accesses, all of a
 * step's loads issued before its stores - the access patterns of the path's
 * kernels without their arithmetic. Two orders:
 *   - grid-stride (u2/u4): one step covers gridDim.x * blockDim.x * U
 *     consecutive chunks, thread t taking t, t + nth, ...;
 *   - blocked (blk8/blk16): workgroup w copies contiguous blocks of
 *     blockDim.x * U chunks, blocks dealt round-robin (w, w + gridDim.x, ...);
 *     the faster of the two for a single read and write stream above a few
 *     hundred MB on MI355X (measured: 1 GB, 349 us against 380 us).
 * Their best time for an op's byte count is what the memory system offers
 * for that many bytes moved half read, half written.
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

template <int U>
__device__ __forceinline__ void stream_copy_blocked(const char * src, char * dst, uint64_t nchunks) {
	const uint64_t blk = (uint64_t) blockDim.x * U;
	for (uint64_t base = (uint64_t) blockIdx.x * blk; base < nchunks; base += (uint64_t) gridDim.x * blk) {
		const uint64_t win = (nchunks - base < blk) ? (nchunks - base) : blk;
		const __amdgpu_buffer_rsrc_t rs = make_rsrc(src + base * 16, (uint32_t) (win * 16));
		const __amdgpu_buffer_rsrc_t rd = make_rsrc(dst + base * 16, (uint32_t) (win * 16));
		R16 r[U];
#pragma unroll
		for (int k = 0; k < U; k++) r[k] = buf_load16_nt(rs, (uint32_t) ((k * blockDim.x + threadIdx.x) * 16), 0);
#pragma unroll
		for (int k = 0; k < U; k++) buf_store16_nt(rd, (uint32_t) ((k * blockDim.x + threadIdx.x) * 16), 0, r[k]);
	}
}

extern "C" __global__ void __launch_bounds__(1024) dataflow_stream_copy_blk8_kernel(const char * src, char * dst, uint64_t nchunks) {
	stream_copy_blocked<8>(src, dst, nchunks);
}
extern "C" __global__ void __launch_bounds__(1024) dataflow_stream_copy_blk16_kernel(const char * src, char * dst, uint64_t nchunks) {
	stream_copy_blocked<16>(src, dst, nchunks);
}
