/*
 * Row gather (token embedding) and KV-cache scatter (copy_to_seq_context):
 * pure data movement, so one byte-generic body serves every storage type,
 * the fp8 ones included.
 *
 * embedding (intended semantics of the reference's
 * src/ops/nvidia/preprocess/embedding.cu:3-119, whose typed-pointer index
 * scales the row offset by the element size a second time):
 *   out[t, :] = table[token_ids[t], :]          t < num_tokens
 * copy_to_seq_context (src/ops/nvidia/attention/copy_to_seq_context.cu:3-100):
 *   ctx_t = (T *) seq_context_ptrs[t], p = seq_positions[t], S = seq_context_sizes[t]
 *   ctx_t[p * kv_dim + d]           = keys[t * kv_dim + d]
 *   ctx_t[(S + p) * kv_dim + d]     = values[t * kv_dim + d]     t < N / kv_dim
 * (a token's context holds S key rows followed by S value rows).
 *
 * gfx950 design: one wave64 per row and token, looping over rows; the row is
 * moved in 16-byte chunks, up to GS_CH per lane in flight (all loads issued
 * before the first store). Source and destination rows are addressed through
 * per-row buffer ranges, so chunks past the row end read zero and their
 * stores are dropped. Rows whose byte length or addresses are not multiples
 * of 16 take a byte/element loop of the same shape.
 */
#include "dtypes.h"
#include "kernel_geometry.h"

/* 16-byte chunks per lane in flight per row pass (4 KB per wave) for rows
 * longer than 2 KB; a row of up to 2 KB is one pass of just the chunks it
 * has (one or two per lane), so no load or store falls past its end.
 * Measured on MI355X: the 2 KB K/V rows of copy_to_seq_context move in 13.00
 * us per 8192 tokens with two chunks per lane against 13.16 us with four
 * (and 14.4 us with eight); 8 KB embedding rows take the same 26 us with
 * four or eight. A token's K and V rows are copied one after the other:
 * issuing both rows' loads before either row's stores took 13.61 us (two
 * chunks) and 14.2 us (four), and one wave per row instead of per token
 * 13.42 us. */
#define GS_CH 4
/* Cache policy of the source rows: the embedding loads its table rows with
 * the default policy (8192 rows of a 128256 x 4096 bf16 table: 25.9 -> 23.2
 * us per launch against the streaming hint), copy_to_seq_context its K and V
 * rows with the streaming hint (13.8 against 13.4 us the other way in
 * bench.py's loop). Both store with the streaming hint: stores without it or
 * at device scope were slower with either load policy. */
#define GS_EMB_LOAD_AUX 0
#define GS_KV_LOAD_AUX BUF_AUX_NT

template <int ELEM>
struct Elem;
template <> struct Elem<1> { typedef uint8_t t; };
template <> struct Elem<2> { typedef uint16_t t; };
template <> struct Elem<4> { typedef uint32_t t; };

/* passes of CH 16-byte chunks per lane over a 16-byte aligned row */
template <int CH, int LAUX>
__device__ __forceinline__ void gs_copy_passes(const char * src, char * dst, uint32_t row_bytes, int lane) {
	const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, row_bytes);
	const __amdgpu_buffer_rsrc_t rd = make_rsrc(dst, row_bytes);
	for (uint32_t base = 0; base < row_bytes; base += 64u * 16u * CH) {
		R16 v[CH];
#pragma unroll
		for (int i = 0; i < CH; i++) v[i] = buf_load16_aux<LAUX>(rs, (uint32_t) (lane + 64 * i) * 16u, base);
#pragma unroll
		for (int i = 0; i < CH; i++) buf_store16_nt(rd, (uint32_t) (lane + 64 * i) * 16u, base, v[i]);
	}
}

/* copy one row of `row_bytes` bytes (a wave; src and dst uniform) */
template <int ELEM, int LAUX>
__device__ __forceinline__ void gs_copy_row(const char * src, char * dst, uint32_t row_bytes, int lane) {
	const bool vec = ((row_bytes | (uint32_t) (uintptr_t) src | (uint32_t) (uintptr_t) dst) & 15u) == 0u;
	if (vec) {
		if (row_bytes <= 64u * 16u) gs_copy_passes<1, LAUX>(src, dst, row_bytes, lane);
		else if (row_bytes <= 2u * 64u * 16u) gs_copy_passes<2, LAUX>(src, dst, row_bytes, lane);
		else gs_copy_passes<GS_CH, LAUX>(src, dst, row_bytes, lane);
	}
	else {
		typedef typename Elem<ELEM>::t E;
		const E * s = reinterpret_cast<const E *>(src);
		E * d = reinterpret_cast<E *>(dst);
		const uint32_t n = row_bytes / ELEM;
		for (uint32_t j = (uint32_t) lane; j < n; j += 64u) d[j] = s[j];
	}
}

template <int ELEM>
__device__ __forceinline__ void embedding_impl(int num_tokens, int embed_dim, const uint32_t * token_ids, const void * table, void * out) {
	const int lane = threadIdx.x & 63;
	/* uniform over the wave: the token index and row addresses live in SGPRs */
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wpb = blockDim.x >> 6;
	const uint32_t row_bytes = (uint32_t) embed_dim * (uint32_t) ELEM;
	for (long t = (long) blockIdx.x * wpb + wave; t < num_tokens; t += (long) gridDim.x * wpb) {
		const uint64_t id = load_scalar(token_ids + t);
		gs_copy_row<ELEM, GS_EMB_LOAD_AUX>(static_cast<const char *>(table) + id * row_bytes, static_cast<char *>(out) + (uint64_t) t * row_bytes, row_bytes, lane);
	}
}

template <int ELEM>
__device__ __forceinline__ void copy_to_seq_context_impl(uint64_t N, int kv_dim, const void * keys, const void * values,
															const int * seq_positions, const uint64_t * seq_context_ptrs,
															const int * seq_context_sizes) {
	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wpb = blockDim.x >> 6;
	const long n_tokens = (long) (N / (uint64_t) kv_dim);
	const uint32_t row_bytes = (uint32_t) kv_dim * (uint32_t) ELEM;
	for (long t = (long) blockIdx.x * wpb + wave; t < n_tokens; t += (long) gridDim.x * wpb) {
		/* per-token metadata, wave-uniform: scalar reads (13.8 -> 13.3 us per
		 * 8192 tokens on MI355X against vector loads) */
		char * ctx = reinterpret_cast<char *>(load_scalar(seq_context_ptrs + t));
		const uint64_t pos = (uint64_t) (int64_t) load_scalar(seq_positions + t);
		const uint64_t size = (uint64_t) (int64_t) load_scalar(seq_context_sizes + t);
		gs_copy_row<ELEM, GS_KV_LOAD_AUX>(static_cast<const char *>(keys) + (uint64_t) t * row_bytes, ctx + pos * row_bytes, row_bytes, lane);
		gs_copy_row<ELEM, GS_KV_LOAD_AUX>(static_cast<const char *>(values) + (uint64_t) t * row_bytes, ctx + (size + pos) * row_bytes, row_bytes, lane);
	}
}

#define GS_KERNELS(SUFFIX, T, ELEM)                                                                                   \
	extern "C" __global__ void __launch_bounds__(64 * GS_WAVES) embedding_##SUFFIX##_kernel(int num_tokens,         \
			int embed_dim, uint32_t * token_ids, T * embedding_table, T * output) {                                  \
		embedding_impl<ELEM>(num_tokens, embed_dim, token_ids, embedding_table, output);                            \
	}                                                                                                               \
	extern "C" __global__ void __launch_bounds__(64 * GS_WAVES) copy_to_seq_context_##SUFFIX##_kernel(uint64_t N,   \
			int total_tokens, int kv_dim, T * keys, T * values, int * seq_positions, uint64_t * seq_context_ptrs,    \
			int * seq_context_sizes) {                                                                               \
		copy_to_seq_context_impl<ELEM>(N, kv_dim, keys, values, seq_positions, seq_context_ptrs, seq_context_sizes); \
	}

GS_KERNELS(fp32, float, 4)
GS_KERNELS(fp16, f16_t, 2)
GS_KERNELS(bf16, bf16_t, 2)
GS_KERNELS(fp8e4m3, uint8_t, 1)
GS_KERNELS(fp8e5m2, uint8_t, 1)
