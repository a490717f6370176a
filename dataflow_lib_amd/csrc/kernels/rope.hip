/*
 * Rotary position embedding, forward and backward, in place on Q and K
 * (semantics of the reference's src/ops/nvidia/attention/rope.cu:3-57,123-180
 * and rope_bwd_x.cu:3-60,120-175; restated in the oracle's rope_* functions).
 *
 * Q is [T x model_dim], K is [T x num_kv_heads*head_dim], T = N / model_dim,
 * row-major, heads contiguous inside a row. Pairs are adjacent elements
 * (2p, 2p+1) of a head; pair p of token t turns by
 *   arg = (float) pos[t] * angle_p,   angle_p = (float) theta^(-(2p)/head_dim)
 * with angle_p and the fp32 product formed exactly as the reference does.
 *
 * One wave64 per token. angle_p is computed once per wave (fp64 pow, rounded
 * to fp32). Per token each lane evaluates cos/sin of one pair argument in
 * fp64 (rounded to fp32) into a per-wave LDS table shared by all 40 heads of
 * the token; the rotation uses a compensated fp32 two-term dot product, so
 * the fp32 result is within ~1 ulp even when the two products cancel.
 */
#include "dtypes.h"
#include "reduce.h"
#include "kernel_geometry.h"

/* a*b + c*d, with the rounding error of c*d added back */
__device__ __forceinline__ float dot2c(float a, float b, float c, float d) {
	const float p = c * d;
	const float pe = fmaf(c, d, -p);
	return fmaf(a, b, p) + pe;
}

template <bool BWD>
__device__ __forceinline__ void rotate(float c, float s, float e, float o, float & e2, float & o2) {
	if (!BWD) {
		e2 = dot2c(c, e, -s, o);   /* c*e - s*o */
		o2 = dot2c(c, o, s, e);    /* c*o + s*e */
	}
	else {
		e2 = dot2c(c, e, s, o);    /* c*e + s*o */
		o2 = dot2c(c, o, -s, e);   /* c*o - s*e */
	}
}

/* orders this wave's LDS table writes and reads (LDS only, so the wave's
 * global loads and stores stay in flight) */
__device__ __forceinline__ void wave_lds_sync() {
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
	__builtin_amdgcn_wave_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/* rotate one row (Q or K) of `width` elements with the token's table; the
 * rotated row is also written to `mirror` when it is not null (16-byte
 * aligned on the vector path) */
template <typename T, bool BWD, bool VECTOR>
__device__ __forceinline__ void rope_row(T * row, int width, int head_dim, const float2 * cs, int lane, T * mirror = nullptr) {
	if (VECTOR) {
		constexpr int VEC = VecOf<T>::N;
		const int nv = width / VEC;
		const int step = (64 * VEC) % head_dim;
		int col = (lane * VEC) % head_dim;
		R16 * rv = reinterpret_cast<R16 *>(row);
		for (int v = lane; v < nv; v += 64) {
			float f[VEC];
			unpack16<T>(rv[v], f);
			const int p0 = col >> 1;
#pragma unroll
			for (int q = 0; q < VEC / 2; q++) {
				const float2 t = cs[p0 + q];
				rotate<BWD>(t.x, t.y, f[2 * q], f[2 * q + 1], f[2 * q], f[2 * q + 1]);
			}
			const R16 o = pack16<T>(f);
			rv[v] = o;
			if (mirror) reinterpret_cast<R16 *>(mirror)[v] = o;
			col += step;
			if (col >= head_dim) col -= head_dim;
		}
	}
	else {
		const int npairs = width >> 1;
		const int step = 128 % head_dim;
		int col = (lane * 2) % head_dim;
		for (int p = lane; p < npairs; p += 64) {
			const float2 t = cs[col >> 1];
			float e2, o2;
			rotate<BWD>(t.x, t.y, to_f(row[2 * p]), to_f(row[2 * p + 1]), e2, o2);
			row[2 * p] = from_f<T>(e2);
			row[2 * p + 1] = from_f<T>(o2);
			if (mirror) {
				mirror[2 * p] = from_f<T>(e2);
				mirror[2 * p + 1] = from_f<T>(o2);
			}
			col += step;
			if (col >= head_dim) col -= head_dim;
		}
	}
}

/* Where the fused RoPE + KV-cache op puts token t's rows: the rotated K row
 * at row pos of the token's context and its V row at row S + pos
 * (copy_to_seq_context's layout, attention/copy_to_seq_context.cu:3-20). */
template <typename T>
struct KvCache {
	const T * values;
	const uint64_t * ctx_ptrs;
	const int * ctx_sizes;
	/* t is uniform over the wave, and so is the row (taken through
	 * readfirstlane, so buffer ranges built on it live in scalar registers) */
	__device__ __forceinline__ T * row(long t, int kv_dim, const int * seq_positions, bool value_row) const {
		const uint64_t c = load_scalar(ctx_ptrs + t);
		const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t) c), hi = __builtin_amdgcn_readfirstlane((uint32_t) (c >> 32));
		T * ctx = reinterpret_cast<T *>(((uint64_t) hi << 32) | lo);
		const int p = __builtin_amdgcn_readfirstlane(load_scalar(seq_positions + t) + (value_row ? load_scalar(ctx_sizes + t) : 0));
		return ctx + (long) p * (long) kv_dim;
	}
};

/* one wave copies a row of n elements (16-byte chunks when both rows and the
 * length allow it) */
template <typename T>
__device__ __forceinline__ void rope_copy_row(const T * src, T * dst, int n, int lane) {
	constexpr int VEC = VecOf<T>::N;
	if ((n % VEC) == 0 && aligned16(src) && aligned16(dst)) {
		const R16 * s = reinterpret_cast<const R16 *>(src);
		R16 * d = reinterpret_cast<R16 *>(dst);
		for (int v = lane; v < n / VEC; v += 64) d[v] = s[v];
	}
	else {
		for (int j = lane; j < n; j += 64) dst[j] = src[j];
	}
}

template <typename T, bool BWD, bool KV = false>
__device__ __forceinline__ void rope_impl(uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
											const int * seq_positions, T * X_q, T * X_k, KvCache<T> kv = KvCache<T>{}) {
	__shared__ float2 tables[ROPE_WAVES][ROPE_MAX_HEAD_DIM / 2];
	const int lane = threadIdx.x & 63;
	const int wave = threadIdx.x >> 6;
	const int wpb = blockDim.x >> 6;
	const long n_tokens = (long) (N / (uint64_t) model_dim);
	const int kv_dim = num_kv_heads * head_dim;
	const int half = head_dim >> 1;
	float2 * cs = tables[wave];

	/* angle_p for p = lane + 64k, exactly as the reference's fp32 expression
	 * powf(theta, -((float) c / (float) head_dim)) evaluated correctly rounded */
	float ang[ROPE_MAX_HEAD_DIM / 128];
#pragma unroll
	for (int k = 0; k < ROPE_MAX_HEAD_DIM / 128; k++) {
		const int p = lane + 64 * k;
		ang[k] = 0.0f;
		if (p < half) {
			const float expo = -((float) (2 * p) / (float) head_dim);
			ang[k] = (float) pow((double) (float) theta, (double) expo);
		}
	}

	constexpr int VEC = VecOf<T>::N;
	const bool vec_ok = (head_dim % VEC == 0) && aligned16(X_q) && aligned16(X_k);

	for (long t = (long) blockIdx.x * wpb + wave; t < n_tokens; t += (long) gridDim.x * wpb) {
		const float fpos = (float) seq_positions[t];
#pragma unroll
		for (int k = 0; k < ROPE_MAX_HEAD_DIM / 128; k++) {
			const int p = lane + 64 * k;
			if (p < half) {
				const float arg = fpos * ang[k];
				double sd, cd;
				sincos((double) arg, &sd, &cd);
				cs[p] = make_float2((float) cd, (float) sd);
			}
		}
		wave_lds_sync();
		T * kmirror = (KV && kv_dim > 0) ? kv.row(t, kv_dim, seq_positions, false) : nullptr;
		if (vec_ok) rope_row<T, BWD, true>(X_q + t * model_dim, model_dim, head_dim, cs, lane);
		else rope_row<T, BWD, false>(X_q + t * model_dim, model_dim, head_dim, cs, lane);
		if (vec_ok && (!KV || aligned16(kmirror))) rope_row<T, BWD, true>(X_k + t * kv_dim, kv_dim, head_dim, cs, lane, kmirror);
		else rope_row<T, BWD, false>(X_k + t * kv_dim, kv_dim, head_dim, cs, lane, kmirror);
		if (KV && kv_dim > 0) rope_copy_row<T>(kv.values + t * kv_dim, kv.row(t, kv_dim, seq_positions, true), kv_dim, lane);
		wave_lds_sync();
	}
}

/* pair index (column / 2) of 16-byte chunk `chunk` of a Q or K row */
template <typename T>
__device__ __forceinline__ int rope_pair_of(int chunk, int head_dim, bool pow2) {
	constexpr int VEC = VecOf<T>::N;
	const int col = pow2 ? ((chunk * VEC) & (head_dim - 1)) : ((chunk * VEC) % head_dim);
	return col >> 1;
}

/* Vector path: one workgroup of ROPE_SLOT_THREADS per group of TG
 * consecutive tokens at a time (TG = rope_tokens_per_group: 2 for fp8, whose
 * rows are half as long, else 1), persistent over groups g = block,
 * block + grid, ... The group's Q rows (and K rows) are contiguous, so they
 * are addressed as one span through one buffer range (chunks past the last
 * token read zero and store nowhere); chunk c of a span belongs to token
 * c / (row chunks). The next group's Q and K chunks are loaded, and waves
 * 0..TG-1 build its tokens' cos/sin tables into the other half of a
 * double-buffered LDS table, while this group is rotated and stored; one
 * barrier per group. */
template <typename T, bool BWD, bool KV = false, int TG = 1, int QJ = ROPE_QJ>
__device__ __forceinline__ void rope_slot(long n_tokens, int model_dim, int head_dim, int kv_dim, int theta,
											const int * seq_positions, T * X_q, T * X_k, KvCache<T> kv = KvCache<T>{}) {
	static_assert(!KV || TG == 1, "the KV-cache scatter runs one token per step");
	constexpr int VEC = VecOf<T>::N;
	constexpr int NT = ROPE_SLOT_THREADS;
	__shared__ float ang[ROPE_MAX_HEAD_DIM / 2];
	__shared__ __attribute__((aligned(16))) float2 tab[2][TG][ROPE_MAX_HEAD_DIM / 2];
	const int tid = threadIdx.x;
	const int lane = tid & 63;
	const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int half = head_dim >> 1;

	const int nvq = model_dim / VEC, nvk = kv_dim / VEC;
	const uint32_t qbytes = (uint32_t) model_dim * (uint32_t) sizeof(T), kbytes = (uint32_t) kv_dim * (uint32_t) sizeof(T);
	const bool pow2 = (head_dim & (head_dim - 1)) == 0;
	const long n_groups = (n_tokens + TG - 1) / TG;
	/* table entry of each owned chunk: its pair index (the same in every Q
	 * and K row, since both rows start at a head boundary) within the table
	 * of the chunk's token in the group (one index per chunk) */
	constexpr int TS = ROPE_MAX_HEAD_DIM / 2;
	int iq[QJ], ik[ROPE_KJ];
#pragma unroll
	for (int j = 0; j < QJ; j++) {
		const int c = tid + NT * j;
		const int tg = (TG == 1) ? 0 : c / nvq;
		iq[j] = (tg < TG ? tg : 0) * TS + rope_pair_of<T>(c, head_dim, pow2);
	}
#pragma unroll
	for (int j = 0; j < ROPE_KJ; j++) {
		const int c = tid + NT * j;
		const int tg = (TG == 1 || nvk == 0) ? 0 : c / nvk;
		ik[j] = (tg < TG ? tg : 0) * TS + rope_pair_of<T>(c, head_dim, pow2);
	}

	/* the cos/sin tables of group g's tokens into tab[b] (wave i builds token i) */
	auto table = [&](long g, int b) {
		const long t = g * TG + wv;
		if (wv >= TG || t >= n_tokens) return;
		const float fpos = (float) load_scalar(seq_positions + t);
		for (int p = lane; p < half; p += 64) {
			const float arg = fpos * ang[p];
			double sd, cd;
			sincos((double) arg, &sd, &cd);
			tab[b][wv][p] = make_float2((float) cd, (float) sd);
		}
	};
	/* byte ranges of group g's Q and K spans */
	auto span = [&](long g, uint32_t row_bytes) {
		const long left = n_tokens - g * TG;
		return (uint32_t) (left < TG ? left : TG) * row_bytes;
	};
	constexpr int VJ = KV ? ROPE_KJ : 1;
	auto load = [&](long g, R16 (&q)[QJ], R16 (&k)[ROPE_KJ], R16 (&v)[VJ]) {
		const long t = g * TG;
		const __amdgpu_buffer_rsrc_t rq = make_rsrc(X_q + t * model_dim, span(g, qbytes));
		const __amdgpu_buffer_rsrc_t rk = make_rsrc(X_k + t * kv_dim, span(g, kbytes));
#pragma unroll
		for (int j = 0; j < QJ; j++)
			if (NT * j < TG * nvq) q[j] = buf_load16_nt(rq, (uint32_t) (tid + NT * j) * 16u, 0);
#pragma unroll
		for (int j = 0; j < ROPE_KJ; j++)
			if (NT * j < TG * nvk) k[j] = buf_load16_nt(rk, (uint32_t) (tid + NT * j) * 16u, 0);
		if (KV) {
			const __amdgpu_buffer_rsrc_t rv = make_rsrc(kv.values + t * kv_dim, kbytes);
#pragma unroll
			for (int j = 0; j < VJ; j++)
				if (NT * j < nvk) v[j] = buf_load16_nt(rv, (uint32_t) (tid + NT * j) * 16u, 0);
		}
	};
	/* fp8 outputs keep 3 (E4M3) or 2 (E5M2) mantissa bits, so they take the
	 * reference's plain fp32 expression (rope.cu:212-213, one rounding per
	 * product) instead of the compensated one the 16- and 32-bit outputs need:
	 * 19.6 -> 17.8 us at the config-3 shapes, outputs within one code */
	auto rot = [&](R16 & r, int p0, const float2 * cs) {
		float f[VEC];
		unpack16<T>(r, f);
#pragma unroll
		for (int q = 0; q < VEC / 2; q++) {
			const float2 c = cs[p0 + q];
			if constexpr (IsFp8<T>::value) {
				const float e = f[2 * q], o = f[2 * q + 1];
				const float s = BWD ? -c.y : c.y;
				f[2 * q] = fmaf(c.x, e, -(s * o));
				f[2 * q + 1] = fmaf(c.x, o, s * e);
			}
			else {
				rotate<BWD>(c.x, c.y, f[2 * q], f[2 * q + 1], f[2 * q], f[2 * q + 1]);
			}
		}
		r = pack16<T>(f);
	};

	long t = blockIdx.x;   /* the group (the token when TG = 1) */
	const long stride = gridDim.x;
	R16 q[QJ], k[ROPE_KJ], v[VJ];
	/* the first group's chunks are requested before the angle setup, whose
	 * fp64 pow latency then overlaps the loads */
	if (t < n_groups) load(t, q, k, v);
	/* angle_p, exactly as the reference's fp32 expression
	 * powf(theta, -((float) c / (float) head_dim)) evaluated correctly rounded */
	for (int p = tid; p < half; p += NT) ang[p] = (float) pow((double) (float) theta, (double) -((float) (2 * p) / (float) head_dim));
	lds_barrier();   /* angles */
	if (t < n_groups) table(t, 0);
	lds_barrier();
	int b = 0;
	for (; t < n_groups; t += stride) {
		const long tn = t + stride;
		/* this token's chunks (requested one token ago) and the previous
		 * token's stores complete here, before the next token's chunks are
		 * requested, so the rotation below waits for nothing issued after
		 * them (left to itself, the compiler's wait for this token's chunks
		 * came after the next token's requests and waited for those too) */
		__builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0) */
		__builtin_amdgcn_sched_barrier(0);
		R16 qn[QJ], kn[ROPE_KJ], vn[VJ];
		if (tn < n_groups) {
			load(tn, qn, kn, vn);
			table(tn, b ^ 1);
		}
		/* fused KV-cache scatter: this token's context rows (scalar reads) */
		T * kctx = nullptr;
		T * vctx = nullptr;
		if (KV && kv_dim > 0) {
			kctx = kv.row(t, kv_dim, seq_positions, false);
			vctx = kv.row(t, kv_dim, seq_positions, true);
		}
		const __amdgpu_buffer_rsrc_t rq = make_rsrc(X_q + t * TG * model_dim, span(t, qbytes));
		const __amdgpu_buffer_rsrc_t rk = make_rsrc(X_k + t * TG * kv_dim, span(t, kbytes));
#pragma unroll
		for (int j = 0; j < QJ; j++) {
			if (NT * j < TG * nvq) {
				rot(q[j], iq[j], &tab[b][0][0]);
				buf_store16_aux<BUF_AUX_DEV | BUF_AUX_NT>(rq, (uint32_t) (tid + NT * j) * 16u, 0, q[j]);
			}
		}
#pragma unroll
		for (int j = 0; j < ROPE_KJ; j++) {
			if (NT * j < TG * nvk) {
				rot(k[j], ik[j], &tab[b][0][0]);
				buf_store16_aux<BUF_AUX_DEV | BUF_AUX_NT>(rk, (uint32_t) (tid + NT * j) * 16u, 0, k[j]);
			}
		}
		if (KV && kv_dim > 0) {
			/* context rows are 16-byte aligned unless the caller's contexts
			 * are not (a workgroup-uniform test per token); they are stored
			 * with the default cache policy (config-3 shapes: 40.8 -> 38.0 us
			 * against the streaming hint) */
			if (aligned16(kctx) && aligned16(vctx)) {
				const __amdgpu_buffer_rsrc_t rkc = make_rsrc(kctx, kbytes), rvc = make_rsrc(vctx, kbytes);
#pragma unroll
				for (int j = 0; j < ROPE_KJ; j++) {
					if (NT * j < nvk) {
						buf_store16_aux<0>(rkc, (uint32_t) (tid + NT * j) * 16u, 0, k[j]);
						buf_store16_aux<0>(rvc, (uint32_t) (tid + NT * j) * 16u, 0, v[j]);
					}
				}
			}
			else {
#pragma unroll
				for (int j = 0; j < ROPE_KJ; j++) {
					const int c = tid + NT * j;
					if (NT * j < nvk && c < nvk) {
						const T * ke = reinterpret_cast<const T *>(&k[j]);
						const T * ve = reinterpret_cast<const T *>(&v[j]);
#pragma unroll
						for (int e = 0; e < VEC; e++) {
							kctx[c * VEC + e] = ke[e];
							vctx[c * VEC + e] = ve[e];
						}
					}
				}
			}
		}
		/* tab[b ^ 1] complete, and every read of tab[b] done before it is
		 * rebuilt; the next group's loads stay in flight across it */
		lds_barrier();
#pragma unroll
		for (int j = 0; j < QJ; j++) q[j] = qn[j];
#pragma unroll
		for (int j = 0; j < ROPE_KJ; j++) k[j] = kn[j];
		if (KV) {
#pragma unroll
			for (int j = 0; j < VJ; j++) v[j] = vn[j];
		}
		b ^= 1;
	}
}

template <typename T, bool BWD, bool KV = false>
__device__ __forceinline__ void rope_dispatch(uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta,
											const int * seq_positions, T * X_q, T * X_k, KvCache<T> kv = KvCache<T>{}) {
	const int kv_dim = num_kv_heads * head_dim;
	unsigned long long ptr_or = (unsigned long long) (uintptr_t) X_q | (unsigned long long) (uintptr_t) X_k;
	if (KV) ptr_or |= (unsigned long long) (uintptr_t) kv.values;
	if (blockDim.x == ROPE_SLOT_THREADS && rope_slot_ok(model_dim, kv_dim, head_dim, (int) sizeof(T), ptr_or)) {
		const long n_tokens = (long) (N / (uint64_t) model_dim);
		if constexpr (!KV && IsFp8<T>::value) {
			if (rope_tokens_per_group(model_dim, kv_dim, (int) sizeof(T)) == 2) {
				rope_slot<T, BWD, false, 2, ROPE_TG2_QJ>(n_tokens, model_dim, head_dim, kv_dim, theta, seq_positions, X_q, X_k);
				return;
			}
		}
		rope_slot<T, BWD, KV>(n_tokens, model_dim, head_dim, kv_dim, theta, seq_positions, X_q, X_k, kv);
	}
	else
		rope_impl<T, BWD, KV>(N, model_dim, head_dim, num_kv_heads, theta, seq_positions, X_q, X_k, kv);
}

#define ROPE_KERNELS(SUFFIX, T)                                                                                     \
	extern "C" __global__ void __launch_bounds__(256) rope_##SUFFIX##_kernel(uint64_t N, int model_dim, int head_dim, \
			int num_kv_heads, int theta, int * seq_positions, T * X_q, T * X_k) {                                    \
		rope_dispatch<T, false>(N, model_dim, head_dim, num_kv_heads, theta, seq_positions, X_q, X_k);              \
	}                                                                                                               \
	extern "C" __global__ void __launch_bounds__(256) rope_bwd_x_##SUFFIX##_kernel(uint64_t N, int model_dim, int head_dim, \
			int num_kv_heads, int theta, int * seq_positions, T * dX_q, T * dX_k) {                                  \
		rope_dispatch<T, true>(N, model_dim, head_dim, num_kv_heads, theta, seq_positions, dX_q, dX_k);             \
	}

/* RoPE fused with the KV-cache scatter (no reference counterpart; the
 * reference notes the fusion at attention/rope.cu:50-54): rope forward on Q
 * and K in place, and the rotated K row and the V row of token t written to
 * rows p and S + p of its context, as copy_to_seq_context does. */
#define ROPE_KV_KERNELS(SUFFIX, T)                                                                                  \
	extern "C" __global__ void __launch_bounds__(256) rope_copy_to_seq_context_##SUFFIX##_kernel(uint64_t N,       \
			int model_dim, int head_dim, int num_kv_heads, int theta, int * seq_positions, T * X_q, T * X_k,         \
			T * values, uint64_t * seq_context_ptrs, int * seq_context_sizes) {                                      \
		rope_dispatch<T, false, true>(N, model_dim, head_dim, num_kv_heads, theta, seq_positions, X_q, X_k,         \
									  KvCache<T>{values, seq_context_ptrs, seq_context_sizes});                      \
	}

ROPE_KERNELS(fp32, float)
ROPE_KERNELS(fp16, f16_t)
ROPE_KERNELS(bf16, bf16_t)
ROPE_KV_KERNELS(fp32, float)
ROPE_KV_KERNELS(fp16, f16_t)
ROPE_KV_KERNELS(bf16, bf16_t)

/* fp8 forward only (reference: rope.cu:183-300; rope_bwd_x has no fp8 kernels) */
#define ROPE_FP8_KERNEL(SUFFIX, T)                                                                                  \
	extern "C" __global__ void __launch_bounds__(256, ROPE_SLOT_WG_PER_CU) rope_##SUFFIX##_kernel(uint64_t N, int model_dim, int head_dim, \
			int num_kv_heads, int theta, int * seq_positions, T * X_q, T * X_k) {                                    \
		rope_dispatch<T, false>(N, model_dim, head_dim, num_kv_heads, theta, seq_positions, X_q, X_k);              \
	}

ROPE_FP8_KERNEL(fp8e4m3, fp8e4m3_t)
ROPE_FP8_KERNEL(fp8e5m2, fp8e5m2_t)
