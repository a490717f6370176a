/*
 * Storage types and 16-byte vector pack/unpack for the gfx950 kernels.
 *
 * Storage: fp32, fp16 (IEEE binary16) and bf16, all row-major. Arithmetic is
 * always fp32. Narrowing conversions round to nearest even: bf16 pairs use
 * the gfx950 packed convert (v_cvt_pk_bf16_f32), fp16 the IEEE convert.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_v;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_v;

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_v;

/* one 16-byte memory vector */
struct __attribute__((aligned(16))) R16 {
	uint32_t w[4];
};

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16_t x) { return __uint_as_float(((uint32_t) x.bits) << 16); }
__device__ __forceinline__ float to_f(f16_t x) { return (float) __builtin_bit_cast(_Float16, x.bits); }

template <typename T> __device__ __forceinline__ T from_f(float f);
template <> __device__ __forceinline__ float from_f<float>(float f) { return f; }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float f) { return bf16_t{__builtin_bit_cast(uint16_t, (__bf16) f)}; }
template <> __device__ __forceinline__ f16_t from_f<f16_t>(float f) { return f16_t{__builtin_bit_cast(uint16_t, (_Float16) f)}; }

/* elements per 16-byte vector */
template <typename T> struct VecOf { static constexpr int N = 16 / (int) sizeof(T); };

/* low / high element of a packed 2 x 16-bit word */
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
	bf16x2_v v = {(__bf16) lo, (__bf16) hi};
	return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
	f16x2_v v = {(_Float16) lo, (_Float16) hi};
	return __builtin_bit_cast(uint32_t, v);
}

template <typename T> __device__ __forceinline__ void unpack16(const R16 & r, float * f);
template <> __device__ __forceinline__ void unpack16<float>(const R16 & r, float * f) {
#pragma unroll
	for (int i = 0; i < 4; i++) f[i] = __uint_as_float(r.w[i]);
}
template <> __device__ __forceinline__ void unpack16<bf16_t>(const R16 & r, float * f) {
#pragma unroll
	for (int i = 0; i < 4; i++) { f[2 * i] = bf16_lo(r.w[i]); f[2 * i + 1] = bf16_hi(r.w[i]); }
}
template <> __device__ __forceinline__ void unpack16<f16_t>(const R16 & r, float * f) {
#pragma unroll
	for (int i = 0; i < 4; i++) {
		f16x2_v h = __builtin_bit_cast(f16x2_v, r.w[i]);
		f[2 * i] = (float) h.x;
		f[2 * i + 1] = (float) h.y;
	}
}

template <typename T> __device__ __forceinline__ R16 pack16(const float * f);
template <> __device__ __forceinline__ R16 pack16<float>(const float * f) {
	R16 r;
#pragma unroll
	for (int i = 0; i < 4; i++) r.w[i] = __float_as_uint(f[i]);
	return r;
}
template <> __device__ __forceinline__ R16 pack16<bf16_t>(const float * f) {
	R16 r;
#pragma unroll
	for (int i = 0; i < 4; i++) r.w[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
	return r;
}
template <> __device__ __forceinline__ R16 pack16<f16_t>(const float * f) {
	R16 r;
#pragma unroll
	for (int i = 0; i < 4; i++) r.w[i] = pack_f16x2(f[2 * i], f[2 * i + 1]);
	return r;
}

/*
 * fp8 storage: the OCP 8-bit formats E4M3 (bias 7, no infinities, max 448)
 * and E5M2 (bias 15, max 57344), which gfx950's conversion instructions
 * implement (v_cvt_pk_f32_fp8 / _bf8 decode two codes, v_cvt_pk_fp8_f32 /
 * _bf8_f32 encode two floats with round to nearest even; out of range they
 * give NaN / inf). Encoding saturates to the largest
 * finite value, as the reference's conversions do (CUDA's fp8 constructors
 * from float, __NV_SATFINITE): the input is clamped to +-max first, NaN kept.
 * fp8 is a forward-only storage type.
 */
struct fp8e4m3_t { uint8_t bits; };
struct fp8e5m2_t { uint8_t bits; };
template <typename T> struct IsFp8 { static constexpr bool value = false; };
template <> struct IsFp8<fp8e4m3_t> { static constexpr bool value = true; };
template <> struct IsFp8<fp8e5m2_t> { static constexpr bool value = true; };

__device__ __forceinline__ float to_f(fp8e4m3_t x) { return __builtin_amdgcn_cvt_f32_fp8((int) x.bits, 0); }
__device__ __forceinline__ float to_f(fp8e5m2_t x) { return __builtin_amdgcn_cvt_f32_bf8((int) x.bits, 0); }

typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <typename T> struct Fp8Traits;
template <> struct Fp8Traits<fp8e4m3_t> {
	static constexpr float MAX = 448.0f;
	/* two floats into bytes 0-1 (hi = false) or 2-3 (hi = true) of `old` */
	__device__ static __forceinline__ uint32_t cvt_pk(float a, float b, uint32_t old, bool hi) {
		return hi ? (uint32_t) __builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int) old, true)
				  : (uint32_t) __builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int) old, false);
	}
	/* bytes 0-1 (hi = false) or 2-3 (hi = true) of w, two per instruction */
	__device__ static __forceinline__ void unpack2(uint32_t w, bool hi, float * f) {
		const f32x2_t v = hi ? __builtin_amdgcn_cvt_pk_f32_fp8((int) w, true) : __builtin_amdgcn_cvt_pk_f32_fp8((int) w, false);
		f[0] = v.x;
		f[1] = v.y;
	}
};
template <> struct Fp8Traits<fp8e5m2_t> {
	static constexpr float MAX = 57344.0f;
	__device__ static __forceinline__ uint32_t cvt_pk(float a, float b, uint32_t old, bool hi) {
		return hi ? (uint32_t) __builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int) old, true)
				  : (uint32_t) __builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int) old, false);
	}
	__device__ static __forceinline__ void unpack2(uint32_t w, bool hi, float * f) {
		const f32x2_t v = hi ? __builtin_amdgcn_cvt_pk_f32_bf8((int) w, true) : __builtin_amdgcn_cvt_pk_f32_bf8((int) w, false);
		f[0] = v.x;
		f[1] = v.y;
	}
};

/* clamp to +-max, NaN kept (the saturating conversion's range) */
template <typename T>
__device__ __forceinline__ float fp8_sat(float f) {
	const float m = Fp8Traits<T>::MAX;
	return (f != f) ? f : __builtin_fminf(__builtin_fmaxf(f, -m), m);
}
/* four floats into one word, byte k = element k */
template <typename T>
__device__ __forceinline__ uint32_t fp8_pack4(float a, float b, float c, float d) {
	const uint32_t lo = Fp8Traits<T>::cvt_pk(fp8_sat<T>(a), fp8_sat<T>(b), 0u, false);
	return Fp8Traits<T>::cvt_pk(fp8_sat<T>(c), fp8_sat<T>(d), lo, true);
}
template <typename T>
__device__ __forceinline__ void fp8_unpack4(uint32_t w, float * f) {
	Fp8Traits<T>::unpack2(w, false, f);
	Fp8Traits<T>::unpack2(w, true, f + 2);
}

template <> __device__ __forceinline__ fp8e4m3_t from_f<fp8e4m3_t>(float f) {
	return fp8e4m3_t{(uint8_t) (fp8_pack4<fp8e4m3_t>(f, 0.0f, 0.0f, 0.0f) & 0xffu)};
}
template <> __device__ __forceinline__ fp8e5m2_t from_f<fp8e5m2_t>(float f) {
	return fp8e5m2_t{(uint8_t) (fp8_pack4<fp8e5m2_t>(f, 0.0f, 0.0f, 0.0f) & 0xffu)};
}

template <> __device__ __forceinline__ void unpack16<fp8e4m3_t>(const R16 & r, float * f) {
#pragma unroll
	for (int i = 0; i < 4; i++) fp8_unpack4<fp8e4m3_t>(r.w[i], f + 4 * i);
}
template <> __device__ __forceinline__ void unpack16<fp8e5m2_t>(const R16 & r, float * f) {
#pragma unroll
	for (int i = 0; i < 4; i++) fp8_unpack4<fp8e5m2_t>(r.w[i], f + 4 * i);
}
/* sixteen floats into sixteen fp8 codes. The clamp to +-max is one v_med3
 * per element, which maps NaN to -max; NaN is looked for one pair at a time
 * (one unordered compare per two elements), and only lanes that hold one
 * redo their chunk with the NaN-keeping clamp. */
template <typename T>
__device__ __forceinline__ R16 fp8_pack16(const float * f) {
	constexpr float m = Fp8Traits<T>::MAX;
	bool nan = false;
#pragma unroll
	for (int i = 0; i < 16; i += 2) nan |= __builtin_isunordered(f[i], f[i + 1]);
	R16 r;
	if (__builtin_expect(nan, 0)) {
#pragma unroll
		for (int i = 0; i < 4; i++) r.w[i] = fp8_pack4<T>(f[4 * i], f[4 * i + 1], f[4 * i + 2], f[4 * i + 3]);
	}
	else {
#pragma unroll
		for (int i = 0; i < 4; i++) {
			const uint32_t lo = Fp8Traits<T>::cvt_pk(__builtin_amdgcn_fmed3f(f[4 * i], -m, m), __builtin_amdgcn_fmed3f(f[4 * i + 1], -m, m), 0u, false);
			r.w[i] = Fp8Traits<T>::cvt_pk(__builtin_amdgcn_fmed3f(f[4 * i + 2], -m, m), __builtin_amdgcn_fmed3f(f[4 * i + 3], -m, m), lo, true);
		}
	}
	return r;
}
template <> __device__ __forceinline__ R16 pack16<fp8e4m3_t>(const float * f) { return fp8_pack16<fp8e4m3_t>(f); }
template <> __device__ __forceinline__ R16 pack16<fp8e5m2_t>(const float * f) { return fp8_pack16<fp8e5m2_t>(f); }

/* 8 bytes: eight fp8 elements, or the fp8 half of a mixed fp8 x 16-bit chunk */
struct __attribute__((aligned(8))) R8 {
	uint32_t w[2];
};
template <typename T>
__device__ __forceinline__ void unpack8_fp8(const R8 & r, float * f) {
	fp8_unpack4<T>(r.w[0], f);
	fp8_unpack4<T>(r.w[1], f + 4);
}

/*
 * A "chunk" is V consecutive elements handled by one lane: V = VecOf<T>::N
 * (one 16-byte access) on the vector path, V = 1 on the element path used
 * for unaligned or ragged rows. raw_t is what sits in registers.
 */
template <typename T, int V> struct Chunk {
	using raw_t = R16;
	static_assert(V == VecOf<T>::N, "vector chunk must be 16 bytes");
	__device__ static __forceinline__ raw_t load(const T * base, long idx) { return reinterpret_cast<const R16 *>(base)[idx]; }
	__device__ static __forceinline__ void store(T * base, long idx, const raw_t & r) { reinterpret_cast<R16 *>(base)[idx] = r; }
	__device__ static __forceinline__ void unpack(const raw_t & r, float * f) { unpack16<T>(r, f); }
	__device__ static __forceinline__ raw_t pack(const float * f) { return pack16<T>(f); }
	__device__ static __forceinline__ raw_t zero() { R16 r; r.w[0] = r.w[1] = r.w[2] = r.w[3] = 0u; return r; }
};
template <typename T> struct Chunk<T, 1> {
	using raw_t = T;
	__device__ static __forceinline__ raw_t load(const T * base, long idx) { return base[idx]; }
	__device__ static __forceinline__ void store(T * base, long idx, const raw_t & r) { base[idx] = r; }
	__device__ static __forceinline__ void unpack(const raw_t & r, float * f) { f[0] = to_f(r); }
	__device__ static __forceinline__ raw_t pack(const float * f) { return from_f<T>(f[0]); }
	__device__ static __forceinline__ raw_t zero() { return from_f<T>(0.0f); }
};

__device__ __forceinline__ bool aligned16(const void * p) { return (((uintptr_t) p) & 15u) == 0; }

/* Empty register barrier: tells the compiler the 16 bytes may have changed,
 * so values derived from them earlier (unpacked floats) are recomputed from
 * the packed registers instead of being kept alive (and spilled) across a pass. */
/* Software-pipelined loops wait here, at the top of each step, for every
 * outstanding vector-memory access (s_waitcnt vmcnt(0): the loads issued one
 * step ago and the stores of the step before), and only then issue the next
 * step's loads. Left to itself the compiler placed its wait for this step's
 * data after the next step's loads (the loads sit under branches), which
 * waited for those too and serialised the pipeline. */
__device__ __forceinline__ void vmem_wait_all() {
	__builtin_amdgcn_s_waitcnt(0x0F70);   /* vmcnt(0); expcnt, lgkmcnt at their maxima */
	__builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void reg_barrier(R16 & r) {
	__asm__ volatile("" : "+v"(r.w[0]), "+v"(r.w[1]), "+v"(r.w[2]), "+v"(r.w[3]));
}

/* A wave-uniform read of memory the kernel does not write, through the
 * scalar cache: an s_load (a read; nothing here stores through that cache),
 * waited for with lgkmcnt, so it does not wait behind the wave's
 * vector-memory traffic. The address must be the same in every lane. */
template <typename T>
__device__ __forceinline__ T load_scalar(const T * p) {
	return *(const __attribute__((address_space(4))) T *) (uintptr_t) p;
}

/* 16-byte global accesses with the non-temporal hint, for data each kernel
 * touches exactly once */
__device__ __forceinline__ R16 ld16_nt(const void * p) {
	const u32x4_v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_v *>(p));
	R16 o;
	o.w[0] = v.x; o.w[1] = v.y; o.w[2] = v.z; o.w[3] = v.w;
	return o;
}
__device__ __forceinline__ void st16_nt(void * p, const R16 & x) {
	const u32x4_v v = {x.w[0], x.w[1], x.w[2], x.w[3]};
	__builtin_nontemporal_store(v, reinterpret_cast<u32x4_v *>(p));
}

/*
 * Raw buffer access: a 128-bit resource (base, byte range) in SGPRs, a
 * per-lane byte offset in one VGPR and a wave-uniform byte offset in an SGPR.
 * Loads past the range return zero and stores past it are dropped, so ragged
 * tails need no branches. dword3 = 0x00020000 is the raw 32-bit data format
 * used by gfx9-family buffer instructions.
 */
#define RAW_BUFFER_DWORD3 0x00020000

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void * base, uint32_t num_bytes) {
	return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short) 0, (int) num_bytes, RAW_BUFFER_DWORD3);
}
__device__ __forceinline__ R16 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
	const u32x4_v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
	R16 o;
	o.w[0] = v.x; o.w[1] = v.y; o.w[2] = v.z; o.w[3] = v.w;
	return o;
}
/* A VALU write to a data VGPR of a wider-than-8-byte buffer store issued just
 * before it can change the data the store writes (observed on gfx950 with an
 * SGPR soffset, where the compiler inserts no wait). So every 16-byte buffer
 * store is followed by two wait states during which its data registers stay
 * unchanged (they are inputs of the s_nop). */
__device__ __forceinline__ void store_data_guard(const u32x4_v & v) {
	__asm__ volatile("s_nop 1" : : "v"(v) : "memory");
}
__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const R16 & x) {
	const u32x4_v v = {x.w[0], x.w[1], x.w[2], x.w[3]};
	__builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, 0);
	store_data_guard(v);
}

/* Cache-policy bits of a gfx950 buffer instruction: bit 0 sc0, bit 1 nt (the
 * streaming hint), bit 4 sc1; sc1:sc0 is the scope at which the access is
 * coherent (2 = device, i.e. across the XCDs' separate L2s).
 * Data touched once is loaded and stored with the streaming hint, so
 * single-use streams do not evict lines that other waves still reuse.
 * BUF_AUX_DEV (device scope, which writes the line through the XCD's L2) is
 * used where a kernel stores to lines it has just read: the RMSNorm backward
 * kernels' dX (8192 x 4096 bf16, fused backward 48.6 -> 46.5 us per launch;
 * fp8-input bwd_x 40.8 -> 33.1 us) and, together with the streaming hint,
 * RoPE's in-place Q and K (30.2 -> 29.9 us). Part of the saving is write
 * traffic that drains while the next kernel runs: in a sequence of different
 * memory-bound ops the ops after these run slower by up to as much (a
 * sequence of the step's seven ops measured 641 us either way). */
#define BUF_AUX_NT 2
#define BUF_AUX_DEV 16
__device__ __forceinline__ R16 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
	const u32x4_v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, BUF_AUX_NT);
	R16 o;
	o.w[0] = v.x; o.w[1] = v.y; o.w[2] = v.z; o.w[3] = v.w;
	return o;
}
template <int AUX>
__device__ __forceinline__ R16 buf_load16_aux(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
	const u32x4_v v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX);
	R16 o;
	o.w[0] = v.x; o.w[1] = v.y; o.w[2] = v.z; o.w[3] = v.w;
	return o;
}
template <int AUX>
__device__ __forceinline__ void buf_store16_aux(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const R16 & x) {
	const u32x4_v v = {x.w[0], x.w[1], x.w[2], x.w[3]};
	__builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, AUX);
	store_data_guard(v);
}
__device__ __forceinline__ void buf_store16_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const R16 & x) {
	buf_store16_aux<BUF_AUX_NT>(r, voff, soff, x);
}
