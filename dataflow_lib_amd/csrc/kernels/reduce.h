/*
 * Wave64 and workgroup reductions for gfx950.
 *
 * Inside a wave: two quad_perm DPP steps, then row_half_mirror and row_mirror
 * (every lane of a 16-lane row ends with the row total), then the four row
 * totals are read with v_readlane and combined in a fixed order. The result is
 * wave-uniform and bitwise reproducible.
 */
#pragma once

#include <hip/hip_runtime.h>

/* Workgroup barrier that orders LDS only. __syncthreads() is a release/acquire
 * fence over all memory, so every wave first waits for all of its outstanding
 * global loads and stores (vmcnt 0), which stalls loads issued early for later
 * work. This barrier waits only for the wave's own LDS accesses (lgkmcnt 0), so
 * such loads stay in flight across it. Use it only where the barrier publishes
 * LDS data (direct-to-LDS buffer loads are vector-memory traffic and are not
 * covered). */
__device__ __forceinline__ void lds_barrier() {
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
	__builtin_amdgcn_s_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
	return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

#define DPP_QUAD_1032 0xB1      /* quad_perm [1,0,3,2] */
#define DPP_QUAD_2301 0x4E      /* quad_perm [2,3,0,1] */
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_HALF_MIRROR 0x141

__device__ __forceinline__ float readlane_f32(float v, int lane) {
	return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
	v += dpp_f32<DPP_QUAD_1032>(v);
	v += dpp_f32<DPP_QUAD_2301>(v);
	v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
	v += dpp_f32<DPP_ROW_MIRROR>(v);
	float a = readlane_f32(v, 0) + readlane_f32(v, 16);
	float b = readlane_f32(v, 32) + readlane_f32(v, 48);
	return a + b;
}

__device__ __forceinline__ float wave_max(float v) {
	v = fmaxf(v, dpp_f32<DPP_QUAD_1032>(v));
	v = fmaxf(v, dpp_f32<DPP_QUAD_2301>(v));
	v = fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
	v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
	float a = fmaxf(readlane_f32(v, 0), readlane_f32(v, 16));
	float b = fmaxf(readlane_f32(v, 32), readlane_f32(v, 48));
	return fmaxf(a, b);
}

/* Sum over the waves of a workgroup (or of a group of NW consecutive waves).
 * slots: LDS array with one float per wave of the group. Includes the
 * barriers it needs; call from every thread of the workgroup. */
template <int NW>
__device__ __forceinline__ float group_sum(float wave_total, float * slots, int wave_in_group) {
	if ((threadIdx.x & 63) == 0) slots[wave_in_group] = wave_total;
	lds_barrier();
	float t = 0.0f;
#pragma unroll
	for (int w = 0; w < NW; w++) t += slots[w];
	return t;
}
