/*
 * Datatype helpers (reference: src/datatype/src/dataflow_datatype.c:4-78).
 * The strings returned by dataflow_datatype_as_string are hashed into op
 * fingerprints, so they must stay byte-identical to the reference's.
 */
#include "dataflow_datatype.h"

size_t dataflow_sizeof_element(DataflowDatatype arr_dtype) {
	switch (arr_dtype) {
		case DATAFLOW_FP64:    return 8;
		case DATAFLOW_FP32:    return 4;
		case DATAFLOW_FP16:    return 2;
		case DATAFLOW_BF16:    return 2;
		case DATAFLOW_FP8E4M3: return 1;
		case DATAFLOW_FP8E5M2: return 1;
		case DATAFLOW_UINT64:  return 8;
		case DATAFLOW_UINT32:  return 4;
		case DATAFLOW_UINT16:  return 2;
		case DATAFLOW_UINT8:   return 1;
		case DATAFLOW_LONG:    return sizeof(long);
		case DATAFLOW_INT:     return sizeof(int);
		/* VOID, BOOL, NONE and every *_SCALAR carry no array element size */
		default:               return 0;
	}
}

char * dataflow_datatype_as_string(DataflowDatatype dtype) {
	static const struct { DataflowDatatype dt; char * name; } names[] = {
		{DATAFLOW_VOID, "VOID"}, {DATAFLOW_FP64, "FP64"}, {DATAFLOW_FP32, "FP32"},
		{DATAFLOW_FP16, "FP16"}, {DATAFLOW_BF16, "BF16"}, {DATAFLOW_FP8E4M3, "FP8E4M3"},
		{DATAFLOW_FP8E5M2, "FP8E5M2"}, {DATAFLOW_UINT64, "UINT64"}, {DATAFLOW_UINT32, "UINT32"},
		{DATAFLOW_UINT16, "UINT16"}, {DATAFLOW_UINT8, "UINT8"}, {DATAFLOW_LONG, "LONG"},
		{DATAFLOW_INT, "INT"},
	};
	for (size_t i = 0; i < sizeof(names) / sizeof(names[0]); i++) {
		if (names[i].dt == dtype) {
			return names[i].name;
		}
	}
	return "UNKNOWN";
}

/* ---- host conversions (round-to-nearest-even on narrowing) ---- */

static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static inline uint16_t f32_to_bf16_rne(float f) {
	uint32_t u = f32_bits(f);
	if ((u & 0x7fffffffu) > 0x7f800000u) {
		/* NaN: keep sign, force a quiet payload bit */
		return (uint16_t) ((u >> 16) | 0x40u);
	}
	u += 0x7fffu + ((u >> 16) & 1u);
	return (uint16_t) (u >> 16);
}

static inline float bf16_to_f32(uint16_t h) { return bits_f32(((uint32_t) h) << 16); }

static inline float f16_to_f32(uint16_t h) {
	uint32_t sign = ((uint32_t) (h & 0x8000u)) << 16;
	uint32_t exp = (h >> 10) & 0x1fu;
	uint32_t man = h & 0x3ffu;
	if (exp == 0) {
		/* zero or subnormal: man * 2^-24 is exact in fp32 */
		float v = (float) man * bits_f32(0x33800000u);
		return sign ? -v : v;
	}
	if (exp == 31) {
		return bits_f32(sign | 0x7f800000u | (man << 13));
	}
	return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

static inline uint16_t f32_to_f16_rne(float f) {
	uint32_t u = f32_bits(f);
	uint16_t sign = (uint16_t) ((u >> 16) & 0x8000u);
	uint32_t a = u & 0x7fffffffu;
	if (a > 0x7f800000u) return (uint16_t) (sign | 0x7e00u);
	if (a >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); /* rounds to inf */
	if (a < 0x38800000u) {
		/* result is subnormal (or zero) in fp16: scale by 2^24 and round */
		float v = bits_f32(a) * 16777216.0f;
		/* v < 1024, integer rounding under the default RNE mode */
		uint32_t r = (uint32_t) __builtin_rintf(v);
		return (uint16_t) (sign | r);
	}
	uint32_t man = a & 0x7fffffu;
	uint32_t exp = (a >> 23) - 112u;
	uint32_t h = (exp << 10) | (man >> 13);
	uint32_t rem = man & 0x1fffu;
	if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
	return (uint16_t) (sign | h);
}

typedef struct {
	void * to; void * from;
	DataflowDatatype to_dt; DataflowDatatype from_dt;
	long start; long end;
} Convert_Range;

static void convert_range(Convert_Range * r) {
	for (long i = r->start; i < r->end; i++) {
		float v;
		switch (r->from_dt) {
			case DATAFLOW_FP32: v = ((const float *) r->from)[i]; break;
			case DATAFLOW_BF16: v = bf16_to_f32(((const uint16_t *) r->from)[i]); break;
			default:            v = f16_to_f32(((const uint16_t *) r->from)[i]); break;
		}
		switch (r->to_dt) {
			case DATAFLOW_FP32: ((float *) r->to)[i] = v; break;
			case DATAFLOW_BF16: ((uint16_t *) r->to)[i] = f32_to_bf16_rne(v); break;
			default:            ((uint16_t *) r->to)[i] = f32_to_f16_rne(v); break;
		}
	}
}

static void * convert_worker(void * arg) {
	convert_range((Convert_Range *) arg);
	return NULL;
}

static bool is_float_storage(DataflowDatatype dt) {
	return dt == DATAFLOW_FP32 || dt == DATAFLOW_FP16 || dt == DATAFLOW_BF16;
}

int dataflow_convert_datatype(void * to, void * from, DataflowDatatype to_dt, DataflowDatatype from_dt, long n, int num_threads) {
	if (!is_float_storage(to_dt) || !is_float_storage(from_dt)) {
		fprintf(stderr, "Error: conversion from %s to %s is not supported...\n",
				dataflow_datatype_as_string(from_dt), dataflow_datatype_as_string(to_dt));
		return -1;
	}
	if (n <= 0) {
		return 0;
	}
	if (num_threads < 1) num_threads = 1;
	if (num_threads > 64) num_threads = 64;
	if ((long) num_threads > n) num_threads = (int) n;

	Convert_Range ranges[64];
	pthread_t threads[64];
	bool spawned[64] = {false};
	long per = n / num_threads, extra = n % num_threads, cur = 0;
	for (int t = 0; t < num_threads; t++) {
		long len = per + (t < extra ? 1 : 0);
		ranges[t] = (Convert_Range) {to, from, to_dt, from_dt, cur, cur + len};
		cur += len;
	}
	for (int t = 1; t < num_threads; t++) {
		spawned[t] = (pthread_create(&threads[t], NULL, convert_worker, &ranges[t]) == 0);
		if (!spawned[t]) {
			/* could not start a thread: convert this range on the caller */
			convert_range(&ranges[t]);
		}
	}
	convert_range(&ranges[0]);
	for (int t = 1; t < num_threads; t++) {
		if (spawned[t]) pthread_join(threads[t], NULL);
	}
	return 0;
}
