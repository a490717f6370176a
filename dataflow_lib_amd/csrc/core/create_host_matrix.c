/*
 * Host matrices and the raw .dat format (reference:
 * src/dataflow_handle/nvidia/test/create_host_matrix.c:4-291): values are made
 * in fp32 and converted to the requested type with dataflow_convert_datatype.
 */
#include "create_host_matrix.h"

#include <math.h>

#define HOST_MATRIX_THREADS 8

static uint64_t g_state = 42;
static int g_generator = HOST_MATRIX_RAND_PORTABLE;

void host_matrix_seed(uint64_t seed) { g_state = seed; }

int host_matrix_set_generator(int generator) {
	if (generator != HOST_MATRIX_RAND_PORTABLE && generator != HOST_MATRIX_RAND_LIBC) {
		fprintf(stderr, "Error: host matrix: unknown generator %d...\n", generator);
		return -1;
	}
	g_generator = generator;
	return 0;
}

/* The reference harnesses' generator (test/create_host_matrix.c:4-29): the
 * polar method of Marsaglia on the C library's rand(), one value kept back
 * for the next call. The evaluation types follow that code exactly (the
 * uniform draws and the square root are fp32, the log ratio fp64), so with
 * the same srand() seed and the same C library the matrices are identical. */
static float g_libc_kept;
static int g_libc_has_kept;

static float libc_polar_normal(float mean, float std) {
	if (std == 0.0f) return mean;
	if (g_libc_has_kept) {
		g_libc_has_kept = 0;
		return mean + std * g_libc_kept;
	}
	float x, y, q;
	for (;;) {
		x = (float) ((double) ((float) rand() / (float) RAND_MAX) * 2.0 - 1.0);
		y = (float) ((double) ((float) rand() / (float) RAND_MAX) * 2.0 - 1.0);
		q = x * x + y * y;
		if (q < 1.0f && q != 0.0f) break;
	}
	const float f = sqrtf((float) (-2.0 * (double) logf(q) / (double) q));
	g_libc_kept = y * f;
	g_libc_has_kept = 1;
	return mean + std * x * f;
}

/* splitmix64 (Steele, Lea, Flood 2014) */
static uint64_t next_u64(void) {
	uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
	z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
	z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
	return z ^ (z >> 31);
}

/* uniform in (0, 1]: 53 random bits, never 0 so log() is finite */
static double next_unit(void) { return ((double) (next_u64() >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

/* standard normal pairs by the Box-Muller transform, in fp64 */
static void normal_pair(double * a, double * b) {
	const double r = sqrt(-2.0 * log(next_unit()));
	const double t = 6.283185307179586476925286766559 * next_unit();
	*a = r * cos(t);
	*b = r * sin(t);
}

static void * dest_or_alloc(void * opt_dest, uint64_t num_els, DataflowDatatype dt, const char * what) {
	const size_t el = dataflow_sizeof_element(dt);
	if (el == 0) {
		fprintf(stderr, "Error: %s: no element size for dtype %s...\n", what, dataflow_datatype_as_string(dt));
		return NULL;
	}
	if (opt_dest) return opt_dest;
	void * p = malloc((num_els * el != 0) ? num_els * el : 1);
	if (!p) fprintf(stderr, "Error: %s: could not allocate %lu elements on the host...\n", what, (unsigned long) num_els);
	return p;
}

/* fp32 values -> dt, into opt_dest or a new buffer; frees `vals` */
static void * finish_from_f32(float * vals, uint64_t num_els, DataflowDatatype dt, void * opt_dest, const char * what) {
	void * dest = dest_or_alloc(opt_dest, num_els, dt, what);
	if (!dest) {
		free(vals);
		return NULL;
	}
	if (dataflow_convert_datatype(dest, vals, dt, DATAFLOW_FP32, (long) num_els, HOST_MATRIX_THREADS)) {
		fprintf(stderr, "Error: %s: conversion from FP32 to %s failed...\n", what, dataflow_datatype_as_string(dt));
		if (!opt_dest) free(dest);
		free(vals);
		return NULL;
	}
	free(vals);
	return dest;
}

static float * f32_buffer(uint64_t num_els, const char * what) {
	float * v = (float *) calloc(num_els ? num_els : 1, sizeof(float));
	if (!v) fprintf(stderr, "Error: %s: could not allocate a temporary fp32 matrix of %lu elements...\n", what, (unsigned long) num_els);
	return v;
}

void * create_zero_host_matrix(uint64_t M, uint64_t N, DataflowDatatype dt, void * opt_dest) {
	void * dest = dest_or_alloc(opt_dest, M * N, dt, "create zero host matrix");
	if (dest) memset(dest, 0, M * N * dataflow_sizeof_element(dt));
	return dest;
}

void * create_rand_host_matrix(uint64_t M, uint64_t N, float mean, float std, DataflowDatatype dt, void * opt_dest) {
	const uint64_t n = M * N;
	float * v = f32_buffer(n, "create rand host matrix");
	if (!v) return NULL;
	if (g_generator == HOST_MATRIX_RAND_LIBC) {
		for (uint64_t i = 0; i < n; i++) v[i] = libc_polar_normal(mean, std);
		return finish_from_f32(v, n, dt, opt_dest, "create rand host matrix");
	}
	for (uint64_t i = 0; i < n; i += 2) {
		double a, b;
		normal_pair(&a, &b);
		v[i] = (float) ((double) mean + (double) std * a);
		if (i + 1 < n) v[i + 1] = (float) ((double) mean + (double) std * b);
	}
	return finish_from_f32(v, n, dt, opt_dest, "create rand host matrix");
}

void * create_identity_host_matrix(uint64_t N, DataflowDatatype dt, void * opt_dest) {
	float * v = f32_buffer(N * N, "create identity host matrix");
	if (!v) return NULL;
	for (uint64_t i = 0; i < N; i++) v[i * N + i] = 1.0f;
	return finish_from_f32(v, N * N, dt, opt_dest, "create identity host matrix");
}

void * create_index_identity_host_matrix(uint64_t M, uint64_t N, DataflowDatatype dt, void * opt_dest) {
	const uint64_t n = M * N;
	float * v = f32_buffer(n, "create index identity host matrix");
	if (!v) return NULL;
	for (uint64_t i = 0; i < n; i++) v[i] = (float) i;
	return finish_from_f32(v, n, dt, opt_dest, "create index identity host matrix");
}

void * load_host_matrix_from_file(char * filepath, uint64_t M, uint64_t N, DataflowDatatype orig_dt, DataflowDatatype new_dt, void * opt_dest) {
	const uint64_t n = M * N;
	const size_t el = dataflow_sizeof_element(orig_dt);
	if (el == 0) {
		fprintf(stderr, "Error: load host matrix: no element size for dtype %s...\n", dataflow_datatype_as_string(orig_dt));
		return NULL;
	}
	FILE * fp = fopen(filepath, "rb");
	if (!fp) {
		fprintf(stderr, "Error: could not load matrix from file: %s\n", filepath);
		return NULL;
	}
	void * orig = malloc((n * el != 0) ? n * el : 1);
	if (!orig) {
		fprintf(stderr, "Error: load host matrix: could not allocate %lu elements...\n", (unsigned long) n);
		fclose(fp);
		return NULL;
	}
	const size_t got = fread(orig, el, n, fp);
	fclose(fp);
	if (got != n) {
		fprintf(stderr, "Error: couldn't read expected number of elements from matrix file: %s. (Expected %lu, read: %lu)\n",
				filepath, (unsigned long) n, (unsigned long) got);
		free(orig);
		return NULL;
	}
	void * dest = dest_or_alloc(opt_dest, n, new_dt, "load host matrix");
	if (!dest) {
		free(orig);
		return NULL;
	}
	int ret = 0;
	if (orig_dt == new_dt) memcpy(dest, orig, n * el);
	else ret = dataflow_convert_datatype(dest, orig, new_dt, orig_dt, (long) n, HOST_MATRIX_THREADS);
	free(orig);
	if (ret) {
		fprintf(stderr, "Error: load host matrix: conversion from %s to %s failed...\n", dataflow_datatype_as_string(orig_dt),
				dataflow_datatype_as_string(new_dt));
		if (!opt_dest) free(dest);
		return NULL;
	}
	return dest;
}

int save_host_matrix(char * filename, void * mat, uint64_t M, uint64_t N, DataflowDatatype dt) {
	const size_t el = dataflow_sizeof_element(dt);
	if (el == 0) {
		fprintf(stderr, "Error: save host matrix: no element size for dtype %s...\n", dataflow_datatype_as_string(dt));
		return -1;
	}
	FILE * fp = fopen(filename, "wb");
	if (!fp) {
		fprintf(stderr, "Error: could not open file with path: %s\n", filename);
		return -1;
	}
	const size_t n = (size_t) (M * N);
	const size_t wrote = fwrite(mat, el, n, fp);
	const int closed = fclose(fp);
	if (wrote != n || closed != 0) {
		fprintf(stderr, "Error: write failed, expected to write %lu els, but only wrote %lu...\n", (unsigned long) n, (unsigned long) wrote);
		return -1;
	}
	return 0;
}
