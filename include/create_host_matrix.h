/*
 * Host matrices and the raw .dat format (reference:
 * src/dataflow_handle/nvidia/test/create_host_matrix.{h,c}).
 *
 * A .dat file is the M x N row-major elements of one DataflowDatatype, with no
 * header; loading converts to another floating type (fp32/fp16/bf16, RNE)
 * through dataflow_convert_datatype. Every create_* returns opt_dest when it
 * is given, else a malloc'd buffer the caller frees; NULL on failure.
 *
 * Differences from the reference: create_identity_host_matrix zeroes the
 * off-diagonal elements (the reference left them uninitialised), and
 * create_rand_host_matrix draws by default from a portable generator
 * (splitmix64 and fp64 Box-Muller) seeded with 42 and reseedable through
 * host_matrix_seed, so matrices are reproducible across hosts.
 * host_matrix_set_generator(HOST_MATRIX_RAND_LIBC) switches to the
 * reference's own generator (Marsaglia's polar method on the C library's
 * rand(), seeded with srand()), which reproduces the reference harnesses'
 * matrices bit for bit on the same C library. Generator state is
 * process-wide and not thread-safe, like rand().
 */
#ifndef CREATE_HOST_MATRIX_H
#define CREATE_HOST_MATRIX_H

#include "dataflow.h"

#ifdef __cplusplus
extern "C" {
#endif

/* create_host_matrix.h:7 */
void * create_zero_host_matrix(uint64_t M, uint64_t N, DataflowDatatype dt, void * opt_dest);
/* create_host_matrix.h:8; N(mean, std) per element, rounded to dt */
void * create_rand_host_matrix(uint64_t M, uint64_t N, float mean, float std, DataflowDatatype dt, void * opt_dest);
/* create_host_matrix.h:9 */
void * create_identity_host_matrix(uint64_t N, DataflowDatatype dt, void * opt_dest);
/* create_host_matrix.h:10; element i = (float) i rounded to dt */
void * create_index_identity_host_matrix(uint64_t M, uint64_t N, DataflowDatatype dt, void * opt_dest);
/* create_host_matrix.h:12; reads M*N elements of orig_dt, converts to new_dt */
void * load_host_matrix_from_file(char * filepath, uint64_t M, uint64_t N, DataflowDatatype orig_dt, DataflowDatatype new_dt, void * opt_dest);
/* create_host_matrix.h:14; 0 or -1 */
int save_host_matrix(char * filename, void * mat, uint64_t M, uint64_t N, DataflowDatatype dt);

/* No counterpart in the reference: reseed create_rand_host_matrix's portable generator. */
void host_matrix_seed(uint64_t seed);

/* No counterpart in the reference: choose create_rand_host_matrix's generator
 * (0, or -1 for an unknown value). */
#define HOST_MATRIX_RAND_PORTABLE 0
#define HOST_MATRIX_RAND_LIBC 1
int host_matrix_set_generator(int generator);

#ifdef __cplusplus
}
#endif

#endif
