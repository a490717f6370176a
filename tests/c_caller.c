/*
 * A C caller of the library's boundary, written the way the reference's C
 * tests use theirs (src/dataflow_handle/nvidia/test/test_cuda_dataflow_handle_raw_ops.c:215-235):
 * a stack-allocated Dataflow_Handle from include/dataflow_handle.h, native
 * ops registered with register_native_ops(), BASELINE config 1 (RMSNorm
 * forward, fp32, 16 x 4096) submitted once through submit_rms_norm() and
 * once as a hand-built raw Op through the handle's submit_op vtable entry.
 * It runs on the CPU test backend (COMPUTE_CPU, oracle/liboracle.so), so it
 * needs no GPU. Both results must be bit-equal and equal the oracle's value
 * rounded to fp32.
 *
 * It also prints the layout of the public structs as C sees them (LAYOUT
 * lines), which the Python test compares with the ctypes mirrors in
 * dataflow_lib_amd/api.py, so a header and its mirror cannot drift apart.
 *
 * usage: c_caller <path of oracle/liboracle.so>; prints OK and exits 0.
 */
#include <math.h>
#include <stddef.h>

#include "dataflow.h"
#include "dataflow_handle.h"
#include "dataflow_ops.h"
#include "hip_dataflow_handle.h"
#include "ops.h"
#include "oracle.h"
#include "set_native_op_skeletons.h"

/* the CPU test backend's init (oracle/cpu_backend.c) */
int init_cpu_dataflow_handle(Dataflow_Handle * h, int num_streams);
int destroy_cpu_dataflow_handle(Dataflow_Handle * h);

/* seeded N(0, 1) samples: splitmix64 uniforms through Box-Muller */
static uint64_t sm_state = 20261202u;
static double uniform01(void) {
	uint64_t z = (sm_state += 0x9e3779b97f4a7c15ull);
	z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
	z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
	z ^= z >> 31;
	return ((double) (z >> 11) + 0.5) / 9007199254740992.0;
}
static float normal01(void) {
	const double u = uniform01(), v = uniform01();
	return (float) (sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v));
}

#define LAYOUT(name, value) printf("LAYOUT %s %ld\n", name, (long) (value))

int main(int argc, char ** argv) {
	if (argc < 2) {
		fprintf(stderr, "usage: %s <oracle library>\n", argv[0]);
		return 2;
	}
	LAYOUT("sizeof_Dataflow_Handle", sizeof(Dataflow_Handle));
	LAYOUT("offset_Dataflow_Handle_stream_prios", offsetof(Dataflow_Handle, stream_prios));
	LAYOUT("offset_Dataflow_Handle_native_function_libs", offsetof(Dataflow_Handle, native_function_libs));
	LAYOUT("offset_Dataflow_Handle_op_table", offsetof(Dataflow_Handle, op_table));
	LAYOUT("offset_Dataflow_Handle_submit_op", offsetof(Dataflow_Handle, submit_op));
	LAYOUT("offset_Dataflow_Handle_submit_peer_transfer", offsetof(Dataflow_Handle, submit_peer_transfer));
	LAYOUT("sizeof_Op", sizeof(Op));
	LAYOUT("sizeof_Op_Skeleton_Header", sizeof(Op_Skeleton_Header));
	LAYOUT("offset_Op_op_args", offsetof(Op, op_args));
	LAYOUT("sizeof_Table", sizeof(Table));
	LAYOUT("sizeof_Hip_Device_Info", sizeof(Hip_Device_Info));
	LAYOUT("offset_Hip_Device_Info_cu_count", offsetof(Hip_Device_Info, cu_count));
	LAYOUT("offset_Hip_Device_Info_arch_name", offsetof(Hip_Device_Info, arch_name));

	Dataflow_Handle h;
	if (init_cpu_dataflow_handle(&h, 2)) {
		fprintf(stderr, "init of the CPU test backend failed\n");
		return 1;
	}
	const int n_registered = register_native_ops(&h, argv[1], "");
	if (n_registered <= 0) {
		fprintf(stderr, "register_native_ops failed (%d)\n", n_registered);
		return 1;
	}

	/* BASELINE config 1: X [16 x 4096] ~ N(0, 1), W = 1 + N(0, 0.02), eps = 1e-5 */
	int n_rows = 16, n_cols = 4096;
	float eps = 1e-5f;
	const long n = (long) n_rows * n_cols;
	float * X = malloc(sizeof(float) * n), * W = malloc(sizeof(float) * n_cols);
	float * Y1 = malloc(sizeof(float) * n), * Y2 = malloc(sizeof(float) * n);
	float ws1[16], rs1[16], ws2[16], rs2[16];
	double * y_pre = malloc(sizeof(double) * n);
	double ws_e[16], rs_e[16], ws_abs[16];
	if (!X || !W || !Y1 || !Y2 || !y_pre) return 1;
	for (long i = 0; i < n; i++) X[i] = normal01();
	for (int j = 0; j < n_cols; j++) W[j] = 1.0f + 0.02f * normal01();

	/* 1. the op API */
	if (submit_rms_norm(&h, 0, DATAFLOW_FP32, n_rows, n_cols, eps, W, X, Y1, ws1, rs1)) {
		fprintf(stderr, "submit_rms_norm failed\n");
		return 1;
	}

	/* 2. the same op built by hand and submitted through the vtable */
	Op op;
	memset(&op, 0, sizeof(op));
	set_native_rms_norm_skeleton(&op.op_skeleton, DATAFLOW_FP32);
	void * w_arg = W, * x_arg = X, * y_arg = Y2, * ws_arg = ws2, * rs_arg = rs2;
	op.op_args[0] = &n_rows;
	op.op_args[1] = &n_cols;
	op.op_args[2] = &eps;
	op.op_args[3] = &w_arg;
	op.op_args[4] = &x_arg;
	op.op_args[5] = &y_arg;
	op.op_args[6] = &ws_arg;
	op.op_args[7] = &rs_arg;
	if (h.submit_op(&h, &op, 0) || h.sync_stream(&h, 0)) {
		fprintf(stderr, "raw op submission failed\n");
		return 1;
	}

	/* 3. an op no backend registered is refused with -1 */
	Op unknown;
	memset(&unknown, 0, sizeof(unknown));
	set_native_rms_norm_skeleton(&unknown.op_skeleton, DATAFLOW_UINT8);
	if (h.submit_op(&h, &unknown, 0) != -1) {
		fprintf(stderr, "an unregistered fingerprint was accepted\n");
		return 1;
	}

	if (oracle_rms_norm(ORACLE_FP32, n_rows, n_cols, eps, W, X, y_pre, ws_e, rs_e, ws_abs)) return 1;
	long bad = 0;
	for (long i = 0; i < n; i++) {
		if (memcmp(&Y1[i], &Y2[i], sizeof(float)) != 0 || Y1[i] != (float) y_pre[i]) bad++;
	}
	for (int r = 0; r < n_rows; r++) {
		if (ws1[r] != ws2[r] || rs1[r] != rs2[r] || rs1[r] != (float) rs_e[r] || ws1[r] != (float) ws_e[r]) bad++;
	}
	destroy_cpu_dataflow_handle(&h);
	free(X); free(W); free(Y1); free(Y2); free(y_pre);
	if (bad) {
		fprintf(stderr, "%ld values differ between the op API, the raw op and the oracle\n", bad);
		return 1;
	}
	printf("OK registered %d, config 1 equal through submit_rms_norm and a raw Op\n", n_registered);
	return 0;
}
