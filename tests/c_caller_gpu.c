/*
 * A C caller of the HIP backend, driving it the way the reference's C tests
 * drive their CUDA handle (src/dataflow_handle/nvidia/test/
 * test_cuda_dataflow_handle_raw_ops.c:215-235): a stack-allocated
 * Dataflow_Handle from include/dataflow_handle.h initialised with
 * init_hip_dataflow_handle(COMPUTE_HSA), the gfx950 code object and the
 * launch-configuration library registered with register_native_ops(),
 * device memory and transfers through the handle's vtable, then
 *   BASELINE config 1 (RMSNorm forward, fp32, 16 x 4096) and
 *   BASELINE config 2 (RMSNorm forward, bf16, 8192 x 4096)
 * each submitted once through submit_rms_norm() on stream 0 and once as a
 * hand-built raw Op through the handle's submit_op on stream 1, plus the
 * config-2 backward through submit_rms_norm_bwd(). The two forward
 * submissions run the same kernel on the same launch shape, so they must be
 * bit-equal; both are checked against the CPU oracle (oracle/liboracle.so,
 * test infrastructure) to the stated tolerances: fp32 outputs within 1e-5
 * relative, bf16 outputs within 1 bf16 ulp of the exact value, fp32 sums
 * within 1e-5 relative plus gamma * sum|terms| (gamma is the fp32 rounding
 * bound of the kernel's reduction depth, passed in by the Python test).
 *
 * usage: c_caller_gpu <code object> <config library> <gamma ws c1> <gamma ws c2> <gamma dW c2>
 * prints OK lines and exits 0, or prints the first mismatch and exits 1.
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

static Dataflow_Handle h;

static void * dev_put(const void * host, uint64_t bytes) {
	void * d = h.alloc_mem(&h, bytes);
	if (!d) return NULL;
	if (h.submit_inbound_transfer(&h, 0, d, (void *) host, bytes) || h.sync_stream(&h, 0)) return NULL;
	return d;
}

static int dev_get(void * host, void * d, uint64_t bytes) {
	return h.submit_outbound_transfer(&h, 0, host, d, bytes) || h.sync_stream(&h, 0);
}

/* o within tol of v (or both NaN) */
static int close_to(double o, double v, double tol) {
	return fabs(o - v) <= tol || (isnan(o) && isnan(v));
}

/* a stored output against its exact value: 1e-5 relative for fp32, one ulp
 * of the output type otherwise (values in the fp32 subnormal range may
 * flush to zero) */
static int out_ok(int dt, double o, double v, double floor_) {
	const double tol = (dt == ORACLE_FP32 ? 1e-5 * fabs(v) : oracle_ulp(v, dt)) + floor_;
	if (close_to(o, v, tol)) return 1;
	return fabs(v) < 0x1p-126 && fabs(o) <= 0x1p-126;
}

static long first_bad = -1;
static long count_bad(long i, int ok) {
	if (!ok && first_bad < 0) first_bad = i;
	return ok ? 0 : 1;
}

/* RMSNorm forward at one config: the op API on stream 0 and a raw Op on
 * stream 1, bit-equal to each other and within tolerance of the oracle */
static int run_fwd(DataflowDatatype dt, int n_rows, int n_cols, double gamma_ws, void ** keep_X, void ** keep_W,
				   void ** keep_rs, void ** host_X, void ** host_W) {
	float eps = 1e-5f;
	const long n = (long) n_rows * n_cols;
	const size_t es = dataflow_sizeof_element(dt);
	float * Xf = malloc(sizeof(float) * n), * Wf = malloc(sizeof(float) * n_cols);
	void * X = malloc(es * n), * W = malloc(es * n_cols);
	void * Y1 = malloc(es * n), * Y2 = malloc(es * n);
	float * ws1 = malloc(4 * n_rows), * rs1 = malloc(4 * n_rows), * ws2 = malloc(4 * n_rows), * rs2 = malloc(4 * n_rows);
	double * y_pre = malloc(sizeof(double) * n), * ws_e = malloc(8 * n_rows), * rs_e = malloc(8 * n_rows), * ws_abs = malloc(8 * n_rows);
	double * y = malloc(sizeof(double) * n);
	if (!Xf || !Wf || !X || !W || !Y1 || !Y2 || !ws1 || !rs1 || !ws2 || !rs2 || !y_pre || !ws_e || !rs_e || !ws_abs || !y) return -1;
	for (long i = 0; i < n; i++) Xf[i] = normal01();
	for (int j = 0; j < n_cols; j++) Wf[j] = 1.0f + 0.02f * normal01();
	if (dataflow_convert_datatype(X, Xf, dt, DATAFLOW_FP32, n, 1) || dataflow_convert_datatype(W, Wf, dt, DATAFLOW_FP32, n_cols, 1)) return -1;

	void * dX = dev_put(X, es * n), * dW = dev_put(W, es * n_cols);
	void * dY1 = h.alloc_mem(&h, es * n), * dY2 = h.alloc_mem(&h, es * n);
	void * dws1 = h.alloc_mem(&h, 4 * n_rows), * drs1 = h.alloc_mem(&h, 4 * n_rows);
	void * dws2 = h.alloc_mem(&h, 4 * n_rows), * drs2 = h.alloc_mem(&h, 4 * n_rows);
	if (!dX || !dW || !dY1 || !dY2 || !dws1 || !drs1 || !dws2 || !drs2) return -1;

	/* 1. the op API, stream 0 */
	if (submit_rms_norm(&h, 0, dt, n_rows, n_cols, eps, dW, dX, dY1, dws1, drs1)) {
		fprintf(stderr, "submit_rms_norm failed\n");
		return -1;
	}
	/* 2. the same op built by hand, through the vtable, stream 1 */
	Op op;
	memset(&op, 0, sizeof(op));
	set_native_rms_norm_skeleton(&op.op_skeleton, dt);
	void * w_arg = dW, * x_arg = dX, * y_arg = dY2, * ws_arg = dws2, * rs_arg = drs2;
	op.op_args[0] = &n_rows;
	op.op_args[1] = &n_cols;
	op.op_args[2] = &eps;
	op.op_args[3] = &w_arg;
	op.op_args[4] = &x_arg;
	op.op_args[5] = &y_arg;
	op.op_args[6] = &ws_arg;
	op.op_args[7] = &rs_arg;
	if (h.submit_op(&h, &op, 1) || h.sync_stream(&h, 1) || h.sync_stream(&h, 0)) {
		fprintf(stderr, "raw op submission failed\n");
		return -1;
	}
	if (dev_get(Y1, dY1, es * n) || dev_get(Y2, dY2, es * n) || dev_get(ws1, dws1, 4 * n_rows) || dev_get(rs1, drs1, 4 * n_rows) ||
		dev_get(ws2, dws2, 4 * n_rows) || dev_get(rs2, drs2, 4 * n_rows)) return -1;

	if (oracle_rms_norm(dt, n_rows, n_cols, eps, W, X, y_pre, ws_e, rs_e, ws_abs)) return -1;
	oracle_load(dt, Y1, n, y);
	long bad = 0;
	first_bad = -1;
	if (memcmp(Y1, Y2, es * n) || memcmp(ws1, ws2, 4 * n_rows) || memcmp(rs1, rs2, 4 * n_rows)) {
		fprintf(stderr, "dtype %d: submit_rms_norm and the raw Op differ\n", (int) dt);
		bad++;
	}
	for (long i = 0; i < n; i++) bad += count_bad(i, out_ok(dt, y[i], y_pre[i], 0.0));
	for (int r = 0; r < n_rows; r++) {
		bad += count_bad(n + r, close_to(rs1[r], rs_e[r], 1e-5 * fabs(rs_e[r])));
		bad += count_bad(2 * n + r, close_to(ws1[r], ws_e[r], 1e-5 * fabs(ws_e[r]) + gamma_ws * ws_abs[r]));
	}
	if (bad) {
		fprintf(stderr, "dtype %d %d x %d forward: %ld values out of tolerance (first at %ld)\n", (int) dt, n_rows, n_cols, bad, first_bad);
		return -1;
	}
	printf("OK forward dtype %d %d x %d: op API and raw Op bit-equal, within tolerance of the oracle\n", (int) dt, n_rows, n_cols);
	h.free_mem(&h, dY1); h.free_mem(&h, dY2); h.free_mem(&h, dws1); h.free_mem(&h, dws2); h.free_mem(&h, drs2);
	*keep_X = dX; *keep_W = dW; *keep_rs = drs1; *host_X = X; *host_W = W;
	free(Xf); free(Wf); free(Y1); free(Y2); free(ws1); free(rs1); free(ws2); free(rs2);
	free(y_pre); free(ws_e); free(rs_e); free(ws_abs); free(y);
	return 0;
}

int main(int argc, char ** argv) {
	if (argc < 6) {
		fprintf(stderr, "usage: %s <code object> <config library> <gamma ws c1> <gamma ws c2> <gamma dW c2>\n", argv[0]);
		return 2;
	}
	const double g_ws1 = atof(argv[3]), g_ws2 = atof(argv[4]), g_dw2 = atof(argv[5]);
	if (init_hip_dataflow_handle(&h, COMPUTE_HSA, 0, 0, 0, 2, NULL, NULL)) {
		fprintf(stderr, "init_hip_dataflow_handle failed\n");
		return 1;
	}
	const int n_registered = register_native_ops(&h, argv[1], argv[2]);
	if (n_registered <= 0) {
		fprintf(stderr, "register_native_ops failed (%d)\n", n_registered);
		return 1;
	}
	printf("OK registered %d\n", n_registered);

	void * dX1, * dW1, * drs1, * X1, * W1;
	if (run_fwd(DATAFLOW_FP32, 16, 4096, g_ws1, &dX1, &dW1, &drs1, &X1, &W1)) return 1;
	void * dX, * dW, * drs, * X, * W;
	const int n_rows = 8192, n_cols = 4096;
	if (run_fwd(DATAFLOW_BF16, n_rows, n_cols, g_ws2, &dX, &dW, &drs, &X, &W)) return 1;

	/* config 2 backward: the exact-gradient op, dX += and dW (fp32) += */
	const long n = (long) n_rows * n_cols;
	float * dYf = malloc(4 * n), * rs = malloc(4 * n_rows), * dWacc = calloc(n_cols, 4);
	uint16_t * dY = malloc(2 * n), * dXh = calloc(n, 2);
	double * dx_pre = malloc(8 * n), * dx_floor = malloc(8 * n), * dw_pre = malloc(8 * n_cols), * dw_abs = malloc(8 * n_cols);
	double * dx = malloc(8 * n);
	if (!dYf || !rs || !dWacc || !dY || !dXh || !dx_pre || !dx_floor || !dw_pre || !dw_abs || !dx) return 1;
	for (long i = 0; i < n; i++) dYf[i] = normal01();
	if (dataflow_convert_datatype(dY, dYf, DATAFLOW_BF16, DATAFLOW_FP32, n, 1)) return 1;
	void * ddY = dev_put(dY, 2 * n), * ddX = dev_put(dXh, 2 * n), * ddW = dev_put(dWacc, 4 * n_cols);
	if (!ddY || !ddX || !ddW || dev_get(rs, drs, 4 * n_rows)) return 1;
	if (submit_rms_norm_bwd(&h, 0, DATAFLOW_BF16, DATAFLOW_BF16, n_rows, n_cols, 1e-5f, drs, dW, dX, ddY, ddX, ddW) ||
		h.sync_stream(&h, 0)) {
		fprintf(stderr, "submit_rms_norm_bwd failed\n");
		return 1;
	}
	if (dev_get(dXh, ddX, 2 * n) || dev_get(dWacc, ddW, 4 * n_cols)) return 1;
	uint16_t * dX_in = calloc(n, 2);
	float * dW_in = calloc(n_cols, 4);
	if (!dX_in || !dW_in) return 1;
	if (oracle_rms_norm_bwd(ORACLE_BF16, n_rows, n_cols, rs, W, X, dY, dX_in, dW_in, dx_pre, dx_floor, dw_pre, dw_abs)) return 1;
	oracle_load(ORACLE_BF16, dXh, n, dx);
	long bad = 0;
	first_bad = -1;
	for (long i = 0; i < n; i++) bad += count_bad(i, out_ok(ORACLE_BF16, dx[i], dx_pre[i], dx_floor[i]));
	for (int j = 0; j < n_cols; j++) bad += count_bad(n + j, close_to(dWacc[j], dw_pre[j], 1e-5 * fabs(dw_pre[j]) + g_dw2 * dw_abs[j]));
	if (bad) {
		fprintf(stderr, "bf16 8192 x 4096 backward: %ld values out of tolerance (first at %ld)\n", bad, first_bad);
		return 1;
	}
	printf("OK backward bf16 %d x %d: dX and dW within tolerance of the oracle\n", n_rows, n_cols);

	/* an op no backend registered is refused with -1 */
	Op unknown;
	memset(&unknown, 0, sizeof(unknown));
	set_native_rms_norm_skeleton(&unknown.op_skeleton, DATAFLOW_UINT8);
	if (h.submit_op(&h, &unknown, 0) != -1) {
		fprintf(stderr, "an unregistered fingerprint was accepted\n");
		return 1;
	}
	h.free_mem(&h, ddY); h.free_mem(&h, ddX); h.free_mem(&h, ddW);
	h.free_mem(&h, dX); h.free_mem(&h, dW); h.free_mem(&h, drs);
	h.free_mem(&h, dX1); h.free_mem(&h, dW1); h.free_mem(&h, drs1);
	free(X1); free(W1); free(X); free(W); free(dYf); free(rs); free(dWacc); free(dY); free(dXh);
	free(dx_pre); free(dx_floor); free(dw_pre); free(dw_abs); free(dx); free(dX_in); free(dW_in);
	if (destroy_dataflow_handle(&h)) {
		fprintf(stderr, "destroy_dataflow_handle failed\n");
		return 1;
	}
	printf("OK done\n");
	return 0;
}
