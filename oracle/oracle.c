/*
 * CPU oracle for the native op path — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Each function restates one reference kernel (file:line cited) in fp64 with
 * the reference's intermediate roundings made explicit. fast-math intrinsics
 * of the reference (expf, sinf, cosf, powf, rsqrtf, division) are replaced by
 * accurate libm results; the GPU kernels are judged against these values.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define U32 (1.0 / 16777216.0)   /* fp32 unit roundoff, 2^-24 */

int oracle_num_threads(void) {
#ifdef _OPENMP
	return omp_get_max_threads();
#else
	return 1;
#endif
}

/* ---------------- formats ---------------- */

/* mantissa bits (implicit bit included), minimum normal exponent and
 * largest finite value. fp8: the OCP 8-bit formats (OCP 8-bit Floating Point
 * Specification, OFP8, rev. 1.0): E4M3 (bias 7, no infinities, S.1111.111 is
 * NaN, max 448) and E5M2 (bias 15, IEEE-style infinities and NaNs, max 57344) */
static int fmt(int dt, int * mant, int * emin, double * maxf) {
	switch (dt) {
		case ORACLE_FP32: *mant = 24; *emin = -126; *maxf = ldexp(2.0 - ldexp(1.0, -23), 127); return 0;
		case ORACLE_FP16: *mant = 11; *emin = -14;  *maxf = 65504.0; return 0;
		case ORACLE_BF16: *mant = 8;  *emin = -126; *maxf = ldexp(2.0 - ldexp(1.0, -7), 127); return 0;
		case ORACLE_FP8E4M3: *mant = 4; *emin = -6; *maxf = 448.0; return 0;
		case ORACLE_FP8E5M2: *mant = 3; *emin = -14; *maxf = 57344.0; return 0;
		default: return -1;
	}
}

static int is_fp8(int dt) { return dt == ORACLE_FP8E4M3 || dt == ORACLE_FP8E5M2; }

/* round-to-nearest-even of v into the format, subnormals included. Overflow
 * gives infinity, except for the fp8 formats, whose conversions saturate to
 * the largest finite value (infinite inputs too): the reference converts to
 * fp8 through the __nv_fp8_e4m3 / __nv_fp8_e5m2 constructors from float, which
 * saturate to finite (the CUDA fp8 types' documented __NV_SATFINITE mode). */
double oracle_round(double v, int dt) {
	int mant, emin;
	double maxf;
	if (fmt(dt, &mant, &emin, &maxf) || v == 0.0 || isnan(v)) return v;
	if (isinf(v)) return is_fp8(dt) ? copysign(maxf, v) : v;
	int e;
	frexp(v, &e);                      /* |v| in [2^(e-1), 2^e) */
	int lead = e - 1;
	if (lead < emin) lead = emin;
	const int q = lead - (mant - 1);   /* quantum exponent */
	double r = ldexp(nearbyint(ldexp(v, -q)), q);   /* default mode: ties to even */
	if (fabs(r) > maxf) r = is_fp8(dt) ? copysign(maxf, v) : copysign(INFINITY, v);
	return r;
}

/* value of an fp8 code */
static double fp8_decode(int dt, uint8_t b) {
	const int s = b >> 7;
	double v;
	if (dt == ORACLE_FP8E4M3) {
		const int e = (b >> 3) & 15, m = b & 7;
		if (e == 15 && m == 7) return NAN;
		v = (e == 0) ? ldexp((double) m, -9) : ldexp((double) (8 + m), e - 10);
	}
	else {
		const int e = (b >> 2) & 31, m = b & 3;
		if (e == 31) return m ? NAN : (s ? -INFINITY : INFINITY);
		v = (e == 0) ? ldexp((double) m, -16) : ldexp((double) (4 + m), e - 17);
	}
	return s ? -v : v;
}

/* code of a value already representable in the fp8 format (NaN -> 0x7f) */
static uint8_t fp8_encode_exact(int dt, double r) {
	if (isnan(r)) return 0x7f;
	const uint8_t s = signbit(r) ? 0x80 : 0;
	const double a = fabs(r);
	if (dt == ORACLE_FP8E5M2 && isinf(r)) return (uint8_t) (s | 0x7c);
	const int mbits = (dt == ORACLE_FP8E4M3) ? 3 : 2;
	const int bias = (dt == ORACLE_FP8E4M3) ? 7 : 15;
	if (a < ldexp(1.0, 1 - bias)) return (uint8_t) (s | (uint8_t) ldexp(a, bias - 1 + mbits));   /* subnormal or zero */
	int e;
	const double f = frexp(a, &e);     /* a = f * 2^e, f in [0.5, 1) */
	const int m = (int) ldexp(f, mbits + 1) - (1 << mbits);
	return (uint8_t) (s | (uint8_t) ((e - 1 + bias) << mbits) | (uint8_t) m);
}

/* spacing of the format at |v| (the ulp of v's binade) */
double oracle_ulp(double v, int dt) {
	int mant, emin;
	double maxf;
	if (fmt(dt, &mant, &emin, &maxf)) return NAN;
	int e;
	if (v == 0.0 || !isfinite(v)) return ldexp(1.0, emin - (mant - 1));
	frexp(v, &e);
	int lead = e - 1;
	if (lead < emin) lead = emin;
	return ldexp(1.0, lead - (mant - 1));
}

static double load1(int dt, const void * p, long i) {
	switch (dt) {
		case ORACLE_FP32: return (double) ((const float *) p)[i];
		case ORACLE_BF16: {
			uint32_t w = ((uint32_t) ((const uint16_t *) p)[i]) << 16;
			float f;
			memcpy(&f, &w, 4);
			return (double) f;
		}
		case ORACLE_FP16: {
			const uint16_t h = ((const uint16_t *) p)[i];
			const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
			double v;
			if (e == 0) v = ldexp((double) m, -24);
			else if (e == 31) v = m ? NAN : INFINITY;
			else v = ldexp((double) (m + 1024), e - 25);
			return s ? -v : v;
		}
		case ORACLE_FP8E4M3:
		case ORACLE_FP8E5M2:
			return fp8_decode(dt, ((const uint8_t *) p)[i]);
		default: return NAN;
	}
}

static void store1(int dt, void * p, long i, double v) {
	const double r = oracle_round(v, dt);
	switch (dt) {
		case ORACLE_FP32: ((float *) p)[i] = (float) r; break;
		case ORACLE_BF16: {
			uint16_t out;
			if (isnan(r)) out = 0x7fc0;
			else {
				float f = (float) r;   /* exact: r is representable in bf16 */
				uint32_t w;
				memcpy(&w, &f, 4);
				out = (uint16_t) (w >> 16);
			}
			((uint16_t *) p)[i] = out;
			break;
		}
		case ORACLE_FP16: {
			uint16_t out;
			if (isnan(r)) out = 0x7e00;
			else if (isinf(r)) out = r > 0 ? 0x7c00 : 0xfc00;
			else {
				const uint16_t s = signbit(r) ? 0x8000 : 0;
				const double a = fabs(r);
				if (a < ldexp(1.0, -14)) out = (uint16_t) (s | (uint16_t) ldexp(a, 24));
				else {
					int e;
					const double f = frexp(a, &e);   /* a = f * 2^e, f in [0.5, 1) */
					const int m = (int) ldexp(f, 11) - 1024;
					out = (uint16_t) (s | (uint16_t) ((e + 14) << 10) | (uint16_t) m);
				}
			}
			((uint16_t *) p)[i] = out;
			break;
		}
		case ORACLE_FP8E4M3:
		case ORACLE_FP8E5M2:
			((uint8_t *) p)[i] = fp8_encode_exact(dt, r);
			break;
		default: break;
	}
}

void oracle_load(int dt, const void * src, long n, double * dst) {
	for (long i = 0; i < n; i++) dst[i] = load1(dt, src, i);
}

void oracle_store(int dt, const double * src, long n, void * dst) {
	for (long i = 0; i < n; i++) store1(dt, dst, i, src[i]);
}

static int dt_ok(int dt) { return dt == ORACLE_FP32 || dt == ORACLE_FP16 || dt == ORACLE_BF16 || is_fp8(dt); }
/* storage types of the backward tensors (fp8 is a forward-only type) */
static int bwd_dt_ok(int dt) { return dt == ORACLE_FP32 || dt == ORACLE_FP16 || dt == ORACLE_BF16; }

/* ---------------- RMSNorm ---------------- */

/* reference: src/ops/nvidia/norm/rms_norm.cu:280-412 (bf16), :4-138 (fp32).
 * ws = sum x*w, rstd = 1/sqrt(sum x^2 / n + eps), y = (x * rstd) * w. */
int oracle_rms_norm(int dt, int n_rows, int n_cols, float eps, const void * W, const void * X,
					double * y_pre, double * ws, double * rstd, double * ws_abs) {
	if (!dt_ok(dt) || n_rows < 0 || n_cols <= 0) return -1;
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) {
		const long base = (long) r * n_cols;
		double ss = 0.0, sw = 0.0, sa = 0.0;
		for (int j = 0; j < n_cols; j++) {
			const double x = load1(dt, X, base + j), w = load1(dt, W, j);
			ss += x * x;
			sw += x * w;
			sa += fabs(x * w);
		}
		const double rs = 1.0 / sqrt(ss / (double) n_cols + (double) eps);
		if (ws) ws[r] = sw;
		if (ws_abs) ws_abs[r] = sa;
		if (rstd) rstd[r] = rs;
		if (y_pre) {
			for (int j = 0; j < n_cols; j++) y_pre[base + j] = (load1(dt, X, base + j) * rs) * load1(dt, W, j);
		}
	}
	return 0;
}

/* the fp8 forward kernels write sum_j x^2 per row where the others write
 * rstd (src/ops/nvidia/norm/rms_norm.cu:511,635) */
int oracle_rms_norm_sq_sums(int dt, int n_rows, int n_cols, const void * X, double * sq_sums) {
	if (!dt_ok(dt) || n_rows < 0 || n_cols <= 0) return -1;
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) {
		double ss = 0.0;
		for (int j = 0; j < n_cols; j++) {
			const double x = load1(dt, X, (long) r * n_cols + j);
			ss += x * x;
		}
		sq_sums[r] = ss;
	}
	return 0;
}

/* reference: src/ops/nvidia/norm/rms_norm_bwd_x.cu:175-256 (bf16), :4-86 (fp32),
 * :259-590 (fp8 W and X, fp16 / bf16 dY and dX):
 *   deriv = w*r - ((x*r^3)/n)*ws;  dX = rnd(dX + rnd(dY * rnd(deriv)))
 * The rounding of deriv is taken at deriv -/+ err_scale * (fp32 error bound of
 * deriv); the two chains bound any fp32 evaluation (err_scale 0: exact chain). */
static int rms_bwd_x_impl(int fdt, int dt, int n_rows, int n_cols, const float * ws, const float * rs, const void * W, const void * X,
							const void * dY, const void * dX_in, double * v_lo, double * v_hi, double err_scale) {
	if (!dt_ok(fdt) || !bwd_dt_ok(dt) || n_rows < 0 || n_cols <= 0) return -1;
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) {
		const long base = (long) r * n_cols;
		const double rr = rs[r], w_s = ws[r];
		const double r3 = rr * rr * rr;
		for (int j = 0; j < n_cols; j++) {
			const double w = load1(fdt, W, j), x = load1(fdt, X, base + j);
			const double a = w * rr, b = ((x * r3) / (double) n_cols) * w_s;
			const double deriv = a - b;
			const double err = err_scale * 8.0 * U32 * (fabs(a) + fabs(b));
			const double g = load1(dt, dY, base + j), d = load1(dt, dX_in, base + j);
			const double p_lo = oracle_round(g * oracle_round(deriv - err, dt), dt);
			const double p_hi = oracle_round(g * oracle_round(deriv + err, dt), dt);
			v_lo[base + j] = d + p_lo;
			if (v_hi) v_hi[base + j] = d + p_hi;
		}
	}
	return 0;
}

int oracle_rms_norm_bwd_x(int dt, int n_rows, int n_cols, const float * ws, const float * rs,
						const void * W, const void * X, const void * dY, const void * dX_in, double * v_lo, double * v_hi) {
	return rms_bwd_x_impl(dt, dt, n_rows, n_cols, ws, rs, W, X, dY, dX_in, v_lo, v_hi, 1.0);
}

/* W and X in fdt (fp8 allowed), dY and dX in dt */
int oracle_rms_norm_bwd_x2(int fdt, int dt, int n_rows, int n_cols, const float * ws, const float * rs,
						const void * W, const void * X, const void * dY, const void * dX_in, double * v_lo, double * v_hi) {
	return rms_bwd_x_impl(fdt, dt, n_rows, n_cols, ws, rs, W, X, dY, dX_in, v_lo, v_hi, 1.0);
}

/* reference: src/ops/nvidia/norm/rms_norm_bwd_w.cu:211-308 (bf16), :4-101 (fp32):
 * dW += sum_rows dY * x * rstd, summed here in fp64 (the reference's bf16
 * atomics have no defined order) */
static void dw_accumulate(int fdt, int dt, int n_rows, int n_cols, const float * rs, const void * X, const void * dY,
							double * dw_pre, double * dw_abs) {
	#pragma omp parallel for schedule(static)
	for (int j = 0; j < n_cols; j++) {
		double s = 0.0, a = 0.0;
		for (int r = 0; r < n_rows; r++) {
			const long i = (long) r * n_cols + j;
			const double t = load1(dt, dY, i) * load1(fdt, X, i) * (double) rs[r];
			s += t;
			a += fabs(t);
		}
		dw_pre[j] += s;
		if (dw_abs) dw_abs[j] += a;
	}
}

int oracle_rms_norm_bwd_w(int dt, int dt_w, int n_rows, int n_cols, const float * rs, const void * X, const void * dY,
						const void * dW_in, double * dw_pre, double * dw_abs) {
	return oracle_rms_norm_bwd_w2(dt, dt, dt_w, n_rows, n_cols, rs, X, dY, dW_in, dw_pre, dw_abs);
}

/* X in fdt (fp8 allowed), dY in dt, dW in dt_w (rms_norm_bwd_w.cu:310-700 for fp8 X) */
int oracle_rms_norm_bwd_w2(int fdt, int dt, int dt_w, int n_rows, int n_cols, const float * rs, const void * X, const void * dY,
						const void * dW_in, double * dw_pre, double * dw_abs) {
	if (!dt_ok(fdt) || !bwd_dt_ok(dt) || !bwd_dt_ok(dt_w) || n_rows < 0 || n_cols <= 0) return -1;
	for (int j = 0; j < n_cols; j++) {
		dw_pre[j] = load1(dt_w, dW_in, j);
		if (dw_abs) dw_abs[j] = fabs(dw_pre[j]);
	}
	dw_accumulate(fdt, dt, n_rows, n_cols, rs, X, dY, dw_pre, dw_abs);
	return 0;
}

/* Exact RMSNorm gradient (no reference kernel; the reference's harness
 * src/dataflow_handle/nvidia/test/check_rms.py:53-63 derives it with autograd):
 *   dX += r*(dY*w) - x * r^3/n * sum_j(dY*w*x);  dW += sum_rows dY*x*r */
int oracle_rms_norm_bwd(int dt, int n_rows, int n_cols, const float * rs, const void * W, const void * X, const void * dY,
						const void * dX_in, const float * dW_in, double * dx_pre, double * dx_floor, double * dw_pre, double * dw_abs) {
	if (!bwd_dt_ok(dt) || n_rows < 0 || n_cols <= 0) return -1;
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) {
		const long base = (long) r * n_cols;
		const double rr = rs[r];
		double dot = 0.0, dabs = 0.0;
		for (int j = 0; j < n_cols; j++) {
			const double t = load1(dt, dY, base + j) * load1(dt, W, j) * load1(dt, X, base + j);
			dot += t;
			dabs += fabs(t);
		}
		const double k = rr * rr * rr / (double) n_cols;
		const double coef = k * dot;
		for (int j = 0; j < n_cols; j++) {
			const double x = load1(dt, X, base + j);
			const double gw = load1(dt, dY, base + j) * load1(dt, W, j);
			const double d = load1(dt, dX_in, base + j);
			dx_pre[base + j] = d + (rr * gw - x * coef);
			if (dx_floor) dx_floor[base + j] = 8.0 * U32 * (fabs(d) + fabs(rr * gw) + fabs(x * coef)) + fabs(x) * k * 64.0 * U32 * dabs;
		}
	}
	for (int j = 0; j < n_cols; j++) {
		dw_pre[j] = (double) dW_in[j];
		if (dw_abs) dw_abs[j] = fabs(dw_pre[j]);
	}
	dw_accumulate(dt, dt, n_rows, n_cols, rs, X, dY, dw_pre, dw_abs);
	return 0;
}

/* ---------------- RoPE ---------------- */

/* reference: src/ops/nvidia/attention/rope.cu:123-180 (fwd), rope_bwd_x.cu:120-175 (bwd).
 * angle = (float) theta^(-(float)c / (float)head_dim) (fp32 result),
 * arg = (float) pos * angle (fp32 product), c/s = cos/sin(arg) as fp32,
 * fwd (e, o) -> (c e - s o, c o + s e); bwd -> (c e + s o, c o - s e). */
static void rope_row(int dt, int bwd, const void * X, long base, int width, int head_dim, const float * cs, const float * sn, double * out) {
	for (int p = 0; p < width / 2; p++) {
		const int c = (2 * p) % head_dim;
		const double cc = cs[c / 2], ss = sn[c / 2];
		const double e = load1(dt, X, base + 2 * p), o = load1(dt, X, base + 2 * p + 1);
		if (!bwd) {
			out[base + 2 * p] = cc * e - ss * o;
			out[base + 2 * p + 1] = cc * o + ss * e;
		}
		else {
			out[base + 2 * p] = cc * e + ss * o;
			out[base + 2 * p + 1] = cc * o - ss * e;
		}
	}
}

int oracle_rope(int dt, int bwd, uint64_t N, int model_dim, int head_dim, int num_kv_heads, int theta, const int * seq_positions,
				const void * X_q, const void * X_k, double * q_pre, double * k_pre) {
	if (!dt_ok(dt) || model_dim <= 0 || head_dim <= 0 || (head_dim & 1) || model_dim % head_dim || N % (uint64_t) model_dim) return -1;
	const long n_tokens = (long) (N / (uint64_t) model_dim);
	const int kv_dim = num_kv_heads * head_dim;
	const int half = head_dim / 2;
	float * angle = (float *) malloc(sizeof(float) * (size_t) half);
	if (!angle) return -1;
	for (int p = 0; p < half; p++) {
		const float expo = -((float) (2 * p) / (float) head_dim);
		angle[p] = (float) pow((double) (float) theta, (double) expo);
	}
	#pragma omp parallel
	{
		float * cs = (float *) malloc(sizeof(float) * (size_t) half);
		float * sn = (float *) malloc(sizeof(float) * (size_t) half);
		#pragma omp for schedule(static)
		for (long t = 0; t < n_tokens; t++) {
			const float fpos = (float) seq_positions[t];
			for (int p = 0; p < half; p++) {
				const float arg = fpos * angle[p];
				cs[p] = (float) cos((double) arg);
				sn[p] = (float) sin((double) arg);
			}
			rope_row(dt, bwd, X_q, t * (long) model_dim, model_dim, head_dim, cs, sn, q_pre);
			if (kv_dim > 0) rope_row(dt, bwd, X_k, t * (long) kv_dim, kv_dim, head_dim, cs, sn, k_pre);
		}
		free(cs);
		free(sn);
	}
	free(angle);
	return 0;
}

/* ---------------- SwiGLU ---------------- */

/* reference: src/ops/nvidia/activations/swiglu.cu:48-68: out = (g / (1 + exp(-g))) * u */
int oracle_swiglu(int dt, long n, const void * g, const void * u, double * out_pre) {
	if (!dt_ok(dt) || n < 0) return -1;
	#pragma omp parallel for schedule(static)
	for (long i = 0; i < n; i++) {
		const double gv = load1(dt, g, i);
		out_pre[i] = (gv / (1.0 + exp(-gv))) * load1(dt, u, i);
	}
	return 0;
}

/* reference: src/ops/nvidia/activations/swiglu_bwd_x.cu:56-80:
 *   e = exp(-g); dU = dO * g/(1+e); dG = dO * (u*(1+e+g*e)) / ((1+e)*(1+e)).
 * Where exp(-g) overflows even in fp64 (g < -709) the same function is
 * evaluated in its sigmoid form. dg_floor bounds the fp32 evaluation noise of
 * dG, whose factor (1 + g*(1-sigmoid(g))) crosses zero near g = -1.28. */
int oracle_swiglu_bwd(int dt, long n, const void * g, const void * u, const void * dO, double * dg_pre, double * dg_floor, double * du_pre) {
	return oracle_swiglu_bwd2(dt, dt, n, g, u, dO, dg_pre, dg_floor, du_pre);
}

/* g and u in fdt (fp8 allowed: swiglu_bwd_x.cu:82-187), dO in dt */
int oracle_swiglu_bwd2(int fdt, int dt, long n, const void * g, const void * u, const void * dO, double * dg_pre, double * dg_floor, double * du_pre) {
	if (!dt_ok(fdt) || !bwd_dt_ok(dt) || n < 0) return -1;
	#pragma omp parallel for schedule(static)
	for (long i = 0; i < n; i++) {
		const double gv = load1(fdt, g, i), uv = load1(fdt, u, i), d = load1(dt, dO, i);
		const double e = exp(-gv);
		double sig, dg;
		if (isfinite(e)) {
			sig = 1.0 / (1.0 + e);
			dg = d * ((uv * (1.0 + e + gv * e)) / ((1.0 + e) * (1.0 + e)));
		}
		else {
			sig = exp(gv) / (1.0 + exp(gv));
			dg = d * uv * sig * (1.0 + gv * (1.0 - sig));
		}
		du_pre[i] = d * (gv / (1.0 + e));
		dg_pre[i] = dg;
		if (dg_floor) dg_floor[i] = 8.0 * U32 * fabs(d * uv * sig) * (1.0 + fabs(gv) * (1.0 - sig));
	}
	return 0;
}

/* ---------------- softmax / cross-entropy ---------------- */

/* reference: src/ops/nvidia/loss/softmax.cu:273-407 (bf16), :3-140 (fp32),
 * :409-960 (fp8 inputs, fp16 / bf16 outputs):
 *   m = max x;  d = rnd((float) x - (float) m);  y = exp(d) / sum exp(d)
 * with rnd the rounding to the input type (the fp32 kernel uses the fp32
 * difference itself); fp8 inputs are converted to the output type first and
 * subtracted there, so `dt_diff` is the output type for them */
static void softmax_row(int dt_in, int dt_diff, const void * X, long base, int n_cols, double * y, double * m_out, double * sx_out) {
	double m = -INFINITY;
	for (int j = 0; j < n_cols; j++) {
		const double x = load1(dt_in, X, base + j);
		if (x > m) m = x;
	}
	double s = 0.0, sx = 0.0;
	for (int j = 0; j < n_cols; j++) {
		const float x = (float) load1(dt_in, X, base + j);
		const float diff = x - (float) m;
		const double d = oracle_round((double) diff, dt_diff);
		const double e = exp(d);
		y[base + j] = e;
		s += e;
		sx += exp((double) x - m);
	}
	for (int j = 0; j < n_cols; j++) y[base + j] /= s;
	if (m_out) *m_out = m;
	if (sx_out) *sx_out = sx;
}

int oracle_softmax(int dt_in, int dt_out, int n_rows, int n_cols, const void * X, double * y_pre) {
	if (!dt_ok(dt_in) || !bwd_dt_ok(dt_out) || n_rows < 0 || n_cols <= 0) return -1;
	const int dt_diff = is_fp8(dt_in) ? dt_out : dt_in;
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) softmax_row(dt_in, dt_diff, X, (long) r * n_cols, n_cols, y_pre, NULL, NULL);
	return 0;
}

/* reference: src/ops/nvidia/loss/cross_entropy.cu:33-44, intended semantics
 * (the kernel's row index i / n_cols is always 0, so it only ever touches
 * row 0): P[r, label_r] = rnd((float) P - 1) in place; labels >= n_cols skip. */
int oracle_cross_entropy_loss(int dt, int n_rows, int n_cols, void * P, const uint32_t * labels) {
	if (!bwd_dt_ok(dt) || n_rows < 0 || n_cols <= 0) return -1;
	for (int r = 0; r < n_rows; r++) {
		if (labels[r] >= (uint32_t) n_cols) continue;
		const long i = (long) r * n_cols + labels[r];
		const float v = (float) load1(dt, P, i) - 1.0f;
		store1(dt, P, i, (double) v);
	}
	return 0;
}

/* Fused softmax + cross-entropy (no single reference kernel: softmax.cu then
 * cross_entropy.cu as the model chains them, dataflow_transformer.c:359-392):
 * y = softmax with the reference's roundings, then y[label] = rnd(y) - 1;
 * loss_r = log(sum_j exp(x_j - m)) + m - x_label, mean = sum loss / n_rows.
 * y_lo/y_hi differ only at the label, where rnd(y) is taken at
 * y (1 -/+ 1e-5) to cover the fp32 error of any evaluation of y. */
static int softmax_xent_impl(int dt, int n_rows, int n_cols, const void * X, const uint32_t * labels,
								double * y_lo, double * y_hi, double * loss, double * mean_loss, double slack) {
	if (!bwd_dt_ok(dt) || n_rows < 0 || n_cols <= 0) return -1;
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) {
		const long base = (long) r * n_cols;
		double m, sx;
		softmax_row(dt, dt, X, base, n_cols, y_lo, &m, &sx);
		if (y_hi) memcpy(y_hi + base, y_lo + base, sizeof(double) * (size_t) n_cols);
		const uint32_t lab = labels[r];
		if (lab < (uint32_t) n_cols) {
			const double p = y_lo[base + lab];
			const double lo = oracle_round(p * (1.0 - slack), dt) - 1.0;
			const double hi = oracle_round(p * (1.0 + slack), dt) - 1.0;
			y_lo[base + lab] = lo;
			if (y_hi) y_hi[base + lab] = hi;
			if (loss) {
				/* -log p_label = log1p(others / exp(x_l - m)), others = the sum
				 * of exp(x_j - m) over the other columns: log(sx) + m - x_l
				 * loses a confident row's small loss in fp64 too (below
				 * ~1e-12); the same form as the kernels, evaluated in fp64 */
				const double xl = load1(dt, X, base + lab), gap = m - xl;
				double others = 0.0;
				for (int j = 0; j < n_cols; j++)
					if ((uint32_t) j != lab) others += exp(load1(dt, X, base + j) - m);
				loss[r] = (gap < 16.0) ? log1p(others / exp(-gap)) : log(others + exp(-gap)) + gap;
			}
		}
		else if (loss) {
			loss[r] = NAN;
		}
	}
	if (mean_loss && loss) {
		double s = 0.0;
		for (int r = 0; r < n_rows; r++) s += loss[r];
		*mean_loss = (n_rows > 0) ? s / (double) n_rows : NAN;
	}
	return 0;
}

int oracle_softmax_cross_entropy(int dt, int n_rows, int n_cols, const void * X, const uint32_t * labels,
								double * y_lo, double * y_hi, double * loss, double * mean_loss) {
	return softmax_xent_impl(dt, n_rows, n_cols, X, labels, y_lo, y_hi, loss, mean_loss, 1e-5);
}

/* exact chains (no evaluation slack), for the CPU dispatch adapters */
int oracle_rms_norm_bwd_x_exact(int dt, int n_rows, int n_cols, const float * ws, const float * rs,
						const void * W, const void * X, const void * dY, const void * dX_in, double * v) {
	return rms_bwd_x_impl(dt, dt, n_rows, n_cols, ws, rs, W, X, dY, dX_in, v, NULL, 0.0);
}

int oracle_rms_norm_bwd_x2_exact(int fdt, int dt, int n_rows, int n_cols, const float * ws, const float * rs,
						const void * W, const void * X, const void * dY, const void * dX_in, double * v) {
	return rms_bwd_x_impl(fdt, dt, n_rows, n_cols, ws, rs, W, X, dY, dX_in, v, NULL, 0.0);
}

int oracle_softmax_cross_entropy_exact(int dt, int n_rows, int n_cols, const void * X, const uint32_t * labels,
								double * y, double * loss, double * mean_loss) {
	return softmax_xent_impl(dt, n_rows, n_cols, X, labels, y, NULL, loss, mean_loss, 0.0);
}

/* ---------------- embedding / copy_to_seq_context ---------------- */

/* reference: src/ops/nvidia/preprocess/embedding.cu:3-119, with the row
 * offset taken in elements (the reference's typed-pointer index multiplies
 * it by the element size once more, :14-20) */
int oracle_embedding(int elem_bytes, int num_tokens, int embed_dim, const uint32_t * ids, const void * table, long vocab, void * out) {
	if ((elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) || num_tokens < 0 || embed_dim < 0) return -1;
	const size_t row = (size_t) embed_dim * (size_t) elem_bytes;
	for (int t = 0; t < num_tokens; t++) {
		if (vocab >= 0 && (long) ids[t] >= vocab) return -1;
		memcpy((char *) out + (size_t) t * row, (const char *) table + (size_t) ids[t] * row, row);
	}
	return 0;
}

/* reference: src/ops/nvidia/attention/copy_to_seq_context.cu:3-100 */
int oracle_copy_to_seq_context(int elem_bytes, uint64_t N, int kv_dim, const void * keys, const void * values,
					const int * seq_positions, const uint64_t * ctx_ptrs, const int * ctx_sizes) {
	if ((elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4) || kv_dim <= 0 || N % (uint64_t) kv_dim) return -1;
	const size_t row = (size_t) kv_dim * (size_t) elem_bytes;
	const long n_tokens = (long) (N / (uint64_t) kv_dim);
	for (long t = 0; t < n_tokens; t++) {
		char * ctx = (char *) (uintptr_t) ctx_ptrs[t];
		const size_t p = (size_t) seq_positions[t], S = (size_t) ctx_sizes[t];
		memcpy(ctx + p * row, (const char *) keys + (size_t) t * row, row);
		memcpy(ctx + (S + p) * row, (const char *) values + (size_t) t * row, row);
	}
	return 0;
}
