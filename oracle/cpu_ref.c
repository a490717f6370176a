/*
 * CPU baseline of the native op path (bench.py's cpu_baseline leg only; not a
 * checker and not part of the product). The same math as the GPU ops on the
 * host's cores: bf16 storage, fp32 element arithmetic, fp64 row (and column)
 * reductions, OpenMP over rows, loops written for the compiler to vectorise
 * (AVX-512 with the build's -march=x86-64-v4). Semantics follow the
 * reference kernels:
 *   rms_norm            src/ops/nvidia/norm/rms_norm.cu:280-412
 *   rms_norm_bwd        the exact-gradient fused backward the GPU path times
 *                       (dX and dW in one pass; dW as rms_norm_bwd_w.cu:4-101)
 *   rope / rope_bwd_x   src/ops/nvidia/attention/rope.cu:123-180, rope_bwd_x.cu:120-175
 *   swiglu / bwd        src/ops/nvidia/activations/swiglu.cu:48-68, swiglu_bwd_x.cu:4-80
 *   softmax + xent      src/ops/nvidia/loss/softmax.cu:273-407, cross_entropy.cu:4-44
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf(uint16_t h) {
	union { uint32_t u; float f; } v;
	v.u = (uint32_t) h << 16;
	return v.f;
}

/* fp32 -> bf16, round to nearest even (NaN kept quiet) */
static inline uint16_t to_bf(float f) {
	union { uint32_t u; float f; } v;
	v.f = f;
	if ((v.u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((v.u >> 16) | 0x40u);
	return (uint16_t) ((v.u + 0x7fffu + ((v.u >> 16) & 1u)) >> 16);
}

int cpu_ref_threads(void) { return omp_get_max_threads(); }

void cpu_ref_rms_norm_bf16(int n_rows, int n_cols, float eps, const uint16_t * W, const uint16_t * X, uint16_t * Y,
						   float * weighted_sums, float * rstd) {
	#pragma omp parallel for schedule(static)
	for (int r = 0; r < n_rows; r++) {
		const uint16_t * x = X + (long) r * n_cols;
		uint16_t * y = Y + (long) r * n_cols;
		double ss = 0.0, ws = 0.0;
		#pragma omp simd reduction(+ : ss, ws)
		for (int j = 0; j < n_cols; j++) {
			const float xv = bf(x[j]);
			ss += (double) (xv * xv);
			ws += (double) (xv * bf(W[j]));
		}
		const float rs = 1.0f / sqrtf((float) (ss / n_cols) + eps);
		#pragma omp simd
		for (int j = 0; j < n_cols; j++) y[j] = to_bf((bf(x[j]) * rs) * bf(W[j]));
		weighted_sums[r] = (float) ws;
		rstd[r] = rs;
	}
}

/* dX += rstd dY w - X rstd^3 / n sum_j(dY w X) per row; dW += sum_rows dY X rstd
 * (per-thread fp64 column partials, added in thread order) */
void cpu_ref_rms_norm_bwd_bf16(int n_rows, int n_cols, const float * rstd, const uint16_t * W, const uint16_t * X,
							   const uint16_t * dY, uint16_t * dX, float * dW) {
	const int nt = omp_get_max_threads();
	double * part = (double *) calloc((size_t) nt * (size_t) n_cols, sizeof(double));
	if (!part) return;
	#pragma omp parallel
	{
		double * mine = part + (long) omp_get_thread_num() * n_cols;
		#pragma omp for schedule(static)
		for (int r = 0; r < n_rows; r++) {
			const uint16_t * x = X + (long) r * n_cols;
			const uint16_t * g = dY + (long) r * n_cols;
			uint16_t * d = dX + (long) r * n_cols;
			const float rs = rstd[r];
			double dot = 0.0;
			#pragma omp simd reduction(+ : dot)
			for (int j = 0; j < n_cols; j++) dot += (double) (bf(g[j]) * bf(W[j]) * bf(x[j]));
			const float coef = (rs * rs * rs) * (float) dot / (float) n_cols;
			#pragma omp simd
			for (int j = 0; j < n_cols; j++) {
				const float gv = bf(g[j]), xv = bf(x[j]);
				d[j] = to_bf(bf(d[j]) + (rs * (gv * bf(W[j])) - xv * coef));
				mine[j] += (double) (gv * xv * rs);
			}
		}
	}
	for (int t = 0; t < nt; t++) {
		const double * p = part + (long) t * n_cols;
		for (int j = 0; j < n_cols; j++) dW[j] += (float) p[j];
	}
	free(part);
}

/* in place on Q [T x model_dim] and K [T x kv_dim]; pair (2p, 2p + 1) of a
 * head turns by pos * theta^(-2p / head_dim) (inverse turn for bwd) */
void cpu_ref_rope_bf16(int bwd, long n_tokens, int model_dim, int head_dim, int num_kv_heads, int theta, const int * pos,
					   uint16_t * Q, uint16_t * K) {
	const int half = head_dim / 2, kv_dim = num_kv_heads * head_dim;
	float * ang = (float *) malloc(sizeof(float) * (size_t) half);
	if (!ang) return;
	for (int p = 0; p < half; p++) ang[p] = powf((float) theta, -((float) (2 * p) / (float) head_dim));
	#pragma omp parallel
	{
		float * cs = (float *) malloc(sizeof(float) * (size_t) head_dim);
		#pragma omp for schedule(static)
		for (long t = 0; t < n_tokens; t++) {
			const float fp = (float) pos[t];
			for (int p = 0; p < half; p++) {
				const float a = fp * ang[p];
				cs[2 * p] = cosf(a);
				cs[2 * p + 1] = bwd ? -sinf(a) : sinf(a);
			}
			for (int which = 0; which < 2; which++) {
				const int width = which ? kv_dim : model_dim;
				uint16_t * row = (which ? K : Q) + t * width;
				for (int h = 0; h < width; h += head_dim) {
					#pragma omp simd
					for (int p = 0; p < half; p++) {
						const float c = cs[2 * p], s = cs[2 * p + 1];
						const float e = bf(row[h + 2 * p]), o = bf(row[h + 2 * p + 1]);
						row[h + 2 * p] = to_bf(c * e - s * o);
						row[h + 2 * p + 1] = to_bf(c * o + s * e);
					}
				}
			}
		}
		free(cs);
	}
	free(ang);
}

void cpu_ref_swiglu_bf16(long n, const uint16_t * g, const uint16_t * u, uint16_t * out) {
	#pragma omp parallel for simd schedule(static)
	for (long i = 0; i < n; i++) {
		const float gv = bf(g[i]);
		out[i] = to_bf(gv / (1.0f + expf(-gv)) * bf(u[i]));
	}
}

void cpu_ref_swiglu_bwd_bf16(long n, const uint16_t * g, const uint16_t * u, const uint16_t * dout, uint16_t * dg, uint16_t * du) {
	#pragma omp parallel for simd schedule(static)
	for (long i = 0; i < n; i++) {
		const float gv = bf(g[i]), uv = bf(u[i]), d = bf(dout[i]);
		const float s = 1.0f / (1.0f + expf(-gv));
		dg[i] = to_bf(d * uv * (s + gv * s * (1.0f - s)));
		du[i] = to_bf(d * gv * s);
	}
}

/* softmax + cross-entropy in place on the logits, per-row loss and mean
 * loss; each row's exponentials are kept in a per-thread fp32 buffer (a row
 * of the config fits the core's L2), so exp is evaluated once per element */
void cpu_ref_softmax_xent_bf16(int n_rows, int n_cols, uint16_t * logits, const uint32_t * labels, float * loss, float * mean_loss) {
	double total = 0.0;
	#pragma omp parallel reduction(+ : total)
	{
		float * e = (float *) malloc(sizeof(float) * (size_t) n_cols);
		#pragma omp for schedule(static)
		for (int r = 0; r < n_rows; r++) {
			uint16_t * x = logits + (long) r * n_cols;
			float m = -INFINITY;
			#pragma omp simd reduction(max : m)
			for (int j = 0; j < n_cols; j++) m = fmaxf(m, bf(x[j]));
			const uint32_t lab = labels[r];
			const float xl = lab < (uint32_t) n_cols ? bf(x[lab]) : 0.0f;
			double s = 0.0;
			#pragma omp simd reduction(+ : s)
			for (int j = 0; j < n_cols; j++) {
				e[j] = expf(bf(x[j]) - m);
				s += (double) e[j];
			}
			const float inv = (float) (1.0 / s);
			#pragma omp simd
			for (int j = 0; j < n_cols; j++) x[j] = to_bf(e[j] * inv);
			if (lab < (uint32_t) n_cols) x[lab] = to_bf(bf(x[lab]) - 1.0f);
			if (lab < (uint32_t) n_cols) {
				/* -log p_label = log1p(others / exp(x_l - m)), as the kernels
				 * form it, with others = s less the label's term */
				const double gap = (double) m - (double) xl, others = s - (double) e[lab];
				loss[r] = (float) (gap < 16.0 ? log1p(others / exp(-gap)) : log(others + exp(-gap)) + gap);
			}
			else {
				loss[r] = NAN;
			}
			total += loss[r];
		}
		free(e);
	}
	*mean_loss = (float) (total / n_rows);
}
