/*
 * Native op skeletons and their registration.
 *
 * Each op is described once by a row of native_op_specs (nickname form and
 * argument dtype list) instead of one hand-written setter per op; the bytes
 * produced are the reference's (src/set_ops/src/set_native_op_skeletons.c:234-611):
 * NUL-padded nickname "<op>_<DT>[_<DT>]", num_args, arg dtypes with the rest
 * DATAFLOW_NONE, and SHA-256 over the whole 388-byte header.
 */
#include "set_native_op_skeletons.h"

#include <ctype.h>
#include <stdatomic.h>

/* placeholders in an argument list, resolved to the op's fwd / bwd dtype */
#define ARG_FWD ((int) -1)
#define ARG_BWD ((int) -2)

typedef enum { NICK_FWD, NICK_BWD, NICK_FWD_BWD } Nick_Form;

typedef struct {
	const char * name;
	Nick_Form nick;
	int num_args;
	int args[12];
	const char * init_symbol;
} Native_Op_Spec;

#define I_S DATAFLOW_INT_SCALAR
#define F_S DATAFLOW_FP32_SCALAR
#define U64_S DATAFLOW_UINT64_SCALAR
#define RMS_INIT "rms_norm_set_attribute_config"
#define SMX_INIT "softmax_set_attribute_config"

static const Native_Op_Spec native_op_specs[] = {
	/* reference set_native_op_skeletons.c:234-270 */
	{"embedding",           NICK_FWD,     5, {I_S, I_S, DATAFLOW_UINT32, ARG_FWD, ARG_FWD}, NULL},
	/* :272-306 (n_rows, n_cols, eps, W, X, out, weighted_sums, rms_vals) */
	{"rms_norm",            NICK_FWD,     8, {I_S, I_S, F_S, ARG_FWD, ARG_FWD, ARG_FWD, DATAFLOW_FP32, DATAFLOW_FP32}, RMS_INIT},
	/* :308-342 (.., eps, weighted_sums, rms_vals, W, X, dY, dX) */
	{"rms_norm_bwd_x",      NICK_FWD_BWD, 9, {I_S, I_S, F_S, DATAFLOW_FP32, DATAFLOW_FP32, ARG_FWD, ARG_FWD, ARG_BWD, ARG_BWD}, RMS_INIT},
	/* :344-376 (.., eps, rms_vals, X, dY, dW) */
	{"rms_norm_bwd_w",      NICK_FWD_BWD, 7, {I_S, I_S, F_S, DATAFLOW_FP32, ARG_FWD, ARG_BWD, ARG_BWD}, RMS_INIT},
	/* fused exact-gradient backward, no reference counterpart:
	 * (n_rows, n_cols, eps, rms_vals, W, X, dY, dX, dW fp32) */
	{"rms_norm_bwd",        NICK_FWD_BWD, 9, {I_S, I_S, F_S, DATAFLOW_FP32, ARG_FWD, ARG_FWD, ARG_BWD, ARG_BWD, DATAFLOW_FP32}, RMS_INIT},
	/* :378-411 (N, model_dim, head_dim, num_kv_heads, theta, seq_positions, X_q, X_k) */
	{"rope",                NICK_FWD,     8, {U64_S, I_S, I_S, I_S, I_S, DATAFLOW_INT, ARG_FWD, ARG_FWD}, NULL},
	/* :413-446 */
	{"rope_bwd_x",          NICK_BWD,     8, {U64_S, I_S, I_S, I_S, I_S, DATAFLOW_INT, ARG_BWD, ARG_BWD}, NULL},
	/* :448-484 */
	{"copy_to_seq_context", NICK_FWD,     8, {U64_S, I_S, I_S, ARG_FWD, ARG_FWD, DATAFLOW_INT, DATAFLOW_UINT64, DATAFLOW_INT}, NULL},
	/* :486-515 (rows, cols, x_w1, x_w3, out) */
	{"swiglu",              NICK_FWD,     5, {I_S, I_S, ARG_FWD, ARG_FWD, ARG_FWD}, NULL},
	/* :517-549 (rows, cols, x_w1, x_w3, dOut, dX_w1, dX_w3) */
	{"swiglu_bwd_x",        NICK_FWD_BWD, 7, {I_S, I_S, ARG_FWD, ARG_FWD, ARG_BWD, ARG_BWD, ARG_BWD}, NULL},
	/* :551-580 (rows, cols, X, out) */
	{"softmax",             NICK_FWD_BWD, 4, {I_S, I_S, ARG_FWD, ARG_BWD}, SMX_INIT},
	/* :582-611 (rows, cols, pred_logits, labels) */
	{"cross_entropy_loss",  NICK_BWD,     4, {I_S, I_S, ARG_BWD, DATAFLOW_UINT32}, NULL},
	/* fused softmax + cross-entropy, no reference counterpart:
	 * (rows, cols, logits (in place), labels, loss fp32 [rows], mean_loss fp32 [1]) */
	{"softmax_cross_entropy_loss", NICK_FWD, 6, {I_S, I_S, ARG_FWD, DATAFLOW_UINT32, DATAFLOW_FP32, DATAFLOW_FP32}, SMX_INIT},
	/* RoPE fused with the KV-cache scatter, no reference counterpart: rope's
	 * 8 args, then values and copy_to_seq_context's context pointers and sizes */
	{"rope_copy_to_seq_context", NICK_FWD, 11, {U64_S, I_S, I_S, I_S, I_S, DATAFLOW_INT, ARG_FWD, ARG_FWD, ARG_FWD,
												 DATAFLOW_UINT64, DATAFLOW_INT}, NULL},
};

#define NUM_NATIVE_OP_SPECS ((int) (sizeof(native_op_specs) / sizeof(native_op_specs[0])))

static const Native_Op_Spec * find_spec(const char * op_name) {
	for (int i = 0; i < NUM_NATIVE_OP_SPECS; i++) {
		if (strcmp(native_op_specs[i].name, op_name) == 0) {
			return &native_op_specs[i];
		}
	}
	return NULL;
}

/* Fingerprints are a pure function of (op, fwd dtype, bwd dtype), so each is
 * computed once per process and kept: every submit_* builds its op's skeleton,
 * and the SHA-256 is most of that cost. An entry goes 0 (empty) -> 1 (being
 * written, by the one thread that won it) -> 2 (ready); a thread that finds it
 * not ready computes the digest itself. */
#define FP_DT_SLOTS 32
typedef struct {
	_Atomic int state;
	uint8_t fingerprint[OP_IDENTIFIER_FINGERPRINT_NUM_BYTES];
} Fingerprint_Cache_Entry;
static Fingerprint_Cache_Entry fingerprint_cache[NUM_NATIVE_OP_SPECS][FP_DT_SLOTS][FP_DT_SLOTS];

static void build_skeleton(Op_Skeleton * skeleton, const Native_Op_Spec * spec, DataflowDatatype fwd_dt, DataflowDatatype bwd_dt) {
	Op_Skeleton_Header * h = &skeleton->header;
	char nick[FUNC_SYMBOL_MAX_LEN];
	switch (spec->nick) {
		case NICK_FWD:
			snprintf(nick, sizeof(nick), "%s_%s", spec->name, dataflow_datatype_as_string(fwd_dt));
			break;
		case NICK_BWD:
			snprintf(nick, sizeof(nick), "%s_%s", spec->name, dataflow_datatype_as_string(bwd_dt));
			break;
		default:
			snprintf(nick, sizeof(nick), "%s_%s_%s", spec->name, dataflow_datatype_as_string(fwd_dt), dataflow_datatype_as_string(bwd_dt));
			break;
	}
	/* zero everything first: unused nickname bytes and dtypes (NONE == 0)
	 * must be zero for the digest to be stable */
	memset(h, 0, sizeof(*h));
	strncpy(h->op_nickname, nick, MAX_OP_NICKNAME_SIZE);
	h->op_nickname[MAX_OP_NICKNAME_SIZE] = '\0';
	h->num_args = spec->num_args;
	for (int i = 0; i < spec->num_args; i++) {
		int a = spec->args[i];
		h->arg_dtypes[i] = (a == ARG_FWD) ? fwd_dt : (a == ARG_BWD) ? bwd_dt : (DataflowDatatype) a;
	}
	Fingerprint_Cache_Entry * e = NULL;
	if ((unsigned) fwd_dt < FP_DT_SLOTS && (unsigned) bwd_dt < FP_DT_SLOTS) {
		e = &fingerprint_cache[spec - native_op_specs][fwd_dt][bwd_dt];
		if (atomic_load_explicit(&e->state, memory_order_acquire) == 2) {
			memcpy(skeleton->identifier.fingerprint, e->fingerprint, OP_IDENTIFIER_FINGERPRINT_NUM_BYTES);
			return;
		}
	}
	do_fingerprinting(h, sizeof(Op_Skeleton_Header), skeleton->identifier.fingerprint, OP_IDENTIFIER_FINGERPRINT_TYPE);
	int empty = 0;
	if (e && atomic_compare_exchange_strong_explicit(&e->state, &empty, 1, memory_order_acq_rel, memory_order_relaxed)) {
		memcpy(e->fingerprint, skeleton->identifier.fingerprint, OP_IDENTIFIER_FINGERPRINT_NUM_BYTES);
		atomic_store_explicit(&e->state, 2, memory_order_release);
	}
}

int set_native_op_skeleton(Op_Skeleton * skeleton, char * op_name, DataflowDatatype fwd_dt, DataflowDatatype bwd_dt) {
	const Native_Op_Spec * spec = find_spec(op_name);
	if (!spec) {
		printf("Cannot set skeleton, unknown op: %s, with fwd_dt: %s, bwd_dt: %s\n", op_name,
				dataflow_datatype_as_string(fwd_dt), dataflow_datatype_as_string(bwd_dt));
		return -1;
	}
	build_skeleton(skeleton, spec, fwd_dt, bwd_dt);
	return 0;
}

#define DEFINE_FWD_SETTER(fn, opname) \
	void fn(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype) { \
		build_skeleton(skeleton, find_spec(opname), fwd_datatype, DATAFLOW_NONE); \
	}
#define DEFINE_BWD_SETTER(fn, opname) \
	void fn(Op_Skeleton * skeleton, DataflowDatatype bwd_datatype) { \
		build_skeleton(skeleton, find_spec(opname), DATAFLOW_NONE, bwd_datatype); \
	}
#define DEFINE_FWD_BWD_SETTER(fn, opname) \
	void fn(Op_Skeleton * skeleton, DataflowDatatype fwd_datatype, DataflowDatatype bwd_datatype) { \
		build_skeleton(skeleton, find_spec(opname), fwd_datatype, bwd_datatype); \
	}

DEFINE_FWD_SETTER(set_native_embedding_skeleton, "embedding")
DEFINE_FWD_SETTER(set_native_rms_norm_skeleton, "rms_norm")
DEFINE_FWD_BWD_SETTER(set_native_rms_norm_bwd_x_skeleton, "rms_norm_bwd_x")
DEFINE_FWD_BWD_SETTER(set_native_rms_norm_bwd_w_skeleton, "rms_norm_bwd_w")
DEFINE_FWD_BWD_SETTER(set_native_rms_norm_bwd_skeleton, "rms_norm_bwd")
DEFINE_FWD_SETTER(set_native_rope_skeleton, "rope")
DEFINE_BWD_SETTER(set_native_rope_bwd_x_skeleton, "rope_bwd_x")
DEFINE_FWD_SETTER(set_native_copy_to_seq_context_skeleton, "copy_to_seq_context")
DEFINE_FWD_SETTER(set_native_swiglu_skeleton, "swiglu")
DEFINE_FWD_BWD_SETTER(set_native_swiglu_bwd_x_skeleton, "swiglu_bwd_x")
DEFINE_FWD_BWD_SETTER(set_native_softmax_skeleton, "softmax")
DEFINE_BWD_SETTER(set_native_cross_entropy_loss_skeleton, "cross_entropy_loss")
DEFINE_FWD_SETTER(set_native_softmax_cross_entropy_loss_skeleton, "softmax_cross_entropy_loss")
DEFINE_FWD_SETTER(set_native_rope_copy_to_seq_context_skeleton, "rope_copy_to_seq_context")

/* ---- registration ---- */

/* Variants provided by the gfx950 code object: the reference's 54
 * (set_native_op_skeletons.c:5-200: fp32 / fp16 / bf16 / fp8e4m3 / fp8e5m2
 * forward ops, fp32 / fp16 / bf16 rope_bwd_x and cross_entropy_loss, and the
 * seven (forward, backward) type pairs of the backward ops and softmax,
 * fp8 forward with fp16 / bf16 backward among them), copy_to_seq_context in
 * all five storage types, and the three fused ops this library adds in fp32 /
 * fp16 / bf16. */
typedef struct { const char * op; DataflowDatatype fwd; DataflowDatatype bwd; } Native_Variant;

#define FWD3(op) {op, DATAFLOW_FP32, DATAFLOW_NONE}, {op, DATAFLOW_FP16, DATAFLOW_NONE}, {op, DATAFLOW_BF16, DATAFLOW_NONE}
#define BWD3(op) {op, DATAFLOW_NONE, DATAFLOW_FP32}, {op, DATAFLOW_NONE, DATAFLOW_FP16}, {op, DATAFLOW_NONE, DATAFLOW_BF16}
#define PAIR3(op) {op, DATAFLOW_FP32, DATAFLOW_FP32}, {op, DATAFLOW_FP16, DATAFLOW_FP16}, {op, DATAFLOW_BF16, DATAFLOW_BF16}

#define FWD5(op) FWD3(op), {op, DATAFLOW_FP8E4M3, DATAFLOW_NONE}, {op, DATAFLOW_FP8E5M2, DATAFLOW_NONE}
/* the reference's seven (fwd, bwd) pairs: the three same-type ones and fp8 x {fp16, bf16} */
#define PAIR7(op) PAIR3(op), {op, DATAFLOW_FP8E4M3, DATAFLOW_FP16}, {op, DATAFLOW_FP8E4M3, DATAFLOW_BF16}, \
				  {op, DATAFLOW_FP8E5M2, DATAFLOW_FP16}, {op, DATAFLOW_FP8E5M2, DATAFLOW_BF16}

static const Native_Variant native_variants[] = {
	FWD5("embedding"),
	FWD5("rms_norm"),
	PAIR7("rms_norm_bwd_x"),
	PAIR7("rms_norm_bwd_w"),
	PAIR3("rms_norm_bwd"),
	FWD5("rope"),
	BWD3("rope_bwd_x"),
	FWD5("copy_to_seq_context"),
	FWD5("swiglu"),
	PAIR7("swiglu_bwd_x"),
	PAIR7("softmax"),
	BWD3("cross_entropy_loss"),
	FWD3("softmax_cross_entropy_loss"),
	FWD3("rope_copy_to_seq_context"),
};

#define NUM_NATIVE_VARIANTS ((int) (sizeof(native_variants) / sizeof(native_variants[0])))

static void append_lower_dt(char * dst, size_t cap, DataflowDatatype dt) {
	const char * s = dataflow_datatype_as_string(dt);
	size_t len = strlen(dst);
	if (len + 1 < cap) dst[len++] = '_';
	for (; *s && len + 1 < cap; s++) dst[len++] = (char) tolower((unsigned char) *s);
	dst[len] = '\0';
}

int register_native_ops(Dataflow_Handle * dataflow_handle, char * native_function_code_filename, char * native_function_config_filename) {
	int n = NUM_NATIVE_VARIANTS;
	Op_Skeleton * skeletons = (Op_Skeleton *) calloc((size_t) n, sizeof(Op_Skeleton));
	char ** func_symbols = (char **) calloc((size_t) n, sizeof(char *));
	char ** launch_symbols = (char **) calloc((size_t) n, sizeof(char *));
	char ** init_symbols = (char **) calloc((size_t) n, sizeof(char *));
	int added = -1;
	if (!skeletons || !func_symbols || !launch_symbols || !init_symbols) {
		fprintf(stderr, "Error: failed to allocate native op registration metadata...\n");
		goto cleanup;
	}

	for (int i = 0; i < n; i++) {
		const Native_Variant * v = &native_variants[i];
		const Native_Op_Spec * spec = find_spec(v->op);
		build_skeleton(&skeletons[i], spec, v->fwd, v->bwd);

		func_symbols[i] = (char *) calloc(FUNC_SYMBOL_MAX_LEN, 1);
		launch_symbols[i] = (char *) calloc(FUNC_SYMBOL_MAX_LEN, 1);
		if (!func_symbols[i] || !launch_symbols[i]) {
			fprintf(stderr, "Error: failed to allocate native op symbol names...\n");
			goto cleanup;
		}
		snprintf(func_symbols[i], FUNC_SYMBOL_MAX_LEN, "%s", v->op);
		if (spec->nick != NICK_BWD) append_lower_dt(func_symbols[i], FUNC_SYMBOL_MAX_LEN, v->fwd);
		if (spec->nick != NICK_FWD) append_lower_dt(func_symbols[i], FUNC_SYMBOL_MAX_LEN, v->bwd);
		strncat(func_symbols[i], "_kernel", FUNC_SYMBOL_MAX_LEN - strlen(func_symbols[i]) - 1);
		snprintf(launch_symbols[i], FUNC_SYMBOL_MAX_LEN, "%s_set_launch_config", v->op);
		if (spec->init_symbol) {
			init_symbols[i] = (char *) calloc(FUNC_SYMBOL_MAX_LEN, 1);
			if (!init_symbols[i]) goto cleanup;
			snprintf(init_symbols[i], FUNC_SYMBOL_MAX_LEN, "%s", spec->init_symbol);
		}
	}

	added = dataflow_handle->register_native_code(dataflow_handle, native_function_code_filename, native_function_config_filename,
													n, skeletons, func_symbols, launch_symbols, init_symbols);
	if (added != n) {
		fprintf(stderr, "WARNING: failed to register all native ops, expected %d functions, got %d...\n", n, added);
	}

cleanup:
	for (int i = 0; i < n; i++) {
		if (func_symbols) free(func_symbols[i]);
		if (launch_symbols) free(launch_symbols[i]);
		if (init_symbols) free(init_symbols[i]);
	}
	free(func_symbols);
	free(launch_symbols);
	free(init_symbols);
	free(skeletons);
	return added;
}
