"""Test helpers: seeded inputs, the oracle binding and the parity criteria.

The oracle (oracle/liboracle.so) is the checker only; the product path under
test is always libdataflow.so + the gfx950 code object.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_LIB = os.path.join(ROOT, "oracle", "liboracle.so")
REF_HOST_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_host.so")

FP32, FP16, BF16 = 3, 4, 5
FP8E4M3, FP8E5M2 = 6, 7   # OCP 8-bit formats, stored as uint8 codes
NP_STORAGE = {FP32: np.float32, FP16: np.float16, BF16: np.uint16, FP8E4M3: np.uint8, FP8E5M2: np.uint8}
# (mantissa bits incl. implicit, emin)
FORMAT = {FP32: (24, -126), FP16: (11, -14), BF16: (8, -126), FP8E4M3: (4, -6), FP8E5M2: (3, -14)}
FP8_MAX = {FP8E4M3: 448.0, FP8E5M2: 57344.0}

_oracle = None


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_LIB):
            raise RuntimeError("oracle library missing: run __graft_entry__.build()")
        L = ctypes.CDLL(ORACLE_LIB)
        vp, i, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_double
        L.oracle_round.restype = d
        L.oracle_round.argtypes = [d, i]
        L.oracle_ulp.restype = d
        L.oracle_ulp.argtypes = [d, i]
        L.oracle_rms_norm.argtypes = [i, i, i, ctypes.c_float, vp, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_bwd_x.argtypes = [i, i, i, vp, vp, vp, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_bwd_w.argtypes = [i, i, i, i, vp, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_bwd.argtypes = [i, i, i, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.oracle_rope.argtypes = [i, i, ctypes.c_uint64, i, i, i, i, vp, vp, vp, vp, vp]
        L.oracle_swiglu.argtypes = [i, ctypes.c_long, vp, vp, vp]
        L.oracle_swiglu_bwd.argtypes = [i, ctypes.c_long, vp, vp, vp, vp, vp, vp]
        L.oracle_softmax.argtypes = [i, i, i, i, vp, vp]
        L.oracle_cross_entropy_loss.argtypes = [i, i, i, vp, vp]
        L.oracle_softmax_cross_entropy.argtypes = [i, i, i, vp, vp, vp, vp, vp, vp]
        L.oracle_embedding.argtypes = [i, i, i, vp, vp, ctypes.c_long, vp]
        L.oracle_copy_to_seq_context.argtypes = [i, ctypes.c_uint64, i, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_bwd_x2.argtypes = [i, i, i, i, vp, vp, vp, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_bwd_x2_exact.argtypes = [i, i, i, i, vp, vp, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_bwd_w2.argtypes = [i, i, i, i, i, vp, vp, vp, vp, vp, vp]
        L.oracle_rms_norm_sq_sums.argtypes = [i, i, i, vp, vp]
        L.oracle_swiglu_bwd2.argtypes = [i, i, ctypes.c_long, vp, vp, vp, vp, vp, vp]
        L.oracle_load.argtypes = [i, vp, ctypes.c_long, vp]
        L.oracle_store.argtypes = [i, vp, ctypes.c_long, vp]
        _oracle = L
    return _oracle


def ptr(a):
    """c_void_p to a numpy array's data; the pointer object keeps the array
    alive, so temporaries survive until the C call returns"""
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------- formats ----------------

def f32_to_bf16_bits(x):
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_storage(x32, dt):
    """fp32 values -> storage array of dtype dt (RNE; fp8 saturates to +-max)."""
    x32 = np.asarray(x32, dtype=np.float32)
    if dt in FP8_MAX:
        v = np.ascontiguousarray(x32, dtype=np.float64)
        out = np.empty(v.shape, np.uint8)
        oracle().oracle_store(dt, ptr(v), v.size, ptr(out))
        return out
    if dt == FP32:
        return x32.copy()
    if dt == FP16:
        return x32.astype(np.float16)
    return f32_to_bf16_bits(x32)


def rope_pair_floor(x, width):
    """fp32 evaluation floor of a rotated pair, per output element: the two
    products of each output are at most |e| + |o| (|cos|, |sin| <= 1), and
    the fp32 tables and products carry a few 2^-24 of that, which remains
    when the products cancel: 8 * 2^-24 * (|e| + |o|), for both outputs of
    the pair. x holds the input rows as floats, `width` columns each."""
    v = np.abs(np.asarray(x, dtype=np.float64).reshape(-1, width))
    m = v[:, 0::2] + v[:, 1::2]
    return np.repeat(m, 2, axis=1).ravel() * 8.0 * 2.0 ** -24


def to_f64(a, dt):
    if dt in FP8_MAX:
        a = np.ascontiguousarray(a, dtype=np.uint8)
        out = np.empty(a.shape)
        oracle().oracle_load(dt, ptr(a), a.size, ptr(out))
        return out
    if dt == BF16:
        return bf16_bits_to_f32(a).astype(np.float64)
    return np.asarray(a).astype(np.float64)


def ulp(v, dt):
    mant, emin = FORMAT[dt]
    a = np.abs(np.asarray(v, dtype=np.float64))
    _, e = np.frexp(np.where(a > 0, a, 1.0))
    lead = np.maximum(e - 1, emin)
    return np.ldexp(1.0, lead - (mant - 1))


def rng(seed):
    return np.random.default_rng(seed)


def normal(seed, shape, mean=0.0, std=1.0):
    return (mean + std * rng(seed).standard_normal(shape)).astype(np.float32)


# ---------------- parity criteria ----------------

FTZ_LIMIT = 2.0 ** -126   # fp32 subnormal range: values below may flush to zero


def check_rounded(o, dt, v_lo, v_hi=None, floor=None, what=""):
    """Half-precision outputs: every element within 1 ulp (of the output type)
    of the exact pre-rounding value, or of the [v_lo, v_hi] interval when the
    reference rounds an intermediate. `floor` adds an fp32-evaluation noise
    bound where the exact expression cancels. Values in the fp32 subnormal
    range may flush to zero. fp32 outputs use 1e-5 relative instead of 1 ulp.
    fp8 outputs saturate: the expected values are clamped to +-max first."""
    of = to_f64(o, dt).ravel()
    lo = np.asarray(v_lo, dtype=np.float64).ravel()
    hi = lo if v_hi is None else np.asarray(v_hi, dtype=np.float64).ravel()
    if dt in FP8_MAX:
        lo, hi = np.clip(lo, -FP8_MAX[dt], FP8_MAX[dt]), np.clip(hi, -FP8_MAX[dt], FP8_MAX[dt])
    a, b = np.minimum(lo, hi), np.maximum(lo, hi)
    fl = 0.0 if floor is None else np.asarray(floor, dtype=np.float64).ravel()
    if dt == FP32:
        tol_a = 1e-5 * np.abs(a) + fl
        tol_b = 1e-5 * np.abs(b) + fl
    else:
        tol_a = ulp(a, dt) + fl
        tol_b = ulp(b, dt) + fl
    ok = (of >= a - tol_a) & (of <= b + tol_b)
    ok |= (np.abs(a) < FTZ_LIMIT) & (np.abs(b) < FTZ_LIMIT) & (np.abs(of) <= FTZ_LIMIT)
    ok |= np.isnan(of) & (np.isnan(a) | np.isnan(b))
    if not ok.all():
        bad = np.flatnonzero(~ok)
        k = bad[0]
        raise AssertionError("%s: %d of %d elements out of tolerance; first at %d: got %r, expected [%r, %r] (+-%r)"
                             % (what, bad.size, of.size, k, of[k], a[k], b[k], max(tol_a[k] if np.ndim(tol_a) else tol_a, 0)))


def check_f32(o, v, rel=1e-5, floor=None, what=""):
    o = np.asarray(o, dtype=np.float64).ravel()
    v = np.asarray(v, dtype=np.float64).ravel()
    tol = rel * np.abs(v) + (0.0 if floor is None else np.asarray(floor, dtype=np.float64).ravel())
    with np.errstate(invalid="ignore"):
        ok = (np.abs(o - v) <= tol) | (np.isnan(o) & np.isnan(v)) | (o == v)
    if not ok.all():
        bad = np.flatnonzero(~ok)
        k = bad[0]
        raise AssertionError("%s: %d of %d fp32 values out of tolerance; first at %d: got %r, expected %r"
                             % (what, bad.size, o.size, k, o[k], v[k]))


# ---------------- fp32 reduction error bounds ----------------
#
# A sum of n terms accumulated in fp32 along a tree of depth d (the most
# roundings any term goes through) is within gamma(d) * sum|terms| of the
# exact sum, gamma(d) = d u / (1 - d u), u = 2^-24 (Higham, Accuracy and
# Stability of Numerical Algorithms, 2nd ed., section 4.2). The RMSNorm
# kernels' depths follow from their launch shapes, restated here from
# dataflow_lib_amd/csrc/kernels/kernel_geometry.h and the kernels' loops.

U32 = 2.0 ** -24
RMS_CH, RMS_MAX_TPR, RMS_STREAM_TPR = 2, 1024, 256
RMS_CELLS_PER_SLOT, RMS_INFLIGHT_BYTES = 64, 64 * 1024
RMS_STREAM_WIDE_COLS, RMS_FIN_GROUPS = 4096, 256 // 16   # finish: RMS_FINISH_THREADS / RMS_FIN_COLS
RMS_DW_SCRATCH_FLOATS = 4 << 20
ELEM_BYTES = {FP32: 4, FP16: 2, BF16: 2, FP8E4M3: 1, FP8E5M2: 1}


def gamma(d):
    return d * U32 / (1.0 - d * U32)


# Config-2 gate for the fp32 sums (weighted_sums, bwd_w dW, the fused dW):
# SUM_GATE_U * u * sum|terms| on top of 1e-5 relative. gamma(d) above holds for
# any input but is the worst case (every rounding error of one sign); on the
# config's random N(0, 1) inputs the kernels' errors are measured at 0.12 u
# (ws) and 0.19 u (fused dW) times sum|terms| (test_fp32_reduction_errors_at_config2),
# and the gate sits 20x above that. Partial sums that lost precision fail it:
# dW partial rows rounded to fp16 exceed it on most columns
# (tests/test_gates.py plants that mistake in a CPU model of the reduction).
SUM_GATE_U = 4.0


def sum_gate(absum):
    return SUM_GATE_U * U32 * np.asarray(absum, dtype=np.float64)


def rms_vec_chunks(n_cols, elem, aligned=True):
    vec = 16 // elem
    if n_cols <= 0 or n_cols % vec or not aligned:
        return 0
    nv = n_cols // vec
    return nv if (nv + RMS_CH - 1) // RMS_CH <= RMS_MAX_TPR else 0


def rms_tpr_for(nv):
    if nv == 0:
        return RMS_STREAM_TPR
    t = (nv + RMS_CH - 1) // RMS_CH
    return ((t + 63) // 64) * 64


def rms_ws_depth(dt, n_cols, aligned=True):
    """roundings along the weighted-sum tree of rms_norm's forward. Vector
    path: four interleaved per-thread sums of RMS_CH * V / 4 terms each, added
    pairwise (2), the wave's DPP tree (6), then the slot's waves in sequence.
    Element path: a thread's terms in sequence, then the same. The first fma
    of an fp32 sum rounds its product (bf16 / fp16 products are exact)."""
    elem = ELEM_BYTES[dt]
    nv = rms_vec_chunks(n_cols, elem, aligned)
    tpr = rms_tpr_for(nv)
    vec = 16 // elem
    if nv:
        per_thread = RMS_CH * vec // 4 + 2
    elif aligned and n_cols % vec == 0:
        per_thread = -(-(n_cols // vec) // tpr) * vec
    else:
        per_thread = -(-n_cols // tpr)
    return per_thread + 6 + tpr // 64


def rms_dw_depth(dt, n_rows, n_cols, arrays, cu_count, max_lds, aligned=True):
    """roundings along the dW reduction of rms_norm_bwd_w (arrays = 2) and the
    fused rms_norm_bwd (arrays = 3), for the launch shape rms_dw_geometry
    picks: a thread's rows in sequence, the workgroup's slots in sequence,
    then the finish pass (a thread's share of the grid's partial rows, its
    RMS_FIN_GROUPS groups, then dW + the total). fp32 inputs add the rounding
    of the product dY * X."""
    elem = ELEM_BYTES[dt]
    nv = rms_vec_chunks(n_cols, elem, aligned)
    tpr = rms_tpr_for(nv) if nv else (RMS_MAX_TPR if n_cols >= RMS_STREAM_WIDE_COLS else RMS_STREAM_TPR)
    per_slot = 2 * n_cols * elem * arrays
    slots = min(max(1, min(RMS_INFLIGHT_BYTES // per_slot, 32)), max(1, RMS_MAX_TPR // tpr))
    while slots >= 1:
        colbuf = n_cols if nv else slots * n_cols
        if (RMS_CELLS_PER_SLOT * slots + colbuf) * 4 <= max_lds:
            break
        slots -= 1
    assert slots >= 1
    grid = min(-(-n_rows // slots), cu_count, RMS_DW_SCRATCH_FLOATS // n_cols)
    rows = -(-n_rows // (grid * slots))
    finish = -(-grid // RMS_FIN_GROUPS) + RMS_FIN_GROUPS + 1
    return rows + (slots - 1) + finish + (1 if dt == FP32 else 0)


def rms_dw_fp8_depth(n_rows, n_cols, cu_count, aligned=True):
    """roundings along the dW reduction of the fp8-input rms_norm_bwd_w
    (fp8_ops.hip, launch shape in hip_ops_config.c; fp8 x 16-bit products are
    exact in fp32). Chunked path (aligned rows of a multiple of 8 columns, up
    to 8 * F8_CPT * 1024): a slot's rows in sequence in registers, the
    workgroup's slots added in LDS, then the finish pass. Element path: the
    workgroup's rows in sequence into its LDS row, then the finish pass."""
    F8_CPT = 2
    tpr = 0
    if aligned and n_cols % 8 == 0:
        t = -(-(n_cols // 8) // F8_CPT)
        tpr = -(-t // 64) * 64
        tpr = tpr if tpr <= 1024 else 0
    slots = max(1, 1024 // tpr) if tpr else 1
    grid = min(-(-n_rows // slots), cu_count, RMS_DW_SCRATCH_FLOATS // n_cols)
    rows = -(-n_rows // (grid * slots))
    return rows + (slots - 1) + (-(-grid // RMS_FIN_GROUPS) + RMS_FIN_GROUPS + 1)


def confident_logits(shape, seed):
    """bf16 logits of a confident model: the label holds the row max 7.03125
    and every other logit sits near 13 below it (N(-13, 0.3)), so about a
    fifth of sum exp(x - m) comes from the bulk, whose differences x - m are
    rounded to bf16 with errors up to 2^-5. A loss built from exp(rnd(x - m))
    corrected only to first order is off by ~2e-4 relative here (the losses
    are ~0.27); to second order by <1e-6. Returns (bf16 bits, labels)."""
    n_rows, n_cols = shape
    x = 7.03125 - 13.0 + normal(seed, shape, std=0.3)
    labels = rng(seed + 1).integers(0, n_cols, size=n_rows).astype(np.uint32)
    x[np.arange(n_rows), labels] = 7.03125
    return to_storage(x, BF16), labels
