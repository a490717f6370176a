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
NP_STORAGE = {FP32: np.float32, FP16: np.float16, BF16: np.uint16}
FORMAT = {FP32: (24, -126), FP16: (11, -14), BF16: (8, -126)}   # (mantissa bits incl. implicit, emin)

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
    """fp32 values -> storage array of dtype dt (RNE)."""
    x32 = np.asarray(x32, dtype=np.float32)
    if dt == FP32:
        return x32.copy()
    if dt == FP16:
        return x32.astype(np.float16)
    return f32_to_bf16_bits(x32)


def to_f64(a, dt):
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
    range may flush to zero. fp32 outputs use 1e-5 relative instead of 1 ulp."""
    of = to_f64(o, dt).ravel()
    lo = np.asarray(v_lo, dtype=np.float64).ravel()
    hi = lo if v_hi is None else np.asarray(v_hi, dtype=np.float64).ravel()
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
