"""Parity of the fp8 variants (gfx950 kernels, through the C ABI) with the oracle.

The reference registers 22 functions with fp8 tensors (OCP E4M3 and E5M2):
the forward rms_norm, rope and swiglu with fp8 storage throughout, and
rms_norm_bwd_x, rms_norm_bwd_w, swiglu_bwd_x and softmax with fp8 forward
tensors and fp16 / bf16 backward ones. Each is called through the submit_*
entry points and compared with oracle/liboracle.so on the same seeded inputs.
Criteria as for the other types (tests/support.py): each output within 1 ulp
of its type of the exact pre-rounding value (fp8 outputs saturate to +-max, so
the expected value is clamped first); fp32 sums within the rounding bound of
the kernel's summation tree.
"""
import numpy as np
import pytest

from support import (BF16, FP16, FP8_MAX, FP8E4M3, FP8E5M2, NP_STORAGE, check_f32, check_rounded, gamma, normal, oracle,
                     ptr, rms_dw_fp8_depth, rms_ws_depth, rng, rope_pair_floor, to_f64, to_storage)
from test_hip_ops import Dev, hdl  # noqa: F401  (the module's handle fixture)

pytestmark = pytest.mark.gpu
F8 = [FP8E4M3, FP8E5M2]
B16 = [FP16, BF16]
IDS = {FP8E4M3: "e4m3", FP8E5M2: "e5m2", FP16: "fp16", BF16: "bf16"}


def dt_id(dt):
    return IDS[dt]


def all_codes(dt):
    """the 256 codes of an fp8 type with finite values"""
    codes = np.arange(256, dtype=np.uint8)
    return codes[np.isfinite(to_f64(codes, dt))]


# ---------------- conversions (through ops whose arithmetic is exact) ----------------

@pytest.mark.parametrize("dt", F8, ids=dt_id)
def test_fp8_decode_encode_every_code(hdl, dt):
    """RoPE at position 0 rotates by cos 0 = 1, sin 0 = 0: q' = q * 1 - q2 * 0
    is q itself for finite q2, so every finite code must come back unchanged
    (decode, then encode)."""
    from dataflow_lib_amd import api
    codes = all_codes(dt)
    hd = 2 * codes.size
    Q = np.concatenate([codes, codes[::-1]]).reshape(1, hd)
    pos = np.zeros(1, np.int32)
    with Dev(hdl) as d:
        pq, pk, pp = d.put(Q), d.put(np.zeros(16, np.uint8)), d.put(pos)
        assert api.submit_rope(hdl, 0, dt, hd, hd, hd, 0, 500000, pp, pq, pk) == 0
        gq = d.get(pq, Q.shape, np.uint8)
    v_in, v_out = to_f64(Q, dt), to_f64(gq, dt)
    assert np.array_equal(v_in, v_out)


@pytest.mark.parametrize("dt", F8, ids=dt_id)
def test_fp8_encode_rounding_and_saturation(hdl, dt):
    """swiglu(g, u) = silu(g) * u with g = max: silu(max) = max exactly in fp32
    (exp(-max) underflows), so out = fp8(max * u) with an exact product. Over
    every code u (and NaN, +-inf for E5M2) this checks round to nearest even
    (ties included: 1.75 * 1.5 = 2.625 lies between 2.5 and 2.75), saturation
    to +-max, and NaN propagation."""
    from dataflow_lib_amd import api
    codes = np.arange(256, dtype=np.uint8)
    u = codes
    g = np.full_like(u, to_storage(np.array([FP8_MAX[dt]], np.float32), dt)[0])
    pre = np.empty(u.size)
    assert oracle().oracle_swiglu(dt, u.size, ptr(g), ptr(u), ptr(pre)) == 0
    with Dev(hdl) as d:
        pg, pu, po = d.put(g), d.put(u), d.empty(u.size)
        assert api.submit_swiglu(hdl, 0, dt, 1, u.size, pg, pu, po) == 0
        out = d.get(po, (u.size,), np.uint8)
    expect = to_storage(np.clip(pre, -FP8_MAX[dt], FP8_MAX[dt]).astype(np.float32), dt)
    vu = to_f64(u, dt)
    fin = np.isfinite(vu)
    # the exact product rounds once: bit-identical codes (a zero may differ in sign only)
    vo, ve = to_f64(out, dt), to_f64(expect, dt)
    assert np.array_equal(vo[fin], ve[fin])
    assert np.isnan(vo[np.isnan(vu)]).all()
    if dt == FP8E5M2:
        inf = np.isinf(vu)
        assert np.array_equal(vo[inf], np.sign(vu[inf]) * FP8_MAX[dt])
    # products past the largest finite value saturate rather than turn into NaN / inf
    assert (np.abs(vo[fin]) <= FP8_MAX[dt]).all() and (np.abs(vo[fin & (np.abs(vu) >= 2)]) == FP8_MAX[dt]).all()


# ---------------- RMSNorm ----------------

RMS_SHAPES = [(16, 4096), (64, 4096), (7, 8192), (33, 1000), (5, 8), (3, 20000), (8192, 4096), (5, 4099), (9, 4112),
              (1024, 8192), (64, 16384)]


def rms_inputs(dt, n_rows, n_cols, seed=1):
    X = to_storage(normal(seed, (n_rows, n_cols)), dt)
    W = to_storage(1.0 + normal(seed + 1, (n_cols,), std=0.02), dt)
    return X, W


@pytest.mark.parametrize("dt", F8, ids=dt_id)
@pytest.mark.parametrize("shape", RMS_SHAPES, ids=lambda s: "%dx%d" % s)
def test_rms_norm_fwd_fp8(hdl, dt, shape):
    """out = fp8((x * rstd) * w); the statistic slot gets sum_j x^2 (not
    rstd) and weighted_sums is left as it was, as in the reference's fp8
    kernels"""
    from dataflow_lib_amd import api
    n_rows, n_cols = shape
    eps = 1e-5
    X, W = rms_inputs(dt, n_rows, n_cols)
    y_pre = np.empty((n_rows, n_cols))
    assert oracle().oracle_rms_norm(dt, n_rows, n_cols, eps, ptr(W), ptr(X), ptr(y_pre), None, None, None) == 0
    ss = np.empty(n_rows)
    assert oracle().oracle_rms_norm_sq_sums(dt, n_rows, n_cols, ptr(X), ptr(ss)) == 0
    sentinel = np.full(n_rows, -12345.5, np.float32)
    with Dev(hdl) as d:
        px, pw, py = d.put(X), d.put(W), d.empty(X.nbytes)
        pws, pss = d.put(sentinel), d.empty(4 * n_rows)
        assert api.submit_rms_norm(hdl, 0, dt, n_rows, n_cols, eps, pw, px, py, pws, pss) == 0
        y = d.get(py, X.shape, np.uint8)
        gss = d.get(pss, (n_rows,), np.float32)
        gws = d.get(pws, (n_rows,), np.float32)
    check_rounded(y, dt, y_pre, what="rms_norm fp8 out")
    # squares of fp8 values are exact in fp32: the sum is bounded by gamma(depth) * sum
    check_f32(gss, ss, rel=0.0, floor=gamma(rms_ws_depth(dt, n_cols)) * ss, what="rms_norm fp8 sum of squares")
    assert np.array_equal(gws, sentinel)


def test_rms_norm_fwd_fp8_unaligned(hdl):
    """X off 16-byte alignment takes the element path"""
    from dataflow_lib_amd import api
    dt, n_rows, n_cols = FP8E4M3, 9, 4096
    X, W = rms_inputs(dt, n_rows, n_cols, seed=5)
    y_pre = np.empty((n_rows, n_cols))
    assert oracle().oracle_rms_norm(dt, n_rows, n_cols, 1e-6, ptr(W), ptr(X), ptr(y_pre), None, None, None) == 0
    with Dev(hdl) as d:
        px, pw, py = d.put(X, offset_bytes=3), d.put(W), d.empty(X.nbytes)
        assert api.submit_rms_norm(hdl, 0, dt, n_rows, n_cols, 1e-6, pw, px, py, None, None) == 0
        y = d.get(py, X.shape, np.uint8)
    check_rounded(y, dt, y_pre, what="rms_norm fp8 unaligned out")


def rms_bwd_inputs(fdt, bdt, n_rows, n_cols, seed=11):
    X, W = rms_inputs(fdt, n_rows, n_cols, seed)
    ws, rs = np.empty(n_rows), np.empty(n_rows)
    assert oracle().oracle_rms_norm(fdt, n_rows, n_cols, 1e-5, ptr(W), ptr(X), None, ptr(ws), ptr(rs), None) == 0
    dY = to_storage(normal(seed + 2, (n_rows, n_cols)), bdt)
    dX = to_storage(normal(seed + 3, (n_rows, n_cols)), bdt)
    return X, W, ws.astype(np.float32), rs.astype(np.float32), dY, dX


MIXED = [(f, b) for f in F8 for b in B16]
MIXED_IDS = ["%s_%s" % (IDS[f], IDS[b]) for f, b in MIXED]
# (32, 16384): the widest rows of the chunked path (TPR 1024); (6, 16392): one chunk past it
BWD_SHAPES = [(16, 4096), (7, 8192), (33, 1000), (5, 8), (3, 20000), (8192, 4096), (5, 4099), (1024, 8192), (32, 16384),
              (6, 16392)]


@pytest.mark.parametrize("fb", MIXED, ids=MIXED_IDS)
@pytest.mark.parametrize("shape", BWD_SHAPES, ids=lambda s: "%dx%d" % s)
def test_rms_norm_bwd_x_fp8(hdl, fb, shape):
    from dataflow_lib_amd import api
    fdt, bdt = fb
    n_rows, n_cols = shape
    X, W, ws, rs, dY, dX = rms_bwd_inputs(fdt, bdt, n_rows, n_cols)
    lo, hi = np.empty((n_rows, n_cols)), np.empty((n_rows, n_cols))
    assert oracle().oracle_rms_norm_bwd_x2(fdt, bdt, n_rows, n_cols, ptr(ws), ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX),
                                           ptr(lo), ptr(hi)) == 0
    with Dev(hdl) as d:
        p = [d.put(a) for a in (ws, rs, W, X, dY, dX)]
        assert api.submit_rms_norm_bwd_x(hdl, 0, fdt, bdt, n_rows, n_cols, 1e-5, *p) == 0
        out = d.get(p[5], X.shape, NP_STORAGE[bdt])
    check_rounded(out, bdt, lo, hi, what="rms_norm_bwd_x fp8 dX")


@pytest.mark.parametrize("fb", MIXED, ids=MIXED_IDS)
@pytest.mark.parametrize("shape", BWD_SHAPES + [(300, 512)], ids=lambda s: "%dx%d" % s)
def test_rms_norm_bwd_w_fp8(hdl, fb, shape):
    from dataflow_lib_amd import api
    fdt, bdt = fb
    n_rows, n_cols = shape
    X, W, ws, rs, dY, _ = rms_bwd_inputs(fdt, bdt, n_rows, n_cols)
    dW = to_storage(normal(21, (n_cols,), std=0.1), bdt)
    pre, absum = np.empty(n_cols), np.empty(n_cols)
    assert oracle().oracle_rms_norm_bwd_w2(fdt, bdt, bdt, n_rows, n_cols, ptr(rs), ptr(X), ptr(dY), ptr(dW), ptr(pre),
                                           ptr(absum)) == 0
    with Dev(hdl) as d:
        prs, px, pdy, pdw = d.put(rs), d.put(X), d.put(dY), d.put(dW)
        assert api.submit_rms_norm_bwd_w(hdl, 0, fdt, bdt, n_rows, n_cols, 1e-5, prs, px, pdy, pdw) == 0
        out = d.get(pdw, (n_cols,), NP_STORAGE[bdt])
        # a second call on the same inputs gives the same bits (fixed-order reduction)
        pdw2 = d.put(dW)
        assert api.submit_rms_norm_bwd_w(hdl, 0, fdt, bdt, n_rows, n_cols, 1e-5, prs, px, pdy, pdw2) == 0
        out2 = d.get(pdw2, (n_cols,), NP_STORAGE[bdt])
    floor = gamma(rms_dw_fp8_depth(n_rows, n_cols, hdl.device_info.cu_count)) * absum
    check_rounded(out, bdt, pre, floor=floor, what="rms_norm_bwd_w fp8 dW")
    assert np.array_equal(out.view(np.uint16), out2.view(np.uint16))


def test_rms_norm_bwd_w_fp8_too_wide_is_refused(hdl):
    """a row whose fp32 LDS accumulator exceeds the workgroup's LDS is an error, not a launch"""
    from dataflow_lib_amd import api
    n_cols = hdl.device_info.max_smem_per_block // 4 + 8
    with Dev(hdl) as d:
        p = d.empty(4 * n_cols)
        assert api.submit_rms_norm_bwd_w(hdl, 0, FP8E4M3, BF16, 1, n_cols, 1e-5, p, p, p, p) == -1


# ---------------- RoPE ----------------

ROPE_CASES = [(8192, 32, 8, 128, 500000), (256, 64, 8, 128, 500000), (64, 32, 8, 128, 500000), (17, 4, 2, 64, 10000),
              (9, 8, 2, 256, 10000), (9, 3, 1, 96, 500000),
              (5, 2, 2, 6, 10000), (3, 2, 0, 128, 500000)]


@pytest.mark.parametrize("dt", F8, ids=dt_id)
@pytest.mark.parametrize("case", ROPE_CASES, ids=lambda c: "T%d_q%d_kv%d_hd%d" % c[:4])
def test_rope_fp8(hdl, dt, case):
    from dataflow_lib_amd import api
    T, nq, nkv, hd, theta = case
    Q = to_storage(normal(51, (T, nq * hd)), dt)
    K = to_storage(normal(52, (T, nkv * hd)), dt)
    pos = rng(53).integers(0, 2048, size=T).astype(np.int32)
    pos[0] = 0
    if T > 2:
        pos[-1] = 131071
    N = T * nq * hd
    qv, kv = np.empty(Q.shape), np.empty(K.shape)
    assert oracle().oracle_rope(dt, 0, N, nq * hd, hd, nkv, theta, ptr(pos), ptr(Q), ptr(K), ptr(qv), ptr(kv)) == 0
    with Dev(hdl) as d:
        pq, pk, pp = d.put(Q), d.put(K), d.put(pos)
        assert api.submit_rope(hdl, 0, dt, N, nq * hd, hd, nkv, theta, pp, pq, pk) == 0
        gq = d.get(pq, Q.shape, np.uint8)
        gk = d.get(pk, K.shape, np.uint8)
    check_rounded(gq, dt, qv, what="rope fp8 Q")
    if K.size:
        check_rounded(gk, dt, kv, what="rope fp8 K")


ROPE_F8_LARGE_STD = {FP8E4M3: 100.0, FP8E5M2: 1.0e4}


@pytest.mark.parametrize("dt", F8, ids=dt_id)
def test_rope_fp8_large_magnitudes(hdl, dt):
    """fp8 inputs spread over the format's range (E4M3 up to its 448
    saturation, E5M2 std 1e4): the plain fp32 rotation the fp8 kernels use
    stays within one fp8 ulp of the exact result, plus the fp32 evaluation
    floor (rope_pair_floor) where the two products cancel, which in E5M2's
    subnormal range is wider than an ulp"""
    from dataflow_lib_amd import api
    T, nq, nkv, hd, theta = 256, 32, 8, 128, 500000
    Q = to_storage(normal(771, (T, nq * hd), std=ROPE_F8_LARGE_STD[dt]), dt)
    K = to_storage(normal(772, (T, nkv * hd), std=ROPE_F8_LARGE_STD[dt]), dt)
    pos = rng(773).integers(0, 131072, size=T).astype(np.int32)
    N = T * nq * hd
    qv, kv = np.empty(Q.shape), np.empty(K.shape)
    assert oracle().oracle_rope(dt, 0, N, nq * hd, hd, nkv, theta, ptr(pos), ptr(Q), ptr(K), ptr(qv), ptr(kv)) == 0
    with Dev(hdl) as d:
        pq, pk, pp = d.put(Q), d.put(K), d.put(pos)
        assert api.submit_rope(hdl, 0, dt, N, nq * hd, hd, nkv, theta, pp, pq, pk) == 0
        gq = d.get(pq, Q.shape, np.uint8)
        gk = d.get(pk, K.shape, np.uint8)
    check_rounded(gq, dt, qv, floor=rope_pair_floor(to_f64(Q, dt), nq * hd), what="rope fp8 Q, large magnitudes")
    check_rounded(gk, dt, kv, floor=rope_pair_floor(to_f64(K, dt), nkv * hd), what="rope fp8 K, large magnitudes")


def test_rope_bwd_has_no_fp8_variant(hdl):
    from dataflow_lib_amd import api
    with Dev(hdl) as d:
        p = d.empty(256)
        assert api.submit_rope_bwd_x(hdl, 0, FP8E4M3, 128, 128, 128, 0, 500000, p, p, p) == -1


# ---------------- SwiGLU ----------------

SWIGLU_SHAPES = [(33, 1000), (8, 14336), (1, 7), (3, 5), (1024, 14336), (5, 1003), (64, 28672)]


def swiglu_inputs(fdt, bdt, shape, seed):
    g = to_storage(normal(seed, shape, std=2.0), fdt)
    u = to_storage(normal(seed + 1, shape), fdt)
    dO = to_storage(normal(seed + 2, shape), bdt) if bdt else None
    if shape[1] > 12:
        vals = np.array([0.0, -0.0, 88.0, -88.0, -89.0, 100.0, -100.0, 448.0, -448.0, -1.2785, 30.0, -30.0], np.float32)
        g.ravel()[:vals.size] = to_storage(vals, fdt)
    return g, u, dO


@pytest.mark.parametrize("dt", F8, ids=dt_id)
@pytest.mark.parametrize("shape", SWIGLU_SHAPES, ids=lambda s: "%dx%d" % s)
def test_swiglu_fwd_fp8(hdl, dt, shape):
    from dataflow_lib_amd import api
    g, u, _ = swiglu_inputs(dt, None, shape, 71)
    pre = np.empty(shape)
    assert oracle().oracle_swiglu(dt, g.size, ptr(g), ptr(u), ptr(pre)) == 0
    with Dev(hdl) as d:
        off = 3 if shape == (5, 1003) else 0
        pg, pu, po = d.put(g, offset_bytes=off), d.put(u), d.empty(g.nbytes)
        assert api.submit_swiglu(hdl, 0, dt, shape[0], shape[1], pg, pu, po) == 0
        out = d.get(po, shape, np.uint8)
    check_rounded(out, dt, pre, what="swiglu fp8 out")


@pytest.mark.parametrize("fb", MIXED, ids=MIXED_IDS)
@pytest.mark.parametrize("shape", SWIGLU_SHAPES, ids=lambda s: "%dx%d" % s)
def test_swiglu_bwd_fp8(hdl, fb, shape):
    from dataflow_lib_amd import api
    fdt, bdt = fb
    g, u, dO = swiglu_inputs(fdt, bdt, shape, 81)
    dg, dgf, du = np.empty(shape), np.empty(shape), np.empty(shape)
    assert oracle().oracle_swiglu_bwd2(fdt, bdt, g.size, ptr(g), ptr(u), ptr(dO), ptr(dg), ptr(dgf), ptr(du)) == 0
    with Dev(hdl) as d:
        off = 3 if shape == (5, 1003) else 0
        pg, pu, pd = d.put(g, offset_bytes=off), d.put(u), d.put(dO)
        pdg, pdu = d.empty(2 * g.size), d.empty(2 * g.size)
        assert api.submit_swiglu_bwd_x(hdl, 0, fdt, bdt, shape[0], shape[1], pg, pu, pd, pdg, pdu) == 0
        gdg, gdu = d.get(pdg, shape, NP_STORAGE[bdt]), d.get(pdu, shape, NP_STORAGE[bdt])
    check_rounded(gdu, bdt, du, what="swiglu fp8 dU")
    check_rounded(gdg, bdt, dg, floor=dgf, what="swiglu fp8 dG")


# ---------------- softmax ----------------

# rows of 32768..131072 columns (a multiple of 16) take the path that prefetches
# the next row: (300, 32768), (520, 65552), (260, 128256) and (1100, 128256)
# give workgroups several rows each (more rows than CUs; four or five in the
# last), 65552 leaves two 8-byte pieces in the register half, (2, 131072) is
# the longest such row
SMX_SHAPES = [(4, 128256), (3, 1000), (2, 1001), (2, 140000), (5, 64), (1, 1), (7, 4104),
              (300, 32768), (520, 65552), (260, 128256), (2, 131072), (5, 65536), (1100, 128256)]
# logits placed off 16-byte alignment: the element-wise loop (for (5, 65536),
# with the long-row path's workgroup size)
SMX_UNALIGNED = ((2, 1001), (5, 65536))


@pytest.mark.parametrize("fb", MIXED, ids=MIXED_IDS)
@pytest.mark.parametrize("shape", SMX_SHAPES, ids=lambda s: "%dx%d" % s)
def test_softmax_fp8(hdl, fb, shape):
    """fp8 logits, fp16 / bf16 probabilities; x - max is taken in the output type"""
    from dataflow_lib_amd import api
    fdt, bdt = fb
    n_rows, n_cols = shape
    x = normal(101, shape, std=2.0)
    if n_cols >= 16:
        x[0, 3] = -np.inf          # E4M3 saturates it to -448
        x[-1, 5] = 30.0
    X = to_storage(x, fdt)
    pre = np.empty(shape)
    assert oracle().oracle_softmax(fdt, bdt, n_rows, n_cols, ptr(X), ptr(pre)) == 0
    with Dev(hdl) as d:
        off = 5 if shape in SMX_UNALIGNED else 0
        px, po = d.put(X, offset_bytes=off), d.empty(2 * X.size)
        assert api.submit_softmax(hdl, 0, fdt, bdt, n_rows, n_cols, px, po) == 0
        out = d.get(po, shape, NP_STORAGE[bdt])
    check_rounded(out, bdt, pre, what="softmax fp8")
    assert np.allclose(to_f64(out, bdt).sum(axis=1), 1.0, atol=2e-2)


@pytest.mark.parametrize("fb", MIXED, ids=MIXED_IDS)
@pytest.mark.parametrize("shape", [(300, 32768), (600, 4104)], ids=lambda s: "%dx%d" % s)
def test_softmax_fp8_special_rows(hdl, fb, shape):
    """workgroups walking several rows (the prefetching path and the
    two-workgroup path) through an all -inf row, a row with +inf and one with
    NaN (E4M3 has no infinities: they saturate to -448 / 448)"""
    from dataflow_lib_amd import api
    fdt, bdt = fb
    n_rows, n_cols = shape
    x = normal(103, shape, std=2.0)
    x[1, :] = -np.inf
    x[n_rows // 2, 17] = np.inf
    x[n_rows - 3, n_cols - 1] = np.nan
    x[4, ::3] = -np.inf
    X = to_storage(x, fdt)
    pre = np.empty(shape)
    assert oracle().oracle_softmax(fdt, bdt, n_rows, n_cols, ptr(X), ptr(pre)) == 0
    with Dev(hdl) as d:
        px, po = d.put(X), d.empty(2 * X.size)
        assert api.submit_softmax(hdl, 0, fdt, bdt, n_rows, n_cols, px, po) == 0
        out = d.get(po, shape, NP_STORAGE[bdt])
    check_rounded(out, bdt, pre, what="softmax fp8, special rows")
    assert np.isnan(to_f64(out, bdt)[n_rows - 3]).all()


def test_softmax_fp8_on_two_streams_matches_one_stream(hdl):
    """The fp8 softmax's long-row path hands rows out from the same counter in
    the code object as the 16-bit fused loss op (and counts finished
    workgroups there), so the handle orders the two across its streams: the
    two ops alternating between streams without waits, with more rows than
    two per workgroup so that both take tickets, give the same bits as the
    same launches on one stream, and the fp8 probabilities match the oracle."""
    from dataflow_lib_amd import api
    from test_hip_ops import logits
    fdt, bdt = FP8E4M3, BF16
    ce_shape, sm_shape = (600, 32000), (600, 65552)
    Xc = logits(BF16, ce_shape, seed=160)
    lab = rng(161).integers(0, ce_shape[1], size=ce_shape[0]).astype(np.uint32)
    Xs = to_storage(normal(162, sm_shape, std=2.0), fdt)
    outs = []
    for two_streams in (False, True):
        with Dev(hdl) as d:
            pc, pl, ploss, pmean = d.put(Xc), d.put(lab), d.empty(4 * ce_shape[0]), d.empty(4)
            ps, po = d.put(Xs), d.empty(2 * Xs.size)
            hdl.sync()
            for rnd in range(3):
                if rnd > 0:
                    hdl.sync()
                    hdl.to_device(np.ascontiguousarray(Xc), pc)   # fresh logits (the loss op works in place)
                assert api.submit_softmax_cross_entropy_loss(hdl, 0, BF16, ce_shape[0], ce_shape[1], pc, pl, ploss, pmean) == 0
                assert api.submit_softmax(hdl, 1 if two_streams else 0, fdt, bdt, sm_shape[0], sm_shape[1], ps, po) == 0
            hdl.sync()
            outs.append([d.get(pc, ce_shape, np.uint16), d.get(ploss, (ce_shape[0],), np.float32),
                         d.get(pmean, (1,), np.float32), d.get(po, sm_shape, NP_STORAGE[bdt])])
    for r, g in zip(outs[0], outs[1]):
        assert np.array_equal(r.view(np.uint8), g.view(np.uint8))
    pre = np.empty(sm_shape)
    assert oracle().oracle_softmax(fdt, bdt, sm_shape[0], sm_shape[1], ptr(Xs), ptr(pre)) == 0
    check_rounded(outs[1][3], bdt, pre, what="softmax fp8 on two streams")


@pytest.mark.parametrize("fb", [(FP8E4M3, BF16), (FP8E5M2, FP16)], ids=["e4m3_bf16", "e5m2_fp16"])
def test_rms_norm_bwd_w_fp8_on_two_streams_matches_one_stream(hdl, fb):
    """The fp8 dW ops keep their partial rows in the same module scratch as the
    16-bit ones, so the handle must order them across streams too: a large
    fp8 bwd_w on stream 0 followed at once by a small one on stream 1, and a
    16-bit fused backward on stream 0 followed by a small fp8 bwd_w on
    stream 1, give the same bits as the same launches one after the other."""
    from dataflow_lib_amd import api
    fdt, bdt = fb
    big, small = (8192, 4096), (64, 4096)
    Xb, Wb, wsb, rsb, dYb, _ = rms_bwd_inputs(fdt, bdt, big[0], big[1], seed=71)
    Xs, Ws, wss, rss, dYs, _ = rms_bwd_inputs(fdt, bdt, small[0], small[1], seed=72)
    # a 16-bit fused backward of the big shape (bdt inputs)
    X16 = to_storage(normal(73, big), bdt)
    W16 = to_storage(1.0 + normal(74, (big[1],), std=0.02), bdt)
    dY16 = to_storage(normal(75, big), bdt)
    rs16 = (1.0 + 0.01 * normal(76, (big[0],))).astype(np.float32)

    def run(first_fused, stream_small):
        with Dev(hdl) as d:
            if first_fused:
                pa = [d.put(a) for a in (rs16, W16, X16, dY16, np.zeros(big, NP_STORAGE[bdt]))] + [d.put(np.zeros(big[1], np.float32))]
            else:
                pa = [d.put(a) for a in (rsb, Xb, dYb)] + [d.put(np.zeros(big[1], NP_STORAGE[bdt]))]
            pb = [d.put(a) for a in (rss, Xs, dYs)] + [d.put(np.zeros(small[1], NP_STORAGE[bdt]))]
            hdl.sync()
            if first_fused:
                assert api.submit_rms_norm_bwd(hdl, 0, bdt, bdt, big[0], big[1], 1e-5, *pa) == 0
                out_a = (pa[5], (big[1],), np.float32)
            else:
                assert api.submit_rms_norm_bwd_w(hdl, 0, fdt, bdt, big[0], big[1], 1e-5, *pa) == 0
                out_a = (pa[3], (big[1],), NP_STORAGE[bdt])
            if stream_small == 0:
                hdl.sync()
            assert api.submit_rms_norm_bwd_w(hdl, stream_small, fdt, bdt, small[0], small[1], 1e-5, *pb) == 0
            return d.get(*out_a), d.get(pb[3], (small[1],), NP_STORAGE[bdt])

    for first_fused in (False, True):
        ref, two = run(first_fused, 0), run(first_fused, 1)
        for r, g in zip(ref, two):
            assert np.array_equal(r.view(np.uint8), g.view(np.uint8))
