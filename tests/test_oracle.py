"""Pins the C oracle (oracle/liboracle.so) before it is trusted as the checker.

The reference publishes no golden vectors for these kernels and its tests
assert nothing, so each oracle function is pinned by what the mathematics
fixes, chosen so a dropped term, a wrong sign or a swapped operand fails:
  rounding      - ties-to-even cases, grid membership, idempotence, fp32-bit RNE
  rms_norm      - constant / zero rows, mean-square identity, numpy dot for ws
  bwd (exact)   - central finite differences of the oracle's own forward
  bwd_x (ref)   - equals the exact gradient when dY is constant along a row
  bwd_w         - finite differences w.r.t. W
  rope          - position 0 identity, c = 0 closed form, pair norms, bwd(fwd(x)) = x,
                  2x2 rotation-matrix brute force
  swiglu        - g = 0 values, finite differences, large-g limit
  softmax / CE  - scipy softmax / logsumexp, constant rows, the bf16 rounding of
                  x - max on a hand-computed row, label arithmetic
"""
import numpy as np
import pytest
from scipy.special import logsumexp, softmax as sp_softmax

from support import BF16, FP16, FP32, bf16_bits_to_f32, f32_to_bf16_bits, normal, oracle, ptr, rng, to_f64, to_storage

O = None


def setup_module():
    global O
    O = oracle()


# ---------------- rounding ----------------

def test_round_ties_to_even_and_subnormals():
    r = lambda v, dt: O.oracle_round(v, dt)
    # bf16 has 8 significant bits: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert r(1.0 + 2 ** -8, BF16) == 1.0
    assert r(1.0 + 3 * 2 ** -8, BF16) == 1.0 + 2 ** -6
    assert r(1.0 + 2 ** -8 + 2 ** -30, BF16) == 1.0 + 2 ** -7
    assert r(-(1.0 + 2 ** -8), BF16) == -1.0
    # fp16: 11 bits; fp32: 24 bits
    assert r(1.0 + 2 ** -11, FP16) == 1.0 and r(1.0 + 3 * 2 ** -11, FP16) == 1.0 + 2 ** -9
    assert r(1.0 + 2 ** -24, FP32) == 1.0 and r(1.0 + 3 * 2 ** -24, FP32) == 1.0 + 2 ** -22
    # subnormal spacing: bf16 2^-133, fp16 2^-24; halfway ties go to the even multiple
    assert r(1.5 * 2 ** -133, BF16) == 2 * 2 ** -133 and r(2.5 * 2 ** -133, BF16) == 2 * 2 ** -133
    assert r(2.5 * 2 ** -24, FP16) == 2 * 2 ** -24 and r(0.4 * 2 ** -24, FP16) == 0.0
    # overflow
    assert r(65520.0, FP16) == np.inf and r(65519.0, FP16) == 65504.0
    assert np.isinf(r(3.4e38 * 1.01, BF16))


def test_round_matches_independent_conversions():
    g = rng(1)
    v = np.concatenate([g.standard_normal(2000) * 10.0 ** g.integers(-30, 30, 2000),
                        g.standard_normal(500) * 1e-40, g.standard_normal(500) * 60000])
    # values beyond the fp16 range round to inf on both sides (numpy warns on that cast)
    with np.errstate(over="ignore"):
        for x in v:
            assert O.oracle_round(x, FP32) == float(np.float32(x))
            assert O.oracle_round(x, FP16) == float(np.float16(x))
    # bf16 of fp32-representable values: integer RNE on the fp32 bit pattern
    f = v.astype(np.float32)
    f = f[np.isfinite(f)]
    want = bf16_bits_to_f32(f32_to_bf16_bits(f)).astype(np.float64)
    got = np.array([O.oracle_round(float(x), BF16) for x in f])
    assert np.array_equal(got, want)


def test_round_is_on_grid_nearest_and_idempotent():
    g = rng(2)
    for x in g.standard_normal(3000) * 10.0 ** g.integers(-20, 20, 3000):
        b = O.oracle_round(x, BF16)
        assert O.oracle_round(b, BF16) == b
        assert (np.float32(b).view(np.uint32) & 0xFFFF) == 0
        assert abs(b - x) <= 0.5 * O.oracle_ulp(x, BF16) * (1 + 1e-12)


# ---------------- RMSNorm ----------------

def rmsf(dt, X, W, eps):
    n_rows, n_cols = X.shape
    y, ws, rs, wa = np.empty(X.shape), np.empty(n_rows), np.empty(n_rows), np.empty(n_rows)
    assert O.oracle_rms_norm(dt, n_rows, n_cols, eps, ptr(W), ptr(X), ptr(y), ptr(ws), ptr(rs), ptr(wa)) == 0
    return y, ws, rs


def test_rms_norm_closed_forms():
    n, eps = 64, 1e-5
    X = np.zeros((3, n), np.float32)
    X[0] = 0.75
    X[2] = normal(3, (n,))
    W = (1 + normal(4, (n,), std=0.1)).astype(np.float32)
    y, ws, rs = rmsf(FP32, X, W, eps)
    e32 = float(np.float32(eps))     # eps is an fp32 kernel argument
    assert np.allclose(y[0], W.astype(np.float64) * 0.75 / np.sqrt(0.75 ** 2 + e32), rtol=1e-14)
    assert np.all(y[1] == 0) and rs[1] == pytest.approx(1 / np.sqrt(e32), rel=1e-14)
    assert ((y[2] / W.astype(np.float64)) ** 2).mean() == pytest.approx(1 - e32 * rs[2] ** 2, rel=1e-12)
    assert ws[2] == pytest.approx(np.dot(X[2].astype(np.float64), W.astype(np.float64)), rel=1e-12)
    # bf16 storage reads the same numbers
    yb, _, rsb = rmsf(BF16, to_storage(X, BF16), to_storage(W, BF16), eps)
    assert rsb[0] == pytest.approx(rs[0], rel=1e-14)


def fd_grad(f, x, h=1e-3):
    """central differences of scalar f over every element of the fp32 array x"""
    g = np.empty(x.shape)
    flat = x.ravel()
    for i in range(flat.size):
        orig = flat[i]
        xp, xm = np.float32(orig + h), np.float32(orig - h)
        flat[i] = xp
        fp = f()
        flat[i] = xm
        fm = f()
        flat[i] = orig
        g.flat[i] = (fp - fm) / (np.float64(xp) - np.float64(xm))
    return g


def test_rms_norm_bwd_exact_matches_finite_differences():
    n_rows, n_cols, eps = 3, 16, 1e-5
    X = normal(5, (n_rows, n_cols))
    W = (1 + normal(6, (n_cols,), std=0.3)).astype(np.float32)
    dY = normal(7, (n_rows, n_cols))
    L = lambda: float((rmsf(FP32, X, W, eps)[0] * dY).sum())
    gx, gw = fd_grad(L, X), fd_grad(L, W)
    _, _, rs = rmsf(FP32, X, W, eps)
    dx, dxf, dw, dwa = np.empty(X.shape), np.empty(X.shape), np.empty(n_cols), np.empty(n_cols)
    zeros = np.zeros_like(X)
    assert O.oracle_rms_norm_bwd(FP32, n_rows, n_cols, ptr(rs.astype(np.float32)), ptr(W), ptr(X), ptr(dY), ptr(zeros),
                                 ptr(np.zeros(n_cols, np.float32)), ptr(dx), ptr(dxf), ptr(dw), ptr(dwa)) == 0
    assert np.allclose(dx, gx, rtol=2e-5, atol=2e-6)
    assert np.allclose(dw, gw, rtol=2e-5, atol=2e-6)
    # bwd_w alone gives the same dW
    dw2, dwa2 = np.empty(n_cols), np.empty(n_cols)
    assert O.oracle_rms_norm_bwd_w(FP32, FP32, n_rows, n_cols, ptr(rs.astype(np.float32)), ptr(X), ptr(dY),
                                   ptr(np.zeros(n_cols, np.float32)), ptr(dw2), ptr(dwa2)) == 0
    assert np.allclose(dw2, gw, rtol=2e-5, atol=2e-6)


def test_rms_norm_bwd_x_reference_formula():
    """with dY constant along each row, the reference's bwd_x formula equals the exact gradient;
    with a non-constant dY it does not (it is not the gradient, by design of the reference)"""
    n_rows, n_cols, eps = 3, 16, 1e-5
    X = normal(8, (n_rows, n_cols))
    W = (1 + normal(9, (n_cols,), std=0.3)).astype(np.float32)
    _, ws, rs = rmsf(FP32, X, W, eps)
    for const in (True, False):
        dY = np.repeat(normal(10, (n_rows, 1)), n_cols, axis=1) if const else normal(11, (n_rows, n_cols))
        L = lambda: float((rmsf(FP32, X, W, eps)[0] * dY).sum())
        gx = fd_grad(L, X)
        lo, hi = np.empty(X.shape), np.empty(X.shape)
        assert O.oracle_rms_norm_bwd_x(FP32, n_rows, n_cols, ptr(ws.astype(np.float32)), ptr(rs.astype(np.float32)),
                                       ptr(W), ptr(X), ptr(dY), ptr(np.zeros_like(X)), ptr(lo), ptr(hi)) == 0
        assert np.allclose(lo, gx, rtol=1e-4, atol=1e-5) == const
        assert np.all(np.abs(hi - lo) <= 1e-6 * (1 + np.abs(lo)))


def test_rms_norm_bwd_x_half_precision_chain_brackets_fp32():
    """the bf16 chain rounds deriv, the product and the sum: its value stays
    within those three roundings of the fp32 result and dX_in carries through"""
    n_rows, n_cols = 2, 32
    X = to_storage(normal(12, (n_rows, n_cols)), BF16)
    W = to_storage(1 + normal(13, (n_cols,), std=0.1), BF16)
    dY = to_storage(normal(14, (n_rows, n_cols)), BF16)
    dX = to_storage(normal(15, (n_rows, n_cols)), BF16)
    _, ws, rs = rmsf(BF16, X, W, 1e-5)
    args = [ptr(ws.astype(np.float32)), ptr(rs.astype(np.float32)), ptr(W), ptr(X), ptr(dY), ptr(dX)]
    lo, hi = np.empty((n_rows, n_cols)), np.empty((n_rows, n_cols))
    assert O.oracle_rms_norm_bwd_x(BF16, n_rows, n_cols, *args, ptr(lo), ptr(hi)) == 0
    xf, wf, gf, df = (to_f64(a, BF16) for a in (X, W, dY, dX))
    deriv = wf * rs[:, None] - (xf * rs[:, None] ** 3 / n_cols) * ws[:, None]
    exact = df + gf * deriv
    bound = np.abs(gf) * np.abs(deriv) * 2 ** -7 + np.abs(gf * deriv) * 2 ** -8
    assert np.all(np.abs(lo - exact) <= bound + 1e-12)


# ---------------- RoPE ----------------

def rope(dt, bwd, Q, K, pos, hd, nkv, theta):
    T = Q.shape[0]
    qv, kv = np.empty(Q.shape), np.empty(K.shape)
    assert O.oracle_rope(dt, bwd, Q.size, Q.shape[1], hd, nkv, theta, ptr(pos), ptr(Q), ptr(K), ptr(qv), ptr(kv)) == 0
    return qv, kv


def test_rope_closed_forms():
    hd, nq, nkv, theta = 8, 2, 1, 10000
    T = 4
    Q, K = normal(20, (T, nq * hd)), normal(21, (T, nkv * hd))
    pos = np.array([0, 1, 7, 1000], np.int32)
    qv, kv = rope(FP32, 0, Q, K, pos, hd, nkv, theta)
    assert np.array_equal(qv[0], Q[0].astype(np.float64)) and np.array_equal(kv[0], K[0].astype(np.float64))
    # pair column 0 of each head turns by exactly (float) pos radians (angle = theta^0 = 1)
    for t in range(T):
        c, s = np.float32(np.cos(np.float64(np.float32(pos[t])))), np.float32(np.sin(np.float64(np.float32(pos[t]))))
        for h in range(nq):
            e, o = np.float64(Q[t, h * hd]), np.float64(Q[t, h * hd + 1])
            assert qv[t, h * hd] == pytest.approx(c * e - s * o, rel=1e-15, abs=1e-15)
            assert qv[t, h * hd + 1] == pytest.approx(c * o + s * e, rel=1e-15, abs=1e-15)
    # pair norms are preserved
    n0 = Q.astype(np.float64).reshape(T, -1, 2)
    n1 = qv.reshape(T, -1, 2)
    assert np.allclose((n1 ** 2).sum(-1), (n0 ** 2).sum(-1), rtol=1e-6)


def test_rope_bruteforce_rotation_matrix_and_inverse():
    hd, nq, nkv, theta = 4, 1, 1, 10000
    Q, K = normal(22, (3, hd)), normal(23, (3, hd))
    pos = np.array([3, 17, 250], np.int32)
    qv, _ = rope(FP32, 0, Q, K, pos, hd, nkv, theta)
    for t in range(3):
        for p in range(hd // 2):
            ang = np.float32(np.power(np.float64(theta), np.float64(np.float32(-(np.float32(2 * p) / np.float32(hd))))))
            arg = np.float32(np.float32(pos[t]) * ang)
            c, s = np.float32(np.cos(np.float64(arg))), np.float32(np.sin(np.float64(arg)))
            R = np.array([[c, -s], [s, c]], np.float64)
            want = R @ Q[t, 2 * p:2 * p + 2].astype(np.float64)
            assert np.allclose(qv[t, 2 * p:2 * p + 2], want, rtol=1e-14, atol=1e-14)
    # backward applies the transpose: bwd(fwd(x)) = x up to the fp32 storage of fwd(x)
    q1 = qv.astype(np.float32)
    k1 = np.zeros_like(K)
    back, _ = rope(FP32, 1, q1, k1, pos, hd, nkv, theta)
    assert np.allclose(back, Q, rtol=1e-6, atol=1e-6)


def textbook_rope(X, pos, hd, theta, inverse=False):
    """RoFormer rotation in fp64 of every head of X [T x heads*hd]: pair
    (2p, 2p+1) turns by pos * theta^(-2p/hd), with the angle, the position and
    their product rounded to fp32 the way the reference forms them
    (attention/rope.cu:26-33) and cos/sin rounded to fp32; written from the
    formula, independently of the oracle's indexing."""
    T, width = X.shape
    out = np.empty((T, width), np.float64)
    for t in range(T):
        for j in range(0, width, 2):
            p = (j % hd) // 2
            ang = np.float32(np.power(np.float64(theta), np.float64(np.float32(-(np.float32(2 * p) / np.float32(hd))))))
            arg = np.float32(np.float32(pos[t]) * ang)
            c, s = np.float64(np.float32(np.cos(np.float64(arg)))), np.float64(np.float32(np.sin(np.float64(arg))))
            if inverse:
                s = -s
            e, o = np.float64(X[t, j]), np.float64(X[t, j + 1])
            out[t, j], out[t, j + 1] = c * e - s * o, c * o + s * e
    return out


def test_rope_k_rows_against_textbook_rotation():
    """The K path on its own row width: fewer K heads than Q heads (kv_dim !=
    model_dim), several tokens and positions other than 0, so a K row
    addressed with Q's row width, or a K head given Q's table, fails."""
    hd, nq, nkv, theta = 16, 4, 2, 500000
    pos = np.array([0, 1, 5, 77, 2047, 123456], np.int32)
    T = pos.size
    Q, K = normal(24, (T, nq * hd)), normal(25, (T, nkv * hd))
    for bwd in (0, 1):
        qv, kv = rope(FP32, bwd, Q, K, pos, hd, nkv, theta)
        assert np.allclose(qv, textbook_rope(Q, pos, hd, theta, inverse=bool(bwd)), rtol=1e-14, atol=1e-14)
        assert np.allclose(kv, textbook_rope(K, pos, hd, theta, inverse=bool(bwd)), rtol=1e-14, atol=1e-14)
        # every K pair keeps its length
        n0 = (K.astype(np.float64).reshape(T, -1, 2) ** 2).sum(-1)
        assert np.allclose((kv.reshape(T, -1, 2) ** 2).sum(-1), n0, rtol=1e-6)
    # bwd(fwd(K)) = K up to the fp32 storage of fwd(K), on K rows alone
    _, kv = rope(FP32, 0, Q, K, pos, hd, nkv, theta)
    _, back = rope(FP32, 1, Q, kv.astype(np.float32), pos, hd, nkv, theta)
    assert np.allclose(back, K, rtol=1e-6, atol=1e-6)
    # bf16 K: the oracle's pre-rounding values are the fp64 rotation of the
    # bf16 inputs
    Kb = to_storage(K, BF16)
    _, kvb = rope(BF16, 0, to_storage(Q, BF16), Kb, pos, hd, nkv, theta)
    assert np.allclose(kvb, textbook_rope(to_f64(Kb, BF16), pos, hd, theta), rtol=1e-14, atol=1e-14)


# ---------------- SwiGLU ----------------

def sw(dt, g, u, dO):
    out, dg, dgf, du = np.empty(g.shape), np.empty(g.shape), np.empty(g.shape), np.empty(g.shape)
    assert O.oracle_swiglu(dt, g.size, ptr(g), ptr(u), ptr(out)) == 0
    assert O.oracle_swiglu_bwd(dt, g.size, ptr(g), ptr(u), ptr(dO), ptr(dg), ptr(dgf), ptr(du)) == 0
    return out, dg, du


def test_swiglu_closed_forms_and_finite_differences():
    g = np.array([0.0, 0.0, 30.0, -3.0, 1.5, -800.0], np.float32)
    u = np.array([2.0, -3.0, 1.5, 0.5, -1.25, 2.0], np.float32)
    dO = np.array([1.0, 2.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    out, dg, du = sw(FP32, g, u, dO)
    assert out[0] == 0 and du[0] == 0 and dg[0] == pytest.approx(1.0) and dg[1] == pytest.approx(3.0 * -1.0)
    assert out[2] == pytest.approx(30.0 * 1.5, rel=1e-12)
    assert np.isfinite(dg).all() and abs(dg[5]) < 1e-300
    ones = np.ones_like(g)
    gg = g[1:5].copy()
    uu = u[1:5].copy()
    fwd = lambda: float(sw(FP32, gg, uu, ones[1:5])[0].sum())
    fd = fd_grad(fwd, gg, h=1e-3)
    _, dg1, du1 = sw(FP32, gg, uu, ones[1:5])
    assert np.allclose(dg1, fd, rtol=1e-5)
    assert np.allclose(du1, sw(FP32, gg, ones[1:5], ones[1:5])[0], rtol=1e-14)


# ---------------- softmax / cross-entropy ----------------

def test_softmax_matches_scipy_and_sums_to_one():
    X = normal(30, (4, 257), std=3.0)
    y = np.empty(X.shape)
    assert O.oracle_softmax(FP32, FP32, 4, 257, ptr(X), ptr(y)) == 0
    assert np.allclose(y, sp_softmax(X.astype(np.float64), axis=1), rtol=1e-6)
    assert np.allclose(y.sum(1), 1.0, rtol=1e-14)
    c = np.full((1, 50), 2.5, np.float32)
    yc = np.empty(c.shape)
    assert O.oracle_softmax(FP32, FP32, 1, 50, ptr(c), ptr(yc)) == 0
    assert np.allclose(yc, 1 / 50, rtol=1e-15)


def test_softmax_rounds_x_minus_max_to_the_input_type():
    # max 3; 2^-8 - 3 = -2.99609375 is not a bf16 value: it rounds to -3.0
    x32 = np.array([[3.0, 2 ** -8]], np.float32)
    yb = np.empty((1, 2))
    assert O.oracle_softmax(BF16, BF16, 1, 2, ptr(to_storage(x32, BF16)), ptr(yb)) == 0
    e = np.exp(-3.0)
    assert yb[0, 0] == pytest.approx(1 / (1 + e), rel=1e-15) and yb[0, 1] == pytest.approx(e / (1 + e), rel=1e-15)
    yf = np.empty((1, 2))
    assert O.oracle_softmax(FP32, FP32, 1, 2, ptr(x32), ptr(yf)) == 0
    ef = np.exp(2 ** -8 - 3.0)
    assert yf[0, 1] == pytest.approx(ef / (1 + ef), rel=1e-12) and yf[0, 1] != yb[0, 1]


def test_cross_entropy_and_fused_loss():
    n_rows, n_cols = 5, 300
    X = to_storage(normal(31, (n_rows, n_cols), std=2.0), BF16)
    lab = np.array([0, 299, 17, 5, 400], np.uint32)   # the last is out of range
    lo, hi, loss, mean = np.empty(X.shape), np.empty(X.shape), np.empty(n_rows), np.zeros(1)
    assert O.oracle_softmax_cross_entropy(BF16, n_rows, n_cols, ptr(X), ptr(lab), ptr(lo), ptr(hi), ptr(loss), ptr(mean)) == 0
    xf = to_f64(X, BF16)
    for r in range(4):
        assert loss[r] == pytest.approx(logsumexp(xf[r]) - xf[r, lab[r]], rel=1e-13)
        assert -1.0 <= lo[r, lab[r]] <= hi[r, lab[r]] <= 0.0
        assert abs(lo[r].sum()) < 2 ** -8     # softmax - onehot sums to zero up to the label rounding
    assert np.isnan(loss[4]) and np.isnan(mean[0])
    # constant row: loss = log n; dominant label: loss -> 0
    C = to_storage(np.array([np.full(64, 1.5), np.r_[100.0, np.zeros(63)]], np.float32), BF16)
    l2 = np.empty(2)
    y2 = np.empty((2, 64))
    assert O.oracle_softmax_cross_entropy(BF16, 2, 64, ptr(C), ptr(np.array([3, 0], np.uint32)), ptr(y2), None, ptr(l2), None) == 0
    assert l2[0] == pytest.approx(np.log(64), rel=1e-14) and 0 <= l2[1] < 1e-40
    # in-place label update of the split op: P - 1 in fp32, rounded to the storage type
    P = to_storage(np.array([[0.25, 0.5], [0.125, 0.75]], np.float32), BF16)
    assert O.oracle_cross_entropy_loss(BF16, 2, 2, ptr(P), ptr(np.array([1, 7], np.uint32))) == 0
    assert np.array_equal(bf16_bits_to_f32(P), np.array([[0.25, -0.5], [0.125, 0.75]], np.float32))


def test_embedding_gathers_rows():
    """Rows that encode their own index come back as the token ids; gathering
    every id in order reproduces the table; a permutation is undone by its
    inverse; an out-of-range id is refused when the vocabulary is known."""
    O = oracle()
    vocab, dim = 50, 7
    table = (np.arange(vocab, dtype=np.float32)[:, None] * 1000 + np.arange(dim, dtype=np.float32)).astype(np.float32)
    ids = rng(200).integers(0, vocab, size=33).astype(np.uint32)
    out = np.empty((ids.size, dim), np.float32)
    assert O.oracle_embedding(4, ids.size, dim, ptr(ids), ptr(table), vocab, ptr(out)) == 0
    assert np.array_equal(np.floor(out[:, 0] / 1000).astype(np.uint32), ids)
    assert np.array_equal(out - out[:, :1], np.tile(np.arange(dim, dtype=np.float32), (ids.size, 1)))
    every = np.arange(vocab, dtype=np.uint32)
    full = np.empty_like(table)
    assert O.oracle_embedding(4, vocab, dim, ptr(every), ptr(table), vocab, ptr(full)) == 0
    assert np.array_equal(full, table)
    perm = rng(201).permutation(vocab).astype(np.uint32)
    once, back = np.empty_like(table), np.empty_like(table)
    assert O.oracle_embedding(4, vocab, dim, ptr(perm), ptr(table), vocab, ptr(once)) == 0
    assert O.oracle_embedding(4, vocab, dim, ptr(np.argsort(perm).astype(np.uint32)), ptr(once), vocab, ptr(back)) == 0
    assert np.array_equal(back, table)
    # 1- and 2-byte elements move the same bytes
    b8 = table.view(np.uint8).reshape(vocab, dim * 4)
    o8 = np.empty((ids.size, dim * 4), np.uint8)
    assert O.oracle_embedding(1, ids.size, dim * 4, ptr(ids), ptr(b8), vocab, ptr(o8)) == 0
    assert np.array_equal(o8.view(np.float32).reshape(out.shape), out)
    bad = ids.copy()
    bad[5] = vocab
    assert O.oracle_embedding(4, bad.size, dim, ptr(bad), ptr(table), vocab, ptr(out)) == -1


def test_copy_to_seq_context_places_keys_then_values():
    """Keys land at row p and values at row S + p of each token's context; no
    other row changes; reading the rows back returns the inputs."""
    O = oracle()
    kv_dim, n_tok = 6, 9
    sizes = np.array([5, 5, 5, 8, 8, 8, 8, 3, 3], np.int32)
    which = np.array([0, 0, 0, 1, 1, 1, 1, 2, 2])            # three sequences
    pos = np.array([0, 1, 4, 0, 2, 5, 7, 2, 0], np.int32)
    ctxs = [np.full((2 * s, kv_dim), -7.0, np.float32) for s in (5, 8, 3)]
    ptrs = np.array([ctxs[w].ctypes.data for w in which], np.uint64)
    K = normal(210, (n_tok, kv_dim))
    V = normal(211, (n_tok, kv_dim))
    assert O.oracle_copy_to_seq_context(4, n_tok * kv_dim, kv_dim, ptr(K), ptr(V), ptr(pos), ptr(ptrs), ptr(sizes)) == 0
    touched = [set() for _ in ctxs]
    for t in range(n_tok):
        c, S = ctxs[which[t]], sizes[t]
        assert np.array_equal(c[pos[t]], K[t]) and np.array_equal(c[S + pos[t]], V[t])
        touched[which[t]] |= {int(pos[t]), int(S + pos[t])}
    for c, tset in zip(ctxs, touched):
        for r in range(c.shape[0]):
            if r not in tset:
                assert np.all(c[r] == -7.0)
    assert O.oracle_copy_to_seq_context(4, n_tok * kv_dim + 1, kv_dim, ptr(K), ptr(V), ptr(pos), ptr(ptrs), ptr(sizes)) == -1


# ---------------- fp8 (OCP E4M3 / E5M2) ----------------

FP8E4M3, FP8E5M2 = 6, 7
FP8_MAX = {FP8E4M3: 448.0, FP8E5M2: 57344.0}


def fp8_decode_all(dt):
    codes = np.arange(256, dtype=np.uint8)
    out = np.empty(256)
    O.oracle_load(dt, ptr(codes), 256, ptr(out))
    return out


def fp8_encode(dt, vals):
    v = np.ascontiguousarray(vals, dtype=np.float64)
    out = np.empty(v.size, np.uint8)
    O.oracle_store(dt, ptr(v), v.size, ptr(out))
    return out


def test_fp8_decode_every_code():
    import torch
    codes = np.arange(256, dtype=np.uint8)
    # E5M2 is the upper byte of IEEE binary16, so numpy's fp16 decodes it independently
    e5 = fp8_decode_all(FP8E5M2)
    ref5 = (codes.astype(np.uint16) << 8).view(np.float16).astype(np.float64)
    assert np.array_equal(np.isnan(e5), np.isnan(ref5)) and np.array_equal(e5[~np.isnan(e5)], ref5[~np.isnan(ref5)])
    for dt, tdt in ((FP8E4M3, torch.float8_e4m3fn), (FP8E5M2, torch.float8_e5m2)):
        got = fp8_decode_all(dt)
        ref = torch.from_numpy(codes.copy()).view(tdt).to(torch.float64).numpy()
        assert np.array_equal(np.isnan(got), np.isnan(ref)), dt
        assert np.array_equal(got[~np.isnan(got)], ref[~np.isnan(ref)]), dt
    e4 = fp8_decode_all(FP8E4M3)
    # E4M3: no infinities, one NaN pattern per sign, largest 448, smallest subnormal 2^-9
    assert np.isnan(e4).sum() == 2 and np.isnan(e4[0x7f]) and np.isnan(e4[0xff])
    assert np.nanmax(e4) == 448.0 and e4[1] == 2.0 ** -9 and not np.isinf(e4).any()
    assert np.isinf(e5).sum() == 2 and np.nanmax(e5[np.isfinite(e5)]) == 57344.0 and e5[1] == 2.0 ** -16


@pytest.mark.parametrize("dt", [FP8E4M3, FP8E5M2], ids=["e4m3", "e5m2"])
def test_fp8_encode_rounding_and_saturation(dt):
    import torch
    tdt = torch.float8_e4m3fn if dt == FP8E4M3 else torch.float8_e5m2
    vals = fp8_decode_all(dt)
    fin = np.sort(np.unique(vals[np.isfinite(vals)]))
    # every code's value comes back to its code (both zeros keep their sign)
    codes = np.arange(256, dtype=np.uint8)
    keep = np.isfinite(vals)
    assert np.array_equal(fp8_encode(dt, vals[keep]), codes[keep])
    # midpoints between neighbours go to the even code, values just off a
    # midpoint to the nearer one; plus random fp32 values across the range
    mid = (fin[1:] + fin[:-1]) / 2
    g = rng(7)
    rand = (g.standard_normal(20000) * 2.0 ** g.integers(-18, 17, 20000)).astype(np.float32).astype(np.float64)
    probe = np.concatenate([mid, np.nextafter(mid, np.inf), np.nextafter(mid, -np.inf), rand])
    probe = probe[np.abs(probe) <= FP8_MAX[dt]].astype(np.float32).astype(np.float64)
    got = fp8_encode(dt, probe)
    ref = torch.from_numpy(probe.astype(np.float32)).to(tdt).view(torch.uint8).numpy()
    same = got == ref
    # +-0 of a value that rounds to zero may differ in sign only
    zero = (vals[got] == 0) & (vals[ref] == 0)
    assert np.all(same | zero)
    # saturating conversion: past the largest finite value (and infinity) to +-max; NaN stays NaN
    big = np.array([FP8_MAX[dt] * 1.0625, FP8_MAX[dt] * 4, 1e30, np.inf, -FP8_MAX[dt] * 2, -np.inf])
    dec = vals[fp8_encode(dt, big)]
    assert np.array_equal(dec, np.sign(big) * FP8_MAX[dt])
    assert np.isnan(vals[fp8_encode(dt, np.array([np.nan]))[0]])
    # oracle_round agrees with the code it stores
    for x in probe[:200]:
        assert O.oracle_round(x, dt) == vals[fp8_encode(dt, np.array([x]))[0]]


def test_fp8_mixed_type_functions_reduce_to_the_single_type_ones():
    """the *2 variants with equal forward and backward types equal the
    single-type functions, and an fp8 forward type reads its tensors as fp8"""
    n_rows, n_cols = 6, 64
    X, W = to_storage(normal(60, (n_rows, n_cols)), BF16), to_storage(1 + normal(61, (n_cols,), std=0.02), BF16)
    dY, dX = to_storage(normal(62, (n_rows, n_cols)), BF16), to_storage(normal(63, (n_rows, n_cols)), BF16)
    ws, rs = normal(64, (n_rows,)), (1 + np.abs(normal(65, (n_rows,)))).astype(np.float32)
    a_lo, a_hi, b_lo, b_hi = (np.empty((n_rows, n_cols)) for _ in range(4))
    assert O.oracle_rms_norm_bwd_x(BF16, n_rows, n_cols, ptr(ws), ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX), ptr(a_lo), ptr(a_hi)) == 0
    assert O.oracle_rms_norm_bwd_x2(BF16, BF16, n_rows, n_cols, ptr(ws), ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX), ptr(b_lo), ptr(b_hi)) == 0
    assert np.array_equal(a_lo, b_lo) and np.array_equal(a_hi, b_hi)
    # fp8 X and W: the same values stored as bf16 give the same result
    X8 = fp8_encode(FP8E4M3, to_f64(X, BF16).ravel()).reshape(X.shape)
    W8 = fp8_encode(FP8E4M3, to_f64(W, BF16))
    X8b = to_storage(fp8_decode_all(FP8E4M3)[X8].astype(np.float32), BF16)
    W8b = to_storage(fp8_decode_all(FP8E4M3)[W8].astype(np.float32), BF16)
    c_lo, c_hi, d_lo, d_hi = (np.empty((n_rows, n_cols)) for _ in range(4))
    assert O.oracle_rms_norm_bwd_x2(FP8E4M3, BF16, n_rows, n_cols, ptr(ws), ptr(rs), ptr(W8), ptr(X8), ptr(dY), ptr(dX), ptr(c_lo), ptr(c_hi)) == 0
    assert O.oracle_rms_norm_bwd_x2(BF16, BF16, n_rows, n_cols, ptr(ws), ptr(rs), ptr(W8b), ptr(X8b), ptr(dY), ptr(dX), ptr(d_lo), ptr(d_hi)) == 0
    assert np.array_equal(c_lo, d_lo) and np.array_equal(c_hi, d_hi)
    # backward-only tensors refuse fp8
    assert O.oracle_rms_norm_bwd_x2(BF16, FP8E4M3, n_rows, n_cols, ptr(ws), ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX), ptr(c_lo), ptr(c_hi)) == -1
    # sum of squares (the fp8 forward's statistic) against numpy
    ss = np.empty(n_rows)
    assert O.oracle_rms_norm_sq_sums(FP8E4M3, n_rows, n_cols, ptr(X8), ptr(ss)) == 0
    xv = fp8_decode_all(FP8E4M3)[X8]
    assert np.allclose(ss, (xv * xv).sum(1), rtol=1e-15)


def test_fp8_functions_equal_the_16_bit_ones_on_the_decoded_values():
    """every fp8 value is exactly a bf16 and an fp16 value, so each fp8
    oracle function must give the pre-rounding values its 16-bit counterpart
    gives on the decoded inputs (the storage type enters only through the
    loads, checked code by code above, and the output rounding, checked here
    against oracle_round); a wrong operand type or a dropped conversion
    breaks an equality"""
    g = rng(71)
    dec = {dt: fp8_decode_all(dt) for dt in (FP8E4M3, FP8E5M2)}
    for f8 in (FP8E4M3, FP8E5M2):
        for b16 in (FP16, BF16):
            def as16(codes):
                return to_storage(dec[f8][codes].astype(np.float32), b16)
            R, C = 5, 48
            X8 = fp8_encode(f8, g.standard_normal(R * C)).reshape(R, C)
            W8 = fp8_encode(f8, 1 + 0.02 * g.standard_normal(C))
            U8 = fp8_encode(f8, g.standard_normal(R * C)).reshape(R, C)
            dY = to_storage(g.standard_normal((R, C)).astype(np.float32), b16)
            dW = to_storage(0.1 * g.standard_normal(C).astype(np.float32), b16)
            rs = (1 + np.abs(g.standard_normal(R))).astype(np.float32)
            # rms_norm_bwd_w: fp8 X with 16-bit dY / dW
            a, aa, b, bb = np.empty(C), np.empty(C), np.empty(C), np.empty(C)
            assert O.oracle_rms_norm_bwd_w2(f8, b16, b16, R, C, ptr(rs), ptr(X8), ptr(dY), ptr(dW), ptr(a), ptr(aa)) == 0
            assert O.oracle_rms_norm_bwd_w(b16, b16, R, C, ptr(rs), ptr(as16(X8)), ptr(dY), ptr(dW), ptr(b), ptr(bb)) == 0
            assert np.array_equal(a, b) and np.array_equal(aa, bb)
            # swiglu_bwd_x: fp8 g, u with 16-bit dO
            n = R * C
            out8 = [np.empty(n) for _ in range(3)]
            out16 = [np.empty(n) for _ in range(3)]
            assert O.oracle_swiglu_bwd2(f8, b16, n, ptr(X8), ptr(U8), ptr(dY), *[ptr(o) for o in out8]) == 0
            assert O.oracle_swiglu_bwd(b16, n, ptr(as16(X8)), ptr(as16(U8)), ptr(dY), *[ptr(o) for o in out16]) == 0
            assert all(np.array_equal(p, q) for p, q in zip(out8, out16))
            # softmax: fp8 logits, x - max rounded in the output type
            L8 = fp8_encode(f8, 2.0 * g.standard_normal(R * 300)).reshape(R, 300)
            y8, y16 = np.empty((R, 300)), np.empty((R, 300))
            assert O.oracle_softmax(f8, b16, R, 300, ptr(L8), ptr(y8)) == 0
            assert O.oracle_softmax(b16, b16, R, 300, ptr(as16(L8)), ptr(y16)) == 0
            assert np.array_equal(y8, y16)
        # single-type forwards: the pre values equal the bf16 ones on the decoded inputs
        R, C = 4, 64
        X8 = fp8_encode(f8, g.standard_normal(R * C)).reshape(R, C)
        W8 = fp8_encode(f8, 1 + 0.02 * g.standard_normal(C))
        xb = to_storage(dec[f8][X8].astype(np.float32), BF16)
        wb = to_storage(dec[f8][W8].astype(np.float32), BF16)
        p8, p16 = [np.empty((R, C)), np.empty(R), np.empty(R), np.empty(R)], [np.empty((R, C)), np.empty(R), np.empty(R), np.empty(R)]
        assert O.oracle_rms_norm(f8, R, C, 1e-5, ptr(W8), ptr(X8), *[ptr(o) for o in p8]) == 0
        assert O.oracle_rms_norm(BF16, R, C, 1e-5, ptr(wb), ptr(xb), *[ptr(o) for o in p16]) == 0
        assert all(np.array_equal(p, q) for p, q in zip(p8, p16))
        s8, s16 = np.empty(n), np.empty(n)
        assert O.oracle_swiglu(f8, n, ptr(X8), ptr(U8), ptr(s8)) == 0
        assert O.oracle_swiglu(BF16, n, ptr(to_storage(dec[f8][X8].astype(np.float32), BF16)),
                               ptr(to_storage(dec[f8][U8].astype(np.float32), BF16)), ptr(s16)) == 0
        assert np.array_equal(s8, s16)
        T, nq, nkv, hd = 3, 2, 1, 16
        Q8 = fp8_encode(f8, g.standard_normal(T * nq * hd)).reshape(T, nq * hd)
        K8 = fp8_encode(f8, g.standard_normal(T * nkv * hd)).reshape(T, nkv * hd)
        pos = np.array([0, 5, 77], np.int32)
        q8, k8, q16, k16 = np.empty(Q8.shape), np.empty(K8.shape), np.empty(Q8.shape), np.empty(K8.shape)
        assert O.oracle_rope(f8, 0, T * nq * hd, nq * hd, hd, nkv, 10000, ptr(pos), ptr(Q8), ptr(K8), ptr(q8), ptr(k8)) == 0
        assert O.oracle_rope(BF16, 0, T * nq * hd, nq * hd, hd, nkv, 10000, ptr(pos),
                             ptr(to_storage(dec[f8][Q8].astype(np.float32), BF16)),
                             ptr(to_storage(dec[f8][K8].astype(np.float32), BF16)), ptr(q16), ptr(k16)) == 0
        assert np.array_equal(q8, q16) and np.array_equal(k8, k16)
        # and the fp8 rounding of those values is the fp8 store's
        for v in (p8[0].ravel()[:50], s8[:50], q8.ravel()[:50]):
            assert np.array_equal(dec[f8][fp8_encode(f8, v)], np.array([O.oracle_round(x, f8) for x in v]))
