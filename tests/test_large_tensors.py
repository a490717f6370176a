"""Tensors past 4 GiB (and, for the flat element-wise ops, past 2^31 elements)
on the GPU: the size class that 288 GB of HBM makes ordinary. Each input is a
small seeded block repeated on the device by doubling device-to-device
copies, so the host uploads only the block. The first block's outputs are
checked against the oracle to the same tolerances as the other GPU tests, and
every later block must be bit-equal to the first (the ops are row- or
element-local and deterministic). Block lengths are chosen so that an offset
wrapped at 2^31 elements or 2^32 bytes, or an access dropped by a 32-bit
buffer range, lands on different data and fails the comparison."""
import numpy as np
import pytest

from support import (BF16, NP_STORAGE, check_f32, check_rounded, gamma, normal, oracle, ptr, rms_ws_depth, rng,
                     to_storage)

pytestmark = pytest.mark.gpu

FOUR_GIB = 1 << 32


@pytest.fixture(scope="module")
def hdl():
    from dataflow_lib_amd import api
    h = api.Handle(0, num_streams=1)
    yield h
    h.destroy()


class Bufs:
    """Device buffers of one test, freed at exit."""

    def __init__(self, h):
        self.h, self.ptrs = h, []

    def __enter__(self):
        return self

    def empty(self, nbytes):
        p = self.h.alloc(nbytes)
        self.ptrs.append(p)
        return p

    def tiled(self, block, reps):
        """`reps` back-to-back copies of `block` in one device buffer."""
        block = np.ascontiguousarray(block)
        bb = block.nbytes
        p = self.empty(bb * reps)
        self.h.to_device(block, p)
        have = 1
        while have < reps:
            n = min(have, reps - have)
            assert self.h.copy(p + have * bb, p, n * bb) == 0
            have += n
        return p

    def get(self, p, shape, dtype):
        self.h.sync()
        return self.h.to_host(p, shape, dtype)

    def __exit__(self, *exc):
        self.h.sync()
        for p in self.ptrs:
            self.h.free(p)


def assert_blocks_equal(out, block_rows, what):
    """out: (reps * block_rows, ...) — every block of `block_rows` rows equals the first, bit for bit."""
    v = out.reshape(out.shape[0] // block_rows, -1)
    first = v[0]
    step = max(1, (1 << 28) // max(1, v.shape[1] * v.itemsize))
    for s in range(1, v.shape[0], step):
        ok = (v[s:s + step] == first).all(axis=1)
        if not ok.all():
            b = s + int(np.flatnonzero(~ok)[0])
            j = int(np.flatnonzero(v[b] != first)[0])
            raise AssertionError("%s: block %d differs from block 0 first at element %d of the block (%r vs %r)"
                                 % (what, b, j, v[b, j], first[j]))


def test_swiglu_past_2g_elements(hdl):
    """fwd and bwd over 2049 x 1048568 bf16 (2.15e9 elements, 4.3 GB per tensor).
    The block is one row of 8 * 131071 elements: 2^31 mod 1048568 = 16384, so a
    wrapped element index reads a different element of the block."""
    from dataflow_lib_amd import api
    dt, L, reps = BF16, 8 * 131071, 2049
    n = L * reps
    assert n > (1 << 31) and 2 * n > FOUR_GIB
    g = to_storage(normal(201, (L,), std=2.0), dt)
    u = to_storage(normal(202, (L,)), dt)
    dO = to_storage(normal(203, (L,)), dt)
    pre = np.empty(L)
    dg, dgf, du = np.empty(L), np.empty(L), np.empty(L)
    assert oracle().oracle_swiglu(dt, L, ptr(g), ptr(u), ptr(pre)) == 0
    assert oracle().oracle_swiglu_bwd(dt, L, ptr(g), ptr(u), ptr(dO), ptr(dg), ptr(dgf), ptr(du)) == 0
    with Bufs(hdl) as d:
        pg, pu, pd = d.tiled(g, reps), d.tiled(u, reps), d.tiled(dO, reps)
        po, pdg, pdu = d.empty(2 * n), d.empty(2 * n), d.empty(2 * n)
        assert api.submit_swiglu(hdl, 0, dt, reps, L, pg, pu, po) == 0
        assert api.submit_swiglu_bwd_x(hdl, 0, dt, dt, reps, L, pg, pu, pd, pdg, pdu) == 0
        for p, what in ((po, "swiglu out"), (pdg, "swiglu dG"), (pdu, "swiglu dU")):
            out = d.get(p, (reps, L), NP_STORAGE[dt])
            if what == "swiglu out":
                check_rounded(out[0], dt, pre, what=what)
            elif what == "swiglu dG":
                check_rounded(out[0], dt, dg, floor=dgf, what=what)
            else:
                check_rounded(out[0], dt, du, what=what)
            assert_blocks_equal(out, 1, what)
            del out


def test_fused_cross_entropy_past_4gib(hdl):
    """16800 x 128256 bf16 logits (4.31 GB), seven distinct rows repeated;
    2^32 bytes is 16744.6 rows, so a wrapped row offset reads across rows."""
    from dataflow_lib_amd import api
    dt, V, B, reps = BF16, 128256, 7, 2400
    R = B * reps
    assert R * V * 2 > FOUR_GIB
    x = normal(211, (B, V), std=2.0)
    x[2, 11] = 40.0
    X = to_storage(x, dt)
    lab = rng(212).integers(0, V, size=B).astype(np.uint32)
    lab[0], lab[B - 1] = 0, V - 1
    lo, hi, loss, mean = np.empty((B, V)), np.empty((B, V)), np.empty(B), np.zeros(1)
    assert oracle().oracle_softmax_cross_entropy(dt, B, V, ptr(X), ptr(lab), ptr(lo), ptr(hi), ptr(loss), ptr(mean)) == 0
    with Bufs(hdl) as d:
        px, pl = d.tiled(X, reps), d.tiled(lab, reps)
        ploss, pmean = d.empty(4 * R), d.empty(4)
        assert api.submit_softmax_cross_entropy_loss(hdl, 0, dt, R, V, px, pl, ploss, pmean) == 0
        gl = d.get(ploss, (R,), np.float32)
        gm = d.get(pmean, (1,), np.float32)
        out = d.get(px, (R, V), NP_STORAGE[dt])
    check_rounded(out[:B], dt, lo, hi, what="fused dlogits")
    assert_blocks_equal(out, B, "fused dlogits")
    del out
    check_f32(gl[:B], loss, rel=1e-4, what="fused loss")
    assert_blocks_equal(gl, B, "fused loss")
    check_f32(gm, mean, rel=1e-4, what="fused mean loss")


def test_rms_norm_past_4gib(hdl):
    """fwd and bwd_x over 524293 x 4096 bf16 rows (4.3 GB per tensor), seven
    distinct rows repeated; 2^32 bytes is exactly 524288 rows, which is not a
    multiple of seven."""
    from dataflow_lib_amd import api
    dt, C, B, reps, eps = BF16, 4096, 7, 74899, 1e-5
    R = B * reps
    assert R * C * 2 > FOUR_GIB and (FOUR_GIB // (2 * C)) % B != 0
    X = to_storage(normal(221, (B, C)), dt)
    W = to_storage(1.0 + normal(222, (C,), std=0.02), dt)
    dY = to_storage(normal(223, (B, C)), dt)
    dX0 = to_storage(normal(224, (B, C)), dt)
    y_pre, ws, rs, ws_abs = np.empty((B, C)), np.empty(B), np.empty(B), np.empty(B)
    assert oracle().oracle_rms_norm(dt, B, C, eps, ptr(W), ptr(X), ptr(y_pre), ptr(ws), ptr(rs), ptr(ws_abs)) == 0
    ws32, rs32 = ws.astype(np.float32), rs.astype(np.float32)
    dlo, dhi = np.empty((B, C)), np.empty((B, C))
    assert oracle().oracle_rms_norm_bwd_x(dt, B, C, ptr(ws32), ptr(rs32), ptr(W), ptr(X), ptr(dY), ptr(dX0),
                                          ptr(dlo), ptr(dhi)) == 0
    with Bufs(hdl) as d:
        pw = d.tiled(W, 1)
        px, pdy, pdx = d.tiled(X, reps), d.tiled(dY, reps), d.tiled(dX0, reps)
        # bwd_x reads the oracle's statistics rounded to fp32, as its oracle did
        pws_in, prs_in = d.tiled(ws32, reps), d.tiled(rs32, reps)
        py, pws, prs = d.empty(R * C * 2), d.empty(4 * R), d.empty(4 * R)
        assert api.submit_rms_norm(hdl, 0, dt, R, C, eps, pw, px, py, pws, prs) == 0
        assert api.submit_rms_norm_bwd_x(hdl, 0, dt, dt, R, C, eps, pws_in, prs_in, pw, px, pdy, pdx) == 0
        gws = d.get(pws, (R,), np.float32)
        grs = d.get(prs, (R,), np.float32)
        check_f32(grs[:B], rs, what="rms_norm rstd")
        check_f32(gws[:B], ws, floor=gamma(rms_ws_depth(dt, C)) * ws_abs, what="rms_norm weighted_sums")
        assert_blocks_equal(grs, B, "rms_norm rstd")
        assert_blocks_equal(gws, B, "rms_norm weighted_sums")
        y = d.get(py, (R, C), NP_STORAGE[dt])
        check_rounded(y[:B], dt, y_pre, what="rms_norm y")
        assert_blocks_equal(y, B, "rms_norm y")
        del y
        dx = d.get(pdx, (R, C), NP_STORAGE[dt])
    check_rounded(dx[:B], dt, dlo, dhi, what="rms_norm_bwd_x dX")
    assert_blocks_equal(dx, B, "rms_norm_bwd_x dX")


def test_rope_past_4gib(hdl):
    """RoPE over 524293 tokens x 4096 (Q, 4.3 GB) and x 1024 (K), seven distinct
    tokens repeated with their positions."""
    from dataflow_lib_amd import api
    dt, B, reps, nq, nkv, hd, theta = BF16, 7, 74899, 32, 8, 128, 500000
    T = B * reps
    assert T * nq * hd * 2 > FOUR_GIB
    Q = to_storage(normal(231, (B, nq * hd)), dt)
    K = to_storage(normal(232, (B, nkv * hd)), dt)
    pos = np.array([0, 1, 17, 4095, 8191, 65535, 131071], np.int32)
    qv, kv = np.empty(Q.shape), np.empty(K.shape)
    assert oracle().oracle_rope(dt, 0, B * nq * hd, nq * hd, hd, nkv, theta, ptr(pos), ptr(Q), ptr(K), ptr(qv), ptr(kv)) == 0
    with Bufs(hdl) as d:
        pq, pk, pp = d.tiled(Q, reps), d.tiled(K, reps), d.tiled(pos, reps)
        assert api.submit_rope(hdl, 0, dt, T * nq * hd, nq * hd, hd, nkv, theta, pp, pq, pk) == 0
        gk = d.get(pk, (T, nkv * hd), NP_STORAGE[dt])
        check_rounded(gk[:B], dt, kv, what="rope k")
        assert_blocks_equal(gk, B, "rope k")
        del gk
        gq = d.get(pq, (T, nq * hd), NP_STORAGE[dt])
    check_rounded(gq[:B], dt, qv, what="rope q")
    assert_blocks_equal(gq, B, "rope q")
