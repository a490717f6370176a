"""The external matmul op (hipBLASLt) and the loss-path driver
submit_transformer_head, on the GPU.

matmul is checked against fp64 products of the same stored inputs: every
output within 1 ulp of its type of the exact value plus an accumulation
allowance of 2^-14 * sum_k |a_mk b_kn| (fp32 accumulation in any order stays
far inside it; a wrong transpose, stride or operand does not).

The head driver is checked stage by stage, each stage from the GPU's own
inputs to it: the norm against the oracle, the projection and both backward
GEMMs as above, dLogits and the loss against the oracle's fused
softmax + cross-entropy, and the norm backward against the oracle's exact
gradient."""
import ctypes

import numpy as np
import pytest

from support import (BF16, FP16, FP32, NP_STORAGE, check_f32, check_rounded, normal, oracle, ptr, rng, to_f64,
                     to_storage, ulp, gamma, rms_dw_depth)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hmm():
    from dataflow_lib_amd import api
    h = api.Handle(0, num_streams=2, matmul=True)
    yield h
    h.destroy()


def stored_f64(a, dt):
    return to_f64(a, dt) if dt != FP32 else np.asarray(a, np.float64)


def gemm_ref(opA, opB):
    """exact product and the accumulation allowance"""
    return opA @ opB, 2.0 ** -14 * (np.abs(opA) @ np.abs(opB))


def check_gemm(out, dt, v, floor, what):
    check_rounded(out, dt, v, floor=floor, what=what) if dt != FP32 else check_f32(out, v, rel=1e-6, floor=floor, what=what)


class Mem:
    def __init__(self, h):
        self.h, self.ptrs = h, []

    def put(self, a):
        p = self.h.to_device(np.ascontiguousarray(a))
        self.ptrs.append(p)
        return p

    def empty(self, n):
        p = self.h.alloc(n)
        self.ptrs.append(p)
        return p

    def get(self, p, shape, dtype):
        self.h.sync()
        return self.h.to_host(p, shape, dtype)

    def free(self):
        self.h.sync()
        for p in self.ptrs:
            self.h.free(p)


@pytest.mark.parametrize("dt", [BF16, FP16, FP32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("ta, tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("M, K, N", [(64, 96, 40), (1000, 256, 64), (33, 7, 5)])
def test_matmul(hmm, dt, ta, tb, M, K, N):
    from dataflow_lib_amd import api
    A = to_storage(normal(500, (M, K) if ta else (K, M)), dt)      # column-major M x K, or K x M when transposed
    B = to_storage(normal(501, (K, N) if tb else (N, K)), dt)
    C = to_storage(normal(502, (N, M), std=0.5), dt)                 # column-major M x N
    opA = stored_f64(A, dt) if ta else stored_f64(A, dt).T
    opB = stored_f64(B, dt) if tb else stored_f64(B, dt).T
    v, fl = gemm_ref(opA, opB)
    m = Mem(hmm)
    try:
        pa, pb, pc = m.put(A), m.put(B), m.put(C)
        pd = m.empty(C.nbytes)
        ws = m.empty(1 << 22)
        assert api.submit_matmul(hmm, 0, dt, dt, api.DATAFLOW_NONE, dt, FP32, ta, tb, M, K, N, 1.0, 0.0, pa, pb, None, pd,
                                 1 << 22, ws) == 0
        d = m.get(pd, (N, M), NP_STORAGE[dt])
        # accumulate: D = 0.5 * A B + 1 * C, C == D in place
        assert api.submit_matmul(hmm, 0, dt, dt, dt, dt, FP32, ta, tb, M, K, N, 0.5, 1.0, pa, pb, pc, pc, 1 << 22, ws) == 0
        acc = m.get(pc, (N, M), NP_STORAGE[dt])
    finally:
        m.free()
    check_gemm(d, dt, v.T, fl.T, "matmul D")
    v2 = 0.5 * v.T + stored_f64(C, dt)
    check_gemm(acc, dt, v2, 0.5 * fl.T + 2.0 ** -20 * np.abs(stored_f64(C, dt)), "matmul D += C")


def test_matmul_rejects_bad_shape_and_dtype(hmm):
    from dataflow_lib_amd import api
    assert api.submit_matmul(hmm, 0, BF16, BF16, api.DATAFLOW_NONE, BF16, FP32, 0, 0, -1, 4, 4, 1.0, 0.0, 0, 0, 0, 0, 0, 0) == -1
    assert api.submit_matmul(hmm, 0, api.DATAFLOW_UINT8, BF16, api.DATAFLOW_NONE, BF16, FP32, 0, 0, 4, 4, 4, 1.0, 0.0,
                             0, 0, 0, 0, 0, 0) == -1


@pytest.mark.parametrize("T, E, V", [(64, 256, 1000), (37, 128, 513)])
def test_transformer_head_fwd_bwd(hmm, T, E, V):
    from dataflow_lib_amd import api
    dt, eps = BF16, 1e-5
    X = to_storage(normal(600, (T, E)), dt)
    wn = to_storage(1.0 + normal(601, (E,), std=0.05), dt)
    Wst = to_storage(normal(602, (V, E), std=E ** -0.5), dt)         # w_head column-major E x V
    dW0 = to_storage(normal(603, (V, E), std=0.01), dt)              # existing weight gradient (accumulated into)
    dwn0 = normal(604, (E,), std=0.01)                               # fp32 norm-weight gradient
    dX0 = to_storage(normal(605, (T, E), std=0.1), dt)               # residual gradient stream (accumulated into)
    labels = rng(606).integers(0, V, size=T).astype(np.uint32)
    bf = NP_STORAGE[dt]
    m = Mem(hmm)
    try:
        px, pwn, pw, pdw, pdwn, pdx = m.put(X), m.put(wn), m.put(Wst), m.put(dW0), m.put(dwn0), m.put(dX0)
        plab = m.put(labels)
        pnorm, pws, prs, pout = m.empty(T * E * 2), m.empty(T * 4), m.empty(T * 4), m.empty(T * V * 2)
        ploss, pprob, pgnorm, pnext = m.empty((T + 1) * 4), m.empty(T * V * 2), m.empty(T * E * 2), m.empty(T * E * 2)
        ws = m.empty(1 << 24)
        head = api.TransformerHead(dt, dt, FP32, eps, api.EmbeddingConfig(V, E), None, pwn, pw)
        acts = api.TransformerHeadActivations(T, None, pnorm, pws, prs, pout, ws, 1 << 24)
        inp = api.TransformerBlockTransition(None, px)
        out = api.TransformerModelOutput(None, None, plab, pprob, ploss, 0.0)
        # inference: logits = softmax(head_norm_out @ w_head)
        assert api.submit_transformer_head(hmm, 0, 1, inp, head, acts, out) == 0
        xn = m.get(pnorm, (T, E), bf)
        logits = m.get(pout, (T, V), bf)
        probs = m.get(pprob, (T, V), bf)
        # training
        ghead = api.TransformerHead(dt, dt, FP32, eps, api.EmbeddingConfig(V, E), None, pdwn, pdw)
        gacts = api.TransformerHeadActivations(T, None, pgnorm, None, None, None, ws, 1 << 24)
        gstream, nxt = api.TransformerBlockTransition(None, pdx), api.TransformerBlockTransition(None, pnext)
        assert api.submit_transformer_head(hmm, 0, 1, inp, head, acts, out, ghead, gacts, gstream, nxt) == 0
        hmm.sync()
        dlogits = m.get(pout, (T, V), bf)
        loss = m.get(ploss, (T + 1,), np.float32)
        gxn = m.get(pgnorm, (T, E), bf)
        dW = m.get(pdw, (V, E), bf)
        dwn = m.get(pdwn, (E,), np.float32)
        dX = m.get(pdx, (T, E), bf)
        nxt_x = m.get(pnext, (T, E), bf)
    finally:
        m.free()
    O = oracle()
    # 1. norm
    y_pre, _, rs, _ = np.empty((T, E)), np.empty(T), np.empty(T), np.empty(T)
    assert O.oracle_rms_norm(dt, T, E, eps, ptr(wn), ptr(X), ptr(y_pre), ptr(np.empty(T)), ptr(rs), ptr(np.empty(T))) == 0
    check_rounded(xn, dt, y_pre, what="head norm")
    # 2. projection from the GPU's norm output
    W = to_f64(Wst, dt).T                                            # E x V
    v, fl = gemm_ref(to_f64(xn, dt), W)
    check_rounded(logits, dt, v, floor=fl, what="head logits")
    # 3. inference softmax of the GPU's logits
    sm = np.empty((T, V))
    assert O.oracle_softmax(dt, dt, T, V, ptr(logits), ptr(sm)) == 0
    check_rounded(probs, dt, sm, what="head probabilities")
    # 4. fused loss on the same logits (the training pass recomputes them identically)
    lo, hi, l_e, mean_e = np.empty((T, V)), np.empty((T, V)), np.empty(T), np.zeros(1)
    assert O.oracle_softmax_cross_entropy(dt, T, V, ptr(logits), ptr(labels), ptr(lo), ptr(hi), ptr(l_e), ptr(mean_e)) == 0
    check_rounded(dlogits, dt, lo, hi, what="head dlogits")
    check_f32(loss[:T], l_e, rel=1e-4, what="head loss")
    check_f32(loss[T:], mean_e, rel=1e-4, what="head mean loss")
    # 5. backward GEMMs from the GPU's dLogits
    dl = to_f64(dlogits, dt)
    v, fl = gemm_ref(dl, W.T)
    check_rounded(gxn, dt, v, floor=fl, what="head grad norm_out")
    v, fl = gemm_ref(to_f64(xn, dt).T, dl)                           # E x V
    check_rounded(dW, dt, v.T + to_f64(dW0, dt), floor=fl.T + 2.0 ** -20 * np.abs(to_f64(dW0, dt)), what="head dW")
    # 6. exact norm backward from the GPU's upstream gradient
    dx_pre, dx_floor, dw_pre, dw_abs = np.empty((T, E)), np.empty((T, E)), np.empty(E), np.empty(E)
    rs32 = rs.astype(np.float32)
    assert O.oracle_rms_norm_bwd(dt, T, E, ptr(rs32), ptr(wn), ptr(X), ptr(gxn), ptr(dX0), ptr(dwn0),
                                 ptr(dx_pre), ptr(dx_floor), ptr(dw_pre), ptr(dw_abs)) == 0
    check_rounded(dX, dt, dx_pre, floor=dx_floor, what="head dX")
    info = hmm.device_info
    check_f32(dwn, dw_pre, floor=gamma(rms_dw_depth(dt, T, E, 3, info.cu_count, info.max_smem_per_block)) * dw_abs,
              what="head dW norm")
    assert np.array_equal(nxt_x, dX)                                 # copied after the compute stream
