"""The registry, fingerprint dispatch and argument marshalling of the product
library, run end to end in a GPU-less process: register_native_ops() and the
submit_* functions of libdataflow.so drive the CPU test backend in
oracle/liboracle.so (COMPUTE_CPU), whose "<op>_<dt>_kernel" adapters read
op_args exactly as the GPU kernels do. BASELINE config 1 (RMSNorm forward,
fp32, 16 x 4096) runs here."""
import ctypes

import numpy as np
import pytest

from support import BF16, FP32, ORACLE_LIB, check_f32, normal, oracle, ptr, to_storage

from dataflow_lib_amd import api


@pytest.fixture(scope="module")
def cpu_handle():
    O = oracle()
    O.init_cpu_dataflow_handle.argtypes = [ctypes.POINTER(api.DataflowHandle), ctypes.c_int]
    O.destroy_cpu_dataflow_handle.argtypes = [ctypes.POINTER(api.DataflowHandle)]
    h = api.DataflowHandle()
    assert O.init_cpu_dataflow_handle(ctypes.byref(h), 2) == 0
    n = api.lib().register_native_ops(ctypes.byref(h), ORACLE_LIB.encode(), b"")
    yield h, n
    O.destroy_cpu_dataflow_handle(ctypes.byref(h))


def test_registers_every_variant(cpu_handle):
    h, n = cpu_handle
    # the reference's 54 functions (its fp8 variants included), copy_to_seq_context x 5 storage
    # types and the three fused ops x fp32/fp16/bf16
    assert n == 68 and h.num_ops == 68 and h.op_table.cnt == 68


def test_config1_rms_norm_fp32_through_handle(cpu_handle):
    """fp32 X [16 x 4096] ~ N(0,1), W = 1 + N(0, 0.02), eps 1e-5"""
    h, _ = cpu_handle
    n_rows, n_cols, eps = 16, 4096, 1e-5
    X = normal(1, (n_rows, n_cols))
    W = (1.0 + normal(2, (n_cols,), std=0.02)).astype(np.float32)
    Y = np.empty_like(X)
    ws, rs = np.empty(n_rows, np.float32), np.empty(n_rows, np.float32)
    assert api.submit_rms_norm(ctypes.byref(h), 0, FP32, n_rows, n_cols, eps, ptr(W), ptr(X), ptr(Y), ptr(ws), ptr(rs)) == 0
    y_pre, ws_e, rs_e, ws_abs = np.empty((n_rows, n_cols)), np.empty(n_rows), np.empty(n_rows), np.empty(n_rows)
    assert oracle().oracle_rms_norm(FP32, n_rows, n_cols, eps, ptr(W), ptr(X), ptr(y_pre), ptr(ws_e), ptr(rs_e), ptr(ws_abs)) == 0
    assert np.array_equal(Y, y_pre.astype(np.float32))
    check_f32(rs, rs_e, rel=1e-7)
    check_f32(ws, ws_e, rel=1e-7)
    # closed form: mean_j (y/w)^2 = r^2 * ss/n = 1 - eps * r^2
    assert np.allclose(((y_pre / W) ** 2).mean(axis=1), 1.0 - eps * rs_e ** 2, rtol=1e-12)


def test_dispatch_uses_fingerprint_not_name(cpu_handle):
    """an Op whose header differs only in one arg dtype must not resolve"""
    h, _ = cpu_handle
    op = api.Op()
    op.op_skeleton = api.native_op_skeleton("swiglu", BF16)
    op.op_skeleton.header.arg_dtypes[4] = FP32
    api.lib().do_fingerprinting(ctypes.byref(op.op_skeleton.header), ctypes.sizeof(api.OpSkeletonHeader),
                                op.op_skeleton.fingerprint, 0)
    submit = ctypes.cast(h.submit_op, ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(api.DataflowHandle),
                                                       ctypes.POINTER(api.Op), ctypes.c_int))
    assert submit(ctypes.byref(h), ctypes.byref(op), 0) == -1


def test_error_paths(cpu_handle):
    h, _ = cpu_handle
    p = np.zeros(64, np.float32)
    # a variant nobody registers (uint8 storage) and an out-of-range stream id
    assert api.submit_rms_norm(ctypes.byref(h), 0, api.DATAFLOW_UINT8, 1, 16, 1e-5, ptr(p), ptr(p), ptr(p), None, None) == -1
    assert api.submit_rms_norm(ctypes.byref(h), 5, FP32, 1, 16, 1e-5, ptr(p), ptr(p), ptr(p), None, None) == -1
    assert api.submit_rms_norm(ctypes.byref(h), -1, FP32, 1, 16, 1e-5, ptr(p), ptr(p), ptr(p), None, None) == 0


@pytest.mark.parametrize("op", ["swiglu", "softmax_xent", "rope", "rms_bwd"])
def test_other_ops_through_handle(cpu_handle, op):
    h, _ = cpu_handle
    H = ctypes.byref(h)
    if op == "swiglu":
        g, u = to_storage(normal(3, (4, 64)), BF16), to_storage(normal(4, (4, 64)), BF16)
        out = np.empty_like(g)
        assert api.submit_swiglu(H, 0, BF16, 4, 64, ptr(g), ptr(u), ptr(out)) == 0
        pre = np.empty((4, 64))
        assert oracle().oracle_swiglu(BF16, g.size, ptr(g), ptr(u), ptr(pre)) == 0
        from support import check_rounded
        check_rounded(out, BF16, pre, what="cpu-dispatched swiglu")
    elif op == "softmax_xent":
        x = to_storage(normal(5, (3, 100), std=2.0), BF16)
        lab = np.array([0, 50, 99], np.uint32)
        loss, mean = np.empty(3, np.float32), np.empty(1, np.float32)
        assert api.submit_softmax_cross_entropy_loss(H, 0, BF16, 3, 100, ptr(x), ptr(lab), ptr(loss), ptr(mean)) == 0
        assert np.isfinite(loss).all() and abs(mean[0] - loss.mean()) < 1e-5
    elif op == "rope":
        q, k = to_storage(normal(6, (2, 256)), BF16), to_storage(normal(7, (2, 128)), BF16)
        pos = np.array([0, 9], np.int32)
        q0 = q.copy()
        assert api.submit_rope(H, 0, BF16, 512, 256, 128, 1, 10000, ptr(pos), ptr(q), ptr(k)) == 0
        assert np.array_equal(q[0], q0[0])     # position 0 is the identity rotation
        assert not np.array_equal(q[1], q0[1])
    else:
        X = normal(8, (3, 32))
        W, dY, dX = np.ones(32, np.float32), normal(9, (3, 32)), np.zeros((3, 32), np.float32)
        rs, dW = np.ones(3, np.float32), np.zeros(32, np.float32)
        assert api.submit_rms_norm_bwd(H, 0, FP32, FP32, 3, 32, 1e-5, ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX), ptr(dW)) == 0
        assert np.allclose(dW, (dY * X).sum(axis=0), rtol=1e-6)


def test_embedding_and_kv_scatter_through_handle(cpu_handle):
    """submit_embedding / submit_copy_to_seq_context marshal their arguments
    the way the kernels read them (fp8 variants move bytes)."""
    h, _ = cpu_handle
    vocab, dim = 40, 16
    table = rng_u8(300, (vocab, dim))
    ids = np.array([3, 0, 39, 3, 17], np.uint32)
    out = np.zeros((ids.size, dim), np.uint8)
    assert api.submit_embedding(ctypes.byref(h), 0, api.DATAFLOW_FP8E4M3, ids.size, dim, ptr(ids), ptr(table), ptr(out)) == 0
    assert np.array_equal(out, table[ids])
    kv_dim, n_tok, S = 8, 4, 6
    ctx = np.zeros((2 * S, kv_dim), np.uint16)
    K, V = rng_u8(301, (n_tok, 2 * kv_dim)).view(np.uint16), rng_u8(302, (n_tok, 2 * kv_dim)).view(np.uint16)
    pos = np.array([0, 3, 1, 5], np.int32)
    ptrs = np.full(n_tok, ctx.ctypes.data, np.uint64)
    sizes = np.full(n_tok, S, np.int32)
    assert api.submit_copy_to_seq_context(ctypes.byref(h), 0, BF16, n_tok * kv_dim, n_tok, kv_dim, ptr(K), ptr(V), ptr(pos),
                                          ptr(ptrs), ptr(sizes)) == 0
    assert np.array_equal(ctx[pos], K) and np.array_equal(ctx[S + pos], V)


def test_rope_copy_to_seq_context_through_handle(cpu_handle):
    """submit_rope_copy_to_seq_context marshals its 11 arguments the way the
    kernel reads them: the same Q and K as submit_rope, and the context rows
    hold the rotated K rows and the V rows."""
    h, _ = cpu_handle
    T, nq, nkv, hd, S = 5, 2, 1, 8, 7
    Q, K, V = normal(310, (T, nq * hd)), normal(311, (T, nkv * hd)), normal(312, (T, nkv * hd))
    pos = np.array([0, 4, 2, 6, 1], np.int32)
    q2, k2 = Q.copy(), K.copy()
    assert api.submit_rope(ctypes.byref(h), 0, FP32, T * nq * hd, nq * hd, hd, nkv, 10000, ptr(pos), ptr(q2), ptr(k2)) == 0
    ctx = np.zeros((2 * S, nkv * hd), np.float32)
    ptrs = np.full(T, ctx.ctypes.data, np.uint64)
    sizes = np.full(T, S, np.int32)
    assert api.submit_rope_copy_to_seq_context(ctypes.byref(h), 0, FP32, T * nq * hd, nq * hd, hd, nkv, 10000, ptr(pos), ptr(Q),
                                               ptr(K), ptr(V), ptr(ptrs), ptr(sizes)) == 0
    assert np.array_equal(Q, q2) and np.array_equal(K, k2)
    assert np.array_equal(ctx[pos], K) and np.array_equal(ctx[S + pos], V)


def rng_u8(seed, shape):
    return np.random.default_rng(seed).integers(0, 256, size=shape).astype(np.uint8)


FP8S = [api.DATAFLOW_FP8E4M3, api.DATAFLOW_FP8E5M2]


def _f8(dt, x):
    from support import to_storage
    return to_storage(np.asarray(x, np.float32), dt)


@pytest.mark.parametrize("f8", FP8S, ids=["e4m3", "e5m2"])
@pytest.mark.parametrize("b16", [api.DATAFLOW_FP16, BF16], ids=["fp16", "bf16"])
def test_fp8_variants_through_handle(cpu_handle, f8, b16):
    """each of the 22 fp8 functions is found by its fingerprint and gets its
    arguments in the order the kernels read them: the results equal the
    oracle's on the same inputs, rounded to the output type"""
    from support import NP_STORAGE, to_f64
    h, _ = cpu_handle
    H = ctypes.byref(h)
    O = oracle()
    g = np.random.default_rng(int(f8) * 10 + int(b16))
    R, C = 3, 32
    X = _f8(f8, g.standard_normal((R, C)))
    W = _f8(f8, 1 + 0.02 * g.standard_normal(C))
    # rms_norm fp8: out in fp8, sum of squares in the statistic slot, weighted sums untouched
    Y = np.zeros_like(X)
    ws, ss = np.full(R, -3.0, np.float32), np.zeros(R, np.float32)
    assert api.submit_rms_norm(H, 0, f8, R, C, 1e-5, ptr(W), ptr(X), ptr(Y), ptr(ws), ptr(ss)) == 0
    pre, e_ss = np.empty((R, C)), np.empty(R)
    assert O.oracle_rms_norm(f8, R, C, 1e-5, ptr(W), ptr(X), ptr(pre), None, None, None) == 0
    assert O.oracle_rms_norm_sq_sums(f8, R, C, ptr(X), ptr(e_ss)) == 0
    assert np.array_equal(to_f64(Y, f8), to_f64(_f8(f8, pre), f8))
    assert np.array_equal(ss, e_ss.astype(np.float32)) and np.all(ws == -3.0)
    # rms_norm_bwd_x / bwd_w with 16-bit backward tensors
    rs = (1 + np.abs(g.standard_normal(R))).astype(np.float32)
    wsum = g.standard_normal(R).astype(np.float32)
    dY = (g.standard_normal((R, C))).astype(np.float32)
    dY = dY.astype(np.float16) if b16 == api.DATAFLOW_FP16 else f32_to_bf16(dY)
    dX = np.zeros_like(dY)
    v = np.empty((R, C))
    assert api.submit_rms_norm_bwd_x(H, 0, f8, b16, R, C, 1e-5, ptr(wsum), ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX)) == 0
    dX0 = np.zeros_like(dY)
    assert O.oracle_rms_norm_bwd_x2_exact(f8, b16, R, C, ptr(wsum), ptr(rs), ptr(W), ptr(X), ptr(dY), ptr(dX0), ptr(v)) == 0
    assert np.array_equal(to_f64(dX, b16), np.array([O.oracle_round(x, b16) for x in v.ravel()]).reshape(R, C))
    dW = np.zeros(C, NP_STORAGE[b16])
    assert api.submit_rms_norm_bwd_w(H, 0, f8, b16, R, C, 1e-5, ptr(rs), ptr(X), ptr(dY), ptr(dW)) == 0
    pw, pa = np.empty(C), np.empty(C)
    assert O.oracle_rms_norm_bwd_w2(f8, b16, b16, R, C, ptr(rs), ptr(X), ptr(dY), ptr(np.zeros(C, NP_STORAGE[b16])), ptr(pw), ptr(pa)) == 0
    assert np.array_equal(to_f64(dW, b16), np.array([O.oracle_round(x, b16) for x in pw]))
    # swiglu fwd (fp8) and bwd (fp8 x 16-bit)
    U = _f8(f8, g.standard_normal((R, C)))
    out = np.zeros_like(X)
    assert api.submit_swiglu(H, 0, f8, R, C, ptr(X), ptr(U), ptr(out)) == 0
    sp = np.empty((R, C))
    assert O.oracle_swiglu(f8, R * C, ptr(X), ptr(U), ptr(sp)) == 0
    assert np.array_equal(to_f64(out, f8), to_f64(_f8(f8, sp), f8))
    dG, dU = np.zeros_like(dY), np.zeros_like(dY)
    assert api.submit_swiglu_bwd_x(H, 0, f8, b16, R, C, ptr(X), ptr(U), ptr(dY), ptr(dG), ptr(dU)) == 0
    eg, eu = np.empty((R, C)), np.empty((R, C))
    assert O.oracle_swiglu_bwd2(f8, b16, R * C, ptr(X), ptr(U), ptr(dY), ptr(eg), None, ptr(eu)) == 0
    assert np.array_equal(to_f64(dU, b16), np.array([O.oracle_round(x, b16) for x in eu.ravel()]).reshape(R, C))
    assert np.array_equal(to_f64(dG, b16), np.array([O.oracle_round(x, b16) for x in eg.ravel()]).reshape(R, C))
    # softmax fp8 -> 16-bit
    P = np.zeros((R, C), NP_STORAGE[b16])
    assert api.submit_softmax(H, 0, f8, b16, R, C, ptr(X), ptr(P)) == 0
    yp = np.empty((R, C))
    assert O.oracle_softmax(f8, b16, R, C, ptr(X), ptr(yp)) == 0
    assert np.array_equal(to_f64(P, b16), np.array([O.oracle_round(x, b16) for x in yp.ravel()]).reshape(R, C))
    # rope fp8 (forward only)
    Q, K = _f8(f8, g.standard_normal((2, 16))), _f8(f8, g.standard_normal((2, 8)))
    pos = np.array([3, 11], np.int32)
    qv, kv = np.empty(Q.shape), np.empty(K.shape)
    assert O.oracle_rope(f8, 0, 32, 16, 8, 1, 10000, ptr(pos), ptr(Q), ptr(K), ptr(qv), ptr(kv)) == 0
    assert api.submit_rope(H, 0, f8, 32, 16, 8, 1, 10000, ptr(pos), ptr(Q), ptr(K)) == 0
    assert np.array_equal(to_f64(Q, f8), to_f64(_f8(f8, qv), f8)) and np.array_equal(to_f64(K, f8), to_f64(_f8(f8, kv), f8))
    assert api.submit_rope_bwd_x(H, 0, f8, 32, 16, 8, 1, 10000, ptr(pos), ptr(Q), ptr(K)) == -1


def f32_to_bf16(x):
    from support import f32_to_bf16_bits
    return f32_to_bf16_bits(x)
