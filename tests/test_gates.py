"""The fp32-sum gate the GPU tests apply at BASELINE config 2 (support.sum_gate:
1e-5 relative plus 4 u * sum|terms|) must reject a reduction that loses
precision. The mistake is planted on the CPU: a model of the dW reduction
(per-workgroup fp32 partial rows over a strided share of the rows, then their
sum, as the RMSNorm dW kernels reduce) against the oracle's exact dW, once as
it is (passes) and once with every partial row rounded to fp16 (fails on most
columns). No GPU involved."""
import numpy as np
import pytest

from support import (BF16, FP32, U32, bf16_bits_to_f32, check_f32, confident_logits, gamma, normal, oracle, ptr, sum_gate,
                     to_storage)

N_ROWS, N_COLS, GROUPS = 8192, 4096, 256


@pytest.fixture(scope="module")
def config2():
    """config-2 inputs (bf16 X, dY ~ N(0, 1); rstd from the oracle forward with
    W = 1 + N(0, 0.02)) and the oracle's exact dW = sum_r dY X rstd with its
    sum of |terms|"""
    seed = 91
    X = to_storage(normal(seed, (N_ROWS, N_COLS)), BF16)
    W = to_storage(1.0 + normal(seed + 1, (N_COLS,), std=0.02), BF16)
    ws, rs, ws_abs = np.empty(N_ROWS), np.empty(N_ROWS), np.empty(N_ROWS)
    assert oracle().oracle_rms_norm(BF16, N_ROWS, N_COLS, 1e-5, ptr(W), ptr(X), None, ptr(ws), ptr(rs), ptr(ws_abs)) == 0
    rs32 = rs.astype(np.float32)
    dY = to_storage(normal(seed + 2, (N_ROWS, N_COLS)), BF16)
    dW_in = np.zeros(N_COLS, np.float32)
    dw_pre, dw_abs = np.empty(N_COLS), np.empty(N_COLS)
    assert oracle().oracle_rms_norm_bwd_w(BF16, FP32, N_ROWS, N_COLS, ptr(rs32), ptr(X), ptr(dY), ptr(dW_in), ptr(dw_pre),
                                          ptr(dw_abs)) == 0
    return bf16_bits_to_f32(X), bf16_bits_to_f32(dY), rs32, dw_pre, dw_abs


def partial_rows(Xf, dYf, rs32):
    """fp32 partial rows: group g adds rows g, g + GROUPS, ... in sequence
    (dY * X is exact in fp32 for bf16 inputs; one fma with rstd per row)"""
    part = np.zeros((GROUPS, N_COLS), np.float32)
    for k in range(N_ROWS // GROUPS):
        rows = slice(k * GROUPS, (k + 1) * GROUPS)
        prod = (dYf[rows] * Xf[rows]).astype(np.float32)
        part = (part + prod * rs32[rows, None]).astype(np.float32)
    return part


def test_sum_gate_passes_an_fp32_reduction(config2):
    Xf, dYf, rs32, dw_pre, dw_abs = config2
    dw = partial_rows(Xf, dYf, rs32).sum(axis=0, dtype=np.float32)
    check_f32(dw, dw_pre, floor=sum_gate(dw_abs), what="fp32 model of the dW reduction")
    # its error is a small fraction of the gate
    assert (np.abs(dw - dw_pre) / (U32 * dw_abs)).max() < 1.0


def test_sum_gate_rejects_fp16_partial_rows(config2):
    Xf, dYf, rs32, dw_pre, dw_abs = config2
    part16 = partial_rows(Xf, dYf, rs32).astype(np.float16).astype(np.float32)
    dw = part16.sum(axis=0, dtype=np.float32)
    with pytest.raises(AssertionError):
        check_f32(dw, dw_pre, floor=sum_gate(dw_abs), what="dW from fp16 partial rows")
    tol = 1e-5 * np.abs(dw_pre) + sum_gate(dw_abs)
    assert (np.abs(dw - dw_pre) > tol).mean() > 0.5
    # the worst-case bound of the kernel's summation tree (depth 65 at this
    # shape) is too wide to see it on many of those columns
    loose = 1e-5 * np.abs(dw_pre) + gamma(65) * dw_abs
    assert (np.abs(dw - dw_pre) > loose).mean() < (np.abs(dw - dw_pre) > tol).mean()


def test_loss_gate_rejects_a_first_order_loss_sum():
    """The fused loss kernel sums exp(x - m) over the unrounded differences
    itself. A cheaper sum built from the softmax's exp(d), d = bf16(x - m),
    corrected in dl = (x - m) - d, must fail the GPU tests' 1e-4 loss gate on
    confident rows (support.confident_logits) when the correction stops at
    first order, and pass it at second order: CPU models of both against the
    oracle."""
    shape = (64, 128256)
    X, labels = confident_logits(shape, 710)
    n_rows, n_cols = shape
    lo, hi, loss, mean = np.empty(shape), np.empty(shape), np.empty(n_rows), np.zeros(1)
    assert oracle().oracle_softmax_cross_entropy(BF16, n_rows, n_cols, ptr(X), ptr(labels), ptr(lo), ptr(hi), ptr(loss),
                                                 ptr(mean)) == 0
    x = bf16_bits_to_f32(X).astype(np.float64)
    m = x.max(axis=1, keepdims=True)
    e = x - m
    d = bf16_bits_to_f32(to_storage(e.astype(np.float32), BF16)).astype(np.float64)
    dl = e - d
    xl = e[np.arange(n_rows), labels]
    second = np.log((np.exp(d) * (1.0 + dl + 0.5 * dl * dl)).sum(axis=1)) - xl
    first = np.log((np.exp(d) * (1.0 + dl)).sum(axis=1)) - xl
    check_f32(second.astype(np.float32), loss, rel=1e-4, what="second-order loss model")
    with pytest.raises(AssertionError):
        check_f32(first.astype(np.float32), loss, rel=1e-4, what="first-order loss model")
