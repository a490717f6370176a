"""The allocation-free entry point (include/dataflow_noalloc.h) against the
handle's submit_rms_norm_bwd, through the C ABI on an AMD GPU.

Both run the same kernels with the same launch shape, so dX and dW must be
bit-identical; each test makes two calls in a row on the no-alloc path, the
second with a smaller input, so partial rows a previous call left in the
shared scratch cannot leak into a later result. Host-side rejections (sizes
past the scratch or LDS, unsupported types) return -1 without launching.
"""
import numpy as np
import pytest

from support import BF16, FP16, FP32, NP_STORAGE, normal, to_storage

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hdl():
    from dataflow_lib_amd import api
    h = api.Handle(0, num_streams=1)
    yield h
    h.destroy()


def inputs(dt, n_rows, n_cols, seed):
    X = to_storage(normal(seed, (n_rows, n_cols)), dt)
    W = to_storage(1.0 + normal(seed + 1, (n_cols,), std=0.02), dt)
    dY = to_storage(normal(seed + 2, (n_rows, n_cols)), dt)
    dX = to_storage(normal(seed + 3, (n_rows, n_cols)), dt)
    dW = normal(seed + 4, (n_cols,), std=0.5)
    return X, W, dY, dX, dW


def run_both(h, dt, n_rows, n_cols, seed):
    """(handle path, no-alloc path) results of one exact backward"""
    from dataflow_lib_amd import api
    X, W, dY, dX, dW = inputs(dt, n_rows, n_cols, seed)
    bufs = []

    def put(a):
        p = h.to_device(np.ascontiguousarray(a))
        bufs.append(p)
        return p
    try:
        px, pw, pdy = put(X), put(W), put(dY)
        prs = h.alloc(4 * n_rows)
        bufs.append(prs)
        py = h.alloc(X.nbytes)
        bufs.append(py)
        assert api.submit_rms_norm(h, 0, dt, n_rows, n_cols, 1e-5, pw, px, py, None, prs) == 0
        out = []
        for path in ("handle", "noalloc"):
            pdx, pdw = put(dX), put(dW)
            if path == "handle":
                rc = api.submit_rms_norm_bwd(h, 0, dt, dt, n_rows, n_cols, 1e-5, prs, pw, px, pdy, pdx, pdw)
            else:
                rc = api.rms_norm_bwd_noalloc(h.stream(0), dt, dt, n_rows, n_cols, 1e-5, prs, pw, px, pdy, pdx, pdw)
            assert rc == 0, path
            h.sync()
            out.append((h.to_host(pdx, X.shape, NP_STORAGE[dt]), h.to_host(pdw, (n_cols,), np.float32)))
        return out
    finally:
        h.sync()
        for p in bufs:
            h.free(p)


def assert_same(a, b, what):
    (xa, wa), (xb, wb) = a, b
    assert np.array_equal(xa.view(np.uint8), xb.view(np.uint8)), what + ": dX differs"
    assert np.array_equal(wa.view(np.uint32), wb.view(np.uint32)), what + ": dW differs"


@pytest.mark.parametrize("dt", [BF16, FP16, FP32], ids=["bf16", "fp16", "fp32"])
def test_noalloc_matches_handle_two_calls_shrinking(hdl, dt):
    # the Llama-3-8B batch (every workgroup writes a partial row), then a
    # smaller call whose partial rows cover only part of what the first left
    big = run_both(hdl, dt, 8192, 4096, seed=71)
    assert_same(big[0], big[1], "8192x4096")
    small = run_both(hdl, dt, 300, 1024, seed=72)
    assert_same(small[0], small[1], "300x1024")


def test_noalloc_element_path_and_repeat(hdl):
    # ragged rows take the element path; the second call is smaller again
    a = run_both(hdl, BF16, 700, 4099, seed=73)
    assert_same(a[0], a[1], "700x4099")
    b = run_both(hdl, BF16, 5, 1001, seed=74)
    assert_same(b[0], b[1], "5x1001")


def test_noalloc_rejects_without_launching(hdl):
    from dataflow_lib_amd import api
    s = hdl.stream(0)
    # unsupported type pairs
    assert api.rms_norm_bwd_noalloc(s, BF16, FP32, 4, 64, 1e-5, None, None, None, None, None, None) == -1
    assert api.rms_norm_bwd_noalloc(s, 6, 6, 4, 64, 1e-5, None, None, None, None, None, None) == -1
    # negative sizes; rows whose dW partial sums exceed the LDS (200000 fp32
    # columns) or the scratch
    assert api.rms_norm_bwd_noalloc(s, BF16, BF16, -1, 64, 1e-5, None, None, None, None, None, None) == -1
    assert api.rms_norm_bwd_noalloc(s, FP32, FP32, 4, 200000, 1e-5, None, None, None, None, None, None) == -1
    # nothing to do: 0, nothing launched
    assert api.rms_norm_bwd_noalloc(s, BF16, BF16, 0, 64, 1e-5, None, None, None, None, None, None) == 0
    assert api.rms_norm_bwd_noalloc(s, BF16, BF16, 4, 0, 1e-5, None, None, None, None, None, None) == 0
    assert hdl.sync() == 0
