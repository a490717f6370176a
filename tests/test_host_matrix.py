"""The raw .dat host-matrix format and the host matrix generators
(reference: src/dataflow_handle/nvidia/test/create_host_matrix.c:4-291),
through libdataflow.so. A .dat file holds exactly the M x N row-major element
bytes; loading converts between fp32/fp16/bf16 with round-to-nearest-even."""
import ctypes

import numpy as np
import pytest

from support import BF16, FP16, FP32, f32_to_bf16_bits, ptr

from dataflow_lib_amd import api

L = api.lib()
vp, u64 = ctypes.c_void_p, ctypes.c_uint64
L.create_zero_host_matrix.restype = vp
L.create_zero_host_matrix.argtypes = [u64, u64, ctypes.c_int, vp]
L.create_rand_host_matrix.restype = vp
L.create_rand_host_matrix.argtypes = [u64, u64, ctypes.c_float, ctypes.c_float, ctypes.c_int, vp]
L.create_identity_host_matrix.restype = vp
L.create_identity_host_matrix.argtypes = [u64, ctypes.c_int, vp]
L.create_index_identity_host_matrix.restype = vp
L.create_index_identity_host_matrix.argtypes = [u64, u64, ctypes.c_int, vp]
L.load_host_matrix_from_file.restype = vp
L.load_host_matrix_from_file.argtypes = [ctypes.c_char_p, u64, u64, ctypes.c_int, ctypes.c_int, vp]
L.save_host_matrix.argtypes = [ctypes.c_char_p, vp, u64, u64, ctypes.c_int]
L.host_matrix_seed.argtypes = [u64]
NP = {FP32: np.float32, FP16: np.float16, BF16: np.uint16}


def into(M, N, dt):
    return np.full((M, N), 0x7F, dtype=NP[dt]) if dt != FP32 else np.full((M, N), np.nan, np.float32)


def test_save_writes_exactly_the_element_bytes(tmp_path):
    a = np.random.default_rng(1).standard_normal((7, 13)).astype(np.float32)
    f = str(tmp_path / "a.dat").encode()
    assert L.save_host_matrix(f, ptr(a), 7, 13, FP32) == 0
    assert open(f, "rb").read() == a.tobytes()
    assert L.save_host_matrix(str(tmp_path / "no/such/dir.dat").encode(), ptr(a), 7, 13, FP32) == -1


@pytest.mark.parametrize("orig, new", [(FP32, BF16), (FP32, FP16), (BF16, FP32), (FP16, BF16), (FP32, FP32)])
def test_load_converts_with_rne(tmp_path, orig, new):
    x = (np.random.default_rng(2).standard_normal((5, 33)) * 3).astype(np.float32)
    x[0, :4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -0.0, 65504.0]   # bf16 ties to even, signed zero
    src = {FP32: x, FP16: x.astype(np.float16), BF16: f32_to_bf16_bits(x)}[orig]
    f = str(tmp_path / "m.dat").encode()
    assert L.save_host_matrix(f, ptr(src), 5, 33, orig) == 0
    dst = into(5, 33, new)
    assert L.load_host_matrix_from_file(f, 5, 33, orig, new, ptr(dst)) == dst.ctypes.data
    as32 = {FP32: lambda a: a, FP16: lambda a: a.astype(np.float32),
            BF16: lambda a: (a.astype(np.uint32) << 16).view(np.float32)}[orig](src)
    with np.errstate(over="ignore"):      # bf16 65536 overflows fp16 to inf, as RNE requires
        expect = {FP32: as32, FP16: as32.astype(np.float16), BF16: f32_to_bf16_bits(as32)}[new]
    assert np.array_equal(dst.view(np.uint8), expect.view(np.uint8))


def test_load_refuses_short_files(tmp_path):
    f = str(tmp_path / "s.dat").encode()
    open(f, "wb").write(b"\0" * 10)
    dst = into(2, 3, FP32)
    assert L.load_host_matrix_from_file(f, 2, 3, FP32, FP32, ptr(dst)) is None
    assert L.load_host_matrix_from_file(str(tmp_path / "missing.dat").encode(), 2, 3, FP32, FP32, ptr(dst)) is None


def test_identity_and_index_identity():
    n = 37
    eye = into(n, n, FP32)
    assert L.create_identity_host_matrix(n, FP32, ptr(eye)) is not None
    assert np.array_equal(eye, np.eye(n, dtype=np.float32))          # off-diagonal zeroed
    idx = into(300, 1000, BF16)
    assert L.create_index_identity_host_matrix(300, 1000, BF16, ptr(idx)) is not None
    assert np.array_equal(idx, f32_to_bf16_bits(np.arange(300 * 1000, dtype=np.float32).reshape(300, 1000)))
    z = into(4, 4, FP16)
    assert L.create_zero_host_matrix(4, 4, FP16, ptr(z)) is not None and not z.any()


def test_rand_is_seeded_normal_and_rounds_to_the_type():
    M, N = 1000, 1000
    a, b, h = into(M, N, FP32), into(M, N, FP32), into(M, N, BF16)
    L.host_matrix_seed(7)
    L.create_rand_host_matrix(M, N, 0.5, 2.0, FP32, ptr(a))
    L.host_matrix_seed(7)
    L.create_rand_host_matrix(M, N, 0.5, 2.0, BF16, ptr(h))
    L.host_matrix_seed(8)
    L.create_rand_host_matrix(M, N, 0.5, 2.0, FP32, ptr(b))
    assert np.array_equal(h, f32_to_bf16_bits(a))                    # same draws, then RNE
    assert not np.array_equal(a, b)
    z = (a.astype(np.float64) - 0.5) / 2.0
    n = z.size
    assert abs(z.mean()) < 5 / np.sqrt(n) and abs(z.var() - 1) < 5 * np.sqrt(2 / n)
    assert abs((z ** 3).mean()) < 5 * np.sqrt(15 / n)               # symmetric
    assert abs(np.mean(np.abs(z) < 1) - 0.682689) < 5 * np.sqrt(0.2167 / n)


def test_libc_generator_reproduces_the_reference_harness_draws():
    """host_matrix_set_generator(HOST_MATRIX_RAND_LIBC): the same values, bit
    for bit, as the reference harnesses' rand_normal (compiled from
    test/create_host_matrix.c into oracle/_ref) after the same srand(), including
    the value kept back across calls and std == 0 drawing nothing"""
    import os
    from support import REF_HOST_LIB
    if not os.path.exists(REF_HOST_LIB):
        pytest.skip("reference host library not built (needs /root/reference)")
    ref = ctypes.CDLL(REF_HOST_LIB)
    if not hasattr(ref, "rand_normal"):
        pytest.skip("reference host library predates rand_normal export")
    ref.rand_normal.restype = ctypes.c_float
    ref.rand_normal.argtypes = [ctypes.c_float, ctypes.c_float]
    libc = ctypes.CDLL("libc.so.6")
    L.host_matrix_set_generator.argtypes = [ctypes.c_int]
    assert L.host_matrix_set_generator(7) == -1
    assert L.host_matrix_set_generator(1) == 0
    try:
        libc.srand(1234)
        a = into(37, 54, FP32)
        L.create_rand_host_matrix(37, 54, 0.5, 2.0, FP32, ptr(a))
        libc.srand(1234)
        e = np.array([ref.rand_normal(0.5, 2.0) for _ in range(a.size)], np.float32)
        assert np.array_equal(a.ravel().view(np.uint32), e.view(np.uint32))
        # an odd count keeps one value back for the next matrix, as rand_normal does
        libc.srand(99)
        p, q = into(1, 5, FP32), into(1, 7, FP32)
        L.create_rand_host_matrix(1, 5, 0.0, 1.0, FP32, ptr(p))
        L.create_rand_host_matrix(1, 7, 0.0, 1.0, FP32, ptr(q))
        libc.srand(99)
        e = np.array([ref.rand_normal(0.0, 1.0) for _ in range(12)], np.float32)
        assert np.array_equal(np.concatenate([p.ravel(), q.ravel()]).view(np.uint32), e.view(np.uint32))
        # std == 0 gives the mean and consumes no draws
        libc.srand(5)
        c, d = into(1, 2, FP32), into(1, 4, FP32)
        L.create_rand_host_matrix(1, 2, 3.0, 0.0, FP32, ptr(c))
        L.create_rand_host_matrix(1, 4, 0.0, 1.0, FP32, ptr(d))
        libc.srand(5)
        e = np.array([ref.rand_normal(0.0, 1.0) for _ in range(4)], np.float32)
        assert np.all(c == 3.0) and np.array_equal(d.ravel(), e)
        # the other types are the same draws rounded to nearest even
        libc.srand(42)
        f = into(8, 16, FP32)
        L.create_rand_host_matrix(8, 16, 0.0, 1.0, FP32, ptr(f))
        libc.srand(42)
        h = into(8, 16, BF16)
        L.create_rand_host_matrix(8, 16, 0.0, 1.0, BF16, ptr(h))
        assert np.array_equal(h, f32_to_bf16_bits(f))
    finally:
        assert L.host_matrix_set_generator(0) == 0
