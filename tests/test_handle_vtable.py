"""The Dataflow_Handle vtable calls around the ops (src/dataflow_handle/include/
dataflow_handle.h:72-118): memory set, the three transfers, stream states and
dependencies, host functions and stream syncs, on an AMD GPU."""
import ctypes

import numpy as np
import pytest

from support import BF16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hdl():
    from dataflow_lib_amd import api
    h = api.Handle(0, num_streams=2)
    yield h
    h.destroy()


def test_set_mem_on_a_stream_and_blocking(hdl):
    n = (1 << 20) + 3
    p = hdl.alloc(n)
    try:
        assert hdl.set_mem(p, 0xA5, n, stream_id=1) == 0
        assert hdl.sync_stream(1) == 0
        assert (hdl.to_host(p, (n,), np.uint8) == 0xA5).all()
        assert hdl.set_mem(p, 0x3C, n // 2) == 0   # stream -1: blocking
        out = hdl.to_host(p, (n,), np.uint8)
        assert (out[: n // 2] == 0x3C).all() and (out[n // 2:] == 0xA5).all()
    finally:
        hdl.free(p)


def test_transfers_round_trip_on_streams(hdl):
    """inbound, device-to-device (dst <- src, the direction the reference's
    D2D copy got backwards) and outbound, each queued on stream 1"""
    x = np.random.default_rng(1).integers(0, 256, 3 * (1 << 20) + 7).astype(np.uint8)
    a, b = hdl.alloc(x.nbytes), hdl.alloc(x.nbytes)
    back = np.zeros_like(x)
    try:
        assert hdl.set_mem(b, 0, x.nbytes) == 0
        assert hdl._fns["submit_inbound_transfer"](hdl.ref, 1, a, x.ctypes.data, x.nbytes) == 0
        assert hdl.copy(b, a, x.nbytes, stream_id=1) == 0
        assert hdl._fns["submit_outbound_transfer"](hdl.ref, 1, back.ctypes.data, b, x.nbytes) == 0
        assert hdl.sync_stream(1) == 0
        assert np.array_equal(back, x)
        assert np.array_equal(hdl.to_host(a, x.shape, np.uint8), x)   # the source is unchanged
    finally:
        hdl.free(a)
        hdl.free(b)


def test_blocking_fill_and_copy_are_done_before_stream_work(hdl):
    """stream -1 set_mem and device-to-device copies are complete when they
    return: a copy queued right after them on a (non-blocking) handle stream
    sees every byte they wrote (256 MiB, long enough that a fill or copy still
    in flight would be caught)"""
    n = 256 << 20
    a, b, c = hdl.alloc(n), hdl.alloc(n), hdl.alloc(n)
    try:
        assert hdl.set_mem(c, 0, n) == 0
        assert hdl.set_mem(a, 0x5A, n) == 0
        assert hdl.copy(c, a, n, stream_id=1) == 0
        assert hdl.sync_stream(1) == 0
        assert (hdl.to_host(c, (n,), np.uint8) == 0x5A).all()
        assert hdl.set_mem(b, 0, n, stream_id=1) == 0
        assert hdl.sync_stream(1) == 0
        assert hdl.set_mem(a, 0xC3, n) == 0
        assert hdl.copy(b, a, n) == 0   # stream -1: blocking
        assert hdl.copy(c, b, n, stream_id=1) == 0
        assert hdl.sync_stream(1) == 0
        assert (hdl.to_host(c, (n,), np.uint8) == 0xC3).all()
    finally:
        for p in (a, b, c):
            hdl.free(p)


def test_dependency_orders_a_copy_after_an_op_on_another_stream(hdl):
    """stream 1 waits for stream 0's state before copying what stream 0's op
    writes, so the copy holds the op's output, not the sentinel before it"""
    from dataflow_lib_amd import api
    rows, cols = 4096, 14336
    n = rows * cols * 2
    g = (np.random.default_rng(2).standard_normal(rows * cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    pg, pu, po, pc = hdl.to_device(g), hdl.to_device(g), hdl.alloc(n), hdl.alloc(n)
    try:
        assert hdl.set_mem(po, 0x7F, n) == 0 and hdl.set_mem(pc, 0, n) == 0
        assert api.submit_swiglu(hdl, 0, BF16, rows, cols, pg, pu, po) == 0
        state = hdl.stream_state(0)
        assert state
        assert hdl.submit_dependency(1, state) == 0
        assert hdl.copy(pc, po, n, stream_id=1) == 0
        assert hdl.sync() == 0
        out, cp = hdl.to_host(po, (rows * cols,), np.uint16), hdl.to_host(pc, (rows * cols,), np.uint16)
        assert not (out == 0x7F7F).all()
        assert np.array_equal(cp, out)
    finally:
        for p in (pg, pu, po, pc):
            hdl.free(p)


def test_host_op_runs_after_the_streams_earlier_work(hdl):
    from dataflow_lib_amd import api
    seen = []
    n = 1 << 16
    p = hdl.alloc(n)
    probe = np.zeros(n, np.uint8)

    def cb(arg):   # runs on a runtime thread once the set_mem before it is done
        seen.append(int(arg or 0))

    fn = api.HostFunc(cb)
    try:
        assert hdl.set_mem(p, 0x11, n, stream_id=0) == 0
        assert hdl.submit_host_op(fn, 1234, stream_id=0) == 0
        assert hdl._fns["submit_outbound_transfer"](hdl.ref, 0, probe.ctypes.data, p, n) == 0
        assert hdl.sync_stream(0) == 0
        assert seen == [1234]
        assert (probe == 0x11).all()
    finally:
        hdl.free(p)


def test_bad_stream_ids_are_errors(hdl):
    assert hdl.sync_stream(2) == -1
    assert hdl.stream_state(5) is None
    assert hdl.submit_dependency(0, None) == -1
    assert hdl.set_mem(0, 0, 0, stream_id=9) == -1
