#!/usr/bin/env python3
"""Per-op HBM throughput of the native op path on one MI355X (gfx950).

Metric: achieved HBM GB/s and % of the 8 TB/s peak per op at
Llama-3-8B token shapes. A "step" is one pass of the hot path: each op below
once, on its next rotating buffer set, through the C ABI (submit_* on stream 0):

  rms_norm_fwd          bf16 X [8192 x 4096]                       (config 2)
  rms_norm_bwd          fused exact-gradient bwd, dX += , dW fp32    (config 2)
  rope_fwd / rope_bwd   bf16 Q [8192 x 32 x 128], K [8192 x 8 x 128] (config 3)
  swiglu_fwd / _bwd     bf16 [8192 x 14336]                          (config 4)
  softmax_xent_fused    bf16 logits [4096 x 128256], loss + mean     (config 5)

Inputs are resident in HBM before timing. Each op rotates through enough
buffer sets that its working set per rotation is >= 1 GiB, so the 256 MB
Infinity Cache cannot serve repeats. The K timed steps run back to back
between two events on the launch stream (an event between kernels would add
several microseconds of stream time to every op). The start event is recorded
behind the queued warm-up launches, with no host synchronization in between,
so the GPU is busy when it fires, and an untimed settle phase (every buffer
set once, then SETTLE_STEPS steps) runs before the warm-up, since the first
steps after the GPU has idled run ~2 % slower: the timed region is steady
state at any K.
`value` = sum of per-op algorithmic bytes / measured step time. Per-op time =
the average launch duration of K back-to-back launches of that op alone
(rotating its sets, behind a few queued untimed launches), between two events
on the launch stream. Timed as extras, outside `value`: the
reference-compatible split ops (rms_norm_bwd_x, rms_norm_bwd_w, softmax,
cross_entropy_loss) and the path's neighbours (embedding gather of 8192 rows
of a 128256 x 4096 bf16 table; copy_to_seq_context of K, V [8192 x 1024] bf16
into 4 contexts of 2048 positions; rope_copy_to_seq_context, RoPE fused with
that scatter, on the config-3 Q, K and those contexts) and the fp8 variants
at the same shapes (E4M3 forward tensors, bf16 backward ones). `storage_types`:
the step again with fp16 and with fp32 storage at the same shapes (each
op's bytes scaled by its element size), its own step time and per-op
times. `transformer_head`:
the loss-path driver
(submit_transformer_head, training pass) at 4096 tokens x 4096 x 128256, whose
time is its three hipBLASLt GEMMs (reported in TFLOP/s).

copy_reference: per op, a streaming copy (a code object of its own, not the
product's) moving the same
total bytes (half read, half written), timed the same way - the ceiling the
memory system offers that many bytes (the op's time over it is reported).

cpu_baseline: a C CPU implementation of the same math (oracle/libcpu_ref.so:
fp32 arithmetic, fp64 reductions, OpenMP over rows, AVX-512) on the full
configs, timed on this host's cores.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
GiB = 1 << 30
BF16 = 5
FP16 = 4
FP32 = 3
ELEM_BYTES = {BF16: 2, FP16: 2, FP32: 4}
NORMAL_FILL = {BF16: "normal_bf16", FP16: "normal_fp16", FP32: "normal_fp32"}


class Hip:
    """hipEvent timing through the same HIP runtime libdataflow.so uses."""

    def __init__(self):
        self.L = ctypes.CDLL(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so"))
        self.L.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.L.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.L.hipEventCreate(ctypes.byref(e)) == 0
        return e.value

    def record(self, ev, stream):
        assert self.L.hipEventRecord(ev, stream) == 0

    def module_function(self, path, name):
        self.L.hipModuleLoad.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p]
        self.L.hipModuleGetFunction.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_char_p]
        if not hasattr(self, "modules"):
            self.modules = {}
        if path not in self.modules:
            m = ctypes.c_void_p()
            assert self.L.hipModuleLoad(ctypes.byref(m), path.encode()) == 0, path
            self.modules[path] = m.value
        f = ctypes.c_void_p()
        assert self.L.hipModuleGetFunction(ctypes.byref(f), self.modules[path], name.encode()) == 0, name
        return f.value

    def launch(self, f, grid, block, args, stream):
        self.L.hipModuleLaunchKernel.argtypes = [ctypes.c_void_p] + [ctypes.c_uint] * 7 + [
            ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p]
        arr = (ctypes.c_void_p * len(args))(*[ctypes.cast(ctypes.pointer(a), ctypes.c_void_p) for a in args])
        assert self.L.hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, 0, stream, arr, None) == 0

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        assert self.L.hipEventSynchronize(b) == 0
        assert self.L.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return float(ms.value)


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def fp8e4m3_bits(x):
    """fp32 -> OCP E4M3 codes (bias 7, 3 mantissa bits), round to nearest
    even, saturating at +-448 (synthetic inputs of the fp8 extras)"""
    x = np.asarray(x, np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    a = np.minimum(np.abs(x), 448.0)
    quantum = np.exp2(np.floor(np.log2(np.maximum(a, 2.0 ** -6))) - 3)
    r = np.round(a / quantum) * quantum
    e = np.floor(np.log2(np.maximum(r, 2.0 ** -6)))
    normal = r >= 2.0 ** -6
    field = np.where(normal, e + 7, 0).astype(np.uint8)
    mant = (np.where(normal, r / np.exp2(e) - 1.0, r / 2.0 ** -6) * 8).astype(np.uint8)
    return sign | (field << 3) | mant


class Pool:
    """Device buffers filled by tiling seeded host blocks (device-to-device copies)."""

    def __init__(self, h, block_elems=1 << 24):
        self.h, self.bufs, self.blocks = h, [], {}
        self.block_elems = block_elems

    def _block(self, key):
        if key not in self.blocks:
            kind, seed, a, b = key
            g = np.random.default_rng(seed)
            if kind == "normal_bf16":
                host = bf16_bits(a + b * g.standard_normal(self.block_elems, dtype=np.float32))
            elif kind == "normal_fp16":
                host = (a + b * g.standard_normal(self.block_elems, dtype=np.float32)).astype(np.float16)
            elif kind == "normal_fp32":
                host = a + b * g.standard_normal(self.block_elems, dtype=np.float32)
            elif kind == "normal_fp8e4m3":
                host = fp8e4m3_bits(a + b * g.standard_normal(self.block_elems, dtype=np.float32))
            elif kind == "zeros":
                host = np.zeros(self.block_elems, np.uint16)
            else:
                raise ValueError(kind)
            self.blocks[key] = (self.h.to_device(host), host.nbytes)
        return self.blocks[key]

    def fill(self, nbytes, kind, seed=0, a=0.0, b=1.0):
        p = self.h.alloc(nbytes)
        self.bufs.append(p)
        src, bb = self._block((kind, seed, a, b))
        off = 0
        while off < nbytes:
            n = min(bb, nbytes - off)
            assert self.h.copy(p + off, src, n) == 0
            off += n
        return p

    def put(self, arr):
        p = self.h.to_device(np.ascontiguousarray(arr))
        self.bufs.append(p)
        return p

    def empty(self, nbytes):
        p = self.h.alloc(nbytes)
        self.bufs.append(p)
        return p

    def free(self, p):
        self.h.sync()
        self.bufs.remove(p)
        self.h.free(p)

    def release(self):
        self.h.sync()
        for p in self.bufs:
            self.h.free(p)
        for p, _ in self.blocks.values():
            self.h.free(p)


def n_sets(set_bytes):
    return max(1, -(-GiB // set_bytes))


def build_ops(h, pool, api, dt=BF16):
    """(name, algorithmic bytes per launch, list of per-set callables); `dt`
    is the storage type of every tensor but the fp32 statistics and dW"""
    es, fill = ELEM_BYTES[dt], NORMAL_FILL[dt]
    ops = []
    T, D = 8192, 4096
    act = T * D * es
    # --- RMSNorm fwd: read X, W; write Y, weighted_sums, rstd
    b_fwd = 2 * act + D * es + 2 * T * 4
    runs = []
    for s in range(n_sets(2 * act)):
        X = pool.fill(act, fill, 1)
        W = pool.fill(D * es, fill, 2, 1.0, 0.02)
        Y, ws, rs = pool.empty(act), pool.empty(T * 4), pool.empty(T * 4)
        runs.append(lambda X=X, W=W, Y=Y, ws=ws, rs=rs: api.submit_rms_norm(h, 0, dt, T, D, 1e-5, W, X, Y, ws, rs))
    ops.append(("rms_norm_fwd", b_fwd, runs))
    # --- fused RMSNorm bwd: read X, dY, dX, W, rstd; write dX; dW fp32 read-modify-write
    b_bwd = 4 * act + D * es + T * 4 + 2 * D * 4
    runs = []
    for s in range(n_sets(4 * act)):
        X = pool.fill(act, fill, 1)
        W = pool.fill(D * es, fill, 2, 1.0, 0.02)
        dY = pool.fill(act, fill, 3)
        dX = pool.fill(act, "zeros")
        rs = pool.empty(T * 4)
        Y = pool.empty(act)
        assert api.submit_rms_norm(h, 0, dt, T, D, 1e-5, W, X, Y, None, rs) == 0
        dW = pool.put(np.zeros(D, np.float32))
        runs.append(lambda X=X, W=W, dY=dY, dX=dX, rs=rs, dW=dW:
                    api.submit_rms_norm_bwd(h, 0, dt, dt, T, D, 1e-5, rs, W, X, dY, dX, dW))
    ops.append(("rms_norm_bwd", b_bwd, runs))
    # --- RoPE fwd / bwd (in place): Q [T x 4096], K [T x 1024], positions t mod 2048
    q, k = T * 4096 * es, T * 1024 * es
    b_rope = 2 * (q + k) + T * 4
    pos = pool.put((np.arange(T) % 2048).astype(np.int32))
    for name, fn in (("rope_fwd", api.submit_rope), ("rope_bwd", api.submit_rope_bwd_x)):
        runs = []
        for s in range(n_sets(2 * (q + k))):
            Q = pool.fill(q, fill, 4)
            K = pool.fill(k, fill, 5)
            runs.append(lambda Q=Q, K=K, fn=fn: fn(h, 0, dt, T * 4096, 4096, 128, 8, 500000, pos, Q, K))
        ops.append((name, b_rope, runs))
    # --- SwiGLU fwd (3T) / bwd (5T), [T x 14336]
    F = 14336
    t = T * F * es
    runs = []
    for s in range(n_sets(3 * t)):
        g, u, o = pool.fill(t, fill, 6), pool.fill(t, fill, 7), pool.empty(t)
        runs.append(lambda g=g, u=u, o=o: api.submit_swiglu(h, 0, dt, T, F, g, u, o))
    ops.append(("swiglu_fwd", 3 * t, runs))
    runs = []
    for s in range(n_sets(5 * t)):
        g, u, d = pool.fill(t, fill, 6), pool.fill(t, fill, 7), pool.fill(t, fill, 8)
        dg, du = pool.empty(t), pool.empty(t)
        runs.append(lambda g=g, u=u, d=d, dg=dg, du=du: api.submit_swiglu_bwd_x(h, 0, dt, dt, T, F, g, u, d, dg, du))
    ops.append(("swiglu_bwd", 5 * t, runs))
    # --- fused softmax + cross-entropy, in place: logits [4096 x 128256]
    R, V = 4096, 128256
    lg = R * V * es
    b_ce = 2 * lg + R * 4 + R * 4 + 4
    labels = pool.put(np.random.default_rng(9).integers(0, V, size=R).astype(np.uint32))
    runs = []
    for s in range(n_sets(2 * lg)):
        L = pool.fill(lg, fill, 10, 0.0, 2.0)
        loss, mean = pool.empty(R * 4), pool.empty(4)
        runs.append(lambda L=L, loss=loss, mean=mean: api.submit_softmax_cross_entropy_loss(h, 0, dt, R, V, L, labels, loss, mean))
    ops.append(("softmax_xent_fused", b_ce, runs))
    return ops


def build_extras(h, pool, api):
    """Reference-compatible split ops (not part of `value`)."""
    ops = []
    T, D = 8192, 4096
    act = T * D * 2
    runs_x, runs_w = [], []
    for s in range(n_sets(4 * act)):
        X = pool.fill(act, "normal_bf16", 1)
        W = pool.fill(D * 2, "normal_bf16", 2, 1.0, 0.02)
        dY = pool.fill(act, "normal_bf16", 3)
        dX = pool.fill(act, "zeros")
        ws, rs, Y = pool.empty(T * 4), pool.empty(T * 4), pool.empty(act)
        assert api.submit_rms_norm(h, 0, BF16, T, D, 1e-5, W, X, Y, ws, rs) == 0
        dW = pool.fill(D * 2, "zeros")
        runs_x.append(lambda X=X, W=W, dY=dY, dX=dX, ws=ws, rs=rs:
                      api.submit_rms_norm_bwd_x(h, 0, BF16, BF16, T, D, 1e-5, ws, rs, W, X, dY, dX))
        runs_w.append(lambda X=X, dY=dY, rs=rs, dW=dW: api.submit_rms_norm_bwd_w(h, 0, BF16, BF16, T, D, 1e-5, rs, X, dY, dW))
    ops.append(("rms_norm_bwd_x", 4 * act + D * 2 + 2 * T * 4, runs_x))
    ops.append(("rms_norm_bwd_w", 2 * act + T * 4 + 2 * D * 2, runs_w))
    R, V = 4096, 128256
    lg = R * V * 2
    runs = []
    for s in range(n_sets(2 * lg)):
        L, O = pool.fill(lg, "normal_bf16", 10, 0.0, 2.0), pool.empty(lg)
        runs.append(lambda L=L, O=O: api.submit_softmax(h, 0, BF16, BF16, R, V, L, O))
    ops.append(("softmax", 2 * lg, runs))
    labels = pool.put(np.random.default_rng(9).integers(0, V, size=R).astype(np.uint32))
    P = pool.fill(lg, "normal_bf16", 11, 0.0, 1e-3)
    ops.append(("cross_entropy_loss", R * 4 + 2 * R * 2, [lambda: api.submit_cross_entropy_loss(h, 0, BF16, R, V, P, labels)]))
    # --- embedding gather (next to the path): 8192 token rows of a 128256 x 4096 bf16 table
    table = pool.fill(V * D * 2, "normal_bf16", 12)
    runs = []
    for s in range(n_sets(2 * act)):
        ids = pool.put(np.random.default_rng(20 + s).integers(0, V, size=T).astype(np.uint32))
        out = pool.empty(act)
        runs.append(lambda ids=ids, out=out: api.submit_embedding(h, 0, BF16, T, D, ids, table, out))
    ops.append(("embedding", 2 * act + T * 4, runs))
    # --- KV-cache scatter: 8192 tokens (4 sequences x 2048 positions) of K and V [8192 x 1024] bf16
    kv = T * 1024 * 2
    pos = np.arange(T, dtype=np.int32) % 2048
    sizes = np.full(T, 2048, np.int32)
    runs = []
    for s in range(n_sets(4 * kv)):
        K, Vv = pool.fill(kv, "normal_bf16", 30), pool.fill(kv, "normal_bf16", 31)
        ctx = [pool.empty(2 * 2048 * 1024 * 2) for _ in range(4)]
        ptrs = pool.put(np.array([ctx[t // 2048] for t in range(T)], np.uint64))
        pp, ps = pool.put(pos), pool.put(sizes)
        runs.append(lambda K=K, Vv=Vv, pp=pp, ptrs=ptrs, ps=ps:
                    api.submit_copy_to_seq_context(h, 0, BF16, T * 1024, T, 1024, K, Vv, pp, ptrs, ps))
    ops.append(("copy_to_seq_context", 4 * kv + T * (4 + 8 + 4), runs))
    # --- RoPE fused with the KV-cache scatter (config 3 shapes, the contexts above):
    # Q and K read + written, the rotated K and V written to the contexts, V read
    q = T * 4096 * 2
    runs = []
    for s in range(n_sets(2 * q + 5 * kv)):
        Q, K, Vv = pool.fill(q, "normal_bf16", 40), pool.fill(kv, "normal_bf16", 41), pool.fill(kv, "normal_bf16", 42)
        ctx = [pool.empty(2 * 2048 * 1024 * 2) for _ in range(4)]
        ptrs = pool.put(np.array([ctx[t // 2048] for t in range(T)], np.uint64))
        pp, ps = pool.put(pos), pool.put(sizes)
        runs.append(lambda Q=Q, K=K, Vv=Vv, pp=pp, ptrs=ptrs, ps=ps:
                    api.submit_rope_copy_to_seq_context(h, 0, BF16, T * 4096, 4096, 128, 8, 500000, pp, Q, K, Vv, ptrs, ps))
    ops.append(("rope_copy_to_seq_context", 2 * q + 5 * kv + T * (4 + 8 + 4), runs))
    ops += build_fp8_extras(h, pool, api)
    return ops


def build_fp8_extras(h, pool, api):
    """The fp8 variants at the step's shapes, E4M3 forward tensors and bf16
    backward ones (E5M2 runs the same kernels with another decode)."""
    E4, ops = api.DATAFLOW_FP8E4M3, []
    T, D, F, R, V = 8192, 4096, 14336, 4096, 128256
    a8, a16 = T * D, T * D * 2
    runs_f, runs_x, runs_w = [], [], []
    for s in range(n_sets(2 * a8 + 3 * a16)):
        X = pool.fill(a8, "normal_fp8e4m3", 50)
        W = pool.fill(D, "normal_fp8e4m3", 51, 1.0, 0.02)
        Y, ws, ss = pool.empty(a8), pool.empty(T * 4), pool.empty(T * 4)
        dY, dX, dW = pool.fill(a16, "normal_bf16", 52), pool.fill(a16, "zeros"), pool.fill(D * 2, "zeros")
        rs = pool.fill(T * 4, "zeros")
        runs_f.append(lambda X=X, W=W, Y=Y, ws=ws, ss=ss: api.submit_rms_norm(h, 0, E4, T, D, 1e-5, W, X, Y, ws, ss))
        runs_x.append(lambda X=X, W=W, dY=dY, dX=dX, ws=ws, rs=rs:
                      api.submit_rms_norm_bwd_x(h, 0, E4, BF16, T, D, 1e-5, ws, rs, W, X, dY, dX))
        runs_w.append(lambda X=X, dY=dY, rs=rs, dW=dW: api.submit_rms_norm_bwd_w(h, 0, E4, BF16, T, D, 1e-5, rs, X, dY, dW))
    ops.append(("rms_norm_fp8e4m3", 2 * a8 + D + T * 4, runs_f))
    ops.append(("rms_norm_bwd_x_fp8e4m3_bf16", a8 + 3 * a16 + D + 2 * T * 4, runs_x))
    ops.append(("rms_norm_bwd_w_fp8e4m3_bf16", a8 + a16 + T * 4 + 2 * D * 2, runs_w))
    q8, k8 = T * 4096, T * 1024
    pos = np.random.default_rng(53).integers(0, 8192, size=T).astype(np.int32)
    runs = []
    for s in range(n_sets(2 * (q8 + k8))):
        Q, K, pp = pool.fill(q8, "normal_fp8e4m3", 54), pool.fill(k8, "normal_fp8e4m3", 55), pool.put(pos)
        runs.append(lambda Q=Q, K=K, pp=pp: api.submit_rope(h, 0, E4, T * 4096, 4096, 128, 8, 500000, pp, Q, K))
    ops.append(("rope_fp8e4m3", 2 * (q8 + k8) + T * 4, runs))
    f8 = T * F
    runs_f, runs_b = [], []
    for s in range(n_sets(3 * f8 + 6 * f8)):
        G, U = pool.fill(f8, "normal_fp8e4m3", 56, 0.0, 2.0), pool.fill(f8, "normal_fp8e4m3", 57)
        O, dO = pool.empty(f8), pool.fill(2 * f8, "normal_bf16", 58)
        dG, dU = pool.empty(2 * f8), pool.empty(2 * f8)
        runs_f.append(lambda G=G, U=U, O=O: api.submit_swiglu(h, 0, E4, T, F, G, U, O))
        runs_b.append(lambda G=G, U=U, dO=dO, dG=dG, dU=dU: api.submit_swiglu_bwd_x(h, 0, E4, BF16, T, F, G, U, dO, dG, dU))
    ops.append(("swiglu_fp8e4m3", 3 * f8, runs_f))
    ops.append(("swiglu_bwd_x_fp8e4m3_bf16", 8 * f8, runs_b))
    lg8 = R * V
    runs = []
    for s in range(n_sets(3 * lg8)):
        L, O = pool.fill(lg8, "normal_fp8e4m3", 59, 0.0, 2.0), pool.empty(2 * lg8)
        runs.append(lambda L=L, O=O: api.submit_softmax(h, 0, E4, BF16, R, V, L, O))
    ops.append(("softmax_fp8e4m3_bf16", 3 * lg8, runs))
    return ops


# launches queued ahead of every timed batch of one op (and of every copy
# shape), so that its start event fires while the GPU is busy
PREROLL = 3
# untimed steps run before the warm-up (time_ops)
SETTLE_STEPS = 10


def time_ops(h, hip, ops, steps, warmup, batches=20):
    """Time `steps` steps (each op once per step, rotating buffer sets) on one
    stream, with events only at the two ends (an event recorded between
    kernels costs the stream several microseconds, which would be counted as
    the ops' time). Every op first runs once on each of its buffer sets and
    SETTLE_STEPS untimed steps follow (the GPU's first steps after idling run
    slower); the host synchronizes, queues the `warmup` steps, and
    synchronizes again after the timed ones; the start event is recorded right behind the queued
    warm-up launches, with no synchronization in between, so it fires when the
    warm-up's last kernel ends and the timed region is steady state whatever
    `steps` is (a start event recorded on an idle GPU charges the ramp from
    idle to the first timed steps). Then, for the per-op figures, each op
    alone: `steps` launches back to back over its rotating sets, again timed
    from two events and again behind PREROLL queued launches, in `batches`
    batches; the op's time is the median batch's average launch duration
    (kernel plus the gap to the next launch)."""
    stream = h.stream(0)
    # settle phase, untimed, before the warm-up: every rotating buffer set of
    # every op once, then SETTLE_STEPS whole steps. Measured on the MI355X
    # boxes, the first ~7 steps after the GPU has been idle run ~2 % slower
    # (20 timed steps after 3 warm-up steps: 0.851 ms per step; after 10, 30
    # or 60: 0.833-0.837 ms; 100 steps after 3: 0.839 ms), so without it the
    # step time depended on `steps`.
    for name, _, runs in ops:
        for r in runs:
            assert r() == 0, name
    for w in range(SETTLE_STEPS):
        for name, _, runs in ops:
            assert runs[w % len(runs)]() == 0, name
    h.sync()
    for w in range(warmup):
        for name, _, runs in ops:
            assert runs[w % len(runs)]() == 0, name
    a, b = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(a, stream)
    for s in range(steps):
        for name, _, runs in ops:
            assert runs[(warmup + s) % len(runs)]() == 0, name
    hip.record(b, stream)
    h.sync()
    wall = time.perf_counter() - t0
    step_ms = hip.elapsed_ms(a, b) / steps
    per_op = {}
    for name, nbytes, runs in ops:
        avgs = []
        for _ in range(batches):
            for k in range(PREROLL):
                assert runs[(steps + k) % len(runs)]() == 0, name
            hip.record(a, stream)
            for k in range(steps):
                assert runs[k % len(runs)]() == 0, name
            hip.record(b, stream)
            h.sync()
            avgs.append(hip.elapsed_ms(a, b) / steps)
        avg = sorted(avgs)[len(avgs) // 2]
        per_op[name] = {"bytes": nbytes, "avg_us": round(avg * 1e3, 2), "launches": steps, "batches": batches,
                        "batch_us_min_max": [round(min(avgs) * 1e3, 2), round(max(avgs) * 1e3, 2)],
                        "gbps": round(nbytes / (avg * 1e-3) / 1e9, 1),
                        "pct_of_peak": round(100.0 * nbytes / (avg * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1),
                        "rotating_sets": len(runs)}
    return per_op, step_ms, wall


def copy_reference(h, hip, pool, api, per_op, launches):
    """What the memory system offers each op's byte count: the bench code
    object's streaming copy (dataflow_stream_copy_*: non-temporal 16-byte buffer loads
    then stores, grid-stride) moving the same total bytes half read, half
    written, timed like the ops (back-to-back launches over at least two
    rotating buffer sets, >= 2 GiB per rotation, between two events; median of three
    batches per shape); the fastest of six
    launch shapes: grid-stride with 2, 3 or 4 workgroups of 512 per CU and 2
    chunks per step or 1 workgroup of 1024 per CU with 4; blocked (contiguous
    blocks per workgroup, dealt round-robin) with 1 workgroup of 1024 per CU
    and 8 chunks per thread or 2 of 512 with 16."""
    stream = h.stream(0)
    cu = h.device_info.cu_count
    shapes = [("dataflow_stream_copy_u2_kernel", m * cu, 512) for m in (2, 3, 4)] + [
        ("dataflow_stream_copy_u4_kernel", cu, 1024), ("dataflow_stream_copy_blk8_kernel", cu, 1024),
        ("dataflow_stream_copy_blk16_kernel", 2 * cu, 512)]
    fns = [(hip.module_function(api.BENCH_COPY_KERNELS, n), g, b) for n, g, b in shapes]
    out = {}
    a, b = hip.event(), hip.event()
    for name, op in per_op.items():
        half = (op["bytes"] // 2) // 16 * 16
        sets = max(2, min(16, (2 * GiB) // (2 * half)))
        bufs = [(pool.empty(half), pool.empty(half)) for _ in range(sets)]
        best, best_shape = None, None
        for (f, grid, block), (kname, _, _) in zip(fns, shapes):
            run = lambda i: hip.launch(f, grid, block, [ctypes.c_void_p(bufs[i % sets][0]), ctypes.c_void_p(bufs[i % sets][1]),
                                                         ctypes.c_uint64(half // 16)], stream)
            batch = []
            for _ in range(3):
                for i in range(PREROLL):
                    run(launches + i)
                hip.record(a, stream)
                for i in range(launches):
                    run(i)
                hip.record(b, stream)
                h.sync()
                batch.append(hip.elapsed_ms(a, b) / launches * 1e3)
            us = sorted(batch)[1]   # median of three batches, so the fastest shape is not a lucky batch
            if best is None or us < best:
                best, best_shape = us, "%s grid %d block %d" % (kname.replace("dataflow_stream_copy_", "").replace("_kernel", ""), grid, block)
        for src, dst in bufs:
            pool.free(src)
            pool.free(dst)
        out[name] = {"bytes": 2 * half, "copy_us": round(best, 2),
                     "copy_pct_of_peak": round(100.0 * 2 * half / (best * 1e-6) / 1e9 / HBM_PEAK_GBPS, 1),
                     "op_us_over_copy_us": round(op["avg_us"] / best, 3), "copy_shape": best_shape}
    return out


def time_head(h, hip, pool, api, iters):
    """submit_transformer_head, training pass (norm, output projection, fused
    loss, both backward GEMMs, norm backward) at 4096 tokens x 4096 x 128256
    bf16; reported beside the path, not in `value`: its time is the three
    hipBLASLt GEMMs' (6 * T * E * V flop)."""
    T, E, V = 4096, 4096, 128256
    X, wn = pool.fill(T * E * 2, "normal_bf16", 40), pool.fill(E * 2, "normal_bf16", 41, 1.0, 0.02)
    W, dW = pool.fill(V * E * 2, "normal_bf16", 42, 0.0, E ** -0.5), pool.fill(V * E * 2, "zeros")
    dwn, dX = pool.fill(E * 4, "zeros"), pool.fill(T * E * 2, "zeros")
    labels = pool.put(np.random.default_rng(43).integers(0, V, size=T).astype(np.uint32))
    norm, wsum, rs, out = pool.empty(T * E * 2), pool.empty(T * 4), pool.empty(T * 4), pool.empty(T * V * 2)
    loss, gnorm, ws = pool.empty((T + 1) * 4), pool.empty(T * E * 2), pool.empty(32 << 20)
    head = api.TransformerHead(BF16, BF16, 3, 1e-5, api.EmbeddingConfig(V, E), None, wn, W)
    acts = api.TransformerHeadActivations(T, None, norm, wsum, rs, out, ws, 32 << 20)
    ghead = api.TransformerHead(BF16, BF16, 3, 1e-5, api.EmbeddingConfig(V, E), None, dwn, dW)
    gacts = api.TransformerHeadActivations(T, None, gnorm, None, None, None, ws, 32 << 20)
    inp, gstream = api.TransformerBlockTransition(None, X), api.TransformerBlockTransition(None, dX)
    mo = api.TransformerModelOutput(None, None, labels, None, loss, 0.0)
    run = lambda: api.submit_transformer_head(h, 0, 0, inp, head, acts, mo, ghead, gacts, gstream, None)
    for _ in range(2):
        assert run() == 0
    h.sync()
    stream = h.stream(0)
    a, b = hip.event(), hip.event()
    hip.record(a, stream)
    for _ in range(iters):
        assert run() == 0
    hip.record(b, stream)
    ms = hip.elapsed_ms(a, b) / iters
    flop = 6.0 * T * E * V
    return {"ms": round(ms, 3), "matmul_tflops": round(flop / (ms * 1e-3) / 1e12, 1), "tokens": T, "embedding": E,
            "vocab": V, "iters": iters, "note": "submit_transformer_head training pass; GEMMs on hipBLASLt"}


def cpu_info():
    """host CPU description from /proc/cpuinfo: full model name, family /
    model / stepping numbers and the vector ISA flags that matter here"""
    info = {"cpu_model": "", "cpu_family_model_stepping": "", "isa": []}
    fam = mod = step = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and not info["cpu_model"]:
                    info["cpu_model"] = v
                elif k == "cpu family" and fam is None:
                    fam = v
                elif k == "model" and mod is None:
                    mod = v
                elif k == "stepping" and step is None:
                    step = v
                elif k == "flags" and not info["isa"]:
                    have = set(v.split())
                    info["isa"] = [x for x in ("avx2", "fma", "avx512f", "avx512bw", "avx512vl", "avx512_bf16",
                                               "avx512_fp16", "amx_bf16") if x in have]
    except OSError:
        pass
    info["cpu_family_model_stepping"] = "%s/%s/%s" % (fam, mod, step)
    return info


def cpu_baseline(budget_s):
    """oracle/libcpu_ref.so (C: bf16 storage, fp32 math, fp64 row and column
    reductions, OpenMP over rows, AVX-512) on the FULL configs 2-5, timed on
    this host: per op one warm-up, then the median of up to five runs (fewer
    if `budget_s` runs out); GB/s from the same algorithmic byte formulas as
    the GPU ops."""
    L = ctypes.CDLL(os.path.join(ROOT, "oracle", "libcpu_ref.so"))
    vp, i, f32, lg = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_long
    L.cpu_ref_rms_norm_bf16.argtypes = [i, i, f32, vp, vp, vp, vp, vp]
    L.cpu_ref_rms_norm_bwd_bf16.argtypes = [i, i, vp, vp, vp, vp, vp, vp]
    L.cpu_ref_rope_bf16.argtypes = [i, lg, i, i, i, i, vp, vp, vp]
    L.cpu_ref_swiglu_bf16.argtypes = [lg, vp, vp, vp]
    L.cpu_ref_swiglu_bwd_bf16.argtypes = [lg, vp, vp, vp, vp, vp]
    L.cpu_ref_softmax_xent_bf16.argtypes = [i, i, vp, vp, vp, vp]
    g = np.random.default_rng(0)
    block = bf16_bits(g.standard_normal(1 << 22, dtype=np.float32))

    def tiled(n, scale=1.0, offset=0.0):
        if scale == 1.0 and offset == 0.0:
            return np.resize(block, n)
        return np.resize(bf16_bits(offset + scale * (block.view(np.uint16).astype(np.uint32) << 16).view(np.float32)), n)

    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    T, D, F, R, V = 8192, 4096, 14336, 4096, 128256
    X, dY, dX = tiled(T * D), np.resize(block[::-1].copy(), T * D), np.zeros(T * D, np.uint16)
    W = tiled(D, 0.02, 1.0)
    Y, ws, rs, dW = np.empty(T * D, np.uint16), np.empty(T, np.float32), np.empty(T, np.float32), np.zeros(D, np.float32)
    L.cpu_ref_rms_norm_bf16(T, D, 1e-5, P(W), P(X), P(Y), P(ws), P(rs))
    Q, K, pos = tiled(T * 4096), tiled(T * 1024), (np.arange(T) % 2048).astype(np.int32)
    G, U, DO = tiled(T * F), np.resize(block[1:], T * F), np.resize(block[2:], T * F)
    SO, DG, DU = np.empty(T * F, np.uint16), np.empty(T * F, np.uint16), np.empty(T * F, np.uint16)
    LG = tiled(R * V, 2.0)
    lab = np.random.default_rng(9).integers(0, V, size=R).astype(np.uint32)
    loss, mean = np.empty(R, np.float32), np.zeros(1, np.float32)
    act = T * D * 2
    work = [
        ("rms_norm_fwd", 2 * act + D * 2 + 2 * T * 4, lambda: L.cpu_ref_rms_norm_bf16(T, D, 1e-5, P(W), P(X), P(Y), P(ws), P(rs))),
        ("rms_norm_bwd", 4 * act + D * 2 + T * 4 + 2 * D * 4, lambda: L.cpu_ref_rms_norm_bwd_bf16(T, D, P(rs), P(W), P(X), P(dY), P(dX), P(dW))),
        ("rope_fwd", 2 * (Q.nbytes + K.nbytes) + T * 4, lambda: L.cpu_ref_rope_bf16(0, T, 4096, 128, 8, 500000, P(pos), P(Q), P(K))),
        ("rope_bwd", 2 * (Q.nbytes + K.nbytes) + T * 4, lambda: L.cpu_ref_rope_bf16(1, T, 4096, 128, 8, 500000, P(pos), P(Q), P(K))),
        ("swiglu_fwd", 3 * G.nbytes, lambda: L.cpu_ref_swiglu_bf16(G.size, P(G), P(U), P(SO))),
        ("swiglu_bwd", 5 * G.nbytes, lambda: L.cpu_ref_swiglu_bwd_bf16(G.size, P(G), P(U), P(DO), P(DG), P(DU))),
        ("softmax_xent_fused", 2 * LG.nbytes + R * 8 + 4, lambda: L.cpu_ref_softmax_xent_bf16(R, V, P(LG), P(lab), P(loss), P(mean))),
    ]
    per, tot_b, tot_t = {}, 0, 0.0
    per_op_budget = budget_s / len(work)
    for name, nb, fn in work:
        t0 = time.perf_counter()
        fn()                                            # warm-up
        first = time.perf_counter() - t0
        runs = max(1, min(5, int(per_op_budget / max(first, 1e-6))))
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        med = sorted(times)[len(times) // 2]
        per[name] = {"ms": round(med * 1e3, 2), "gbps": round(nb / med / 1e9, 2), "runs": runs}
        tot_b += nb
        tot_t += med
    out = {"value": round(tot_b / tot_t / 1e9, 3), "unit": "GB/s", "cores": int(L.cpu_ref_threads()), "kind": "port",
           "nproc": os.cpu_count(),
           "sample": "oracle/libcpu_ref.so (C: bf16 storage, fp32 math, fp64 reductions, OpenMP over rows, "
                     "gcc -O3 -march=x86-64-v4 -ffast-math) on the full configs 2-5 (rms_norm fwd+fused bwd 8192x4096, "
                     "rope fwd+bwd 8192x(32+8)x128, swiglu fwd+bwd 8192x14336, fused softmax+xent 4096x128256); "
                     "per op 1 warm-up + median of up to 5 runs; same byte formulas; value = total bytes / total time",
           "ops": per}
    out.update(cpu_info())
    return out


def host_submit_cost(api):
    """microseconds per submit_* call from C (lib/bench_submit_cost): batches
    of submits at the step's shapes, the queue drained between batches"""
    import subprocess
    exe = os.path.join(api.LIB_DIR, "bench_submit_cost")
    if not os.path.exists(exe):
        return None
    r = subprocess.run([exe, api.KERNELS, api.CONFIG_LIB], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        print("bench: submit-cost program failed (%d): %s" % (r.returncode, r.stderr[-500:]), file=sys.stderr)
        return None
    return json.loads(r.stdout.strip().splitlines()[-1])


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(name)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-head", action="store_true", help="skip the transformer-head (GEMM) line")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-types", action="store_true", help="skip the fp16 and fp32 storage steps (storage_types)")
    ap.add_argument("--no-copy-reference", action="store_true",
                    help="skip timing the streaming copy of each op's byte count (copy_reference)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 4 device-to-device copies of 1 GiB (the HIP runtime's copy kernel), the known-size "
                         "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: every GPU box here has a single MI355X and this build has no "
              "multi-GPU path (the ops shard by tokens with no exchange; only the dW and mean-loss sums would cross GPUs). "
              "Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    from dataflow_lib_amd import api
    # host cost of the op API, timed from C in a child process started before
    # this process makes its first HIP call
    submit_us = host_submit_cost(api)
    hip = Hip()
    h = api.Handle(0, num_streams=1, matmul=not args.no_head)
    pool = Pool(h)
    try:
        print("bench: allocating and filling rotating buffer sets", file=sys.stderr, flush=True)
        ops = build_ops(h, pool, api)
        extras = [] if args.no_extras else build_extras(h, pool, api)
        types = {} if args.no_types else {name: build_ops(h, pool, api, dt) for name, dt in (("fp16", FP16), ("fp32", FP32))}
        h.sync()
        print("bench: timing %d steps after %d warmup" % (args.steps, args.warmup), file=sys.stderr, flush=True)
        per_op, step_ms, wall = time_ops(h, hip, ops, args.steps, args.warmup)
        # extras and the other storage types with the same launch count per
        # batch as their copy_reference: the two events around a batch add a
        # few microseconds to it, which a shorter batch would charge to each
        # launch more heavily than the copy's
        per_extra = time_ops(h, hip, extras, args.steps, 1)[0] if extras else {}
        per_type = {}
        for name, tops in types.items():
            t_op, t_ms, _ = time_ops(h, hip, tops, args.steps, 1)
            t_bytes = sum(v["bytes"] for v in t_op.values())
            per_type[name] = {"ms_per_step": round(t_ms, 4), "gbps": round(t_bytes / (t_ms * 1e-3) / 1e9, 1),
                              "pct_of_peak": round(100.0 * t_bytes / (t_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 1), "ops": t_op}
        copy_ref = None
        if not args.no_copy_reference:
            sized = dict(per_op)
            sized.update({k: v for k, v in per_extra.items() if v["bytes"] >= (1 << 20)})
            copy_ref = copy_reference(h, hip, pool, api, sized, args.steps)
        head = None if args.no_head else time_head(h, hip, pool, api, 5)
        if args.copy_calibration:
            src, dst = pool.empty(GiB), pool.empty(GiB)
            for _ in range(4):
                assert h.copy(dst, src, GiB, 0) == 0
            h.sync()
        info = h.device_info
        dev = {"arch": info.arch_name.decode(), "cu_count": info.cu_count, "num_xcds": info.num_xcds}
    finally:
        pool.release()
        h.destroy()

    total_bytes = sum(v["bytes"] for v in per_op.values())
    value = total_bytes / (step_ms * 1e-3) / 1e9
    dom = max(per_op, key=lambda k: per_op[k]["avg_us"])
    d = per_op[dom]
    roofline = {"bound": "hbm", "kernel": dom, "achieved": d["gbps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(d["gbps"] / HBM_PEAK_GBPS, 4), "traffic": load_traffic(dom)}
    cpu = None
    if not args.no_cpu:
        print("bench: CPU baseline (oracle/libcpu_ref.so, full configs) ~%.0f s" % args.cpu_budget, file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_budget)
    line = {
        "metric": "Achieved HBM GB/s and % of 8 TB/s peak per op at Llama-3-8B token shapes",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded normal blocks tiled in HBM; labels uniform)",
        "config": {"workload": "llama3-8b native-op step: rms_norm fwd+bwd 8192x4096, rope fwd+bwd 8192x(32+8)x128, "
                               "swiglu fwd+bwd 8192x14336, fused softmax+xent 4096x128256",
                   "tokens": 8192, "hidden": 4096, "ffn": 14336, "vocab": 128256, "ce_rows": 4096},
        "pct_of_peak": round(100.0 * value / HBM_PEAK_GBPS, 1),
        "ops": per_op, "extras": per_extra, "storage_types": per_type, "copy_reference": copy_ref, "transformer_head": head,
        "host_submit_us": submit_us, "roofline": roofline,
        "cpu_baseline": cpu,
        "device": dev,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
