"""The C ABI libraries load and export every function include/*.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

from support import ROOT

from dataflow_lib_amd import api

INCLUDE = os.path.join(ROOT, "include")


def declared_functions(path):
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    src = re.sub(r"^\s*#[^\n]*(\\\n[^\n]*)*", "", src, flags=re.M)
    # drop struct / enum / extern "C" bodies' braces content of aggregates
    while True:
        new = re.sub(r"\b(struct|enum|union)\s*\w*\s*\{[^{}]*\}", r"\1", src)
        if new == src:
            break
        src = new
    src = src.replace('extern "C" {', "").replace("}", "")
    names = []
    for stmt in src.split(";"):
        stmt = " ".join(stmt.split())
        if not stmt or stmt.startswith("typedef") or "(*" in stmt:
            continue
        m = re.match(r"^[\w\s\*]+?\b(\w+)\s*\(", stmt)
        if m and m.group(1) not in ("if", "while", "for", "return"):
            names.append(m.group(1))
    return names


def test_every_declared_symbol_is_exported():
    core = api.lib()
    cfg = ctypes.CDLL(api.CONFIG_LIB)
    noalloc = api.noalloc_lib()
    headers = sorted(f for f in os.listdir(INCLUDE) if f.endswith(".h"))
    seen = 0
    for h in headers:
        names = declared_functions(os.path.join(INCLUDE, h))
        lib = {"hip_ops_config.h": cfg, "dataflow_noalloc.h": noalloc}.get(h, core)
        missing = [n for n in names if not hasattr(lib, n)]
        assert not missing, "%s declares functions missing from %s: %s" % (h, lib._name, missing)
        seen += len(names)
    assert seen >= 55


def test_parser_sees_the_op_api():
    names = declared_functions(os.path.join(INCLUDE, "dataflow_ops.h"))
    assert {"submit_rms_norm", "submit_rope_bwd_x", "submit_softmax_cross_entropy_loss", "submit_embedding",
            "submit_copy_to_seq_context", "submit_matmul", "submit_rope_copy_to_seq_context"} <= set(names)
    assert len(names) == 15


def test_kernel_code_object_present():
    data = open(api.KERNELS, "rb").read()
    assert data[:4] == b"\x7fELF" or data.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    for sym in (b"rms_norm_bf16_kernel", b"rms_norm_bwd_bf16_bf16_kernel_finish", b"rope_bwd_x_bf16_kernel",
                b"swiglu_bwd_x_bf16_bf16_kernel", b"softmax_cross_entropy_loss_bf16_kernel", b"embedding_fp8e5m2_kernel",
                b"copy_to_seq_context_bf16_kernel", b"rope_copy_to_seq_context_bf16_kernel"):
        assert sym in data
    # the 22 functions with fp8 tensors: every kernel name the registry derives for them
    for f in ("fp8e4m3", "fp8e5m2"):
        for name in ("rms_norm_%s_kernel", "rope_%s_kernel", "swiglu_%s_kernel"):
            assert (name % f).encode() in data
        for b in ("fp16", "bf16"):
            for op in ("rms_norm_bwd_x", "rms_norm_bwd_w", "swiglu_bwd_x", "softmax"):
                assert ("%s_%s_%s_kernel" % (op, f, b)).encode() in data
            assert ("rms_norm_bwd_w_%s_%s_kernel_finish" % (f, b)).encode() in data
    # the measurement-only streaming copies live in bench.py's own code object
    assert b"dataflow_stream_copy" not in data
    bench = open(api.BENCH_COPY_KERNELS, "rb").read()
    assert b"dataflow_stream_copy_blk8_kernel" in bench
