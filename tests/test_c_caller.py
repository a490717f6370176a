"""A C program compiled against include/*.h drives the boundary the way the
reference's C callers do (tests/c_caller.c): stack-allocated handle,
register_native_ops, config 1 through submit_rms_norm and through a raw Op
on the handle's submit_op. tests/c_caller.c runs on the CPU test backend (no
GPU); the struct layouts it prints must equal the ctypes mirrors in
dataflow_lib_amd/api.py. tests/c_caller_gpu.c does the same on the HIP
backend (marked gpu)."""
import ctypes
import os
import subprocess

import pytest

from support import ORACLE_LIB, ROOT

from dataflow_lib_amd import api

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build_and_run(tmp_path):
    exe = str(tmp_path / "c_caller")
    lib, odir = api.LIB_DIR, os.path.dirname(ORACLE_LIB)
    cmd = ["gcc", "-std=gnu11", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", odir, "-I", os.path.join(ROCM, "include"), os.path.join(ROOT, "tests", "c_caller.c"), "-o", exe,
           "-L", lib, "-ldataflow", "-L", odir, "-loracle", "-Wl,-rpath," + lib, "-Wl,-rpath," + odir, "-lm"]
    b = subprocess.run(cmd, capture_output=True, text=True)
    assert b.returncode == 0, b.stderr
    return subprocess.run([exe, ORACLE_LIB], capture_output=True, text=True, timeout=60)


def test_c_caller_config1_and_layouts(tmp_path):
    r = build_and_run(tmp_path)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "OK registered 68" in r.stdout
    layout = {}
    for line in r.stdout.splitlines():
        if line.startswith("LAYOUT "):
            _, name, value = line.split()
            layout[name] = int(value)
    H, O, HI = api.DataflowHandle, api.Op, api.HipDeviceInfo
    want = {
        "sizeof_Dataflow_Handle": ctypes.sizeof(H),
        "offset_Dataflow_Handle_stream_prios": H.stream_prios.offset,
        "offset_Dataflow_Handle_native_function_libs": H.native_function_libs.offset,
        "offset_Dataflow_Handle_op_table": H.op_table.offset,
        "offset_Dataflow_Handle_submit_op": H.submit_op.offset,
        "offset_Dataflow_Handle_submit_peer_transfer": H.submit_peer_transfer.offset,
        "sizeof_Op": ctypes.sizeof(O),
        "sizeof_Op_Skeleton_Header": ctypes.sizeof(api.OpSkeletonHeader),
        "offset_Op_op_args": O.op_args.offset,
        "sizeof_Table": ctypes.sizeof(api.Table),
        "sizeof_Hip_Device_Info": ctypes.sizeof(HI),
        "offset_Hip_Device_Info_cu_count": HI.cu_count.offset,
        "offset_Hip_Device_Info_arch_name": HI.arch_name.offset,
    }
    assert layout == want
    # the op skeleton header is the 388-byte SHA-256 input
    assert layout["sizeof_Op_Skeleton_Header"] == 388


@pytest.mark.gpu
def test_c_caller_on_the_hip_backend(tmp_path):
    """tests/c_caller_gpu.c: a gcc-built C program that initialises the HIP
    backend on a stack-allocated Dataflow_Handle, registers the gfx950 code
    object and the launch-configuration library, and runs BASELINE configs 1
    and 2 through submit_rms_norm and through a raw Op on the handle's
    submit_op (bit-equal), plus the config-2 backward through
    submit_rms_norm_bwd, each checked against the oracle inside the program.
    The reduction-depth bounds of the fp32 sums come from tests/support.py,
    for this device's CU count and LDS size."""
    from support import BF16, FP32, gamma, rms_dw_depth, rms_ws_depth
    h = api.Handle(0, num_streams=1)
    cu, lds = h.device_info.cu_count, h.device_info.max_smem_per_block
    h.destroy()
    exe = str(tmp_path / "c_caller_gpu")
    lib, odir = api.LIB_DIR, os.path.dirname(ORACLE_LIB)
    cmd = ["gcc", "-std=gnu11", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
           "-I", odir, "-I", os.path.join(ROCM, "include"), os.path.join(ROOT, "tests", "c_caller_gpu.c"), "-o", exe,
           "-L", lib, "-ldataflow", "-L", odir, "-loracle", "-Wl,-rpath," + lib, "-Wl,-rpath," + odir, "-lm"]
    b = subprocess.run(cmd, capture_output=True, text=True)
    assert b.returncode == 0, b.stderr
    args = [exe, api.KERNELS, api.CONFIG_LIB, repr(gamma(rms_ws_depth(FP32, 4096))), repr(gamma(rms_ws_depth(BF16, 4096))),
            repr(gamma(rms_dw_depth(BF16, 8192, 4096, 3, cu, lds)))]
    r = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "OK registered 68" in r.stdout
    assert "OK forward dtype 3 16 x 4096" in r.stdout
    assert "OK forward dtype 5 8192 x 4096" in r.stdout
    assert "OK backward bf16 8192 x 4096" in r.stdout
    assert "OK done" in r.stdout
