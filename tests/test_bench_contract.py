"""bench.py's contract pieces that need no GPU: the single-GPU guard, the CPU
baseline object and the committed traffic figures the roofline line reads."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

STEP_OPS = ["rms_norm_fwd", "rms_norm_bwd", "rope_fwd", "rope_bwd", "swiglu_fwd", "swiglu_bwd", "softmax_xent_fused"]


def run_bench(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, capture_output=True, text=True,
                          timeout=120, env=env, cwd=ROOT)


@pytest.mark.parametrize("args,env", [(["--gpus", "2"], None), (["--gpus", "8"], None), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_exits_with_a_message(args, env):
    r = run_bench(args, env)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_cpu_baseline_object():
    import bench
    cpu = bench.cpu_baseline(0.2)
    assert cpu["kind"] == "port" and cpu["unit"] == "GB/s"
    assert cpu["value"] > 0 and cpu["cores"] >= 1
    assert "oracle" in cpu["sample"]
    assert cpu["nproc"] >= 1 and isinstance(cpu["cpu_model"], str) and isinstance(cpu["isa"], list)
    assert sorted(cpu["ops"]) == sorted(STEP_OPS)
    assert all(v["gbps"] > 0 and v["ms"] > 0 and v["runs"] >= 1 for v in cpu["ops"].values())
    assert "full configs" in cpu["sample"] and cpu["cpu_family_model_stepping"]


def test_traffic_figures_cover_the_step():
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        t = json.load(f)
    import bench
    for op in STEP_OPS:
        assert bench.load_traffic(op) == t[op]
        assert t[op] > 0
    # the scales come from a copy of known size: FETCH_SIZE counts half the bytes, WRITE_SIZE all of them
    assert abs(t["fetch_scale"] - 2.0) < 0.01 and abs(t["write_scale"] - 1.0) < 0.01


def test_cpu_baseline_library_keeps_the_process_float_mode():
    """loading the CPU baseline (compiled with -ffast-math) must not switch the
    process to flush-to-zero: the oracle tests in the same process rely on
    subnormals"""
    import ctypes
    import numpy as np
    ctypes.CDLL(os.path.join(ROOT, "oracle", "libcpu_ref.so"))
    tiny = np.float32(2.0 ** -140)                      # an fp32 subnormal, exactly representable
    assert tiny != 0 and tiny * np.float32(2) == np.float32(2.0 ** -139)
