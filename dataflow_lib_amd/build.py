"""Build recipe for the product library (no cmake/ninja: direct compiler calls).

Outputs (in-tree, under dataflow_lib_amd/lib/):
  libdataflow.so                 C ABI: datatype, fingerprint, table, op skeletons,
                                 submit_* op API and the HIP backend of Dataflow_Handle
  libdataflow_hip_config.so      launch configurations (dlopen'ed by the backend)
  dataflow_kernels_gfx950.hsaco  gfx950 code object (hipModuleLoad'ed by the backend)
  libdataflow_hipblaslt.so       the external matmul op on hipBLASLt (register_external_matmul)
  libdataflow_noalloc.so         the allocation-free entry point (include/dataflow_noalloc.h):
                                 host code and its gfx950 kernels in one HIP fat binary
  bench_submit_cost              C program bench.py runs to time the host side of the op API
  bench_stream_copy_gfx950.hsaco streaming copies bench.py times as the memory system's
                                 ceiling (not part of the product; loaded by bench.py only)
"""
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
CC = os.environ.get("CC", "gcc")

ARCH = "gfx950"
KERNELS_OUT = os.path.join(LIB, "dataflow_kernels_gfx950.hsaco")
CORE_OUT = os.path.join(LIB, "libdataflow.so")
CONFIG_OUT = os.path.join(LIB, "libdataflow_hip_config.so")
MATMUL_OUT = os.path.join(LIB, "libdataflow_hipblaslt.so")
BENCH_COPY_OUT = os.path.join(LIB, "bench_stream_copy_gfx950.hsaco")
NOALLOC_OUT = os.path.join(LIB, "libdataflow_noalloc.so")
SUBMIT_COST_OUT = os.path.join(LIB, "bench_submit_cost")
CXX = os.environ.get("CXX", "g++")

C_FLAGS = ["-O2", "-fPIC", "-std=gnu11", "-Wall", "-Wextra", "-Werror=format", "-Wno-unused-parameter", "-Wno-stringop-truncation",
           "-D__HIP_PLATFORM_AMD__", "-I", INCLUDE, "-I", os.path.join(CSRC, "kernels"),
           "-I", os.path.join(ROCM, "include")]
HIP_LINK = ["-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib")]
# packed fp32 VALU forms are kept out of every code object
HIP_FLAGS = ["--offload-arch=" + ARCH, "-O3", "--genco", "-std=c++17",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", os.path.join(CSRC, "kernels")]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "--hip-link", "warning: argument unused")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError("build step failed (%d): %s\n%s\n%s" % (res.returncode, " ".join(cmd), res.stdout, err))
    # warnings are printed on every build, not only verbose ones
    if err.strip():
        print(err, file=sys.stderr)


def _atomic(out, build_fn):
    tmp = out + ".tmp%d" % os.getpid()
    try:
        build_fn(tmp)
        os.replace(tmp, out)
    finally:
        if os.path.exists(tmp):
            os.remove(tmp)


def _sources(*subdirs):
    out = []
    for d in subdirs:
        full = os.path.join(CSRC, d)
        out += sorted(os.path.join(full, f) for f in os.listdir(full) if f.endswith(".c"))
    return out


def build(verbose=False):
    if not os.path.exists(HIPCC):
        raise RuntimeError("hipcc not found at %s" % HIPCC)
    os.makedirs(LIB, exist_ok=True)
    _atomic(KERNELS_OUT, lambda o: _run([HIPCC] + HIP_FLAGS + [os.path.join(CSRC, "kernels", "dataflow_kernels.hip"), "-o", o], verbose))
    _atomic(CORE_OUT, lambda o: _run([CC, "-shared"] + C_FLAGS + _sources("core", "ops", "backend/hip") +
                                      ["-o", o, "-lcrypto", "-ldl", "-lpthread"] + HIP_LINK, verbose))
    _atomic(CONFIG_OUT, lambda o: _run([CC, "-shared"] + C_FLAGS + _sources("config") +
                                        ["-o", o, "-L", LIB, "-ldataflow", "-Wl,-rpath,$ORIGIN"] + HIP_LINK, verbose))
    _atomic(MATMUL_OUT, lambda o: _run([CXX, "-shared", "-O2", "-fPIC", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__",
                                        "-I", INCLUDE, "-I", os.path.join(ROCM, "include"),
                                        os.path.join(CSRC, "external", "hipblaslt_matmul.cpp"), "-o", o,
                                        "-L", os.path.join(ROCM, "lib"), "-lhipblaslt"] + HIP_LINK, verbose))
    _atomic(NOALLOC_OUT, lambda o: _run([HIPCC, "--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-shared",
                                         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                                         "-I", INCLUDE, "-I", os.path.join(CSRC, "kernels"),
                                         os.path.join(CSRC, "noalloc", "rms_norm_bwd_noalloc.hip"), "-o", o,
                                         "-L", LIB, "-ldataflow", "-Wl,-rpath,$ORIGIN"], verbose))
    _atomic(SUBMIT_COST_OUT, lambda o: _run([CC] + C_FLAGS + [os.path.join(CSRC, "bench", "submit_cost.c"), "-o", o,
                                             "-L", LIB, "-ldataflow", "-Wl,-rpath,$ORIGIN"] + HIP_LINK, verbose))
    _atomic(BENCH_COPY_OUT, lambda o: _run([HIPCC] + HIP_FLAGS + [os.path.join(CSRC, "bench", "stream_copy.hip"), "-o", o], verbose))
    return {"kernels": KERNELS_OUT, "core": CORE_OUT, "config": CONFIG_OUT, "matmul": MATMUL_OUT,
            "noalloc": NOALLOC_OUT, "bench_copy": BENCH_COPY_OUT, "submit_cost": SUBMIT_COST_OUT}


if __name__ == "__main__":
    for k, v in build(verbose="-v" in sys.argv).items():
        print(k, v)
