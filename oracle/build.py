"""Build recipe for the test oracle (TEST INFRASTRUCTURE ONLY).

  oracle/liboracle.so    the C restatement (oracle.c) plus the CPU test backend
                         (cpu_backend.c), linked against the product's libdataflow.so
  oracle/libcpu_ref.so   the CPU baseline bench.py times (cpu_ref.c: fp32 math, fp64
                         reductions, OpenMP, AVX-512); built for x86-64-v4 rather
                         than -march=native, since it is compiled in this container
                         and runs on the GPU box's host (another x86 vendor)
  oracle/_ref/libref_host.so
                         the reference's own host C for the op registry, compiled
                         from its sources where they lie under /root/reference
                         (datatype strings, SHA-256 fingerprints, op skeletons, op
                         table) and its harnesses' random-matrix generator. Built
                         only when /root/reference is present; its kernels are
                         CUDA for sm_90a and cannot be built here.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
REF = os.environ.get("DATAFLOW_REFERENCE_ROOT", "/root/reference")
ORACLE_OUT = os.path.join(HERE, "liboracle.so")
CPU_REF_OUT = os.path.join(HERE, "libcpu_ref.so")
REF_OUT = os.path.join(HERE, "_ref", "libref_host.so")
PRODUCT_LIB = os.path.join(ROOT, "dataflow_lib_amd", "lib")

# reference host files for the registry path, compiled where they lie
REF_SOURCES = [
    "src/datatype/src/dataflow_datatype.c",
    "src/fingerprint/src/fingerprint.c",
    "src/set_ops/src/set_native_op_skeletons.c",
    "src/set_ops/src/set_external_op_skeletons.c",
    "src/table/src/table.c",
    "src/dataflow_handle/nvidia/test/create_host_matrix.c",
]
# exported registry-path entry points; everything else is local and
# --gc-sections drops what they do not reach (dataflow_convert_datatype's AVX-512
# conversion sources need -mavx512fp16, which this gcc lacks, so they are not built)
REF_EXPORTS = [
    "dataflow_sizeof_element", "dataflow_datatype_as_string",
    "do_fingerprinting", "fingerprint_to_least_sig64", "get_fingerprint_num_bytes",
    "set_native_op_skeleton", "set_native_embedding_skeleton", "set_native_rms_norm_skeleton",
    "set_native_rms_norm_bwd_x_skeleton", "set_native_rms_norm_bwd_w_skeleton", "set_native_rope_skeleton",
    "set_native_rope_bwd_x_skeleton", "set_native_copy_to_seq_context_skeleton", "set_native_swiglu_skeleton",
    "set_native_swiglu_bwd_x_skeleton", "set_native_softmax_skeleton", "set_native_cross_entropy_loss_skeleton",
    "register_native_ops", "set_external_matmul_skeleton", "init_table", "insert_table", "find_table", "remove_table", "destroy_table",
    "rand_normal",
]
REF_INCLUDES = [
    "include", "src/datatype/include", "src/fingerprint/include", "src/ops/include",
    "src/set_ops/include", "src/dataflow_handle/include", "src/table/include", "src/dataflow_handle/nvidia/test",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("build step failed: %s\n%s%s" % (" ".join(cmd), res.stdout, res.stderr))


def build_oracle(verbose=False):
    tmp = ORACLE_OUT + ".tmp%d" % os.getpid()
    _run(["gcc", "-O2", "-fopenmp", "-fPIC", "-shared", "-std=gnu11", "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(ROOT, "include"), "-I", HERE, "-I", "/opt/rocm/include",
          os.path.join(HERE, "oracle.c"), os.path.join(HERE, "cpu_backend.c"),
          "-o", tmp, "-L", PRODUCT_LIB, "-ldataflow", "-Wl,-rpath," + PRODUCT_LIB, "-lm"], verbose)
    os.replace(tmp, ORACLE_OUT)
    return ORACLE_OUT


def build_cpu_ref(verbose=False):
    """The CPU baseline; -ffast-math lets expf vectorise (glibc's vector math
    library), the counterpart of the GPU kernels' hardware exp2. It is given
    to the compile step only: linked with -ffast-math, gcc adds a start-up
    object that turns on flush-to-zero for the whole process loading the
    library."""
    tmp = CPU_REF_OUT + ".tmp%d" % os.getpid()
    obj = tmp + ".o"
    try:
        _run(["gcc", "-c", "-O3", "-march=x86-64-v4", "-ffast-math", "-fopenmp", "-fPIC", "-std=gnu11",
              os.path.join(HERE, "cpu_ref.c"), "-o", obj], verbose)
        _run(["gcc", "-shared", "-fopenmp", obj, "-o", tmp, "-lm"], verbose)
    finally:
        if os.path.exists(obj):
            os.remove(obj)
    os.replace(tmp, CPU_REF_OUT)
    return CPU_REF_OUT


def build_reference_host(verbose=False):
    """Returns the path of the built library, or None when the reference is absent."""
    if not all(os.path.exists(os.path.join(REF, s)) for s in REF_SOURCES):
        return None
    os.makedirs(os.path.dirname(REF_OUT), exist_ok=True)
    tmp = REF_OUT + ".tmp%d" % os.getpid()
    vscript = os.path.join(os.path.dirname(REF_OUT), "exports.map")
    with open(vscript, "w") as f:
        f.write("{ global: %s; local: *; };\n" % "; ".join(REF_EXPORTS))
    cmd = ["gcc", "-O1", "-fPIC", "-shared", "-w", "-std=gnu11", "-ffunction-sections", "-fdata-sections"]
    for inc in REF_INCLUDES:
        cmd += ["-I", os.path.join(REF, inc)]
    cmd += [os.path.join(REF, s) for s in REF_SOURCES]
    cmd += ["-o", tmp, "-Wl,--gc-sections", "-Wl,--version-script=" + vscript, "-lcrypto", "-lm"]
    _run(cmd, verbose)
    os.replace(tmp, REF_OUT)
    return REF_OUT


if __name__ == "__main__":
    v = "-v" in sys.argv
    print(build_oracle(v))
    print(build_cpu_ref(v))
    print(build_reference_host(v))
