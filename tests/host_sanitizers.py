"""Host code under AddressSanitizer + UBSan: builds libdataflow.so's C sources
(registry, op table, fingerprints, op API, host data plane, HIP backend) and
the oracle's C with gcc -fsanitize=address,undefined into a scratch copy of
the repository and
runs the CPU test suite against it with the sanitizer runtimes preloaded.
Run by hand: python3 tests/host_sanitizers.py (no GPU needed; ~1 minute)."""
import os
import shutil
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def main():
    work = tempfile.mkdtemp(prefix="dataflow_sanitize_")
    try:
        shutil.copytree(ROOT, os.path.join(work, "repo"), ignore=shutil.ignore_patterns(".git", "_work", "gpurun_out", "__pycache__"))
        repo = os.path.join(work, "repo")
        sys.path.insert(0, repo)
        from dataflow_lib_amd import build as B
        flags = [f for f in B.C_FLAGS if f != "-O2"]
        cmd = (["gcc", "-shared", "-g", "-O1", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                "-fno-sanitize-recover=undefined"] + flags + B._sources("core", "ops", "backend/hip") +
               ["-o", B.CORE_OUT, "-lcrypto", "-ldl", "-lpthread"] + B.HIP_LINK)
        subprocess.run(cmd, check=True, cwd=repo)
        oracle_dir = os.path.join(repo, "oracle")
        subprocess.run(["gcc", "-shared", "-g", "-O1", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                        "-fno-sanitize-recover=undefined", "-fopenmp", "-fPIC", "-std=gnu11", "-D__HIP_PLATFORM_AMD__",
                        "-I", os.path.join(repo, "include"), "-I", oracle_dir, "-I", "/opt/rocm/include",
                        os.path.join(oracle_dir, "oracle.c"), os.path.join(oracle_dir, "cpu_backend.c"),
                        "-o", os.path.join(oracle_dir, "liboracle.so"), "-L", B.LIB, "-ldataflow", "-Wl,-rpath," + B.LIB, "-lm"],
                       check=True, cwd=repo)
        rt = [subprocess.run(["gcc", "-print-file-name=" + n], capture_output=True, text=True).stdout.strip()
              for n in ("libasan.so", "libubsan.so")]
        env = dict(os.environ, LD_PRELOAD=" ".join(rt), ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
        return subprocess.run([sys.executable, "-m", "pytest", "tests", "-x", "-q", "-m", "not gpu", "-p", "no:cacheprovider"],
                              cwd=repo, env=env).returncode
    finally:
        shutil.rmtree(work, ignore_errors=True)


if __name__ == "__main__":
    sys.exit(main())
