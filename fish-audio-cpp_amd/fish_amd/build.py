"""Builds the HIP library (gfx950) and the CPU oracle, in-tree.

`build_library()` compiles every source under ``fish-audio-cpp_amd/csrc`` with
hipcc into ``fish-audio-cpp_amd/lib/libfish_w8a8.so``.  `build_oracle()` runs
``make`` in ``oracle/`` (the test checker, built next to the product but never
linked into it).
"""
import os
import subprocess
import sys

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))  # fish-audio-cpp_amd/
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
LIB_DIR = os.path.join(PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libfish_w8a8.so")
ORACLE_DIR = os.path.join(REPO_ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "_build", "liboracle_w8a8.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every FMA in the kernels is written as __builtin_fmaf, so
# the rounding sequence is the one the code states.  Packed fp32 ops are off
# (they have produced silent wrong results on these boxes).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

HIP_SOURCES = ["quant.hip", "gemv.hip", "gemv_dot.hip", "gemv_dot_pro.hip", "gemv_dot_swiglu.hip", "gemv_mfma_fused.hip",
               "gemv_f16.hip", "gemm.hip", "chain.hip", "attn.hip"]
HOST_SOURCES = ["api.cpp", "loader.cpp", "kernels_cxx.cpp"]


def _run(cmd, cwd=None):
    res = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    return out


def build_library(verbose=False):
    """Compile each source to an object in parallel, then link the .so."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(LIB_DIR, exist_ok=True)
    obj_dir = os.path.join(PKG_ROOT, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    inc = ["-I", os.path.join(PKG_ROOT, "include")]
    flags = [f for f in HIP_FLAGS if f != "-shared"]
    jobs = []
    for src in HIP_SOURCES + HOST_SOURCES:   # the shared kernel header is not a unit
        obj = os.path.join(obj_dir, src + ".o")
        lang = [] if src.endswith(".hip") else ["-x", "hip"]
        jobs.append((obj, [HIPCC] + flags + inc + ["-c"] + lang + [os.path.join(CSRC, src), "-o", obj]))
    with ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        outs = list(ex.map(lambda j: _run(j[1]), jobs))
    tmp = LIB_PATH + ".tmp"
    outs.append(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + [o for o, _ in jobs]
                     + ["-o", tmp]))
    os.replace(tmp, LIB_PATH)
    out = "\n".join(o for o in outs if o.strip())
    if verbose and out.strip():
        print(out)
    return LIB_PATH


TEST_DRIVER_SRC = os.path.join(REPO_ROOT, "tests", "cxx", "engine_prefill.cpp")
TEST_DRIVER = os.path.join(LIB_DIR, "engine_prefill")


def build_test_driver(verbose=False):
    """The C++ test driver (tests/cxx/engine_prefill.cpp): the engine's
    prefill attention block through the C++ mirror, linked to the library."""
    out = _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-x", "hip",
                "-I", os.path.join(PKG_ROOT, "include"), TEST_DRIVER_SRC,
                "-L", LIB_DIR, "-lfish_w8a8", "-Wl,-rpath,$ORIGIN", "-o", TEST_DRIVER + ".tmp"])
    os.replace(TEST_DRIVER + ".tmp", TEST_DRIVER)
    if verbose and out.strip():
        print(out)
    return TEST_DRIVER


def build_oracle(verbose=False):
    out = _run(["make", "-s", "-C", ORACLE_DIR])
    if verbose and out.strip():
        print(out)
    return ORACLE_LIB


if __name__ == "__main__":
    print(build_library(verbose=True))
    print(build_test_driver(verbose=True))
    print(build_oracle(verbose=True))
    sys.exit(0)
