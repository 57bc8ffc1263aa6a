"""Build libgpic_fp8.so (the HIP kernels and their C ABI) for gfx950 with hipcc, in-tree.

    python nano-gpic_amd/gpic_fp8/build.py        (or gpic_fp8.build.build() from Python)
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "csrc")
INCLUDE = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include")
LIB = os.path.join(HERE, "libgpic_fp8.so")
SOURCES = ["api.hip", "cast.hip", "gemm.hip", "norm.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",                                        # every float op rounds as written
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",  # no v_pk_*_f32 (unreliable on this pool)
    "-Wall", "-Wno-unused-function",
]


def build(verbose=False):
    """Each source compiled to an object in its own hipcc process (in parallel), then linked into the library."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    procs = []
    for name in SOURCES:
        obj = os.path.join(objdir, name.replace(".hip", ".o"))
        cmd = [HIPCC, *compile_flags, "-c", "-I", INCLUDE, "-o", obj, os.path.join(CSRC, name)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((name, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    objs = []
    for name, obj, pr in procs:
        _, err = pr.communicate()
        if pr.returncode != 0:
            raise RuntimeError(f"hipcc failed on {name} ({pr.returncode}):\n{err[-6000:]}")
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc link failed ({r.returncode}):\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    return LIB


TEST_LIBS = {"bf16_selfcheck.hip": "libbf16_selfcheck.so", "mfma_ceiling.hip": "libmfma_ceiling.so",
             "hbm_floor.hip": "libhbm_floor.so"}


def build_test_libs(verbose=False):
    """The test-side libraries under tests/hip (the bf16 rounding self-check, the MFMA ceiling and HBM floor
    measurements), with the same compiler flags as the product."""
    root = os.path.dirname(os.path.dirname(HERE))
    outs = []
    for src_name, lib_name in TEST_LIBS.items():
        src = os.path.join(root, "tests", "hip", src_name)
        out = os.path.join(root, "tests", "hip", lib_name)
        cmd = [HIPCC, *FLAGS, "-o", out + ".tmp", src]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stderr[-6000:]}")
        os.replace(out + ".tmp", out)
        outs.append(out)
    return outs


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_test_libs(verbose="-v" in sys.argv))
