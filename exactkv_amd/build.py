"""Build libexactkv_hip.so (gfx950) in-tree.

Each csrc/*.hip is compiled with hipcc for gfx950 only, then the objects are linked
into one shared library against the HIP runtime that PyTorch-ROCm itself loads
(torch/lib/libamdhip64.so), so that the library and torch share one runtime: the
same device context, allocations and streams (torch's current stream is passed to
every entry point).

    python -m exactkv_amd.build          # or __graft_entry__.build()
"""
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libexactkv_hip.so")
BUILD_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

# Packed-FP32 VALU forms are kept out of generated code (the compiler would otherwise
# form v_pk_* f32 ops from scalar float code).
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


def _torch_lib_dir():
    import torch
    return os.path.join(os.path.dirname(torch.__file__), "lib")


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the exactkv HIP library)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in r.stdout.splitlines() if "packed-fp32-ops" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(verbose=False):
    """Compile every csrc/*.hip for gfx950 and link libexactkv_hip.so. Always rebuilds."""
    hipcc = _hipcc()
    tlib = _torch_lib_dir()
    if not os.path.exists(os.path.join(tlib, "libamdhip64.so")):
        raise RuntimeError(f"PyTorch-ROCm HIP runtime not found in {tlib}")
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = []
    for src in sorted(glob.glob(os.path.join(CSRC, "*.hip"))):
        obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
        _run([hipcc, *HIP_FLAGS, "-c", src, "-o", obj], verbose)
        objs.append(obj)
    tmp = OUT + ".tmp"
    # plain host link (device code is already embedded in each object): only torch's
    # HIP runtime is named, so the loader reuses the copy torch has loaded
    _run([shutil.which("g++") or "g++", "-shared", "-fPIC", "-o", tmp, *objs, f"-L{tlib}", "-l:libamdhip64.so",
          f"-Wl,-rpath,{tlib}", "-Wl,--no-undefined"], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
