"""Build libmhsa_hip.so (the C-ABI library) for gfx950 with hipcc, in-tree.

Usage: python mlx-nemo-rs_amd/build.py [--jobs N]

Every call recompiles all sources (the build is the "does it build" check);
objects go to mlx-nemo-rs_amd/_build/, the library to
mlx-nemo-rs_amd/libmhsa_hip.so.
"""
import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmhsa_hip.so")
SOURCES = ["gemm.hip", "attention.hip", "misc.hip", "mhsa_api.hip", "block_api.hip", "conv.hip", "checkpoint.cpp"]
ARCH = "gfx950"


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


# Packed fp32 VALU ops are disabled for all device code (gfx950 forms of
# v_pk_*_f32 are not trusted on this hardware); hipcc's host pass ignores it.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-Wall", "-Wno-unused-result"]


# The attention kernels feed every MFMA result to vector ALU work (softmax,
# rel_shift remap), so their accumulators are kept in VGPRs: with the AGPR
# form the compiler copies them through v_accvgpr_read/write on every tile.
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc()] + FLAGS + FILE_FLAGS.get(src, []) + ["-I", os.path.join(os.path.dirname(HERE), "include"), "-c",
                                                         os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l and "(ignoring feature)" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def build(jobs: int = 4, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        results = list(ex.map(_compile, SOURCES))
    for obj, warn in results:
        if verbose and warn.strip():
            print(warn)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
    sys.exit(0)
