"""Build libmhsa_hip.so (the C-ABI library) for gfx950 with hipcc, in-tree.

Usage: python mlx-nemo-rs_amd/build.py [--jobs N] [--sanitize-host]

Every call recompiles all sources (the build is the "does it build" check);
objects go to mlx-nemo-rs_amd/_build/, the library to
mlx-nemo-rs_amd/libmhsa_hip.so.

--sanitize-host builds a second library, _build/san/libmhsa_hip_san.so, whose
host code is instrumented with AddressSanitizer and UndefinedBehaviorSanitizer
(device code is built as usual; the sanitizers apply to host code only). It
leaves the sanitizer runtime unresolved: load it into a process started with
LD_PRELOAD=<sanitizer_runtime()>. With --ubsan-only it builds
_build/san/libmhsa_hip_ubsan.so (UBSan alone, runtime
sanitizer_runtime("ubsan_standalone")): the HIP runtime does not start in a
process that preloads the ASan runtime, so GPU runs use this one.
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
SOURCES = ["gemm.hip", "attention.hip", "misc.hip", "mhsa_api.hip", "block_api.hip", "encoder_api.hip", "conv.hip",
           "checkpoint.cpp"]
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


# Host-only instrumentation: each -fsanitize= sits behind -Xarch_host so that
# no device code is built with it.
SAN_BASE = ["-O3", "-Xarch_host", "-g", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature",
            "-Xclang", "-packed-fp32-ops", "-Xarch_host", "-fno-omit-frame-pointer"]


def san_flags(kinds):
    flags = list(SAN_BASE)
    for k in kinds:
        flags += ["-Xarch_host", f"-fsanitize={k}"]
    if "undefined" in kinds:
        flags += ["-Xarch_host", "-fno-sanitize-recover=undefined"]
    return flags


SAN_BUILD = os.path.join(BUILD, "san")
SAN_LIB = os.path.join(SAN_BUILD, "libmhsa_hip_san.so")
UBSAN_LIB = os.path.join(SAN_BUILD, "libmhsa_hip_ubsan.so")


def sanitizer_runtime(name: str = "asan") -> str:
    """A sanitizer runtime of the ROCm clang that builds the sanitized
    library: "asan" (it carries UBSan's handlers too) or "ubsan_standalone"."""
    clang = os.path.join(os.path.dirname(os.path.realpath(hipcc())), "..", "llvm", "bin", "clang")
    if not os.path.exists(clang):
        clang = "/opt/rocm/llvm/bin/clang"
    r = subprocess.run([clang, f"-print-file-name=libclang_rt.{name}-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    if r.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
        raise RuntimeError(f"the {name} runtime of ROCm's clang was not found")
    return path


def _compile(src, flags=None, out_dir=None):
    obj = os.path.join(out_dir or BUILD, os.path.splitext(src)[0] + ".o")
    base = FLAGS if flags is None else flags
    cmd = [hipcc()] + base + FILE_FLAGS.get(src, []) + ["-I", os.path.join(os.path.dirname(HERE), "include"), "-c",
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


def build_sanitized(jobs: int = 4, ubsan_only: bool = False) -> str:
    """The host-sanitized library (see the module docstring); with ubsan_only,
    UBSan alone (for processes that cannot preload the ASan runtime)."""
    kinds = ("undefined",) if ubsan_only else ("address", "undefined")
    lib = UBSAN_LIB if ubsan_only else SAN_LIB
    out_dir = os.path.join(SAN_BUILD, "ubsan" if ubsan_only else "asan")
    os.makedirs(out_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        results = list(ex.map(lambda s: _compile(s, san_flags(kinds), out_dir), SOURCES))
    tmp = lib + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--sanitize-host", action="store_true")
    ap.add_argument("--ubsan-only", action="store_true", help="with --sanitize-host: UBSan without ASan")
    a = ap.parse_args()
    if a.sanitize_host:
        print(build_sanitized(a.jobs, a.ubsan_only))
        sys.exit(0)
    print(build(a.jobs, a.verbose))
    sys.exit(0)
