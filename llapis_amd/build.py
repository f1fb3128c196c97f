"""Build libllapis_moe.so in-tree: hand-written gfx950 HIP kernels + the C ABI.

    python -m llapis_amd.build          # or: python llapis_amd/build.py

The host quantisers are compiled with g++ -ffp-contract=off (their float
rounding must match ggml's own build); everything else with hipcc for gfx950
only.  Objects go to llapis_amd/_build/, the library next to this file.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libllapis_moe.so"
ARCH = "gfx950"

HIP_SOURCES = ["mmv.hip", "decode.hip", "prefill.hip", "small_kernels.hip", "transfer.hip", "model_files.hip",
               "residency.hip", "api.hip"]
HOST_SOURCES = ["quantize.cpp", "policy.cpp", "kfit.cpp"]


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def gelu_table():
    """Generate the fp16 GELU table of the CPU path's GEGLU (gen_gelu_table.c:
    host float arithmetic and glibc tanhf, as the CPU path fills its own)."""
    gen = BUILD / "gen_gelu_table"
    _run(["gcc", "-O2", "-ffp-contract=off", "-mf16c", str(CSRC / "gen_gelu_table.c"), "-o", str(gen), "-lm"])
    out = subprocess.run([str(gen)], stdout=subprocess.PIPE, check=True, text=True).stdout
    inc = BUILD / "gelu_table.inc"
    if not inc.exists() or inc.read_text() != out:
        inc.write_text(out)
    return inc


def build(verbose=False):
    BUILD.mkdir(exist_ok=True)
    hipcc = _hipcc()
    gelu_table()
    hip_flags = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
                 "-Wno-unused-variable",
                 # packed fp32 VALU ops are kept out of every kernel
                 "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                 f"-I{CSRC}", f"-I{BUILD}", f"-I{PKG.parent / 'include'}"]
    jobs = []
    for src in HIP_SOURCES:
        obj = BUILD / (src + ".o")
        jobs.append([hipcc, *hip_flags, "-c", str(CSRC / src), "-o", str(obj)])
    for src in HOST_SOURCES:
        obj = BUILD / (src + ".o")
        jobs.append(["g++", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-pthread", "-Wall",
                     f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for out in ex.map(_run, jobs):
            if verbose and out.strip():
                print(out)
    objs = [str(BUILD / (s + ".o")) for s in HIP_SOURCES + HOST_SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o", str(tmp), *objs, "-pthread"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
