"""Build libgehtp.so (the runlist engine + gfx950 kernels) in-tree with hipcc.

    python -m gehtp_amd.build        # or gehtp_amd.build.build()

Objects go to gehtp_amd/_build/, the library to gehtp_amd/libgehtp.so, and the
resident decode server (host code over the library's C ABI) to
gehtp_amd/gehtp_persistent. Every source is compiled on every call (the build is a
correctness check as much as a build); the compile units run in parallel.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = PKG / "libgehtp.so"
SERVER = PKG / "gehtp_persistent"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# packed-fp32 instructions are disabled for all device code.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # No FP contraction: ops the reference rounds through f16 must not be fused
    # (clang otherwise narrows f32 mul/add of f16 values to f16 and fuses them).
    "-ffp-contract=off",
    "-Wall", "-Wno-unused-result", "-Wno-unused-variable",
]
SOURCES = ["wt_parse.cpp", "engine.cpp", "capi.cpp",
           "k_w4g.hip", "k_rows.hip", "k_f16mm.hip", "k_attn.hip", "k_data.hip"]


def _compile(src: Path, verbose: bool) -> Path:
    obj = OUT / (src.name + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[cmd.index("-c"):cmd.index("-c")] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip() and verbose:
        print(r.stderr, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    OUT.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    tmp = SERVER.with_name(SERVER.name + ".tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", f"-I{ROOT / 'include'}",
           str(CSRC / "persistent.cpp"), f"-L{PKG}", "-lgehtp", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"server build failed\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, SERVER)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
