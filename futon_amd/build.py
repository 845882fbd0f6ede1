"""Builds futon_amd/libfuton_hip.so (HIP kernels + C ABI + C++ host layer)
for gfx950 in-tree.

Each ``csrc/*.hip`` is compiled by hipcc and each ``csrc/host/*.cpp`` (the
host side: pack loading, tokenizer, provider) by the host C++ compiler, in
parallel; everything is linked into one shared library next to this file.
Flags:

* ``--offload-arch=gfx950`` — MI355X only; no other targets, no host fallback.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` — keep the compiler from
  emitting packed-FP32 VALU ops.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libfuton_hip.so")
CLI = os.path.join(HERE, "futon_embed")
OBJ = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
HOST = os.path.join(CSRC, "host")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(os.path.dirname(HERE), "include"),
]


HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(os.path.dirname(HERE), "include")]

# Per-file code-generation options.  attention.hip: keep MFMA results in
# VGPRs (its softmax reads every score tile right after the MFMA; in AGPRs
# each element would cost an extra v_accvgpr_read), and let fmaxf skip the
# NaN-quieting copy of each operand (scores are finite or −inf for masked
# keys, so the results are bit-identical; ~2% faster).
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"]}


def sources() -> list[str]:
    hip = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    host = sorted(os.path.join(HOST, f) for f in os.listdir(HOST) if f.endswith(".cpp"))
    return hip + host


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    if src.endswith(".cpp"):
        cmd = [CXX, *HOST_FLAGS, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libfuton_hip.so failed")
    os.replace(tmp, LIB)
    # The `futon embed` command on this library (csrc/cli/futon_embed.cpp).
    cmd = [CXX, *HOST_FLAGS, os.path.join(CSRC, "cli", "futon_embed.cpp"), "-o", CLI + ".tmp", "-L", HERE,
           "-lfuton_hip", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("build of futon_embed failed")
    os.replace(CLI + ".tmp", CLI)
    if verbose:
        print(f"built {LIB} and {CLI}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
