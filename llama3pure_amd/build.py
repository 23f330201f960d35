"""Builds libl3p.so (HIP, gfx950) in-tree with hipcc, and the Node.js N-API
addon js/l3p_napi.node over it when Node's headers are installed.

    python -m llama3pure_amd.build

Every source is compiled with -ffp-contract=off (elementwise code must round
like the reference's scalar C; the kernels request fused multiply-adds
explicitly where the summation tolerance allows them) and without packed
fp32 instructions.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libl3p.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["gemv.hip", "gemm.hip", "blocks.hip", "layers.hip", "api.cpp", "model.cpp"]
ARCH = os.environ.get("L3P_ARCH", "gfx950")

FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-result", f"-I{os.path.join(HERE, '..', 'include')}"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src + ".o")
    cmd = [hipcc(), *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    return obj


def build() -> str:
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, OUT)
    build_napi()
    return OUT


NAPI_SRC = os.path.join(HERE, "..", "js", "l3p_napi.c")
NAPI_OUT = os.path.join(HERE, "..", "js", "l3p_napi.node")


def node_include() -> str | None:
    for d in ("/usr/include/node", "/usr/local/include/node"):
        if os.path.exists(os.path.join(d, "node_api.h")):
            return d
    return None


def build_napi() -> str | None:
    """js/l3p_napi.node, linked against libl3p.so through an $ORIGIN rpath."""
    inc = node_include()
    if inc is None:
        sys.stderr.write("node_api.h not found: the N-API addon is not built\n")
        return None
    tmp = NAPI_OUT + ".tmp"
    cmd = ["gcc", "-O2", "-Wall", "-shared", "-fPIC", "-DNODE_GYP_MODULE_NAME=l3p_napi", f"-I{inc}", NAPI_SRC,
           "-o", tmp, f"-L{HERE}", "-l:libl3p.so", "-Wl,-rpath,$ORIGIN/../llama3pure_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("N-API addon build failed")
    os.replace(tmp, NAPI_OUT)
    return NAPI_OUT


if __name__ == "__main__":
    print(build())
