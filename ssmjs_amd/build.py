"""Builds ssmjs_amd/libssm_hip.so (the C ABI in include/ssm_hip.h) for gfx950 with hipcc.

Each .hip source under ssmjs_amd/csrc is compiled separately (in parallel) and linked
against rocBLAS. When Node's headers are installed, the Node-API addon
ssmjs_amd/napi/ssm_napi.node (the binding the TypeScript host loads) is built next to it
with the host compiler. Usage:  python -m ssmjs_amd.build  [-j N]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_obj")
LIB = os.path.join(HERE, "libssm_hip.so")
SOURCES = ["conv1d.hip", "scan_m1.hip", "ssd.hip", "ssd_f32.hip", "glue.hip", "rowgemm.hip",
           "stepproj.hip", "head.hip", "gemm.hip", "sample.hip", "model.hip"]
ARCH = os.environ.get("SSM_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
NAPI_SRC = os.path.join(HERE, "napi", "ssm_napi.cc")
NAPI_OUT = os.path.join(HERE, "napi", "ssm_napi.node")
NODE_INCLUDE = os.environ.get("NODE_INCLUDE", "/usr/include/node")

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    # packed-FP32 VALU forms stay off (only the scalar and vector FP32 paths are emitted)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-command-line-argument",
    "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-6000:]}")
    return obj


# host-only C++ (no device code), built with the host compiler
HOST_SOURCES = ["ssmw.cpp"]


def _compile_host(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".host.o")
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-Wall", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed on {src}:\n{r.stderr[-6000:]}")
    return obj


def build(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(SOURCES)))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    objs += [_compile_host(src) for src in HOST_SOURCES]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-lrocblas", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    if build_napi() and verbose:
        print("built", NAPI_OUT)
    return LIB


def build_napi() -> bool:
    """Node-API addon over libssm_hip.so; skipped (False) when node_api.h is absent."""
    if not os.path.exists(os.path.join(NODE_INCLUDE, "node_api.h")):
        return False
    tmp = NAPI_OUT + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-shared", "-fPIC", "-Wall",
           "-DNODE_GYP_MODULE_NAME=ssm_napi", "-I", NODE_INCLUDE, NAPI_SRC, "-o", tmp,
           "-L" + HERE, "-lssm_hip", "-Wl,-rpath,$ORIGIN/.."]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"Node-API addon build failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, NAPI_OUT)
    return True


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    try:
        build(a.j, verbose=True)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
