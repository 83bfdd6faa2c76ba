"""Builds libforge_amd.so for gfx950 in-tree with hipcc (no cmake/ninja needed).

    python -m forge_amd.build          # or forge_amd.build.build()

Objects go to forge_amd/_build/, the library to forge_amd/lib/libforge_amd.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libforge_amd.so")
# Measurement probes (bench.py --probes), a library of their own: not part of the product.
PROBE_LIB = os.path.join(LIBDIR, "libforge_probes.so")
PROBE_SOURCES = ["probes.hip"]

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 VALU forms (v_pk_*_f32) are disabled for all device code: some of their forms
# have given wrong results on these GPUs without any error.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-x", "hip",
    "-Wall", "-Wno-unused-result", "-ffp-contract=on",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
] + DEVICE_FLAGS

SOURCES = [
    "runtime.hip",
    "quantize.hip",
    "sparsity.hip",
    "gemm_dense.hip",
    "gemm_skinny.hip",
    "gemm_decode.hip",
    "gemm_sparse.hip",
    "gemm_sparse_wide.hip",
    "conv.hip",
    "conv_window.hip",
    "conv_transpose.hip",
    "conv_depthwise.hip",
    "noalloc.hip",
    "forge_api.cpp",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + COMMON_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # The host pass does not know the device-only feature flag: that warning is expected.
    noise = [l for l in r.stderr.splitlines() if l.strip() and "packed-fp32-ops" not in l]
    if noise:
        sys.stderr.write(f"[{src}]\n" + "\n".join(noise) + "\n")
    return obj


def _link(objs: list, lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = dict(zip(srcs, ex.map(_compile, srcs)))
    _link([objs[s] for s in SOURCES], LIB)
    _link([objs[s] for s in PROBE_SOURCES], PROBE_LIB)
    return LIB


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    print(build())
