"""Builds tests/cpp/lib/abi_args_san: the C-ABI argument checks (abi_args.cpp) as a host program
with AddressSanitizer + UndefinedBehaviorSanitizer, linked against the host-sanitized library
(forge_amd.build_san, built first when missing or stale). CPU only: run by
tests/test_sanitizers.py, never on a GPU."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
EXE = os.path.join(HERE, "lib", "abi_args_san")
CLANGXX = os.environ.get("FORGE_SAN_CXX", "/opt/rocm/llvm/bin/clang++")


def build() -> str:
    sys.path.insert(0, ROOT)
    from forge_amd import build_san
    if build_san.stale():
        build_san.build()
    os.makedirs(os.path.dirname(EXE), exist_ok=True)
    cmd = [CLANGXX, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           f"-I{os.path.join(ROOT, 'include')}", os.path.join(HERE, "abi_args.cpp"),
           f"-L{build_san.LIBDIR}", "-lforge_amd_san", f"-Wl,-rpath,{build_san.LIBDIR}",
           "-o", EXE + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(EXE + ".tmp", EXE)
    return EXE


if __name__ == "__main__":
    sys.stdout.write(build() + "\n")
