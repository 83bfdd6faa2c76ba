"""Builds tests/cpp/lib/libforge_caller.so: a C++ program's view of the drop-in API
(include/forge/**.h), linked against forge_amd/lib/libforge_amd.so. Test infrastructure,
built by __graft_entry__.build() after the library itself."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
LIB = os.path.join(HERE, "lib", "libforge_caller.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def build() -> str:
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    libdir = os.path.join(ROOT, "forge_amd", "lib")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           f"-I{os.path.join(ROOT, 'include')}", os.path.join(HERE, "forge_caller.hip"),
           f"-L{libdir}", "-lforge_amd", "-Wl,-rpath,$ORIGIN/../../../forge_amd/lib", "-o", LIB + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    sys.stdout.write(build() + "\n")
