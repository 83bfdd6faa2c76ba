"""Host-sanitized build of the library, for CPU-only argument-check tests.

    python -m forge_amd.build_san

Compiles the same sources as forge_amd.build with AddressSanitizer and UndefinedBehaviorSanitizer
on the host side only (each flag passed with -Xarch_host; the gfx950 device code is built as
usual), into forge_amd/_build_san/ and forge_amd/lib_san/libforge_amd_san.so. The library
leaves the sanitizer runtime symbols to the program that loads it, which must itself be built
with -fsanitize=address,undefined by the same clang (tests/cpp/build_san.py). Not used on a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

from . import build as _b

BUILD = os.path.join(_b.HERE, "_build_san")
LIBDIR = os.path.join(_b.HERE, "lib_san")
LIB = os.path.join(LIBDIR, "libforge_amd_san.so")

HOST_SAN = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=all",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-g",
]


def _newest_header() -> float:
    t = 0.0
    for d in (_b.CSRC, os.path.join(_b.ROOT, "include")):
        for base, _, files in os.walk(d):
            for f in files:
                if f.endswith((".h", ".hpp")):
                    t = max(t, os.path.getmtime(os.path.join(base, f)))
    return t


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if os.path.exists(obj) and os.path.getmtime(obj) > max(_newest_header(),
                                                           os.path.getmtime(os.path.join(_b.CSRC, src))):
        return obj   # up to date
    cmd = [_b.HIPCC] + _b.COMMON_FLAGS + HOST_SAN + ["-c", os.path.join(_b.CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def stale() -> bool:
    """True when the sanitized library is missing or older than a source or header."""
    if not os.path.exists(LIB):
        return True
    t = os.path.getmtime(LIB)
    for d in (_b.CSRC, os.path.join(_b.ROOT, "include")):
        for base, _, files in os.walk(d):
            if any(os.path.getmtime(os.path.join(base, f)) > t for f in files):
                return True
    return False


def build(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = jobs or min(len(_b.SOURCES), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, _b.SOURCES))
    tmp = LIB + ".tmp"
    cmd = [_b.HIPCC, f"--offload-arch={_b.ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    sys.stdout.write(build() + "\n")
