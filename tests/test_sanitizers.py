"""Host AddressSanitizer + UndefinedBehaviorSanitizer runs, on the CPU only:

- the oracle, built with both sanitizers (`make -C oracle sanitize`), driven over every function
  on exact-size buffers and edge shapes (oracle/sanity_main.c);
- the C ABI's argument checks: every entry point of include/forge_amd.h called with empty
  shapes, null operands, contract violations and extreme sizes from a sanitized host program
  (tests/cpp/abi_args.cpp) linked against the library built with host-side sanitizers
  (forge_amd/build_san.py; the device code is the ordinary gfx950 build). No GPU is touched:
  calls that pass the checks fail with "no device".
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1",
               HIP_VISIBLE_DEVICES="", ROCR_VISIBLE_DEVICES="")


def test_oracle_under_asan_ubsan():
    r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    exe = os.path.join(ROOT, "oracle", "lib", "oracle_sanity")
    r = subprocess.run([exe], capture_output=True, text=True, env=SAN_ENV, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout


def test_c_abi_argument_checks_under_asan_ubsan():
    import importlib.util
    spec = importlib.util.spec_from_file_location("forge_build_san_driver",
                                                  os.path.join(ROOT, "tests", "cpp", "build_san.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    exe = mod.build()
    r = subprocess.run([exe], capture_output=True, text=True, env=SAN_ENV, timeout=300, cwd="/tmp")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all expectations hold" in r.stdout
