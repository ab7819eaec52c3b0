"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

The reference runs its device probes under compute-sanitizer
(cuda-rust-probe/run.sh:3-24). GPU-side sanitizers are not available for
gfx950 here, so the host code that takes untrusted input or owns resources
runs under clang's ASan + UBSan instead:

- libribn_amd built by `python -m engine_amd.build --sanitize` (the host side
  of every source instrumented; device code as in the product). A child
  interpreter preloads the clang ASan runtime, loads that library through
  RIBN_AMD_LIBRARY and runs the CPU tests of the GGUF reader (the reference's
  error cases, every truncation of a well-formed file, mutated headers and
  directories), of the C-ABI validation, handle ownership and exit release,
  and of the serving rules and backend adapter.
- The C oracle built by `make -C oracle asan`, loaded by the same child
  through KQUANT_ORACLE_LIBRARY, under its golden-vector and decode tests.
- tests/cpp/serving_rules_test.cpp (submission ownership, row scattering)
  compiled with g++ -fsanitize=address,undefined.

Any report ends the sanitized process (-fno-sanitize-recover, halt_on_error)
and fails the test. Leak detection is off: the interpreter itself holds
allocations at exit that LeakSanitizer would report. Nothing here launches a
kernel; the child sees no GPU.
"""
import os
import subprocess
import sys

import pytest

from engine_amd import build as B

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

# CPU tests run again under the sanitizers (the product library and the
# oracle both replaced by their sanitized builds).
CHILD_TESTS = ["test_gguf.py", "test_abi.py", "test_exit_release.py", "test_serving.py", "test_oracle.py",
               "test_oracle_decode.py", "test_oracle_q8_1.py"]


def asan_runtime() -> str:
    out = subprocess.run([B.hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True).stdout.strip()
    if not out or not os.path.exists(out):
        pytest.skip("clang ASan runtime not found next to hipcc")
    return out


@pytest.fixture(scope="module")
def sanitized_libs():
    if not B.sanitized_is_current():
        B.build_sanitized()
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    return B.ASAN_LIB, os.path.join(ROOT, "oracle", "build", "libkquant_oracle_asan.so")


def test_host_code_under_asan_and_ubsan(sanitized_libs):
    lib, oracle_lib = sanitized_libs
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": asan_runtime(),
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:detect_stack_use_after_return=1:strict_string_checks=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "RIBN_AMD_LIBRARY": lib,
        "KQUANT_ORACLE_LIBRARY": oracle_lib,
        "HIP_VISIBLE_DEVICES": "-1",
    })
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
           *[os.path.join(HERE, t) for t in CHILD_TESTS]]
    res = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    report = res.stdout[-4000:] + res.stderr[-8000:]
    assert "AddressSanitizer" not in res.stderr and "runtime error:" not in res.stderr, report
    assert res.returncode == 0, report
    assert " passed" in res.stdout and " failed" not in res.stdout, report


def test_child_really_loads_the_sanitized_builds(sanitized_libs):
    """The libraries the child runs are the instrumented ones."""
    lib, oracle_lib = sanitized_libs
    for path in (lib, oracle_lib):
        undefined = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True, text=True).stdout
        assert "__asan_report_load" in undefined, path
        assert "__ubsan_handle_" in undefined, path
    env = dict(os.environ, LD_PRELOAD=asan_runtime(), ASAN_OPTIONS="detect_leaks=0", RIBN_AMD_LIBRARY=lib,
               KQUANT_ORACLE_LIBRARY=oracle_lib, HIP_VISIBLE_DEVICES="-1")
    probe = ("from engine_amd import _lib; from oracle import kquant_oracle as O; "
             "_lib.load(); O.lib(); print(_lib.LIB_PATH); print(O.LIB_PATH)")
    out = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True,
                         check=True).stdout.split()
    assert out == [lib, oracle_lib]


def test_serving_rules_cpp_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "serving_rules_test_asan"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", "-Wall", "-Werror", "-I", os.path.join(ROOT, "engine_amd", "csrc"),
                    os.path.join(HERE, "cpp", "serving_rules_test.cpp"), "-o", str(exe)], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    env.pop("LD_PRELOAD", None)
    out = subprocess.run([str(exe)], capture_output=True, text=True, env=env)
    assert out.returncode == 0, out.stderr[-4000:]
    assert out.stdout.strip() == "ok"
