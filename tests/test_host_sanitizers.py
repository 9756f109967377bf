"""The library's host C++ under AddressSanitizer and UBSan, on the CPU.

The reference's own checks compile to nothing in Release builds
(include/utils/utils.h:108-116), so the BlockManager, scheduler and weight
loader here are also run instrumented. `make -C atomflow_amd/csrc asan` builds
libatomflow_kv_asan.so: the regular HIP objects plus the host sources
(block_manager.cpp, scheduler.cpp, weight_loader.cpp, launchers.cpp,
runtime_abi.cpp) compiled by g++ with -fsanitize=address,undefined and
-fno-sanitize-recover=undefined. The BlockManager random traces, the scheduler
traces, the weight-file and prefill-plan tests then run against it in a child
process (ATOMFLOW_KV_LIB) with libasan preloaded (and libstdc++, so the
runtime's exception interceptor resolves in a C program such as python), and
the C++ memory-API program is built instrumented and linked against it. Any
sanitizer report fails the test.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "atomflow_amd", "csrc")
LIBDIR = os.path.join(ROOT, "atomflow_amd")
ASAN_LIB = os.path.join(LIBDIR, "libatomflow_kv_asan.so")
HOST_TESTS = ["tests/test_block_manager.py", "tests/test_scheduler.py", "tests/test_weights.py",
              "tests/test_prefill_plan.py", "tests/test_abi.py"]
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:verify_asan_link_order=0:halt_on_error=1",
           "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _gcc_file(name):
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    p = r.stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _clean(out):
    return "ERROR: AddressSanitizer" not in out and "runtime error:" not in out


@pytest.fixture(scope="module")
def asan_lib():
    if shutil.which("g++") is None or _gcc_file("libasan.so") is None:
        pytest.skip("g++ with the AddressSanitizer runtime is not available")
    r = subprocess.run(["make", "-C", CSRC, "-j8", "asan"], capture_output=True, text=True,
                       timeout=1200)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return ASAN_LIB


def test_host_code_is_instrumented(asan_lib):
    nm = subprocess.run(["nm", "-D", asan_lib], capture_output=True, text=True).stdout
    assert "__asan_report_load8" in nm and "__ubsan_handle" in nm


def test_host_tests_under_sanitizers(asan_lib):
    env = dict(os.environ, **SAN_ENV, ATOMFLOW_KV_LIB=asan_lib,
               LD_PRELOAD=f"{_gcc_file('libasan.so')} {_gcc_file('libstdc++.so')}")
    r = subprocess.run([sys.executable, "-m", "pytest", *HOST_TESTS, "-q", "-m", "not gpu",
                        "-p", "no:cacheprovider"], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=900)
    out = r.stdout + r.stderr
    print(out[-1500:])
    assert r.returncode == 0 and _clean(out), out[-6000:]
    assert " passed" in out


def test_memory_api_under_sanitizers(asan_lib, tmp_path):
    exe = str(tmp_path / "memory_api_asan")
    src = os.path.join(ROOT, "tests", "cpp", "memory_api.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-I",
                    os.path.join(ROOT, "include"), src, asan_lib, f"-Wl,-rpath,{LIBDIR}",
                    "-Wl,-rpath-link,/opt/rocm/lib", "-o", exe], check=True)
    env = dict(os.environ, **SAN_ENV)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    out = r.stdout + r.stderr
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok") and _clean(out), out[-4000:]
