"""The memory API kept from the reference, on the CPU: tests/cpp/memory_api.cpp
(ArenaAllocator 128-B bump allocation and out-of-memory throw,
include/memory/alloc.h:17-29; MemoryPlanner 16-B allocation,
memory_planner.h:11-26; the engine's [L0_K | L0_V | ...] KV pool carve as
64-bit Views, src/core/engine.cu:187-215) built with g++ against the library."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "atomflow_amd")


def test_memory_api_cpp(tmp_path):
    exe = str(tmp_path / "memory_api")
    src = os.path.join(ROOT, "tests", "cpp", "memory_api.cpp")
    assert os.path.exists(os.path.join(LIBDIR, "libatomflow_kv.so")), "build the library first"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "include"), src,
                    "-L", LIBDIR, "-latomflow_kv", f"-Wl,-rpath,{LIBDIR}",
                    "-Wl,-rpath-link,/opt/rocm/lib", "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.returncode, r.stdout, r.stderr)
