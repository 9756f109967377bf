"""The C ABI library builds, loads without a GPU, and exports every symbol the
public headers declare; the C++ headers compile and link in a host program."""
import os
import re
import subprocess

import pytest

import atomflow_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = ["include/af_kv.h", "include/af_runtime.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(os.path.join(ROOT, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(af_\w+)\s*\(", text, re.M):
            names.add(m.group(1))
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", atomflow_amd.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_every_declared_function_is_exported():
    decl = declared_functions()
    assert len(decl) > 50
    missing = decl - exported_symbols()
    assert not missing, sorted(missing)


def test_ctypes_prototypes_cover_the_headers():
    from atomflow_amd import _abi

    assert declared_functions() == set(_abi.PROTOTYPES), (
        sorted(declared_functions() ^ set(_abi.PROTOTYPES)))


def test_library_loads_and_reports_status_strings():
    lib = atomflow_amd.lib()
    assert lib.af_version() > 0
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10):
        assert lib.af_status_string(code)
        assert lib.af_status_string(code).decode() != "unknown status", code
    assert lib.af_status_string(-1).decode() == "block pool exhausted"
    assert atomflow_amd.AF_ERR_TIMEOUT == -10


def test_host_only_entry_points_without_gpu():
    from atomflow_amd import kv
    import oracle

    c, s = kv.rope_table_host(300, 128, 500000.0)
    oc, os_ = oracle.rope_table(300, 128, 500000.0)
    assert (c.view("u4") == oc.view("u4")).all() and (s.view("u4") == os_.view("u4")).all()
    lib = atomflow_amd.lib()
    assert lib.af_attention_workspace_size(1, 24, 8, 128, 64) > 64 * 1024
    assert lib.af_attention_workspace_size(0, 24, 8, 128, 64) == 0
    p = kv.make_pool(0, atomflow_amd.AF_KV_FP16, 16, 28, 8, 128, 1000)
    assert kv.pool_bytes(p) == 28 * 2 * 1000 * 16 * 1024 * 2
    # argument validation happens before any device call
    assert lib.af_rope_append(None, None, None, None, None, 0, None, 16, 24, 8, 128, None,
                              None) == atomflow_amd.AF_ERR_INVALID_ARG


def test_default_split_counts():
    """The split heuristic on a 256-CU device (the CU count a host without a GPU
    assumes, MI355X's). Batch 1, 8 KV heads: ~3/4 of a workgroup per CU up to
    ctx 24k, then ~1024-row spans but never more workgroups than CUs (33 splits
    at ctx 32k put two workgroups on 8 CUs and ran a third slower). Batches:
    ~512 rows per split."""
    from atomflow_amd import kv
    assert kv.default_splits(8193, 1, 8) == 24
    assert kv.default_splits(24577, 1, 8) == 25  # ceil(24577 / 1024)
    # one workgroup per CU at most, counting each pair's combiner and one spare CU per pair
    assert kv.default_splits(32769, 1, 8) == 30
    assert kv.default_splits(131072, 1, 8) == 30
    assert kv.default_splits(1025, 1, 8) == 17   # one 64-row step per split
    assert kv.default_splits(8193, 32, 8) == 17  # batched: ceil(8193 / 512)
    assert kv.default_splits(0, 1, 8) == 1
    # more splits than the combiner form takes (32): no CUs held back for combiners
    assert kv.default_splits(200000, 1, 2) == 128  # kMaxSplits; 126 with the combiner's room
    assert kv.default_splits(32769, 1, 4) == 48    # 3/4 of a workgroup per CU


def test_shared_prefix_argument_checks_without_gpu():
    """af_paged_attention_shared_prefix validates its arguments before any device
    call: a negative prefix, a missing prefix table, more key splits than 64-row
    tiles, a prefix past the table, head_dim other than 128, an empty pool."""
    import ctypes
    from atomflow_amd import kv
    lib = atomflow_amd.lib()
    fake = 0x10000  # never dereferenced: every call below fails validation first
    pool = kv.make_pool(fake, atomflow_amd.AF_KV_FP16, 16, 2, 8, 128, 1000)

    def call(p, prefix_table, prefix, psplits, max_blocks=64):
        return lib.af_paged_attention_shared_prefix(
            fake, 3072, ctypes.byref(p), 0, prefix_table, prefix, psplits, fake, max_blocks, fake,
            4, 1000, fake, 3072, 24, 0, fake, 1 << 30, None)

    assert call(pool, fake, -1, 0) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(pool, None, 200, 0) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(pool, fake, 200, -1) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(pool, fake, 200, 5) == atomflow_amd.AF_ERR_INVALID_ARG  # ceil(200 / 64) = 4
    assert call(pool, fake, 64 * 16 + 1, 0) == atomflow_amd.AF_ERR_OUT_OF_RANGE
    p64 = kv.make_pool(fake, atomflow_amd.AF_KV_FP16, 16, 2, 8, 64, 1000)
    assert call(p64, fake, 200, 0) == atomflow_amd.AF_ERR_UNSUPPORTED
    empty = kv.make_pool(fake, atomflow_amd.AF_KV_FP16, 16, 2, 8, 128, 0)
    assert call(empty, fake, 200, 0) == atomflow_amd.AF_ERR_INVALID_ARG
    # pool flags: AF_KV_POOL_SHARED_BLOCKS is the only defined bit
    odd = kv.make_pool(fake, atomflow_amd.AF_KV_FP16, 16, 2, 8, 128, 1000, flags=2)
    assert call(odd, fake, 200, 0) == atomflow_amd.AF_ERR_INVALID_ARG
    shared = kv.make_pool(fake, atomflow_amd.AF_KV_FP16, 16, 2, 8, 128, 1000,
                          flags=atomflow_amd.AF_KV_POOL_SHARED_BLOCKS)
    assert lib.af_kv_pool_bytes(ctypes.byref(shared)) == lib.af_kv_pool_bytes(ctypes.byref(pool))


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(atomflow_amd, "_lib", None)
    monkeypatch.setattr(atomflow_amd, "LIB_PATH", "/nonexistent/libatomflow_kv.so")
    with pytest.raises(RuntimeError, match="missing"):
        atomflow_amd.lib()


def test_cpp_headers_compile_and_link(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text(r'''
#include "core/view.h"
#include "memory/block_manager.h"
#include "memory/memory_planner.h"
#include <cstdio>
#include <vector>
int main() {
    using namespace atomflow::server;
    BlockManager bm;
    PoolConfig c; c.total_blocks = 8; c.block_size = 16; c.n_layers = 2; c.n_kv_heads = 8;
    c.head_dim = 128;
    bm.initialize(c, false, nullptr);
    if (bm.allocate_block() != 0 || bm.num_free_blocks() != 7) return 1;
    bm.free_block(0);
    bool threw = false;
    try { bm.free_block(0); } catch (const std::invalid_argument&) { threw = true; }
    if (!threw) return 2;
    int s = bm.create_sequence();
    AppendSlot a;
    if (bm.append_token(s, &a) != 0 || a.position != 0 || a.slot != 0) return 3;
    std::vector<char> arena(1024);
    MemoryPlanner mp(arena.data(), arena.size());
    float* f = mp.allocate<float>(3);
    if (mp.get_offset() != 16 || !f) return 4;
    threw = false;
    try { mp.allocate<char>(2000); } catch (const std::runtime_error&) { threw = true; }
    if (!threw) return 5;
    View v = create_contiguous_view(nullptr, DataType::FP16, {32769, 1024});
    if (v.strides[0] != 1024 || v.offset(32768, 5) != size_t(32768) * 1024 + 5) return 6;
    View big = create_contiguous_view(nullptr, DataType::FP8_E4M3, {28, 2, 50000 * 32, 1024});
    if (big.numel() != int64_t(28) * 2 * 50000 * 32 * 1024) return 7;
    std::puts("ok");
    return 0;
}
''')
    exe = tmp_path / "t"
    libdir = os.path.dirname(atomflow_amd.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), str(src),
                    "-L", libdir, "-latomflow_kv", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
