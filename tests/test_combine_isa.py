"""The split-K combine of decode_attn_kernel publishes its partials without a
release/acquire fence. It relies on gfx950 instruction semantics instead:
agent-scope stores (`sc1`) retired by `s_waitcnt vmcnt(0)`, an `s_barrier`,
then one returning `global_atomic_add`; the last arrival reads with
agent-scope loads (`sc1`) issued after that atomic. The dedicated-combiner
form publishes with an agent-scope ready-flag store behind the same wait and
barrier, and the persistent form's arrival follows the same rule. This test
compiles decode_attention.hip for gfx950 (device code only, assembly out) and
checks that order in every instantiation, read to the end of each function,
so a compiler change that reorders or drops any of it fails here, on the CPU.
The key pieces of prefill_attention_kernel publish and merge the same way and
are checked too."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "atomflow_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _compile(tmp_path, arch="gfx950", src="decode_attention"):
    out = str(tmp_path / f"{src}.s")
    cmd = [HIPCC, f"--offload-arch={arch}", "-O3", "-std=c++17", "--cuda-device-only", "-S",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(ROOT, "include"), "-I", CSRC,
           os.path.join(CSRC, f"{src}.hip"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    return r, out


@pytest.fixture(scope="module")
def decode_asm(tmp_path_factory):
    """decode_attention.hip's gfx950 assembly, compiled once for the tests below."""
    if not os.path.exists(HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    r, out = _compile(tmp_path_factory.mktemp("decode_asm"))
    assert r.returncode == 0, r.stderr[-2000:]
    return open(out).read()


def _functions(asm, kernel="decode_attn_kernel", end=r"\.Lfunc_end"):
    """(name, instructions) of every function whose name contains `kernel`, read
    to its end (early exits end in s_endpgm blocks of their own)."""
    pat = re.compile(r"^(_Z\S*" + kernel + r"\S*):[^\n]*\n(.*?)" + end, re.S | re.M)
    for name, body in pat.findall(asm):
        lines = [l.strip() for l in body.splitlines()]
        yield name, [l for l in lines if l and not l.startswith(";") and not l.startswith(".")]


def _is_mem(l):
    return l.startswith(("global_", "buffer_", "flat_"))


def _full_wait(l):
    return l.startswith("s_waitcnt") and ("vmcnt(0)" in l or l == "s_waitcnt 0")


def _sc1_stores(ins):
    return [i for i, l in enumerate(ins) if l.startswith("global_store") and " sc1" in l]


def _publication(name, ins, signal):
    """The partial records' agent-scope stores, a full vector-memory wait, an
    s_barrier and then the instruction at index `signal` (the arrival atomic or
    the ready-flag store), with no memory instruction between the wait and it.
    Returns the wait's index."""
    bar = max(i for i in range(signal) if ins[i].startswith("s_barrier"))
    wait = max(i for i in range(bar) if ins[i].startswith("s_waitcnt"))
    assert _full_wait(ins[wait]), (name, ins[wait])
    assert not any(_is_mem(l) for l in ins[wait + 1:signal]), (name, ins[wait + 1:signal])
    # partial records (o pair, m, l) go out with agent-scope stores before the wait
    records = [i for i in _sc1_stores(ins) if i < wait]
    assert len(records) >= 3, (name, [ins[i] for i in records])
    return wait


def _arrival_atomics(ins):
    return [i for i, l in enumerate(ins) if l.startswith("global_atomic")]


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_combine_publication_order(decode_asm):
    asm = decode_asm
    grid = comb = persistent = 0
    for name, ins in _functions(asm, "decode_attn_kernel"):
        atomics = _arrival_atomics(ins)
        m = re.search(r"decode_attn_kernelILi\d+ELi\d+E((?:Lb[01]E)+)E", name)
        # bool arguments: FP8, PAGED, FUSED, PAIR, COMB, CACHED
        if m and re.findall(r"Lb([01])E", m.group(1))[4] == "1":
            # dedicated-combiner form: no arrival counter; each split publishes
            # with its ready flag, an agent-scope store behind the same wait and
            # barrier, and the combiner polls the flags and loads the records
            # with agent-scope loads
            assert not atomics, (name, [ins[i] for i in atomics])
            flags = [i for i in _sc1_stores(ins) if ins[i].startswith("global_store_dword ")]
            published = []
            for f in flags:
                try:
                    published.append(_publication(name, ins, f))
                except (AssertionError, ValueError):
                    continue
            assert len(published) == 1, (name, [ins[i] for i in flags])
            loads = [i for i, l in enumerate(ins) if l.startswith("global_load") and " sc1" in l]
            assert len(loads) >= 3, (name, len(loads))  # poison word, flags, records
            comb += 1
            continue
        # every other instantiation: one returning, agent-scope arrival atomic
        assert len(atomics) == 1, (name, [ins[i] for i in atomics])
        a = atomics[0]
        assert re.match(r"global_atomic_add\s+v\d+, v\d+, v\d+, s\[\d+:\d+\]\s+sc0$", ins[a]), \
            (name, ins[a])  # returning (sc0), agent scope: no sc1 / nt bits
        wait = _publication(name, ins, a)
        after = [i for i in _sc1_stores(ins) if i > a]
        assert len(after) <= 1, (name, [ins[i] for i in after])  # the counter re-arm only
        # the combine's reads: agent-scope loads, none before the atomic
        loads = [i for i, l in enumerate(ins) if l.startswith("global_load") and " sc1" in l]
        assert loads and min(loads) > a, (name, min(loads) if loads else None, a)
        assert not any(wait < i < a for i in _sc1_stores(ins))
        grid += 1
    for name, ins in _functions(asm, "decode_attn_persistent"):
        # item claim, arrival, finished-workgroup count: the arrival is the one
        # behind the records' publication
        atomics = _arrival_atomics(ins)
        assert len(atomics) == 3, (name, [ins[i] for i in atomics])
        arrivals = []
        for a in atomics:
            try:
                _publication(name, ins, a)
                arrivals.append(a)
            except (AssertionError, ValueError):
                continue
        assert len(arrivals) == 1, (name, [ins[i] for i in atomics])
        a = arrivals[0]
        assert re.match(r"global_atomic_add\s+v\d+, v\d+, v\d+, s\[\d+:\d+\]\s+sc0$", ins[a]), \
            (name, ins[a])
        loads = [i for i, l in enumerate(ins) if l.startswith("global_load") and " sc1" in l and i > a]
        assert len(loads) >= 3, (name, len(loads))  # (m, l) and the first batch of records
        persistent += 1
    # 100 grid-form kernels (contiguous / paged, fp16 / FP8, fused, pairs, 3wg;
    # paged ones with both KV load policies), 8 dedicated-combiner kernels, 60
    # persistent kernels (both policies)
    assert grid >= 100 and comb == 8 and persistent == 60, (grid, comb, persistent)


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_other_targets_refused(tmp_path):
    r, _ = _compile(tmp_path, arch="gfx942")
    assert r.returncode != 0
    assert "target gfx950 only" in r.stderr


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_prefill_key_piece_publication_order(tmp_path):
    r, out = _compile(tmp_path, src="prefill_attention")
    assert r.returncode == 0, r.stderr[-2000:]
    asm = open(out).read()
    checked = 0
    # the whole function: early exits (a piece a lighter tile does not need) end
    # in s_endpgm blocks of their own
    for name, ins in _functions(asm, "prefill_attention_kernel"):
        atomics = [i for i, l in enumerate(ins) if l.startswith("global_atomic")]
        assert len(atomics) == 1, (name, [ins[i] for i in atomics])
        a = atomics[0]
        assert re.match(r"global_atomic_add\s+v\d+, v\d+, v\d+, s\[\d+:\d+\]\s+sc0$", ins[a]), \
            (name, ins[a])
        bar = max(i for i in range(a) if ins[i].startswith("s_barrier"))
        # the full vector-memory wait before that barrier (an LDS wait may follow it)
        wait = max(i for i in range(bar) if ins[i].startswith("s_waitcnt") and
                   ("vmcnt(0)" in ins[i] or ins[i] == "s_waitcnt 0"))
        assert not any(l.startswith(("global_", "buffer_", "flat_")) for l in ins[wait + 1:a])
        stores = [i for i, l in enumerate(ins) if l.startswith("global_store") and " sc1" in l]
        before = [i for i in stores if i < wait]
        after = [i for i in stores if i > a]
        assert len(before) >= 32 + 2, (name, len(before))  # 32 o words per lane + m + l
        assert len(after) <= 1, (name, [ins[i] for i in after])  # the counter re-arm only
        loads = [i for i, l in enumerate(ins) if l.startswith("global_load") and " sc1" in l]
        assert loads and min(loads) > a, (name, min(loads) if loads else None, a)
        checked += 1
    assert checked == 3, checked  # contiguous, paged fp16, paged FP8


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_kv_rows_load_policy(decode_asm):
    """Decode kernels read KV rows with non-temporal 16-byte loads (`global_load_dwordx4 ...
    nt`), except the CACHED instantiations (pools with AF_KV_POOL_SHARED_BLOCKS), which use no
    non-temporal load at all."""
    asm = decode_asm
    seen = {False: 0, True: 0}
    for kernel in ("decode_attn_kernel", "decode_attn_persistent"):
        for name, ins in _functions(asm, kernel):
            m = re.search(kernel + r"(?:_3wg)?ILi\d+ELi\d+E((?:Lb[01]E)+)E", name)
            assert m, name
            cached = re.findall(r"Lb([01])E", m.group(1))[-1] == "1"  # the last: CACHED
            nt = [l for l in ins if l.startswith("global_load_dwordx4") and l.endswith(" nt")]
            assert (not nt) if cached else len(nt) >= 4, (name, len(nt))
            seen[cached] += 1
    assert seen[False] >= 98 and seen[True] >= 70, seen
