"""The split-K combine of decode_attn_kernel publishes its partials without a
release/acquire fence. It relies on gfx950 instruction semantics instead:
agent-scope stores (`sc1`) retired by `s_waitcnt vmcnt(0)`, an `s_barrier`,
then one returning `global_atomic_add`; the last arrival reads with
agent-scope loads (`sc1`) issued after that atomic. This test compiles
decode_attention.hip for gfx950 (device code only, assembly out) and checks
that order in every instantiation that has a combine, so a compiler change
that reorders or drops any of it fails here, on the CPU. The key pieces of
prefill_attention_kernel publish and merge the same way and are checked too."""
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


def _functions(asm, kernel="decode_attn_kernel", end="s_endpgm"):
    pat = re.compile(r"^(_Z\S*" + kernel + r"\S*):[^\n]*\n(.*?)" + end, re.S | re.M)
    for name, body in pat.findall(asm):
        lines = [l.strip() for l in body.splitlines()]
        yield name, [l for l in lines if l and not l.startswith(";") and not l.startswith(".")]


@pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_combine_publication_order(tmp_path):
    r, out = _compile(tmp_path)
    assert r.returncode == 0, r.stderr[-2000:]
    asm = open(out).read()
    checked = 0
    for name, ins in _functions(asm):
        atomics = [i for i, l in enumerate(ins) if l.startswith("global_atomic")]
        if not atomics:
            continue  # an instantiation whose grid never splits has no combine
        assert len(atomics) == 1, (name, [ins[i] for i in atomics])
        a = atomics[0]
        assert re.match(r"global_atomic_add\s+v\d+, v\d+, v\d+, s\[\d+:\d+\]\s+sc0$", ins[a]), \
            (name, ins[a])  # returning (sc0), agent scope: no sc1 / nt bits
        # the barrier the atomic waits behind, and the full vmcnt wait before it
        bar = max(i for i in range(a) if ins[i].startswith("s_barrier"))
        wait = max(i for i in range(bar) if ins[i].startswith("s_waitcnt"))
        assert "vmcnt(0)" in ins[wait] or ins[wait] == "s_waitcnt 0", (name, ins[wait])
        between = ins[wait + 1:a]
        assert not any(l.startswith(("global_", "buffer_", "flat_")) for l in between), \
            (name, between)
        # partial records: agent-scope stores, all before that wait
        stores = [i for i, l in enumerate(ins) if l.startswith("global_store") and " sc1" in l]
        before = [i for i in stores if i < wait]
        after = [i for i in stores if i > a]
        assert len(before) >= 3, (name, [ins[i] for i in stores])  # o pair + m + l
        assert len(after) <= 1, (name, [ins[i] for i in after])  # the counter re-arm only
        assert not any(wait < i < a for i in stores)
        # the combine's reads: agent-scope loads, none before the atomic
        loads = [i for i, l in enumerate(ins) if l.startswith("global_load") and " sc1" in l]
        assert loads and min(loads) > a, (name, min(loads) if loads else None, a)
        checked += 1
    assert checked >= 30, checked


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
    for name, ins in _functions(asm, "prefill_attention_kernel", end=r"\.Lfunc_end"):
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
