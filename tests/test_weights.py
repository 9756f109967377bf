"""AtomFlow .bin weights: the exporter (atomflow_amd.weights) and the C++
WeightLoader (af_weights_*), host side."""
import os
import struct
import subprocess

import numpy as np
import pytest

import atomflow_amd
from atomflow_amd import weights as W
from inputs import rng

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SMALL = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300,
             max_seq_len=1024)


def small_model(seed, cfg=SMALL):
    r = rng(seed)
    D, F, V = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    KV = cfg["n_kv_heads"] * D // cfg["n_heads"]
    t = {"embed": r.standard_normal((V, D)).astype(np.float32),
         "final_norm": r.standard_normal(D).astype(np.float32),
         "lm_head": r.standard_normal((V, D)).astype(np.float16)}
    for l in range(cfg["n_layers"]):
        t[f"{l}.input_norm"] = r.standard_normal(D).astype(np.float32)
        t[f"{l}.post_norm"] = r.standard_normal(D).astype(np.float32)
        for name, shape in (("qkv", (D + 2 * KV, D)), ("o_proj", (D, D)), ("gate", (F, D)),
                            ("up", (F, D)), ("down", (D, F))):
            t[f"{l}.{name}"] = (r.standard_normal(shape) * 0.05).astype(np.float32)
    t["0.qkv"][3, :128] = 0.0  # an all-zero group: scale 1
    return t


def test_quantize_fp8_matches_reference_convention_in_torch():
    """quantize_weights.py:220-268 with torch's float8_e4m3fn cast as the encoder."""
    import torch
    r = rng(51)
    w = (r.standard_normal((64, 512)) * r.uniform(0.01, 3.0, (64, 1))).astype(np.float32)
    w[5, 128:256] = 0.0
    w[7, 3] = 1e4  # one group dominated by an outlier
    codes, scales = W.quantize_fp8(w)
    t = torch.from_numpy(w).view(64, 4, 128)
    absmax = t.abs().amax(dim=2)
    sc = torch.where(absmax > 0, absmax / 448.0, torch.ones_like(absmax))
    q = (t / sc.unsqueeze(2)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    assert np.array_equal(codes, q.view(torch.uint8).numpy().reshape(64, 512))
    assert np.array_equal(scales.view(np.uint16), sc.to(torch.float16).numpy().view(np.uint16))


def test_export_and_loader_round_trip(tmp_path):
    path = tmp_path / "m.bin"
    t = small_model(52)
    W.export_bin(path, SMALL, t)
    raw = path.read_bytes()
    magic, ver, gs, *dims = struct.unpack_from("<4si i 7i", raw, 0)
    assert magic == b"ATOM" and ver == 1 and gs == 128
    wf = W.WeightFile(path)
    assert wf.header == dict(version=1, group_size=128, **SMALL)
    assert wf.payload_bytes == len(raw) - 256
    D, F, V = 256, 512, 300
    expect_off = 256

    def check_tensor(kind, layer, arr, dims):
        nonlocal expect_off
        off, nb, shape = wf.tensor(kind, layer)
        assert off + 256 == expect_off and shape == dims and nb == arr.nbytes, (kind, layer)
        assert raw[expect_off:expect_off + nb] == arr.tobytes(), (kind, layer)
        expect_off += -(-nb // 256) * 256

    check_tensor(W.EMBED, -1, t["embed"], (V, D))
    for l in range(2):
        check_tensor(W.INPUT_NORM, l, t[f"{l}.input_norm"], (D, 1))
        check_tensor(W.POST_NORM, l, t[f"{l}.post_norm"], (D, 1))
        kinds = ((W.QKV, W.QKV_SCALES, "qkv"), (W.O_PROJ, W.O_SCALES, "o_proj"),
                 (W.GATE, W.GATE_SCALES, "gate"), (W.UP, W.UP_SCALES, "up"),
                 (W.DOWN, W.DOWN_SCALES, "down"))
        for kw, ks, name in kinds:
            codes, scales = W.quantize_fp8(t[f"{l}.{name}"])
            check_tensor(kw, l, codes, codes.shape)
            check_tensor(ks, l, scales, scales.shape)
    check_tensor(W.FINAL_NORM, -1, t["final_norm"], (D, 1))
    check_tensor(W.LM_HEAD, -1, t["lm_head"], (V, D))
    assert expect_off == len(raw)
    with pytest.raises(atomflow_amd.AfError):
        wf.tensor(W.QKV, 2)  # no layer 2
    wf.close()


def test_loader_rejects_bad_files(tmp_path):
    good = tmp_path / "g.bin"
    W.export_bin(good, SMALL, small_model(53))
    raw = good.read_bytes()
    for name, data in (("magic", b"ATOX" + raw[4:]), ("short", raw[:-300]),
                       ("header", raw[:200]), ("dims", raw[:12] + struct.pack("<i", 100) + raw[16:])):
        p = tmp_path / f"{name}.bin"
        p.write_bytes(data)
        with pytest.raises(atomflow_amd.AfError) as e:
            W.WeightFile(p)
        assert e.value.status == atomflow_amd.AF_ERR_BAD_FILE, name
    with pytest.raises(atomflow_amd.AfError):
        W.WeightFile(tmp_path / "missing.bin")


def test_cpp_weight_loader_layout_and_cursor(tmp_path):
    """The C++ API: the reference cursor (next_block / next<T>) walks the file in
    format order; the layout of the Llama-3.2-3B header equals the byte count of
    the reference engine's own pool arithmetic (engine.cu:57-73, without its
    headroom) plus the header, since every block is already a multiple of 256."""
    path = tmp_path / "m.bin"
    W.export_bin(path, SMALL, small_model(54))
    src = tmp_path / "t.cpp"
    src.write_text(r'''
#include "memory/weight_loader.h"
#include <cstdio>
#include <cstring>
int main(int argc, char** argv) {
    WeightLoader w(argv[1]);
    const AtomHeader& h = w.header;
    if (h.dim != 256 || h.n_layers != 2) return 1;
    const float* emb = w.next<float>(size_t(h.vocab_size) * h.dim);
    if ((const void*)emb != w.data() + 256) return 2;
    for (int l = 0; l < h.n_layers; ++l) {
        w.next<float>(h.dim); w.next<float>(h.dim);
        const int qkv = h.dim + 2 * h.n_kv_heads * (h.dim / h.n_heads);
        const int rows[5] = {qkv, h.dim, h.hidden_dim, h.hidden_dim, h.dim};
        const int cols[5] = {h.dim, h.dim, h.dim, h.dim, h.hidden_dim};
        for (int i = 0; i < 5; ++i) {
            const uint8_t* q = w.next<uint8_t>(size_t(rows[i]) * cols[i]);
            w.next<uint16_t>(size_t(rows[i]) * (cols[i] / h.group_size));
            if (i == 0 && (const void*)q != w.data() + w.tensor(atomflow::WeightKind::Qkv, l).offset) return 3;
        }
    }
    w.next<float>(h.dim);
    w.next<uint16_t>(size_t(h.vocab_size) * h.dim);
    if (w.current_offset() != w.file_size()) return 4;
    bool threw = false;
    try { w.next_block(1); } catch (const std::runtime_error&) { threw = true; }
    if (!threw) return 5;
    AtomHeader L{{'A','T','O','M'}, 1, 128, 3072, 8192, 28, 24, 8, 128256, 131072};
    const size_t D = 3072, F = 8192, V = 128256, GS = 128, NL = 28, QKV = 3072 + 2 * 1024;
    size_t pool = V * D * 4;
    for (size_t i = 0; i < NL; ++i)
        pool += 2 * D * 4 + QKV * D + QKV * (D / GS) * 2 + D * D + D * (D / GS) * 2 +
                2 * (F * D + F * (D / GS) * 2) + D * F + D * (F / GS) * 2;
    pool += D * 4 + V * D * 2;
    if (atomflow::atom_file_bytes(L) != 256 + pool) return 6;
    std::puts("ok");
    return 0;
}
''')
    exe = tmp_path / "t"
    libdir = os.path.dirname(atomflow_amd.LIB_PATH)
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), str(src),
                    "-L", libdir, "-latomflow_kv", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe), str(path)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
