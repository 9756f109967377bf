"""AtomFlow .bin weights on the GPU: the payload uploaded by af_weights_upload is
the file's bytes, and the layer weights used in place by the W8A16 GEMV and the
fused QKV projection give the oracle's results for the arrays that were written."""
import numpy as np
import pytest

import oracle
from atomflow_amd import device as dev
from atomflow_amd import kv
from atomflow_amd import weights as W
from inputs import fp16_ulp, gemv_abs_terms, rng
from test_weights import SMALL, small_model

pytestmark = pytest.mark.gpu

LLAMA_LIKE = dict(dim=3072, hidden_dim=8192, n_layers=2, n_heads=24, n_kv_heads=8,
                  vocab_size=1000, max_seq_len=4096)


def say(msg):
    print(f"[case] {msg}", flush=True)


def test_upload_is_bit_exact(gpu, tmp_path):
    say("weights upload: small model, payload compared byte for byte")
    path = tmp_path / "m.bin"
    W.export_bin(path, SMALL, small_model(60))
    wf = W.WeightFile(path)
    buf = wf.upload()
    raw = np.frombuffer(path.read_bytes(), np.uint8)[256:]
    assert np.array_equal(buf.download(np.uint8), raw)


def test_loaded_weights_drive_qkv_projection(gpu, tmp_path):
    say("weights: Llama-3.2-3B-shaped layers, QKV GEMV and fused QKV + RoPE + append from the upload")
    cfg = LLAMA_LIKE
    r = rng(61)
    D, F, V = cfg["dim"], cfg["hidden_dim"], cfg["vocab_size"]
    QKV = D + 2 * 1024
    t = {"embed": np.zeros((V, D), np.float32), "final_norm": np.ones(D, np.float32),
         "lm_head": np.zeros((V, D), np.float16)}
    for l in range(2):
        t[f"{l}.input_norm"] = np.ones(D, np.float32)
        t[f"{l}.post_norm"] = np.ones(D, np.float32)
        for name, shape in (("qkv", (QKV, D)), ("o_proj", (D, D)), ("gate", (F, D)),
                            ("up", (F, D)), ("down", (D, F))):
            t[f"{l}.{name}"] = (r.standard_normal(shape) * 0.02).astype(np.float32)
    path = tmp_path / "m.bin"
    W.export_bin(path, cfg, t)
    wf = W.WeightFile(path)
    base = wf.upload()
    x = r.standard_normal(D).astype(np.float16)
    d_x = dev.DeviceBuffer.from_array(x)
    for l, (kw, ks, name, n, k) in enumerate([(W.QKV, W.QKV_SCALES, "qkv", QKV, D),
                                              (W.DOWN, W.DOWN_SCALES, "down", D, F)]):
        codes, scales = W.quantize_fp8(t[f"1.{name}"])
        xin = x if k == D else r.standard_normal(k).astype(np.float16)
        d_in = dev.DeviceBuffer.from_array(xin)
        y = dev.DeviceBuffer(n * 2)
        kv.launch_w8a16_gemv(d_in, wf.view(base, kw, 1), wf.view(base, ks, 1), y, n, k)
        got = y.download(np.float16, (n,)).astype(np.float64)
        y64 = oracle.w8a16_gemv_f64(codes, xin, scales)
        bound = k * 2.0 ** -24 * gemv_abs_terms(codes, xin, scales)
        assert np.all(np.abs(got - y64) <= 0.5 * fp16_ulp(y64) + bound), name
    # fused projection + RoPE + append at position 7 from the uploaded layer-0 weights
    max_seq = 64
    c, s = oracle.rope_table(max_seq, 128, 500000.0)
    kc = np.zeros((max_seq, 1024), np.float16)
    vc = np.zeros((max_seq, 1024), np.float16)
    d_kc, d_vc = dev.DeviceBuffer.from_array(kc), dev.DeviceBuffer.from_array(vc)
    d_c, d_s = dev.DeviceBuffer.from_array(c), dev.DeviceBuffer.from_array(s)
    qkv = dev.DeviceBuffer(QKV * 2)
    kv.launch_qkv_rope_append(d_x, wf.view(base, W.QKV, 0), wf.view(base, W.QKV_SCALES, 0), D, qkv,
                              d_kc, d_vc, d_c, d_s, 7, max_seq, 24, 8, 128)
    plain = dev.DeviceBuffer(QKV * 2)
    kv.launch_w8a16_gemv(d_x, wf.view(base, W.QKV, 0), wf.view(base, W.QKV_SCALES, 0), plain, QKV, D)
    y = plain.download(np.float16, (QKV,))
    ref = oracle.rope_append(y, kc, vc, c, s, 7, 24, 8, 128)
    assert np.array_equal(qkv.download(np.uint16), ref.view(np.uint16))
    assert np.array_equal(d_kc.download(np.uint16, kc.shape), kc.view(np.uint16))
    assert np.array_equal(d_vc.download(np.uint16, vc.shape), vc.view(np.uint16))
