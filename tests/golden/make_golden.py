"""Writes the golden fixtures in tests/golden/ from library routines (torch, CPU).

The reference ships no vectors for the KV path (its ground_truth *.bin files are
full-model activations at seq_len 1), so the oracle is pinned against
textbook library routines instead:

* ``fp8_e4m3fn.npz`` — torch.float8_e4m3fn: the decode value of all 256 codes,
  and the encoding of a dense grid over [-448, 448] plus every midpoint
  between adjacent codes (ties) and the clamp convention of
  tools/quantize_weights.py:256-260.
* ``sdpa_cases.npz`` — torch.nn.functional.scaled_dot_product_attention in
  float64 (GQA via repeat_interleave) for seeded decode cases. Inputs are not
  stored: they are regenerated from the seed (tests/inputs.py) and checked
  against the stored sha256.

Run from the repo root:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from inputs import randn_f16  # noqa: E402

# (n_q_heads, n_kv_heads, head_dim, L, seed)
SDPA_CASES = [
    (24, 8, 128, 513, 0xA70F10 + 1),  # BASELINE configs[0] shape and length
    (24, 8, 128, 1, 0xA70F10 + 101),
    (24, 8, 128, 77, 0xA70F10 + 102),
    (8, 8, 128, 300, 0xA70F10 + 103),
    (16, 4, 128, 1000, 0xA70F10 + 104),
    (8, 1, 128, 129, 0xA70F10 + 105),
    (16, 8, 64, 250, 0xA70F10 + 106),
]


def sdpa_inputs(nq, nkv, hd, L, seed):
    q = randn_f16(nq * hd, seed)
    k = randn_f16((L, nkv * hd), seed + 1)
    v = randn_f16((L, nkv * hd), seed + 2)
    return q, k, v


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def sdpa_ref(q, k, v, nq, nkv, hd, L):
    qt = torch.from_numpy(q.astype(np.float64)).view(1, nq, 1, hd)
    kt = torch.from_numpy(k.astype(np.float64)).view(L, nkv, hd).permute(1, 0, 2).unsqueeze(0)
    vt = torch.from_numpy(v.astype(np.float64)).view(L, nkv, hd).permute(1, 0, 2).unsqueeze(0)
    rep = nq // nkv
    kt = kt.repeat_interleave(rep, dim=1).contiguous()
    vt = vt.repeat_interleave(rep, dim=1).contiguous()
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=1.0 / np.sqrt(hd))
    return out.reshape(nq * hd).numpy()


def fp8_fixture():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    decode = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    finite = np.sort(np.unique(decode[np.isfinite(decode)]))
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    grid = np.linspace(-448.0, 448.0, 20001, dtype=np.float32)
    rng = np.random.Generator(np.random.PCG64(7))
    small = (rng.standard_normal(5000) * 0.01).astype(np.float32)
    x = np.concatenate([grid, mids, -mids, finite, small]).astype(np.float32)
    enc = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # reference convention: scale = absmax / 448, q = e4m3fn(clamp(x / scale, +-448))
    t = torch.from_numpy(rng.standard_normal((64, 128)).astype(np.float16).astype(np.float32))
    absmax = t.abs().max()
    scale = absmax / 448.0
    q = (t / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.savez_compressed(os.path.join(HERE, "fp8_e4m3fn.npz"), decode=decode, x=x, encoded=enc,
                        quant_src=t.numpy().astype(np.float16), quant_scale=np.float32(scale),
                        quant_codes=q)


def sdpa_fixture():
    rows = []
    outs = []
    for (nq, nkv, hd, L, seed) in SDPA_CASES:
        q, k, v = sdpa_inputs(nq, nkv, hd, L, seed)
        outs.append(sdpa_ref(q, k, v, nq, nkv, hd, L))
        rows.append((nq, nkv, hd, L, seed, digest(q, k, v)))
    np.savez_compressed(
        os.path.join(HERE, "sdpa_cases.npz"),
        shapes=np.array([r[:5] for r in rows], np.int64),
        digests=np.array([r[5] for r in rows]),
        **{f"out{i}": o for i, o in enumerate(outs)})


if __name__ == "__main__":
    fp8_fixture()
    sdpa_fixture()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
