"""AtomFlow .bin weights: writer and loader (C ABI af_weights_*).

The format is the one tools/quantize_weights.py:320-427 writes and the
reference's WeightLoader (include/memory/weight_loader.h:23-130) reads: a
256-byte header ("ATOM", version, group_size, dim, hidden_dim, n_layers, n_heads,
n_kv_heads, vocab_size, max_seq_len as little-endian int32), then every tensor
zero-padded to a multiple of 256 bytes: embed_tokens fp32; per layer the two
RMSNorm weights fp32 and the fused QKV, o_proj, gate, up and down weights as
E4M3 codes followed by fp16 group scales; model.norm fp32; lm_head fp16.

``quantize_fp8`` follows quantize_weights.py:220-268: scale = absmax / 448 per
group of ``group_size`` along K (1 for an all-zero group), computed in fp32;
codes = E4M3FN(round to nearest even of clamp(w / scale, -448, 448)); the scale
is stored as fp16.
"""
import ctypes
import struct

import numpy as np

from . import AfError, check, lib
from .device import DeviceBuffer, _s

FP8_MAX = 448.0
ALIGN = 256

# af_weights_tensor kinds (include/af_kv.h)
EMBED, INPUT_NORM, POST_NORM = 0, 1, 2
QKV, QKV_SCALES, O_PROJ, O_SCALES, GATE, GATE_SCALES = 3, 4, 5, 6, 7, 8
UP, UP_SCALES, DOWN, DOWN_SCALES, FINAL_NORM, LM_HEAD = 9, 10, 11, 12, 13, 14

_E4M3_POS = None


def _e4m3_values():
    """The 127 finite non-negative E4M3FN values, indexed by code 0..126."""
    global _E4M3_POS
    if _E4M3_POS is None:
        v = []
        for c in range(127):
            e, m = c >> 3, c & 7
            v.append(m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10))
        _E4M3_POS = np.array(v, np.float64)
    return _E4M3_POS


def e4m3_codes(x):
    """E4M3FN codes of values already within +-448, rounding to nearest even."""
    vals = _e4m3_values()
    a = np.abs(np.asarray(x, np.float64))
    hi = np.clip(np.searchsorted(vals, a), 1, 126)
    lo = hi - 1
    d_lo, d_hi = a - vals[lo], vals[hi] - a
    up = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(up, hi, lo).astype(np.uint8)
    return code | np.where(np.signbit(x), np.uint8(0x80), np.uint8(0))


def quantize_fp8(w, group_size=128):
    """[N, K] float -> (E4M3 codes uint8 [N, K], fp16 scales [N, K / group_size])."""
    t = np.asarray(w, np.float32)
    n, k = t.shape
    if k % group_size:
        raise ValueError(f"K={k} is not divisible by group_size={group_size}")
    g = t.reshape(n, k // group_size, group_size)
    absmax = np.abs(g).max(axis=2)
    scale = np.where(absmax > 0, absmax / np.float32(FP8_MAX), np.float32(1.0)).astype(np.float32)
    q = np.clip(g / scale[..., None], -FP8_MAX, FP8_MAX).astype(np.float32)
    return e4m3_codes(q).reshape(n, k), scale.astype(np.float16)


def _pad(f):
    r = f.tell() % ALIGN
    if r:
        f.write(b"\0" * (ALIGN - r))


def export_bin(path, cfg, tensors, group_size=128, version=1):
    """Writes an AtomFlow .bin. cfg: dim, hidden_dim, n_layers, n_heads, n_kv_heads,
    vocab_size, max_seq_len. tensors: "embed" [V, D], "final_norm" [D], "lm_head"
    [V, D], and per layer l: f"{l}.input_norm", f"{l}.post_norm" [D] and
    f"{l}.qkv" [D + 2 KV, D], f"{l}.o_proj" [D, D], f"{l}.gate" [F, D], f"{l}.up"
    [F, D], f"{l}.down" [D, F] as float arrays (quantised here) or as
    (codes, scales) pairs (written as given)."""
    with open(path, "wb") as f:
        f.write(header_bytes(cfg, group_size, version))

        def raw(a, dtype):
            f.write(np.ascontiguousarray(a, dtype).tobytes())
            _pad(f)

        def fp8(a):
            codes, scales = a if isinstance(a, tuple) else quantize_fp8(a, group_size)
            raw(codes, np.uint8)
            raw(scales, np.float16)

        raw(tensors["embed"], np.float32)
        for l in range(cfg["n_layers"]):
            raw(tensors[f"{l}.input_norm"], np.float32)
            raw(tensors[f"{l}.post_norm"], np.float32)
            for name in ("qkv", "o_proj", "gate", "up", "down"):
                fp8(tensors[f"{l}.{name}"])
        raw(tensors["final_norm"], np.float32)
        raw(tensors["lm_head"], np.float16)


def layout_bytes(cfg, group_size=128, version=1):
    """Size of a .bin file for this model configuration (header included)."""
    f = np.array([version, group_size, cfg["dim"], cfg["hidden_dim"], cfg["n_layers"],
                  cfg["n_heads"], cfg["n_kv_heads"], cfg["vocab_size"], cfg["max_seq_len"]],
                 np.int32)
    n = int(lib().af_weights_layout_bytes(f.ctypes.data))
    if n == 0:
        raise ValueError(f"inconsistent model configuration {cfg}")
    return n


def header_bytes(cfg, group_size=128, version=1):
    """The 256-byte file header for cfg."""
    h = struct.pack("<4sii", b"ATOM", version, group_size) + struct.pack(
        "<iiiiiii", cfg["dim"], cfg["hidden_dim"], cfg["n_layers"], cfg["n_heads"],
        cfg["n_kv_heads"], cfg["vocab_size"], cfg["max_seq_len"])
    return h + b"\0" * (ALIGN - len(h))


class WeightFile:
    """A mapped .bin file (af_weights_open); ``upload`` copies its payload to the
    device in one streamed block and ``view`` gives a tensor's device address."""

    HEADER_FIELDS = ("version", "group_size", "dim", "hidden_dim", "n_layers", "n_heads",
                     "n_kv_heads", "vocab_size", "max_seq_len")

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().af_weights_open(str(path).encode(), ctypes.byref(h)), f"af_weights_open({path})")
        self.h = h.value
        f = np.zeros(9, np.int32)
        check(lib().af_weights_header(self.h, f.ctypes.data), "af_weights_header")
        self.header = dict(zip(self.HEADER_FIELDS, (int(x) for x in f)))
        self.payload_bytes = int(lib().af_weights_payload_bytes(self.h))

    def close(self):
        if self.h:
            lib().af_weights_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, kind, layer=-1):
        """(payload offset, bytes, (rows, cols)) of one tensor."""
        off, nb = ctypes.c_int64(0), ctypes.c_int64(0)
        dims = np.zeros(2, np.int64)
        check(lib().af_weights_tensor(self.h, kind, layer, ctypes.byref(off), ctypes.byref(nb),
                                      dims.ctypes.data), "af_weights_tensor")
        return off.value, nb.value, (int(dims[0]), int(dims[1]))

    def upload(self, dst=None, stream=None):
        """Copies the payload into `dst` (a DeviceBuffer, allocated when None)."""
        if dst is None:
            dst = DeviceBuffer(self.payload_bytes)
        check(lib().af_weights_upload(self.h, dst.ptr, dst.nbytes, _s(stream)), "af_weights_upload")
        return dst

    def view(self, base, kind, layer=-1):
        """Device address of a tensor in a payload uploaded at `base` (DeviceBuffer or int)."""
        b = base.ptr if isinstance(base, DeviceBuffer) else int(base)
        return b + self.tensor(kind, layer)[0]


__all__ = ["AfError", "WeightFile", "e4m3_codes", "export_bin", "header_bytes", "layout_bytes",
           "quantize_fp8"]
