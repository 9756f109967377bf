"""Benchmark of the KV-cache hot path on one MI355X (BASELINE.json metric).

Default workload = BASELINE configs[1] at ctx 8192: a 28-layer contiguous KV
stack (Llama-3.2-3B attention shape: 24 Q heads, 8 KV heads, head_dim 128,
fp16), batch 1. One step = per layer fused RoPE+append at pos = ctx, then GQA
decode attention over L = ctx + 1 tokens; the 56 launches are captured in one
hipGraph. Inputs are synthetic N(0,1) fp16, generated on the device and
resident in HBM before timing.

Printed JSON line:
  value      whole-step KV-read throughput: 28 * L * 4096 B / step time (GB/s)
  roofline   attention kernel alone: algorithmic KV bytes per launch / its mean
             duration (HIP events around a graph of 28 attention launches, on
             the stream they run on), against 8 TB/s HBM; traffic = HBM bytes
             per launch from the committed rocprofv3 PMC summary, or null
  cpu_baseline  the scalar C++ oracle (oracle/) timed on this host on one full
             28-layer step, 1 thread

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--ctx 8192]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

NQ, NKV, HD, LAYERS = 24, 8, 128, 28
Q_DIM, KV_DIM = NQ * HD, NKV * HD
QKV = Q_DIM + 2 * KV_DIM
THETA = 500000.0
HBM_PEAK_GBS = 8000.0
PMC_SUMMARY = os.path.join(ROOT, "profiles", "decode_attn_c2_ctx8k_pmc.txt")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=8192, choices=[1024, 8192, 32768])
    ap.add_argument("--splits", type=int, default=0, help="attention split count (0 = library default)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain copy kernel of known size (scales PMC byte counters)")
    return ap.parse_args()


def read_traffic(ctx):
    """HBM bytes per attention launch from the committed PMC summary (or None)."""
    if ctx != 8192 or not os.path.exists(PMC_SUMMARY):
        return None
    for line in open(PMC_SUMMARY):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(ctx):
    """One 28-layer decode step (append + attention) on the scalar oracle, 1 thread."""
    import oracle

    L = ctx + 1
    r = np.random.Generator(np.random.PCG64(0xA70F10 + 2))
    k = np.zeros((L, KV_DIM), np.float16)
    v = np.zeros((L, KV_DIM), np.float16)
    k[:ctx] = r.standard_normal((ctx, KV_DIM)).astype(np.float16)
    v[:ctx] = r.standard_normal((ctx, KV_DIM)).astype(np.float16)
    cos, sin = oracle.rope_table(L, HD, THETA)
    qkv = r.standard_normal((LAYERS, QKV)).astype(np.float16)
    t0 = time.perf_counter()
    for l in range(LAYERS):  # same K/V bytes every layer: only the time is used
        rq = oracle.rope_append(qkv[l], k, v, cos, sin, ctx, NQ, NKV, HD)
        oracle.cached_attention(rq[:Q_DIM], k, v, L, NQ, NKV, HD)
    dt = time.perf_counter() - t0
    gbs = LAYERS * L * KV_DIM * 2 * 2 / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"one 28-layer decode step at ctx {ctx} (RoPE+append + attention over "
                      f"{L} tokens per layer) on the scalar C++ oracle, 1 thread, {dt:.1f} s",
            "ms_per_step": round(dt * 1e3, 1)}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the KV path is single-GPU; see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    import atomflow_amd
    from atomflow_amd import device as dev
    from atomflow_amd import kv

    atomflow_amd.lib()
    dev.set_device(0)
    info = dev.device_info()
    ctx = args.ctx
    L = ctx + 1
    max_seq = (L + 127) // 128 * 128
    slab = max_seq * KV_DIM * 2
    log(f"device {info}; ctx {ctx}, cache rows {max_seq}, pool {LAYERS * 2 * slab / 2**30:.2f} GiB")

    stream = dev.Stream()
    pool = dev.DeviceBuffer(LAYERS * 2 * slab)          # [L0_K | L0_V | L1_K | ...]
    qkv = dev.DeviceBuffer(LAYERS * QKV * 2)             # one qkv_out row per layer
    out = dev.DeviceBuffer(LAYERS * Q_DIM * 2)
    d_cos = dev.DeviceBuffer(max_seq * HD // 2 * 4)
    d_sin = dev.DeviceBuffer(max_seq * HD // 2 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA, stream)
    lib = atomflow_amd.lib()
    atomflow_amd.check(lib.af_rt_fill_randn_f16(pool.ptr, LAYERS * 2 * slab // 2, 7, 1.0, stream.handle))
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, LAYERS * QKV, 11, 1.0, stream.handle))
    splits = args.splits or kv.default_splits(L, 1, NKV)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    stream.sync()

    def k_ptr(l):
        return pool.ptr + (2 * l) * slab

    def v_ptr(l):
        return pool.ptr + (2 * l + 1) * slab

    def step():
        for l in range(LAYERS):
            q = qkv.ptr + l * QKV * 2
            kv.launch_rope_append(q, k_ptr(l), v_ptr(l), d_cos, d_sin, ctx, max_seq, NQ, NKV, HD,
                                  stream=stream)
            kv.launch_cached_attention_ex(q, k_ptr(l), v_ptr(l), out.ptr + l * Q_DIM * 2, L,
                                          max_seq, HD, NQ, NKV, ws, num_splits=splits,
                                          stream=stream)

    def attention_only():
        for l in range(LAYERS):
            q = qkv.ptr + l * QKV * 2
            kv.launch_cached_attention_ex(q, k_ptr(l), v_ptr(l), out.ptr + l * Q_DIM * 2, L,
                                          max_seq, HD, NQ, NKV, ws, num_splits=splits,
                                          stream=stream)

    def append_only():
        for l in range(LAYERS):
            q = qkv.ptr + l * QKV * 2
            kv.launch_rope_append(q, k_ptr(l), v_ptr(l), d_cos, d_sin, ctx, max_seq, NQ, NKV, HD,
                                  stream=stream)

    g_step = dev.Graph.capture(stream, step)
    g_attn = dev.Graph.capture(stream, attention_only)
    g_app = dev.Graph.capture(stream, append_only)
    e0, e1 = dev.Event(), dev.Event()

    def timed(graph, reps):
        for _ in range(args.warmup):
            graph.launch(stream)
        dev.synchronize()
        e0.record(stream)
        for _ in range(reps):
            graph.launch(stream)
        e1.record(stream)
        e1.sync()
        dev.synchronize()
        return e0.elapsed_ms(e1) / reps

    log(f"splits {splits}; warmup {args.warmup}, timing {args.steps} graph replays")
    ms_step = timed(g_step, args.steps)
    ms_attn = timed(g_attn, args.steps) / LAYERS
    ms_app = timed(g_app, args.steps) / LAYERS
    log(f"step {ms_step * 1e3:.1f} us, attention {ms_attn * 1e3:.2f} us/launch, "
        f"append {ms_app * 1e3:.2f} us/launch")

    kv_bytes = L * KV_DIM * 2 * 2          # K and V rows attended, each byte once
    step_gbs = LAYERS * kv_bytes / (ms_step * 1e-3) / 1e9
    attn_gbs = kv_bytes / (ms_attn * 1e-3) / 1e9
    traffic = read_traffic(ctx)

    result = {
        "metric": "decode-attn KV-read GB/s (% of 8 TB/s HBM) + us/layer-step at ctx 8k",
        "value": round(step_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "us_per_layer_step": round(ms_step * 1e3 / LAYERS, 3),
        "pct_of_hbm_peak": round(100 * step_gbs / HBM_PEAK_GBS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic N(0,1) fp16 K/V/qkv generated on device",
        "config": {"workload": f"BASELINE configs[1]: 28-layer contiguous KV, batch 1, ctx {ctx}, "
                               "24 Q / 8 KV heads x 128, fp16, hipGraph step = 28 x "
                               "(RoPE+append + GQA attention)",
                   "ctx": ctx, "attended_tokens": L, "layers": LAYERS, "splits": splits,
                   "device": info["name"], "arch": info["arch"], "cus": info["compute_units"]},
        "kernels": {"decode_attn_us": round(ms_attn * 1e3, 3),
                    "rope_append_us": round(ms_app * 1e3, 3),
                    "attn_kv_bytes_per_launch": kv_bytes},
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("cpu baseline (scalar oracle, 1 thread) ...")
        result["cpu_baseline"] = cpu_baseline(ctx)
    print(json.dumps(result), flush=True)
    for g in (g_step, g_attn, g_app):
        g.destroy()
    if args.calibrate_copy:
        calibrate_copy(stream)


def calibrate_copy(stream, mib=256, reps=3):
    """paged_gather over an identity table: reads 2 x `mib` MiB, writes 2 x `mib` MiB."""
    from atomflow_amd import device as dev
    from atomflow_amd import kv

    rows = mib * 2**20 // (KV_DIM * 2)
    src = dev.DeviceBuffer(2 * rows * KV_DIM * 2)
    dst_k = dev.DeviceBuffer(rows * KV_DIM * 2)
    dst_v = dev.DeviceBuffer(rows * KV_DIM * 2)
    src.fill_u32(0x3c003c00, stream)
    pool = kv.make_pool(src, 1, 16, 1, NKV, HD, rows // 16)
    table = dev.DeviceBuffer.from_array(np.arange(rows // 16, dtype=np.int32))
    for _ in range(reps):
        kv.paged_gather(pool, 0, table, rows, dst_k, dst_v, stream)
    stream.sync()
    log(f"copy calibration: {reps} x paged_gather of {2 * rows * KV_DIM * 2} B read + same written")


if __name__ == "__main__":
    main()
