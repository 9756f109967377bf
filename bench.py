"""Benchmark of the KV-cache hot path on one MI355X (BASELINE.json metric).

Default (``--config 2``) = BASELINE configs[1] at ctx 8192: a 28-layer
contiguous KV stack (Llama-3.2-3B attention shape: 24 Q heads, 8 KV heads,
head_dim 128, fp16), batch 1. One decode step = per layer RoPE+append at
pos = ctx and GQA attention over L = ctx + 1 tokens, as one fused launch per
layer (af_decode_attention_fused); the 28 launches are one hipGraph. Inputs are
synthetic N(0,1) fp16 generated on the device and resident in HBM before timing.

``--config 3|4|5`` run the paged workloads (BASELINE configs[2..4]) through the
BlockManager: paged fp16 (B=32, L~U[128,8192], 16-token blocks), paged with a
2048-token shared prefix (64 forks through the shared-prefix entry points, the
plain paged kernel timed beside them, copy-on-write measured separately), FP8
E4M3 paged (B=128, L~U[8192,16384], 32-token blocks, ~100 GB pool).

Printed JSON line (one per run):
  value      KV-read throughput of the whole step: layers * KV bytes attended /
             step time (GB/s); ms_per_step and us_per_layer_step alongside
  roofline   the attention kernel alone: algorithmic KV bytes per launch / its
             mean duration (HIP events around a graph of 28 attention launches,
             on the stream they run on) against 8 TB/s; traffic = HBM bytes per
             launch from the committed rocprofv3 PMC summary (configs[1] only)
  cpu_baseline  (default config) the scalar C++ oracle timed on this host on one
             28-layer step, 1 thread

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2..5] [--ctx 8192]
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
HIDDEN = 3072                              # model width: the QKV projection's input
THETA = 500000.0
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak
PMC_SUMMARY = os.path.join(ROOT, "profiles", "decode_attn_c2_ctx8k_pmc.txt")
PAGED_PMC_SUMMARY = os.path.join(ROOT, "profiles", "paged_attn_pmc.txt")
PMC_SUMMARY_32K = os.path.join(ROOT, "profiles", "decode_attn_c2_ctx32k_pmc.txt")
METRIC = "decode-attn KV-read GB/s (% of 8 TB/s HBM) + us/layer-step at ctx 8k"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4, 5],
                    help="BASELINE configs[n-1]: 2 contiguous, 3 paged, 4 paged+CoW, 5 paged FP8")
    ap.add_argument("--ctx", type=int, default=8192, choices=[1024, 8192, 32768])
    ap.add_argument("--splits", type=int, default=0, help="attention split count (0 = library default)")
    ap.add_argument("--prefix-splits", type=int, default=0,
                    help="configs[3]: key splits of the shared-prefix launch (0 = library default)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-prefill", action="store_true", help="skip the prefill measurements")
    ap.add_argument("--no-serving", action="store_true", help="skip the continuous-batching step")
    ap.add_argument("--serving-grouped", action="store_true",
                    help="also run the shared-prefix serving step with decode grouped by share "
                         "group (its groups fall below the sharing threshold)")
    ap.add_argument("--weights", action="store_true",
                    help="also time writing and loading a 4.9 GiB Llama-3.2-3B-shaped .bin")
    ap.add_argument("--no-weights", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-matrix", action="store_true",
                    help="skip the per-config matrix (configs[1] ctx 1k/32k, configs[2..4])")
    ap.add_argument("--compare-lib", default=None,
                    help="in-process A/B: time the in-tree library (A) against this build (B) on the "
                         "same buffers and workspaces, graphs replayed alternately; prints one line "
                         "per workload and launch kind")
    ap.add_argument("--compare-work", default="ctx8k,ctx32k,cfg3,cfg4,cfg5",
                    help="workloads of --compare-lib: ctx8k, ctx32k (configs[1]), cfg3 (configs[2]), "
                         "cfg4 (configs[3], plain and shared-prefix), cfg5 (configs[4])")
    ap.add_argument("--compare-rounds", type=int, default=8)
    ap.add_argument("--fanout-only", action="store_true",
                    help="run only the fan-out decode measurement and print its JSON object")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain copy kernel of known size (scales PMC byte counters)")
    ap.add_argument("--stamps", action="store_true",
                    help="run only the per-phase timeline of the configs[1] attention launch "
                         "(with --config 3: of the configs[2] paged launch; needs "
                         "libatomflow_kv_stamps.so: make -C atomflow_amd/csrc stamps) and "
                         "print its JSON object")
    ap.add_argument("--read-probe", action="store_true",
                    help="run only the streaming-read probes (per-launch read ceilings of each "
                         "workload's bytes) and print their JSON object")
    return ap.parse_args()


def read_traffic(path=PMC_SUMMARY, key="traffic_bytes_per_launch:"):
    """HBM bytes per attention launch from a committed PMC summary (or None)."""
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith(key):
            return float(line.split(":", 1)[1])
    return None


def host_cpu():
    """CPU model, logical cores on the host, and the cores this process may run on."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1, len(os.sched_getaffinity(0))


def cpu_threads():
    """Worker threads for the CPU baselines: the cores this process may use, at most 16
    (the GPU box's CPU share per GPU)."""
    return max(1, min(16, len(os.sched_getaffinity(0))))


def cpu_baseline(ctx, runs_threaded=5, runs_single=3):
    """One 28-layer decode step (append + attention) on the scalar C++ oracle: the
    median of `runs_threaded` runs with one thread per query head (up to the cores this
    process may use, at most 16) is the value; the median of `runs_single` one-thread
    runs is reported beside it."""
    import oracle

    L = ctx + 1
    r = np.random.Generator(np.random.PCG64(0xA70F10 + 2))
    k = np.zeros((L, KV_DIM), np.float16)
    v = np.zeros((L, KV_DIM), np.float16)
    k[:ctx] = r.standard_normal((ctx, KV_DIM)).astype(np.float16)
    v[:ctx] = r.standard_normal((ctx, KV_DIM)).astype(np.float16)
    cos, sin = oracle.rope_table(L, HD, THETA)
    qkv = r.standard_normal((LAYERS, QKV)).astype(np.float16)
    threads = min(cpu_threads(), NQ)

    def step(nt):
        t0 = time.perf_counter()
        for l in range(LAYERS):  # same K/V bytes every layer: only the time is used
            rq = oracle.rope_append(qkv[l], k, v, cos, sin, ctx, NQ, NKV, HD)
            oracle.cached_attention(rq[:Q_DIM], k, v, L, NQ, NKV, HD, threads=nt)
        return time.perf_counter() - t0

    tn = [step(threads) for _ in range(runs_threaded)]
    t1 = [step(1) for _ in range(runs_single)]
    dtn, dt1 = float(np.median(tn)), float(np.median(t1))
    gbs = lambda dt: LAYERS * L * KV_DIM * 2 * 2 / dt / 1e9
    model, host_cores, allowed = host_cpu()
    return {"value": round(gbs(dtn), 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"one 28-layer decode step at ctx {ctx} (RoPE+append + attention over "
                      f"{L} tokens per layer) on the C++ oracle; value = median of "
                      f"{runs_threaded} runs with {threads} threads over query heads "
                      f"({dtn:.3f} s); 1 thread: median of {runs_single} runs ({dt1:.2f} s)",
            "ms_per_step": round(dtn * 1e3, 1), "runs": runs_threaded,
            "single_thread_gbs": round(gbs(dt1), 3),
            "single_thread_ms_per_step": round(dt1 * 1e3, 1), "single_thread_runs": runs_single,
            "cpu_model": model, "host_logical_cores": host_cores, "cores_allowed": allowed}


def cpu_baseline_paged(cfg, host, runs=3):
    """The oracle's paged attention (ok_paged_attention_f16 / _fp8) over one layer of
    BASELINE configs[cfg - 1] with the GPU run's block tables and lengths, on host
    data of the same layout: every sequence for configs[2] and [3], 8 sequences
    (the first 8 of the batch) for configs[4]. Sequences run in parallel on
    cpu_threads() threads (ctypes releases the GIL); value = median of `runs` runs,
    one single-thread run beside it."""
    from concurrent.futures import ThreadPoolExecutor

    import oracle

    lens, bs, fp8 = host["lens"], host["bs"], host["fp8"]
    B = len(lens) if cfg != 5 else 8
    r = np.random.Generator(np.random.PCG64(0xA70F10 + 40 + cfg))
    # The blocks the sampled sequences name, renumbered in random order into compact
    # host slabs (shared blocks stay shared): the same rows per sequence and a
    # scattered block order, as on the GPU.
    nblk = [(int(lens[b]) + bs - 1) // bs for b in range(B)]
    used = np.unique(np.concatenate([host["tables"][b, :nblk[b]] for b in range(B)]))
    remap = np.full(int(used.max()) + 1, -1, np.int64)
    remap[used] = r.permutation(len(used))
    tables = [remap[host["tables"][b, :nblk[b]]].astype(np.int32) for b in range(B)]
    rows = len(used) * bs
    # timing only: values are fp16 bit patterns of magnitude in [2^-7, 4) or E4M3 codes
    if fp8:
        kslab = r.integers(0, 0x7F, (rows, KV_DIM), dtype=np.uint8)
        vslab = r.integers(0, 0x7F, (rows, KV_DIM), dtype=np.uint8)
        sc = np.full(NKV, 5.0 / 448.0, np.float32)
    else:
        kslab = r.integers(0x2000, 0x4400, (rows, KV_DIM), dtype=np.uint16).view(np.float16)
        vslab = r.integers(0x2000, 0x4400, (rows, KV_DIM), dtype=np.uint16).view(np.float16)
    q = r.standard_normal((B, Q_DIM), dtype=np.float32).astype(np.float16)

    def one(b):
        if fp8:
            oracle.paged_attention_fp8(q[b], kslab, vslab, sc, sc, tables[b], int(lens[b]), bs,
                                       NQ, NKV, HD)
        else:
            oracle.paged_attention_f16(q[b], kslab, vslab, tables[b], int(lens[b]), bs, NQ, NKV,
                                       HD)

    threads = cpu_threads()

    def layer(nt):
        t0 = time.perf_counter()
        if nt == 1:
            for b in range(B):
                one(b)
        else:
            with ThreadPoolExecutor(nt) as ex:
                list(ex.map(one, range(B)))
        return time.perf_counter() - t0

    tn = [layer(threads) for _ in range(runs)]
    t1 = layer(1)
    dtn = float(np.median(tn))
    esz = 1 if fp8 else 2
    nbytes = int(sum(int(lens[b]) for b in range(B))) * KV_DIM * esz * 2
    model, host_cores, allowed = host_cpu()
    return {"value": round(nbytes / dtn / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"one layer of configs[{cfg - 1}]: paged attention of {B} sequences "
                      f"({nbytes} KV bytes attended) on the C++ oracle, the GPU run's block "
                      f"tables; value = median of {runs} runs on {threads} threads "
                      f"({dtn:.3f} s); 1 thread: one run ({t1:.2f} s)",
            "runs": runs, "single_thread_gbs": round(nbytes / t1 / 1e9, 3),
            "cpu_model": model, "host_logical_cores": host_cores, "cores_allowed": allowed}


class Timer:
    """Times graph replays with one HIP event pair per replay, on the replay stream
    (the reference's own timing takes the median of graph replays, main.cu:125-150).
    graph_ms returns the median; mean_ms holds the mean of the same replays."""

    def __init__(self, dev, stream, warmup):
        self.dev, self.stream, self.warmup = dev, stream, warmup
        self.events = []
        self.mean_ms = None

    def graph_ms(self, graph, reps):
        """Median ms per replay of `graph` over `reps` replays (after the warmup)."""
        for _ in range(self.warmup):
            graph.launch(self.stream)
        self.dev.synchronize()
        while len(self.events) < reps + 1:
            self.events.append(self.dev.Event())
        ev = self.events
        for i in range(reps):
            ev[i].record(self.stream)
            graph.launch(self.stream)
        ev[reps].record(self.stream)
        ev[reps].sync()
        self.dev.synchronize()
        t = [ev[i].elapsed_ms(ev[i + 1]) for i in range(reps)]
        self.mean_ms = float(np.mean(t))
        return float(np.median(t))


def bench_contiguous(args, dev, kv, lib, info, ctx=None, lean=False):
    """configs[1] at one context length. lean: the fused step, the two-launch step
    and the attention kernel only (the matrix entries); otherwise also the QKV
    projection and the prefill / serving / GEMV legs."""
    import atomflow_amd

    ctx = args.ctx if ctx is None else ctx
    L = ctx + 1
    max_seq = (L + 127) // 128 * 128
    slab = max_seq * KV_DIM * 2
    log(f"configs[1]: ctx {ctx}, cache rows {max_seq}, pool {LAYERS * 2 * slab / 2**30:.2f} GiB")
    stream = dev.Stream()
    pool = dev.DeviceBuffer(LAYERS * 2 * slab)          # [L0_K | L0_V | L1_K | ...]
    qkv = dev.DeviceBuffer(LAYERS * QKV * 2)             # one qkv_out row per layer
    out = dev.DeviceBuffer(LAYERS * Q_DIM * 2)
    d_cos = dev.DeviceBuffer(max_seq * HD // 2 * 4)
    d_sin = dev.DeviceBuffer(max_seq * HD // 2 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA, stream)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(pool.ptr, LAYERS * 2 * slab // 2, 7, 1.0, stream.handle))
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, LAYERS * QKV, 11, 1.0, stream.handle))
    splits = args.splits or kv.default_splits(L, 1, NKV)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    # The projection either side of the path: FP8 E4M3 QKV weights [QKV, HIDDEN]
    # with fp16 per-128 group scales and an fp16 activation row, per layer.
    proj_layers = 1 if lean else LAYERS
    w_qkv = dev.DeviceBuffer(proj_layers * QKV * HIDDEN)
    s_qkv = dev.DeviceBuffer(proj_layers * QKV * (HIDDEN // 128) * 2)
    x_act = dev.DeviceBuffer(proj_layers * HIDDEN * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_fp8(w_qkv.ptr, proj_layers * QKV * HIDDEN, 13, 20.0,
                                                stream.handle))
    atomflow_amd.check(lib.af_rt_fill_randn_f16(s_qkv.ptr, proj_layers * QKV * (HIDDEN // 128),
                                                17, 0.002, stream.handle))
    atomflow_amd.check(lib.af_rt_fill_randn_f16(x_act.ptr, proj_layers * HIDDEN, 19, 1.0,
                                                stream.handle))
    stream.sync()

    def ptrs(l):
        return (qkv.ptr + l * QKV * 2, pool.ptr + 2 * l * slab, pool.ptr + (2 * l + 1) * slab,
                out.ptr + l * Q_DIM * 2)

    def step():  # one fused launch per layer: RoPE + append + attention
        for l in range(LAYERS):
            q, k, v, o = ptrs(l)
            kv.launch_decode_attention_fused(q, k, v, d_cos, d_sin, ctx, max_seq, o, NQ, NKV, HD,
                                             ws, num_splits=splits, stream=stream)

    def step_two_launch():  # the reference's order as two launches: append, then attention
        for l in range(LAYERS):
            q, k, v, o = ptrs(l)
            kv.launch_rope_append(q, k, v, d_cos, d_sin, ctx, max_seq, NQ, NKV, HD, stream=stream)
            kv.launch_cached_attention_ex(q, k, v, o, L, max_seq, HD, NQ, NKV, ws,
                                          num_splits=splits, stream=stream)

    def attention_only():
        for l in range(LAYERS):
            q, k, v, o = ptrs(l)
            kv.launch_cached_attention_ex(q, k, v, o, L, max_seq, HD, NQ, NKV, ws,
                                          num_splits=splits, stream=stream)

    def qkv_args(l):
        return (x_act.ptr + l * HIDDEN * 2, w_qkv.ptr + l * QKV * HIDDEN,
                s_qkv.ptr + l * QKV * (HIDDEN // 128) * 2)

    def step_with_projection():  # QKV GEMV + RoPE + append, then attention
        for l in range(LAYERS):
            q, k, v, o = ptrs(l)
            x, w, sc = qkv_args(l)
            kv.launch_qkv_rope_append(x, w, sc, HIDDEN, q, k, v, d_cos, d_sin, ctx, max_seq, NQ, NKV,
                                      HD, stream=stream)
            kv.launch_cached_attention_ex(q, k, v, o, L, max_seq, HD, NQ, NKV, ws,
                                          num_splits=splits, stream=stream)

    def projection_only():
        for l in range(LAYERS):
            q, k, v, _ = ptrs(l)
            x, w, sc = qkv_args(l)
            kv.launch_qkv_rope_append(x, w, sc, HIDDEN, q, k, v, d_cos, d_sin, ctx, max_seq, NQ, NKV,
                                      HD, stream=stream)

    legs = [("step", step), ("two", step_two_launch), ("attn", attention_only)]
    if not lean:
        legs += [("proj_step", step_with_projection), ("proj", projection_only)]
    graphs = {name: dev.Graph.capture(stream, fn) for name, fn in legs}
    t = Timer(dev, stream, args.warmup)
    log(f"splits {splits}; warmup {args.warmup}, timing {args.steps} graph replays (median)")
    ms_step = t.graph_ms(graphs["step"], args.steps)
    ms_step_mean = t.mean_ms
    ms_two = t.graph_ms(graphs["two"], args.steps)
    ms_attn = t.graph_ms(graphs["attn"], args.steps) / LAYERS
    ms_proj_step = ms_proj = None
    if not lean:
        ms_proj_step = t.graph_ms(graphs["proj_step"], args.steps)
        ms_proj = t.graph_ms(graphs["proj"], args.steps) / LAYERS
    log(f"step {ms_step * 1e3:.1f} us (two-launch {ms_two * 1e3:.1f} us), "
        f"attention {ms_attn * 1e3:.2f} us/launch")
    for g in graphs.values():
        g.destroy()
    for b in (pool, qkv, out, d_cos, d_sin, w_qkv, s_qkv, x_act):
        b.free()

    kv_bytes = L * KV_DIM * 2 * 2          # K and V rows attended, each byte once
    proj_bytes = QKV * HIDDEN + QKV * (HIDDEN // 128) * 2 + HIDDEN * 2 + QKV * 2
    step_gbs = LAYERS * kv_bytes / (ms_step * 1e-3) / 1e9
    attn_gbs = kv_bytes / (ms_attn * 1e-3) / 1e9
    pmc = {8192: PMC_SUMMARY, 32768: PMC_SUMMARY_32K}.get(ctx)
    result = {
        "metric": METRIC, "value": round(step_gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "ms_per_step_mean": round(ms_step_mean, 4),
        "us_per_layer_step": round(ms_step * 1e3 / LAYERS, 3),
        "pct_of_hbm_peak": round(100 * step_gbs / HBM_PEAK_GBS, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 KV, fp32 softmax/accumulate",
        "data": "synthetic N(0,1) fp16 K/V/qkv generated on device",
        "config": {"workload": f"BASELINE configs[1]: 28-layer contiguous KV, batch 1, ctx {ctx}, "
                               "24 Q / 8 KV heads x 128, fp16, hipGraph step = 28 fused "
                               "RoPE+append+GQA-attention launches",
                   "ctx": ctx, "attended_tokens": L, "layers": LAYERS, "splits": splits,
                   "device": info["name"], "arch": info["arch"], "cus": info["compute_units"]},
        "kernels": {"decode_attn_us": round(ms_attn * 1e3, 3),
                    "two_launch_us_per_layer_step": round(ms_two * 1e3 / LAYERS, 3),
                    "attn_kv_bytes_per_launch": kv_bytes},
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(pmc) if pmc else None},
        "cpu_baseline": None,
    }
    if lean:
        return result
    result["kernels"].update({
        "qkv_rope_append_us": round(ms_proj * 1e3, 3),
        "qkv_weight_bytes_per_launch": proj_bytes,
        "qkv_rope_append_gbs": round(proj_bytes / (ms_proj * 1e-3) / 1e9, 1),
        "layer_step_with_qkv_projection_us": round(ms_proj_step * 1e3 / LAYERS, 3)})
    if not args.no_prefill:
        log("prefill (one layer) ...")
        result["prefill"] = bench_prefill(dev, kv, lib, stream, 3, 10)
    if not args.no_serving:
        log("serving (scheduler-driven continuous batching) ...")
        result["serving"] = bench_serving(dev, kv, lib)
        log("serving with a shared 1544-token prompt prefix and the prefix cache ...")
        result["serving_shared_prefix"] = bench_serving(dev, kv, lib, shared_prefix=1544)
        if args.serving_grouped:
            # groups of ~5 forks over the 1544-row prefix are below the sharing
            # threshold (kv.SHARE_MIN_SAVED_ROWS), so this leg only runs on request
            log("the same, decode attention grouped by the plan's share groups ...")
            result["serving_shared_prefix_grouped"] = bench_serving(
                dev, kv, lib, shared_prefix=1544, group_decode=True)
        log("fan-out: 64 forks of one cached 4096-token prompt, plain vs grouped decode ...")
        result["serving_fanout"] = bench_fanout(dev, kv, lib)
    log("projection GEMVs ...")
    result["gemv"] = bench_gemv(dev, kv, lib, args.steps, args.warmup)
    if args.weights:
        log("weights (.bin load) ...")
        result["weights"] = bench_weights(dev)
    if args.calibrate_copy:
        calibrate_copy(dev, kv, stream)
    return result


def prefill_flops(p0, n, kv_len):
    """Algorithmic FLOPs of causal chunk attention: 2 (QK) + 2 (PV) per head_dim
    element per attended (query, key) pair, over all Q heads."""
    keys = sum(min(p0 + i + 1, kv_len) for i in range(n))
    return 4.0 * HD * NQ * keys


def bench_prefill(dev, kv, lib, stream, warmup, reps):
    """One layer of prefill: the ctx-8k prompt as one causal chunk, a 2048-token
    chunk at p0 = 6144 (contiguous cache and a bs-16 paged pool with a permuted
    block table), a 512-token chunk at p0 = 6144, and the 2048-row RoPE + append.
    Attention runs through the key-piece entry points with the library's choice
    of pieces (heavy query tiles of a chunk too small to fill the device are
    cut into key ranges); the 512-token chunk is also timed uncut."""
    import atomflow_amd
    e0, e1 = dev.Event(), dev.Event()

    def time_us(fn):
        for _ in range(warmup):
            fn()
        dev.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.sync()
        return e0.elapsed_ms(e1) * 1e3 / reps

    L, LMAX = 8192, 16384
    k = dev.DeviceBuffer(LMAX * KV_DIM * 2)
    v = dev.DeviceBuffer(LMAX * KV_DIM * 2)
    qkv = dev.DeviceBuffer(LMAX * QKV * 2)
    out = dev.DeviceBuffer(LMAX * Q_DIM * 2)
    def randn(b, seed):
        atomflow_amd.check(lib.af_rt_fill_randn_f16(b.ptr, b.nbytes // 2, seed, 1.0, stream.handle))

    for i, b in enumerate((k, v, qkv)):
        randn(b, 0xA70F90 + i)

    wss = {}

    def ws(p0_, n_, kv_len_):  # key-piece workspace of one chunk shape
        key = (p0_, n_, kv_len_)
        if key not in wss:
            wss[key] = kv.PrefillWorkspace(p0_, n_, kv_len_, NQ, 0, stream)
        return wss[key]

    def attn(p0_, n_, kv_len_):
        w = ws(p0_, n_, kv_len_)
        return lambda: kv.launch_prefill_attention_ws(qkv, QKV, k, v, out, Q_DIM, p0_, n_, kv_len_,
                                                      LMAX, NQ, NKV, HD, w, stream=stream)

    def prompt(lp):  # an lp-token prompt as one causal chunk
        return attn(0, lp, lp)
    full = prompt(L)
    p0, n = 6144, 2048
    chunk = attn(p0, n, p0 + n)
    chunk512 = attn(p0, 512, p0 + 512)
    chunk512_plain = lambda: kv.launch_prefill_attention(qkv, QKV, k, v, out, Q_DIM, p0, 512,
                                                         p0 + 512, LMAX, NQ, NKV, HD, stream=stream)
    bs = 16
    nblocks = L // bs
    pool_buf = dev.DeviceBuffer(2 * nblocks * bs * KV_DIM * 2)
    randn(pool_buf, 0xA70F93)
    pool = kv.make_pool(pool_buf, atomflow_amd.AF_KV_FP16, bs, 1, NKV, HD, nblocks)
    table = dev.DeviceBuffer.from_array(
        np.random.default_rng(0xA70F94).permutation(nblocks).astype(np.int32))
    paged = lambda: kv.launch_paged_prefill_attention_ws(qkv, QKV, pool, 0, table, nblocks, p0, n,
                                                         p0 + n, out, Q_DIM, NQ, ws(p0, n, p0 + n),
                                                         stream=stream)
    pool8_buf = dev.DeviceBuffer(2 * nblocks * bs * KV_DIM)
    atomflow_amd.check(lib.af_rt_fill_randn_fp8(pool8_buf.ptr, pool8_buf.nbytes, 0xA70F95, 20.0,
                                                stream.handle))
    scales8 = dev.DeviceBuffer.from_array(np.full(2 * NKV, 0.05, np.float32))
    pool8 = kv.make_pool(pool8_buf, atomflow_amd.AF_KV_FP8_E4M3, bs, 1, NKV, HD, nblocks, scales8)
    paged8 = lambda: kv.launch_paged_prefill_attention_ws(qkv, QKV, pool8, 0, table, nblocks, p0,
                                                          n, p0 + n, out, Q_DIM, NQ,
                                                          ws(p0, n, p0 + n), stream=stream)
    cos = dev.DeviceBuffer(L * (HD // 2) * 4)
    sin = dev.DeviceBuffer(L * (HD // 2) * 4)
    kv.build_rope_cache(cos, sin, L, HD, THETA)
    append = lambda: kv.launch_prefill_rope_append(qkv, n, k, v, cos, sin, p0, L, NQ, NKV, HD,
                                                   stream=stream)
    us_full, us_chunk, us_paged, us_paged8, us_app, us_2k, us_16k, us_512, us_512p = (
        time_us(f) for f in (full, chunk, paged, paged8, append, prompt(2048), prompt(LMAX),
                             chunk512, chunk512_plain))
    tf = lambda fl, us: fl / (us * 1e-6) / 1e12
    f_full, f_chunk = prefill_flops(0, L, L), prefill_flops(p0, n, p0 + n)
    f_2k, f_16k = prefill_flops(0, 2048, 2048), prefill_flops(0, LMAX, LMAX)
    f_512 = prefill_flops(p0, 512, p0 + 512)
    app_bytes = n * (QKV * 2 * 2 + 2 * KV_DIM * 2)  # qkv rows read + written, K/V rows written
    res = {
        "workload": "one layer, 24 Q / 8 KV heads x 128, fp16: 2048-, 8192- and 16384-token "
                    "prompts, each as one causal chunk; 2048-token chunk at p0 6144 (contiguous, paged bs 16 with a "
                    "permuted block table, fp16 and FP8-E4M3 pools); 512-token chunk at p0 6144 "
                    "with and without key pieces; 2048-row RoPE + append",
        "attn_8k_us": round(us_full, 1), "attn_8k_tflops": round(tf(f_full, us_full), 1),
        "attn_2k_us": round(us_2k, 1), "attn_2k_tflops": round(tf(f_2k, us_2k), 1),
        "attn_16k_us": round(us_16k, 1), "attn_16k_tflops": round(tf(f_16k, us_16k), 1),
        "chunk_2k_at_6k_us": round(us_chunk, 1),
        "chunk_2k_at_6k_tflops": round(tf(f_chunk, us_chunk), 1),
        "paged_chunk_2k_at_6k_us": round(us_paged, 1),
        "paged_chunk_2k_at_6k_tflops": round(tf(f_chunk, us_paged), 1),
        "paged_fp8_chunk_2k_at_6k_us": round(us_paged8, 1),
        "paged_fp8_chunk_2k_at_6k_tflops": round(tf(f_chunk, us_paged8), 1),
        "chunk_512_at_6k_us": round(us_512, 1), "chunk_512_at_6k_tflops": round(tf(f_512, us_512), 1),
        "chunk_512_at_6k_uncut_us": round(us_512p, 1),
        "chunk_512_at_6k_uncut_tflops": round(tf(f_512, us_512p), 1),
        "rope_append_2k_us": round(us_app, 2),
        "rope_append_2k_gbs": round(app_bytes / (us_app * 1e-6) / 1e9, 1),
        "roofline": {"bound": "mfma", "achieved": round(tf(f_full, us_full), 1),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf(f_full, us_full) / MFMA_F16_PEAK_TFLOPS, 4)},
    }
    for b in (k, v, qkv, out, pool_buf, pool8_buf, scales8, table, cos, sin):
        b.free()
    for w in wss.values():
        w.buf.free()
    return res


def bench_serving(dev, kv, lib, steps=12, warmup=3, shared_prefix=0, group_decode=False):
    """Continuous batching through the Scheduler (the intended caller of the paged path,
    server_engine.cu:55-68): configs[2]'s
    32 sequences (contexts uniform in [128, 8192]) decoding while a 2048-token prompt
    arrives every step and is prefilled in 512-token chunks under a 2048-token step
    budget. A step = the host plan (af_sched_step) + upload of slots / positions /
    block tables / chunk descriptors / CoW copies + the copies + 28 layers of three
    launches: one paged append for every new row (decode tokens and chunk tokens),
    decode attention for the batch, and one batched prefill attention for all chunks.
    With shared_prefix > 0 every arriving prompt starts with the same shared_prefix
    tokens and the scheduler's prefix cache is on (4 entries). With group_decode the
    decode batch is ordered by the plan's share groups (kv.decode_share_segments) and
    each group that saves at least kv.SHARE_MIN_SAVED_ROWS row reads is attended
    through the shared-prefix entry (its prompt prefix read once per layer), the
    other sequences by one plain launch."""
    import atomflow_amd
    r = np.random.Generator(np.random.PCG64(0xA70F10 + 6))
    bs, chunk, budget, max_running = 16, 512, 2048, 64
    ctx = r.integers(128, 8193, 32)
    n_new, new_prompt, new_gen, old_gen = steps + warmup + 8, 2048, 64, 1000
    total_blocks = (sum(-(-(int(c) + old_gen) // bs) for c in ctx)
                    + n_new * -(-(new_prompt + new_gen) // bs) + 64)
    bm = kv.BlockManager(total_blocks, bs, LAYERS, NKV, HD, atomflow_amd.AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(total_blocks)]
    for b in r.permutation(ids):
        bm.free_block(int(b))
    stream = dev.Stream()
    nbytes = kv.pool_bytes(bm.pool())
    pool_buf = dev.DeviceBuffer(nbytes)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(pool_buf.ptr, nbytes // 2, 7, 1.0, stream.handle))
    bm.attach_pool(pool_buf.ptr)
    pool = bm.pool()
    if shared_prefix:  # requests fork cached prompt prefixes: keep KV rows cached
        pool.flags = atomflow_amd.AF_KV_POOL_SHARED_BLOCKS
    sched = kv.Scheduler(bm, max_running, budget, chunk, 16, 4 if shared_prefix else 0)
    for i, c in enumerate(ctx):
        assert sched.add_request(i, int(c), old_gen)
    while True:  # host-only steps until the 32 contexts are in the cache and decoding
        p = sched.step()
        if not p["prefill"] and len(p["decode"]) == len(ctx):
            break
    max_pos = 16384
    max_blocks = max_pos // bs
    d_cos = dev.DeviceBuffer(max_pos * HD // 2 * 4)
    d_sin = dev.DeviceBuffer(max_pos * HD // 2 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_pos, HD, THETA, stream)
    rows = max_running + budget  # per layer: decode rows, then the chunks' rows
    qkv = dev.DeviceBuffer(LAYERS * rows * QKV * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, qkv.nbytes // 2, 11, 1.0, stream.handle))
    out = dev.DeviceBuffer(rows * Q_DIM * 2)
    ws = kv.AttentionWorkspace(max_running, NQ, NKV, HD, 0, stream)
    dev.synchronize()
    e0, e1 = dev.Event(), dev.Event()
    rec = []
    arrived, ttft = {}, []  # steps from arrival to the first output token
    pf_ws = None  # key-piece workspace of the batched prefill, grown to the largest step
    for k in range(warmup + steps):
        t0 = time.perf_counter()
        if shared_prefix:
            sched.add_request(1000 + k, new_prompt, new_gen, 7, shared_prefix)
        else:
            sched.add_request(1000 + k, new_prompt, new_gen)
        arrived[1000 + k] = k
        p = sched.step()
        t1 = time.perf_counter()
        for c in p["prefill"]:
            if c[4] and c[0] in arrived and arrived[c[0]] >= warmup:
                ttft.append(k - arrived[c[0]] + 1)
        a = p["arrays"]
        nd = len(p["decode"])
        segs = [(0, nd, 0)] if nd else []
        if group_decode and nd:
            order, segs = kv.decode_share_segments(a["decode_share_groups"],
                                                   a["decode_share_rows"])
            for key in ("decode_seqs", "decode_slots", "decode_positions"):
                a[key] = a[key][order]
        # host -> device: slots / positions of every new row, block tables, chunk descriptors
        slots = np.concatenate([a["decode_slots"], a["prefill_slots"]])
        positions = np.concatenate([a["decode_positions"], a["prefill_positions"]])
        bufs = [dev.DeviceBuffer.from_array(slots), dev.DeviceBuffer.from_array(positions)]
        if nd:
            tables, lens = bm.export_tables(a["decode_seqs"], max_blocks)
            bufs += [dev.DeviceBuffer.from_array(tables), dev.DeviceBuffer.from_array(lens)]
        nch = len(p["prefill"])
        if nch:
            ctab, _ = bm.export_tables([c[1] for c in p["prefill"]], max_blocks)
            desc = np.array([(p0, n, p0 + n, nd + int(a["chunks"][i, 3]))
                             for i, (_, _, p0, n, _, _) in enumerate(p["prefill"])], np.int32)
            pmap, groups, most, pf_bytes = kv.prefill_piece_map(desc, NQ)
            if pf_ws is None or pf_ws.nbytes < pf_bytes:
                if pf_ws is not None:
                    pf_ws.buf.free()
                pf_ws = kv.RecordWorkspace(pf_bytes, stream)
                stream.sync()
            cb = [dev.DeviceBuffer.from_array(ctab), dev.DeviceBuffer.from_array(desc),
                  dev.DeviceBuffer.from_array(pmap)]
            bufs += cb
        ncp = len(p["copies"])
        if ncp:
            cpb = [dev.DeviceBuffer.from_array(np.ascontiguousarray(a["copies"], np.int32)),
                   dev.DeviceBuffer.from_array(np.array([ncp], np.int32))]
            bufs += cpb
        n_rows = len(slots)
        e0.record(stream)
        if ncp:  # copy-on-write of shared partial blocks, all layers, before the appends
            kv.kv_copy_blocks(pool, cpb[0], cpb[1], ncp, stream)
        for l in range(LAYERS):
            q = qkv.ptr + l * rows * QKV * 2
            kv.launch_paged_rope_append(q, n_rows, pool, l, bufs[0], bufs[1], d_cos, d_sin,
                                        max_pos, NQ, stream=stream)
            for s0, sn, prefix in segs:
                tab = bufs[2].ptr + s0 * max_blocks * 4
                args = (tab, max_blocks, bufs[3].ptr + s0 * 4, sn, int(lens[s0:s0 + sn].max()),
                        out.ptr + s0 * Q_DIM * 2, Q_DIM, NQ, ws)
                if prefix:
                    kv.launch_paged_attention_shared_prefix(q + s0 * QKV * 2, QKV, pool, l, tab,
                                                            prefix, *args, stream=stream)
                else:
                    kv.launch_paged_attention(q + s0 * QKV * 2, QKV, pool, l, *args,
                                              stream=stream)
            if nch:
                kv.launch_paged_prefill_attention_batched_ws(q, QKV, pool, l, cb[0], max_blocks,
                                                             cb[1], cb[2], len(pmap), groups, most,
                                                             out, Q_DIM, NQ, pf_ws, stream=stream)
        e1.record(stream)
        e1.sync()
        t2 = time.perf_counter()
        for b in bufs:
            b.free()
        if k >= warmup:
            rec.append((nd, sum(c[3] for c in p["prefill"]), nch, (t1 - t0) * 1e6,
                        e0.elapsed_ms(e1), (t2 - t0) * 1e3, len(p["prefix_hits"]), ncp,
                        sum(sn for _, sn, pre in segs if pre)))
    rec = np.array(rec)
    dec, pf, nch, plan_us, gpu_ms, wall_ms, hits, ncopies, grouped = rec.mean(axis=0)
    res = {
        "workload": "configs[2] pool (bs 16, permuted free list), 32 sequences with contexts in "
                    "[128, 8192] decoding + one 2048-token prompt arriving per step, prefill chunk "
                    "512, step budget 2048 tokens, 28 layers x (one paged append for all new rows, "
                    "decode attention for the batch, one batched prefill attention for the "
                    "chunks, heavy query tiles cut into key pieces)" + (f"; every prompt shares its first {shared_prefix} tokens, prefix "
                                 "cache of 4 entries" if shared_prefix else "")
                    + ("; decode batch grouped by share group, each group's prefix attended "
                       "once (shared-prefix entry)" if group_decode else ""),
        "steps": steps, "decode_seqs_per_step": round(float(dec), 1),
        "prefill_tokens_per_step": round(float(pf), 1), "chunks_per_step": round(float(nch), 1),
        "host_plan_us": round(float(plan_us), 1), "gpu_ms_per_step": round(float(gpu_ms), 3),
        "wall_ms_per_step": round(float(wall_ms), 3),
        "tokens_per_s_gpu": round(float((dec + pf) / (gpu_ms * 1e-3)), 0),
        "decode_tokens_per_s_gpu": round(float(dec / (gpu_ms * 1e-3)), 0),
        "steps_to_first_token": round(float(np.mean(ttft)), 2) if ttft else None,
    }
    if shared_prefix:
        res["prefix_hits_per_step"] = round(float(hits), 2)
        res["cow_copies_per_step"] = round(float(ncopies), 2)
    if group_decode:
        res["grouped_decode_seqs_per_step"] = round(float(grouped), 2)
    for b in (pool_buf, d_cos, d_sin, qkv, out):
        b.free()
    if pf_ws is not None:
        pf_ws.buf.free()
    sched.close()
    bm.close()
    return res


def bench_fanout(dev, kv, lib, steps=8, n_req=64, prefix=4096, suffix=16, prefix_splits=0):
    """Decode of n_req requests that share one cached prompt prefix (the prefix cache
    forks it; the fan-out of n samples or of one system prompt, paged_kv_manager.h:61).
    Once all are decoding, steps alternate between the batch's plain decode
    attention and the same batch grouped by the plan's share groups
    (kv.decode_share_segments, the group through af_paged_attention_shared_prefix);
    each step runs 28 layers of one paged append plus the attention. GPU time per
    step of each form, same running set."""
    import atomflow_amd
    bs, max_blocks = 16, 512
    prompt = prefix + suffix
    total_blocks = n_req * (-(-(prompt + 64) // bs)) + 64
    bm = kv.BlockManager(total_blocks, bs, LAYERS, NKV, HD, atomflow_amd.AF_KV_FP16)
    stream = dev.Stream()
    nbytes = kv.pool_bytes(bm.pool())
    pool_buf = dev.DeviceBuffer(nbytes)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(pool_buf.ptr, nbytes // 2, 9, 1.0, stream.handle))
    bm.attach_pool(pool_buf.ptr)
    pool = bm.pool()
    pool.flags = atomflow_amd.AF_KV_POOL_SHARED_BLOCKS  # every request forks the cached prefix
    sched = kv.Scheduler(bm, n_req, 8192, 4096, 0, 1)
    assert sched.add_request(0, prompt, 64, 3, prefix)
    while sched.step()["cache_entries"] == 0:
        pass
    for i in range(1, n_req):
        assert sched.add_request(i, prompt, 64, 3, prefix)
    p = sched.step()
    while len(p["decode"]) < n_req:  # host-only steps: the forks prefill their suffixes
        p = sched.step()
    max_pos = prompt + 64
    d_cos = dev.DeviceBuffer(max_pos * HD // 2 * 4)
    d_sin = dev.DeviceBuffer(max_pos * HD // 2 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_pos, HD, THETA, stream)
    qkv = dev.DeviceBuffer(LAYERS * n_req * QKV * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, qkv.nbytes // 2, 13, 1.0, stream.handle))
    out = dev.DeviceBuffer(n_req * Q_DIM * 2)
    ws = kv.AttentionWorkspace(n_req, NQ, NKV, HD, 0, stream)
    dev.synchronize()
    e0, e1 = dev.Event(), dev.Event()
    times = {False: [], True: []}
    for k in range(2 * steps + 2):
        grouped = bool(k % 2)
        a = p["arrays"]
        nd = len(p["decode"])
        segs = [(0, nd, 0)]
        if grouped:
            order, segs = kv.decode_share_segments(a["decode_share_groups"],
                                                   a["decode_share_rows"])
            for key in ("decode_seqs", "decode_slots", "decode_positions"):
                a[key] = a[key][order]
        tables, lens = bm.export_tables(a["decode_seqs"], max_blocks)
        bufs = [dev.DeviceBuffer.from_array(x) for x in
                (a["decode_slots"], a["decode_positions"], tables, lens)]
        e0.record(stream)
        for l in range(LAYERS):
            q = qkv.ptr + l * n_req * QKV * 2
            kv.launch_paged_rope_append(q, nd, pool, l, bufs[0], bufs[1], d_cos, d_sin, max_pos,
                                        NQ, stream=stream)
            for s0, sn, pre in segs:
                tab = bufs[2].ptr + s0 * max_blocks * 4
                args = (tab, max_blocks, bufs[3].ptr + s0 * 4, sn, int(lens[s0:s0 + sn].max()),
                        out.ptr + s0 * Q_DIM * 2, Q_DIM, NQ, ws)
                if pre:
                    kv.launch_paged_attention_shared_prefix(q + s0 * QKV * 2, QKV, pool, l, tab,
                                                            pre, *args, stream=stream,
                                                            prefix_splits=prefix_splits)
                else:
                    kv.launch_paged_attention(q + s0 * QKV * 2, QKV, pool, l, *args,
                                              stream=stream)
        e1.record(stream)
        e1.sync()
        if k >= 2:
            times[grouped].append(e0.elapsed_ms(e1))
        for b in bufs:
            b.free()
        p = sched.step()
        assert len(p["decode"]) == n_req
    plain, grp = float(np.mean(times[False])), float(np.mean(times[True]))
    for b in (pool_buf, d_cos, d_sin, qkv, out):
        b.free()
    sched.close()
    bm.close()
    return {
        "workload": f"{n_req} requests forking one cached {prefix}-token prompt prefix "
                    f"({suffix} own prompt tokens each), decoding; fp16 pool bs 16; a step = "
                    "28 layers x (paged append of the batch's new rows + decode attention), "
                    "plain and grouped steps alternating over the same running set",
        "steps_each": steps, "plain_ms_per_step": round(plain, 3),
        "grouped_ms_per_step": round(grp, 3), "speedup": round(plain / grp, 3),
        "decode_tokens_per_s_plain": round(n_req / (plain * 1e-3), 0),
        "decode_tokens_per_s_grouped": round(n_req / (grp * 1e-3), 0),
    }


def bench_gemv(dev, kv, lib, steps, warmup):
    """The W8A16 projections either side of the path at the engine's shapes
    (engine.cu:315-459), each timed as a graph of 28 launches over 28 layers'
    weights: o_proj 3072 x 3072, gate and up 8192 x 3072 (two launches, and the
    pair in one af_w8a16_gemv_pair launch), down 3072 x 8192. Algorithmic bytes
    = E4M3 weights + fp16 group scales + activation in + output out."""
    import atomflow_amd
    FFN = 8192
    stream = dev.Stream()
    shapes = {"o_proj": (HIDDEN, HIDDEN), "gate": (FFN, HIDDEN), "up": (FFN, HIDDEN),
              "down": (HIDDEN, FFN)}
    bufs = {}
    for i, (name, (n, k)) in enumerate(shapes.items()):
        w = dev.DeviceBuffer(LAYERS * n * k)
        sc = dev.DeviceBuffer(LAYERS * n * (k // 128) * 2)
        atomflow_amd.check(lib.af_rt_fill_randn_fp8(w.ptr, w.nbytes, 0xA70FA0 + i, 20.0,
                                                    stream.handle))
        atomflow_amd.check(lib.af_rt_fill_randn_f16(sc.ptr, sc.nbytes // 2, 0xA70FB0 + i, 0.002,
                                                    stream.handle))
        bufs[name] = (w, sc)
    x = dev.DeviceBuffer(LAYERS * FFN * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(x.ptr, x.nbytes // 2, 0xA70FC0, 1.0, stream.handle))
    y = dev.DeviceBuffer(LAYERS * 2 * FFN * 2)
    stream.sync()

    def args(name, l):
        n, k = shapes[name]
        w, sc = bufs[name]
        return (w.ptr + l * n * k, sc.ptr + l * n * (k // 128) * 2, n, k)

    def single(name):
        def run():
            for l in range(LAYERS):
                w, sc, n, k = args(name, l)
                kv.launch_w8a16_gemv(x.ptr + l * FFN * 2, w, sc, y.ptr + l * 2 * FFN * 2, n, k,
                                     stream=stream)
        return run

    def gate_up_two():
        single("gate")()
        single("up")()

    def gate_up_pair():
        for l in range(LAYERS):
            wg, sg, n, k = args("gate", l)
            wu, su, _, _ = args("up", l)
            yl = y.ptr + l * 2 * FFN * 2
            kv.launch_w8a16_gemv_pair(x.ptr + l * FFN * 2, wg, sg, yl, n, wu, su, yl + FFN * 2, n,
                                      k, stream=stream)

    # batched QKV projection (one token per sequence of a serving step), weights 5120 x 3072
    wq = dev.DeviceBuffer(LAYERS * QKV * HIDDEN)
    sq = dev.DeviceBuffer(LAYERS * QKV * (HIDDEN // 128) * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_fp8(wq.ptr, wq.nbytes, 0xA70FD0, 20.0, stream.handle))
    atomflow_amd.check(lib.af_rt_fill_randn_f16(sq.ptr, sq.nbytes // 2, 0xA70FD1, 0.002,
                                                stream.handle))
    xb = dev.DeviceBuffer(LAYERS * 32 * HIDDEN * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(xb.ptr, xb.nbytes // 2, 0xA70FD2, 1.0,
                                                stream.handle))
    yb = dev.DeviceBuffer(LAYERS * 32 * QKV * 2)
    stream.sync()

    def batched(m):
        def run():
            for l in range(LAYERS):
                kv.launch_w8a16_gemm_batched(xb.ptr + l * 32 * HIDDEN * 2, HIDDEN, m,
                                             wq.ptr + l * QKV * HIDDEN,
                                             sq.ptr + l * QKV * (HIDDEN // 128) * 2,
                                             yb.ptr + l * 32 * QKV * 2, QKV, QKV, HIDDEN,
                                             stream=stream)
        return run

    def per_token(m):  # the same projection as m single-token GEMVs
        def run():
            for l in range(LAYERS):
                for i in range(m):
                    kv.launch_w8a16_gemv(xb.ptr + (l * 32 + i) * HIDDEN * 2,
                                         wq.ptr + l * QKV * HIDDEN,
                                         sq.ptr + l * QKV * (HIDDEN // 128) * 2,
                                         yb.ptr + (l * 32 + i) * QKV * 2, QKV, HIDDEN,
                                         stream=stream)
        return run

    shapes["qkv"] = (QKV, HIDDEN)
    fns = {"o_proj": single("o_proj"), "gate": single("gate"), "down": single("down"),
           "gate_up_two_launches": gate_up_two, "gate_up_pair": gate_up_pair,
           "qkv_batched_m1": batched(1), "qkv_batched_m8": batched(8),
           "qkv_batched_m32": batched(32), "qkv_per_token_gemv_m8": per_token(8)}
    t = Timer(dev, stream, warmup)
    res = {"workload": "W8A16 GEMV, E4M3 weights with fp16 scales per 128-group, fp16 in/out, "
                       "28 layers' weights per graph (each launch reads its own layer's)"}
    for name, fn in fns.items():
        g = dev.Graph.capture(stream, fn)
        us = t.graph_ms(g, steps) * 1e3 / LAYERS
        g.destroy()
        mats = {"gate_up_two_launches": ["gate", "up"], "gate_up_pair": ["gate", "up"]}.get(
            name, ["qkv"] if name.startswith("qkv") else [name])
        tokens = int(name.rsplit("_m", 1)[1]) if name.startswith("qkv") else 1
        nbytes = sum(shapes[m][0] * shapes[m][1] * (1 + 2 / 128)
                     + tokens * (shapes[m][1] + shapes[m][0]) * 2 for m in mats)
        res[f"{name}_us"] = round(us, 3)
        res[f"{name}_gbs"] = round(nbytes / (us * 1e-6) / 1e9, 1)
    res["qkv_note"] = ("qkv_*: the 5120 x 3072 QKV projection of m tokens; batched = one "
                       "af_w8a16_gemm_batched launch (weights read once), per_token = m "
                       "af_w8a16_gemv launches; GB/s counts the weights once")
    for w, sc in bufs.values():
        w.free()
        sc.free()
    for b in (x, y, wq, sq, xb, yb):
        b.free()
    return res


def bench_weights(dev, path_dir="/tmp"):
    """Loading the reference's .bin format (weight_loader.h:23-130): a
    Llama-3.2-3B-shaped file (header of the real model, random contents) is
    uploaded by af_weights_upload (one streamed block through pinned double
    buffers) and, for comparison, the way the reference engine does it
    (engine.cu:97-148): one pageable copy per tensor from the mapped file."""
    from atomflow_amd import weights as W
    cfg = dict(dim=3072, hidden_dim=8192, n_layers=28, n_heads=24, n_kv_heads=8,
               vocab_size=128256, max_seq_len=131072)
    total = W.layout_bytes(cfg)
    path = os.path.join(path_dir, f"af_bench_{os.getpid()}.bin")
    block = np.random.default_rng(0xA70F96).integers(0, 256, 64 << 20, dtype=np.uint8).tobytes()
    try:
        with open(path, "wb") as f:
            f.write(W.header_bytes(cfg))
            left = total - 256
            while left > 0:
                n = min(left, len(block))
                f.write(block[:n])
                left -= n
        wf = W.WeightFile(path)
        dst = dev.DeviceBuffer(wf.payload_bytes)
        wf.upload(dst)  # warm the page cache and the pinned-allocation path
        reps = 3
        t0 = time.perf_counter()
        for _ in range(reps):
            wf.upload(dst)
        t_stream = (time.perf_counter() - t0) / reps
        mm = np.memmap(path, np.uint8, "r")
        kinds = [(W.EMBED, -1)] + [(k, l) for l in range(cfg["n_layers"])
                                   for k in range(W.INPUT_NORM, W.DOWN_SCALES + 1)]
        kinds += [(W.FINAL_NORM, -1), (W.LM_HEAD, -1)]
        specs = [wf.tensor(k, l) for k, l in kinds]
        t0 = time.perf_counter()
        for off, nb, _ in specs:
            dst.upload(mm[256 + off:256 + off + nb], offset=off)
        dev.synchronize()
        t_ref = time.perf_counter() - t0
        del mm
        gb = wf.payload_bytes / 1e9
        res = {"workload": "Llama-3.2-3B-shaped .bin (dim 3072, ffn 8192, 28 layers, vocab 128256): "
                           f"{wf.payload_bytes / 2**30:.2f} GiB payload, file in the page cache",
               "tensors": len(specs),
               "upload_s": round(t_stream, 3), "upload_gbs": round(gb / t_stream, 1),
               "per_tensor_pageable_s": round(t_ref, 3),
               "per_tensor_pageable_gbs": round(gb / t_ref, 1)}
        dst.free()
        wf.close()
        return res
    finally:
        if os.path.exists(path):
            os.remove(path)


def bench_paged(args, dev, kv, lib, info, cfg=None, cpu=False):
    """BASELINE configs[cfg - 1] (cfg 3, 4, 5) through the BlockManager. cpu: also the
    oracle's time on a bounded sample of the same layer (cpu_baseline_paged)."""
    import atomflow_amd
    from atomflow_amd import AF_KV_FP16, AF_KV_FP8_E4M3

    cfg = args.config if cfg is None else cfg
    r = np.random.Generator(np.random.PCG64(0xA70F10 + cfg))
    if cfg == 3:
        bs, fp8 = 16, False
        ctx_lens = r.integers(128, 8193, 32)
    elif cfg == 4:
        bs, fp8 = 16, False
        suffix = r.integers(1, 1025, 64)
    else:
        bs, fp8 = 32, True
        ctx_lens = r.integers(8192, 16385, 128)
    esz = 1 if fp8 else 2
    if cfg == 4:
        prefix = 2048
        B = len(suffix)
        lens_after = prefix + suffix + 1
        unique_tokens = prefix + int(suffix.sum()) + B
        need = prefix // bs + sum((int(s) + 1 + bs - 1) // bs for s in suffix)
    else:
        B = len(ctx_lens)
        lens_after = ctx_lens + 1
        unique_tokens = int(lens_after.sum())
        need = sum((int(n) + bs - 1) // bs for n in lens_after)
    total_blocks = int(need * 1.1) + 8        # 10% free-list headroom
    bm = kv.BlockManager(total_blocks, bs, LAYERS, NKV, HD, AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(total_blocks)]
    for b in r.permutation(ids):               # blocks come back in random order
        bm.free_block(int(b))
    if cfg == 4:
        root = bm.seq_create()
        bm.seq_extend(root, prefix)
        seqs = [root] + [bm.seq_fork(root) for _ in range(B - 1)]
        for s, n in zip(seqs, suffix):
            assert not isinstance(bm.seq_extend(s, int(n)), int)
    else:
        seqs = []
        for n in ctx_lens:
            s = bm.seq_create()
            assert not isinstance(bm.seq_extend(s, int(n)), int)
            seqs.append(s)
    plan = bm.plan_decode(seqs)
    assert not isinstance(plan, int), plan
    slots, positions, copies = plan
    max_len = int(lens_after.max())
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    assert np.array_equal(lens, lens_after)
    desc = bm.pool()
    nbytes = kv.pool_bytes(desc)
    log(f"configs[{cfg - 1}]: B {B}, block {bs}, {total_blocks} blocks, pool {nbytes / 2**30:.1f} GiB, "
        f"max len {max_len}, fp8 {fp8}")
    stream = dev.Stream()
    pool = dev.DeviceBuffer(nbytes)
    scales = None
    if fp8:  # N(0,1) values, absmax-style scale fixed at 5 sigma / 448
        scale = 5.0 / 448.0
        scales = dev.DeviceBuffer.from_array(np.full((LAYERS, 2, NKV), scale, np.float32))
        atomflow_amd.check(lib.af_rt_fill_randn_fp8(pool.ptr, nbytes, 7, 1.0 / scale, stream.handle))
    else:
        atomflow_amd.check(lib.af_rt_fill_randn_f16(pool.ptr, nbytes // 2, 7, 1.0, stream.handle))
    bm.attach_pool(pool.ptr, scales.ptr if scales else None)
    desc = bm.pool()
    if cfg == 4:  # the forks map the prefix blocks: keep KV rows cached
        desc.flags = atomflow_amd.AF_KV_POOL_SHARED_BLOCKS
    max_pos = max_len + 1
    d_cos = dev.DeviceBuffer(max_pos * HD // 2 * 4)
    d_sin = dev.DeviceBuffer(max_pos * HD // 2 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_pos, HD, THETA, stream)
    qkv = dev.DeviceBuffer(LAYERS * B * QKV * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, LAYERS * B * QKV, 11, 1.0, stream.handle))
    out = dev.DeviceBuffer(LAYERS * B * Q_DIM * 2)
    d_tables, d_lens = dev.DeviceBuffer.from_array(tables), dev.DeviceBuffer.from_array(lens)
    d_slots, d_pos = dev.DeviceBuffer.from_array(slots), dev.DeviceBuffer.from_array(positions)
    # 0 = the library's default partition (for batches: ~512 tokens per split,
    # so each sequence's split count follows its length)
    launch_splits = args.splits
    splits = args.splits or max(kv.default_splits(max_len, B, NKV), 1)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, splits, stream)
    stream.sync()

    def step():
        for l in range(LAYERS):
            kv.launch_paged_decode_fused(qkv.ptr + l * B * QKV * 2, B, desc, l, d_slots, d_pos,
                                         d_cos, d_sin, max_pos, d_tables, max_blocks, max_len,
                                         out.ptr + l * B * Q_DIM * 2, Q_DIM, NQ, ws,
                                         num_splits=launch_splits, stream=stream)

    def attention_only():
        for l in range(LAYERS):
            kv.launch_paged_attention(qkv.ptr + l * B * QKV * 2, QKV, desc, l, d_tables,
                                      max_blocks, d_lens, B, max_len,
                                      out.ptr + l * B * Q_DIM * 2, Q_DIM, NQ, ws,
                                      num_splits=launch_splits, stream=stream)

    graphs = {"step": dev.Graph.capture(stream, step), "attn": dev.Graph.capture(stream, attention_only)}
    if cfg == 4:
        # Shared-prefix form: rows [0, 2048) of every fork are the root's, attended
        # once for the batch (matrix-core launch), the suffixes per sequence.
        d_root = dev.DeviceBuffer.from_array(np.ascontiguousarray(tables[0]))
        ws_sp = kv.AttentionWorkspace(B, NQ, NKV, HD, 0, stream)
        stream.sync()

        def step_sp():
            for l in range(LAYERS):
                kv.launch_paged_decode_fused_shared_prefix(
                    qkv.ptr + l * B * QKV * 2, B, desc, l, d_slots, d_pos, d_cos, d_sin, max_pos,
                    d_root, prefix, d_tables, max_blocks, max_len, out.ptr + l * B * Q_DIM * 2,
                    Q_DIM, NQ, ws_sp, num_splits=launch_splits, prefix_splits=args.prefix_splits,
                    stream=stream)

        def attention_sp():
            for l in range(LAYERS):
                kv.launch_paged_attention_shared_prefix(
                    qkv.ptr + l * B * QKV * 2, QKV, desc, l, d_root, prefix, d_tables, max_blocks,
                    d_lens, B, max_len, out.ptr + l * B * Q_DIM * 2, Q_DIM, NQ, ws_sp,
                    num_splits=launch_splits, prefix_splits=args.prefix_splits, stream=stream)

        graphs["step_sp"] = dev.Graph.capture(stream, step_sp)
        graphs["attn_sp"] = dev.Graph.capture(stream, attention_sp)
    t = Timer(dev, stream, args.warmup)
    ms_step = t.graph_ms(graphs["step"], args.steps)
    ms_step_mean = t.mean_ms
    ms_attn = t.graph_ms(graphs["attn"], args.steps) / LAYERS
    ms_step_plain = ms_attn_plain = None
    if cfg == 4:
        ms_step_plain, ms_attn_plain = ms_step, ms_attn
        ms_step = t.graph_ms(graphs["step_sp"], args.steps)
        ms_step_mean = t.mean_ms
        ms_attn = t.graph_ms(graphs["attn_sp"], args.steps) / LAYERS
    for g in graphs.values():
        g.destroy()
    row = KV_DIM * esz
    logical = int(lens_after.sum()) * row * 2
    step_gbs = LAYERS * logical / (ms_step * 1e-3) / 1e9
    # Roofline bytes: every KV row the step must read once. With a shared prefix
    # (configs[3]) that is the unique rows: the prefix once, then each suffix.
    algo_bytes = unique_tokens * row * 2 if cfg == 4 else logical
    attn_gbs = algo_bytes / (ms_attn * 1e-3) / 1e9
    result = {
        "metric": METRIC + f" [paged configs[{cfg - 1}]]", "value": round(step_gbs, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4), "ms_per_step_mean": round(ms_step_mean, 4),
        "us_per_layer_step": round(ms_step * 1e3 / LAYERS, 3),
        "pct_of_hbm_peak": round(100 * step_gbs / HBM_PEAK_GBS, 1), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": ("fp8 e4m3" if fp8 else "f16") + " KV, fp32 softmax/accumulate",
        "data": "synthetic N(0,1) KV generated on device; block tables from the BlockManager "
                "over a randomly permuted free list",
        "config": {"workload": f"BASELINE configs[{cfg - 1}]", "batch": B, "block_size": bs,
                   "total_blocks": total_blocks, "pool_gib": round(nbytes / 2**30, 2),
                   "max_len": max_len, "mean_len": float(lens_after.mean()), "splits": splits,
                   "logical_kv_bytes_per_layer": logical,
                   "unique_kv_bytes_per_layer": unique_tokens * row * 2, "layers": LAYERS},
        "kernels": {"paged_attn_us": round(ms_attn * 1e3, 3)},
        "roofline_bytes": "unique KV rows (shared prefix once)" if cfg == 4 else "KV rows attended",
        # traffic: measured HBM bytes per attention call (FETCH_SIZE + WRITE_SIZE passes, scaled
        # by a copy kernel) from the committed PMC summary of this config
        "roofline": {"bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(PAGED_PMC_SUMMARY,
                                             f"traffic_bytes_per_launch configs[{cfg - 1}]:")},
        "cpu_baseline": None,
    }
    if cfg == 4:
        result["path"] = ("af_paged_decode_fused_shared_prefix (step) / "
                          "af_paged_attention_shared_prefix (attention)")
        result["kernels"].update({
            "plain_paged_attn_us": round(ms_attn_plain * 1e3, 3),
            "plain_us_per_layer_step": round(ms_step_plain * 1e3 / LAYERS, 3),
            "plain_step_gbs_logical": round(LAYERS * logical / (ms_step_plain * 1e-3) / 1e9, 1)})
        result["kernels"].update(cow_copy_timing(dev, kv, bm, prefix, B, stream, desc))
        # The same algorithmic bytes as the shared-prefix path (the answer needs
        # every unique row once); the plain kernel re-reads the prefix per fork,
        # mostly from L2/MALL, which logical_gbs shows.
        plain_gbs = algo_bytes / (ms_attn_plain * 1e-3) / 1e9
        result["plain"] = {
            "us_per_layer_step": round(ms_step_plain * 1e3 / LAYERS, 3),
            "attn_us": round(ms_attn_plain * 1e3, 3),
            "logical_gbs": round(logical / (ms_attn_plain * 1e-3) / 1e9, 1),
            "roofline": {"bound": "hbm", "achieved": round(plain_gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(plain_gbs / HBM_PEAK_GBS, 4),
                         "bytes": "unique KV rows (shared prefix once)",
                         "traffic": read_traffic(PAGED_PMC_SUMMARY,
                                                 "traffic_bytes_per_launch configs[3] plain:")}}
    if args.calibrate_copy:
        calibrate_copy(dev, kv, stream)
    if cpu:
        host = {"tables": tables, "lens": lens_after, "bs": bs, "fp8": fp8,
                "total_blocks": total_blocks, "unique_rows": unique_tokens}
    bm.close()
    pool.free()
    for b in (qkv, out, d_tables, d_lens, d_slots, d_pos, d_cos, d_sin):
        b.free()
    if cpu:
        log(f"configs[{cfg - 1}] cpu baseline (oracle on a sample of one layer) ...")
        result["cpu_baseline"] = cpu_baseline_paged(cfg, host)
    return result


def cow_copy_timing(dev, kv, bm, prefix, B, stream, desc):
    """configs[3] with a shared partial tail: fork -> first append triggers B-1 copies."""
    root = bm.seq_create()
    if isinstance(bm.seq_extend(root, prefix + 8), int):
        return {"cow": "skipped: pool full"}
    forks = [bm.seq_fork(root) for _ in range(B - 1)]
    plan = bm.plan_decode([root] + forks, max_copies=B)
    if isinstance(plan, int):
        return {"cow": f"skipped: status {plan}"}
    copies = plan[2]
    d_copies = dev.DeviceBuffer.from_array(np.ascontiguousarray(copies, np.int32))
    d_count = dev.DeviceBuffer.from_array(np.array([len(copies)], np.int32))
    g = dev.Graph.capture(stream, lambda: kv.kv_copy_blocks(desc, d_copies, d_count, B, stream))
    ms = Timer(dev, stream, 3).graph_ms(g, 20)
    g.destroy()
    return {"cow_copies": len(copies), "cow_rows_per_copy": int(copies[0][2]) if len(copies) else 0,
            "cow_copy_us_all_layers": round(ms * 1e3, 3)}


def calibrate_copy(dev, kv, stream, mib=256, reps=3):
    """paged_gather over an identity table: reads 2 x `mib` MiB, writes 2 x `mib` MiB."""
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


def matrix_entry(res, name, attn_key="paged_attn_us"):
    """The per-workload summary kept in the default run's `matrix` object."""
    k = res["kernels"]
    return {"workload": name, "us_per_layer_step": res["us_per_layer_step"],
            "attn_us_per_launch": k.get(attn_key),
            "attn_gbs": res["roofline"]["achieved"], "roofline": res["roofline"],
            "ms_per_step": res["ms_per_step"], "config": res["config"],
            "cpu_baseline": res.get("cpu_baseline")}


def bench_matrix(args, dev, kv, lib, info, headline):
    """Every BASELINE config point on the GPU, in the default run: configs[1] at ctx
    1024 / 8192 / 32768, configs[2] (paged fp16), configs[3] (64 forks of a shared
    prefix: the shared-prefix path and the plain paged kernel), configs[4] (paged
    FP8, ~93 GiB pool). Paged entries carry an oracle CPU baseline on a sample."""
    cpu = not args.no_cpu
    m = {"configs[1] ctx 8192": matrix_entry(headline, "configs[1] ctx 8192", "decode_attn_us")}
    m["configs[1] ctx 8192"]["cpu_baseline"] = headline.get("cpu_baseline")
    for ctx in (1024, 32768):
        log(f"matrix: configs[1] ctx {ctx} ...")
        r = bench_contiguous(args, dev, kv, lib, info, ctx=ctx, lean=True)
        m[f"configs[1] ctx {ctx}"] = matrix_entry(r, f"configs[1] ctx {ctx}", "decode_attn_us")
    for cfg in (3, 4, 5):
        log(f"matrix: configs[{cfg - 1}] ...")
        r = bench_paged(args, dev, kv, lib, info, cfg=cfg, cpu=cpu)
        if cfg == 4:
            m["configs[3] shared-prefix path"] = matrix_entry(r, "configs[3] shared-prefix path "
                                                             "(af_paged_attention_shared_prefix)")
            p = r["plain"]
            m["configs[3] plain paged kernel"] = {
                "workload": "configs[3] through af_paged_attention (each fork reads the prefix)",
                "us_per_layer_step": p["us_per_layer_step"], "attn_us_per_launch": p["attn_us"],
                "attn_gbs": p["roofline"]["achieved"], "logical_gbs": p["logical_gbs"],
                "roofline": p["roofline"],
                "cpu_baseline": r.get("cpu_baseline")}
        else:
            name = {3: "configs[2] paged fp16", 5: "configs[4] paged fp8"}[cfg]
            m[name] = matrix_entry(r, name)
    return m


# (name, bytes per launch, layers rotated, head-row bytes, segment bytes): the
# attention kernel's bytes per launch for each BASELINE workload, rotated over
# enough layers that the 256 MB MALL does not serve re-reads.
READ_PROBE_WORKLOADS = [
    ("configs[1] ctx 8192", 8193 * 2 * 2048, 28, 2048, 256),
    ("configs[1] ctx 32768", 32769 * 2 * 2048, 12, 2048, 256),
    ("configs[2] (549 MB)", 134104 * 2 * 2048, 4, 2048, 256),
    ("configs[4] (3.25 GB, FP8 rows)", 1585518 * 2 * 1024, 2, 1024, 128),
    # the same rows read as 256-B pieces: two KV heads per workgroup (the FP8 pair form)
    ("configs[4] (3.25 GB, FP8 rows, KV-head pairs)", 1585518 * 2 * 1024, 2, 1024, 256),
    # the E4M3 weights of the projections either side of the path (K = 3072 rows of 3 KB)
    # (contiguous reads only: segment 0)
    ("QKV weights 5120 x 3072 (15.7 MB)", QKV * HIDDEN, 28, HIDDEN, 0),
    ("o_proj weights 3072 x 3072 (9.4 MB)", HIDDEN * HIDDEN, 28, HIDDEN, 0),
]


def bench_read_probe(args, dev):
    """Streaming-read ceilings (af_rt_read_probe): for each workload's bytes per
    launch, the median time of a launch that only reads them, over a sweep of
    workgroup counts, for contiguous chunks and for the decode kernel's head-row
    access pattern, each with the default and the non-temporal load policy (`_nt`
    keys; the decode kernels' KV rows use the latter). Times are per launch from
    graphs of `layers` launches, each on its own region."""
    stream = dev.Stream()
    sink = dev.DeviceBuffer(256)
    t = Timer(dev, stream, args.warmup)
    out = {}
    for name, nbytes, layers, row_bytes, seg in READ_PROBE_WORKLOADS:
        log(f"read probe: {name}, {nbytes} B per launch x {layers} regions ...")
        buf = dev.DeviceBuffer(nbytes * layers)
        buf.fill_u32(0x3C003C00, stream)
        n_seg = row_bytes // seg if seg else 0
        entry = {"bytes_per_launch": nbytes, "regions": layers, "head_row_bytes": row_bytes,
                 "segment_bytes": seg}
        kinds = [("contiguous", (256, 512, 1024, 2048, 4096, 8192))]
        if n_seg:
            kinds.append(("head_rows", tuple(n_seg * sp for sp in (24, 32, 64, 128, 256, 512))))
        kinds = [(k + ("_nt_us" if nt else "_us"), grid, nt) for k, grid in kinds for nt in (0, 1)]
        for kind, _, _ in kinds:
            entry[kind] = {}
        for kind, grid, nt in kinds:
            for g in grid:
                def launches(g=g, kind=kind, nt=nt):
                    for l in range(layers):
                        if kind.startswith("contiguous"):
                            dev.read_probe(buf.ptr + l * nbytes, nbytes, g, sink.ptr, stream=stream,
                                           nontemporal=nt)
                        else:
                            dev.read_probe(buf.ptr + l * nbytes, nbytes, g, sink.ptr, seg,
                                           row_bytes, stream=stream, nontemporal=nt)
                graph = dev.Graph.capture(stream, launches)
                us = t.graph_ms(graph, args.steps) * 1e3 / layers
                graph.destroy()
                entry[kind][str(g)] = round(us, 3)
        for kind in ("contiguous_us", "contiguous_nt_us", "head_rows_us", "head_rows_nt_us"):
            if not entry.get(kind):
                continue
            g, us = min(entry[kind].items(), key=lambda kv_: kv_[1])
            gbs = nbytes / (us * 1e-6) / 1e9
            entry["best_" + kind[:-3]] = {"workgroups": int(g), "us": us, "gbs": round(gbs, 1),
                                         "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}
        out[name] = entry
        buf.free()
    sink.free()
    stream.destroy()
    return out


STAMP_PHASES = ["split start", "ring prologue issued", "main loop entered", "rows streamed",
                "partials in LDS", "partial stores issued", "stores acknowledged, flag set"]
COMBINER_PHASES = {0: "combiner start", 6: "combiner: last flag seen", 7: "combiner: output written"}


STAMP_WGS, STAMP_SLOTS = 4096, 12  # the stamps build's table: [workgroup][slot]
# slots of the grid form beyond STAMP_PHASES: 8 kernel entry, 9 hardware ids
# (XCC_ID | HW_ID << 32), 10 last-arrival combine done, 11 block table staged;
# a slot counts only if it is later than the same workgroup's entry (no clearing)
GRID_PHASES = [(8, "entry"), (0, "mapped (split start)"), (11, "block table staged"),
               (1, "ring prologue issued"), (2, "main loop entered"), (3, "rows streamed"),
               (4, "partials in LDS"), (5, "partial stores issued"), (6, "stores acknowledged")]


def bench_stamps_paged(args, dev, kv, lib):
    """Timeline of one configs[2] attention launch (paged fp16, B = 32, the compact
    grid) from the stamps build: each workgroup's phases, how many workgroups are in
    each state over time, and per CU the share of the launch during which none of
    its workgroups is streaming rows. 4 layers (549 MB of KV each, past the MALL)
    in a graph; the last launch of each of `steps` replays; medians over replays."""
    import ctypes
    import atomflow_amd
    from atomflow_amd import AF_KV_FP16

    layers = 4
    r = np.random.Generator(np.random.PCG64(0xA70F10 + 3))  # bench_paged's configs[2] draw
    bs, ctx_lens = 16, r.integers(128, 8193, 32)
    B = len(ctx_lens)
    lens_after = ctx_lens + 1
    need = sum((int(n) + bs - 1) // bs for n in lens_after)
    total_blocks = int(need * 1.1) + 8
    bm = kv.BlockManager(total_blocks, bs, layers, NKV, HD, AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(total_blocks)]
    for b in r.permutation(ids):
        bm.free_block(int(b))
    seqs = []
    for n in lens_after:
        sq = bm.seq_create()
        assert not isinstance(bm.seq_extend(sq, int(n)), int)
        seqs.append(sq)
    max_len = int(lens_after.max())
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    stream = dev.Stream()
    nbytes = kv.pool_bytes(bm.pool())
    pool = dev.DeviceBuffer(nbytes)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(pool.ptr, nbytes // 2, 7, 1.0, stream.handle))
    bm.attach_pool(pool.ptr, None)
    desc = bm.pool()
    qkv = dev.DeviceBuffer(layers * B * QKV * 2)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, layers * B * QKV, 11, 1.0, stream.handle))
    out = dev.DeviceBuffer(layers * B * Q_DIM * 2)
    d_tables, d_lens = dev.DeviceBuffer.from_array(tables), dev.DeviceBuffer.from_array(lens)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0, stream)
    stream.sync()
    raw = ctypes.CDLL(atomflow_amd.LIB_PATH)
    raw.af_dbg_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    table = np.zeros((STAMP_WGS, STAMP_SLOTS), np.uint64)

    def attention():
        for l in range(layers):
            kv.launch_paged_attention(qkv.ptr + l * B * QKV * 2, QKV, desc, l, d_tables, max_blocks,
                                      d_lens, B, max_len, out.ptr + l * B * Q_DIM * 2, Q_DIM, NQ,
                                      ws, stream=stream)

    graph = dev.Graph.capture(stream, attention)
    for _ in range(args.warmup):
        graph.launch(stream)
    stream.sync()
    per = []
    for _ in range(args.steps):
        graph.launch(stream)
        stream.sync()
        atomflow_amd.check(raw.af_dbg_phase_stamps(table.ctypes.data, table.nbytes))
        st = table.astype(np.int64)
        hwids = st[:, 9].copy()
        # this launch's entries (within 1 ms of the latest), and slots after them
        fresh = st[:, 8] > st[:, 8].max() - 100000
        st[:, 9] = 0
        valid = (st > st[:, 8:9]) | (np.arange(STAMP_SLOTS) == 8)
        st = np.where(valid & fresh[:, None], st, 0)
        real = (st[:, 0] > 0) & (st[:, 8] > 0)  # workgroups with a split (not past the batch)
        t0 = st[st[:, 8] > 0, 8].min()
        us = np.where(st > 0, (st - t0) * 0.01, np.nan)[real]
        end = np.where(np.isnan(us[:, 10]), us[:, 6], us[:, 10])
        row = {"workgroups": int(real.sum()), "launched": int(fresh.sum()),
               "span_us": float(np.nanmax(end))}
        for (pa, na), (pb, nb) in zip(GRID_PHASES[:-1], GRID_PHASES[1:]):
            d = us[:, pb] - us[:, pa]
            row[f"{na} -> {nb}"] = (float(np.nanmedian(d)), float(np.nanpercentile(d, 90)))
        d = us[:, 10] - us[:, 6]
        row["stores acknowledged -> combine done (last arrivals)"] = (
            float(np.nanmedian(d)), float(np.nanpercentile(d, 90)), int(np.sum(~np.isnan(d))))
        life = end - us[:, 8]
        row["streaming share of a workgroup's life"] = float(np.nanmedian((us[:, 3] - us[:, 2]) / life))
        # per CU: the share of the launch with no workgroup streaming rows
        hw = hwids[real]
        cu = (hw & 0xF) * 1024 + ((hw >> 32) >> 8 & 0xFF)  # XCC, then CU / SH / SE bits of HW_ID
        span = row["span_us"]
        grid_t = np.arange(0.0, span, 0.1)
        idle = []
        for c in np.unique(cu):
            m = cu == c
            on = np.zeros(len(grid_t), bool)
            for a0, a1 in zip(us[m, 2], us[m, 3]):
                on |= (grid_t >= a0) & (grid_t < a1)
            idle.append(1.0 - on.mean())
        row["CUs"] = int(len(idle))
        row["CU share with no workgroup streaming"] = float(np.mean(idle))
        states = []
        for t in np.arange(0.0, span, 4.0):
            pre = int(np.sum((us[:, 8] <= t) & (us[:, 2] > t)))
            strm = int(np.sum((us[:, 2] <= t) & (us[:, 3] > t)))
            epi = int(np.sum((us[:, 3] <= t) & (end > t)))
            states.append((round(float(t)), pre, strm, epi))
        row["states"] = states
        per.append(row)
    graph.destroy()
    result = {"workload": f"configs[2] paged fp16, B={B}, 16-token blocks, {layers} layers rotated; "
                          "attention only (af_paged_attention, compact grid)",
              "replays": args.steps, "unit": "us from the launch's first workgroup entry"}
    for k, v in per[0].items():
        if k == "states":
            continue
        vals = [r[k] for r in per]
        if isinstance(v, tuple):
            result[k] = [round(float(np.median([x[i] for x in vals])), 3) for i in range(len(v))]
        else:
            result[k] = round(float(np.median(vals)), 4)
    mid = sorted(per, key=lambda r: r["span_us"])[len(per) // 2]
    result["states (t us: prologue / streaming / epilogue workgroups), median-span replay"] = \
        mid["states"]
    bm.close()
    for b in (pool, qkv, out, d_tables, d_lens):
        b.free()
    stream.destroy()
    return result


def bench_stamps(args, dev, kv, lib):
    """Where one attention launch's time goes (configs[1], batch 1): the stamps
    build records s_memrealtime (10 ns ticks) per workgroup at each phase of the
    decode kernel (split workgroups, then the dedicated combiners). For the last
    launch of a 28-layer graph (fused step, then attention only), after each of
    `steps` replays: every phase's median and slowest workgroup, in us from the
    first workgroup's start; the medians over replays are reported."""
    import ctypes
    import atomflow_amd

    ctx = args.ctx
    L = ctx + 1
    max_seq = (L + 127) // 128 * 128
    slab = max_seq * KV_DIM * 2
    stream = dev.Stream()
    pool = dev.DeviceBuffer(LAYERS * 2 * slab)
    qkv = dev.DeviceBuffer(LAYERS * QKV * 2)
    out = dev.DeviceBuffer(LAYERS * Q_DIM * 2)
    d_cos = dev.DeviceBuffer(max_seq * HD // 2 * 4)
    d_sin = dev.DeviceBuffer(max_seq * HD // 2 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA, stream)
    atomflow_amd.check(lib.af_rt_fill_randn_f16(pool.ptr, LAYERS * 2 * slab // 2, 7, 1.0, stream.handle))
    atomflow_amd.check(lib.af_rt_fill_randn_f16(qkv.ptr, LAYERS * QKV, 11, 1.0, stream.handle))
    splits = args.splits or kv.default_splits(L, 1, NKV)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    stream.sync()
    raw = ctypes.CDLL(atomflow_amd.LIB_PATH)
    raw.af_dbg_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    table = np.zeros((STAMP_WGS, STAMP_SLOTS), np.uint64)

    def ptrs(l):
        return (qkv.ptr + l * QKV * 2, pool.ptr + 2 * l * slab, pool.ptr + (2 * l + 1) * slab,
                out.ptr + l * Q_DIM * 2)

    def fused():
        for l in range(LAYERS):
            q, k, v, o = ptrs(l)
            kv.launch_decode_attention_fused(q, k, v, d_cos, d_sin, ctx, max_seq, o, NQ, NKV, HD,
                                             ws, num_splits=splits, stream=stream)

    def attention():
        for l in range(LAYERS):
            q, k, v, o = ptrs(l)
            kv.launch_cached_attention_ex(q, k, v, o, L, max_seq, HD, NQ, NKV, ws,
                                          num_splits=splits, stream=stream)

    result = {"workload": f"configs[1] ctx {ctx}, batch 1, {splits} splits x {NKV} KV heads",
              "splits": splits, "phases": STAMP_PHASES + list(COMBINER_PHASES.values()),
              "unit": "us from the first workgroup's start", "replays": args.steps}
    for name, fn in (("fused", fused), ("attention", attention)):
        graph = dev.Graph.capture(stream, fn)
        for _ in range(args.warmup):
            graph.launch(stream)
        stream.sync()
        per = []
        for _ in range(args.steps):
            atomflow_amd.check(raw.af_dbg_phase_stamps_clear())
            graph.launch(stream)
            stream.sync()
            atomflow_amd.check(raw.af_dbg_phase_stamps(table.ctypes.data, table.nbytes))
            t = table[: splits * NKV].astype(np.float64)
            c = table[splits * NKV: splits * NKV + NKV].astype(np.float64)
            t0 = min(t[:, 0][t[:, 0] > 0].min(), c[:, 0][c[:, 0] > 0].min() if (c[:, 0] > 0).any() else np.inf)
            row = {}
            for rows, phases in ((t, dict(enumerate(STAMP_PHASES))), (c, COMBINER_PHASES)):
                for ph, pname in phases.items():
                    v = rows[:, ph]
                    v = (v[v > 0] - t0) * 0.01
                    if len(v):
                        row[pname] = (float(np.median(v)), float(v.max()), int(len(v)))
            # per KV head (workgroup id = split * heads + head: every split of
            # head h runs on XCD h when heads = 8)
            heads = np.arange(splits * NKV) % NKV
            for ph in (1, 3):
                row[f"by_kv_head {STAMP_PHASES[ph]}"] = [
                    float(np.median((t[heads == h, ph] - t0) * 0.01)) for h in range(NKV)]
            per.append(row)
        graph.destroy()
        summary = {}
        for pname in STAMP_PHASES + list(COMBINER_PHASES.values()):
            vals = [r[pname] for r in per if pname in r]
            if vals:
                summary[pname] = {"median_us": round(float(np.median([v[0] for v in vals])), 3),
                                  "slowest_us": round(float(np.median([v[1] for v in vals])), 3),
                                  "workgroups": vals[0][2]}
        for ph in (1, 3):
            key = f"by_kv_head {STAMP_PHASES[ph]}"
            summary[key] = [round(float(np.median([r[key][h] for r in per])), 3) for h in range(NKV)]
        result[name] = summary
    for b in (pool, qkv, out, d_cos, d_sin):
        b.free()
    stream.destroy()
    return result


def bench_compare(args):
    """In-process A/B of two builds of the library. Both are loaded with RTLD_LOCAL (each
    resolves its own symbols), the buffers are allocated once, and every workload's graph
    is captured once per build, on a workspace of that build's own (sized and initialised by
    it, so the builds may lay their workspaces out differently); the graphs are then replayed
    alternately, `compare_rounds` rounds of `steps`
    replays, and the median per-launch microseconds of each build are printed with B/A. The
    spread between processes (a fresh pool lands on different memory) does not enter."""
    import ctypes
    import atomflow_amd
    from atomflow_amd import AF_KV_FP16, AF_KV_FP8_E4M3, _abi

    paths = [atomflow_amd.LIB_PATH, os.path.abspath(args.compare_lib)]
    libs = [_abi.bind(ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL)) for p in paths]
    atomflow_amd._lib = libs[0]
    from atomflow_amd import device as dev
    from atomflow_amd import kv
    dev.set_device(0)
    stream = dev.Stream()
    lib0 = libs[0]
    print(f"A = {paths[0]}\nB = {paths[1]}", flush=True)

    def timed(graph):
        e0, e1 = dev.Event(), dev.Event()
        ts = []
        for _ in range(args.steps):
            e0.record(stream)
            graph.launch(stream)
            e1.record(stream)
            stream.sync()
            ts.append(e0.elapsed_ms(e1) * 1e3 / LAYERS)
        e0.destroy()
        e1.destroy()
        return float(np.median(ts))

    def ab(name, mkws, kinds):
        graphs, wss = {}, []
        for li, L in enumerate(libs):
            atomflow_amd._lib = L
            ws = mkws()
            wss.append(ws)
            for kind, fn in kinds.items():
                g = dev.Graph.capture(stream, lambda: fn(ws))
                for _ in range(max(args.warmup, 1)):
                    g.launch(stream)
                stream.sync()
                graphs[(li, kind)] = g
        atomflow_amd._lib = libs[0]
        res = {k: [] for k in graphs}
        for r in range(args.compare_rounds):
            order = list(graphs)
            for k in (order if r % 2 == 0 else order[::-1]):
                res[k].append(timed(graphs[k]))
        for kind in kinds:
            va, vb = np.array(res[(0, kind)]), np.array(res[(1, kind)])
            print(f"{name:7s} {kind:10s} A {np.median(va):9.2f} us  B {np.median(vb):9.2f} us  "
                  f"B/A {np.median(vb) / np.median(va):.4f}   (A {va.min():.2f}-{va.max():.2f}, "
                  f"B {vb.min():.2f}-{vb.max():.2f})", flush=True)
        for g in graphs.values():
            g.destroy()
        for ws in wss:
            ws.buf.free()

    def contiguous(ctx):
        L = ctx + 1
        max_seq = (L + 127) // 128 * 128
        slab = max_seq * KV_DIM * 2
        pool = dev.DeviceBuffer(LAYERS * 2 * slab)
        qkv = dev.DeviceBuffer(LAYERS * QKV * 2)
        out = dev.DeviceBuffer(LAYERS * Q_DIM * 2)
        d_cos = dev.DeviceBuffer(max_seq * HD // 2 * 4)
        d_sin = dev.DeviceBuffer(max_seq * HD // 2 * 4)
        kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA, stream)
        atomflow_amd.check(lib0.af_rt_fill_randn_f16(pool.ptr, LAYERS * 2 * slab // 2, 7, 1.0,
                                                     stream.handle))
        atomflow_amd.check(lib0.af_rt_fill_randn_f16(qkv.ptr, LAYERS * QKV, 11, 1.0, stream.handle))
        stream.sync()

        def ptrs(l):
            return (qkv.ptr + l * QKV * 2, pool.ptr + 2 * l * slab, pool.ptr + (2 * l + 1) * slab,
                    out.ptr + l * Q_DIM * 2)

        def fused(ws):
            for l in range(LAYERS):
                q, k, v, o = ptrs(l)
                kv.launch_decode_attention_fused(q, k, v, d_cos, d_sin, ctx, max_seq, o, NQ, NKV, HD,
                                                 ws, stream=stream)

        def attention(ws):
            for l in range(LAYERS):
                q, k, v, o = ptrs(l)
                kv.launch_cached_attention_ex(q, k, v, o, L, max_seq, HD, NQ, NKV, ws, stream=stream)
        ab(f"ctx{ctx // 1024}k", lambda: kv.AttentionWorkspace(1, NQ, NKV, HD, 0, stream),
           {"fused": fused, "attention": attention})
        for b in (pool, qkv, out, d_cos, d_sin):
            b.free()

    def paged(cfg):
        r = np.random.Generator(np.random.PCG64(0xA70F10 + cfg))  # bench_paged's draws
        fp8 = cfg == 5
        bs = 32 if fp8 else 16
        if cfg == 3:
            lens_new = r.integers(128, 8193, 32)
        elif cfg == 5:
            lens_new = r.integers(8192, 16385, 128)
        else:
            prefix, suffix = 2048, r.integers(1, 1025, 64)
        B = 64 if cfg == 4 else len(lens_new)
        if cfg == 4:
            need = prefix // bs + sum((int(x) + 1 + bs - 1) // bs for x in suffix)
        else:
            need = sum((int(n) + 1 + bs - 1) // bs for n in lens_new)
        total_blocks = int(need * 1.1) + 8
        bm = kv.BlockManager(total_blocks, bs, LAYERS, NKV, HD, AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16)
        ids = [bm.allocate_block() for _ in range(total_blocks)]
        for b in r.permutation(ids):
            bm.free_block(int(b))
        if cfg == 4:
            root = bm.seq_create()
            bm.seq_extend(root, prefix)
            seqs = [root] + [bm.seq_fork(root) for _ in range(B - 1)]
            for sq, n in zip(seqs, suffix):
                assert not isinstance(bm.seq_extend(sq, int(n)), int)
        else:
            seqs = []
            for n in lens_new:
                sq = bm.seq_create()
                assert not isinstance(bm.seq_extend(sq, int(n)), int)
                seqs.append(sq)
        plan = bm.plan_decode(seqs)
        assert not isinstance(plan, int), plan
        slots, positions, _ = plan
        max_len = int(positions.max()) + 1
        max_blocks = (max_len + bs - 1) // bs
        tables, lens = bm.export_tables(seqs, max_blocks)
        nbytes = kv.pool_bytes(bm.pool())
        pool = dev.DeviceBuffer(nbytes)
        scales = None
        if fp8:
            sc = 5.0 / 448.0
            scales = dev.DeviceBuffer.from_array(np.full((LAYERS, 2, NKV), sc, np.float32))
            atomflow_amd.check(lib0.af_rt_fill_randn_fp8(pool.ptr, nbytes, 7, 1.0 / sc, stream.handle))
        else:
            atomflow_amd.check(lib0.af_rt_fill_randn_f16(pool.ptr, nbytes // 2, 7, 1.0, stream.handle))
        bm.attach_pool(pool.ptr, scales.ptr if scales else None)
        desc = bm.pool()
        if cfg == 4:  # the forks map the prefix blocks: keep KV rows cached
            desc.flags = atomflow_amd.AF_KV_POOL_SHARED_BLOCKS
        max_pos = max_len + 1
        d_cos = dev.DeviceBuffer(max_pos * HD // 2 * 4)
        d_sin = dev.DeviceBuffer(max_pos * HD // 2 * 4)
        kv.build_rope_cache(d_cos, d_sin, max_pos, HD, THETA, stream)
        qkv = dev.DeviceBuffer(LAYERS * B * QKV * 2)
        atomflow_amd.check(lib0.af_rt_fill_randn_f16(qkv.ptr, LAYERS * B * QKV, 11, 1.0,
                                                     stream.handle))
        out = dev.DeviceBuffer(LAYERS * B * Q_DIM * 2)
        d_t, d_l = dev.DeviceBuffer.from_array(tables), dev.DeviceBuffer.from_array(lens)
        d_sl, d_p = dev.DeviceBuffer.from_array(slots), dev.DeviceBuffer.from_array(positions)
        bufs = [pool, d_cos, d_sin, qkv, out, d_t, d_l, d_sl, d_p] + ([scales] if scales else [])
        stream.sync()
        qp = lambda l: qkv.ptr + l * B * QKV * 2
        op = lambda l: out.ptr + l * B * Q_DIM * 2
        kinds = {}
        if cfg == 4:
            d_root = dev.DeviceBuffer.from_array(np.ascontiguousarray(tables[0]))
            bufs.append(d_root)
            kinds["shared"] = lambda ws: [kv.launch_paged_attention_shared_prefix(
                qp(l), QKV, desc, l, d_root, prefix, d_t, max_blocks, d_l, B, max_len, op(l), Q_DIM,
                NQ, ws, stream=stream) for l in range(LAYERS)]
        else:
            kinds["fused"] = lambda ws: [kv.launch_paged_decode_fused(
                qp(l), B, desc, l, d_sl, d_p, d_cos, d_sin, max_pos, d_t, max_blocks, max_len, op(l),
                Q_DIM, NQ, ws, stream=stream) for l in range(LAYERS)]
        kinds["attention" if cfg != 4 else "plain"] = lambda ws: [kv.launch_paged_attention(
            qp(l), QKV, desc, l, d_t, max_blocks, d_l, B, max_len, op(l), Q_DIM, NQ, ws,
            stream=stream) for l in range(LAYERS)]
        ab(f"cfg{cfg}", lambda: kv.AttentionWorkspace(B, NQ, NKV, HD, 0, stream), kinds)
        bm.close()
        for b in bufs:
            b.free()

    for w in args.compare_work.split(","):
        if w.startswith("ctx"):
            contiguous(int(w[3:-1]) * 1024)
        else:
            paged(int(w[3:]))
    stream.destroy()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the KV path runs on one GPU here; sharding is a design note only)", file=sys.stderr)
        sys.exit(2)
    import atomflow_amd
    from atomflow_amd import device as dev
    from atomflow_amd import kv

    if args.stamps:  # the measurement build of the same library
        atomflow_amd.LIB_PATH = os.environ.get(
            "AF_STAMPS_LIB", os.path.join(ROOT, "atomflow_amd", "libatomflow_kv_stamps.so"))
    if args.compare_lib:
        bench_compare(args)
        return
    lib = atomflow_amd.lib()
    dev.set_device(0)
    info = dev.device_info()
    log(f"device {info}")
    if args.fanout_only:
        print(json.dumps({"serving_fanout": bench_fanout(dev, kv, lib)}), flush=True)
        return
    if args.read_probe:
        print(json.dumps({"read_probe": bench_read_probe(args, dev)}), flush=True)
        return
    if args.stamps:
        fn = bench_stamps_paged if args.config == 3 else bench_stamps
        print(json.dumps({"stamps": fn(args, dev, kv, lib)}), flush=True)
        return
    if args.config == 2:
        result = bench_contiguous(args, dev, kv, lib, info)
        if not args.no_cpu:
            log("cpu baseline (C++ oracle, threaded and 1 thread) ...")
            result["cpu_baseline"] = cpu_baseline(args.ctx)
        if not args.no_matrix and args.ctx == 8192:
            result["matrix"] = bench_matrix(args, dev, kv, lib, info, result)
    else:
        result = bench_paged(args, dev, kv, lib, info)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
