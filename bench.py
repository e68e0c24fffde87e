"""Benchmark of the sampling hot path on one MI355X.

A step is one bfi_smp_sample_rows call (or bfi_smp_verify for C4) over a batch that is
already resident in HBM. The default workload is C2: B=64 rows of V=151936 f32 logits with
per-row temperature/top-k/top-p/min-p and repetition/presence/frequency penalties over
512-id Zipf histories. The timed steps rotate over copies of the batch that together exceed
the 256 MiB last-level cache, so every step streams its logits from HBM. A separate
profiling pass (outside the timed loop) records HIP events in the dispatch packets of each
kernel of every call: the whole call's time (first kernel's start to last kernel's end)
gives the headline roofline, each kernel's its own entry. Output: one JSON line with
whole-job rows/s, the roofline, and the CPU oracle's rows/s on this host (all cores, and
one core).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "builderforce-inference_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0
METRIC = "sampled rows/sec + achieved HBM GB/s (% of peak) at B=64, V=151936 fp32"
WORKLOAD_DESC = {
    "C1": "C1: B=1, V=151936 f32, rep 1.1 over 64 ids, T 0.7 / top-k 40 / top-p 0.95",
    "C2": "C2: B=64, V=151936 f32, per-row T U[0.2,1.5], top-k {0,20,50,100}, top-p U[0.8,1], min-p 0.05, "
          "rep 1.1 + presence 0.5 + frequency 0.3 over 512-id Zipf(1.1) histories",
    "C2M": "C2M: C2 under packed grammar allow-masks (0.1%-30% allowed, runs 1-64)",
    "C3": "C3: B=32, V=151936 f32, packed allow-mask (0.1%-30% allowed, runs 1-64), T 1.0 / top-p 0.9",
    "C4": "C4: spec verify, 16 seq x (4 drafts + 1) rows, V=151936 f32, T 0.8 / top-p 0.95",
    "C5": "C5: B=256, V=262144 bf16, top-p 0.9 over the full vocabulary, rep 1.05 over 1024-id histories",
}


def read_traffic(name):
    """HBM bytes per call (all three kernels) from the committed rocprofv3 counter summary
    (profiles/sample_rows_<config>.txt or verify_<config>.txt, line 'traffic_bytes: N'), if
    present."""
    entry = "verify" if name == "C4" else "sample_rows"
    p = os.path.join(ROOT, "profiles", f"{entry}_{name}.txt")
    try:
        for line in open(p):
            if line.startswith("traffic_bytes:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_threads():
    """The cores this process may run on (its CPU affinity)."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        return max(1, os.cpu_count() or 1)


def cpu_baseline(cfg, seconds, threads):
    """The oracle (C restatement of the reference sampler) on this host, `threads` threads
    splitting each batch's rows, over whole batches of the same workload until `seconds`
    have elapsed."""
    import oracle as O
    import workloads

    x = cfg["logits"]
    dtype = 1 if cfg["dtype"] == "bf16" else 0
    rows = 0
    t0 = time.perf_counter()
    batches = 0
    while True:
        if "drafts" in cfg:
            S, R = cfg["n_seq"], cfg["rows_per_seq"]
            xf = workloads.bf16_bits_to_f32(x) if dtype else x
            for s in range(S):
                p = {k: (int(cfg["params"][s][k]) if k == "top_k" else float(cfg["params"][s][k]))
                     for k in cfg["params"].dtype.names if k != "reserved"}
                h = cfg["hist"][cfg["hist_off"][s]:cfg["hist_off"][s + 1]]
                O.verify_seq(xf[s * R:(s + 1) * R], p, h, cfg["drafts"][s], cfg["u_pairs"][s].reshape(-1),
                             float(cfg["u_bonus"][s]))
            rows += S * R
        else:
            O.sample_rows(x, cfg["params"], cfg["hist"], cfg["hist_off"], cfg["u"], cfg["mask"], dtype=dtype,
                          threads=threads)
            rows += cfg["B"]
        batches += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    if "drafts" in cfg:
        threads = 1
    return dict(value=rows / el, unit="rows/s", cores=threads, kind="port",
                sample=f"{batches} whole batches of the {cfg['name']} workload ({rows} rows, {el:.1f} s) through "
                       f"the C restatement of sample.rs/spec.rs (oracle/bfi_oracle.c), rows split over "
                       f"{threads} thread{'s' if threads > 1 else ''}")


def bench_mask(args):
    """One step = one bfi_mask_build call (host scan of the generated text + the k_mask
    launch) for the named tool-call constraint over the synthetic vocabulary; timed with
    events on the stream. The CPU baseline is the oracle's restatement of apply_constraint
    (sample.rs:63-90: a rescan of so_far + piece per id) on a sample of ids."""
    import numpy as np
    import torch

    import bfi_smp
    import workloads

    V = 151936
    pieces = workloads.synthetic_vocab(V, seed=args.seed)
    mp = bfi_smp.MaskProducer(0)
    mp.set_vocab(pieces)
    nw = (V + 31) // 32
    d = torch.empty(nw, dtype=torch.int32, device="cuda:0")
    c = workloads.MASK_TOOLS
    so_far = workloads.MASK_SO_FAR
    for _ in range(args.warmup):
        mp.build(so_far, d, **c)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        mp.build(so_far, d, **c)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    piece_bytes = sum(len(p) for p in pieces)
    moved = piece_bytes + 4 * (V + 1) + 4 * nw
    line = {"metric": "allow-mask ids/sec (named tool-call constraint, V=151936)", "value": round(V / (ms / 1e3), 1),
            "unit": "ids/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 5), "wall_ms_per_step": round(wall * 1e3 / args.steps, 5),
            "higher_is_better": True, "dtype": "u8", "data": "synthetic vocabulary (workloads.synthetic_vocab)",
            "config": {"workload": "F1: named tool-call constraint", "n_vocab": V, "so_far_bytes": len(so_far),
                       "piece_bytes": piece_bytes},
            "bytes_per_step": moved, "step_gbs": round(moved / (ms / 1e3) / 1e9, 1)}
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import constraint as K

        n, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < args.cpu_seconds and n < V:
            K.allow_mask(pieces[n:n + 2000], so_far, dict(c))
            n += 2000
        dt = time.perf_counter() - t1
        line["cpu_baseline"] = {"value": round(n / dt, 1), "unit": "ids/s", "cores": 1, "kind": "port",
                                "sample": f"{n} ids of the same vocabulary through oracle/constraint.py "
                                          f"(apply_constraint restated: one rescan of so_far + piece per id), "
                                          f"{dt:.1f} s"}
    print(json.dumps(line), flush=True)
    mp.close()


def bench_head(args):
    """The device output head (bfi_smp_head: rms_norm + lm_head with the reference's
    rounding) and the fused head + sample step (bfi_smp_head_sample_rows) on a
    Qwen3-0.6B-shaped head: 64 rows (C2's batch), n_embd 1024, n_vocab 151936, f32 weights
    (622 MB), C2's per-row parameters and histories. Timed with events on the stream over
    `--steps` calls after `--warmup`. The CPU baseline is the oracle's head (one thread) on
    one row."""
    import numpy as np
    import torch

    import bfi_smp
    import oracle as O
    import workloads

    T, d, V = 64, 1024, 151936
    rng = np.random.default_rng(args.seed)
    dev = torch.device("cuda:0")
    x = torch.from_numpy((rng.standard_normal((T, d)) * 3).astype(np.float32)).to(dev)
    nw = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).to(dev)
    w = torch.from_numpy((rng.standard_normal((V, d)) * (8 / np.sqrt(d))).astype(np.float32)).to(dev)
    cfg = workloads.config("C2", seed=args.seed)
    dd = workloads.to_device(cfg, dev)
    smp = bfi_smp.Sampler(0)
    logits = torch.empty((T, V), dtype=torch.float32, device=dev)
    out = torch.zeros(T, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream()

    def timed(fn, steps, warm):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(steps):
            fn()
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps * 1e-3

    steps, warm = max(5, min(args.steps, 50)), max(2, min(args.warmup, 5))
    t_head = timed(lambda: smp.head(x, nw, 1e-6, w, out=logits), steps, warm)
    t_fused = timed(lambda: smp.head_sample_rows(x, nw, 1e-6, w, dd["params"], dd["u"], out, dd["hist"],
                                                 dd["hist_off"]), steps, warm)
    flops = 2.0 * T * V * d
    achieved = flops / t_head / 1e12
    # the same head over Q8_0 weights (a GGUF lm_head format): dequantized once, then the
    # block dot order (each 32-weight block summed apart)
    wq = (rng.standard_normal((V, d)) * (8 / np.sqrt(d))).astype(np.float32).reshape(-1, 32)
    dq = np.maximum(np.abs(wq).max(1), 1e-8) / 127.0
    q8 = np.zeros((wq.shape[0], 34), np.uint8)
    q8[:, 0:2] = dq.astype(np.float16).view(np.uint8).reshape(-1, 2)
    q8[:, 2:] = np.clip(np.rint(wq / dq[:, None]), -127, 127).astype(np.int8).view(np.uint8)
    src = torch.from_numpy(q8.reshape(-1)).to(dev)
    w8 = torch.empty((V, d), dtype=torch.float32, device=dev)
    t_deq = timed(lambda: smp.dequant(8, src, V * d, out=w8), 3, 1)
    t_head_q8 = timed(lambda: smp.head_typed(x, nw, 1e-6, w8, 8, out=logits), steps, warm)
    xs = x[:1].cpu().numpy()
    ws = w.cpu().numpy()
    t0 = time.perf_counter()
    O.matmul_f32(ws, O.rms_norm(xs, nw.cpu().numpy(), 1e-6))
    t_cpu = time.perf_counter() - t0
    line = {"metric": "device head + sample rows/sec (Qwen3-0.6B-shaped head, B=64)",
            "value": round(T / t_fused, 1), "unit": "rows/s", "n_gpus": 1, "higher_is_better": True,
            "head_ms": round(t_head * 1e3, 3), "head_sample_ms": round(t_fused * 1e3, 3),
            "head_q8_0_ms": round(t_head_q8 * 1e3, 3), "dequant_q8_0_ms": round(t_deq * 1e3, 3),
            "readback_bytes_per_row": 4, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "F2 head + sample", "rows": T, "n_embd": d, "n_vocab": V},
            "roofline": {"bound": "valu", "achieved": round(achieved, 2), "peak": 157.3, "unit": "TFLOP/s",
                         "frac": round(achieved / 157.3, 4), "traffic": V * d * 4 + T * (d + V) * 4,
                         "note": "products and sums separately rounded (the reference's order): one "
                                 "unpacked multiply and one add a term, no MFMA"},
            "cpu_baseline": {"value": round(1.0 / t_cpu, 3), "unit": "rows/s", "cores": 1, "kind": "port",
                             "sample": "the oracle's head on one row"}}
    print(json.dumps(line), flush=True)
    smp.close()


def bench_prefix(args):
    """The prefix cache (include/bfi_prefix.h, engine/prefix.rs) on a Qwen3-0.6B-shaped state:
    28 layers x (K, V) of [4096 positions, 8 heads x 128] f32 rows (4 KiB a row), 2048 positions
    used, the logits of a 151,936-id vocabulary. One insert copies the used rows device to
    device; one restore copies them back into full-capacity tensors and zeroes the other 2048
    rows. Timed with events on the stream; lookup timed on the host with 64 cached entries.
    The CPU baseline is the same cache in host memory (memcpy) on the same state."""
    import numpy as np
    import torch

    import bfi_smp

    L, cap, n, row = 28, 4096, 2048, 8 * 128
    dev = torch.device("cuda:0")
    kv = [torch.randn(cap, row, device=dev) for _ in range(2 * L)]
    logits = torch.randn(151936, device=dev)
    rng = np.random.default_rng(args.seed)
    toks = rng.integers(0, 151936, n).tolist()
    pc = bfi_smp.PrefixCache(8 << 30, 0)
    s = torch.cuda.current_stream()
    kept = 2 * L * n * row * 4

    def timed(fn, reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        fn()
        torch.cuda.synchronize()
        e0.record(s)
        for _ in range(reps):
            fn()
        e1.record(s)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3

    src_st = pc.prepare(n, kv, [], logits)  # (the tensors' descriptions built once, as a native caller keeps them)
    t_ins = timed(lambda: pc.insert(toks, stream=s.cuda_stream, prepared=src_st), 10)
    hit = pc.lookup(toks + [1, 2, 3])
    dst = [torch.empty_like(t) for t in kv]
    ld = torch.empty_like(logits)
    dst_st = pc.prepare(0, dst, [], ld)
    t_res = timed(lambda: pc.restore(hit, stream=s.cuda_stream, prepared=dst_st), 20)
    ok = all(torch.equal(a[:n], b[:n]) and not a[n:].any().item() for a, b in zip(dst, kv))
    # lookup among 64 entries (short states: only the index is timed)
    small = [torch.zeros(cap, 8, device=dev)]
    prompts = [rng.integers(0, 151936, 2048).tolist() for _ in range(64)]
    for p in prompts:
        pc.insert(p, len(p), small, [], logits[:8], stream=s.cuda_stream)
    q = prompts[17][:1500] + rng.integers(0, 151936, 2596).tolist()
    t0 = time.perf_counter()
    for _ in range(200):
        h = pc.lookup(q)
    t_look = (time.perf_counter() - t0) / 200
    assert h is not None and h[1] == 1500
    restore_bytes = 2 * kept + 2 * L * (cap - n) * row * 4 + logits.numel() * 4 * 2
    # CPU baseline: the host-memory cache restoring the same state (memcpy + memset)
    hkv = [np.random.default_rng(1).standard_normal((cap, row)).astype(np.float32) for _ in range(2 * L)]
    hl = np.zeros(151936, np.float32)
    hc = bfi_smp.PrefixCache(8 << 30, -1)
    hc.insert(toks, n, hkv, [], hl)
    hh = hc.lookup(toks + [1])
    hdst = [np.empty_like(t) for t in hkv]
    hld = np.empty_like(hl)
    t0 = time.perf_counter()
    reps = 3
    for _ in range(reps):
        hc.restore(hh, hdst, [], hld)
    t_cpu = (time.perf_counter() - t0) / reps
    achieved = restore_bytes / t_res / 1e9
    line = {"metric": "prefix-cache restore GB/s (Qwen3-0.6B-shaped state, 2048 of 4096 positions)",
            "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "restore_ms": round(t_res * 1e3, 3), "insert_ms": round(t_ins * 1e3, 3),
            "insert_GBps": round(2 * kept / t_ins / 1e9, 1), "lookup_us_64_entries": round(t_look * 1e6, 1),
            "exact": ok, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "F4 prefix cache", "layers": L, "kv_row_bytes": row * 4, "capacity": cap,
                       "used": n},
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                         "frac": round(achieved / 8000.0, 4), "traffic": restore_bytes},
            "cpu_baseline": {"value": round(restore_bytes / t_cpu / 1e9, 2), "unit": "GB/s", "cores": 1,
                             "kind": "port", "sample": "the same restore with the cache in host memory"}}
    print(json.dumps(line), flush=True)
    pc.close()
    hc.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="C2", choices=sorted(WORKLOAD_DESC))
    ap.add_argument("--profile-launches", type=int, default=200,
                    help="calls of the profiling pass (events in every kernel's dispatch), before the timed steps")
    ap.add_argument("--rotate-mib", type=int, default=320,
                    help="the timed steps cycle through copies of the logits totalling at least this many MiB "
                         "(0: one batch, cache-resident)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a device-to-device copy of 256 MiB (10 launches), the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--mask", action="store_true",
                    help="measure the allow-mask producer (include/bfi_mask.h) instead: a named "
                         "tool-call constraint over a synthetic 151,936-piece vocabulary")
    ap.add_argument("--head", action="store_true",
                    help="measure the device output head (rms_norm + lm_head, the reference's rounding) and "
                         "the fused head + sample step on a Qwen3-0.6B-shaped head instead")
    ap.add_argument("--prefix", action="store_true",
                    help="measure the prefix cache (include/bfi_prefix.h) instead: insert, restore and "
                         "lookup of a Qwen3-0.6B-shaped state in device memory")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's path runs on a single MI355X "
              "(rows shard across GPUs with no exchange between them). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if args.copy_calibration:
        n = 64 << 20  # 256 MiB of f32
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "launches": 10}), flush=True)
        return

    import bfi_smp
    import workloads

    if args.mask:
        bench_mask(args)
        return
    if args.prefix:
        bench_prefix(args)
        return
    if args.head:
        bench_head(args)
        return

    cfg = workloads.config(args.config, seed=args.seed)
    dev = torch.device("cuda:0")
    d = workloads.to_device(cfg, dev)
    smp = bfi_smp.Sampler(0)
    verify = "drafts" in cfg
    # copies of the logits, together above the last-level cache, one per step in turn
    batch_bytes = d["logits"].numel() * d["logits"].element_size()
    ncopy = 1 if args.rotate_mib <= 0 else max(1, -(-(args.rotate_mib << 20) // batch_bytes))
    logits = [d["logits"]] + [d["logits"].clone() for _ in range(ncopy - 1)]

    def step(i):
        x = logits[i % ncopy]
        if verify:
            smp.verify(x, cfg["rows_per_seq"], d["params"], d["drafts"], d["draft_len"], d["u_pairs"],
                       d["u_bonus"], d["out_accepted"], d["out_next"], d["hist"], d["hist_off"], d["mask"])
        else:
            smp.sample_rows(x, d["params"], d["u"], d["out"], d["hist"], d["hist_off"], d["mask"])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # the profiling pass: start/stop events in each kernel's dispatch packet, every launch
    smp.set_profiling(True)
    for i in range(args.profile_launches):
        step(i)
    smp.set_profiling(False)
    torch.cuda.synchronize()
    kern_ms, n = smp.profile()
    # the timed steps (no events)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0

    rows = cfg["B"]
    ms_step = el * 1e3 / args.steps
    value = rows * args.steps / el
    alg = workloads.algorithmic_bytes(cfg)
    us = {k: v * 1e3 / max(n, 1) for k, v in kern_ms.items()}
    traffic = read_traffic(args.config)

    def gbs(t_us):
        return round(alg / (t_us * 1e-6) / 1e9, 1) if t_us > 0 else None

    achieved = gbs(us["call"])
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg["dtype"] == "bf16" else "f32",
        "data": "synthetic (seeded generator, builderforce-inference_amd/workloads.py)",
        "config": {"workload": WORKLOAD_DESC[args.config], "batch_rows": rows, "n_vocab": cfg["V"],
                   "seed": args.seed, "rotating_copies": ncopy,
                   "rotating_mib": round(ncopy * batch_bytes / 2 ** 20, 1)},
        "roofline": {
            "bound": "hbm",
            "kernel": "whole call (k_stream + k_quant + k_row, first start to last end)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": traffic,
            "algorithmic_bytes": alg,
            "call_us": round(us["call"], 3),
            "timed_launches": n,
            "per_kernel": {k: {"us": round(us[k], 3), "achieved": gbs(us[k]),
                               "frac": round(gbs(us[k]) / HBM_PEAK_GBS, 4) if us[k] > 0 else None}
                           for k in ("k_stream", "k_quant", "k_row")},
        },
        "step_hbm_gbs": round(alg / (ms_step * 1e-3) / 1e9, 1),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds, cpu_threads())
        out["cpu_baseline_1core"] = cpu_baseline(cfg, args.cpu_seconds, 1)
    smp.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
