"""Benchmark of the sampling hot path on one MI355X.

A step is one bfi_smp_sample_rows call (or bfi_smp_verify for C4) over a batch that is
already resident in HBM. The default workload is C2: B=64 rows of V=151936 f32 logits with
per-row temperature/top-k/top-p/min-p and repetition/presence/frequency penalties over
512-id Zipf histories. Output: one JSON line with whole-job rows/s, the HBM roofline of the
streaming pass (the kernel that moves the bytes; its duration from HIP events recorded in
its dispatch packets on every 32nd step of the timed region) and the CPU oracle's rows/s on
this host.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "builderforce-inference_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0
PROFILE_EVERY = 32
METRIC = "sampled rows/sec + achieved HBM GB/s (% of peak) at B=64, V=151936 fp32"
WORKLOAD_DESC = {
    "C1": "C1: B=1, V=151936 f32, rep 1.1 over 64 ids, T 0.7 / top-k 40 / top-p 0.95",
    "C2": "C2: B=64, V=151936 f32, per-row T U[0.2,1.5], top-k {0,20,50,100}, top-p U[0.8,1], min-p 0.05, "
          "rep 1.1 + presence 0.5 + frequency 0.3 over 512-id Zipf(1.1) histories",
    "C3": "C3: B=32, V=151936 f32, packed allow-mask (0.1%-30% allowed, runs 1-64), T 1.0 / top-p 0.9",
    "C4": "C4: spec verify, 16 seq x (4 drafts + 1) rows, V=151936 f32, T 0.8 / top-p 0.95",
    "C5": "C5: B=256, V=262144 bf16, top-p 0.9 over the full vocabulary, rep 1.05 over 1024-id histories",
}


def read_traffic(name):
    """HBM bytes per launch of the streaming kernel from the committed rocprofv3 counter
    summary (profiles/k_stream_<config>_traffic.txt, line 'traffic_bytes: N'), if present."""
    p = os.path.join(ROOT, "profiles", f"k_stream_{name}_traffic.txt")
    try:
        for line in open(p):
            if line.startswith("traffic_bytes:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def cpu_baseline(cfg, seconds):
    """The oracle (C restatement of the reference sampler) on this host's cores, over whole
    batches of the same workload until `seconds` have elapsed."""
    import numpy as np

    import oracle as O
    import workloads

    threads = max(1, min(os.cpu_count() or 1, 16))
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
                       f"{threads} threads")


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="C2", choices=sorted(WORKLOAD_DESC))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a device-to-device copy of 256 MiB (10 launches), the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--mask", action="store_true",
                    help="measure the allow-mask producer (include/bfi_mask.h) instead: a named "
                         "tool-call constraint over a synthetic 151,936-piece vocabulary")
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

    cfg = workloads.config(args.config, seed=args.seed)
    dev = torch.device("cuda:0")
    d = workloads.to_device(cfg, dev)
    smp = bfi_smp.Sampler(0)
    verify = "drafts" in cfg

    def step():
        if verify:
            smp.verify(d["logits"], cfg["rows_per_seq"], d["params"], d["drafts"], d["draft_len"], d["u_pairs"],
                       d["u_bonus"], d["out_accepted"], d["out_next"], d["hist"], d["hist_off"], d["mask"])
        else:
            smp.sample_rows(d["logits"], d["params"], d["u"], d["out"], d["hist"], d["hist_off"], d["mask"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Kernel durations come from HIP events recorded in the dispatch packets of every
    # PROFILE_EVERY-th step of the timed region: events on every step would add about 10 us
    # of event processing per step to the wall time.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if i % PROFILE_EVERY == 0:
            smp.set_profiling(True)
            step()
            smp.set_profiling(False)
        else:
            step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    stream_ms, select_ms, n = smp.profile()

    rows = cfg["B"]
    ms_step = el * 1e3 / args.steps
    value = rows * args.steps / el
    alg = workloads.algorithmic_bytes(cfg)
    k_us = stream_ms * 1e3 / max(n, 1)
    s_us = select_ms * 1e3 / max(n, 1)
    achieved = alg / (k_us * 1e-6) / 1e9
    traffic = read_traffic(args.config)
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
                   "seed": args.seed},
        "roofline": {
            "bound": "hbm",
            "kernel": "k_stream",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes": alg,
            "kernel_us": round(k_us, 3),
            "timed_launches": n,
        },
        "step_breakdown_us": {"k_stream": round(k_us, 3), "k_select": round(s_us, 3),
                              "wall": round(ms_step * 1e3, 3)},
        "step_hbm_gbs": round(alg / (ms_step * 1e-3) / 1e9, 1),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    smp.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
