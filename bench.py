#!/usr/bin/env python3
"""Benchmark of the MI355X token-selection path.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one strim_sample call over one batch of synthetic logits already resident
in HBM. The headline workload is configuration 2 (B=8, V=151,936 bf16, per-row
T / top-k / top-p, min-p 0.05, presence/frequency penalties over a 4,096-token history,
one uniform per row). Inputs rotate through a pool larger than 512 MB (twice the
256 MB Infinity Cache) so the streaming kernels read HBM, not the cache. The B=64
stress configuration (5) is reported beside it. Per-kernel durations come from HIP
events recorded on the launch stream over a second pass of the same steps.

Prints ONE JSON line on stdout; diagnostics go to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "strim-engine_amd"))

HBM_PEAK_GBS = 8000.0
METRIC = "µs/sample step at B=8,V=151,936 bf16; rows/s at B=64; HBM GB/s vs peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_pool_cfg2(torch, dev, n_sets, B, V, H, seed=2):
    """Distinct cfg2-shaped inputs: N(0, 2.5^2) + Zipf(1.1) rank bias over a permutation."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    perm = torch.from_numpy(rng.permutation(V)).to(dev)
    bias = torch.empty(V, device=dev)
    bias[perm] = -1.1 * torch.log(torch.arange(V, device=dev, dtype=torch.float32) + 1.0)
    xs, hs, ns = [], [], []
    perm_np = perm.cpu().numpy()
    for s in range(n_sets):
        x = torch.randn(B, V, device=dev, generator=g) * 2.5 + bias
        xs.append(x.to(torch.bfloat16).contiguous())
        r = rng.zipf(1.1, size=(B, H)).astype(np.int64) - 1
        hs.append(torch.from_numpy(perm_np[r % V].astype(np.int32)).to(dev))
        ns.append(torch.from_numpy(rng.random((B, 2), dtype=np.float32)).to(dev))
    return xs, hs, ns


def make_pool_cfg5(torch, dev, n_sets, B, V, H, seed=5):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    from strim_amd.ops import pack_mask

    xs, hs, ms = [], [], []
    for s in range(n_sets):
        x = torch.randn(B, V, device=dev, generator=g) * 2.0
        dom = torch.rand(B, device=dev, generator=g) < 0.3
        col = torch.randint(0, V, (B,), device=dev, generator=g)
        x[dom, col[dom]] = 20.0
        xs.append(x.to(torch.bfloat16).contiguous())
        hs.append(torch.randint(0, V, (B, H), device=dev, generator=g, dtype=torch.int32))
        ms.append(pack_mask(torch.rand(B, V, device=dev, generator=g) < 0.05).contiguous())
    return xs, hs, ms


def time_steps(torch, fn, n_sets, steps, warmup):
    for i in range(warmup):
        fn(i % n_sets)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i % n_sets)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def kernel_times(ctx, torch, fn, n_sets, steps):
    ctx.profile_begin(6 * steps + 16)
    for i in range(steps):
        fn(i % n_sets)
    prof = ctx.profile_end()
    return {k: (ms / n * 1e3 if n else 0.0, n) for k, (ms, n) in prof.items()}


def cpu_baseline_cfg2(seconds: float):
    """The oracle (a C port of the reference sampler, OpenMP over rows) on host cores,
    on the cfg2 workload, repeated for about `seconds`."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    from strim_amd import workloads as W

    O.build()
    w = W.cfg2()
    threads = min(os.cpu_count() or 1, 16)
    n = 0
    t0 = time.perf_counter()
    while True:
        O.sample(w["x"], w["params"], history=w["history"], history_len=w["history_len"],
                 noise_mode=O.NOISE_ICDF, noise=w["noise"], nthreads=threads)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    return {"value": round(el * 1e6 / n, 1), "unit": "us/step", "cores": threads,
            "kind": "port",
            "sample": f"cfg2 B=8 V=151936 (bf16 values as f32), {n} steps in {el:.1f}s, "
                      f"OpenMP over rows"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--pool-mb", type=float, default=600.0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b64", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the token "
              "selection shards over rows with no communication); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from strim_amd import _native as N
    from strim_amd import ops
    from strim_amd import workloads as W

    dev = torch.device("cuda:0")
    V, B, H = W.V_DEFAULT, 8, 4096
    per_set = B * V * 2 + B * H * 4 + B * 8
    n_sets = int(np.ceil(args.pool_mb * 2**20 / per_set))
    log(f"[bench] cfg2 pool: {n_sets} sets x {per_set / 2**20:.2f} MiB")
    xs, hs, ns = make_pool_cfg2(torch, dev, n_sets, B, V, H)
    params = W.cfg2()["params"]
    hl = torch.full((B,), H, dtype=torch.int32, device=dev)
    ctx = ops.Context(0, max_rows=64, max_vocab=V)
    out_ids = torch.empty(B, dtype=torch.int32, device=dev)
    out_st = torch.empty(B, dtype=torch.int32, device=dev)

    def step2(i):
        ctx.sample(xs[i], params, history=hs[i], history_len=hl, noise_mode=N.NOISE_ICDF,
                   noise=ns[i], out_ids=out_ids, out_status=out_st)

    ms2 = time_steps(torch, step2, n_sets, args.steps, args.warmup)
    st = out_st.cpu().numpy()
    assert (st == 0).all(), f"row status {st}"
    kt2 = kernel_times(ctx, torch, step2, n_sets, args.steps)
    bytes2 = W.algorithmic_bytes(B, V, 2, mask=False, H=H, noise_floats=2)
    stream_us = kt2["k_stream"][0]
    log(f"[bench] cfg2 {ms2 * 1e3:.2f} us/step; kernels (us/launch): "
        + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt2.items() if v[1]))
    del xs, hs, ns
    torch.cuda.empty_cache()

    # cfg3: grammar masks + T 0.8 + top-p 0.9 (the general path: scan, collect, finalize)
    w3 = W.cfg3()
    per3 = B * V * 2 + B * ((V + 31) // 32) * 4
    n3 = int(np.ceil(args.pool_mb * 2**20 / per3))
    g3 = torch.Generator(device=dev)
    g3.manual_seed(3)
    m3 = torch.from_numpy(w3["mask"].view(np.int32)).to(dev)
    x3 = [(torch.randn(B, V, device=dev, generator=g3) * 2.5).to(torch.bfloat16) for _ in range(n3)]
    n3s = [torch.from_numpy(np.random.default_rng(i).random((B, 2), dtype=np.float32)).to(dev)
           for i in range(n3)]

    def step3(i):
        ctx.sample(x3[i], w3["params"], mask=m3, noise_mode=N.NOISE_ICDF, noise=n3s[i],
                   out_ids=out_ids, out_status=out_st)

    ms3 = time_steps(torch, step3, n3, args.steps, args.warmup)
    st3 = out_st.cpu().numpy()
    assert (st3 == 0).all(), f"row status {st3}"
    kt3 = kernel_times(ctx, torch, step3, n3, args.steps)
    log(f"[bench] cfg3 {ms3 * 1e3:.2f} us/step; kernels (us/launch): "
        + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt3.items() if v[1]))
    del x3, n3s
    torch.cuda.empty_cache()

    result = {
        "metric": METRIC,
        "value": round(ms2 * 1e3, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms2, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 in, f32/f64 math",
        "data": "synthetic (seeded N(0,2.5^2)+Zipf bias logits, Zipf histories), rotating "
                f"{n_sets}-set pool > 512 MB",
        "config": {"workload": "cfg2: B=8 V=151936 bf16, per-row T{0.6,0.8,1.0} top-k{0,20,50} "
                               "top-p U[0.8,1], min-p 0.05, presence 0.5, frequency 0.3 over "
                               "4096-token history, icdf draw (one uniform per row)",
                   "B": B, "V": V, "history": H},
        "roofline": {"kernel": "k_stream", "bound": "hbm",
                     "achieved": round(bytes2 / (stream_us * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(bytes2 / (stream_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "bytes_per_launch": bytes2, "us_per_launch": round(stream_us, 3)},
        "kernel_us": {k: round(v[0], 3) for k, v in kt2.items() if v[1]},
        "cfg3": {"workload": "cfg3: B=8 bf16 + packed grammar masks (0.01-30% density), "
                             "T 0.8, top-p 0.9, icdf", "us_per_step": round(ms3 * 1e3, 3),
                 "kernel_us": {k: round(v[0], 3) for k, v in kt3.items() if v[1]}},
    }

    if not args.no_b64:
        B5, H5 = 64, 2048
        per5 = B5 * V * 2 + B5 * ((V + 31) // 32) * 4 + B5 * H5 * 4
        n5 = int(np.ceil(args.pool_mb * 2**20 / per5))
        log(f"[bench] cfg5 pool: {n5} sets x {per5 / 2**20:.2f} MiB")
        xs5, hs5, ms5 = make_pool_cfg5(torch, dev, n5, B5, V, H5)
        p5 = W.cfg5()["params"]
        hl5 = torch.full((B5,), H5, dtype=torch.int32, device=dev)
        o5 = torch.empty(B5, dtype=torch.int32, device=dev)
        s5 = torch.empty(B5, dtype=torch.int32, device=dev)
        pos = W.cfg5()["params"].copy()

        def step5(i):
            ctx.sample(xs5[i], p5, mask=ms5[i], history=hs5[i], history_len=hl5,
                       noise_mode=N.NOISE_ICDF, noise=None, out_ids=o5, out_status=s5)

        ms_5 = time_steps(torch, step5, n5, args.steps, args.warmup)
        st5 = s5.cpu().numpy()
        assert (st5 == 0).all(), f"row status {st5}"
        kt5 = kernel_times(ctx, torch, step5, n5, args.steps)
        bytes5 = W.algorithmic_bytes(B5, V, 2, mask=True, H=H5, noise_floats=0)
        us5 = kt5["k_stream"][0]
        log(f"[bench] cfg5 {ms_5 * 1e3:.2f} us/step; kernels (us/launch): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt5.items() if v[1]))
        result["b64"] = {
            "workload": "cfg5: B=64 bf16, 2048-token history, 5% masks, T 0.8, top-k 40, "
                        "top-p 0.95, min-p 0.02, Philox per row",
            "us_per_step": round(ms_5 * 1e3, 3),
            "rows_per_s": round(B5 / (ms_5 * 1e-3), 1),
            "roofline": {"kernel": "k_stream", "bound": "hbm",
                         "achieved": round(bytes5 / (us5 * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(bytes5 / (us5 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": bytes5, "us_per_launch": round(us5, 3)},
            "step_hbm_frac": round(bytes5 / (ms_5 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel_us": {k: round(v[0], 3) for k, v in kt5.items() if v[1]},
        }
        del xs5, hs5, ms5, pos
    ctx.close()

    if not args.no_cpu:
        log("[bench] cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline_cfg2(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
