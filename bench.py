#!/usr/bin/env python3
"""Benchmark of the MI355X token-selection path.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one strim_sample call over one batch of synthetic logits already resident in
HBM. The headline workload is the north-star chain (n1): B=8, V=151,936 bf16, presence
and frequency penalties over a 4,096-token history, packed grammar allow-masks, T 0.8,
top-p 0.9, one uniform per row (icdf draw). Inputs rotate through a pool larger than
512 MB (twice the 256 MB Infinity Cache), so the streaming kernel reads HBM.

Timing:
  value        the pool's steps captured once in a HIP graph (the way a decode loop
               launches a fixed step) and replayed at least 5 times and for at least
               1,000 steps (more when --steps asks): each replay's wall clock between two
               device synchronisations over its steps; `value` is the median over the
               replays and `steps` the number of steps timed. Host launch overhead is
               outside the measurement.
  kernel_us    per-kernel durations from HIP events bound to each dispatch, with the steps
               queued behind a bounded GPU sleep so they run back to back; the roofline
               uses the streaming kernel's average.
  eager_us     the same steps launched one by one from Python (host-bound reference).
Beside it: cfg3 (masks + top-p), cfg2 (heterogeneous rows with penalties and min-p), the
B=64 stress configuration (rows/s, roofline), the general-q verify (cfg4) and the
reference's one-hot verify (both graph-timed), a wide-nucleus row on the exact
resolution, grammar-mask production, the logits producer (final RMSNorm + lm_head
GEMV) alone and followed by the n1 chain, and the CPU oracle (a C port of the reference
sampler) single-threaded and on every host core.

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
    """Distinct cfg2-shaped inputs: N(0, 2.5^2) + Zipf(1.1) rank bias over a permutation,
    Zipf-distributed histories, one uniform per row."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    perm = torch.from_numpy(rng.permutation(V)).to(dev)
    bias = torch.empty(V, device=dev)
    bias[perm] = -1.1 * torch.log(torch.arange(V, device=dev, dtype=torch.float32) + 1.0)
    xs, hs, ns = [], [], []
    perm_np = perm.cpu().numpy()
    for _ in range(n_sets):
        x = torch.randn(B, V, device=dev, generator=g) * 2.5 + bias
        xs.append(x.to(torch.bfloat16).contiguous())
        r = rng.zipf(1.1, size=(B, H)).astype(np.int64) - 1
        hs.append(torch.from_numpy(perm_np[r % V].astype(np.int32)).to(dev))
        ns.append(torch.from_numpy(rng.random((B, 2), dtype=np.float32)).to(dev))
    return xs, hs, ns


def make_masks_cfg3(torch, x, hist=None, presence=0.5, frequency=0.3, T=0.8, P=0.9,
                    gen=None):
    """cfg3's allow masks for one pool set, built from that set's own logits (the
    workloads.py layout on the device): rows 0-3 clustered runs of 64 at densities
    0.01 / 1 / 10 / 30 %, rows 4-5 scattered at 0.01 / 1 %, row B-2 allows exactly one
    token, row B-1 masks the whole top-p nucleus of its own penalised logits at (T, P)
    and allows 30 % of the other tokens at random. `hist` gives the penalty histories
    (presence / frequency as the chain applies them); None for a chain without them.
    Returns packed int32 words [B, ceil(V/32)]."""
    from strim_amd.ops import pack_mask

    B, V = x.shape
    dev = x.device
    dens = [0.0001, 0.01, 0.10, 0.30]
    allowed = torch.zeros(B, V, dtype=torch.bool, device=dev)
    for r in range(B):
        d = dens[r % 4]
        n = max(1, int(round(d * V)))
        if (r // 4) % 2 == 0:  # clustered: seeded contiguous runs of 64
            run = 64
            starts = torch.randperm(V // run, device=dev, generator=gen)[: max(1, n // run)] * run
            idx = (starts[:, None] + torch.arange(run, device=dev)[None, :]).reshape(-1)
            allowed[r, idx] = True
        else:  # scattered
            allowed[r, torch.randperm(V, device=dev, generator=gen)[:n]] = True
    # one row allows exactly one token
    allowed[B - 2] = False
    allowed[B - 2, int(torch.randint(0, V, (1,), device=dev, generator=gen))] = True
    # one row's top-p nucleus (of its penalised logits at T, P) lies in masked tokens
    r = B - 1
    v = x[r].float()
    if hist is not None:
        c = torch.bincount(hist[r].long().clamp(0, V - 1), minlength=V)[:V].float()
        hit = c > 0
        v = torch.where(hit, (v - frequency * c) - presence, v)
    l = (v / T).double()
    order = torch.argsort(l, descending=True, stable=True)
    w = torch.exp(l[order] - l[order[0]])
    cum = torch.cumsum(w, 0) / w.sum()
    cut = int(torch.searchsorted(cum, torch.tensor([P], dtype=cum.dtype, device=dev))) + 1
    allowed[r] = torch.rand(V, device=dev, generator=gen) < 0.3
    allowed[r, order[:cut]] = False
    return pack_mask(allowed).contiguous()


def make_pool_n1(torch, dev, n_sets, B, V, H, seed=6, penalties=True):
    """The n1 (penalties=True) or cfg3 (False) pool: cfg2-shaped logits, histories and
    uniforms, each set with its own cfg3 masks made from its own penalised logits, so
    every set has an active one-token row and a row whose nucleus is masked."""
    xs, hs, ns = make_pool_cfg2(torch, dev, n_sets, B, V, H, seed=seed)
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1000)
    ms = [make_masks_cfg3(torch, xs[i], hs[i] if penalties else None, gen=g)
          for i in range(n_sets)]
    return xs, hs, ns, ms


def make_pool_cfg5(torch, dev, n_sets, B, V, H, seed=5):
    """cfg5-shaped inputs: 70 % rows N(0, 2^2), 30 % rows with one +20 logit; uniform
    2,048-token histories; 5 %-density allow masks."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    from strim_amd.ops import pack_mask

    xs, hs, ms = [], [], []
    for _ in range(n_sets):
        x = torch.randn(B, V, device=dev, generator=g) * 2.0
        dom = torch.rand(B, device=dev, generator=g) < 0.3
        col = torch.randint(0, V, (B,), device=dev, generator=g)
        x[dom, col[dom]] = 20.0
        xs.append(x.to(torch.bfloat16).contiguous())
        hs.append(torch.randint(0, V, (B, H), device=dev, generator=g, dtype=torch.int32))
        ms.append(pack_mask(torch.rand(B, V, device=dev, generator=g) < 0.05).contiguous())
    return xs, hs, ms


def make_pool_cfg4(torch, dev, n_sets, B, k, V, Vd, T=0.7, seed=4):
    """cfg4-shaped verify inputs: target [B,k+1,V] bf16 (cfg2-style logits), draft logits
    [B,k,Vd] bf16 biased toward the target, an ascending injective table, drafts drawn
    from q = softmax(draft / T)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    perm = torch.from_numpy(rng.permutation(V)).to(dev)
    bias = torch.empty(V, device=dev)
    bias[perm] = -1.1 * torch.log(torch.arange(V, device=dev, dtype=torch.float32) + 1.0)
    table = torch.from_numpy(np.sort(rng.choice(V, size=Vd, replace=False)).astype(np.int32)).to(dev)
    ts, ds, dr = [], [], []
    for _ in range(n_sets):
        t = (torch.randn(B, k + 1, V, device=dev, generator=g) * 2.5 + bias).to(torch.bfloat16)
        d = (0.5 * torch.randn(B, k, Vd, device=dev, generator=g) * 2.5
             + 0.8 * t[:, :k, :].float()[:, :, table.long()]).to(torch.bfloat16)
        q = torch.softmax(d.float() / T, dim=-1).reshape(B * k, Vd)
        pick = torch.multinomial(q, 1, generator=g).reshape(B, k)
        ts.append(t.contiguous())
        ds.append(d.contiguous())
        dr.append(table[pick].to(torch.int32).contiguous())
    return ts, ds, dr, table


MIN_TIMED_STEPS = 1000  # at least this many steps are timed, whatever --steps asks
MIN_REPLAYS = 5


def graph_median(torch, calls, steps, warmup):
    """Capture `calls` (one step each) into a HIP graph and replay it R times (at least
    MIN_REPLAYS, and at least max(steps, MIN_TIMED_STEPS) steps in all), each replay
    timed alone between two device synchronisations. Returns (median µs per step over
    the replays, steps timed, [µs per step of each replay])."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls[: min(3, len(calls))]:  # warm the launch path outside capture
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in calls:
            c()
    want = max(steps, MIN_TIMED_STEPS)
    reps = max(MIN_REPLAYS, (want + len(calls) - 1) // len(calls))
    for _ in range(max(1, warmup // len(calls))):
        g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        per.append((time.perf_counter() - t0) * 1e6 / len(calls))
    del g
    return float(np.median(per)), reps * len(calls), per


def kernel_times(torch, ctx, calls, steps, window=96, sleep_cycles=30_000_000):
    """Per-kernel average durations (µs) from HIP events around each launch, the steps
    queued behind a bounded GPU sleep so they execute back to back."""
    tot = {}
    done = 0
    while done < steps:
        n = min(window, steps - done)
        torch.cuda.synchronize()
        ctx.profile_begin(8 * n + 8)
        torch.cuda._sleep(sleep_cycles)
        for i in range(n):
            calls[(done + i) % len(calls)]()
        prof = ctx.profile_end()
        for k, (ms, cnt) in prof.items():
            a = tot.setdefault(k, [0.0, 0])
            a[0] += ms
            a[1] += cnt
        done += n
    return {k: (v[0] * 1e3 / v[1], v[1]) for k, v in tot.items() if v[1]}


def eager_us_per_step(torch, calls, steps):
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        calls[i % len(calls)]()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e6 / steps


GRAMMAR_ROWS = 8  # mask rows per launch (one per row of the B=8 configuration)


def _grammar_launch_us(torch, g, keys, steps):
    """µs per strim_grammar_masks launch: 32 launches captured in a HIP graph (the host's
    per-call cost stays out of the timing; each replay's launches carry their captured
    sequence numbers), replayed until about `steps` launches ran."""
    m = g.masks(keys)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(4):
            g.masks(keys, out=m)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    per = 32
    with torch.cuda.graph(graph):
        for _ in range(per):
            g.masks(keys, out=m)
    for _ in range(3):
        graph.replay()
    n = max(1, steps // per)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(n):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) * 1e3 / (n * per)


def grammar_mask_bench(torch, dev, args):
    """strim_grammar_masks at the configuration's width (V=151,936, 151,665 byte strings):
    8 rows per launch in a string's in-string state, where nearly every token walks all
    its bytes, for a JSON-string DFA (4 states: the walk reads an LDS copy of the table)
    and a JSON-object DFA (22 states: the walk reads the table through the caches).
    "produce" runs with the mask cache off (every launch walks the vocabulary once for the
    8 equal keys and writes the words to the 8 rows), "cached" with it on (every launch
    after the first copies the rows); "produce_distinct" walks 8 different states of the
    JSON-object DFA per launch."""
    from strim_amd import workloads as W
    from strim_amd.grammar import DeviceGrammar

    toks, skip = W.grammar_vocab()
    steps = 500
    res = {}
    nt_o, fl_o, s_o = W.json_object_dfa()
    for dfa, (nt, fl), state in (("json_string", W.json_string_dfa(), 1),
                                 ("json_object", (nt_o, fl_o), s_o)):
        keys = torch.full((GRAMMAR_ROWS,), state, dtype=torch.int32, device=dev)
        out = {}
        for name, cache in (("produce", 0), ("cached", 4 if dfa == "json_string" else 32)):
            g = DeviceGrammar(toks, W.V_DEFAULT, eos=W.GRAMMAR_EOS, skip=skip,
                              cache_slots=cache)
            g.set_dfa(nt, fl)
            out[name] = _grammar_launch_us(torch, g, keys, steps)
            g.close()
        if dfa == "json_object":
            con = [i for i in range(nt.shape[0]) if fl[i] & 2][:GRAMMAR_ROWS]
            kd = torch.tensor(con, dtype=torch.int32, device=dev)
            g = DeviceGrammar(toks, W.V_DEFAULT, eos=W.GRAMMAR_EOS, skip=skip, cache_slots=0)
            g.set_dfa(nt, fl)
            out["produce_distinct"] = _grammar_launch_us(torch, g, kd, steps)
            out["distinct_rows"] = len(con)
            g.close()
        res[dfa] = out
        log(f"[bench] grammar masks ({dfa}, {nt.shape[0]} states): produce "
            f"{out['produce']:.2f} us/launch, cached {out['cached']:.2f} us/launch "
            f"({GRAMMAR_ROWS} rows of one state)"
            + (f"; {out['distinct_rows']} distinct states produced "
               f"{out['produce_distinct']:.2f} us/launch" if "produce_distinct" in out else ""))
    words = (W.V_DEFAULT + 31) // 32
    # algorithmic bytes of a launch: each token's 16-byte head and 8-byte meta read once
    # (the 8 equal keys are walked once), the words of every row written
    launch_bytes = len(toks) * 24 + words * 4 * GRAMMAR_ROWS
    out = res["json_string"]
    gbs = launch_bytes / (out["produce"] * 1e-6) / 1e9
    oo = res["json_object"]
    return {"workload": f"strim_grammar_masks: {GRAMMAR_ROWS} rows x V=151936, 151665 byte "
                        "strings (mean 6.5 bytes), JSON-string DFA, in-string state",
            "produce_us_per_launch": round(out["produce"], 3),
            "cached_us_per_launch": round(out["cached"], 3),
            "roofline_produce": {"bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0,
                                 "unit": "GB/s", "frac": round(gbs / 8000.0, 4),
                                 "launch_bytes": launch_bytes},
            "json_object_dfa": {
                "workload": f"{GRAMMAR_ROWS} rows, 22-state JSON-object DFA "
                            "({\"name\":\"<string>\",\"age\":<integer>}), in-string state; "
                            "the table is walked through the caches",
                "produce_us_per_launch": round(oo["produce"], 3),
                "cached_us_per_launch": round(oo["cached"], 3),
                "produce_distinct_us_per_launch": round(oo["produce_distinct"], 3),
                "distinct_states": oo["distinct_rows"]}}


def cpu_baseline_grammar(seconds: float):
    """The reference's host mask production (the trie walk, restated in the oracle) for
    the same state, one thread, repeated for about `seconds`."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    from strim_amd import workloads as W

    O.build()
    toks, skip = W.grammar_vocab()
    nt, fl = W.json_string_dfa()
    o = O.GrammarOracle(toks, W.V_DEFAULT, W.GRAMMAR_EOS, skip)
    o.set_dfa(nt, fl)
    n = 0
    t0 = time.perf_counter()
    while True:
        o.mask(1)
        n += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    return {"value": round(el * 1e6 / n, 1), "unit": "us/row", "cores": 1, "kind": "port",
            "sample": f"trie walk of the in-string state, {n} rows in {el:.1f}s"}


# k_stream instantiation -> workload
# (dtype, aligned, history counts, mask, segments per thread, general rows)
STREAM_CASES = {"k_stream<1, true, 2, true, 1, true>": "n1",
                "k_stream<1, true, 2, false, 1, false>": "cfg2",
                "k_stream<1, true, 2, true, 4, false>": "cfg5",
                "k_stream<1, true, 0, true, 1, true>": "cfg3",
                "k_stream<1, true, 0, false, 1, true>": "cfg4"}
TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_bench_workloads.md"


def head_bench(torch, ops, dev, ctx, args, w1, m1, hl, B=8, K=5120):
    """The producer of the logits (final RMSNorm + dense bf16 lm_head, K=5120 hidden,
    V=151,936) on its own and followed by the n1 chain: graph-timed like the headline.
    The 1.56 GB weight matrix is read once per call, so it streams from HBM."""
    from strim_amd import workloads as W
    V = W.V_DEFAULT
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    x = (2.0 * torch.randn(B, K, device=dev, generator=g)).to(torch.bfloat16)
    nw = (1.0 + 0.1 * torch.randn(K, device=dev, generator=g)).to(torch.bfloat16)
    wt = (0.05 * torch.randn(V, K, device=dev, generator=g)).to(torch.bfloat16)
    xn = torch.empty(B, K, dtype=torch.bfloat16, device=dev)
    lg = torch.empty(B, V, dtype=torch.bfloat16, device=dev)
    head = lambda: ops.head_logits(x, wt, nw, out=lg, xn=xn)
    n = 20
    steps = max(200, args.steps // 4)
    ush, kh, _ = graph_median(torch, [head] * n, steps, n)
    hs = torch.from_numpy(w1["history"]).to(dev)
    ns = torch.from_numpy(w1["noise"]).to(dev)
    samp = ctx.bind_sample(lg, w1["params"], mask=m1, history=hs, history_len=hl, noise=ns)
    def step():
        head()
        samp()
    usc, kc, _ = graph_median(torch, [step] * n, steps, n)
    st = samp.out_status.cpu().numpy()
    assert (st == 0).all(), f"head chain status {st}"
    # greedy rows: the producer then strim_sample at T = 0, against the pick fused into
    # the producer's epilogue (strim_head_greedy), with and without the logits written
    pg = W.params_array(B, temperature=0.0)
    sg = ctx.bind_sample(lg, pg)
    def step_g():
        head()
        sg()
    usg, _, _ = graph_median(torch, [step_g] * n, steps, n)
    gid = torch.empty(B, dtype=torch.int32, device=dev)
    gst = torch.empty(B, dtype=torch.int32, device=dev)
    fused = lambda: ops.head_greedy(ctx, x, wt, nw, out_logits=lg, xn=xn, ids=gid, status=gst)
    fused_nl = lambda: ops.head_greedy(ctx, x, wt, nw, xn=xn, ids=gid, status=gst)
    usf, _, _ = graph_median(torch, [fused] * n, steps, n)
    usf_nl, _, _ = graph_median(torch, [fused_nl] * n, steps, n)
    assert torch.equal(gid, sg.out_ids) and (gst == 0).all(), "fused greedy differs"
    byt = V * K * 2 + B * V * 2 + B * K * 2 * 3 + K * 2
    flops = 2.0 * B * V * K
    log(f"[bench] head B={B} K={K} V={V}: {ush:.1f} us/call; head + n1 chain {usc:.1f} us/step; "
        f"greedy: head + sample {usg:.1f}, fused {usf:.1f} (no logits written {usf_nl:.1f}) "
        f"us/step")
    # the producer at B = 64 (four 16-row batch tiles per MFMA step)
    B64 = 64
    x64 = (2.0 * torch.randn(B64, K, device=dev, generator=g)).to(torch.bfloat16)
    xn64 = torch.empty(B64, K, dtype=torch.bfloat16, device=dev)
    lg64 = torch.empty(B64, V, dtype=torch.bfloat16, device=dev)
    head64 = lambda: ops.head_logits(x64, wt, nw, out=lg64, xn=xn64)
    us64, _, _ = graph_median(torch, [head64] * n, steps, n)
    byt64 = V * K * 2 + B64 * V * 2 + B64 * K * 2 * 3 + K * 2
    log(f"[bench] head B={B64}: {us64:.1f} us/call, "
        f"{byt64 / (us64 * 1e-6) / 1e9:.0f} GB/s, {2.0 * B64 * V * K / (us64 * 1e-6) / 1e12:.1f} TFLOP/s")
    del wt
    torch.cuda.empty_cache()
    return {
        "workload": f"final RMSNorm + dense bf16 lm_head: hidden [{B},{K}] x lm_head [{V},{K}] "
                    "-> bf16 logits (k_head_norm + k_head_gemv, MFMA 16x16x32 bf16)",
        "us_per_call": round(ush, 2), "steps": kh,
        "roofline": {"bound": "hbm", "achieved": round(byt / (ush * 1e-6) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(byt / (ush * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "bytes_per_call": int(byt), "kernel": "k_head_norm + k_head_gemv"},
        "mfma_tflops": round(flops / (ush * 1e-6) / 1e12, 2),
        "then_n1_chain_us_per_step": round(usc, 2),
        "sampler_share_us": round(usc - ush, 2),
        "greedy": {"head_then_sample_us_per_step": round(usg, 2),
                   "fused_us_per_step": round(usf, 2),
                   "fused_no_logits_us_per_step": round(usf_nl, 2),
                   "workload": f"B={B} greedy rows (T=0, no penalties, mask or filters): "
                               "strim_head_logits then strim_sample, against strim_head_greedy"},
        "b64": {"us_per_call": round(us64, 2),
                "roofline": {"bound": "hbm", "achieved": round(byt64 / (us64 * 1e-6) / 1e9, 1),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(byt64 / (us64 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             "bytes_per_call": int(byt64)},
                "mfma_tflops": round(2.0 * B64 * V * K / (us64 * 1e-6) / 1e12, 2)},
    }


def measured_traffic():
    """HBM bytes per launch of k_stream per workload, from the committed rocprofv3 counter
    summary (lines `traffic <kernel> <workload> <bytes>`); {} when absent."""
    out = {}
    if TRAFFIC_FILE.exists():
        for line in TRAFFIC_FILE.read_text().splitlines():
            f = line.strip().strip("`").split()
            if len(f) == 4 and f[0] == "traffic" and f[3].isdigit():
                out[(f[1], f[2])] = int(f[3])
    return out


def roofline(bytes_per_launch, us, traffic=None):
    gbs = bytes_per_launch / (us * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "k_stream",
            "bytes_per_launch": int(bytes_per_launch), "us_per_launch": round(us, 3)}


def _kname(n):
    import re
    return re.sub(r"\(.*", "", n).replace("strim::", "").replace("void ", "").strip()


def summarize(d):
    """Markdown summary of a profile directory made by the commands it prints: kernel
    trace statistics of the bench (d/trace), and FETCH_SIZE / WRITE_SIZE per dispatch of a
    counter pass (d/fetch, d/write) scaled by the 256 MiB copy's counters."""
    import csv
    import glob
    d = Path(d)
    print("## Kernel trace (rocprofv3 --kernel-trace --stats)\n")
    print("| kernel | calls | avg us | min us | max us |\n|---|---|---|---|---|")
    for f in glob.glob(str(d / "trace" / "*kernel_stats.csv")):
        for r in csv.DictReader(open(f)):
            if "strim::" in r["Name"]:
                print(f"| {_kname(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                      f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} |")
    for f in glob.glob(str(d / "trace" / "*kernel_trace.csv")):
        rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Start_Timestamp"]))
        acc, case, pending = {}, None, {}
        for r in rows:
            if "strim::" not in r["Kernel_Name"]:
                continue
            k = _kname(r["Kernel_Name"])
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            if k == "k_qprep":  # runs before its call's k_stream
                pending.setdefault(k, []).append(us)
                continue
            if k.startswith("k_head"):
                case = "head"
            if k.startswith("k_stream"):
                case = STREAM_CASES.get(k, k)
                for kk, v in pending.items():
                    acc.setdefault((kk, case), []).extend(v)
                pending = {}
            # grammar masks: the cache-off grammar comes first; the cached one's set_dfa
            # (its k_gclear) starts the cached launches
            if k == "k_gclear":
                case = "grammar cached"
            elif k == "k_gmask" and not str(case).startswith("grammar"):
                case = "grammar produce"
            kk = "k_stream" if k.startswith("k_stream") else k
            acc.setdefault((kk, case), []).append(us)
        acc = {key: v for key, v in acc.items() if v}
        print("\nThe same trace per workload (a kernel belongs to the k_stream variant it "
              "follows; k_gmask to the grammar-mask timings, "
              "cache off, then cache on):\n")
        print("| kernel | workload | calls | avg us | median us |\n|---|---|---|---|---|")
        for (k, c), v in sorted(acc.items(), key=lambda t: (str(t[0][1]), t[0][0])):
            v = sorted(v)
            print(f"| {k} | {c} | {len(v)} | {sum(v) / len(v):.2f} | {v[len(v) // 2]:.2f} |")
    per = {}
    scale = {}
    for cn in ("FETCH_SIZE", "WRITE_SIZE"):
        sub = "fetch" if cn == "FETCH_SIZE" else "write"
        for f in glob.glob(str(d / sub / "*counter_collection.csv")):
            rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Dispatch_Id"]))
            case, pend, gm = None, [], False
            for r in rows:
                k = _kname(r["Kernel_Name"])
                v = float(r["Counter_Value"])
                # grammar masks: cache off first; a table install (k_gclear) after mask
                # launches starts the cached ones
                if k == "k_gclear":
                    case = "grammar cached" if gm else "grammar produce"
                    continue
                if k == "k_gmask":
                    gm = True
                    if not str(case).startswith("grammar"):
                        case = "grammar produce"
                if k == "k_qprep":  # runs before its call's k_stream
                    pend.append((k, v))
                    continue
                if k.startswith("k_stream"):
                    case = STREAM_CASES.get(k, k)
                    for kk, vv in pend:
                        per.setdefault((kk, case, cn), []).append(vv)
                    pend = []
                if k.startswith("k_head"):
                    case = "head"
                if "copyBuffer" in k and int(r["Grid_Size"]) >= 131072:
                    scale[cn] = 256 * 1024 / v  # KiB moved / KiB counted
                if "strim::" in r["Kernel_Name"]:
                    kk = k.split("<")[0] if k.startswith(("k_stream", "k_head")) else k
                    per.setdefault((kk, case, cn), []).append(v)
    print("\n## HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)\n")
    print(f"Calibration: a 256 MiB device copy reads FETCH_SIZE x {scale.get('FETCH_SIZE', 0):.3f} "
          f"and writes WRITE_SIZE x {scale.get('WRITE_SIZE', 0):.3f} KiB; the factors scale "
          "the counters below to bytes.\n")
    print("| kernel | workload | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | bytes/launch |")
    print("|---|---|---|---|---|---|")
    keys = sorted({(k, c) for k, c, _ in per})
    lines = []
    for k, c in keys:
        fe = per.get((k, c, "FETCH_SIZE"), [0.0])
        wr = per.get((k, c, "WRITE_SIZE"), [0.0])
        fa, wa = sum(fe) / len(fe), sum(wr) / len(wr)
        b = int((fa * scale.get("FETCH_SIZE", 1.0) + wa * scale.get("WRITE_SIZE", 1.0)) * 1024)
        print(f"| {k} | {c} | {len(fe)} | {fa:.0f} | {wa:.0f} | {b} |")
        lines.append(f"traffic {k} {c} {b}")
    print("\nMachine-readable (bench.py reads these lines):\n")
    for ln in lines:
        print(f"    {ln}")
    # any other counter pass (d/<name>/*counter_collection.csv): per-kernel averages
    for sub in sorted(p for p in d.iterdir() if p.is_dir() and p.name not in
                      ("trace", "fetch", "write")):
        vals = {}
        for f in glob.glob(str(sub / "*counter_collection.csv")):
            for r in csv.DictReader(open(f)):
                if "strim::" in r["Kernel_Name"]:
                    key = (_kname(r["Kernel_Name"]), r["Counter_Name"])
                    vals.setdefault(key, []).append(float(r["Counter_Value"]))
        if not vals:
            continue
        names = sorted({c for _, c in vals})
        print(f"\n## Counters per dispatch ({sub.name}: rocprofv3 --pmc {' '.join(names)})\n")
        print("| kernel | dispatches | " + " | ".join(names) + " |")
        print("|---|---|" + "---|" * len(names))
        for k in sorted({k for k, _ in vals}):
            n = len(vals.get((k, names[0]), []))
            cells = [f"{sum(v) / len(v):.4g}" if (v := vals.get((k, c))) else "" for c in names]
            print(f"| {k} | {n} | " + " | ".join(cells) + " |")


def pmc_pass(torch, ops, W, dev, steps, pool_mb):
    """A short eager run for hardware-counter passes: `steps` steps of n1, cfg3, cfg2,
    cfg5 and the cfg4 verify over pools of distinct inputs, then one copy of 256 MiB
    (read 256 MiB + write 256 MiB) to scale FETCH_SIZE / WRITE_SIZE."""
    V, B, H = W.V_DEFAULT, 8, 4096
    ctx = ops.Context(0, max_rows=64, max_vocab=V)
    hl = torch.full((B,), H, dtype=torch.int32, device=dev)

    def run(calls):
        for i in range(steps):
            calls[i % len(calls)]()
        torch.cuda.synchronize()

    n2 = int(np.ceil(pool_mb * 2**20 / (B * V * 2 + B * H * 4 + B * ((V + 31) // 32) * 4)))
    w1, w3 = W.n1(), W.cfg3()
    # the same pools as the timed lines: every set carries masks made from its own logits
    xs, hs, ns, ms = make_pool_n1(torch, dev, n2, B, V, H, seed=6)
    run([ctx.bind_sample(xs[i], w1["params"], mask=ms[i], history=hs[i], history_len=hl,
                         noise=ns[i]) for i in range(n2)])
    del xs, hs, ns, ms
    xs, hs, ns, ms = make_pool_n1(torch, dev, n2, B, V, 1, seed=3, penalties=False)
    run([ctx.bind_sample(xs[i], w3["params"], mask=ms[i], noise=ns[i]) for i in range(n2)])
    del xs, hs, ns, ms
    xs, hs, ns = make_pool_cfg2(torch, dev, n2, B, V, H, seed=2)
    run([ctx.bind_sample(xs[i], W.cfg2()["params"], history=hs[i], history_len=hl,
                         noise=ns[i]) for i in range(n2)])
    del xs, hs, ns
    n5 = int(np.ceil(pool_mb * 2**20 / (64 * V * 2 + 64 * 4748 * 4 + 64 * 2048 * 4)))
    xs5, hs5, ms5 = make_pool_cfg5(torch, dev, n5, 64, V, 2048)
    hl5 = torch.full((64,), 2048, dtype=torch.int32, device=dev)
    p5 = W.cfg5()["params"]
    run([ctx.bind_sample(xs5[i], p5, mask=ms5[i], history=hs5[i], history_len=hl5)
         for i in range(n5)])
    del xs5, hs5, ms5
    B4, K4, VD4 = 4, 3, W.VD_DEFAULT
    n4 = int(np.ceil(pool_mb * 2**20 / (B4 * (K4 + 1) * V * 2 + B4 * K4 * VD4 * 2)))
    ts4, ds4, dr4, tab4 = make_pool_cfg4(torch, dev, n4, B4, K4, V, VD4)
    p4 = W.params_array(B4, temperature=0.7, seed=np.arange(B4, dtype=np.uint64) + 40,
                        position=3)
    run([ctx.bind_verify(ts4[i], dr4[i], p4, draft_logits=ds4[i], draft_to_full=tab4,
                         noise_mode=1) for i in range(n4)])
    del ts4, ds4, dr4
    # the logits producer (B=8, K=5120, V=151,936): a few calls over the 1.56 GB weights
    K = 5120
    x = torch.randn(B, K, device=dev).to(torch.bfloat16)
    nw = torch.ones(K, device=dev).to(torch.bfloat16)
    wt = (0.05 * torch.randn(V, K, device=dev)).to(torch.bfloat16)
    for _ in range(3):
        ops.head_logits(x, wt, nw)
    torch.cuda.synchronize()
    del wt
    # grammar masks (the JSON-string DFA's in-string state, 8 rows of one state and 8 of
    # distinct JSON-object states): with the mask cache off, then on
    from strim_amd.grammar import DeviceGrammar
    toks, skip = W.grammar_vocab()
    nt_s, fl_s = W.json_string_dfa()
    nt_o, fl_o, _ = W.json_object_dfa()
    con = [i for i in range(nt_o.shape[0]) if fl_o[i] & 2][:GRAMMAR_ROWS]
    for cache in (0, 4):
        for nt, fl, keys in ((nt_s, fl_s, [1] * GRAMMAR_ROWS), (nt_o, fl_o, con)):
            g = DeviceGrammar(toks, V, eos=W.GRAMMAR_EOS, skip=skip, cache_slots=cache)
            g.set_dfa(nt, fl)
            kd = torch.tensor(keys, dtype=torch.int32, device=dev)
            for _ in range(steps):
                g.masks(kd)
            torch.cuda.synchronize()
            g.close()
    src = torch.empty(256 * 2**20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    ctx.close()
    print(f"pmc pass: {steps} steps each of n1, cfg3, cfg2, cfg5 and cfg4, 3 logits-producer "
          f"calls, {steps} grammar-mask launches per case, one 256 MiB copy",
          flush=True)


def host_cpu():
    """The host's logical CPU count and model name (for the CPU baseline)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return os.cpu_count() or 1, model


def cpu_baseline_n1(seconds: float):
    """The oracle (a C port of the reference sampler) on the north-star chain's own
    inputs, single-threaded and on every host core (OpenMP over rows), each repeated for
    about `seconds`."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O
    from strim_amd import workloads as W

    O.build()
    w = W.n1()
    nproc, model = host_cpu()
    out = {}
    for name, threads in (("single", 1), ("all", nproc)):
        n = 0
        t0 = time.perf_counter()
        while True:
            O.sample(w["x"], w["params"], mask=w["mask"], history=w["history"],
                     history_len=w["history_len"], noise_mode=O.NOISE_ICDF, noise=w["noise"],
                     nthreads=threads)
            n += 1
            if time.perf_counter() - t0 >= seconds:
                break
        out[name] = ((time.perf_counter() - t0) * 1e6 / n, n, threads)
    us1, n1s, _ = out["single"]
    usa, nas, th = out["all"]
    return {"value": round(usa, 1), "unit": "us/step", "cores": th, "kind": "port",
            "single_thread_us_per_step": round(us1, 1), "nproc": nproc, "cpu_model": model,
            "sample": f"n1 B=8 V=151936 (bf16 values as f32) with the bench's masks, 4096-id "
                      f"histories and uniforms: {nas} steps on {th} threads (OpenMP over rows), "
                      f"{n1s} steps on 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000,
                    help=f"steps to time per workload (at least {MIN_TIMED_STEPS} are timed)")
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--pool-mb", type=float, default=600.0)
    ap.add_argument("--cpu-seconds", type=float, default=5.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-b64", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the cfg2, cfg3, verify, wide-nucleus and grammar-mask timings")
    ap.add_argument("--summarize", metavar="DIR",
                    help="print the markdown summary of a profile directory (trace/, fetch/, "
                         "write/ as made by the commands in profiles/) and exit")
    ap.add_argument("--pmc-pass", type=int, default=0, metavar="N",
                    help="profiling pass for rocprofv3 counters: N eager steps of each "
                         "workload over a pool, then a 256 MiB device copy (the calibration "
                         "kernel for FETCH_SIZE / WRITE_SIZE); prints a summary line only")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: every box here has one GPU, and this path shards "
              "over rows with no communication (see the sharding design); run --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from strim_amd import ops
    from strim_amd import workloads as W

    dev = torch.device("cuda:0")
    if args.pmc_pass:
        pmc_pass(torch, ops, W, dev, args.pmc_pass, args.pool_mb)
        return
    traffic = measured_traffic()
    V, B, H = W.V_DEFAULT, 8, 4096
    ctx = ops.Context(0, max_rows=64, max_vocab=V)

    # ---- headline: the north-star chain (penalties + grammar masks + top-p) ----------
    w1 = W.n1()
    per_set = B * V * 2 + B * ((V + 31) // 32) * 4 + B * H * 4 + B * 8
    n_sets = int(np.ceil(args.pool_mb * 2**20 / per_set))
    log(f"[bench] n1 pool: {n_sets} sets x {per_set / 2**20:.2f} MiB")
    # every set has its own masks, made from its own penalised logits: the one-token row
    # and the masked-nucleus row are active in every step
    xs, hs, ns, ms = make_pool_n1(torch, dev, n_sets, B, V, H, seed=6)
    hl = torch.full((B,), H, dtype=torch.int32, device=dev)
    calls = [ctx.bind_sample(xs[i], w1["params"], mask=ms[i], history=hs[i], history_len=hl,
                             noise=ns[i]) for i in range(n_sets)]
    for i in range(args.warmup):
        calls[i % n_sets]()
    torch.cuda.synchronize()
    eager = [c.out_ids.clone() for c in calls[:4]]
    us1, k1, per1 = graph_median(torch, calls, args.steps, args.warmup)
    # the graph replays must reproduce the eager results
    for c, e in zip(calls[:4], eager):
        assert torch.equal(c.out_ids, e), "graph replay differs from eager launch"
    st = torch.stack([c.out_status for c in calls]).cpu().numpy()
    assert (st == 0).all(), f"row status {st}"
    kt1 = kernel_times(torch, ctx, calls, min(max(args.steps, 480), 960))
    eg1 = eager_us_per_step(torch, calls, 500)
    bytes1 = W.algorithmic_bytes(B, V, 2, mask=True, H=H, noise_floats=2)
    log(f"[bench] n1 graph {us1:.2f} us/step median of {len(per1)} replays (eager {eg1:.2f}); "
        "kernels (us): " + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt1.items()))
    m1 = ms[0]  # kept for the logits-producer line
    del xs, hs, ns, ms, calls
    torch.cuda.empty_cache()

    result = {
        "metric": METRIC,
        "value": round(us1, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": k1,
        "steps_requested": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us1 * 1e-3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 logits; f32 processing, f64 decisions",
        "data": f"synthetic (seeded N(0,2.5^2)+Zipf bias logits, Zipf histories, cfg3 "
                f"grammar masks made per set from its own penalised logits), rotating "
                f"{n_sets}-set pool > 512 MB",
        "config": {"workload": "n1 north-star chain: B=8 V=151936 bf16, presence 0.5 + "
                               "frequency 0.3 over a 4096-id history, packed grammar masks "
                               "(0.01-30% density, clustered and scattered, a one-token row, "
                               "a row whose top-p nucleus is masked; every pool set's masks "
                               "made from its own logits), T 0.8, top-p 0.9, icdf draw",
                   "B": B, "V": V, "history": H,
                   "timing": f"hip-graph replay, median of {len(per1)} replays "
                             f"({k1} steps timed, at least {MIN_TIMED_STEPS})"},
        "roofline": roofline(bytes1, kt1["k_stream"][0], traffic.get(("k_stream", "n1"))),
        "kernel_us": {k: round(v[0], 3) for k, v in kt1.items()},
        "replay_us_per_step": [round(x, 3) for x in per1],
        "eager_us_per_step": round(eg1, 3),
    }

    if not args.no_extra:
        # ---- cfg3: masks + top-p, no penalties ----------------------------------------
        w3 = W.cfg3()
        n3 = int(np.ceil(args.pool_mb * 2**20 / (B * V * 2 + B * ((V + 31) // 32) * 4)))
        xs3, _, ns3, ms3 = make_pool_n1(torch, dev, n3, B, V, 1, seed=3, penalties=False)
        calls3 = [ctx.bind_sample(xs3[i], w3["params"], mask=ms3[i], noise=ns3[i])
                  for i in range(n3)]
        us3, k3, per3 = graph_median(torch, calls3, args.steps, 20)
        kt3 = kernel_times(torch, ctx, calls3, 480)
        log(f"[bench] cfg3 graph {us3:.2f} us/step; kernels (us): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt3.items()))
        result["cfg3"] = {
            "workload": "cfg3: B=8 bf16 + packed allow masks (0.01-30% density, clustered and "
                        "scattered, a one-token row, a row whose nucleus is masked; every "
                        "pool set's masks made from its own logits), T 0.8, top-p 0.9, icdf",
            "us_per_step": round(us3, 3), "steps": k3,
            "roofline": roofline(W.algorithmic_bytes(B, V, 2, mask=True, noise_floats=2),
                                 kt3["k_stream"][0], traffic.get(("k_stream", "cfg3"))),
            "kernel_us": {k: round(v[0], 3) for k, v in kt3.items()}}
        del xs3, ns3, ms3, calls3
        # ---- cfg2: heterogeneous rows, penalties, min-p -------------------------------
        w2 = W.cfg2()
        n2 = int(np.ceil(args.pool_mb * 2**20 / per_set))
        xs2, hs2, ns2 = make_pool_cfg2(torch, dev, n2, B, V, H)
        calls2 = [ctx.bind_sample(xs2[i], w2["params"], history=hs2[i], history_len=hl,
                                  noise=ns2[i]) for i in range(n2)]
        us2, k2, per2 = graph_median(torch, calls2, args.steps, 20)
        kt2 = kernel_times(torch, ctx, calls2, 480)
        log(f"[bench] cfg2 graph {us2:.2f} us/step; kernels (us): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt2.items()))
        result["cfg2"] = {
            "workload": "cfg2: B=8 V=151936 bf16, per-row T{0.6,0.8,1.0} top-k{0,20,50} "
                        "top-p U[0.8,1], min-p 0.05, presence 0.5, frequency 0.3 over "
                        "4096-token history, icdf draw",
            "us_per_step": round(us2, 3), "steps": k2,
            "roofline": roofline(W.algorithmic_bytes(B, V, 2, mask=False, H=H, noise_floats=2),
                                 kt2["k_stream"][0], traffic.get(("k_stream", "cfg2"))),
            "kernel_us": {k: round(v[0], 3) for k, v in kt2.items()}}
        del xs2, hs2, ns2, calls2
        torch.cuda.empty_cache()

    if not args.no_b64:
        # ---- cfg5: B=64 stress ----------------------------------------------------------
        B5, H5 = 64, 2048
        per5 = B5 * V * 2 + B5 * ((V + 31) // 32) * 4 + B5 * H5 * 4
        n5 = int(np.ceil(args.pool_mb * 2**20 / per5))
        log(f"[bench] cfg5 pool: {n5} sets x {per5 / 2**20:.2f} MiB")
        xs5, hs5, ms5 = make_pool_cfg5(torch, dev, n5, B5, V, H5)
        p5 = W.cfg5()["params"]
        hl5 = torch.full((B5,), H5, dtype=torch.int32, device=dev)
        calls5 = [ctx.bind_sample(xs5[i], p5, mask=ms5[i], history=hs5[i], history_len=hl5)
                  for i in range(n5)]
        for i in range(min(args.warmup, 50)):
            calls5[i % n5]()
        us5, k5, per5l = graph_median(torch, calls5, args.steps, 50)
        st5 = torch.stack([c.out_status for c in calls5]).cpu().numpy()
        assert (st5 == 0).all(), f"row status {st5}"
        kt5 = kernel_times(torch, ctx, calls5, 480)
        bytes5 = W.algorithmic_bytes(B5, V, 2, mask=True, H=H5, noise_floats=0)
        log(f"[bench] cfg5 graph {us5:.2f} us/step; kernels (us): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt5.items()))
        result["b64"] = {
            "workload": "cfg5: B=64 bf16, 2048-token history (presence 0.5, frequency 0.3), "
                        "5% masks, T 0.8, top-k 40, top-p 0.95, min-p 0.02, Philox per row",
            "us_per_step": round(us5, 3),
            "rows_per_s": round(B5 / (us5 * 1e-6), 1),
            "steps": k5,
            "roofline": roofline(bytes5, kt5["k_stream"][0], traffic.get(("k_stream", "cfg5"))),
            "step_hbm_frac": round(bytes5 / (us5 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "kernel_us": {k: round(v[0], 3) for k, v in kt5.items()},
        }
        del xs5, hs5, ms5, calls5
        torch.cuda.empty_cache()

    if not args.no_extra:
        # ---- cfg4: general-q verify (graph) ----------------------------------------------
        B4, K4, VD4 = 4, 3, W.VD_DEFAULT
        n4 = int(np.ceil(args.pool_mb * 2**20 / (B4 * (K4 + 1) * V * 2 + B4 * K4 * VD4 * 2)))
        ts4, ds4, dr4, tab4 = make_pool_cfg4(torch, dev, n4, B4, K4, V, VD4)
        p4 = W.params_array(B4, temperature=0.7, seed=np.arange(B4, dtype=np.uint64) + 40,
                            position=3)
        calls4 = [ctx.bind_verify(ts4[i], dr4[i], p4, draft_logits=ds4[i], draft_to_full=tab4,
                                  noise_mode=1) for i in range(n4)]
        for c in calls4[:4]:
            c()
        torch.cuda.synchronize()
        us4, k4, _ = graph_median(torch, calls4, args.steps, 20)
        st4 = torch.stack([c.status for c in calls4]).cpu().numpy()
        assert (st4 == 0).all(), f"verify status {st4}"
        kt4 = kernel_times(torch, ctx, calls4, 192, window=32)
        # the step's algorithmic bytes: target rows, draft logits, the index table, and per
        # sequence its params, drafts and outputs (the k_stream launch reads all of the
        # inputs: its extra workgroups take the draft logits and the table)
        bytes4 = (B4 * (K4 + 1) * V * 2 + B4 * K4 * VD4 * 2 + VD4 * 4
                  + B4 * (48 + 4 * K4 + 8))
        log(f"[bench] cfg4 graph {us4:.2f} us/step; kernels (us): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt4.items()))
        result["cfg4"] = {
            "workload": "cfg4: general-q verify B=4 k=3 V=151936 bf16, draft logits "
                        "[4,3,32768] bf16 + ascending table, T 0.7, Philox Gumbel",
            "us_per_step": round(us4, 3), "steps": k4,
            "roofline": roofline(bytes4, kt4["k_stream"][0], traffic.get(("k_stream", "cfg4"))),
            "kernel_us": {k: round(v[0], 3) for k, v in kt4.items()}}
        # ---- the reference's verify: one-hot drafts, Gumbel noise (graph) -----------------
        calls4o = [ctx.bind_verify(ts4[i], dr4[i], p4, noise_mode=1) for i in range(n4)]
        for c in calls4o[:4]:
            c()
        torch.cuda.synchronize()
        us4o, k4o, _ = graph_median(torch, calls4o, args.steps, 20)
        kt4o = kernel_times(torch, ctx, calls4o, 192, window=32)
        log(f"[bench] one-hot verify graph {us4o:.2f} us/step; kernels (us): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in kt4o.items()))
        result["verify_onehot"] = {
            "workload": "SpecSampling.verify as the reference runs it: B=4 k=3 V=151936 bf16 "
                        "target rows, one-hot drafts, T 0.7, no filter, Philox Gumbel noise",
            "us_per_step": round(us4o, 3), "steps": k4o,
            "kernel_us": {k: round(v[0], 3) for k, v in kt4o.items()}}
        del ts4, ds4, dr4, calls4, calls4o
        torch.cuda.empty_cache()
        # ---- wide nuclei: rows whose kept set is wider than the chunks' candidates ----
        # B=8 rows of N(0,1) logits at T 1.0: seven with top-p 0.95 (a nucleus of tens of
        # thousands of tokens) and one unfiltered (its icdf draw ranges over the whole
        # vocabulary); a rotating pool, so the logits stream from HBM
        nwd = int(np.ceil(args.pool_mb * 2**20 / (B * V * 2)))
        gw = torch.Generator(device=dev)
        gw.manual_seed(21)
        xws = [torch.randn(B, V, device=dev, generator=gw).to(torch.bfloat16).contiguous()
               for _ in range(nwd)]
        nws = [torch.rand(B, 2, device=dev, generator=gw) for _ in range(nwd)]
        pw = W.params_array(B, temperature=1.0, top_p=[0.95] * (B - 1) + [1.0],
                            seed=np.arange(B, dtype=np.uint64) + 90, position=17)
        callsw = [ctx.bind_sample(xws[i], pw, noise=nws[i]) for i in range(nwd)]
        for c in callsw[:2]:
            c()
        torch.cuda.synchronize()
        usw, kw, _ = graph_median(torch, callsw, min(args.steps, MIN_TIMED_STEPS), 2)
        stw = torch.stack([c.out_status for c in callsw]).cpu().numpy()
        assert (stw == 0).all(), f"wide-nucleus status {stw}"
        ktw = kernel_times(torch, ctx, callsw, 96, window=16)
        log(f"[bench] wide nuclei graph {usw:.2f} us/step; kernels (us): "
            + ", ".join(f"{k}={v[0]:.2f}" for k, v in ktw.items()))
        result["wide_nucleus"] = {
            "workload": "B=8 V=151936 bf16 N(0,1) logits, T 1.0: 7 rows top-p 0.95 (nuclei of "
                        "tens of thousands of tokens) and 1 unfiltered row, icdf draw; "
                        f"rotating {nwd}-set pool > 512 MB",
            "us_per_step": round(usw, 3), "steps": kw,
            "kernel_us": {k: round(v[0], 3) for k, v in ktw.items()}}
        del xws, nws, callsw
        torch.cuda.empty_cache()
        result["head"] = head_bench(torch, ops, dev, ctx, args, w1, m1, hl)
        result["grammar_masks"] = grammar_mask_bench(torch, dev, args)
    ctx.close()

    if not args.no_cpu:
        log("[bench] cpu baseline (oracle) ...")
        result["cpu_baseline"] = cpu_baseline_n1(args.cpu_seconds)
        if "grammar_masks" in result:
            result["grammar_masks"]["cpu_baseline"] = cpu_baseline_grammar(2.0)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
