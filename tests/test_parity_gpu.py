"""GPU parity: the HIP path against the CPU oracle on identical seeded inputs.

Full-size cases use the benchmark configurations; the sweep covers small and ragged
shapes, ties, masks, penalties, both noise modes, the Sampler flags and error rows.
"""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import (check_sample, check_verify, dev, dev_logits, host_logits, run_sample,
                      run_verify)
from strim_amd import ops
from strim_amd import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


# ------------------------------------------------------------ small sweep ----
def _sweep_case(rng, V, B):
    x = rng.normal(0, rng.choice([0.5, 2.0, 4.0]), size=(B, V)).astype(np.float32)
    if rng.random() < 0.3:  # heavy exact ties
        x = (rng.integers(-4, 4, size=(B, V)) * 0.5).astype(np.float32)
    allowed = None
    if rng.random() < 0.5:
        allowed = rng.random((B, V)) < rng.choice([0.01, 0.3, 0.9])
        for r in range(B):
            if not allowed[r].any():
                allowed[r, rng.integers(0, V)] = True
    H = int(rng.choice([0, 0, 8, 64]))
    hist = rng.integers(-2, V + 2, size=(B, H)).astype(np.int32) if H else None
    hl = rng.integers(0, H + 1, size=B).astype(np.int32) if H else None
    p = O.make_params(
        B, temperature=rng.choice([0.0, -0.5, 0.5, 0.8, 1.0, 1.5], size=B),
        top_k=rng.choice([0, 0, 1, 5, 40, V, V + 3], size=B),
        top_p=rng.choice([1.0, 0.95, 0.8, 0.3], size=B),
        min_p=rng.choice([0.0, 0.0, 0.02, 0.2], size=B),
        repetition_penalty=rng.choice([1.0, 1.2], size=B),
        presence_penalty=rng.choice([0.0, 0.4], size=B),
        frequency_penalty=rng.choice([0.0, 0.2], size=B),
        flags=rng.choice([0, 0, 1, 7], size=B),
        seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
        position=rng.integers(0, 1000, size=B).astype(np.uint64))
    mask = None if allowed is None else W.pack_mask(allowed)
    return x, p, mask, hist, hl


@pytest.mark.parametrize("V", [1, 7, 64, 1000, 4096, 4097, 9001, 40000])
def test_sweep_small(ctx, V):
    rng = np.random.default_rng(1000 + V)
    for it in range(6):
        B = int(rng.choice([1, 3, 8, 16]))
        x, p, mask, hist, hl = _sweep_case(rng, V, B)
        for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
            for injected in (False, True):
                noise = None
                if injected:
                    n = (V + 1) if mode == O.NOISE_GUMBEL else 2
                    noise = rng.random((B, n), dtype=np.float32)
                say(f"sweep V={V} it={it} B={B} mode={mode} injected={injected}")
                dt = "bf16" if it % 2 == 0 else "f32"
                check_sample(ctx, x, p, dt, mask, hist, hl, mode, noise,
                             label=f"V={V} it={it} mode={mode}")


@pytest.mark.parametrize("V", [1000, 9001, 40000])
def test_sweep_large_batch(ctx, V):
    # 40 rows take the large-launch k_stream variants (128-thread workgroups, four
    # segments per thread), with and without penalties
    rng = np.random.default_rng(3000 + V)
    for it in range(4):
        x, p, mask, hist, hl = _sweep_case(rng, V, 40)
        if it % 2 == 1:  # no penalty anywhere: the variant without the history table
            p["repetition_penalty"] = 1.0
            p["presence_penalty"] = 0.0
            p["frequency_penalty"] = 0.0
        for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
            dt = "bf16" if it < 2 else "f32"
            say(f"sweep-large V={V} it={it} mode={mode} dtype={dt}")
            check_sample(ctx, x, p, dt, mask, hist, hl, mode, None,
                         label=f"large V={V} it={it} mode={mode}")


@pytest.mark.parametrize("V", [163840, 163841, 262144, 300007, 1 << 20])
def test_vocab_past_64_chunks(V):
    # rows at and past the lattice's 40 chunks (163,840 tokens) and past 64 chunks (up to
    # the 2^20 maximum): up to 64 chunks every wave reduces the chunk statistics alone,
    # past that they merge across waves; general rows past 40 chunks take the exact
    # resolution
    rng = np.random.default_rng(V % 1000)
    B = 4
    x = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    hist = rng.integers(0, V, size=(B, 500)).astype(np.int32)
    p = O.make_params(B, temperature=[0.8, 1.0, 0.0, 0.7], top_k=[0, 50, 0, 0],
                      top_p=[0.9, 1.0, 1.0, 0.95], min_p=[0.0, 0.0, 0.0, 0.05],
                      presence_penalty=np.float32(0.4),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                      position=np.arange(B, dtype=np.uint64))
    c = ops.Context(0, max_rows=B, max_vocab=V)
    try:
        for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
            say(f"vocab {V} mode={mode}")
            check_sample(c, x, p, "bf16", None, hist, None, mode, None, label=f"V={V}")
    finally:
        c.close()


@pytest.mark.parametrize("H", [300, 4096, 8192, 9000])
def test_large_batch_long_histories(ctx, H):
    # Launches of 32 rows or more run four 8-token segments per thread. Every chunk's
    # workgroup counts the row's history ids that fall inside it: the first 4,096 ids from
    # registers loaded before the logits, a longer history's rest read in a loop.
    # Zipf-skewed ids put hundreds of ids in one chunk; ids out of range and lengths
    # below H are dropped.
    rng = np.random.default_rng(4000 + H)
    B, V = 36, 20000
    x = rng.normal(0, 2.0, size=(B, V)).astype(np.float32)
    perm = rng.permutation(V)
    hist = W.zipf_ids(rng, B * H, V, perm).reshape(B, H).astype(np.int32)
    hist[:, ::97] = rng.integers(-3, 0, size=hist[:, ::97].shape)
    hist[:, 1::89] = V + rng.integers(0, 3, size=hist[:, 1::89].shape)
    hl = rng.integers(0, H + 1, size=B).astype(np.int32)
    hl[:4] = H
    p = O.make_params(B, temperature=rng.choice([0.7, 1.0], size=B),
                      top_k=rng.choice([0, 40], size=B), top_p=rng.choice([1.0, 0.9], size=B),
                      min_p=rng.choice([0.0, 0.02], size=B),
                      repetition_penalty=rng.choice([1.0, 1.1], size=B),
                      presence_penalty=0.5, frequency_penalty=0.3,
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=3)
    allowed = rng.random((B, V)) < 0.3
    allowed[:, perm[:50]] = True
    for dt in ("bf16", "f32"):
        for mask in (None, W.pack_mask(allowed)):
            say(f"large-batch history H={H} dtype={dt} mask={mask is not None}")
            check_sample(ctx, x, p, dt, mask, hist, hl, O.NOISE_ICDF, None,
                         label=f"long history H={H} {dt}")


def test_verify_large_batch_history(ctx):
    # 10 sequences x (k + 1) = 40 rows: the grouped history plus each row's draft prefix
    rng = np.random.default_rng(77)
    B, k, V, H = 10, 3, 9001, 2048
    tgt = rng.normal(0, 2.0, size=(B, k + 1, V)).astype(np.float32)
    drafts = tgt[:, :k, :].argmax(-1).astype(np.int32)
    drafts[::3, 1] = rng.integers(0, V, size=drafts[::3, 1].shape)
    perm = rng.permutation(V)
    hist = W.zipf_ids(rng, B * H, V, perm).reshape(B, H).astype(np.int32)
    hist[:, :8] = drafts[:, :1]  # the drafts are in the history too
    p = O.make_params(B, temperature=rng.choice([0.0, 0.7, 1.0], size=B),
                      top_k=rng.choice([0, 20], size=B), top_p=rng.choice([1.0, 0.9], size=B),
                      repetition_penalty=1.2, presence_penalty=0.4, frequency_penalty=0.1,
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=5)
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        say(f"verify large batch history mode={mode}")
        check_verify(ctx, tgt, k, drafts, p, "bf16", None, hist, None, mode,
                     label="verify large batch history")


# ------------------------------------------------------------- configs ----
def test_cfg1_fp32_chain_and_greedy(ctx):
    w = W.cfg1()
    say("cfg1 icdf")
    check_sample(ctx, w["x"], w["params"], "f32", None, w["history"], w["history_len"],
                 O.NOISE_ICDF, w["noise"], label="cfg1")
    say("cfg1 gumbel philox")
    check_sample(ctx, w["x"], w["params"], "f32", None, w["history"], w["history_len"],
                 O.NOISE_GUMBEL, None, label="cfg1 gumbel")
    say("cfg1 greedy")
    ids, st, ref = check_sample(ctx, w["x"], w["greedy_params"], "f32", None, w["history"],
                                w["history_len"], label="cfg1 greedy")
    assert ids[0] in set(w["spikes"].tolist())


@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
@pytest.mark.parametrize("injected", [False, True])
def test_cfg2_heterogeneous(ctx, mode, injected):
    w = W.cfg2()
    B, V = w["x"].shape
    noise = w["noise"] if mode == O.NOISE_ICDF else np.random.default_rng(9).random(
        (B, V + 1), dtype=np.float32)
    say(f"cfg2 mode={mode} injected={injected}")
    check_sample(ctx, w["x"], w["params"], "bf16", None, w["history"], w["history_len"], mode,
                 noise if injected else None, label="cfg2")


@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
def test_cfg3_masks(ctx, mode):
    w = W.cfg3()
    say(f"cfg3 mode={mode}")
    ids, st, ref = check_sample(ctx, w["x"], w["params"], "bf16", w["mask"], None, None, mode,
                                w["noise"] if mode == O.NOISE_ICDF else None, label="cfg3")
    assert (st == 0).all()
    for r in range(len(ids)):
        assert w["allowed"][r, ids[r]]
    assert ids[6] == int(np.nonzero(w["allowed"][6])[0][0])


@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
@pytest.mark.parametrize("injected", [False, True])
def test_n1_north_star_chain(ctx, mode, injected):
    # B=8 x V=151,936 bf16: presence/frequency penalties over 4,096 history ids, cfg3's
    # masks (every density and edge row), T 0.8, top-p 0.9, no top-k or min-p
    w = W.n1()
    B, V = w["x"].shape
    noise = None
    if injected:
        noise = w["noise"] if mode == O.NOISE_ICDF else np.random.default_rng(19).random(
            (B, V + 1), dtype=np.float32)
    say(f"n1 mode={mode} injected={injected}")
    ids, st, ref = check_sample(ctx, w["x"], w["params"], "bf16", w["mask"], w["history"],
                                w["history_len"], mode, noise, label="n1")
    assert (st == 0).all()
    for r in range(B):
        assert w["allowed"][r, ids[r]]


@pytest.mark.parametrize("seed", [7, 8, 9, 10, 11, 12])
def test_n1_other_sets(ctx, seed):
    # more n1 sets: each masked-nucleus row's top-p cut falls in a lattice bin of 50-180
    # keys on two or three values of l, and its draw often in another crowded bin
    w = W.n1(seed=seed)
    say(f"n1 seed={seed}")
    ids, st, ref = check_sample(ctx, w["x"], w["params"], "bf16", w["mask"], w["history"],
                                w["history_len"], O.NOISE_ICDF, w["noise"], label="n1-sets")
    assert (st == 0).all()


def _grid_logits(rng, n, V):
    # rows of N(0, s^2) rounded to a grid of 1/16 .. 1/128: every lattice bin near a
    # decision holds tens to hundreds of keys on one to eight values of l
    s = rng.choice([1.0, 1.5, 2.0], size=n)
    q = rng.choice([16.0, 32.0, 64.0, 128.0], size=n)
    x = rng.normal(0, 1, size=(n, V)) * s[:, None]
    return (np.round(x * q[:, None]) / q[:, None]).astype(np.float32)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_crowded_bins_few_values(ctx, seed):
    # top-k (a count decision), kept ties, min-p, top-p and the draw over zones whose keys
    # share a few values of l
    rng = np.random.default_rng(500 + seed)
    B, V = 16, 60000
    x = _grid_logits(rng, B, V)
    p = O.make_params(B, temperature=rng.choice([0.7, 1.0, 1.3], size=B),
                      top_k=rng.choice([0, 0, 300, 1000, 2500], size=B),
                      top_p=rng.choice([1.0, 0.5, 0.8, 0.9, 0.95, 0.99], size=B),
                      min_p=rng.choice([0.0, 0.0, 0.01, 0.05], size=B),
                      flags=rng.choice([0, 0, 1], size=B),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                      position=np.arange(B, dtype=np.uint64))
    noise = rng.random((B, 2), dtype=np.float32)
    say(f"crowded bins seed={seed}")
    check_sample(ctx, x, p, "bf16", None, None, None, O.NOISE_ICDF, noise, label="crowded")
    check_sample(ctx, x, p, "bf16", None, None, None, O.NOISE_ICDF, None, label="crowded-own")


def test_crowded_bins_verify(ctx):
    # verify rows over the same kind of zones: the draft is excluded from the residual draw
    rng = np.random.default_rng(510)
    B, k, V = 6, 3, 60000
    x = _grid_logits(rng, B * (k + 1), V).reshape(B, k + 1, V)
    drafts = np.empty((B, k), np.int32)
    for b in range(B):
        for j in range(k):  # drafts among each row's leading values
            drafts[b, j] = int(rng.choice(np.argsort(-x[b, j], kind="stable")[:400]))
    p = O.make_params(B, temperature=np.float32(1.0), top_p=rng.choice([0.8, 0.9, 0.95], size=B),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64))
    say("crowded bins verify")
    check_verify(ctx, x, k, drafts, p, "bf16", None, None, None, O.NOISE_ICDF, None,
                 label="crowded-verify")


def test_cfg5_stress_batch(ctx):
    w = W.cfg5()
    say("cfg5")
    check_sample(ctx, w["x"], w["params"], "bf16", w["mask"], w["history"], w["history_len"],
                 O.NOISE_ICDF, None, label="cfg5")


# ------------------------------------------------------------ large kept sets ----
@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
def test_unfiltered_full_vocab(ctx, mode):
    # no top-k / top-p / min-p: the kept set is the whole row (histogram-summary path)
    rng = np.random.default_rng(31)
    B, V = 8, W.V_DEFAULT
    x = rng.normal(0, 1.5, size=(B, V)).astype(np.float32)
    p = O.make_params(B, temperature=np.float32(0.9), seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                      position=np.arange(B, dtype=np.uint64))
    say(f"unfiltered mode={mode}")
    check_sample(ctx, x, p, "bf16", None, None, None, mode, None, label="unfiltered")


def test_large_nucleus_top_p(ctx):
    rng = np.random.default_rng(32)
    B, V = 8, W.V_DEFAULT
    x = rng.normal(0, 1.0, size=(B, V)).astype(np.float32)
    p = O.make_params(B, top_p=np.linspace(0.3, 0.99, B).astype(np.float32),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64))
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        say(f"large nucleus mode={mode}")
        check_sample(ctx, x, p, "bf16", None, None, None, mode, None, label="nucleus")


@pytest.mark.parametrize("injected", [False, True])
def test_rank_noise_wide_nucleus(ctx, injected):
    # Sampler-compat rows (ties kept, noise by rank, no log-sum-exp) whose nucleus holds
    # tens of thousands of tokens: the rank-ordered walk of the exact path
    rng = np.random.default_rng(33)
    B, V = 4, W.V_DEFAULT
    x = rng.normal(0, 0.7, size=(B, V)).astype(np.float32)
    p = O.make_params(B, temperature=np.float32(1.3), top_p=[0.5, 0.9, 0.99, 0.7],
                      top_k=[0, 0, 0, 60000], flags=O.FLAG_SAMPLER_COMPAT,
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                      position=np.arange(B, dtype=np.uint64))
    noise = rng.random((B, V + 1), dtype=np.float32) if injected else None
    say(f"rank noise wide nucleus injected={injected}")
    check_sample(ctx, x, p, "bf16", None, None, None, O.NOISE_GUMBEL, noise, label="rank-wide")


@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
def test_minp_slot_overflow(ctx, mode):
    # min-p rows (fast class) over near-flat logits: every chunk overflows its local
    # candidate slots and the row is resolved by the exact path
    rng = np.random.default_rng(34)
    B, V = 8, W.V_DEFAULT
    x = rng.normal(0, 0.2, size=(B, V)).astype(np.float32)
    hist = rng.integers(0, V, size=(B, 512), dtype=np.int32)
    p = O.make_params(B, temperature=np.float32(1.0), min_p=np.float32(0.05),
                      top_k=[0, 0, 300, 5000, 0, 0, 0, 0],
                      top_p=[1.0, 0.9, 1.0, 0.8, 1.0, 0.95, 1.0, 0.6],
                      repetition_penalty=np.float32(1.2), frequency_penalty=np.float32(0.1),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                      position=np.arange(B, dtype=np.uint64))
    say(f"minp overflow mode={mode}")
    check_sample(ctx, x, p, "bf16", None, hist, None, mode, None, label="minp-overflow")


@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
def test_tie_blocks(ctx, mode):
    # logits quantised to a few values: huge exact-tie groups ordered by id
    rng = np.random.default_rng(35)
    B, V = 6, 50000
    x = rng.integers(-3, 2, size=(B, V)).astype(np.float32)
    p = O.make_params(B, top_k=[0, 20000, 0, 777, 0, 30000], top_p=[0.9, 1.0, 0.3, 0.99, 1.0, 0.5],
                      flags=[0, 1, 7, 1, 0, 7], seed=rng.integers(0, 2**63, size=B, dtype=np.uint64))
    say(f"tie blocks mode={mode}")
    check_sample(ctx, x, p, "bf16", None, None, None, mode, None, label="ties")


def test_verify_flat_exact(ctx):
    # verification over near-flat target rows with penalties over history and the draft
    # prefix: draft rows resolved by the exact path
    rng = np.random.default_rng(36)
    B, k, V = 3, 3, 60000
    x = rng.normal(0, 0.3, size=(B, k + 1, V)).astype(np.float32)
    drafts = rng.integers(0, V, size=(B, k), dtype=np.int32)
    hist = rng.integers(0, V, size=(B, 300), dtype=np.int32)
    p = O.make_params(B, temperature=np.float32(0.9), top_p=[0.95, 1.0, 0.8], min_p=[0.0, 0.05, 0.0],
                      presence_penalty=np.float32(0.4),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64))
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        say(f"verify flat mode={mode}")
        check_verify(ctx, x, k, drafts, p, "bf16", None, hist, None, mode, None, label="verify-flat")


def test_flat_row_ties(ctx):
    # every logit equal: order is by id; top-k keeps the K smallest ids
    V, B = 10000, 4
    x = np.zeros((B, V), np.float32)
    p = O.make_params(B, top_k=[100, 0, 3000, 7], top_p=[1.0, 0.5, 0.9, 1.0], flags=[0, 0, 1, 1],
                      seed=5, position=np.arange(B, dtype=np.uint64))
    say("flat ties")
    ids, st, ref = check_sample(ctx, x, p, "bf16", label="flat")


# ------------------------------------------------------------ errors / layout ----
def test_row_errors(ctx):
    V, B = 5000, 5
    rng = np.random.default_rng(3)
    x = rng.normal(size=(B, V)).astype(np.float32)
    x[1, 17] = np.nan
    x[4, 9] = np.inf
    allowed = np.ones((B, V), bool)
    allowed[3] = False
    allowed[2, :100] = False  # row 2 stays valid
    p = O.make_params(B)
    say("row errors")
    ids, st, ref = check_sample(ctx, x, p, "f32", W.pack_mask(allowed), label="errors")
    assert st.tolist() == [0, O.STRIM_ENONFINITE, 0, O.STRIM_EEMPTY, O.STRIM_ENONFINITE]
    assert (ids[[1, 3, 4]] == -1).all()
    # invalid params fail the whole call synchronously, like ChatRequest validation
    from strim_amd import _native as N

    bad = p.copy()
    bad["top_p"][2] = 0.0
    with pytest.raises(N.StrimError) as ei:
        run_sample(ctx, x, bad, "f32")
    assert ei.value.code == N.EINVAL


def test_strided_and_unaligned_rows(ctx):
    rng = np.random.default_rng(4)
    B, V = 4, 3001
    x = rng.normal(size=(B, V + 13)).astype(np.float32)
    p = O.make_params(B, top_k=10, seed=3)
    for dt in ("f32", "bf16"):
        full = dev_logits(x, dt)
        view = full[:, 1:V + 1]  # row stride V+13, base not 16-byte aligned
        say(f"strided dtype={dt}")
        ids, st, _ = ctx.sample(view, p, noise=dev(np.full((B, 2), 0.3, np.float32)))
        torch.cuda.synchronize()
        xh = W.bf16_round(x[:, 1:V + 1]) if dt == "bf16" else x[:, 1:V + 1]
        ref = O.sample(np.ascontiguousarray(xh), p, noise=np.full((B, 2), 0.3, np.float32))
        np.testing.assert_array_equal(ids.cpu().numpy(), ref["token"])


def test_reproducible(ctx):
    w = W.cfg2()
    say("reproducible")
    a = run_sample(ctx, w["x"], w["params"], "bf16", None, w["history"], w["history_len"],
                   O.NOISE_GUMBEL, None, probs=False)[0]
    b = run_sample(ctx, w["x"], w["params"], "bf16", None, w["history"], w["history_len"],
                   O.NOISE_GUMBEL, None, probs=False)[0]
    np.testing.assert_array_equal(a, b)
    p2 = w["params"].copy()
    p2["position"] += 1
    c = run_sample(ctx, w["x"], p2, "bf16", None, w["history"], w["history_len"],
                   O.NOISE_GUMBEL, None, probs=False)[0]
    assert (a != c).any()


# ------------------------------------------------------------------ verify ----
def test_verify_accept_count_semantics(ctx):
    # SpecSamplingTests.verifyAcceptCountSemantics (SpecSamplingTests.swift:181-197)
    V = 8
    r0 = np.full(V, -50, np.float32); r0[1] = 0
    r1 = r0.copy(); r1[1] = -50; r1[2] = 0
    r2 = np.full(V, -50, np.float32); r2[5] = 0
    logits = np.stack([r0, r1, r2, r2])[None]
    say("verify KAT")
    for first in range(20):
        p = O.make_params(1, temperature=1.0, seed=1, position=first)
        for mode in (O.NOISE_GUMBEL, O.NOISE_ICDF):
            g, _ = check_verify(ctx, logits, 3, [[1, 2, 3]], p, "f32", noise_mode=mode)
            assert g["accepted"][0] == 2 and g["token"][0] == 5


@pytest.mark.parametrize("k", [0, 1, 3])
def test_verify_random(ctx, k):
    rng = np.random.default_rng(50 + k)
    for it in range(6):
        B = int(rng.choice([1, 4, 8]))
        V = int(rng.choice([50, 4096, 20000, W.V_DEFAULT]))
        tgt = rng.normal(0, rng.choice([1.0, 3.0]), size=(B, k + 1, V)).astype(np.float32)
        drafts = rng.integers(0, V, size=(B, k)).astype(np.int32)
        # sometimes draft the argmax so accepts happen
        am = tgt[:, :k, :].argmax(-1)
        pick = rng.random((B, k)) < 0.5
        drafts[pick] = am[pick]
        p = O.make_params(B, temperature=rng.choice([0.0, 0.7, 1.0], size=B),
                          top_k=rng.choice([0, 20], size=B), top_p=rng.choice([1.0, 0.9], size=B),
                          min_p=rng.choice([0.0, 0.05], size=B),
                          seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                          position=rng.integers(0, 100, size=B).astype(np.uint64))
        mask = None
        if it % 2 == 1:
            allowed = rng.random((B, k + 1, V)) < 0.5
            mask = W.pack_mask(allowed)
        H = 16 if it % 3 == 0 else 0
        hist = rng.integers(0, V, size=(B, H)).astype(np.int32) if H else None
        if H:
            p["repetition_penalty"] = 1.3
        for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
            say(f"verify k={k} it={it} B={B} V={V} mode={mode}")
            check_verify(ctx, tgt, k, drafts, p, "bf16", mask, hist, None, mode,
                         label=f"verify k={k} it={it}")


def test_verify_error_after_rejection(ctx):
    # a bad draft or an empty row after the first rejection leaves the sequence alone;
    # only the rows the accept chain reaches count (SpecSampling.swift:101-105)
    rng = np.random.default_rng(17)
    V, k = 300, 3
    tgt = rng.normal(size=(3, k + 1, V)).astype(np.float32)
    allowed = np.ones((3, k + 1, V), bool)
    allowed[:, 0, 9] = False
    allowed[1, 2, :] = False
    drafts = np.array([[9, V + 5, 7], [9, 5, 6], [V + 5, 1, 2]], np.int32)
    p = O.make_params(3, temperature=1.0, seed=4)
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        say(f"verify error after rejection mode={mode}")
        g, ref = check_verify(ctx, tgt, k, drafts, p, "f32", W.pack_mask(allowed),
                              noise_mode=mode, label="error-after-reject")
        assert g["status"].tolist() == [0, 0, O.STRIM_EINVAL]
        assert g["token"][2] == -1 and g["token"][0] == ref["token"][0]
        assert g["row_token"][0, 1] == -1 and g["row_token"][1, 2] == -1


# ------------------------------------------------------------ general-q verify ----
@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
def test_verify_general_q_cfg4(ctx, mode):
    # configuration 4: target [4,4,V] bf16, draft logits [4,3,32768] over an ascending
    # injective table, drafts sampled from q, T 0.7, Philox uniforms per position
    # Without per-row outputs only (accepted, token) is computed: k_finalize takes the
    # accept tests and the residual draw serves each sequence's first rejection alone.
    w = W.cfg4()
    for rows in (True, False):
        say(f"verify general-q cfg4 mode={mode} row_outputs={rows}")
        check_verify(ctx, w["target"], w["k"], w["drafts"], w["params"], "bf16", noise_mode=mode,
                     draft_logits=w["draft_logits"], table=w["table"],
                     label=f"cfg4 mode={mode} rows={rows}", row_outputs=rows)


@pytest.mark.parametrize("k", [1, 3])
def test_verify_general_q_random(ctx, k):
    rng = np.random.default_rng(70 + k)
    for it in range(4):
        B = int(rng.choice([2, 5]))
        V = int(rng.choice([300, 5000, 20000]))
        Vd = int(rng.choice([V // 4, V // 2]))
        table = np.sort(rng.choice(V, size=Vd, replace=False)).astype(np.int32)
        tgt = rng.normal(0, 2.0, size=(B, k + 1, V)).astype(np.float32)
        dl = (0.6 * tgt[:, :k, :][:, :, table]
              + rng.normal(0, 1.0, size=(B, k, Vd))).astype(np.float32)
        T = rng.choice([0.0, 0.7, 1.0], size=B)
        Tq = np.where(T > 0, T, 1.0)
        q = W.bf16_round(dl).astype(np.float64) / Tq[:, None, None]
        q = np.exp(q - q.max(-1, keepdims=True))
        q /= q.sum(-1, keepdims=True)
        drafts = np.zeros((B, k), np.int32)
        for b in range(B):
            for j in range(k):
                drafts[b, j] = table[rng.choice(Vd, p=q[b, j])]
        p = O.make_params(B, temperature=T, top_k=rng.choice([0, 20], size=B),
                          top_p=rng.choice([1.0, 0.9], size=B),
                          min_p=rng.choice([0.0, 0.05], size=B),
                          seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                          position=rng.integers(0, 100, size=B).astype(np.uint64))
        mask = W.pack_mask(rng.random((B, k + 1, V)) < 0.6) if it % 2 else None
        hist = rng.integers(0, V, size=(B, 8)).astype(np.int32) if it == 2 else None
        if hist is not None:
            p["presence_penalty"] = 0.4
        for mode, rows in ((O.NOISE_ICDF, True), (O.NOISE_GUMBEL, True), (O.NOISE_GUMBEL, False)):
            say(f"verify general-q k={k} it={it} B={B} V={V} Vd={Vd} mode={mode} rows={rows}")
            check_verify(ctx, tgt, k, drafts, p, "bf16", mask, hist, None, mode,
                         draft_logits=dl, table=table, label=f"general-q k={k} it={it}",
                         row_outputs=rows)


def test_verify_general_q_table_errors(ctx):
    rng = np.random.default_rng(90)
    B, k, V, Vd = 3, 2, 400, 100
    table = np.sort(rng.choice(V, size=Vd, replace=False)).astype(np.int32)
    tgt = rng.normal(size=(B, k + 1, V)).astype(np.float32)
    dl = rng.normal(size=(B, k, Vd)).astype(np.float32)
    drafts = rng.choice(table, size=(B, k)).astype(np.int32)
    outside = np.setdiff1d(np.arange(V), table)
    drafts[1, 1] = outside[0]  # sequence 1: a draft the draft vocabulary cannot produce
    p = O.make_params(B, temperature=0.8, seed=np.arange(B, dtype=np.uint64))
    say("verify general-q draft outside the table")
    g, ref = check_verify(ctx, tgt, k, drafts, p, "f32", draft_logits=dl, table=table,
                          label="draft outside table")
    assert g["status"][1] == O.STRIM_EINVAL and g["status"][0] == 0
    bad = table.copy()
    bad[[10, 11]] = bad[[11, 10]]  # not ascending
    say("verify general-q unsorted table")
    g = run_verify(ctx, host_logits(tgt, "f32"), k, drafts, p, "f32", draft_logits=dl,
                   table=bad)
    assert (g["status"] == O.STRIM_EINVAL).all()
    assert (g["accepted"] == 0).all() and (g["token"] == -1).all()


# ------------------------------------------------------------------ aux ops ----
def test_mask_logits(ctx):
    rng = np.random.default_rng(6)
    R, V = 3, 1003
    x = rng.normal(size=(R, V)).astype(np.float32)
    allowed = rng.random((R, V)) < 0.4
    for dt in ("f32", "bf16"):
        say(f"mask_logits {dt}")
        out = ops.mask_logits(dev_logits(x, dt), dev(W.pack_mask(allowed))).cpu().numpy()
        xh = W.bf16_round(x) if dt == "bf16" else x
        np.testing.assert_array_equal(out, np.where(allowed, xh, -np.inf).astype(np.float32))


def test_draft_argmax(ctx):
    rng = np.random.default_rng(7)
    R, Vd = 5, 32768
    dl = rng.normal(size=(R, Vd)).astype(np.float32)
    table = np.sort(rng.choice(W.V_DEFAULT, size=Vd, replace=False)).astype(np.int32)
    say("draft_argmax")
    got = ops.draft_argmax(dev_logits(dl, "bf16"), dev(table)).cpu().numpy()
    xh = W.bf16_round(dl)
    np.testing.assert_array_equal(got, table[xh.argmax(-1)])


# ------------------------------------------------------------ mirror API ----
def test_sampler_mirror_matches_oracle(ctx):
    from strim_amd.sampler import GenParams, Sampler, SamplingConfig, SpecSampling

    rng = np.random.default_rng(8)
    V = 4000
    x = rng.normal(size=V).astype(np.float32)
    xd = dev_logits(x, "f32")
    s = Sampler(GenParams(temperature=0.9, top_k=20, top_p=0.9, seed=123), ctx=ctx)
    say("mirror Sampler.sample")
    for i in range(5):
        got = s.sample(xd)
        p = O.make_params(1, temperature=0.9, top_k=20, top_p=0.9, seed=123, position=i,
                          flags=O.FLAG_SAMPLER_COMPAT)
        ref = O.sample(x[None], p, noise_mode=O.NOISE_GUMBEL)
        assert got == ref["token"][0] or ref["margin"][0] < O.TIE_EPS
    cfg = SamplingConfig(temperature=1.0, top_k=0, top_p=1.0, seed=77)
    say("mirror SpecSampling.sample")
    a = [SpecSampling.sample(xd, cfg, i, ctx=ctx) for i in range(20)]
    b = [SpecSampling.sample(xd, cfg, i, ctx=ctx) for i in range(20)]
    assert a == b and len(set(a)) > 5


# ------------------------------------------------------------ statistics ----
@pytest.mark.parametrize("t,k,pp", [(1.0, 0, 1.0), (0.8, 5, 1.0), (1.0, 0, 0.8), (1.0, 6, 0.9)])
@pytest.mark.parametrize("mode", [O.NOISE_ICDF, O.NOISE_GUMBEL])
def test_gpu_verify_marginal(ctx, t, k, pp, mode):
    # SpecSamplingTests.marginalMatchesTarget (SpecSamplingTests.swift:104-118) on the GPU
    # verifier, at the reference's strength: the four parameter sets, drafts the mode,
    # the third most likely token and (where one exists) a token of zero filtered mass,
    # n = 200,000 draws each with seeds 2000 + j, accept-or-residual ~ P by chi-square
    # and the accept rate within 0.01 of P(draft)
    from test_oracle import _chi2

    rng = np.random.default_rng(11)
    V, n, chunk = 16, 200_000, 4000
    row = (rng.normal(size=V) * 2).astype(np.float32)
    P = O.sample(row[None], O.make_params(1, temperature=t, top_k=k, top_p=pp),
                 want_probs=True)["probs"][0].astype(np.float64)
    order = np.argsort(-P, kind="stable")
    drafts = [int(order[0]), int(order[2])]
    zero = np.nonzero(P == 0)[0]
    if zero.size:
        drafts.append(int(zero[0]))
    tgt = dev_logits(np.repeat(np.repeat(row[None, None], 2, 1), chunk, 0), "f32")
    for jd, d in enumerate(drafts):
        say(f"marginal T={t} k={k} p={pp} mode={mode} draft={d}")
        dd = dev(np.full((chunk, 1), d, np.int32))
        emitted, accs = [], []
        for c0 in range(0, n, chunk):
            p = O.make_params(chunk, temperature=t, top_k=k, top_p=pp, seed=2000 + jd)
            p["position"] = (np.arange(chunk, dtype=np.uint64) + c0) * 2
            g = ctx.verify(tgt, dd, p, noise_mode=mode)
            acc = g["row_accept"][:, 0].cpu().numpy().astype(bool)
            emitted.append(np.where(acc, d, g["row_token"][:, 0].cpu().numpy()))
            accs.append(acc)
        e = np.concatenate(emitted)
        stat, crit = _chi2(np.bincount(e, minlength=V).astype(np.float64), P)
        assert stat < crit, (t, k, pp, mode, d, stat, crit)
        assert abs(np.concatenate(accs).mean() - P[d]) < 0.01


def test_gpu_verify_reproducible_and_seed_sensitive(ctx):
    # the verify half of SpecSamplingTests.verifyIsReproducibleAndSeedSensitive
    # (SpecSamplingTests.swift:158-170) through strim_verify: a (seed, first index) pair
    # repeats its outcome, and 40 seeds or 40 first indices give more than three
    # distinct outcomes; every outcome equals the oracle's. (A flat row, as in the
    # oracle's version of this test: the reference's MLX-drawn row is not reproducible
    # here.)
    rng = np.random.default_rng(3)
    V, k = 32, 3
    logits = (rng.normal(size=(k + 1, V)) * 0.5).astype(np.float32)
    cases = [(9, 5), (9, 5)] + [(s, 5) for s in range(40)] + [(9, f) for f in range(40)]
    B = len(cases)
    p = O.make_params(B, temperature=1, top_k=20, top_p=0.95,
                      seed=np.array([c[0] for c in cases], np.uint64),
                      position=np.array([c[1] for c in cases], np.uint64))
    tgt = np.repeat(logits[None], B, 0)
    dr = np.tile(np.array([[1, 2, 3]], np.int32), (B, 1))
    say("verify reproducible")
    g = ctx.verify(dev_logits(tgt, "f32"), dev(dr), p, noise_mode=O.NOISE_GUMBEL)
    torch.cuda.synchronize()
    got = list(zip(g["accepted"].cpu().numpy().tolist(), g["token"].cpu().numpy().tolist()))
    ref = O.verify(tgt, k, dr, p, noise_mode=O.NOISE_GUMBEL)
    assert got == list(zip(ref["accepted"].tolist(), ref["token"].tolist()))
    assert got[0] == got[1]
    assert len(set(got[2:42])) > 3
    assert len(set(got[42:])) > 3


@pytest.mark.parametrize("const_noise", [True, False])
def test_gumbel_unfiltered_ties_across_waves(ctx, const_noise):
    # Unfiltered Gumbel rows (no top-k / top-p / min-p) with quantised logits whose maximum
    # is held by ids in several waves and chunks. With one injected uniform for every
    # token the proxy scores tie exactly across lanes, waves and chunks, so the chunks'
    # two-best shortlist cannot be certain and the rows take the exact resolution (ties
    # to the smallest id); with random uniforms the shortlist decides. strim_sample and
    # strim_verify (the draft among the tied ids) against the oracle.
    rng = np.random.default_rng(71 if const_noise else 72)
    B, V, k = 4, 20000, 2
    x = (np.round(rng.normal(0.0, 1.0, size=(B, V)) * 2.0) / 2.0).astype(np.float32)
    tied = np.array([5, 700, 1100, 4095, 4100, 9000, 13313, 19999])
    x[:, tied] = 6.0
    p = O.make_params(B, seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=3)
    if const_noise:
        noise = np.full((B, V + 1), 0.5, np.float32)
    else:
        noise = rng.random((B, V + 1), dtype=np.float32)
    say(f"gumbel ties sample const={const_noise}")
    ids, _, _ = check_sample(ctx, x, p, "f32", noise_mode=O.NOISE_GUMBEL, noise=noise,
                             probs=False, label="gumbel-ties")
    if const_noise:
        assert (ids == tied[0]).all(), ids
    xt = np.repeat(x[:, None, :], k + 1, axis=1)
    drafts = np.stack([tied[[0, 3]], tied[[2, 1]], tied[[7, 0]], [3, tied[4]]]).astype(np.int32)
    nv = np.repeat(noise[:, None, :], k + 1, axis=1).copy()
    say(f"gumbel ties verify const={const_noise}")
    check_verify(ctx, xt, k, drafts, p, "f32", noise_mode=O.NOISE_GUMBEL, noise=nv,
                 label="gumbel-ties-verify")


def test_gumbel_unfiltered_near_ties(ctx):
    # Tokens of one chunk whose Gumbel scores differ by less than the fp32 proxy's error:
    # equal logits and adjacent uniforms (u ~ 0.9 + k 2^-24, scores ~6e-7 apart), so the
    # chunk's proxy order may differ from the fp64 one and every near tie must reach the
    # fp64 decision. Row 1 holds a whole chunk of equal logits under one uniform: more near
    # ties than a chunk keeps, decided by the exact resolution. Sample and verify (drafts
    # among the near ties) against the oracle.
    rng = np.random.default_rng(73)
    B, V, k = 3, 20000, 2
    x = (np.round(rng.normal(0.0, 1.0, size=(B, V)) * 2.0) / 2.0).astype(np.float32)
    noise = (rng.random((B, V + 1), dtype=np.float32) * np.float32(0.5)).astype(np.float32)
    near = np.array([9, 130, 2000, 4090, 8200, 8201, 12000])
    x[:, near] = 7.0
    steps = rng.permutation(len(near))
    for r in range(B):
        noise[r, near] = (np.float32(0.9) + steps.astype(np.float32) * np.float32(2.0 ** -24))
    x[1, 4096:8192] = 7.0
    noise[1, 4096:8192] = np.float32(0.75)
    p = O.make_params(B, seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=5)
    say("gumbel near ties sample")
    check_sample(ctx, x, p, "f32", noise_mode=O.NOISE_GUMBEL, noise=noise, probs=False,
                 label="gumbel-near")
    xt = np.repeat(x[:, None, :], k + 1, axis=1)
    drafts = np.stack([near[[3, 2]], near[[4, 5]], [4100, near[1]]]).astype(np.int32)
    nv = np.repeat(noise[:, None, :], k + 1, axis=1).copy()
    say("gumbel near ties verify")
    check_verify(ctx, xt, k, drafts, p, "f32", noise_mode=O.NOISE_GUMBEL, noise=nv,
                 label="gumbel-near-verify")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_exact_resolution_penalised_aligned(ctx, dtype):
    # Aligned rows with penalties whose nucleus is wider than both candidate tiers, so the
    # exact streaming resolution decides them. Its windows rebuild the history counts in
    # LDS one after another; the history ids carry a +6 logit that their penalty takes off
    # again, so a window that lost a count would move most of the row's mass.
    rng = np.random.default_rng(75)
    B, V, H = 8, W.V_DEFAULT, 4096
    x = rng.normal(0, 0.3, size=(B, V)).astype(np.float32)
    hist = np.stack([rng.choice(V, size=H, replace=False) for _ in range(B)]).astype(np.int32)
    hist[:, H // 2:] = hist[:, : H // 2]  # every id twice
    for r in range(B):
        x[r, hist[r]] += 6.0
    p = O.make_params(B, temperature=np.float32(1.0),
                      top_p=np.array([0.95, 0.9, 0.99, 0.8, 0.95, 0.97, 0.85, 0.9], np.float32),
                      frequency_penalty=np.float32(2.0), presence_penalty=np.float32(2.0),
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                      position=np.arange(B, dtype=np.uint64))
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        say(f"exact penalised aligned dtype={dtype} mode={mode}")
        check_sample(ctx, x, p, dtype, None, hist, None, mode, None, probs=False,
                     label="exact-pen")
    k = 2
    xt = np.repeat(x[:, None, :], k + 1, axis=1)
    drafts = hist[:, :k].copy()
    say(f"exact penalised aligned verify dtype={dtype}")
    check_verify(ctx, xt, k, drafts, p, dtype, None, hist, None, O.NOISE_ICDF, None,
                 label="exact-pen-verify")


def _gumbel_u(g):
    # the uniform whose Gumbel transform -log(-log u) is g
    return np.float32(np.exp(-np.exp(-np.float64(g))))


def test_gumbel_three_near_ties_one_lane(ctx):
    # Unfiltered Gumbel rows whose three best scores lie in one 8-token segment (one lane)
    # within a few 1e-6 of each other, and every other score far below: the lane holds
    # both of its wave's winners and the third near tie, which must still reach the fp64
    # decision. Sample, and verify with a rejected draft (the residual decides).
    rng = np.random.default_rng(76)
    B, V, k = 32, W.V_DEFAULT, 1
    x = np.full((B, V), -12.0, np.float32)
    noise = rng.random((B, V + 1), dtype=np.float32)
    for r in range(B):
        seg = 8 * int(rng.integers(0, V // 8))
        pos = seg + rng.choice(8, size=3, replace=False)
        x[r, pos] = 30.0
        gaps = np.array([0.0, 1.5e-6, 3.0e-6])[rng.permutation(3)]
        for q in range(3):
            noise[r, pos[q]] = _gumbel_u(0.4 + gaps[q])
    p = O.make_params(B, temperature=np.float32(1.0), position=7,
                      seed=rng.integers(0, 2**63, size=B, dtype=np.uint64))
    say("gumbel three near ties in one lane: sample")
    check_sample(ctx, x, p, "f32", noise_mode=O.NOISE_GUMBEL, noise=noise, probs=False,
                 label="gumbel-3near")
    xt = np.repeat(x[:, None, :], k + 1, axis=1)
    drafts = np.zeros((B, k), np.int32)
    nv = np.repeat(noise[:, None, :], k + 1, axis=1).copy()
    say("gumbel three near ties in one lane: verify")
    check_verify(ctx, xt, k, drafts, p, "f32", noise_mode=O.NOISE_GUMBEL, noise=nv,
                 label="gumbel-3near-verify")
