"""The reference's own known-answer and distributional tests, and the injected-uniform
layout cases, run through the HIP path (strim_sample / strim_verify via the C ABI).

  - uniform_kats.py: hand-solved cases pinning which uniform drives which decision;
  - SpecSamplingTests.filteredMatchesReference (SpecSamplingTests.swift:58-68) on the
    processed probabilities (out_probs);
  - SpecSamplingTests.temperatureZeroPathEqualsArgmax (:70-88) through strim_sample and
    strim_verify;
  - SpecSamplingTests.chainK3MatchesTarget (:120-156): a k = 3 chain on the GPU
    verifier, chi-square per position;
  - the SpecSampling.sample / verify facade against the oracle.
"""
import numpy as np
import pytest
import torch

import oracle as O
import uniform_kats as K
from gpu_util import dev, dev_logits
from test_oracle import _chi2

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def test_uniform_layout_kats_gpu(ctx):
    for name, x, kw, mode, nz, want in K.sample_cases():
        say(f"kat {name}")
        ids, st, _ = ctx.sample(dev_logits(x, "f32"), O.make_params(len(x), **kw),
                                noise_mode=mode, noise=dev(nz, np.float32))
        torch.cuda.synchronize()
        assert st.cpu().numpy().tolist() == [0] * len(x)
        assert ids.cpu().numpy().tolist() == want, name
    for name, t, d, kw, mode, nz, want_acc, want_tok in K.verify_cases():
        say(f"kat {name}")
        g = ctx.verify(dev_logits(t, "f32"), dev(d, np.int32), O.make_params(len(t), **kw),
                       noise_mode=mode, noise=dev(nz, np.float32))
        torch.cuda.synchronize()
        assert g["status"].cpu().numpy().tolist() == [0] * len(t)
        assert g["accepted"].cpu().numpy().tolist() == want_acc, name
        assert g["token"].cpu().numpy().tolist() == want_tok, name


def test_filtered_matches_reference_gpu(ctx):
    # ln([8,4,2,1,1]) -> [.5,.25,.125,.0625,.0625]; top-k 2 -> [2/3,1/3]; top-p 0.7 ->
    # [2/3,1/3] (the third token has mass 0.75 > 0.7 before it)
    row = np.log(np.array([8, 4, 2, 1, 1], np.float64)).astype(np.float32)[None]
    cases = [(dict(), [0.5, 0.25, 0.125, 0.0625, 0.0625]),
             (dict(top_k=2), [2 / 3, 1 / 3, 0, 0, 0]),
             (dict(top_p=0.7), [2 / 3, 1 / 3, 0, 0, 0])]
    for kw, want in cases:
        say(f"filtered {kw}")
        _, st, pr = ctx.sample(dev_logits(row, "f32"), O.make_params(1, **kw), want_probs=True)
        torch.cuda.synchronize()
        assert st.item() == 0
        got = pr.cpu().numpy()[0].astype(np.float64)
        np.testing.assert_allclose(got, want, atol=1e-6)
        assert (got[np.asarray(want) == 0] == 0).all()


def test_temperature_zero_path_equals_argmax_gpu(ctx):
    n, V = 1000, 64
    rng = np.random.default_rng(7)
    x = (rng.normal(size=(n, V)) * 3).astype(np.float32)
    best = x.argmax(-1).astype(np.int32)
    nz = rng.random((n, V + 1), dtype=np.float32)
    p = O.make_params(n, temperature=1e-4)
    say("T=1e-4 sample == argmax")
    ids, st, _ = ctx.sample(dev_logits(x, "f32"), p, noise_mode=O.NOISE_GUMBEL,
                            noise=dev(nz, np.float32))
    torch.cuda.synchronize()
    assert (st.cpu().numpy() == 0).all()
    np.testing.assert_array_equal(ids.cpu().numpy(), best)
    # verify rows: draft == argmax always accepted, any other draft never (its residual
    # is then the argmax)
    tgt = np.stack([x, x], 1)
    nz2 = np.stack([nz, nz], 1)
    for drafts, accepted in ((best, True), ((best + 1) % V, False)):
        say(f"T=1e-4 verify draft==argmax {accepted}")
        g = ctx.verify(dev_logits(tgt, "f32"), dev(drafts.reshape(n, 1), np.int32), p,
                       noise_mode=O.NOISE_GUMBEL, noise=dev(nz2, np.float32))
        torch.cuda.synchronize()
        acc = g["row_accept"].cpu().numpy()[:, 0]
        assert (acc == (1 if accepted else 0)).all()
        if not accepted:
            np.testing.assert_array_equal(g["row_token"].cpu().numpy()[:, 0], best)


def test_chain_k3_matches_target_gpu(ctx):
    # Prefix-dependent target (SpecSamplingTests.chainK3MatchesTarget): row j is consulted
    # only while drafts[0..j) were accepted; the emitted token at every reached position
    # must follow that row's filtered target P_j.
    V, n, k = 16, 98304, 3
    rng = np.random.default_rng(40)
    rows = (rng.normal(size=(k + 1, V)) * 2).astype(np.float32)
    t, tk, tp = 1.0, 8, 0.95
    P = O.sample(rows, O.make_params(k + 1, temperature=t, top_k=tk, top_p=tp),
                 want_probs=True)["probs"].astype(np.float64)
    drafts = np.array([P[0].argmax(), P[1].argmax(), np.argsort(-P[2], kind="stable")[1]],
                      np.int32)
    tgt = np.broadcast_to(rows[None], (8192, k + 1, V)).copy()
    counts = np.zeros((k + 1, V), np.int64)
    reached = np.zeros(k + 1, np.int64)
    for mode in (O.NOISE_GUMBEL, O.NOISE_ICDF):
        counts[:] = 0
        reached[:] = 0
        for c0 in range(0, n, 8192):
            p = O.make_params(8192, temperature=t, top_k=tk, top_p=tp, seed=500 + mode)
            p["position"] = (np.arange(8192, dtype=np.uint64) + c0) * (k + 1)
            say(f"chain k=3 mode={mode} chunk={c0}")
            g = ctx.verify(dev_logits(tgt, "f32"), dev(np.broadcast_to(drafts, (8192, k)), np.int32),
                           p, noise_mode=mode, row_outputs=False)
            torch.cuda.synchronize()
            acc = g["accepted"].cpu().numpy()
            tok = g["token"].cpu().numpy()
            assert (g["status"].cpu().numpy() == 0).all()
            for j in range(k + 1):
                hit = acc >= j
                reached[j] += hit.sum()
                emitted = np.where(acc[hit] > j, drafts[min(j, k - 1)], tok[hit])
                counts[j] += np.bincount(emitted, minlength=V)
        for j in range(k + 1):
            assert reached[j] > 1000, (mode, j, reached[j])
            stat, crit = _chi2(counts[j].astype(np.float64), P[j])
            assert stat < crit, f"mode {mode} position {j}: chi2 {stat:.1f} >= {crit:.1f}"


def test_spec_sampling_facade_matches_oracle(ctx):
    from strim_amd.sampler import SamplingConfig, SpecSampling

    rng = np.random.default_rng(12)
    V, k = 3000, 3
    x = (rng.normal(size=(k + 1, V)) * 2).astype(np.float32)
    xd = dev_logits(x, "f32")
    cfg = SamplingConfig(temperature=0.9, top_k=40, top_p=0.9, seed=31)
    for first in range(12):
        am = x[:k].argmax(-1)
        drafts = [int(am[0]), int(am[1]) if first % 2 else int(rng.integers(V)), int(am[2])]
        say(f"facade verify first={first}")
        got = SpecSampling.verify(xd, drafts, cfg, first, ctx=ctx)
        ref = O.verify(x[None], k, np.array([drafts], np.int32),
                       O.make_params(1, temperature=0.9, top_k=40, top_p=0.9, seed=31,
                                     position=first), noise_mode=O.NOISE_GUMBEL)
        assert got == (ref["accepted"][0], ref["token"][0]) or ref["margin"][0] < O.TIE_EPS
        say(f"facade sample index={first}")
        s = SpecSampling.sample(xd[0], cfg, first, ctx=ctx)
        r = O.sample(x[:1], O.make_params(1, temperature=0.9, top_k=40, top_p=0.9, seed=31,
                                          position=first), noise_mode=O.NOISE_GUMBEL)
        assert s == r["token"][0] or r["margin"][0] < O.TIE_EPS
