"""Batched decode integration (strim_amd/batch.py).

CPU: MTPStats restates the reference's accounting tests (MTPStatsTests.swift:4-88) case
for case. GPU: one BatchPicker call over a mixed batch (greedy, sampled, grammar rows)
equals the reference's per-row pick loop (EngineCore.swift:968-1011) run on the oracle,
row by row, and a constrained speculative round records each request's MTPStats from
the verifier's accepted counts.
"""
import numpy as np
import pytest

from strim_amd.batch import POSITION_LIMIT, MTPStats, draft_depth


# ------------------------------------------------------------- MTPStats (CPU) ----
def test_every_prefix_at_every_depth():
    for depth in range(5):
        for accepted in range(depth + 1):
            s = MTPStats()
            s.record_round(depth, accepted)
            assert s.rounds == 1 and s.emitted == accepted + 1
            for j in range(4):
                assert s.proposed[j] == (1 if j < depth else 0)
                assert s.reached[j] == (1 if j < depth and accepted >= j else 0)
                assert s.accepted_prefix[j] == (1 if j < accepted else 0)


def test_zero_depth_and_budget_truncation():
    for remaining in range(1, 6):
        d = draft_depth(4, remaining)
        s = MTPStats()
        s.record_round(d, d)
        assert s.emitted == remaining and sum(s.proposed) == remaining - 1
    e = MTPStats()
    assert e.rounds == 0 and e.proposed == [0, 0, 0, 0]


def test_fixed_and_adaptive_sequences_match_trace_accounting():
    for depths in ([4, 4, 4, 1, 0], [3, 3, 2, 3, 1, 0], [1, 1, 1, 0]):
        s = MTPStats()
        prop, reach, acc = [0] * 4, [0] * 4, [0] * 4
        tokens = 0
        for n, d in enumerate(depths):
            a = min(d, n % 3)
            s.record_round(d, a)
            tokens += a + 1
            for i in range(1, 5):
                if i <= d:
                    prop[i - 1] += 1
                if i <= d and a >= i - 1:
                    reach[i - 1] += 1
                if a >= i:
                    acc[i - 1] += 1
        assert (s.proposed, s.reached, s.accepted_prefix) == (prop, reach, acc)
        assert s.emitted == tokens and s.rounds == len(depths)


def test_resolved_outcome_fixtures():
    for depth, accepted, reached, prefix in [(4, 4, [1, 1, 1, 1], [1, 1, 1, 1]),
                                             (3, 0, [1, 0, 0, 0], [0, 0, 0, 0]),
                                             (4, 2, [1, 1, 1, 0], [1, 1, 0, 0])]:
        s = MTPStats()
        s.record_round(depth, accepted)
        assert s.reached == reached and s.accepted_prefix == prefix


def test_delta_and_baselines():
    s = MTPStats()
    s.record_round(3, 1)
    before = s.copy()
    assert s.delta(before) == MTPStats()
    s.record_round(2, 0)
    d = s.delta(before)
    assert d.rounds == 1 and d.proposed == [1, 1, 0, 0]
    stream, total = MTPStats(), MTPStats()
    base = stream.copy()
    stream.record_round(4, 2)
    total.add(stream.delta(base))
    base = stream.copy()
    total.add(stream.delta(base))  # the same snapshot cannot count twice
    first = total.copy()
    stream.record_round(2, 0)
    total.add(stream.delta(base))
    assert total.rounds == 2 and first.rounds == 1
    assert total.proposed == [2, 2, 1, 1] and total.accepted_prefix == [1, 1, 0, 0]


def test_bounded_counters_expose_overflow():
    s = MTPStats()
    s.record_round(9, 7)
    assert len(s.proposed) == POSITION_LIMIT and s.proposed == [1, 1, 1, 1]
    assert s.overflow_proposed == 5 and s.emitted == 8


# ------------------------------------------------------------------ GPU ----
@pytest.mark.gpu
def test_gpu_batch_pick_equals_per_row_loop(oracle_mod, ctx):
    import torch

    import grammar_util as G
    from strim_amd.batch import BatchPicker
    from strim_amd.grammar import DeviceGrammar, FREE, forced

    O = oracle_mod
    V = G.FAKE_VOCAB
    width = len(V) + 8
    nt, fl = G.object_int_dfa()
    g = DeviceGrammar(V, width, eos=[G.FAKE_EOS], skip=G.FAKE_SKIP)
    g.set_dfa(nt, fl)
    go = O.GrammarOracle(V, width, [G.FAKE_EOS], G.FAKE_SKIP)
    go.set_dfa(nt, fl)
    rng = np.random.default_rng(21)
    B = 8
    keys = np.array([0, 5, 7, FREE, forced(40), 1, FREE, 5], dtype=np.int32)
    T = np.array([0.0, 0.8, 1.0, 0.0, 0.7, 1.2, 0.9, 0.0])
    p = O.make_params(B, temperature=T, top_k=rng.choice([0, 20], size=B),
                      top_p=rng.choice([1.0, 0.9], size=B), seed=np.arange(B, dtype=np.uint64),
                      position=3)
    x = rng.normal(0, 2.0, size=(B, width)).astype(np.float32)
    picker = BatchPicker(ctx, g)
    ids, status, nxt = picker.pick(torch.from_numpy(x).cuda(), p,
                                   torch.from_numpy(keys).cuda())
    ids, status, nxt = ids.cpu().numpy(), status.cpu().numpy(), nxt.cpu().numpy()
    for b in range(B):  # the reference's loop: mask the row, then sample or argmax it
        m = go.mask(int(keys[b]))[None]
        ref = O.sample(x[b:b + 1], p[b:b + 1], mask=m)
        assert status[b] == 0 and ids[b] == ref["token"][0], (b, ids[b], ref["token"][0])
        k = int(keys[b])
        want = go.advance(k, V[ids[b]]) if 0 <= k < len(fl) and ids[b] < len(V) else k
        assert nxt[b] == want
    g.close()


@pytest.mark.gpu
def test_gpu_constrained_round_records_stats(oracle_mod, ctx):
    import torch

    import grammar_util as G
    from gpu_util import dev_logits
    from strim_amd.batch import BatchPicker
    from strim_amd.grammar import DeviceGrammar, FREE

    O = oracle_mod
    V = G.FAKE_VOCAB
    width = len(V) + 8
    nt, fl = G.object_int_dfa()
    g = DeviceGrammar(V, width, eos=[G.FAKE_EOS], skip=G.FAKE_SKIP)
    g.set_dfa(nt, fl)
    go = O.GrammarOracle(V, width, [G.FAKE_EOS], G.FAKE_SKIP)
    go.set_dfa(nt, fl)
    rng = np.random.default_rng(22)
    B, k = 3, 3
    op, q, a, x = V.index(b"{"), V.index(b"\""), V.index(b"a"), V.index(b"x")
    drafts = np.array([[op, q, a], [op, x, op], [1, 2, 3]], dtype=np.int32)
    keys = np.array([0, 0, FREE], dtype=np.int32)
    tgt = rng.normal(0, 1.0, size=(B, k + 1, width)).astype(np.float32)
    for b in range(B):  # make the drafts likely so that some are accepted
        for j in range(k):
            tgt[b, j, drafts[b, j]] += 6.0
    p = O.make_params(B, temperature=1.0, seed=np.array([3, 4, 5], dtype=np.uint64),
                      position=1)
    stats = [MTPStats() for _ in range(B)]
    out = BatchPicker(ctx, g).verify_round(dev_logits(tgt, "f32"), torch.from_numpy(drafts).cuda(),
                                           p, stats=stats, keys=torch.from_numpy(keys).cuda())
    vk = go.verify_keys(keys, drafts)
    assert np.array_equal(out["keys"].cpu().numpy(), vk)
    masks = np.stack([np.stack([go.mask(int(kk)) for kk in row]) for row in vk])
    ref = O.verify(tgt, k, drafts, p, mask=masks)
    acc = out["accepted"].cpu().numpy()
    assert np.array_equal(acc, ref["accepted"]), (acc, ref["accepted"])
    assert acc[1] <= 1  # "x" after "{" is masked out: the second draft is never accepted
    for b in range(B):
        s = MTPStats()
        s.record_round(k, int(ref["accepted"][b]))
        assert stats[b] == s
    g.close()
