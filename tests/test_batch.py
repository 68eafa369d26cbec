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
def _budget_oracle_states(O, G):
    """RequestConstraint.budget test fixture (GrammarTests.swift:356-371) on the oracle."""
    from strim_amd.grammar import request_states

    V = G.FAKE_VOCAB
    width = len(V) + 8
    close = V.index(b"</think>")
    go = O.GrammarOracle(V, width, [G.FAKE_EOS], G.FAKE_SKIP)
    go.set_dfa(*G.object_int_dfa())
    st = request_states(1, grammar_state=-1, in_think=True, budget=3, close_id=close)
    return go, st, close


def test_oracle_thinking_budget(oracle_mod):
    # GrammarTests.swift:356-371: free while thinking under the budget, forced close id
    # once three thinking tokens are spent, free again after the close id
    import grammar_util as G

    go, st, close = _budget_oracle_states(oracle_mod, G)
    assert go.request_keys(st)[0, 0] == -1
    st = go.request_advance(st, [65])
    st = go.request_advance(st, [66])
    assert go.request_keys(st)[0, 0] == -1
    st = go.request_advance(st, [67])
    key = int(go.request_keys(st)[0, 0])
    assert key == -2 - close
    m = go.mask(key)
    bits = np.unpackbits(m.view(np.uint8), bitorder="little")
    assert bits.sum() == 1 and bits[close] == 1
    st = go.request_advance(st, [close])
    assert go.request_keys(st)[0, 0] == -1 and st["in_think"][0] == 0 and st["count"][0] == 3


def test_oracle_request_keys_walk(oracle_mod):
    # the verify walk across the thinking boundary: drafts "a", close, "{" from a request
    # one token short of its budget whose grammar starts at state 0
    import grammar_util as G
    from strim_amd.grammar import request_states

    O = oracle_mod
    V = G.FAKE_VOCAB
    go = O.GrammarOracle(V, len(V) + 8, [G.FAKE_EOS], G.FAKE_SKIP)
    nt, fl = G.object_int_dfa()
    go.set_dfa(nt, fl)
    close = V.index(b"</think>")
    st = request_states(1, grammar_state=0, in_think=True, budget=2, close_id=close)
    st["count"] = 1
    a, op, x = V.index(b"a"), V.index(b"{"), V.index(b"x")
    keys = go.request_keys(st, [[a, close, op, x]])[0].tolist()
    g1 = go.advance(0, b"{")
    # row 0 free (count 1 < 2); after "a" the budget is spent: forced close; after the
    # close id the grammar's start state; after "{" its successor; "x" then kills it
    assert keys == [-1, -2 - close, 0, g1, -1]
    # advancing by the same tokens: "x" steps the grammar dead and marks the violation
    st2 = go.request_advance(st, [x], [[a, close, op]], [3])
    assert st2["in_think"][0] == 0 and st2["g"][0] == -1 and st2["violated"][0] == 1


@pytest.mark.gpu
def test_gpu_batch_pick_equals_per_row_loop(oracle_mod, ctx):
    import torch

    import grammar_util as G
    from strim_amd.batch import BatchPicker
    from strim_amd.grammar import (DeviceGrammar, request_states, states_from_device,
                                   states_to_device)

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
    close = V.index(b"</think>")
    # grammar rows, a row without grammar, thinking rows under and at their budget
    st = request_states(B, grammar_state=[0, 5, 7, -1, 0, 1, 0, 5],
                        in_think=[0, 0, 0, 0, 1, 0, 1, 0], budget=4, close_id=close)
    st["count"] = [0, 0, 0, 0, 4, 0, 1, 0]
    T = np.array([0.0, 0.8, 1.0, 0.0, 0.7, 1.2, 0.9, 0.0])
    p = O.make_params(B, temperature=T, top_k=rng.choice([0, 20], size=B),
                      top_p=rng.choice([1.0, 0.9], size=B), seed=np.arange(B, dtype=np.uint64),
                      position=3)
    x = rng.normal(0, 2.0, size=(B, width)).astype(np.float32)
    picker = BatchPicker(ctx, g)
    sd = states_to_device(st)
    ids, status, keys = picker.pick(torch.from_numpy(x).cuda(), p, sd)
    ids, status, keys = ids.cpu().numpy(), status.cpu().numpy(), keys.cpu().numpy()
    ref_keys = go.request_keys(st)[:, 0]
    np.testing.assert_array_equal(keys, ref_keys)
    assert keys[4] == -2 - close and keys[6] == -1
    for b in range(B):  # the reference's loop: mask the row, then sample or argmax it
        m = go.mask(int(ref_keys[b]))[None]
        ref = O.sample(x[b:b + 1], p[b:b + 1], mask=m)
        assert status[b] == 0 and ids[b] == ref["token"][0], (b, ids[b], ref["token"][0])
    assert ids[4] == close
    want = go.request_advance(st, ids)
    got = states_from_device(sd)
    np.testing.assert_array_equal(got.view(np.int32), want.view(np.int32))
    g.close()


@pytest.mark.gpu
def test_gpu_batch_two_programs_one_pick(oracle_mod, ctx):
    # requests under two different grammars in one batch (GrammarEngine's programs,
    # GrammarVocab.swift:116-147): one DeviceGrammar table holds both, interned lazily;
    # every step is one BatchPicker call, and each row equals the reference's loop over
    # the row's own program (its mask, then the draw), for six steps
    import torch

    import grammar_util as G
    from strim_amd.batch import BatchPicker
    from strim_amd.grammar import DeviceGrammar, request_states, states_from_device, \
        states_to_device

    O = oracle_mod
    V = G.FAKE_VOCAB
    width = len(V) + 8
    progs = {"obj": G.object_int_dfa(), "lit": G.literal_dfa(b'{"name": "Paris"}')}
    g = DeviceGrammar(V, width, eos=[G.FAKE_EOS], skip=G.FAKE_SKIP, cache_slots=8)
    oracles, starts = {}, {}
    for name, (nt, fl) in progs.items():
        go = O.GrammarOracle(V, width, [G.FAKE_EOS], G.FAKE_SKIP)
        go.set_dfa(nt, fl)
        oracles[name] = go
        starts[name] = g.add_program(name, G.LazyTable(nt, fl))
    B = 8
    which = ["obj", "lit", "obj", "lit", "lit", "obj", "obj", "lit"]
    st = request_states(B, grammar_state=[starts[w] for w in which])
    sd = states_to_device(st)
    picker = BatchPicker(ctx, g)
    rng = np.random.default_rng(23)
    local = [0] * B  # each request's state in its program; -1 once it ended (end of turn:
    # the engine stops advancing a finished request, RequestConstraint.swift:104)
    for step in range(6):
        T = rng.choice([0.0, 0.7, 1.0], size=B)
        p = O.make_params(B, temperature=T, seed=np.arange(B, dtype=np.uint64) + 100 * step,
                          position=step)
        x = rng.normal(0, 2.0, size=(B, width)).astype(np.float32)
        ids, status, keys = picker.pick(torch.from_numpy(x).cuda(), p, sd)
        ids, status, keys = ids.cpu().numpy(), status.cpu().numpy(), keys.cpu().numpy()
        for b in range(B):
            if local[b] < 0:
                continue
            prog, ls = g._owner[int(keys[b])]
            assert prog.key == which[b] and ls == local[b], (step, b)
            m = oracles[which[b]].mask(ls)[None]
            ref = O.sample(x[b:b + 1], p[b:b + 1], mask=m)
            assert status[b] == 0 and ids[b] == ref["token"][0], (step, b)
            nl = oracles[which[b]].advance(ls, V[ids[b]]) if ids[b] != G.FAKE_EOS else -1
            local[b] = nl
        got = states_from_device(sd)
        for b in range(B):
            if local[b] >= 0:
                assert g._owner[int(got["g"][b])][1] == local[b], (step, b)
    g.close()


@pytest.mark.gpu
def test_gpu_thinking_budget(oracle_mod, ctx):
    # GrammarTests.swift:356-371 through the device state machine
    import torch

    import grammar_util as G
    from strim_amd.grammar import DeviceGrammar, states_from_device, states_to_device

    go, st, close = _budget_oracle_states(oracle_mod, G)
    V = G.FAKE_VOCAB
    g = DeviceGrammar(V, len(V) + 8, eos=[G.FAKE_EOS], skip=G.FAKE_SKIP)
    g.set_dfa(*G.object_int_dfa())
    sd = states_to_device(st)

    def key():
        return int(g.request_keys(sd)[0, 0].item())

    def emit(t):
        g.request_advance(sd, torch.tensor([t], dtype=torch.int32, device="cuda"))

    assert key() == -1
    emit(65)
    emit(66)
    assert key() == -1
    emit(67)
    assert key() == -2 - close
    m = g.mask(key()).cpu().numpy()
    bits = np.unpackbits(m.view(np.uint8), bitorder="little")
    assert bits.sum() == 1 and bits[close] == 1
    emit(close)
    assert key() == -1
    s = states_from_device(sd)
    assert s["in_think"][0] == 0 and s["count"][0] == 3
    g.close()


@pytest.mark.gpu
def test_gpu_constrained_round_records_stats(oracle_mod, ctx):
    import torch

    import grammar_util as G
    from gpu_util import dev_logits
    from strim_amd.batch import BatchPicker, SpecRounds
    from strim_amd.grammar import (DeviceGrammar, request_states, states_from_device,
                                   states_to_device)

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
    st = request_states(B, grammar_state=[0, 0, -1])
    tgt = rng.normal(0, 1.0, size=(B, k + 1, width)).astype(np.float32)
    for b in range(B):  # make the drafts likely so that some are accepted
        for j in range(k):
            tgt[b, j, drafts[b, j]] += 6.0
    p = O.make_params(B, temperature=1.0, seed=np.array([3, 4, 5], dtype=np.uint64))
    sd = states_to_device(st)
    rounds = SpecRounds(BatchPicker(ctx, g), p, states=sd, next_index=1)
    out = rounds.round(dev_logits(tgt, "f32"), torch.from_numpy(drafts).cuda(), noise_mode=0)
    vk = go.request_keys(st, drafts)
    assert np.array_equal(out["keys"].cpu().numpy(), vk)
    masks = np.stack([np.stack([go.mask(int(kk)) for kk in row]) for row in vk])
    p1 = p.copy()
    p1["position"] = 1  # SpecSampling.verify's firstIndex = sampleIndex (SpecStream.swift:249)
    ref = O.verify(tgt, k, drafts, p1, mask=masks)
    acc = out["accepted"].cpu().numpy()
    assert np.array_equal(acc, ref["accepted"]), (acc, ref["accepted"])
    assert np.array_equal(out["token"].cpu().numpy(), ref["token"])
    assert acc[1] <= 1  # "x" after "{" is masked out: the second draft is never accepted
    for b in range(B):
        s = MTPStats()
        s.record_round(k, int(ref["accepted"][b]))
        assert rounds.stats[b] == s
    # sampleIndex += accepted + 1 (SpecStream.swift:255)
    np.testing.assert_array_equal(rounds.sample_index, 1 + ref["accepted"] + 1)
    want = go.request_advance(st, ref["token"], drafts, ref["accepted"])
    np.testing.assert_array_equal(states_from_device(sd).view(np.int32), want.view(np.int32))
    # a round without drafts samples at the advanced index (SpecStream.swift:315-317)
    x0 = rng.normal(0, 1.0, size=(B, width)).astype(np.float32)
    idx_before = rounds.sample_index.copy()
    keys0 = go.request_keys(want)[:, 0]
    ids, status, _ = rounds.plain(torch.from_numpy(x0).cuda(), noise_mode=0)
    p2 = p.copy()
    p2["position"] = idx_before
    ref0 = O.sample(x0, p2, mask=np.stack([go.mask(int(kk)) for kk in keys0]))
    np.testing.assert_array_equal(ids.cpu().numpy(), ref0["token"])
    np.testing.assert_array_equal(rounds.sample_index, idx_before + 1)
    g.close()
