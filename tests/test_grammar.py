"""On-device grammar masks (include/strim_grammar.h) against the CPU oracle.

CPU: the oracle's trie walk (oracle/grammar_oracle.c, the reference's algorithm) is pinned
against a brute-force per-token DFA walk on random vocabularies and DFAs, and against
closed-form masks of hand-built DFAs over the reference's FakeVocab fixture
(GrammarTests.swift:7-27); the verify keys follow ConstraintRowTests.verifyRows
(GrammarTests.swift:324-354). GPU: strim_grammar_masks / strim_grammar_advance equal the
oracle bit for bit, on first production and from the mask cache, and a masked strim_sample
only ever picks allowed ids.
"""
import numpy as np
import pytest

import grammar_util as G


# ------------------------------------------------------------------ oracle pins (CPU) ----
def _oracle(oracle_mod, tokens, width, eos, skip, nt, fl):
    o = oracle_mod.GrammarOracle(tokens, width, eos, skip)
    o.set_dfa(nt, fl)
    return o


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_trie_walk_matches_brute_force(oracle_mod, seed):
    rng = np.random.default_rng(seed)
    toks = G.random_vocab(rng, 1500)
    width = 1500 + 37 if seed == 0 else 1400  # wider than the vocabulary, or narrower
    skip = (rng.random(len(toks)) < 0.02).astype(np.uint8)
    eos = [3, 1499, width + 5]
    nt, fl = G.random_dfa(rng, 40)
    o = _oracle(oracle_mod, toks, width, eos, skip, nt, fl)
    for key in list(range(40)) + [-1, G_forced(7), G_forced(width + 3), 40, 1000]:
        want = G.brute_mask(toks, width, eos, skip, nt, fl, key)
        assert np.array_equal(o.mask(key), want), key


def G_forced(i):
    return -2 - i


def test_oracle_fake_vocab_closed_forms(oracle_mod):
    V = G.FAKE_VOCAB
    width = len(V) + 8
    # one literal: the non-empty prefixes of "true", then only the end-of-turn id
    nt, fl = G.literal_dfa(b"true")
    o = _oracle(oracle_mod, V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    want = sorted(i for i, t in enumerate(V)
                  if t and b"true".startswith(t) and i != G.FAKE_EOS)
    assert G.bits(o.mask(0), width) == want
    assert want == [ord("t"), V.index(b"true")]
    assert G.bits(o.mask(4), width) == [G.FAKE_EOS]
    assert o.advance(0, b"true") == 4 and o.advance(0, b"tru") == 3 and o.advance(0, b"x") == -1
    # digits: the all-digit pieces and the end-of-turn id
    nt, fl = G.digits_dfa()
    o = _oracle(oracle_mod, V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    want = sorted([i for i, t in enumerate(V) if t and t.isdigit() and i != G.FAKE_EOS]
                  + [G.FAKE_EOS])
    assert G.bits(o.mask(0), width) == want
    assert V.index(b"123") in want and V.index(b"-1") not in want
    # free and forced rows (DeviceMasks.all / only)
    assert G.bits(o.mask(-1), width) == list(range(width))
    assert G.bits(o.mask(-2 - 300), width) == [300]
    # the skipped end-of-turn piece is never walked: a literal DFA for its bytes allows its
    # single-byte prefix only
    nt, fl = G.literal_dfa(b"<|im_end|>")
    o = _oracle(oracle_mod, V, width, [], G.FAKE_SKIP, nt, fl)
    assert G.bits(o.mask(0), width) == [ord("<")]


def test_oracle_duplicates_and_trie_shape(oracle_mod):
    toks = [b"ab", b"a", b"ab", b"", b"abc", b"b", b"ab"]
    nt = np.full((1, 256), 0, dtype=np.int32)  # every byte allowed
    fl = np.array([G.CON], dtype=np.uint8)
    o = _oracle(oracle_mod, toks, 8, [], None, nt, fl)
    assert o.nodes() == 1 + 3 + 1  # root, a-b-c, b
    assert G.bits(o.mask(0), 8) == [0, 1, 2, 4, 5, 6]
    o2 = _oracle(oracle_mod, toks, 3, [], None, nt, fl)  # ids at or above width dropped
    assert G.bits(o2.mask(0), 3) == [0, 1, 2]


def test_oracle_verify_keys_follow_reference_rules(oracle_mod):
    # ConstraintRowTests.verifyRows: drafts "{" (valid), "x" (invalid after "{"), "{" (after
    # the violation): rows 0, 1 constrained; rows 2, 3 free
    V = G.FAKE_VOCAB
    width = len(V) + 8
    nt, fl = G.object_int_dfa()
    o = _oracle(oracle_mod, V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    op, x, q = V.index(b"{"), V.index(b"x"), V.index(b"\"")
    keys = o.verify_keys([0], [[op, x, op]])
    assert keys.tolist() == [[0, 1, -1, -1]]
    m0, m1 = G.bits(o.mask(0), width), G.bits(o.mask(1), width)
    assert op in m0 and x not in m0 and q in m1 and x not in m1
    assert G.bits(o.mask(-1), width) == list(range(width))
    # an unconstrained request stays free; a multi-byte draft steps through its bytes
    assert o.verify_keys([-1], [[1, 2]]).tolist() == [[-1, -1, -1]]
    assert o.verify_keys([0], [[V.index(b"{\""), V.index(b"a"), V.index(b"\":")]]).tolist() \
        == [[0, 2, 3, 5]]


# ------------------------------------------------------------------------ GPU parity ----
def _dev_grammar(tokens, width, eos, skip, nt, fl, cache_states=64):
    from strim_amd.grammar import DeviceGrammar

    g = DeviceGrammar(tokens, width, eos=eos, skip=skip, cache_slots=cache_states)
    g.set_dfa(nt, fl)
    return g


def _keys(lst):
    import torch

    return torch.tensor(lst, dtype=torch.int32, device="cuda")


@pytest.mark.gpu
@pytest.mark.parametrize("seed,count,width,S,cache", [
    (0, 1500, 1537, 40, 64),      # width past the vocabulary
    (1, 3000, 2900, 300, 16),     # narrower; states past the cache
    (2, 20000, 20000, 12, 64),
])
def test_gpu_masks_match_oracle(oracle_mod, seed, count, width, S, cache):
    rng = np.random.default_rng(seed)
    toks = G.random_vocab(rng, count)
    skip = (rng.random(count) < 0.02).astype(np.uint8)
    eos = [5, count - 1, width + 9]
    nt, fl = G.random_dfa(rng, S)
    o = _oracle(oracle_mod, toks, width, eos, skip, nt, fl)
    g = _dev_grammar(toks, width, eos, skip, nt, fl, cache_states=cache)
    keys = [int(k) for k in rng.integers(S, size=24)] + [-1, -2 - 11, -2 - (width - 1), S, S + 7]
    keys += keys[:6]  # repeated keys inside one launch
    for rep in range(2):  # first production, then (for cached states) from the cache
        got = g.masks(_keys(keys)).cpu().numpy().view(np.uint32)
        for r, k in enumerate(keys):
            assert np.array_equal(got[r], o.mask(k)), (rep, r, k)
    g.close()


@pytest.mark.gpu
def test_gpu_masks_full_vocab_and_cache_reset(oracle_mod):
    # a vocabulary of the benchmark's size: cached rows survive until the DFA changes
    rng = np.random.default_rng(7)
    V = 151936
    toks = G.random_vocab(rng, 151665, alphabet=5)
    nt, fl = G.random_dfa(rng, 64, alphabet=5, p_dead=0.3)
    o = _oracle(oracle_mod, toks, V, [151643, 151645], None, nt, fl)
    g = _dev_grammar(toks, V, [151643, 151645], None, nt, fl, cache_states=64)
    keys = [0, 3, 17, 0, 63]
    for _ in range(2):
        got = g.masks(_keys(keys)).cpu().numpy().view(np.uint32)
        for r, k in enumerate(keys):
            assert np.array_equal(got[r], o.mask(k)), k
    nt2, fl2 = G.random_dfa(rng, 64, alphabet=5, p_dead=0.3)
    g.set_dfa(nt2, fl2)
    o.set_dfa(nt2, fl2)
    got = g.masks(_keys(keys)).cpu().numpy().view(np.uint32)
    for r, k in enumerate(keys):
        assert np.array_equal(got[r], o.mask(k)), ("after set_dfa", k)
    g.close()


@pytest.mark.gpu
def test_gpu_fake_vocab_verify_rows(oracle_mod):
    import torch

    V = G.FAKE_VOCAB
    width = len(V) + 8
    nt, fl = G.object_int_dfa()
    o = _oracle(oracle_mod, V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    g = _dev_grammar(V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    op, x = V.index(b"{"), V.index(b"x")
    drafts = [[op, x, op], [V.index(b"{\""), V.index(b"a"), V.index(b"\":")], [1, 2, 3]]
    state = [0, 0, -1]
    keys, masks = g.verify_masks(_keys(state), torch.tensor(drafts, dtype=torch.int32,
                                                                 device="cuda"))
    want = o.verify_keys(state, drafts)
    assert np.array_equal(keys.cpu().numpy(), want)
    assert want.tolist() == [[0, 1, -1, -1], [0, 2, 3, 5], [-1, -1, -1, -1]]
    got = masks.cpu().numpy().view(np.uint32)
    for r, k in enumerate(want.reshape(-1)):
        assert np.array_equal(got[r], o.mask(int(k))), (r, k)
    g.close()


@pytest.mark.gpu
def test_gpu_advance_matches_oracle(oracle_mod):
    import torch

    rng = np.random.default_rng(11)
    toks = G.random_vocab(rng, 5000)
    nt, fl = G.random_dfa(rng, 50, p_dead=0.05)
    o = _oracle(oracle_mod, toks, 5000, [], None, nt, fl)
    g = _dev_grammar(toks, 5000, [], None, nt, fl)
    B, k = 300, 5
    state = rng.integers(-3, 52, size=B).astype(np.int32)  # forced, free, states, past S
    drafts = rng.integers(-2, 5002, size=(B, k)).astype(np.int32)  # ids outside the vocab
    got = g.advance(torch.from_numpy(state).cuda(), torch.from_numpy(drafts).cuda())
    assert np.array_equal(got.cpu().numpy(), o.verify_keys(state, drafts))
    g.close()


@pytest.mark.gpu
def test_gpu_masked_sampling_walk(oracle_mod, ctx):
    """The reference's random walk (GrammarTests.swift:37-55) on the device: sample under
    the produced mask, advance by the sampled token, and the grammar stays alive."""
    import torch
    from strim_amd import params_array

    V = G.FAKE_VOCAB
    width = len(V) + 8
    nt, fl = G.object_int_dfa()
    g = _dev_grammar(V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    o = _oracle(oracle_mod, V, width, [G.FAKE_EOS], G.FAKE_SKIP, nt, fl)
    rng = np.random.default_rng(5)
    state = torch.zeros(1, dtype=torch.int32, device="cuda")
    for step in range(12):
        m = g.masks(state)
        logits = torch.from_numpy(rng.normal(size=(1, width)).astype(np.float32)).cuda()
        p = params_array(1, temperature=1.0, seed=step, position=step)
        ids, status, _ = ctx.sample(logits, p, mask=m)
        tok = int(ids[0])
        assert int(status[0]) == 0
        s = int(state[0])
        assert tok in G.bits(o.mask(s), width)
        if tok == G.FAKE_EOS:
            assert fl[s] & G.ACC
            break
        state = g.advance(state, torch.tensor([[tok]], dtype=torch.int32, device="cuda"))[:, 1]
        assert int(state[0]) >= 0 and int(state[0]) == o.advance(s, V[tok])
    g.close()


@pytest.mark.gpu
def test_gpu_grammar_argument_errors():
    from strim_amd import _native as N
    from strim_amd.grammar import DeviceGrammar

    g = DeviceGrammar([b"a", b"b"], 2)
    with pytest.raises(N.StrimError):  # no DFA yet
        g.mask(0)
    with pytest.raises(N.StrimError):  # entry past the state count
        g.set_dfa(np.full((1, 256), 1, dtype=np.int32), np.array([2], dtype=np.uint8))
    with pytest.raises(N.StrimError):  # an entry below UNKNOWN
        g.set_dfa(np.full((1, 256), -3, dtype=np.int32), np.array([2], dtype=np.uint8))
    g.set_dfa(np.full((1, 256), -2, dtype=np.int32), np.array([2], dtype=np.uint8))
    with pytest.raises(N.StrimError):  # an appended entry past the new state count
        g.append_states(np.full((1, 256), 2, dtype=np.int32), np.array([2], dtype=np.uint8))
    with pytest.raises(N.StrimError):  # a target past the state count
        g.set_next([5], [1])
    with pytest.raises(N.StrimError):  # an entry past the table
        g.set_next([256], [0])
    g.close()


# ---------------------------------------------- growing table, programs, cache (GPU) ----
def _lazy_bfs(g, o, prog_key, dfa, toks, n_states_max, rng):
    """Visits the program's states breadth first through the device: each visited state's
    mask is produced with the lazy table filled on demand and compared with the oracle's
    mask of the local state; its successors (by the tokens the mask allows) are interned
    by stepping the device state with strim_grammar_advance."""
    import torch

    start = g.add_program(prog_key, dfa)
    seen = {dfa.start: start}
    queue = [dfa.start]
    checked = 0
    while queue and checked < n_states_max:
        ls = queue.pop(0)
        gs = seen[ls]
        got = g.masks(_keys([gs])).cpu().numpy().view(np.uint32)[0]
        assert np.array_equal(got, o.mask(ls)), (prog_key, ls, gs)
        checked += 1
        allowed = np.nonzero(np.unpackbits(got.view(np.uint8), bitorder="little"))[0]
        allowed = [int(t) for t in allowed if t < len(toks) and toks[t]]
        # (end-of-turn ids join an accepting state's mask without a walk)
        allowed = [t for t in allowed if o.advance(ls, toks[t]) >= 0]
        for t in rng.permutation(allowed)[:6].tolist():
            # every entry on an allowed token's path is known once the mask is resolved
            nxt = g.advance(_keys([gs]), torch.tensor([[t]], dtype=torch.int32, device="cuda"))
            ng = int(nxt[0, 1])
            nl = o.advance(ls, toks[t])
            assert ng >= 0, (ls, t, ng, nl)
            if nl not in seen:
                seen[nl] = ng
                queue.append(nl)
            assert seen[nl] == ng, (ls, t)
    return checked


@pytest.mark.gpu
def test_gpu_lazy_programs_share_one_table(oracle_mod):
    # GrammarDFA interns states as walks reach them (GrammarDFA.swift:36-58): two
    # programs start with one UNKNOWN row each and grow through the walks' pending
    # entries; every visited state's mask equals the oracle's for the program's full
    # table, and one call over keys of both programs gives both programs' rows
    rng = np.random.default_rng(31)
    count, width = 4000, 4100
    toks = G.random_vocab(rng, count)
    eos = [7, count - 1]
    ntA, flA = G.random_dfa(rng, 60, p_dead=0.1)
    ntB, flB = G.random_dfa(rng, 25, p_dead=0.3)
    flA[0] |= G.CON
    flB[0] |= G.CON
    oA = _oracle(oracle_mod, toks, width, eos, None, ntA, flA)
    oB = _oracle(oracle_mod, toks, width, eos, None, ntB, flB)
    from strim_amd.grammar import DeviceGrammar

    g = DeviceGrammar(toks, width, eos=eos, cache_slots=64)
    A, B = G.LazyTable(ntA, flA), G.LazyTable(ntB, flB)
    assert _lazy_bfs(g, oA, "A", A, toks, 12, rng) >= 5
    assert _lazy_bfs(g, oB, "B", B, toks, 12, rng) >= 3
    # the host was asked only for transitions a walk needed (the alphabet's six bytes of
    # interned states), never for a whole table row
    assert A.calls <= 6 * 60 and B.calls <= 6 * 25
    # one call, rows of both programs interleaved (and repeated): cached or produced
    ga = {ls: gs for gs, (p, ls) in g._owner.items() if p.key == "A"}
    gb = {ls: gs for gs, (p, ls) in g._owner.items() if p.key == "B"}
    la, lb = sorted(ga)[:6], sorted(gb)[:6]
    keys = [ga[s] for s in la] + [gb[s] for s in lb] + [ga[la[0]], -1, gb[lb[-1]]]
    want = [oA.mask(s) for s in la] + [oB.mask(s) for s in lb] + [oA.mask(la[0]),
                                                                  oA.mask(-1), oB.mask(lb[-1])]
    for rep in range(2):
        got = g.masks(_keys(keys)).cpu().numpy().view(np.uint32)
        for r in range(len(keys)):
            assert np.array_equal(got[r], want[r]), (rep, r, keys[r])
    g.close()


@pytest.mark.gpu
def test_gpu_pending_entries_and_unresolved_keys(oracle_mod):
    # an UNKNOWN entry met by a walk is listed once, handed out once, and met again when
    # not filled; a key walk through it gives UNRESOLVED (an all-zero row); a known entry
    # cannot be changed
    import torch
    from strim_amd import _native as N
    from strim_amd.grammar import UNKNOWN, UNRESOLVED, DeviceGrammar

    toks = [b"ab", b"a", b"b", b"ba"]
    nt = np.full((2, 256), -1, dtype=np.int32)
    nt[0, ord("a")] = 1
    nt[0, ord("b")] = UNKNOWN
    nt[1, ord("b")] = UNKNOWN
    fl = np.array([G.CON, G.CON | G.ACC], dtype=np.uint8)
    g = DeviceGrammar(toks, 8, eos=[5], cache_slots=8)
    g.set_dfa(nt, fl)
    m = g.masks(_keys([0, 0, 1]), resolve=False).cpu().numpy().view(np.uint32)
    # from 0: "a" -> 1 allowed; "ab" and "b", "ba" meet unknown entries (not allowed yet)
    assert m[0, 0] == 0b0010 and m[1, 0] == 0b0010
    assert m[2, 0] == 1 << 5  # from 1: every token meets an unknown or dead entry; eos
    p = sorted(g.pending().tolist())
    assert p == [0 * 256 + ord("b"), 1 * 256 + ord("b")]
    assert g.pending().size == 0  # handed out once
    keys = g.advance(_keys([0]), torch.tensor([[0, 1]], dtype=torch.int32, device="cuda"))
    assert keys.cpu().tolist() == [[0, UNRESOLVED, UNRESOLVED]]
    assert g.masks(keys.reshape(-1)[1:2], resolve=False).abs().sum().item() == 0
    assert g.pending().tolist() == [1 * 256 + ord("b")]  # met again: listed again
    g.set_next([1 * 256 + ord("b"), 0 * 256 + ord("b")], [0, -1])
    with pytest.raises(N.StrimError):  # a known entry keeps its value
        g.set_next([0 * 256 + ord("a")], [0])
    g.set_next([0 * 256 + ord("a")], [1])  # (the same value is accepted)
    keys = g.advance(_keys([0]), torch.tensor([[0, 1]], dtype=torch.int32, device="cuda"))
    assert keys.cpu().tolist() == [[0, 0, 1]]
    m = g.masks(_keys([0, 1]), resolve=False).cpu().numpy().view(np.uint32)
    assert m[0, 0] == 0b0011  # "ab" -> 0, "a" -> 1; "b" dead
    assert m[1, 0] == 0b1100 | (1 << 5)  # from 1: "b" -> 0, "ba" -> 1; eos
    assert g.pending().size == 0  # every entry a walk meets is known now
    g.close()


@pytest.mark.gpu
@pytest.mark.parametrize("slots", [2, 6])
def test_gpu_mask_cache_eviction(oracle_mod, slots):
    # more states than cache slots, over several calls and within one call: every row
    # equals the oracle's whichever slot it took, was evicted from or could not take
    rng = np.random.default_rng(41 + slots)
    count, width = 3000, 3000
    toks = G.random_vocab(rng, count)
    nt, fl = G.random_dfa(rng, 40, p_dead=0.2)
    o = _oracle(oracle_mod, toks, width, [3], None, nt, fl)
    g = _dev_grammar(toks, width, [3], None, nt, fl, cache_states=slots)
    for call in range(8):
        keys = [int(k) for k in rng.integers(40, size=int(rng.integers(1, 12)))]
        got = g.masks(_keys(keys)).cpu().numpy().view(np.uint32)
        for r, k in enumerate(keys):
            assert np.array_equal(got[r], o.mask(k)), (call, r, k)
        if call == 4:
            g.drop_masks(0, 20)
    g.close()


@pytest.mark.gpu
def test_gpu_duplicate_keys_produced_once(oracle_mod):
    # 1,100 rows over three keys (past the 1,024 duplicates a producing workgroup lists)
    rng = np.random.default_rng(43)
    toks = G.random_vocab(rng, 700)
    nt, fl = G.random_dfa(rng, 9)
    o = _oracle(oracle_mod, toks, 700, [1], None, nt, fl)
    g = _dev_grammar(toks, 700, [1], None, nt, fl, cache_states=4)
    keys = [2] * 1060 + [5] * 20 + [-1] * 20
    keys = [2] + [int(k) for k in rng.permutation(keys[1:])]
    for rep in range(2):
        got = g.masks(_keys(keys)).cpu().numpy().view(np.uint32)
        want = {k: o.mask(k) for k in (2, 5, -1)}
        for r, k in enumerate(keys):
            assert np.array_equal(got[r], want[k]), (rep, r, k)
    g.close()


@pytest.mark.gpu
def test_gpu_program_lru_drops_masks(oracle_mod):
    # past max_programs the least recently used program's masks are dropped; its rows are
    # produced again, still right
    rng = np.random.default_rng(47)
    toks = G.random_vocab(rng, 1200)
    from strim_amd.grammar import DeviceGrammar

    g = DeviceGrammar(toks, 1200, eos=[0], cache_slots=16, max_programs=2)
    progs = []
    for i in range(4):
        nt, fl = G.random_dfa(rng, 8, p_dead=0.1)
        fl[0] |= G.CON
        progs.append((G.LazyTable(nt, fl), _oracle(oracle_mod, toks, 1200, [0], None, nt, fl)))
    for rnd in range(2):
        for i, (dfa, o) in enumerate(progs):
            s = g.add_program(f"p{i}", dfa)
            got = g.masks(_keys([s])).cpu().numpy().view(np.uint32)[0]
            assert np.array_equal(got, o.mask(dfa.start)), (rnd, i)
        assert sum(p.resident for p in g._programs.values()) == 2
    g.close()
