"""Seeded synthetic inputs for the five benchmark configurations.

Host generation uses numpy PCG64. Logits are returned as float32 arrays holding
exact bfloat16 values (bf16 rows) so the same numbers can feed the device path and
any host-side check. Shapes and distributions follow the configuration table:
  cfg1  B=1,  V=151,936 fp32  N(0,3^2) + 5 spikes at +15, 256-token history,
        repetition 1.05 -> T 0.7 -> top-k 20 -> top-p 0.95, one uniform per row
  cfg2  B=8,  bf16 N(0,2.5^2) + Zipf(1.1) bias over a seeded permutation, 4,096-token
        Zipf history, per-row T {0.6,0.8,1.0} / top-k {0,20,50} / top-p U[0.8,1],
        min-p 0.05, presence 0.5, frequency 0.3
  cfg3  cfg2 logits + packed masks (densities 0.01/1/10/30 %, clustered or scattered;
        one row allows one token; one row's top-p mass is entirely masked), T 0.8,
        top-p 0.9
  cfg4  verify B=4, k=3: target [4,4,V] bf16, draft [4,3,32,768] bf16 over a seeded
        ascending injective table, drafts sampled from q = softmax(draft/T), T 0.7
  cfg5  B=64 bf16: 70 % rows N(0,2^2), 30 % rows with one +20 logit; 2,048-token
        history; 5 % masks; T 0.8, top-k 40, top-p 0.95, min-p 0.02, per-row seed
  n1    the north-star chain: cfg2 logits and penalty history + cfg3 masks, T 0.8,
        top-p 0.9 (no top-k, no min-p)
"""
from __future__ import annotations

import numpy as np

from ._native import params_array

V_DEFAULT = 151_936
VD_DEFAULT = 32_768


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16 value (as float32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).copy()


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 arrays of exact bf16 values -> uint16 bit patterns."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def pack_mask(allowed: np.ndarray) -> np.ndarray:
    """bool [..., V] -> uint32 [..., ceil(V/32)]: bit (i & 31) of word (i >> 5)."""
    allowed = np.asarray(allowed, dtype=bool)
    V = allowed.shape[-1]
    W = (V + 31) // 32
    pad = np.zeros(allowed.shape[:-1] + (W * 32,), dtype=bool)
    pad[..., :V] = allowed
    packed = np.packbits(pad.reshape(allowed.shape[:-1] + (W, 4, 8)), axis=-1,
                         bitorder="little")
    return np.ascontiguousarray(packed.reshape(allowed.shape[:-1] + (W, 4))).view(
        np.uint32).reshape(allowed.shape[:-1] + (W,))


def zipf_ids(rng, n, V, perm, a=1.1):
    r = rng.zipf(a, size=n).astype(np.int64) - 1
    return perm[r % V].astype(np.int32)


def cfg1(seed=1, V=V_DEFAULT):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, size=(1, V)).astype(np.float32)
    spikes = rng.choice(V, size=5, replace=False)
    x[0, spikes] = 15.0
    hist = rng.integers(0, V, size=(1, 256), dtype=np.int32)
    params = params_array(1, temperature=0.7, top_k=20, top_p=0.95, repetition_penalty=1.05,
                          seed=seed, position=0)
    noise = rng.random((1, 2), dtype=np.float32)
    greedy = params.copy()
    greedy["temperature"] = 0.0
    return dict(x=x, dtype="f32", params=params, greedy_params=greedy, history=hist,
                history_len=np.full(1, 256, np.int32), mask=None, noise=noise, spikes=spikes)


def _cfg2_logits(rng, B, V, sigma=2.5):
    perm = rng.permutation(V)
    bias = np.empty(V, dtype=np.float32)
    bias[perm] = -1.1 * np.log(np.arange(V, dtype=np.float64) + 1.0)
    x = rng.normal(0.0, sigma, size=(B, V)).astype(np.float32) + bias[None, :]
    return bf16_round(x), perm


def cfg2(seed=2, B=8, V=V_DEFAULT, H=4096):
    rng = np.random.default_rng(seed)
    x, perm = _cfg2_logits(rng, B, V)
    hist = np.stack([zipf_ids(rng, H, V, perm) for _ in range(B)])
    T = np.array([0.6, 0.8, 1.0], np.float32)[np.arange(B) % 3]
    K = np.array([0, 20, 50], np.int32)[(np.arange(B) // 3) % 3]
    P = rng.uniform(0.8, 1.0, size=B).astype(np.float32)
    params = params_array(B, temperature=T, top_k=K, top_p=P, min_p=0.05,
                          presence_penalty=0.5, frequency_penalty=0.3,
                          seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=7)
    noise = rng.random((B, 2), dtype=np.float32)
    return dict(x=x, dtype="bf16", params=params, history=hist.astype(np.int32),
                history_len=np.full(B, H, np.int32), mask=None, noise=noise)


def _cfg3_masks(rng, x_proc, T=0.8, P=0.9):
    """cfg3's allow masks over B rows: densities 0.01/1/10/30 % (clustered runs of 64 for
    the first four rows, scattered for the next four), one row allowing exactly one token
    and one row whose top-p nucleus (of the penalised logits x_proc at T, P) is masked."""
    B, V = x_proc.shape
    dens = [0.0001, 0.01, 0.10, 0.30]
    allowed = np.zeros((B, V), dtype=bool)
    for r in range(B):
        d = dens[r % 4]
        n = max(1, int(round(d * V)))
        if (r // 4) % 2 == 0:  # clustered: seeded contiguous runs of 64
            run = 64
            starts = rng.choice(V // run, size=max(1, n // run), replace=False) * run
            for s0 in starts:
                allowed[r, s0:s0 + run] = True
        else:  # scattered
            allowed[r, rng.choice(V, size=n, replace=False)] = True
    # edge: one row allows exactly one token
    allowed[B - 2] = False
    allowed[B - 2, int(rng.integers(0, V))] = True
    # edge: one row's top-p mass (at T, P) lies entirely in masked tokens
    r = B - 1
    l = x_proc[r] / np.float32(T)
    order = np.argsort(-l.astype(np.float64), kind="stable")
    w = np.exp(l[order].astype(np.float64) - l[order[0]])
    cut = int(np.searchsorted(np.cumsum(w) / w.sum(), P)) + 1
    allowed[r] = rng.random(V) < 0.3
    allowed[r, order[:cut]] = False
    return allowed


def cfg3(seed=3, B=8, V=V_DEFAULT):
    rng = np.random.default_rng(seed)
    x, _ = _cfg2_logits(rng, B, V)
    allowed = _cfg3_masks(rng, x)
    params = params_array(B, temperature=0.8, top_p=0.9,
                          seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=11)
    noise = rng.random((B, 2), dtype=np.float32)
    return dict(x=x, dtype="bf16", params=params, history=None, history_len=None,
                mask=pack_mask(allowed), allowed=allowed, noise=noise)


def penalised(x, history, presence=0.5, frequency=0.3):
    """The penalty stage of the chain on float32 values (v - f*c - p for ids seen c > 0
    times), each step one float32 rounding as the kernels round it."""
    out = np.array(x, dtype=np.float32, copy=True)
    for r in range(out.shape[0]):
        c = np.bincount(history[r], minlength=out.shape[1])[:out.shape[1]].astype(np.float32)
        hit = c > 0
        v = out[r, hit] - np.float32(frequency) * c[hit]
        out[r, hit] = v - np.float32(presence)
    return out


def n1(seed=6, B=8, V=V_DEFAULT, H=4096):
    """The north-star chain: cfg2's logits and 4,096-id Zipf penalty history (presence
    0.5, frequency 0.3), cfg3's masks (every density, both placements, the one-token row
    and the masked-nucleus row), then T 0.8 and top-p 0.9 without top-k or min-p, one
    uniform per row."""
    rng = np.random.default_rng(seed)
    x, perm = _cfg2_logits(rng, B, V)
    hist = np.stack([zipf_ids(rng, H, V, perm) for _ in range(B)]).astype(np.int32)
    allowed = _cfg3_masks(rng, penalised(x, hist))
    params = params_array(B, temperature=0.8, top_p=0.9, presence_penalty=0.5,
                          frequency_penalty=0.3,
                          seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=13)
    noise = rng.random((B, 2), dtype=np.float32)
    return dict(x=x, dtype="bf16", params=params, history=hist,
                history_len=np.full(B, H, np.int32), mask=pack_mask(allowed), allowed=allowed,
                noise=noise)


def cfg4(seed=4, B=4, k=3, V=V_DEFAULT, Vd=VD_DEFAULT, T=0.7):
    rng = np.random.default_rng(seed)
    tgt, perm = _cfg2_logits(rng, B * (k + 1), V)
    tgt = tgt.reshape(B, k + 1, V)
    table = np.sort(rng.choice(V, size=Vd, replace=False)).astype(np.int32)
    dl = bf16_round(rng.normal(0.0, 2.5, size=(B, k, Vd)).astype(np.float32))
    # bias the draft toward the target so drafts are sometimes accepted
    dl = bf16_round(0.5 * dl + 0.8 * tgt[:, :k, :][:, :, table])
    q = dl.astype(np.float64) / T
    q = np.exp(q - q.max(-1, keepdims=True))
    q /= q.sum(-1, keepdims=True)
    drafts = np.zeros((B, k), np.int32)
    for b in range(B):
        for j in range(k):
            drafts[b, j] = table[rng.choice(Vd, p=q[b, j])]
    params = params_array(B, temperature=T, seed=rng.integers(0, 2**63, size=B, dtype=np.uint64),
                          position=3)
    return dict(target=tgt, draft_logits=dl, table=table, drafts=drafts, params=params, k=k)


def cfg5(seed=5, B=64, V=V_DEFAULT, H=2048):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 2.0, size=(B, V)).astype(np.float32)
    dom = rng.random(B) < 0.3
    for r in np.nonzero(dom)[0]:
        x[r, int(rng.integers(0, V))] = 20.0
    x = bf16_round(x)
    hist = rng.integers(0, V, size=(B, H), dtype=np.int32)
    allowed = rng.random((B, V)) < 0.05
    # the 2,048-token history penalises as in cfg2 (presence 0.5, frequency 0.3)
    params = params_array(B, temperature=0.8, top_k=40, top_p=0.95, min_p=0.02,
                          presence_penalty=0.5, frequency_penalty=0.3,
                          seed=rng.integers(0, 2**63, size=B, dtype=np.uint64), position=0)
    return dict(x=x, dtype="bf16", params=params, history=hist,
                history_len=np.full(B, H, np.int32), mask=pack_mask(allowed), allowed=allowed,
                noise=None)


def algorithmic_bytes(B, V, dtype_bytes, mask=False, H=0, noise_floats=0):
    """Bytes one sampling step must move: logits, mask words, history, params,
    noise and the output id (the out_probs validation output is excluded)."""
    return (B * V * dtype_bytes + (B * ((V + 31) // 32) * 4 if mask else 0) + B * H * 4
            + B * (48 + 4 * noise_floats + 4))


# ---------------------------------------------------------------------------------
# grammar masks: a vocabulary of the configuration's size and a JSON-string DFA
# ---------------------------------------------------------------------------------
GRAMMAR_COUNT = 151_665  # ids with byte strings; the logits width stays V_DEFAULT
GRAMMAR_EOS = (151_643, 151_645)


def grammar_vocab(seed=12, count=GRAMMAR_COUNT):
    """Synthetic byte-level BPE vocabulary: the 256 single bytes, then pieces of 2..64
    bytes (mean about 6.5) over printable ASCII with a leading space on a third of them
    and a sprinkling of quotes, backslashes and UTF-8 continuation bytes; the end-of-turn
    ids are control tokens (skipped by the mask)."""
    rng = np.random.default_rng(seed)
    toks = [bytes([b]) for b in range(256)]
    n = count - 256
    lens = np.minimum(64, 2 + rng.geometric(0.22, size=n))
    alpha = np.frombuffer(b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789"
                          b"_.,:;-+=()[]{}<>/!?'", dtype=np.uint8)
    special = np.frombuffer(b"\"\\\x80\xa0\xc3\xe4", dtype=np.uint8)
    for i in range(n):
        L = int(lens[i])
        b = alpha[rng.integers(len(alpha), size=L)]
        if rng.random() < 0.33:
            b[0] = 0x20
        if rng.random() < 0.08:
            b[rng.integers(L)] = special[rng.integers(len(special))]
        toks.append(b.tobytes())
    skip = np.zeros(count, dtype=np.uint8)
    for e in GRAMMAR_EOS:
        toks[e] = b"<|ctrl%d|>" % e
        skip[e] = 1
    return toks, skip


def json_string_dfa():
    """A JSON string value: 0 -"-> 1 (inside); 1: bytes >= 0x20 except quote and backslash
    stay, backslash -> 2, quote -> 3 (accepting, done); 2: one escape character -> 1."""
    nt = np.full((4, 256), -1, dtype=np.int32)
    nt[0, ord('"')] = 1
    nt[1, 0x20:] = 1
    nt[1, ord('"')] = 3
    nt[1, ord("\\")] = 2
    for c in b'"\\/bfnrtu':
        nt[2, c] = 1
    flags = np.array([2, 2, 2, 1], dtype=np.uint8)
    return nt, flags


def json_object_dfa():
    """The object {"name":"<string>","age":<integer>} without whitespace: the literal
    {"name":" (states 0..8), the string (9; 10 after a backslash), the literal ,"age":
    after the string's closing quote (11..18), the first digit (18), more digits (19),
    the closing brace after a lone 0 (21) and the end (20, accepting). 22 states, so a
    mask walks from the caches rather than from an LDS copy of the table.
    Returns (next_table, flags, in_string_state)."""
    lit1, lit2 = b'{"name":"', b',"age":'
    S = len(lit1)            # inside the string
    E = S + 1                # after a backslash
    L2 = E + 1               # after the closing quote: expects lit2
    D0 = L2 + len(lit2)      # the first digit
    D = D0 + 1               # more digits
    F = D + 1                # done (accepting)
    Z = F + 1                # after a lone 0: only the brace
    nt = np.full((Z + 1, 256), -1, dtype=np.int32)
    for i, c in enumerate(lit1):
        nt[i, c] = i + 1 if i + 1 < len(lit1) else S
    nt[S, 0x20:] = S
    nt[S, ord('"')] = L2
    nt[S, ord("\\")] = E
    for c in b'"\\/bfnrtu':
        nt[E, c] = S
    for i, c in enumerate(lit2):
        nt[L2 + i, c] = L2 + i + 1
    for c in b"123456789":
        nt[D0, c] = D
    nt[D0, ord("0")] = Z
    nt[D, ord("0"):ord("9") + 1] = D
    nt[D, ord("}")] = F
    nt[Z, ord("}")] = F
    flags = np.full(Z + 1, 2, dtype=np.uint8)
    flags[F] = 1
    return nt, flags, S
