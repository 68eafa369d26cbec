"""Known-answer cases that pin which injected uniform drives which decision.

Each case is small enough to solve by hand; the expected answer is written next to it,
not computed by the code under test. A case puts a uniform near 1 (Gumbel noise of
about +16.6) at exactly one index, so the token that reads that index wins by a wide
margin, and puts distractors at the indices a plausible indexing mistake would read:

  A  Gumbel, no filter: noise of candidate i is u[i], i the token id
     (SpecSampling.swift:78-80, takeAlong(gumbel, ids) with ids = 0..V-1).
  B  Gumbel, top-k: candidates are sorted, but noise is still u[id]
     (SpecSampling.swift:49-54,80); a distractor sits at the sorted position.
  C  NOISE_BY_RANK under top-p: noise by sorted rank (Sampler.swift:44-51); the
     distractor sits at the winning token's id.
  D  verify, Gumbel: accept uniform is u[V] (SpecSampling.swift:83); u[0] and u[V-1]
     point the other way. Two sequences in one call also pin the [B][k+1][V+1] stride.
  E  verify, icdf: layout [B][k+1][2] = (draw, accept); swapping them flips the outcome.
  F  sample, icdf: element 0 of the [B][2] pair is the draw.

The same cases run on the oracle (tests/test_uniform_layout.py, together with mutated
oracles that must fail them) and through the HIP path (tests/test_kats_gpu.py).
"""
from __future__ import annotations

import numpy as np

V = 16
# largest float32 below 1: Gumbel transform ~ +16.6355
U_HI = np.float32(1.0 - 2.0 ** -24)
U_MID = np.float32(0.5)

# sixteen distinct logits; descending order of ids:
#   4 13 7 1 10 3 9 12 0 15 6 8 14 2 11 5
ROW = np.array([0.3, 1.2, -0.5, 0.9, 2.0, -1.0, 0.0, 1.5, -0.2, 0.6, 1.0, -0.8, 0.4, 1.8, -0.3,
                0.2], np.float32)
ORDER = [4, 13, 7, 1, 10, 3, 9, 12, 0, 15, 6, 8, 14, 2, 11, 5]


def _gumbel_row(hot: dict[int, float]) -> np.ndarray:
    u = np.full(V + 1, U_MID, np.float32)
    for i, val in hot.items():
        u[i] = val
    return u


def sample_cases():
    """(name, logits [B,V], params kwargs, noise_mode, noise, expected ids [B])."""
    cases = []
    # A: no filter -> u[id]; id 2 (rank 13) holds U_HI. Reading by sorted position would
    # give ORDER[2] = 7.
    cases.append(("A gumbel unfiltered by id", ROW[None], dict(temperature=1.0), 1,
                  _gumbel_row({2: U_HI})[None], [2]))
    # B: top-5 keeps 4 13 7 1 10 (sorted). u[10] = U_HI -> token 10 (position 4). The
    # distractor u[3] = U_HI: position 3 is token 1, and id 3 itself is outside the top 5.
    cases.append(("B gumbel top-k by id", ROW[None], dict(temperature=1.0, top_k=5), 1,
                  _gumbel_row({10: U_HI, 3: U_HI})[None], [10]))
    # C: top-p 0.9 with NOISE_BY_RANK: u[6] = U_HI is read by rank 6 = token 9. Id 6
    # (rank 10) is also in the nucleus, so an id reading would return 6.
    cases.append(("C gumbel by rank under top-p", ROW[None],
                  dict(temperature=1.0, top_p=0.9, flags=2), 1, _gumbel_row({6: U_HI})[None],
                  [9]))
    # F: two equal tokens 3 and 8 (order 3, 8); draw u = 0.75 -> the second; the accept
    # element 0.25 would pick the first.
    two = np.full((1, V), -50.0, np.float32)
    two[0, 3] = two[0, 8] = 0.0
    cases.append(("F icdf draw element 0", two, dict(temperature=1.0), 0,
                  np.array([[0.75, 0.25]], np.float32), [8]))
    return cases


def nucleus_c() -> list[int]:
    """Ids kept by top-p 0.9 on ROW at T=1 (closed form: drop a token iff the mass before
    it exceeds 0.9 of the total), for checking that case C's distractor is live."""
    w = np.exp(ROW.astype(np.float64) - ROW.max())
    o = ORDER
    before = np.concatenate([[0.0], np.cumsum(w[o])[:-1]])
    return [o[i] for i in range(V) if before[i] <= 0.9 * w.sum()]


def verify_cases():
    """(name, target [B,2,V], drafts [B,1], params kwargs, noise_mode, noise,
    expected accepted [B], expected token [B])."""
    # row 0: tokens 0 and 1 tie at the top, p = 1/2 each; the draft is 0; a rejection
    # leaves token 1 as the only residual. Row 1 (bonus): token 5 only.
    tgt = np.full((2, 2, V), -50.0, np.float32)
    tgt[:, 0, 0] = tgt[:, 0, 1] = 0.0
    tgt[:, 1, 5] = 0.0
    drafts = np.zeros((2, 1), np.int32)
    cases = []
    # D: sequence 0 accepts (u[V] = 0.25 < 1/2) while u[0] = u[V-1] = 0.75 would reject;
    # sequence 1 rejects (u[V] = 0.75) while u[0] = u[V-1] = 0.25 would accept.
    nz = np.full((2, 2, V + 1), U_MID, np.float32)
    nz[0, 0, V] = 0.25
    nz[0, 0, 0] = nz[0, 0, V - 1] = 0.75
    nz[1, 0, V] = 0.75
    nz[1, 0, 0] = nz[1, 0, V - 1] = 0.25
    cases.append(("D gumbel accept at V", tgt, drafts, dict(temperature=1.0), 1, nz, [1, 0],
                  [5, 1]))
    # E: icdf pairs (draw, accept): sequence 0 (0.9, 0.1) accepts, sequence 1 (0.1, 0.9)
    # rejects; exchanging the elements flips both.
    nz = np.zeros((2, 2, 2), np.float32)
    nz[0, 0] = (0.9, 0.1)
    nz[1, 0] = (0.1, 0.9)
    nz[:, 1] = (0.5, 0.5)
    cases.append(("E icdf (draw, accept)", tgt, drafts, dict(temperature=1.0), 0, nz, [1, 0],
                  [5, 1]))
    return cases
