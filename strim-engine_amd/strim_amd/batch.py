"""Batched decode integration: the whole batch's token choice in one call, and the MTP
round accounting.

The reference picks a batched decode step's tokens with a per-row loop, each row masked
by its constraint and sampled (or argmaxed) on its own, one launch and one host sync per
row (`EngineCore.pick` / `decodeBatch`, Sources/StrimEngine/EngineCore.swift:968-1011).
`BatchPicker.pick` makes it one `strim_sample` call: greedy rows are T <= 0 rows of the
same params array, constrained rows take their mask words from the device grammar
(`strim_request_keys` + `strim_grammar_masks`) and their request states (thinking
budget, grammar state) are stepped by the chosen tokens on the device
(`strim_request_advance`), so the step needs no host sync at all.
`BatchPicker.verify_round` does the same for a speculative round (`strim_verify` with
the verify-row masks) and records each request's round in its `MTPStats`, with one host
read of the B accepted counts. `SpecRounds` keeps each request's output position
(SpecStream's sampleIndex) across rounds.

`MTPStats` mirrors the reference's completed-round accounting
(Sources/StrimCore/QwenModel.swift:3-77): one-based positions, bounded counters for
depths 1..4, deeper proposals counted in overflow_proposed.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

POSITION_LIMIT = 4


def draft_depth(requested: int, remaining_tokens: int) -> int:
    """QwenModel.draftDepth (QwenModel.swift:149-151)."""
    return min(max(requested, 0), max(remaining_tokens - 1, 0))


@dataclass
class MTPStats:
    proposed: list = field(default_factory=lambda: [0] * POSITION_LIMIT)
    reached: list = field(default_factory=lambda: [0] * POSITION_LIMIT)
    accepted_prefix: list = field(default_factory=lambda: [0] * POSITION_LIMIT)
    rounds: int = 0
    emitted: int = 0
    overflow_proposed: int = 0

    def record_round(self, depth: int, accepted: int) -> None:
        """MTPStats.recordRound (QwenModel.swift:21-48): position i (one-based) is proposed
        when i <= depth, reached when the i - 1 drafts before it were accepted, and in the
        accepted prefix when i <= accepted."""
        depth = max(int(depth), 0)
        a = min(max(int(accepted), 0), depth)
        self.rounds += 1
        self.emitted += a + 1
        self.overflow_proposed += max(0, depth - POSITION_LIMIT)
        for i in range(1, POSITION_LIMIT + 1):
            if depth >= i:
                self.proposed[i - 1] += 1
                if a >= i - 1:
                    self.reached[i - 1] += 1
                if a >= i:
                    self.accepted_prefix[i - 1] += 1

    def add(self, other: "MTPStats") -> None:
        """MTPStats.add (QwenModel.swift:49-58)."""
        for name in ("proposed", "reached", "accepted_prefix"):
            mine, theirs = getattr(self, name), getattr(other, name)
            for i in range(POSITION_LIMIT):
                mine[i] += theirs[i]
        self.rounds += other.rounds
        self.emitted += other.emitted
        self.overflow_proposed += other.overflow_proposed

    def delta(self, since: "MTPStats") -> "MTPStats":
        """MTPStats.delta (QwenModel.swift:60-72): both snapshots of one stream, in order."""
        d = MTPStats()
        for name in ("proposed", "reached", "accepted_prefix"):
            setattr(d, name, [x - y for x, y in zip(getattr(self, name), getattr(since, name))])
        d.rounds = self.rounds - since.rounds
        d.emitted = self.emitted - since.emitted
        d.overflow_proposed = self.overflow_proposed - since.overflow_proposed
        return d

    def copy(self) -> "MTPStats":
        return self.delta(MTPStats())


class BatchPicker:
    """One call per decode step for the whole batch (see the module docstring).

    ctx: a `strim_amd.ops.Context`; grammar: a `strim_amd.grammar.DeviceGrammar` shared by
    the constrained requests (its one table holds every request's program, so a batch
    under several grammars is one call), or None. Constrained requests carry a device tensor of
    per-request states (`grammar.REQUEST_STATE` rows, int32 [B, 6]): the thinking phase
    and budget, the grammar state and the violation flag of RequestConstraint
    (RequestConstraint.swift:62-109). Each call reads the rows' keys from the states and
    steps the states by the emitted tokens, on the device.
    """

    def __init__(self, ctx, grammar=None):
        self.ctx = ctx
        self.grammar = grammar

    def _need_grammar(self):
        if self.grammar is None:
            raise ValueError("request states need a grammar")

    def pick(self, logits: torch.Tensor, params, states: torch.Tensor | None = None,
             noise_mode: int = 0):
        """Tokens [B] for logits [B, V] and per-row params (T <= 0 = greedy), each row
        masked by its request's next-token key (RequestConstraint.apply). states is
        advanced in place by the picked tokens (RequestConstraint.advance). Returns
        (ids, status, keys): the keys the rows were masked by."""
        mask = keys = None
        if states is not None:
            self._need_grammar()
            keys = self.grammar.request_keys(states)[:, 0].contiguous()
            mask = self.grammar.masks(keys)
        ids, status, _ = self.ctx.sample(logits, params, mask=mask, noise_mode=noise_mode)
        if states is not None:
            self.grammar.request_advance(states, ids)
        return ids, status, keys

    def verify_round(self, target: torch.Tensor, drafts: torch.Tensor, params,
                     stats: list | None = None, states: torch.Tensor | None = None,
                     depth=None, noise_mode: int = 0, **kw):
        """A speculative round over target [B, k + 1, V] and drafts [B, k]. With states,
        the k + 1 verify rows of each request are masked by its keys
        (RequestConstraint.verifyMask on the device) and the states are advanced by the
        accepted drafts and the decided token. stats: a list of B MTPStats, one per
        request, each given its round (depth defaults to k). Returns strim_verify's
        outputs plus "keys" [B, k + 1]."""
        B, k1, _ = target.shape
        mask = vkeys = None
        if states is not None:
            self._need_grammar()
            vkeys = self.grammar.request_keys(states, drafts)
            mask = self.grammar.masks(vkeys.reshape(-1)).view(B, k1, -1)
        out = self.ctx.verify(target, drafts, params, mask=mask, noise_mode=noise_mode, **kw)
        out["keys"] = vkeys
        if states is not None:
            self.grammar.request_advance(states, out["token"], drafts, out["accepted"])
        if stats is not None:
            acc = out["accepted"].cpu().numpy()  # the round's one host read
            d = np.full(B, k1 - 1) if depth is None else np.broadcast_to(np.asarray(depth), (B,))
            for b in range(B):
                stats[b].record_round(int(d[b]), int(acc[b]))
        return out


class SpecRounds:
    """SpecStream's output-position bookkeeping for B sampled requests
    (SpecStream.swift:48-55,248-256,310-317) on top of BatchPicker.

    Every request keeps `sample_index`, the output position of the token its next round
    decides first (enableSampling's nextIndex, 1 after sampleFirst took position 0). A
    verify round samples its row j at position sample_index + j (SpecSampling.verify's
    firstIndex) and then advances it by accepted + 1; a round without drafts samples at
    sample_index and advances it by one. Greedy requests (T <= 0) keep their index, as the
    reference's greedy branch has none. The per-request positions go into the params'
    `position` field, so the noise of every decision is keyed exactly as the reference
    keys it.
    """

    def __init__(self, picker: BatchPicker, params, states: torch.Tensor | None = None,
                 next_index: int = 1):
        self.picker = picker
        self.params = np.array(params, copy=True)
        self.states = states
        self.sample_index = np.full(len(self.params), next_index, dtype=np.uint64)
        self.stats = [MTPStats() for _ in range(len(self.params))]

    def _sampled(self) -> np.ndarray:
        return self.params["temperature"] > 0

    def _params_now(self) -> np.ndarray:
        p = self.params.copy()
        p["position"] = self.sample_index
        return p

    def round(self, target: torch.Tensor, drafts: torch.Tensor, noise_mode: int = 1,
              depth=None) -> dict:
        """One verify round (SpecStream.round's verify branch); returns strim_verify's
        outputs. Reads the B accepted counts on the host once."""
        out = self.picker.verify_round(target, drafts, self._params_now(), stats=self.stats,
                                       states=self.states, depth=depth, noise_mode=noise_mode)
        acc = out["accepted"].cpu().numpy().astype(np.uint64)
        self.sample_index += np.where(self._sampled(), acc + 1, 0).astype(np.uint64)
        return out

    def plain(self, logits: torch.Tensor, noise_mode: int = 1):
        """A round without drafts (SpecStream.round's depth-0 branch): one token per
        request at its sample_index."""
        ids, status, keys = self.picker.pick(logits, self._params_now(), states=self.states,
                                             noise_mode=noise_mode)
        self.sample_index += self._sampled().astype(np.uint64)
        for s in self.stats:
            s.record_round(0, 0)
        return ids, status, keys
