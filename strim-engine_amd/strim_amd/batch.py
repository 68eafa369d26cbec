"""Batched decode integration: the whole batch's token choice in one call, and the MTP
round accounting.

The reference picks a batched decode step's tokens with a per-row loop, each row masked
by its constraint and sampled (or argmaxed) on its own, one launch and one host sync per
row (`EngineCore.pick` / `decodeBatch`, Sources/StrimEngine/EngineCore.swift:968-1011).
`BatchPicker.pick` makes it one `strim_sample` call: greedy rows are T <= 0 rows of the
same params array, constrained rows take their mask words from the device grammar
(`strim_grammar_masks`) and their grammar states are stepped by the chosen tokens on
the device (`strim_grammar_advance`), so the step needs no host sync at all.
`BatchPicker.verify_round` does the same for a speculative round (`strim_verify` with
the verify-row masks) and records each request's round in its `MTPStats`, with one host
read of the B accepted counts.

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
    the constrained rows, or None.
    """

    def __init__(self, ctx, grammar=None):
        self.ctx = ctx
        self.grammar = grammar

    def pick(self, logits: torch.Tensor, params, keys: torch.Tensor | None = None,
             noise_mode: int = 0):
        """Tokens [B] for logits [B, V] and per-row params (T <= 0 = greedy). keys: device
        int32 [B] grammar keys (state, -1 free, -2 - id forced) or None. Returns
        (ids, status, next_keys); next_keys are the keys after each row's token."""
        mask = None
        if keys is not None:
            if self.grammar is None:
                raise ValueError("keys need a grammar")
            mask = self.grammar.masks(keys)
        ids, status, _ = self.ctx.sample(logits, params, mask=mask, noise_mode=noise_mode)
        nxt = None
        if keys is not None:
            nxt = self.grammar.advance(keys, ids.view(-1, 1))[:, 1].contiguous()
        return ids, status, nxt

    def verify_round(self, target: torch.Tensor, drafts: torch.Tensor, params,
                     stats: list | None = None, keys: torch.Tensor | None = None,
                     depth=None, noise_mode: int = 0, **kw):
        """A speculative round over target [B, k + 1, V] and drafts [B, k]. With keys, the
        k + 1 verify rows of each request are masked by its grammar (verifyMask on the
        device). stats: a list of B MTPStats, one per request, each given its round
        (depth defaults to k). Returns strim_verify's outputs plus "keys" [B, k + 1]."""
        B, k1, _ = target.shape
        mask = None
        vkeys = None
        if keys is not None:
            if self.grammar is None:
                raise ValueError("keys need a grammar")
            vkeys, words = self.grammar.verify_masks(keys, drafts)
            mask = words.view(B, k1, -1)
        out = self.ctx.verify(target, drafts, params, mask=mask, noise_mode=noise_mode, **kw)
        out["keys"] = vkeys
        if stats is not None:
            acc = out["accepted"].cpu().numpy()  # the round's one host read
            d = np.full(B, k1 - 1) if depth is None else np.broadcast_to(np.asarray(depth), (B,))
            for b in range(B):
                stats[b].record_round(int(d[b]), int(acc[b]))
        return out
