"""Host-side mirror of strim's sampling API over the HIP path.

Names, argument meaning and error behaviour follow the reference's Swift types so a
caller (and the parity tests) read like the reference:
  SamplingConfig  <- Sources/StrimCore/SpecSampling.swift:7-15
  GenParams       <- Sources/StrimEngine/EngineAPI.swift:47-67 (sampling fields only)
  Sampler         <- Sources/StrimEngine/Sampler.swift:8-54
  SpecSampling    <- Sources/StrimCore/SpecSampling.swift:28-116
  mask_logits     <- Sources/StrimCore/TokenMask.swift:15-17
The min-p and penalty fields are extensions; their defaults are exact no-ops.
Randomness is position-keyed Philox (noise=None) or caller-injected uniforms.
"""
from __future__ import annotations

import random
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _native as N
from .ops import Context, mask_logits  # noqa: F401  (re-exported)

_MASK64 = (1 << 64) - 1


def mix(seed: int, position: int) -> int:
    """SpecSampling.mix (SpecSampling.swift:29-34), host copy for callers that key
    their own noise."""
    z = (seed + 0x9E3779B97F4A7C15 * ((position + 1) & _MASK64)) & _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return z ^ (z >> 31)


@dataclass
class SamplingConfig:
    temperature: float
    top_k: int = 0
    top_p: float = 1.0
    seed: int = 0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0

    def params(self, position: int = 0, flags: int = 0) -> np.ndarray:
        return N.params_array(1, temperature=self.temperature, top_k=self.top_k,
                              top_p=self.top_p, min_p=self.min_p,
                              repetition_penalty=self.repetition_penalty,
                              presence_penalty=self.presence_penalty,
                              frequency_penalty=self.frequency_penalty, flags=flags,
                              seed=self.seed, position=position)


@dataclass
class GenParams:
    max_tokens: int = 256
    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    seed: int | None = None
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    stop_ids: list = field(default_factory=list)

    @property
    def is_greedy(self) -> bool:
        return self.temperature <= 0


_default_ctx: dict[int, Context] = {}


def default_context(device: int = 0) -> Context:
    if device not in _default_ctx:
        _default_ctx[device] = Context(device=device, max_rows=256, max_vocab=262144)
    return _default_ctx[device]


def _words(mask, V, device):
    """Accepts packed int32 words [.., ceil(V/32)] or a bool row [.., V]."""
    if mask is None:
        return None
    if mask.dtype == torch.bool:
        from .ops import pack_mask
        return pack_mask(mask.to(device)).contiguous()
    return mask.to(device).contiguous()


class SpecSampling:
    """Position-keyed sampling and speculative verification (SpecSampling.swift:28-116)."""

    mix = staticmethod(mix)

    @staticmethod
    def sample(logits: torch.Tensor, config: SamplingConfig, index: int, mask=None,
               noise=None, noise_mode: int = N.NOISE_GUMBEL, ctx: Context | None = None) -> int:
        """Plain sample at output position `index` (SpecSampling.swift:109-116). Syncs."""
        V = logits.shape[-1]
        ctx = ctx or default_context(logits.device.index or 0)
        ids, st, _ = ctx.sample(logits.reshape(1, V).contiguous(), config.params(index),
                                mask=_words(mask, V, logits.device), noise_mode=noise_mode,
                                noise=noise)
        s = int(st.item())
        N.check(s, "SpecSampling.sample")
        return int(ids.item())

    @staticmethod
    def verify(logits: torch.Tensor, drafts, config: SamplingConfig, first_index: int,
               mask=None, noise=None, noise_mode: int = N.NOISE_GUMBEL,
               ctx: Context | None = None) -> tuple[int, int]:
        """One verify round over logits [k+1, V] (SpecSampling.swift:93-106): returns
        (accepted draft count, token decided at row `accepted`). Syncs once."""
        k1, V = logits.shape
        dev = logits.device
        ctx = ctx or default_context(dev.index or 0)
        d = torch.tensor(list(drafts), dtype=torch.int32, device=dev).reshape(1, k1 - 1)
        out = ctx.verify(logits.reshape(1, k1, V).contiguous(), d, config.params(first_index),
                         mask=_words(mask, V, dev), noise_mode=noise_mode, noise=noise)
        N.check(int(out["status"].item()), "SpecSampling.verify")
        return int(out["accepted"].item()), int(out["token"].item())


class Sampler:
    """Non-MTP sampler (Sampler.swift:8-54): keeps ties at the k-th value, indexes the
    Gumbel noise by sorted rank under top-p and scores logits without the lse shift.
    The reference advances an MLX split-key chain per call; this sampler advances a
    Philox position instead (SamplingConfig.seed, position = calls made)."""

    def __init__(self, params: GenParams, ctx: Context | None = None):
        self.temperature = params.temperature
        self.top_k = params.top_k
        self.top_p = params.top_p
        self.seed = params.seed if params.seed is not None else random.getrandbits(64)
        self._ext = dict(min_p=params.min_p, repetition_penalty=params.repetition_penalty,
                         presence_penalty=params.presence_penalty,
                         frequency_penalty=params.frequency_penalty)
        self._ctx = ctx
        self._calls = 0

    @property
    def config(self) -> SamplingConfig:
        return SamplingConfig(self.temperature, self.top_k, self.top_p, self.seed, **self._ext)

    def sample_first(self, logits: torch.Tensor) -> int:
        """Output token 0, position-keyed (Sampler.swift:29-31)."""
        return SpecSampling.sample(logits, self.config, 0, ctx=self._ctx)

    def sample(self, logits: torch.Tensor, mask=None, history: torch.Tensor | None = None) -> int:
        """Next token from one position's logits [V] (Sampler.swift:34-54). Syncs."""
        V = logits.shape[-1]
        dev = logits.device
        ctx = self._ctx or default_context(dev.index or 0)
        p = self.config.params(self._calls, flags=N.FLAG_SAMPLER_COMPAT)
        self._calls += 1
        hist = None if history is None else history.reshape(1, -1).to(dev, torch.int32).contiguous()
        ids, st, _ = ctx.sample(logits.reshape(1, V).contiguous(), p,
                                mask=_words(mask, V, dev), history=hist,
                                noise_mode=N.NOISE_GUMBEL)
        N.check(int(st.item()), "Sampler.sample")
        return int(ids.item())
