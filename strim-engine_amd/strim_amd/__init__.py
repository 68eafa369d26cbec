"""strim_amd — MI355X-native (gfx950) token selection for strim.

The work runs in libstrim_sampler.so (hand-written HIP kernels behind the C ABI in
include/strim_sampler.h and include/strim_grammar.h). This package binds it and mirrors
the reference's Swift sampling API (sampler.py), its grammar-mask runtime (grammar.py),
its batched decode pick and MTP accounting (batch.py) and its draft-vocabulary loader
(draft_vocab.py).
"""
from . import _native
from ._native import (ECAPACITY, EEMPTY, EINVAL, ENONFINITE, FLAG_NOISE_BY_RANK,
                      FLAG_SAMPLER_COMPAT, FLAG_SCORE_NO_LSE, FLAG_TOPK_KEEP_TIES, NOISE_GUMBEL,
                      NOISE_ICDF, OK, PARAMS_DTYPE, StrimError, params_array)

__all__ = [
    "_native", "ECAPACITY", "EEMPTY", "EINVAL", "ENONFINITE", "FLAG_NOISE_BY_RANK",
    "FLAG_SAMPLER_COMPAT", "FLAG_SCORE_NO_LSE", "FLAG_TOPK_KEEP_TIES", "NOISE_GUMBEL",
    "NOISE_ICDF", "OK", "PARAMS_DTYPE", "StrimError", "params_array",
]
