"""CPU restatement of the logits producer: the decode step's final RMSNorm and dense
lm_head linear (Sources/StrimCore/QwenModel.swift:202-212: store.rmsNorm then
OpTimer.linear; Sources/StrimCore/Weights.swift:244-255 `linear` = matmul(x, w^T) for
dense weights, :270-273 `rmsNorm` = MLXFast.rmsNorm(x, weight, eps 1e-6)).

TEST INFRASTRUCTURE ONLY: the parity checker for strim_head_logits. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it.

rms_norm follows the published MLX algorithm as the kernel states it: inv = 1 /
sqrt(mean(x^2) + eps) in float32, out = w * bf16(x * inv) rounded to bf16. The MLX fork the
reference pins (mlx-swift 0.32.3-strim.1, not under /root/reference) is absent, so the
exact rounding order of its Metal kernel is parity unpinned; this restatement sums the
squares in float64. It is pinned by: eps = 0 power-of-two scale invariance (exact),
unit weights giving rows of unit RMS to bf16 precision, and a brute-force float64
evaluation on small rows. gemv_ref is the float64 product of the bf16 operands, the
reference for the float32-accumulated MFMA result, and is pinned against numpy's own
matmul and a hand-computed case in tests/test_head_oracle.py.
"""
from __future__ import annotations

import numpy as np


def bf16_round(x) -> np.ndarray:
    """float32 -> nearest-even bf16, returned as float32 (NaN stays NaN)."""
    a = np.ascontiguousarray(np.asarray(x, np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = np.nan
    return out


def rms_norm(x, w, eps: float = 1e-6) -> np.ndarray:
    """x: float32 [B, K] (bf16 values), w: float32 [K] (bf16 values) -> bf16-valued
    float32 [B, K]."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    K = x.shape[-1]
    ss = (x.astype(np.float64) ** 2).sum(-1)
    mean = (ss / K).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    t = bf16_round(x * inv[:, None])
    return bf16_round(w[None, :] * t)


def gemv_ref(xn, W) -> np.ndarray:
    """float64 logits of bf16-valued operands: xn [B, K], W [V, K] -> [B, V]."""
    return np.asarray(xn, np.float64) @ np.asarray(W, np.float64).T


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bf16 values at |x| (2^-126 -> 2^-133 below the normal range)."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)
