"""A second, independent restatement of the filtering/draw semantics in plain Python
(full stable sort, no selection tricks), used only to cross-check the C oracle on tiny
rows. It follows the same reference lines: Sources/StrimCore/SpecSampling.swift:44-68
and Sources/StrimEngine/Sampler.swift:37-53.
"""
from __future__ import annotations

import math

import numpy as np


def process(x, params, mask=None, hist=()):
    """Penalties -> mask -> temperature, each float32 step rounded separately."""
    f32 = np.float32
    T, rep = f32(params["temperature"]), f32(params["repetition_penalty"])
    pres, freq = f32(params["presence_penalty"]), f32(params["frequency_penalty"])
    V = len(x)
    cnt = [0] * V
    for h in hist:
        if 0 <= h < V:
            cnt[h] += 1
    out = []
    for i in range(V):
        v = f32(x[i])
        if cnt[i] > 0:
            v = f32(v / rep) if v > 0 else f32(v * rep)
            v = f32(v - f32(freq * f32(cnt[i])))
            v = f32(v - pres)
        if mask is not None and not mask[i]:
            out.append(-math.inf)
            continue
        out.append(float(v if T <= 0 else f32(v / T)))
    return out


def filtered(l, params):
    """-> list of (id, prob) for the kept set in (l desc, id asc) order."""
    V = len(l)
    allowed = [i for i in range(V) if l[i] > -math.inf]
    m = max(l[i] for i in allowed)
    order = sorted(allowed, key=lambda i: (-l[i], i))
    if params["min_p"] > 0:
        lmp = math.log(float(np.float32(params["min_p"])))
        order = [i for i in order if l[i] - m >= lmp]
    K = int(params["top_k"])
    if 0 < K < V:
        if params["flags"] & 1:  # keep ties
            if len(order) > K:
                kth = l[order[K - 1]]
                order = [i for i in order if l[i] >= kth]
        else:
            order = order[:K]
    w = [math.exp(l[i] - m) for i in order]
    P = float(np.float32(params["top_p"]))
    if P < 1.0:
        S = sum(w)
        before, cut = 0.0, len(order)
        for j, wj in enumerate(w):
            if before / S - P > 0:
                cut = j
                break
            before += wj
        order, w = order[:cut], w[:cut]
    S = sum(w)
    return [(i, wi / S) for i, wi in zip(order, w)]


def icdf_draw(kept, u):
    S = sum(p for _, p in kept)
    t = float(u) * S
    c = 0.0
    for i, p in kept:
        c += p
        if c > t:
            return i
    return kept[-1][0]
