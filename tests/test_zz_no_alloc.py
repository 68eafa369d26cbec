"""strim_sample_noalloc (the entry point that allocates nothing) against strim_sample.

The call goes straight through the C ABI (ctypes) and must return the same ids and
statuses as strim_sample on the same inputs, bit for bit, on two calls in a row, the
second one smaller (the fixed scratch keeps the first call's contents).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev, dev_logits
from strim_amd import _native as N
from strim_amd import ops
from strim_amd import workloads as W

pytestmark = pytest.mark.gpu


def _noalloc(x, params, mask=None, history=None, history_len=None, noise_mode=0, noise=None):
    B, V = x.shape
    p = ops.host_params(params)
    ids = torch.full((B,), -7, dtype=torch.int32, device=x.device)
    st = torch.full((B,), -7, dtype=torch.int32, device=x.device)
    H = 0 if history is None else history.shape[-1]
    ms = 0 if mask is None else mask.shape[-1]
    rc = N.lib().strim_sample_noalloc(
        ops._stream(None), ops._ptr(x), ops._dtype_code(x), B, V, x.stride(0) if B > 1 else V,
        p.ctypes.data_as(ctypes.c_void_p), ops._ptr(mask), ms, ops._ptr(history),
        ops._ptr(history_len), H, noise_mode, ops._ptr(noise), ops._ptr(ids), ops._ptr(st))
    assert rc == N.OK, rc
    torch.cuda.synchronize()
    return ids.cpu().numpy(), st.cpu().numpy()


def test_noalloc_matches_strim_sample(ctx):
    # call 1: the north-star chain at full width (penalties, masks, top-p) with 40 rows
    # (two groups of the fixed scratch); call 2: a smaller, different batch
    w = W.n1()
    rng = np.random.default_rng(5)
    x = np.concatenate([w["x"]] * 5)
    hist = np.concatenate([w["history"]] * 5)
    mask = np.concatenate([w["mask"]] * 5)
    p = np.concatenate([w["params"]] * 5)
    p["seed"] = rng.integers(0, 2**63, size=len(p), dtype=np.uint64)
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        print(f"[case] noalloc call 1 n1 x5 mode={mode}", flush=True)
        xd, md, hd = dev_logits(x, "bf16"), dev(mask), dev(hist, np.int32)
        got = _noalloc(xd, p, md, hd, None, mode)
        ids, st, _ = ctx.sample(xd, p, mask=md, history=hd, noise_mode=mode)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[0], ids.cpu().numpy())
        np.testing.assert_array_equal(got[1], st.cpu().numpy())
        assert (got[1] == 0).all()
    # call 2: smaller rows and batch, cfg2's fast rows plus an empty-mask row
    V = 50000
    x2 = rng.normal(0, 2.0, size=(5, V)).astype(np.float32)
    allowed = rng.random((5, V)) < 0.5
    allowed[3] = False
    p2 = O.make_params(5, temperature=[0.0, 0.7, 1.0, 0.9, 1.3], top_k=[0, 20, 0, 0, 300],
                       top_p=[1.0, 0.9, 0.8, 1.0, 1.0], min_p=[0.0, 0.05, 0.0, 0.0, 0.0],
                       seed=rng.integers(0, 2**63, size=5, dtype=np.uint64))
    print("[case] noalloc call 2 V=50000 B=5", flush=True)
    xd, md = dev_logits(x2, "f32"), dev(W.pack_mask(allowed))
    got = _noalloc(xd, p2, md)
    ids, st, _ = ctx.sample(xd, p2, mask=md)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got[0], ids.cpu().numpy())
    np.testing.assert_array_equal(got[1], st.cpu().numpy())
    assert got[1][3] == N.EEMPTY and (np.delete(got[1], 3) == 0).all()


def test_noalloc_rejects_beyond_capacity():
    # checked on the host before any launch: no device work happens
    x = torch.zeros((1, N.NOALLOC_MAX_VOCAB + 1), dtype=torch.float32, device="cuda")
    p = ops.host_params(O.make_params(1))
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = N.lib().strim_sample_noalloc(ops._stream(None), ops._ptr(x), N.DTYPE_F32, 1,
                                      N.NOALLOC_MAX_VOCAB + 1, N.NOALLOC_MAX_VOCAB + 1,
                                      p.ctypes.data_as(ctypes.c_void_p), None, 0, None, None, 0,
                                      0, None, ops._ptr(out), None)
    assert rc == N.ECAPACITY
