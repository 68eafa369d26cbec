"""strim_head_logits (final RMSNorm + dense lm_head on MFMA) against the CPU
restatement, and the logits it produces through the sampler against the oracle.

The bar: the normalised rows bit-exact with head_oracle.rms_norm; each logit within half
a bf16 spacing of the float64 product of the same bf16 operands, plus 1e-6 of the sum of
|products| for the float32 accumulation; the sampled tokens equal to the oracle's on the
very logits the kernel wrote (the usual tie exemption)."""
import ctypes

import numpy as np
import pytest
import torch

import head_oracle as H
import oracle as O
from gpu_util import check_sample
from strim_amd import _native as N
from strim_amd import ops

pytestmark = pytest.mark.gpu


def bf16_dev(a: np.ndarray) -> torch.Tensor:
    bits = (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def check_logits(got, xn, W, label):
    ref = H.gemv_ref(xn, W)
    tol = 0.5 * H.bf16_ulp(ref) + 1e-6 * (np.abs(xn.astype(np.float64)) @
                                          np.abs(W.astype(np.float64)).T) + 1e-30
    err = np.abs(got.astype(np.float64) - ref)
    bad = np.argwhere(err > tol)
    assert bad.size == 0, f"{label}: {len(bad)} logits off, first {bad[0]} err {err[tuple(bad[0])]:.3g}"


@pytest.mark.parametrize("B,K,V", [(1, 256, 1000), (8, 512, 4133), (20, 256, 777),
                                   (64, 256, 300), (3, 5120, 2050)])
def test_head_logits_match_fp64_product(B, K, V):
    print(f"[head] B={B} K={K} V={V}", flush=True)
    rng = np.random.default_rng(B * 1000 + K + V)
    x = H.bf16_round(rng.normal(0, 2.0, (B, K)).astype(np.float32))
    g = H.bf16_round(rng.normal(1.0, 0.2, K).astype(np.float32))
    W = H.bf16_round(rng.normal(0, 0.05, (V, K)).astype(np.float32))
    xn = torch.empty(B, K, dtype=torch.bfloat16, device="cuda")
    out = ops.head_logits(bf16_dev(x), bf16_dev(W), bf16_dev(g), eps=1e-6, xn=xn)
    torch.cuda.synchronize()
    xn_ref = H.rms_norm(x, g, 1e-6)
    np.testing.assert_array_equal(to_np(xn), xn_ref, err_msg="normalised rows")
    check_logits(to_np(out), xn_ref, W, f"B={B} K={K} V={V}")


def test_head_logits_no_norm_and_strided_output():
    # hidden already normalised (norm_weight NULL); logits rows at a stride that is not a
    # multiple of 4 (the element-wise store path) inside a larger buffer
    B, K, V, OS = 5, 512, 1030, 1037
    rng = np.random.default_rng(7)
    xn = H.bf16_round(rng.normal(0, 1.0, (B, K)).astype(np.float32))
    W = H.bf16_round(rng.normal(0, 0.05, (V, K)).astype(np.float32))
    buf = torch.full((B, OS), 7.0, dtype=torch.bfloat16, device="cuda")
    xd, Wd = bf16_dev(xn), bf16_dev(W)
    st = N.lib().strim_head_logits(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                   ctypes.c_void_p(xd.data_ptr()), K, B, K, None, 1e-6, None,
                                   ctypes.c_void_p(Wd.data_ptr()), K, V,
                                   ctypes.c_void_p(buf.data_ptr()), OS)
    assert st == 0
    torch.cuda.synchronize()
    got = to_np(buf)
    check_logits(got[:, :V], xn, W, "strided")
    assert (got[:, V:] == 7.0).all(), "wrote past V"


def test_head_logits_rejects_bad_sizes():
    lib = N.lib()
    t = torch.zeros(64 * 512, dtype=torch.bfloat16, device="cuda")
    o = torch.zeros(64 * 16, dtype=torch.bfloat16, device="cuda")
    p, po = ctypes.c_void_p(t.data_ptr()), ctypes.c_void_p(o.data_ptr())
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ok = dict(hs=512, B=4, K=512, nw=None, xn=None, ws=512, V=16, os=16)
    def call(**kw):
        a = {**ok, **kw}
        return lib.strim_head_logits(s, p, a["hs"], a["B"], a["K"], a["nw"], 1e-6, a["xn"], p,
                                     a["ws"], a["V"], po, a["os"])
    assert call() == 0
    torch.cuda.synchronize()
    assert call(K=384, hs=384, ws=384) == O.STRIM_EINVAL   # K not a multiple of 256
    assert call(B=0) == O.STRIM_EINVAL
    assert call(B=65) == O.STRIM_EINVAL
    assert call(os=15) == O.STRIM_EINVAL                    # out stride below V
    assert call(hs=500) == O.STRIM_EINVAL                   # hidden stride below K
    assert call(nw=p) == O.STRIM_EINVAL                     # norm weight without workspace


def test_head_then_sample_matches_oracle(ctx):
    # hidden -> logits on the GPU -> the north-star chain's sampler (penalties, mask,
    # T 0.8, top-p 0.9) on those logits, against the oracle on the same logits
    B, K, V, Hn = 8, 1024, 20000, 256
    rng = np.random.default_rng(11)
    x = H.bf16_round(rng.normal(0, 2.0, (B, K)).astype(np.float32))
    g = H.bf16_round(rng.normal(1.0, 0.1, K).astype(np.float32))
    W = H.bf16_round(rng.normal(0, 0.08, (V, K)).astype(np.float32))
    logits = ops.head_logits(bf16_dev(x), bf16_dev(W), bf16_dev(g))
    torch.cuda.synchronize()
    lx = to_np(logits)
    check_logits(lx, H.rms_norm(x, g, 1e-6), W, "chain")
    hist = rng.integers(0, V, size=(B, Hn)).astype(np.int32)
    allowed = rng.random((B, V)) < np.array([1.0, 0.5, 0.1, 0.02, 1.0, 0.3, 0.8, 1.0])[:, None]
    allowed[:, 0] = True
    params = O.make_params(B, temperature=0.8, top_p=0.9, presence_penalty=0.5,
                           frequency_penalty=0.3, seed=rng.integers(0, 2**63, B, dtype=np.uint64),
                           position=5)
    noise = rng.random((B, 2)).astype(np.float32)
    check_sample(ctx, lx, params, "bf16", mask=O.pack_mask(allowed), history=hist,
                 history_len=np.full(B, Hn, np.int32), noise=noise, label="head chain")


@pytest.mark.parametrize("B,K,V", [(1, 256, 1000), (8, 512, 4133), (17, 256, 777),
                                   (64, 256, 2049), (8, 1024, 151936)])
def test_head_greedy_equals_greedy_sample(ctx, B, K, V):
    # the fused pick (strim_head_greedy) against strim_sample at T = 0 (no penalties, mask
    # or filters) on the very logits the producer wrote, and against the numpy first
    # maximum of those logits; then with the logits left unwritten. Quantised weights make
    # exact ties across workgroup tiles, so the first-index rule is exercised.
    rng = np.random.default_rng(B * 7 + V)
    x = H.bf16_round(rng.normal(0, 1.0, (B, K)).astype(np.float32))
    g = H.bf16_round(rng.normal(1.0, 0.1, K).astype(np.float32))
    W = H.bf16_round((rng.integers(-3, 4, (V, K)) * 0.03125).astype(np.float32))
    W[V - 1] = W[min(V - 1, 5)]  # the same row at both ends of the vocabulary
    xd, gd, Wd = bf16_dev(x), bf16_dev(g), bf16_dev(W)
    lg = torch.empty(B, V, dtype=torch.bfloat16, device="cuda")
    ids, st = ops.head_greedy(ctx, xd, Wd, gd, out_logits=lg)
    torch.cuda.synchronize()
    lx = to_np(lg)
    assert (st.cpu().numpy() == 0).all()
    np.testing.assert_array_equal(ids.cpu().numpy(), np.argmax(lx, axis=1))
    sid, sst, _ = ctx.sample(lg, O.make_params(B, temperature=0.0))
    np.testing.assert_array_equal(ids.cpu().numpy(), sid.cpu().numpy())
    ids2, st2 = ops.head_greedy(ctx, xd, Wd, gd)  # logits not written
    np.testing.assert_array_equal(ids2.cpu().numpy(), ids.cpu().numpy())


def test_head_greedy_statuses(ctx):
    # a NaN or +inf logit gives STRIM_ENONFINITE and every logit -inf STRIM_EEMPTY, as
    # strim_sample reports them for a greedy row (ids -1)
    B, K, V = 4, 256, 700
    rng = np.random.default_rng(3)
    x = H.bf16_round(rng.normal(0, 1.0, (B, K)).astype(np.float32))
    W = H.bf16_round(rng.normal(0, 0.05, (V, K)).astype(np.float32))
    x[1, 0] = np.nan                         # row 1: every logit NaN
    x[2] = 0.0
    x[2, 0] = np.inf                         # row 2: +inf or NaN logits
    W[:, 0] = np.where(np.arange(V) % 2 == 0, 1.0, -1.0).astype(np.float32)
    x[3] = 0.0
    x[3, 0] = -np.inf
    W3 = W.copy()
    W3[:, 0] = 1.0                           # row 3: every logit -inf
    lg = torch.empty(B, V, dtype=torch.bfloat16, device="cuda")
    Wd = bf16_dev(W3)
    ids, st = ops.head_greedy(ctx, bf16_dev(x), Wd, out_logits=lg)
    sid, sst, _ = ctx.sample(lg, O.make_params(B, temperature=0.0))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(st.cpu().numpy(), sst.cpu().numpy())
    np.testing.assert_array_equal(ids.cpu().numpy(), sid.cpu().numpy())
    assert st.cpu().numpy()[0] == 0 and (st.cpu().numpy()[1:3] == O.STRIM_ENONFINITE).all()
    assert st.cpu().numpy()[3] == O.STRIM_EEMPTY
