"""Pins of the logits-producer restatement (oracle/head_oracle.py) on the CPU."""
import numpy as np

import head_oracle as H


def _bf16(rng, shape, scale=1.0):
    return H.bf16_round(rng.normal(0.0, scale, size=shape).astype(np.float32))


def test_bf16_round_known_values():
    # nearest even at the halfway point, sign kept, NaN kept
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 1.0 + 2 ** -9,
                  np.nan], np.float32)
    want = np.array([1.0, 1.0, 1.0 + 2 ** -6, -1.0, 1.0, np.nan], np.float32)
    np.testing.assert_array_equal(H.bf16_round(x), want)
    assert H.bf16_ulp(1.0) == 2 ** -7 and H.bf16_ulp(3.0) == 2 ** -6


def test_rms_norm_power_of_two_scale_invariance():
    # with eps = 0, scaling a row by 2^j scales the mean of squares by 4^j and the inverse
    # root by 2^-j, all exactly, so the output is unchanged bit for bit
    rng = np.random.default_rng(1)
    x, w = _bf16(rng, (5, 512)), _bf16(rng, 512, 0.5)
    base = H.rms_norm(x, w, eps=0.0)
    for j in (-3, 1, 4):
        np.testing.assert_array_equal(H.rms_norm(x * np.float32(2.0 ** j), w, eps=0.0), base)


def test_rms_norm_unit_weights_give_unit_rms():
    rng = np.random.default_rng(2)
    x = _bf16(rng, (7, 1024), 3.0)
    y = H.rms_norm(x, np.ones(1024, np.float32), eps=0.0)
    rms = np.sqrt((y.astype(np.float64) ** 2).mean(-1))
    np.testing.assert_allclose(rms, 1.0, rtol=2 ** -8)


def test_rms_norm_brute_force_small():
    rng = np.random.default_rng(3)
    x, w = _bf16(rng, (3, 16)), _bf16(rng, 16)
    eps = 1e-6
    got = H.rms_norm(x, w, eps)
    for b in range(3):
        m = sum(float(v) * float(v) for v in x[b]) / 16
        inv = np.float32(1.0) / np.sqrt(np.float32(m) + np.float32(eps))
        for k in range(16):
            t = H.bf16_round(np.float32(x[b, k]) * inv)
            assert got[b, k] == H.bf16_round(np.float32(w[k]) * t)


def test_gemv_ref_hand_case_and_matmul():
    xn = np.array([[1.0, 2.0, -1.0, 0.5]], np.float32)
    W = np.array([[1.0, 0.0, 0.0, 0.0], [0.5, 0.5, 0.5, 0.5], [-2.0, 1.0, 0.0, 4.0]], np.float32)
    np.testing.assert_array_equal(H.gemv_ref(xn, W), [[1.0, 1.25, 2.0]])
    rng = np.random.default_rng(4)
    a, b = _bf16(rng, (4, 64)), _bf16(rng, (9, 64))
    np.testing.assert_allclose(H.gemv_ref(a, b), a.astype(np.float64) @ b.astype(np.float64).T)
