"""CPU checks of the C ABI library: it loads, exports every declared symbol, and
validates host-checkable arguments synchronously (no GPU work is issued)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(strim_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from strim_amd import _native as N

    L = N.lib()
    decl = _declared_symbols()
    assert set(decl) == set(N.EXPORTS)
    for name in decl:
        assert hasattr(L, name), name
    assert "gfx950" in N.version()


def test_default_params_are_reference_defaults():
    from strim_amd import _native as N

    p = N.SamplingParams()
    N.lib().strim_default_params(ctypes.byref(p))
    assert (p.temperature, p.top_k, p.top_p, p.min_p) == (1.0, 0, 1.0, 0.0)
    assert (p.repetition_penalty, p.presence_penalty, p.frequency_penalty) == (1.0, 0.0, 0.0)
    assert (p.flags, p.seed, p.position) == (0, 0, 0)


@pytest.mark.parametrize("field,value,ok", [
    ("temperature", 0.0, True), ("temperature", -0.1, True), ("temperature", np.nan, False),
    ("top_p", 1.0, True), ("top_p", 0.0, False), ("top_p", 1.01, False),
    ("top_k", 0, True), ("top_k", -1, False),
    ("min_p", 1.0, True), ("min_p", -0.01, False),
    ("repetition_penalty", 0.0, False), ("presence_penalty", np.inf, False),
    ("flags", 7, True), ("flags", 8, False),
])
def test_check_params_mirrors_request_validation(field, value, ok):
    # GenParams as the engine takes it (T <= 0 greedy, EngineAPI.swift:66) and the
    # ChatRequest.parse ranges (Sources/StrimServer/ChatRequest.swift:150-160)
    from strim_amd import _native as N

    p = N.params_array(3)
    p[field][1] = value
    assert (N.check_params(p) == N.OK) == ok


def test_sample_rejects_bad_arguments_synchronously():
    from strim_amd import _native as N

    L = N.lib()
    dummy = ctypes.c_void_p(16)
    # NULL context / logits / params / outputs -> EINVAL before any device call
    assert L.strim_sample(None, None, dummy, 1, 8, 100, 100, dummy, None, 0, None, None, 0, 0,
                          None, dummy, None, None) == N.EINVAL
    assert L.strim_verify(None, None, dummy, 1, 1, 1, 100, None, 0, None, dummy, dummy, None, 0,
                          None, None, 0, 0, None, dummy, dummy, None, None, None) == N.EINVAL
    assert L.strim_mask_logits(None, dummy, 7, 1, 10, 10, None, 0, dummy) == N.EINVAL
    assert L.strim_draft_argmax(None, dummy, 1, 1, 0, 0, None, dummy) == N.EINVAL
    assert L.strim_ctx_create(ctypes.byref(ctypes.c_void_p()), 0, 0, 10) == N.EINVAL
    assert L.strim_ctx_destroy(None) == N.EINVAL


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from strim_amd import _native as N

    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setattr(N, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(RuntimeError, match="not built"):
        N.lib()


def test_params_layout_matches_oracle():
    import oracle
    from strim_amd import _native as N

    assert N.PARAMS_DTYPE == oracle.PARAMS_DTYPE
    assert ctypes.sizeof(N.SamplingParams) == N.PARAMS_DTYPE.itemsize == 48


def test_workload_shapes():
    from strim_amd import workloads as W

    w = W.cfg3(V=4096)
    assert w["mask"].shape == (8, 128) and w["mask"].dtype == np.uint32
    assert w["allowed"][6].sum() == 1
    unpacked = ((w["mask"][:, :, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(8, -1)
    np.testing.assert_array_equal(unpacked.astype(bool), w["allowed"])
    w4 = W.cfg4(V=5000, Vd=512)
    assert np.all(np.diff(w4["table"]) > 0) and w4["table"][-1] < 5000
    assert np.isin(w4["drafts"], w4["table"]).all()


def test_mirror_mix_matches_oracle():
    import oracle
    from strim_amd.sampler import mix

    for s, p in [(0, 0), (1, 2), (2**64 - 1, 2**63), (1234, 7)]:
        assert mix(s, p) == oracle.mix(s, p)
