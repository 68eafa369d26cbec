"""The draft-vocabulary table: the loader's checks (Weights.swift:154-210) on the CPU, and
the reference's real 32k table (tests/golden/draft_vocab_32k.npz, from the reference's
bench/draft_vocab_32k.json) through the on-device index map and a general-q verify."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from strim_amd import draft_vocab as DV

GOLD = Path(__file__).resolve().parent / "golden" / "draft_vocab_32k.npz"
# the real table's ids reach 248,076: its model's lm_head is wider than the benchmark's
# 151,936 columns; 248,320 rows stand for it
ROWS = 248320


def _real():
    z = np.load(GOLD)
    return z["ids"], int(z["k"]), str(z["tokenizer_sha256"])


def _write(d: Path, ids, k, sha):
    body = {"k": k, "ids": [int(i) for i in ids]}
    if sha is not None:
        body["tokenizer_sha256"] = sha
    (d / "draft_vocab.json").write_text(json.dumps(body))


def test_real_table_passes_the_reference_checks():
    ids, k, sha = _real()
    assert k == 32768 and ids.size == k and len(sha) == 64
    assert DV.check_ids(ids, k, ROWS)
    assert not DV.check_ids(ids, k, int(ids[-1]))  # the last id must be below the rows


def test_loader_rules(tmp_path):
    ids, k, sha = _real()
    model = tmp_path / "model"
    model.mkdir()
    tok = b'{"tokenizer": "stand-in"}'
    (model / "tokenizer.json").write_bytes(tok)
    good = hashlib.sha256(tok).hexdigest()
    env = {}
    # no file anywhere: full vocabulary
    assert DV.load_draft_vocab(ROWS, model, env, cwd=tmp_path) is None
    # a matching hash loads (upper-case hex accepted, as the reference lower-cases it)
    _write(model, ids, k, good.upper())
    got = DV.load_draft_vocab(ROWS, model, env, cwd=tmp_path)
    assert got is not None and got.dtype == np.int32 and np.array_equal(got, ids)
    # a hash of another tokenizer (the table's own) is refused
    _write(model, ids, k, sha)
    assert DV.load_draft_vocab(ROWS, model, env, cwd=tmp_path) is None
    # no hash, wrong k, unsorted, out of range: refused
    _write(model, ids, k, None)
    assert DV.load_draft_vocab(ROWS, model, env, cwd=tmp_path) is None
    _write(model, ids, k + 1, good)
    assert DV.load_draft_vocab(ROWS, model, env, cwd=tmp_path) is None
    bad = ids.copy()
    bad[[10, 11]] = bad[[11, 10]]
    _write(model, bad, k, good)
    assert DV.load_draft_vocab(ROWS, model, env, cwd=tmp_path) is None
    _write(model, ids, k, good)
    assert DV.load_draft_vocab(int(ids[-1]), model, env, cwd=tmp_path) is None
    # STRIM_DRAFT_VOCAB: off wins; a path is tried first; then bench/draft_vocab_48k.json
    assert DV.load_draft_vocab(ROWS, model, {"STRIM_DRAFT_VOCAB": "off"}, cwd=tmp_path) is None
    other = tmp_path / "other.json"
    other.write_text(json.dumps({"k": 3, "ids": [1, 5, 9], "tokenizer_sha256": good}))
    got = DV.load_draft_vocab(ROWS, model, {"STRIM_DRAFT_VOCAB": str(other)}, cwd=tmp_path)
    assert got.tolist() == [1, 5, 9]
    (tmp_path / "bench").mkdir()
    (tmp_path / "bench" / "draft_vocab_48k.json").write_text(
        json.dumps({"k": 2, "ids": [3, 4], "tokenizer_sha256": good}))
    got = DV.load_draft_vocab(ROWS, None, {}, cwd=tmp_path)
    assert got.tolist() == [3, 4]


@pytest.mark.gpu
def test_gpu_real_table_index_map_and_verify(ctx):
    from gpu_util import check_verify, dev_logits
    import oracle as O
    from strim_amd import ops
    from strim_amd import workloads as W

    ids, k_tab, _ = _real()
    table = DV.device_table(ids)
    rng = np.random.default_rng(33)
    dl = rng.normal(size=(6, k_tab)).astype(np.float32)
    got = ops.draft_argmax(dev_logits(dl, "bf16"), table).cpu().numpy()
    np.testing.assert_array_equal(got, ids[W.bf16_round(dl).argmax(-1)])
    # general-q verify over the real table at its model's width
    B, k, V = 2, 3, ROWS
    tgt = rng.normal(0, 2.0, size=(B, k + 1, V)).astype(np.float32)
    dlg = (0.6 * tgt[:, :k, :][:, :, ids] + rng.normal(0, 1.0, size=(B, k, k_tab))).astype(np.float32)
    drafts = ids[rng.integers(k_tab, size=(B, k))].astype(np.int32)
    p = O.make_params(B, temperature=0.7, seed=np.array([5, 6], dtype=np.uint64), position=2)
    for mode in (O.NOISE_ICDF, O.NOISE_GUMBEL):
        check_verify(ctx, tgt, k, drafts, p, "bf16", None, None, None, mode,
                     draft_logits=dlg, table=ids, label=f"real table mode={mode}")
