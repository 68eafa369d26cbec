"""Draft-vocabulary table for MTP drafting: the loader and its checks, with the index map
kept on the GPU for `draft_argmax` / `Context.verify(draft_to_full=...)`.

Follows the reference loader `ModelWeights.loadDraftVocab`
(Sources/StrimCore/Weights.swift:154-210): the first existing file of the environment's
STRIM_DRAFT_VOCAB, `<model_dir>/draft_vocab.json` and `bench/draft_vocab_48k.json` under
the working directory; STRIM_DRAFT_VOCAB=off, no file, a file without `tokenizer_sha256`,
a hash that differs from `<model_dir>/tokenizer.json`'s sha256, or ids that are not `k`
strictly ascending ids below the lm_head's rows all give None (the full vocabulary).
The quantized lm_head rows the reference gathers with the ids belong to the model side
and are not part of this path.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys
from pathlib import Path

import numpy as np


def _notice(msg: str) -> None:
    print(msg, file=sys.stderr)


def check_ids(ids, k: int, rows: int) -> bool:
    """`ids.count == k`, non-empty, the last below `rows`, strictly ascending
    (Weights.swift:193-197)."""
    a = np.asarray(ids, dtype=np.int64)
    return (a.ndim == 1 and a.size == k and a.size > 0 and int(a[-1]) < rows
            and int(a[0]) >= 0 and bool(np.all(a[1:] > a[:-1])))


def load_draft_vocab(rows: int, model_dir=None, env=None, cwd=None):
    """The draft table as int32 numpy ids, or None (use the full vocabulary)."""
    env = os.environ if env is None else env
    cwd = Path.cwd() if cwd is None else Path(cwd)
    choice = env.get("STRIM_DRAFT_VOCAB") or None
    if choice == "off":
        _notice("draft vocab: off (STRIM_DRAFT_VOCAB=off); using full vocab")
        return None
    cands = [choice]
    if model_dir is not None:
        cands.append(str(Path(model_dir) / "draft_vocab.json"))
    cands.append(str(cwd / "bench" / "draft_vocab_48k.json"))
    path = next((Path(c) for c in cands if c and Path(c).is_file()), None)
    if path is None:
        _notice("draft vocab: none found; using full vocab")
        return None
    try:
        d = json.loads(path.read_text())
        k, ids = int(d["k"]), d["ids"]
    except (OSError, ValueError, KeyError, TypeError) as e:
        _notice(f"draft vocab {path}: {e}")
        return None
    want = d.get("tokenizer_sha256")
    if not want:
        _notice(f"draft vocab {path}: no tokenizer_sha256; using full vocab")
        return None
    if model_dir is not None and (Path(model_dir) / "tokenizer.json").is_file():
        got = hashlib.sha256((Path(model_dir) / "tokenizer.json").read_bytes()).hexdigest()
        if got != str(want).lower():
            _notice("draft vocab hash mismatch; using full vocab")
            return None
    if not check_ids(ids, k, rows):
        _notice(f"draft vocab {path}: need k ascending ids < {rows}; ignored")
        return None
    _notice(f"draft vocab: loaded {path}")
    return np.asarray(ids, dtype=np.int32)


def device_table(ids, device: int = 0):
    """The index map as a device int32 tensor (the `draft_to_full` argument)."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).to(f"cuda:{device}")
