"""Writes tests/golden/draft_vocab_32k.npz from the reference's real draft-vocabulary table
(bench/draft_vocab_32k.json in the reference tree): the ascending ids and the tokenizer
sha256 it is bound to. Run in a tree where the reference is present:

    python tests/golden/make_draft_vocab_fixture.py /path/to/reference
"""
import json
import sys
from pathlib import Path

import numpy as np

src = Path(sys.argv[1]) / "bench" / "draft_vocab_32k.json"
d = json.loads(src.read_text())
out = Path(__file__).resolve().parent / "draft_vocab_32k.npz"
np.savez_compressed(out, ids=np.asarray(d["ids"], dtype=np.int32), k=np.int32(d["k"]),
                    tokenizer_sha256=np.array(d["tokenizer_sha256"]))
print(out, len(d["ids"]))
