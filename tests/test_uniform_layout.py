"""Which injected uniform drives which decision, pinned on the oracle (CPU).

The hand-solved cases in uniform_kats.py must hold on the oracle, and each of three
mutated oracles (strim_oracle.c's SO_MUTANT: Gumbel noise by the wrong index, the
accept uniform read from element 0, the icdf pair exchanged) must fail at least one of
them, so the cases can tell the right layout from each plausible wrong one.
"""
import numpy as np
import pytest

import oracle as O
import uniform_kats as K


def _sample_outcomes():
    out = []
    for name, x, kw, mode, nz, want in K.sample_cases():
        r = O.sample(x, O.make_params(len(x), **kw), noise_mode=mode, noise=nz)
        out.append((name, r["token"].tolist(), list(want)))
    return out


def _verify_outcomes():
    out = []
    for name, t, d, kw, mode, nz, want_acc, want_tok in K.verify_cases():
        r = O.verify(t, 1, d, O.make_params(len(t), **kw), noise_mode=mode, noise=nz)
        out.append((name, (r["accepted"].tolist(), r["token"].tolist()),
                    (list(want_acc), list(want_tok))))
    return out


def test_case_c_distractor_is_in_the_nucleus():
    # the by-id reading of case C would pick id 6, so id 6 must be a kept token
    assert 6 in K.nucleus_c() and K.ORDER[6] == 9


def test_uniform_layout_kats(oracle_mod):
    for name, got, want in _sample_outcomes() + _verify_outcomes():
        assert got == want, f"{name}: oracle {got}, hand-solved {want}"


@pytest.mark.parametrize("mutant,fails", [
    (1, {"A gumbel unfiltered by id", "B gumbel top-k by id", "C gumbel by rank under top-p"}),
    (2, {"D gumbel accept at V"}),
    (3, {"E icdf (draw, accept)", "F icdf draw element 0"}),
])
def test_mutated_oracles_fail_the_kats(oracle_mod, tmp_path, mutant, fails):
    lib = O.build_mutant(mutant, tmp_path / f"libstrim_oracle_mut{mutant}.so")
    with O.use_library(lib):
        failed = {name for name, got, want in _sample_outcomes() + _verify_outcomes()
                  if got != want}
    assert failed == fails, f"mutant {mutant}: failed {sorted(failed)}, expected {sorted(fails)}"
