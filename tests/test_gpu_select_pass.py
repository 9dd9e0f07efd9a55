# SPDX-License-Identifier: MIT
"""The one-wavefront select pass against the oracle and against the
256-thread workgroup pass on the same inputs.

Unconstrained decodes of at most 16 beams with shortlists take one wavefront
per example by default; dbs_hip_set_select_pass(1) keeps the workgroup pass.
Both must give the oracle's bits in every path the narrow pass has: the
candidates ranked in the lanes, the running best list (more than 64
survivors: shortlists shorter than K leave tau at -inf), rows that fail the
exactness check read in full (shortlists of 1, 3 or 8 entries), carried
beams after EOS, per-example steps, the overlapped decode and logits rows.
"""

import pytest

from tests.cases import first_difference, make_case

pytestmark = pytest.mark.gpu


def _unconstrained(seed, **kw):
    case = make_case(seed, **kw)
    case["kw"] = dict(case["kw"], no_repeat_ngram_size=0, repetition_penalty=1.0)
    return case


def _check_both(hip, oracle, case):
    want = oracle.decode(case["xin"], dtype=case["dtype"], **case["kw"])
    lib = hip.lib
    prev = lib.dbs_hip_set_select_pass(1)
    try:
        wide = hip.decode(case["xin"], case["dtype"], **case["kw"])
    finally:
        lib.dbs_hip_set_select_pass(prev)
    narrow = hip.decode(case["xin"], case["dtype"], **case["kw"])
    tag = f"seed {case['seed']} {case['dtype']} B{case['B']} T{case['T']} K{case['K']} V{case['V']} {case['kw']}"
    diff = first_difference(narrow, want)
    assert diff is None, f"narrow pass, {tag}: {diff}"
    diff = first_difference(wide, want)
    assert diff is None, f"workgroup pass, {tag}: {diff}"


def test_select_pass_setting(hip):
    lib = hip.lib
    assert lib.dbs_hip_set_select_pass(2) == -2
    assert lib.dbs_hip_set_select_pass(-1) == -2
    assert lib.dbs_hip_set_select_pass(0) == 0  # automatic by default
    assert lib.dbs_hip_set_select_pass(0) == 0


@pytest.mark.parametrize("seed", range(0, 40))
def test_narrow_matches_oracle(hip, oracle, seed):
    _check_both(hip, oracle, _unconstrained(21000 + seed))


@pytest.mark.parametrize("shortlist", ["1", "3", "8"])
@pytest.mark.parametrize("seed", range(0, 10))
def test_narrow_rescans_and_long_lists(hip, oracle, seed, shortlist, monkeypatch):
    monkeypatch.setenv("DBS_HIP_SHORTLIST", shortlist)
    _check_both(hip, oracle, _unconstrained(22000 + seed, vocabs=[40, 257, 1000, 3000]))


@pytest.mark.parametrize("overlap", [1, 0])
@pytest.mark.parametrize("seed", range(0, 8))
def test_narrow_overlapped(hip, oracle, seed, overlap):
    lib = hip.lib
    prev = lib.dbs_hip_set_decode_overlap(overlap)
    try:
        _check_both(hip, oracle, _unconstrained(23000 + seed, dtypes=["bf16", "f16"], vocabs=[1000, 4104, 8201]))
    finally:
        lib.dbs_hip_set_decode_overlap(prev)


def test_narrow_many_survivors(hip, oracle, monkeypatch):
    """Sixteen beams with eight-entry shortlists: 128 survivors a step go
    through the running list, and most rows fail the check."""
    monkeypatch.setenv("DBS_HIP_SHORTLIST", "8")
    for seed in range(24000, 24012):
        case = _unconstrained(seed, vocabs=[300, 2048])
        if case["K"] != 16:
            continue
        _check_both(hip, oracle, case)
    case = _unconstrained(24100, vocabs=[2048])
    import numpy as np

    rng = np.random.default_rng(5)
    B, T, V = 2, 5, 2048
    x = np.log(rng.dirichlet(np.ones(V), size=(B, T, 16))).astype(np.float32)
    from tests.cases import to_bits

    case.update(B=B, T=T, K=16, V=V, dtype="f32", x=x, xin=to_bits(x, "f32"))
    case["kw"] = dict(from_logits=False, eos_token=3, extra_eos=[], min_length=2, alpha=0.6,
                      no_repeat_ngram_size=0, repetition_penalty=1.0, steps=None, banned=None,
                      banned_per_example=None)
    _check_both(hip, oracle, case)
