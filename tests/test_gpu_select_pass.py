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

Constrained decodes (n-gram blocking of n >= 2, a repetition penalty) of at
most 16 beams take it too, with each beam's prefix, signature and n-gram list
in LDS: small vocabularies and long decodes make blocking and penalties
frequent, prefixes longer than a wavefront, and signatures of 16 to 64 words
(the most that fit).
"""

import numpy as np
import pytest

from tests.cases import first_difference, log_softmax, make_case, to_bits

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
    rng = np.random.default_rng(5)
    B, T, V = 2, 5, 2048
    x = np.log(rng.dirichlet(np.ones(V), size=(B, T, 16))).astype(np.float32)
    case.update(B=B, T=T, K=16, V=V, dtype="f32", x=x, xin=to_bits(x, "f32"))
    case["kw"] = dict(from_logits=False, eos_token=3, extra_eos=[], min_length=2, alpha=0.6,
                      no_repeat_ngram_size=0, repetition_penalty=1.0, steps=None, banned=None,
                      banned_per_example=None)
    _check_both(hip, oracle, case)


def _constrained(seed, *, T_range=(10, 41), vocabs=(3, 7, 40, 257, 1000), ks=(1, 2, 3, 4, 5, 8, 16), B_max=4):
    """A decode with n-gram blocking (n = 2, 3, 4) and/or a repetition
    penalty over T_range steps."""
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, B_max + 1))
    T = int(rng.integers(*T_range))
    K = int(rng.choice(ks))
    V = int(rng.choice(vocabs))
    dtype = str(rng.choice(["f32", "f16", "bf16"]))
    from_logits = bool(rng.integers(0, 2))
    x = rng.normal(0.0, float(rng.choice([0.5, 2.0])), size=(B, T, K, V)).astype(np.float32)
    if not from_logits:
        x = log_softmax(x)
    if rng.random() < 0.4:  # exact ties
        pool = rng.choice(x.reshape(-1), size=6)
        mask = rng.random(x.shape) < 0.05
        x[mask] = rng.choice(pool, size=int(mask.sum()))
    ngram = int(rng.choice([0, 2, 3, 4]))
    rep = float(rng.choice([1.0, 1.2, 2.0])) if ngram else float(rng.choice([1.2, 2.0]))
    eos = int(rng.integers(-1, V)) if rng.random() < 0.6 else -1
    kw = dict(
        from_logits=from_logits,
        eos_token=eos,
        extra_eos=[],
        min_length=int(rng.integers(0, 6)),
        alpha=float(rng.choice([0.0, 0.6, 1.0])),
        no_repeat_ngram_size=ngram,
        repetition_penalty=rep,
        steps=[int(s) for s in rng.integers(1, T + 1, size=B)] if rng.random() < 0.4 else None,
        banned=(rng.random(V) < 0.1).astype(np.uint8) if rng.random() < 0.25 and V > 3 else None,
        banned_per_example=(rng.random((B, V)) < 0.05).astype(np.uint8) if rng.random() < 0.25 else None,
    )
    return dict(seed=seed, B=B, T=T, K=K, V=V, dtype=dtype, x=x, xin=to_bits(x, dtype), kw=kw, invalid=False)


@pytest.mark.parametrize("seed", range(0, 40))
def test_narrow_constrained_matches_oracle(hip, oracle, seed):
    _check_both(hip, oracle, _constrained(25000 + seed))


@pytest.mark.parametrize("seed", range(0, 8))
def test_narrow_constrained_long_prefixes(hip, oracle, seed):
    """Prefixes of 70 to 100 tokens over 7 or 40 tokens: blocking at most
    steps, copies and list builds over several rounds."""
    _check_both(hip, oracle, _constrained(26000 + seed, T_range=(70, 101), vocabs=(7, 40), ks=(2, 4, 5, 8), B_max=2))


@pytest.mark.parametrize("shortlist", ["1", "3"])
@pytest.mark.parametrize("seed", range(0, 8))
def test_narrow_constrained_rescans(hip, oracle, seed, shortlist, monkeypatch):
    """Short shortlists: rows fail the check and are read in full under the
    constraints."""
    monkeypatch.setenv("DBS_HIP_SHORTLIST", shortlist)
    _check_both(hip, oracle, _constrained(27000 + seed, vocabs=(40, 257, 1000)))


@pytest.mark.parametrize("overlap", [1, 0])
@pytest.mark.parametrize("seed", range(0, 6))
def test_narrow_constrained_overlapped(hip, oracle, seed, overlap):
    lib = hip.lib
    prev = lib.dbs_hip_set_decode_overlap(overlap)
    try:
        _check_both(hip, oracle, _constrained(28000 + seed, vocabs=(40, 1000, 4104)))
    finally:
        lib.dbs_hip_set_decode_overlap(prev)
