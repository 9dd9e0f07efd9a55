# SPDX-License-Identifier: MIT
"""GPU parity of the decode through the C ABI (dbs_cuda_decode_ex2 /
dbs_hip_decode_ex3) against the CPU oracle on identical seeded inputs.

The bar is bit-exact for every field: tokens, parents, lengths, from_logprob,
scores, raw scores, final scores, row logsumexp and the NaN/+inf flags. (The
tolerance the north star allows for logits and 16-bit rows, 2 ulp of float32,
is not used: the engine reproduces the reference's operation order.)
"""

import os

import numpy as np
import pytest

from tests.cases import first_difference, make_case

pytestmark = pytest.mark.gpu


def _oracle_decode(oracle, case):
    kw = dict(case["kw"])
    return oracle.decode(case["xin"], dtype=case["dtype"], **kw)


def _check(hip, oracle, case, **extra):
    want = _oracle_decode(oracle, case)
    got = hip.decode(case["xin"], case["dtype"], **case["kw"], **extra)
    diff = first_difference(got, want)
    assert diff is None, f"seed {case['seed']} {case['dtype']} B{case['B']} T{case['T']} K{case['K']} V{case['V']} {case['kw']}: {diff}"


@pytest.mark.parametrize("seed", range(0, 60))
def test_decode_matches_oracle(hip, oracle, seed):
    _check(hip, oracle, make_case(1000 + seed))


@pytest.mark.parametrize("seed", range(0, 12))
def test_decode_wide_beams_and_vocab(hip, oracle, seed):
    _check(hip, oracle, make_case(5000 + seed, big=True))


@pytest.mark.parametrize("shortlist", ["0", "1", "3"])
@pytest.mark.parametrize("seed", range(0, 8))
def test_decode_rescan_paths(hip, oracle, seed, shortlist, monkeypatch):
    """Shortlists of 0, 1 or 3 entries force the exact row rescans."""
    monkeypatch.setenv("DBS_HIP_SHORTLIST", shortlist)
    _check(hip, oracle, make_case(7000 + seed))


def test_decode_without_caller_workspace(hip, oracle):
    _check(hip, oracle, make_case(42), workspace=False)


def test_ties_pick_lowest_token(hip):
    # reference tests/dbs_tests.cpp:128-142: all entries equal -> tokens 0, 1
    x = np.full((1, 1, 2, 5), -1.0, np.float32)
    out = hip.decode(x, "f32")
    assert out["tokens"][0, 0].tolist() == [0, 1]


def test_golden_two_step(hip):
    # reference tests/dbs_tests.cpp:489-508
    x = np.array([0.0, -1.0, -2.0, -3.0, -4.0, -5.0, -0.5, -0.1, -2.0, -0.2, -0.3, -2.0], np.float32)
    out = hip.decode(x.reshape(1, 2, 2, 3), "f32")
    assert out["tokens"][0, 0, 0] == 0 and out["tokens"][0, 1, 0] == 1


def test_c_api_example(hip):
    # reference examples/c_api.c: best beam tokens 0 1 with score -0.300
    x = np.array([-0.1, -1.0, -2.0, -9.0, -9.0, -9.0, -0.5, -0.2, -2.0, -0.3, -0.9, -2.0], np.float32)
    out = hip.decode(x.reshape(1, 2, 2, 3), "f32")
    assert out["tokens"][0, 0, out["parents"][0, 1, 0]] == 0 and out["tokens"][0, 1, 0] == 1
    assert out["final_scores"][0, 0] == np.float32(-0.1) + np.float32(-0.2)


def test_invalid_rows_flagged_only_when_read(hip, oracle):
    rng = np.random.default_rng(3)
    x = np.log(rng.dirichlet(np.ones(50), size=(3, 4, 2))).astype(np.float32)
    x[0, 0, 1, 7] = np.nan  # beam 1 at t = 0 is never read
    x[1, 2, 0, 3] = np.inf  # read
    x[2, 3, 1, 9] = np.nan  # read
    out = hip.decode(x, "f32")
    want = oracle.decode(x)
    assert out["invalid"].tolist() == want["invalid"].tolist() == [0, 1, 1]
