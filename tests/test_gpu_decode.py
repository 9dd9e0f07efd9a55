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


# 16-bit rows have three row-pass kernels with identical results: the
# pipelined one (the default; any V, rows at any 2-byte offset), the resident
# one (V % 8 == 0) and the two-pass one. Each runs on the same inputs.
_ROW_PASS_VOCABS = [8, 40, 255, 256, 257, 1000, 2047, 2048, 3000, 4104, 8200, 8201]


@pytest.fixture
def row_pass(hip):
    def select(kind):
        hip.lib.dbs_hip_set_row_pass(kind)

    yield select
    hip.lib.dbs_hip_set_row_pass(-1)


@pytest.mark.parametrize("kind", [2, 1, 0, 5])
@pytest.mark.parametrize("seed", range(0, 30))
def test_decode_16bit_row_passes(hip, oracle, row_pass, seed, kind):
    row_pass(kind)
    case = make_case(9000 + seed, dtypes=["bf16", "f16"], vocabs=_ROW_PASS_VOCABS, scales=[0.05, 0.5, 2.0, 3.0, 8.0])
    _check(hip, oracle, case)


# Log-prob rows of every dtype take the one-read kernel where the row fits on
# chip (the default) and the two-pass kernel otherwise; both run on the same
# inputs, with the rows at every alignment (an element offset of 0-4 from the
# allocation), vocabularies at the block and on-chip limits (fp32 rows up to
# 40956 elements, 16-bit up to 81912), and one past them.
_LOGPROB_VOCABS = [2, 7, 8, 255, 256, 257, 1000, 1021, 4097, 8192, 32000, 40956, 40957, 50257, 81912, 81913]


@pytest.mark.parametrize("kind", [3, 0])
@pytest.mark.parametrize("seed", range(0, 24))
def test_decode_logprob_row_passes(hip, oracle, row_pass, seed, kind):
    row_pass(kind)
    case = make_case(9700 + seed, vocabs=_LOGPROB_VOCABS, logits=False)
    _check(hip, oracle, case, x_offset=seed % 5)


@pytest.mark.parametrize("seed", range(0, 6))
def test_decode_16bit_wide_beams(hip, oracle, seed):
    """K > 64: no shortlist (every read row is rescanned); the row pass still
    gives the logsumexp and the flags."""
    case = make_case(9500 + seed, big=True, dtypes=["bf16"], vocabs=[1000, 4104])
    _check(hip, oracle, case)


def _bf16_exact(values):
    """float32 values that bfloat16 represents exactly (checked)."""
    from tests.cases import to_bits

    v = np.asarray(values, np.float32)
    bits = to_bits(v, "bf16")
    back = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(back.view(np.uint32), v.view(np.uint32)), "not exact in bfloat16"
    return v


@pytest.mark.parametrize("m", [1.0, 1.5, 2.0, 4.0, 0.98828125, 0.5, 7.5, 63.5, 126.0, 127.0, 200.0, 2.0 ** 20,
                               1.5 * 2.0 ** 99, (2.0 - 2.0 ** -7) * 2.0 ** 127])
@pytest.mark.parametrize("kind", [-1, 5])
def test_logsumexp_table_edges(hip, oracle, row_pass, m, kind):
    """Rows whose terms sit at the edges of the bfloat16 term tables:
    magnitudes around 2^(E-25) (where fl(x - max) stops depending on x) and
    around 2^-25 (the fixed-base table's first slot), +-0, subnormals, terms
    at exp(-87) and just past it, magnitudes around 127.5 (the fixed-base
    table's last slot), -inf, maxima at and below 1 and from 127 up (the
    Cephes fallback)."""
    rng = np.random.default_rng(int(abs(np.log2(m)) * 1000) + 7)
    V = 4104
    m = float(_bf16_exact([m])[0])
    E = int(np.floor(np.log2(m)))
    specials = []
    for k in range(-28, -20):
        t = 2.0 ** (E + k)
        specials += [t, -t, t * 1.0078125, -t * 1.0078125, t * 0.9921875, -t * 0.9921875]
    for k in (-26, -25, -24):
        t = 2.0 ** k
        specials += [t, -t, t * 1.0078125, -t * 1.0078125, t * 0.9921875, -t * 0.9921875]
    specials += [-126.5, -127.0, -127.5, -128.0, -200.0]
    specials += [0.0, -0.0, 1e-40, -1e-40, 2.0 ** -133, -(2.0 ** -133), -np.inf]
    for d in (86.0, 86.5, 87.0, 87.5, 88.0, 120.0, 127.0, 128.0, 130.0):
        specials += [m - d]
    specials = [s for s in specials if not (s > m)]
    rows = []
    for r in range(6):
        base = rng.normal(0.0, 1.0, V).astype(np.float32) * np.float32(min(m, 3.0)) * 0.3
        base = np.minimum(base, np.float32(m))
        idx = rng.choice(V, size=len(specials) + 1, replace=False)
        base[idx[:-1]] = np.asarray(specials, np.float32)
        base[idx[-1]] = m
        rows.append(base)
    x = np.stack(rows).reshape(1, 3, 2, V).astype(np.float32)
    from tests.cases import to_bits

    xin = to_bits(x, "bf16")
    kw = dict(from_logits=True, eos_token=3, min_length=2, alpha=1.0)
    row_pass(kind)
    want = oracle.decode(xin, dtype="bf16", **kw)
    got = hip.decode(xin, "bf16", **kw)
    diff = first_difference(got, want)
    assert diff is None, f"m={m}: {diff}"


@pytest.mark.parametrize("V,dtype", [(151936, "bf16"), (128256, "bf16"), (155648, "bf16"), (155656, "bf16"),
                                     (151936, "f16")])
def test_decode_large_vocab_16bit(hip, oracle, V, dtype):
    """Full-size vocabularies around the on-chip limit (155648 entries; one
    more stripe falls back to the two-pass kernel)."""
    rng = np.random.default_rng(V % 1000 + 11)
    x = rng.normal(0.0, 3.0, size=(1, 3, 4, V)).astype(np.float32)
    x += (-1.1 * np.log(rng.permutation(V) + 1.0)).astype(np.float32)
    from tests.cases import to_bits

    xin = to_bits(x, dtype)
    kw = dict(from_logits=True, eos_token=V - 7, min_length=2, alpha=1.0)
    want = oracle.decode(xin, dtype=dtype, **kw)
    got = hip.decode(xin, dtype, **kw)
    diff = first_difference(got, want)
    assert diff is None, f"V={V} {dtype}: {diff}"


# A multi-step decode can run its select pass alongside the row pass (a second
# stream that follows the row pass step by step; dbs_hip_set_decode_overlap:
# 1 always, 0 never, -1 constrained decodes only). Every order gives the
# oracle's bits, with every row-pass kernel, and no wait for a step gives up.
@pytest.mark.parametrize("kind", [-1, 2, 0])
@pytest.mark.parametrize("overlap", [1, 0, -1])
@pytest.mark.parametrize("seed", range(0, 10))
def test_decode_overlapped_select(hip, oracle, row_pass, seed, overlap, kind):
    import ctypes as C

    lib = hip.lib
    row_pass(kind)
    prev = lib.dbs_hip_set_decode_overlap(overlap)
    try:
        lib.dbs_hip_profile_enable(1)  # clears the counters
        case = make_case(9700 + seed, dtypes=["bf16", "f16", "f32"], vocabs=[40, 1000, 4104, 8201])
        _check(hip, oracle, case)
        ms, n = C.c_double(), C.c_int64()
        assert lib.dbs_hip_profile_read(6, C.byref(ms), C.byref(n)) == 0
        assert n.value == 0, "a wait of the overlapped decode gave up"
    finally:
        lib.dbs_hip_profile_enable(0)
        lib.dbs_hip_set_decode_overlap(prev)
