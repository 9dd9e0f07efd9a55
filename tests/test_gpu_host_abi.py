# SPDX-License-Identifier: MIT
"""The libdbs host C ABI (include/dbs.h) of libdbs_hip.so, computed on the
GPU, against the reference's own CPU library (oracle/_ref/libdbs_ref.so):
the same entry points called with identical arguments and host arrays, every
output compared bit for bit. Covers dbs_decode_batch_into(_ex) and
dbs_backward_batch_into(_ex) on the golden cases, random cases (f32/f16/bf16,
logits, EOS and extra EOS, min_length from the options and from the
constraints, banned tokens, n-gram blocking, repetition penalty, per-example
steps) and a C1-sized batch; the backward accumulates into a non-zero
buffer (+= semantics, untouched elements included); validate_inputs errors
give the reference's status and text."""

import os

import numpy as np
import pytest

from beamgrad_amd import _build
from tests.cases import first_difference, load_golden, log_softmax, make_case
from tests.host_abi import HostLib

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libdbs_ref.so")
OUT_KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
            "raw_scores", "from_logprob")


@pytest.fixture(scope="module")
def libs():
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref is not built")
    return HostLib(_build.lib_path()), HostLib(REF_LIB)


def _run_both(libs, fn, **opts):
    res = []
    for lib in libs:
        h = lib.create(**opts)
        try:
            res.append(fn(lib, h))
        finally:
            lib.destroy(h)
    return res


def _options(K, kw, validate=0):
    return dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], validate_inputs=validate)


def _decode_both(libs, xin, K, dtype, kw, *, ex=True, cons_kw=None, validate=0):
    def fn(lib, h):
        if kw.get("extra_eos"):
            assert lib.set_extra_eos(h, kw["extra_eos"]) == 0, lib.error()
        keep = {}
        cons = None
        if cons_kw is not None:
            cons = HostLib.constraints(keep=keep, **cons_kw)
        st, out = lib.decode(h, xin, K, dtype=dtype, from_logits=kw["from_logits"], steps=kw["steps"],
                             constraints=cons, ex=ex)
        return st, out, lib.error()

    return _run_both(libs, fn, **_options(K, kw, validate))


def _constraints_of(kw, min_length_override=None):
    if kw.get("banned") is None and not kw.get("no_repeat_ngram_size") and kw.get("repetition_penalty", 1.0) <= 1.0 \
            and min_length_override is None:
        return None
    return dict(banned=kw.get("banned"), no_repeat_ngram_size=int(kw.get("no_repeat_ngram_size") or 0),
                repetition_penalty=float(kw.get("repetition_penalty", 1.0)),
                min_length=-1 if min_length_override is None else min_length_override)


def _check_decode(libs, xin, K, dtype, kw, **more):
    (s0, o0, e0), (s1, o1, e1) = _decode_both(libs, xin, K, dtype, kw, **more)
    assert (s0, e0) == (s1, e1)
    assert s0 == 0, e0
    keys = OUT_KEYS + (("row_lse",) if "row_lse" in o0 else ())
    diff = first_difference(o0, o1, keys)
    assert diff is None, diff
    return o0


def _check_backward(libs, trace, V, K, kw, xin=None, dtype="f32", steps=None, seed=0):
    B, T = trace["parents"].shape[:2]
    rng = np.random.default_rng(seed)
    # a buffer with values, including -0.0, that the backward must leave alone
    # where it adds nothing
    init = rng.normal(size=(B, T, K, V)).astype(np.float32)
    init[rng.random(init.shape) < 0.1] = -0.0
    gf = rng.normal(size=(B, K)).astype(np.float32)
    grads = dict(grad_final=gf, grad_final_raw=rng.normal(size=(B, K)).astype(np.float32),
                 grad_scores=rng.normal(size=(B, T, K)).astype(np.float32),
                 grad_raw=rng.normal(size=(B, T, K)).astype(np.float32))
    runs = [dict(ex=False, grad_final=gf), dict(ex=True, grad_final=gf), dict(ex=True, **grads)]
    if kw["from_logits"]:
        runs = [dict(ex=True, grad_final=gf, logits=xin, logits_dtype=dtype, row_lse=trace["row_lse"]),
                dict(ex=True, logits=xin, logits_dtype=dtype, row_lse=trace["row_lse"], **grads)]
    for run in runs:
        def fn(lib, h):
            st, g = lib.backward(h, trace, V, init, steps=steps, **run)
            return st, g, lib.error()

        (s0, g0, e0), (s1, g1, e1) = _run_both(libs, fn, **_options(K, kw))
        assert (s0, e0) == (s1, e1)
        assert s0 == 0, e0
        bad = np.argwhere(g0.view(np.uint32) != g1.view(np.uint32))
        assert bad.size == 0, (sorted(run), tuple(bad[0]), g0[tuple(bad[0])], g1[tuple(bad[0])])


@pytest.mark.parametrize("case", load_golden(), ids=lambda c: f"golden{c['index']}")
def test_golden_cases_decode_and_backward(libs, case):
    kw = dict(case["kw"])
    if kw.get("banned_per_example") is not None:
        pytest.skip("per-example banned masks are not part of the host ABI")
    out = _check_decode(libs, case["xin"], case["K"], case["dtype"], kw, cons_kw=_constraints_of(kw))
    _check_backward(libs, out, case["V"], case["K"], kw, xin=case["xin"], dtype=case["dtype"], steps=kw["steps"],
                    seed=case["index"])


@pytest.mark.parametrize("seed", range(24))
def test_random_cases_decode_and_backward(libs, seed):
    case = make_case(9900 + seed, allow_invalid=False)
    kw = dict(case["kw"])
    kw["banned_per_example"] = None
    K = case["K"]
    ml = None
    if seed % 3 == 0:
        ml = int(seed % 5)  # min_length from the constraints overrides the options'
    out = _check_decode(libs, case["xin"], K, case["dtype"], kw, cons_kw=_constraints_of(kw, ml))
    if case["dtype"] == "f32" and not kw["from_logits"] and ml is None and _constraints_of(kw) is None:
        # the plain f32 entry point gives the same bits
        _check_decode(libs, case["xin"], K, "f32", kw, ex=False)
    _check_backward(libs, out, case["V"], K, kw, xin=case["xin"], dtype=case["dtype"], steps=kw["steps"], seed=seed)


def test_c1_sized_batch(libs):
    """C1's shape and options: fp32 log-probs [8, 32, 4, 32000], EOS 2, alpha 0.6."""
    rng = np.random.default_rng(1001)
    x = log_softmax(rng.normal(0.0, 2.0, size=(8, 32, 4, 32000)).astype(np.float32))
    kw = dict(from_logits=False, eos_token=2, extra_eos=[], min_length=0, alpha=0.6, steps=None)
    out = _check_decode(libs, x, 4, "f32", kw)
    _check_backward(libs, out, 32000, 4, kw, seed=1)


@pytest.mark.parametrize("from_logits", [False, True])
def test_validate_inputs_errors_match(libs, from_logits):
    rng = np.random.default_rng(5)
    B, T, K, V = 3, 4, 3, 50
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    if not from_logits:
        x = log_softmax(x)
    x[1, 2, :, 7] = np.nan  # example 1 reads a NaN at step 2
    x[2, 3, 1, 9] = np.inf
    kw = dict(from_logits=from_logits, eos_token=-1, extra_eos=[], min_length=0, alpha=0.0, steps=None)
    (s0, _, e0), (s1, _, e1) = _decode_both(libs, x, K, "f32", kw, validate=1)
    assert s0 == s1 == -1
    assert e0 == e1 and "NaN or +inf" in e0 and e0.startswith("example 1:"), (e0, e1)
    # without validation both decode it (NaN/+inf entries are never selected)
    _check_decode(libs, x, K, "f32", kw)


def test_handle_reused_across_shapes(libs):
    """One handle, calls of different sizes in a row (its device buffers grow
    and are reused)."""
    ours, ref = libs
    rng = np.random.default_rng(3)
    hs = [lib.create(beam_size=4, eos_token=3, length_penalty_alpha=0.6) for lib in libs]
    try:
        for B, T, V in ((2, 5, 300), (5, 9, 1000), (1, 3, 40)):
            x = log_softmax(rng.normal(0, 2, size=(B, T, 4, V)).astype(np.float32))
            outs = []
            for lib, h in zip(libs, hs):
                st, o = lib.decode(h, x, 4)
                assert st == 0, lib.error()
                outs.append(o)
            assert first_difference(outs[0], outs[1], OUT_KEYS + ("row_lse",)) is None
    finally:
        for lib, h in zip(libs, hs):
            lib.destroy(h)


@pytest.mark.parametrize("seed", range(4))
def test_logits_backward_in_small_chunks(libs, monkeypatch, seed):
    """The from-logits backward works a bounded chunk of examples at a time
    (at most 1 GiB of logits and gradient rows on the device); with the
    bound forced down to one example per chunk the bits are still the
    reference library's."""
    case = make_case(9950 + seed, dtypes=["bf16", "f32"], logits=True, allow_invalid=False)
    while case["B"] < 2:
        case = make_case(case["seed"] + 100, dtypes=["bf16", "f32"], logits=True, allow_invalid=False)
    kw = dict(case["kw"])
    kw["banned_per_example"] = None
    out = _check_decode(libs, case["xin"], case["K"], case["dtype"], kw, cons_kw=_constraints_of(kw))
    monkeypatch.setenv("DBS_HIP_TEST_BACKWARD_CHUNK_BYTES", "1")
    _check_backward(libs, out, case["V"], case["K"], kw, xin=case["xin"], dtype=case["dtype"], steps=kw["steps"],
                    seed=seed)
