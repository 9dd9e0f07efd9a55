# SPDX-License-Identifier: MIT
"""Per-example beams, EOS tokens and minimum lengths through the device ABI
(DBSCudaDecodeArgs.beam_sizes_per_example / eos_tokens_per_example /
min_lengths_per_example, reference include/dbs_cuda.h:80-85). The oracle is
each example decoded alone with its own options on its first beams[b] rows,
its slots past them empty (pinned against the reference library's
dbs_decode_batch_variable in tests/test_oracle.py); compared bit for bit."""

import numpy as np
import pytest

from beamgrad_amd import _abi
from tests.cases import first_difference, make_case

pytestmark = pytest.mark.gpu


def _per_example(case, seed, which):
    rng = np.random.default_rng(10_000 + seed)
    B, K, V = case["B"], case["K"], case["V"]
    beams = [int(v) for v in rng.integers(1, K + 1, size=B)] if "beams" in which else None
    eos = [int(v) for v in rng.integers(-1, V, size=B)] if "eos" in which else None
    mins = [int(v) for v in rng.integers(0, 6, size=B)] if "min" in which else None
    return beams, eos, mins


@pytest.mark.parametrize("which", [("beams",), ("eos",), ("min",), ("beams", "eos", "min")])
@pytest.mark.parametrize("seed", range(12))
def test_per_example_options_match_oracle(hip, oracle, seed, which):
    case = make_case(7000 + seed)
    kw = dict(case["kw"])
    beams, eos, mins = _per_example(case, seed, which)
    if eos is not None and kw["eos_token"] < 0:
        # extra EOS tokens need an EOS token somewhere; they count per example
        kw["extra_eos"] = [int(eos[0]) if eos[0] >= 0 else 0]
    got = hip.decode(case["xin"], case["dtype"], beams=beams, eos_tokens=eos, min_lengths=mins, **kw)
    want = oracle.decode_per_example(case["xin"], dtype=case["dtype"], beams=beams, eos_tokens=eos,
                                     min_lengths=mins, **kw)
    assert first_difference(got, want) is None, (case["seed"], which)


@pytest.mark.parametrize("seed", range(6))
def test_per_example_options_large_vocab_16bit(hip, oracle, seed):
    """Rows through the persistent 16-bit row passes (and the overlapped
    select pass) with per-example options."""
    case = make_case(7100 + seed, vocabs=[4096, 20000], dtypes=["bf16", "f16"], logits=True, allow_invalid=False)
    kw = dict(case["kw"])
    beams, eos, mins = _per_example(case, seed, ("beams", "eos", "min"))
    if kw["eos_token"] < 0:
        kw["extra_eos"] = []
    got = hip.decode(case["xin"], case["dtype"], beams=beams, eos_tokens=eos, min_lengths=mins, **kw)
    want = oracle.decode_per_example(case["xin"], dtype=case["dtype"], beams=beams, eos_tokens=eos,
                                     min_lengths=mins, **kw)
    assert first_difference(got, want) is None


@pytest.mark.parametrize("seed", range(6))
def test_step_api_with_per_example_options(hip, oracle, seed):
    rng = np.random.default_rng(seed)
    B, T, K, V = 3, 5, 4, 23
    x = rng.normal(0, 2, (B, T, K, V)).astype(np.float32)
    x = (x - np.log(np.exp(x).sum(-1, keepdims=True))).astype(np.float32)
    beams, eos, mins = [int(v) for v in rng.integers(1, K + 1, B)], [2, -1, 5], [0, 2, 4]
    # (no extra EOS tokens: without prefixes the step API reports a carried
    # finished beam's token as the example's EOS token)
    got = hip.steps(x, "f32", eos_token=2, alpha=0.6, beams=beams, eos_tokens=eos, min_lengths=mins)
    want = oracle.decode_per_example(x, dtype="f32", beams=beams, eos_tokens=eos, min_lengths=mins, eos_token=2,
                                     alpha=0.6)
    keys = ("tokens", "parents", "lengths", "scores", "raw_scores", "from_logprob", "final_scores",
            "final_raw_scores", "final_lengths")
    assert first_difference(got, want, keys) is None


@pytest.mark.parametrize("seed", range(6))
def test_backward_with_per_example_beams(hip, oracle, seed):
    case = make_case(7200 + seed, allow_invalid=False, dtypes=["f32"], logits=False)
    kw = dict(case["kw"])
    B, T, K, V = case["B"], case["T"], case["K"], case["V"]
    beams, eos, mins = _per_example(case, seed, ("beams",))
    trace = oracle.decode_per_example(case["xin"], dtype="f32", beams=beams, **kw)
    rng = np.random.default_rng(seed)
    gf = rng.normal(size=(B, K)).astype(np.float32)
    got = hip.backward(trace, V, alpha=kw["alpha"], steps=kw["steps"], beams=beams, grad_final=gf)
    want = oracle.backward(trace, V, alpha=kw["alpha"], steps=kw["steps"], grad_final=gf)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # a slot past its example's beams carries nothing, whatever the trace holds there
    bad = {k: np.array(v) for k, v in trace.items()}
    for b in range(B):
        if beams[b] < K:
            bad["parents"][b, :, beams[b]:] = 0
            bad["tokens"][b, :, beams[b]:] = 0
            bad["from_logprob"][b, :, beams[b]:] = 1
    got_bad = hip.backward(bad, V, alpha=kw["alpha"], steps=kw["steps"], beams=beams, grad_final=gf)
    assert np.array_equal(got_bad.view(np.uint32), want.view(np.uint32))
    draws = hip.path_gradient(trace, V, gf, alpha=kw["alpha"], steps=kw["steps"], beams=beams)
    assert np.array_equal(draws.view(np.uint32),
                          oracle.path_gradient(trace, V, gf, alpha=kw["alpha"], steps=kw["steps"]).view(np.uint32))


def test_per_example_arrays_are_validated(hip):
    x = np.zeros((2, 3, 4, 9), np.float32)
    for bad in (dict(beams=[0, 2]), dict(beams=[1, 5]), dict(eos_tokens=[-2, 1]), dict(eos_tokens=[9, 1]),
                dict(min_lengths=[0, -1])):
        assert hip.decode(x, "f32", expect_status=True, **bad) == _abi.STATUS_INVALID_ARGUMENT, bad
    # extra EOS tokens need an EOS token: the scalar one or per example
    assert hip.decode(x, "f32", extra_eos=(3,), expect_status=True) == _abi.STATUS_INVALID_ARGUMENT
    assert hip.decode(x, "f32", extra_eos=(3,), eos_tokens=[-1, 2], expect_status=True) == _abi.STATUS_OK
