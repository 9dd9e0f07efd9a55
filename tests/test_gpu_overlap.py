# SPDX-License-Identifier: MIT
"""The overlapped decode's contract: the select pass follows the row pass
step by step on a second stream (one per caller stream), waits for exactly the
rows the row pass reads, and reports a wait that gave up as an error instead
of reading rows that may not be written.

* per-example beams below K (the row pass reads, and counts, only the
  example's beams): bit-exact vs the oracle, and no wait gives up;
* a forced give-up (DBS_HIP_TEST_WAIT_GIVE_UP=1 makes every wait need one
  row more than the row pass ever counts, with a 10 us bound, so every kernel
  still exits normally): invalid_input[b] == 2, the example's trace is
  padding, and a synchronising call (dbs_cuda_set_synchronization(1), or the
  legacy DBS_CUDA_DEBUG_SYNC=1 environment switch) returns LAUNCH_FAILED;
* two host threads decoding on two streams at once, each bit-exact.
"""

import ctypes as C
import os
import threading

import numpy as np
import pytest
import torch

from beamgrad_amd import _abi
from tests.cases import first_difference, make_case

pytestmark = pytest.mark.gpu


def _timeouts(lib) -> int:
    ms, n = C.c_double(), C.c_int64()
    assert lib.dbs_hip_profile_read(6, C.byref(ms), C.byref(n)) == 0
    return n.value


@pytest.fixture
def overlap_on(hip):
    lib = hip.lib
    prev = lib.dbs_hip_set_decode_overlap(1)
    lib.dbs_hip_profile_enable(1)  # clears the counters
    try:
        yield lib
    finally:
        lib.dbs_hip_profile_enable(0)
        lib.dbs_hip_set_decode_overlap(prev)


def _big_case(seed):
    """A multi-step 16-bit from-logits case for the persistent row passes."""
    return make_case(seed, vocabs=[4096, 20000], dtypes=["bf16", "f16"], logits=True, allow_invalid=False)


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("constrained", [False, True])
def test_per_example_beams_below_k_do_not_wait(hip, oracle, overlap_on, seed, constrained):
    case = _big_case(7300 + seed) if not constrained else make_case(7350 + seed, allow_invalid=False)
    kw = dict(case["kw"])
    if constrained:
        kw["no_repeat_ngram_size"], kw["repetition_penalty"] = 2, 1.2
    B, K = case["B"], case["K"]
    rng = np.random.default_rng(seed)
    beams = [int(v) for v in rng.integers(1, K + 1, size=B)]
    beams[0] = max(1, K - 1) if K > 1 else 1  # at least one example below K where K allows
    got = hip.decode(case["xin"], case["dtype"], beams=beams, **kw)
    want = oracle.decode_per_example(case["xin"], dtype=case["dtype"], beams=beams, **kw)
    assert first_difference(got, want) is None, (case["seed"], beams)
    assert _timeouts(overlap_on) == 0, "a wait of the overlapped decode gave up"


def _forced_give_up(monkeypatch):
    monkeypatch.setenv("DBS_HIP_TEST_WAIT_GIVE_UP", "1")


def _check_abandoned(res, B, T, K):
    assert (res["invalid"] == 2).all(), res["invalid"]
    assert (res["tokens"] == -1).all() and (res["parents"] == -1).all()
    assert (res["lengths"] == 0).all() and (res["from_logprob"] == 0).all()
    assert np.isneginf(res["final_scores"]).all() and np.isneginf(res["final_raw_scores"]).all()
    assert (res["final_lengths"] == 0).all()


@pytest.mark.parametrize("seed", range(3))
def test_given_up_wait_is_reported_async(hip, overlap_on, monkeypatch, seed):
    case = _big_case(7400 + seed)
    kw = dict(case["kw"])
    _forced_give_up(monkeypatch)
    status, res = hip.decode(case["xin"], case["dtype"], with_status=True, **kw)
    assert status == _abi.STATUS_OK  # asynchronous call: the flags carry the failure
    if case["T"] > 1:
        _check_abandoned(res, case["B"], case["T"], case["K"])
        assert _timeouts(overlap_on) >= case["B"]


@pytest.mark.parametrize("how", ["api", "env_legacy", "env"])
def test_given_up_wait_fails_a_synchronising_call(hip, oracle, overlap_on, monkeypatch, how):
    case = _big_case(7410)
    while case["T"] < 2:
        case = _big_case(case["seed"] + 1)
    kw = dict(case["kw"])
    lib = overlap_on
    _forced_give_up(monkeypatch)
    prev = lib.dbs_cuda_get_synchronization()
    try:
        if how == "api":
            assert lib.dbs_cuda_set_synchronization(1) == 0
        elif how == "env_legacy":
            monkeypatch.setenv("DBS_CUDA_DEBUG_SYNC", "1")
        else:
            monkeypatch.setenv("DBS_CUDA_SYNC_CHECK", "1")
        status, res = hip.decode(case["xin"], case["dtype"], with_status=True, **kw)
        assert status == _abi.STATUS_LAUNCH_FAILED, lib.dbs_cuda_status_string(status)
        _check_abandoned(res, case["B"], case["T"], case["K"])
    finally:
        lib.dbs_cuda_set_synchronization(prev)
    # the switches off again: the same decode completes and matches the oracle
    monkeypatch.delenv("DBS_HIP_TEST_WAIT_GIVE_UP")
    monkeypatch.delenv("DBS_CUDA_DEBUG_SYNC", raising=False)
    monkeypatch.delenv("DBS_CUDA_SYNC_CHECK", raising=False)
    got = hip.decode(case["xin"], case["dtype"], **kw)
    assert first_difference(got, oracle.decode(case["xin"], dtype=case["dtype"], **kw)) is None


def test_legacy_debug_sync_is_read_per_call(hip, monkeypatch):
    lib = hip.lib
    assert lib.dbs_cuda_get_synchronization() == 0
    monkeypatch.setenv("DBS_CUDA_DEBUG_SYNC", "1")
    # the flag getter reports the API flag only (reference semantics); the
    # environment switch acts on the calls
    assert lib.dbs_cuda_get_synchronization() == 0
    x = np.zeros((1, 2, 2, 9), np.float32)
    assert hip.decode(x, "f32", expect_status=True) == _abi.STATUS_OK


def test_two_threads_two_streams(hip, oracle, overlap_on):
    cases = [_big_case(7500 + i) for i in range(2)]
    wants = [oracle.decode(c["xin"], dtype=c["dtype"], **c["kw"]) for c in cases]
    results = [[None] * 4 for _ in cases]
    errors = []
    barrier = threading.Barrier(2)

    def run(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                barrier.wait()
                for rep in range(4):
                    results[i][rep] = hip.decode(cases[i]["xin"], cases[i]["dtype"], **cases[i]["kw"])
        except BaseException as e:  # reported below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for i, c in enumerate(cases):
        for rep in range(4):
            assert first_difference(results[i][rep], wants[i]) is None, (i, rep)
    assert _timeouts(overlap_on) == 0


def _torch_case(seed):
    """A multi-step 16-bit from-logits case (decoded overlapped by default)
    as a torch tensor, with its options."""
    import beamgrad_amd as bg

    case = _big_case(seed)
    while case["T"] < 2:
        case = _big_case(case["seed"] + 1)
    # no constraints: the options below carry EOS, min_length and alpha only
    case["kw"] = kw = dict(case["kw"], banned=None, banned_per_example=None, no_repeat_ngram_size=0,
                           repetition_penalty=1.0)
    x = torch.from_numpy(case["xin"].view(np.int16)).cuda()
    x = x.view(torch.bfloat16 if case["dtype"] == "bf16" else torch.float16)
    eos = [kw["eos_token"], *kw["extra_eos"]] if kw["eos_token"] >= 0 and kw["extra_eos"] else kw["eos_token"]

    def opts(validate):
        return bg.BeamOptions(beam_size=case["K"], eos_token=eos, min_length=kw["min_length"],
                              length_penalty_alpha=kw["alpha"], validate_inputs=validate)

    return case, x, opts


@pytest.mark.parametrize("validate", [True, False])
def test_given_up_wait_raises_from_the_torch_ops(oracle, monkeypatch, validate):
    """decode / final_scores raise a RuntimeError of their own (not the NaN
    ValueError) whether or not the inputs are validated: with validate the
    example's flag says 2, without it the decode's fault word is read back.
    The same calls without the knob match the oracle."""
    import beamgrad_amd as bg

    case, x, opts = _torch_case(7430)
    kw = case["kw"]
    _forced_give_up(monkeypatch)
    with pytest.raises(RuntimeError, match="gave up waiting for the row pass"):
        bg.decode(x, opts(validate), kw["steps"], from_logits=True)
    with pytest.raises(RuntimeError, match="gave up waiting for the row pass"):
        bg.final_scores(x.detach().clone().requires_grad_(True), opts(validate), kw["steps"], from_logits=True)
    monkeypatch.delenv("DBS_HIP_TEST_WAIT_GIVE_UP")
    out = bg.decode(x, opts(validate), kw["steps"], from_logits=True)
    want = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    got = {k: getattr(out, k).cpu().numpy() for k in ("final_scores", "final_raw_scores", "scores", "raw_scores")}
    for k in ("final_lengths", "tokens", "parents", "lengths"):
        got[k] = getattr(out, k).cpu().numpy().astype(np.int32)
    assert first_difference(got, want, tuple(got)) is None
    scores = bg.final_scores(x, opts(validate), kw["steps"], from_logits=True)
    assert np.array_equal(scores.detach().cpu().numpy().view(np.uint32), want["final_scores"].view(np.uint32))


@pytest.mark.parametrize("validate", [0, 1])
def test_given_up_wait_fails_the_host_abi_decode(oracle, monkeypatch, validate):
    """dbs_decode_batch_into_ex on the GPU returns DBS_ERROR_RUNTIME with its
    own error text for a given-up wait, and decodes as the oracle without
    the knob."""
    from beamgrad_amd import _build
    from tests.host_abi import HostLib

    case, _x, _opts = _torch_case(7440)
    kw = case["kw"]
    lib = HostLib(_build.lib_path())
    h = lib.create(beam_size=case["K"], eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                   min_length=kw["min_length"], validate_inputs=validate)
    try:
        if kw["extra_eos"]:
            assert lib.set_extra_eos(h, kw["extra_eos"]) == 0, lib.error()
        _forced_give_up(monkeypatch)
        st, _out = lib.decode(h, case["xin"], case["K"], dtype=case["dtype"], from_logits=True, steps=kw["steps"])
        assert st == -2, (st, lib.error())  # DBS_ERROR_RUNTIME
        assert "gave up waiting for the row pass" in lib.error()
        monkeypatch.delenv("DBS_HIP_TEST_WAIT_GIVE_UP")
        st, out = lib.decode(h, case["xin"], case["K"], dtype=case["dtype"], from_logits=True, steps=kw["steps"])
        assert st == 0, lib.error()
    finally:
        lib.destroy(h)
    want = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    assert first_difference(out, want, ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents",
                                        "lengths", "scores", "raw_scores", "from_logprob", "row_lse")) is None


def test_more_caller_streams_than_overlap_sets(hip, oracle, overlap_on):
    """A decode on each of 70 caller streams (the library keeps 64 sets of
    an auxiliary stream and two events; the least recently used set of the
    device is rebound to a new caller), then again on the first ones: every
    decode bit-exact, no wait given up."""
    case = _big_case(7600)
    want = oracle.decode(case["xin"], dtype=case["dtype"], **case["kw"])
    streams = [torch.cuda.Stream() for _ in range(70)]
    for rep in range(2):
        for i, s in enumerate(streams if rep == 0 else streams[:8]):
            with torch.cuda.stream(s):
                got = hip.decode(case["xin"], case["dtype"], **case["kw"])
            assert first_difference(got, want) is None, (rep, i)
    torch.cuda.synchronize()
    assert _timeouts(overlap_on) == 0


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("overlap", [1, 0])
def test_read_back_after_a_decode(hip, oracle, monkeypatch, seed, overlap):
    """dbs_hip_decode_read_back after dbs_hip_decode_ex4: the flags and the
    fault word it copies equal a plain copy taken after the stream is
    synchronised, overlapped (the copy runs on the select pass's stream) or
    not (on the caller's stream), with and without a forced give-up; the
    trace matches the oracle."""
    lib = hip.lib
    prev = lib.dbs_hip_set_decode_overlap(overlap)
    try:
        case = _big_case(7700 + seed)
        give_up = overlap == 1 and seed % 2 == 1
        if give_up:
            _forced_give_up(monkeypatch)
        res = hip.decode(case["xin"], case["dtype"], read_back=True, **case["kw"])
    finally:
        lib.dbs_hip_set_decode_overlap(prev)
    assert np.array_equal(res["read_back_flags"], res["invalid"])
    assert res["read_back_fault"] == res["fault_word"]
    overlapped = res["fault_word"] is not None
    assert overlapped == (overlap == 1 and case["T"] > 1)
    if give_up and overlapped:
        assert res["fault_word"] != 0 and (res["invalid"] == 2).all()
    else:
        assert (res["invalid"] == 0).all() and not res["fault_word"]
        want = oracle.decode(case["xin"], dtype=case["dtype"], **case["kw"])
        assert first_difference(res, want) is None


def test_read_back_on_many_caller_streams(hip, oracle, overlap_on):
    """Decodes read back through the torch ops on 70 caller streams (more
    than the library's 64 overlap sets, so sets are rebound between a decode
    and the next): every result matches the oracle, no wait gives up."""
    import beamgrad_amd as bg

    case, x, opts = _torch_case(7720)
    kw = case["kw"]
    want = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    streams = [torch.cuda.Stream() for _ in range(70)]
    for i, s in enumerate(streams + streams[:6]):
        with torch.cuda.stream(s):
            out = bg.decode(x, opts(i % 2 == 0), kw["steps"], from_logits=True)
            s.synchronize()
        got = {k: getattr(out, k).cpu().numpy() for k in ("final_scores", "final_raw_scores", "scores",
                                                             "raw_scores")}
        for k in ("final_lengths", "tokens", "parents", "lengths"):
            got[k] = getattr(out, k).cpu().numpy().astype(np.int32)
        assert first_difference(got, want, tuple(got)) is None, i
    torch.cuda.synchronize()
    assert _timeouts(overlap_on) == 0
