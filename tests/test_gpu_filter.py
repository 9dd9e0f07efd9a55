# SPDX-License-Identifier: MIT
"""Token filters (DBSAdvancedConstraintsC.token_filter) in libdbs_hip.so
against the reference's own CPU library (oracle/_ref/libdbs_ref.so), both
called with identical arguments and the same recording filter.

The reference calls the filter for each read beam in order and each token
in order that passes the forced, banned, minimum-length and n-gram checks,
with the beam's prefix, before the value check (reference
src/decoder.cpp:259-282); a refused token is not a candidate. The HIP
library decodes such a decode step by step on the device step API and asks
the filter on the host in that order. Compared: every output bit for bit,
statuses and messages as text, and the filter's calls (batch index, step,
parent beam, prefix, token) of each example in order. Cases: batch decodes
into caller arrays (f32/f16/bf16, logits with row_lse, EOS and extra EOS,
min_length, banned tokens, n-gram blocking, repetition penalty, forced
tokens, per-example steps, a relaxed pool), validate_inputs errors,
dbs_decode_constrained_ex and model-step decodes."""

import ctypes as C
import os

import numpy as np
import pytest

from beamgrad_amd import _build
from tests.cases import first_difference, log_softmax, make_case, to_bits
from tests.host_abi import HostLib, enable_results, read_result

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libdbs_ref.so")
OUT_KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
            "raw_scores", "from_logprob", "row_lse")
POOL_KEYS = ("pool_parents", "pool_tokens", "pool_lengths", "pool_scores", "pool_raw_scores", "pool_from_logprob")
FILTER_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int32), C.c_int, C.c_int)


@pytest.fixture(scope="module")
def libs():
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref is not built")
    return enable_results(HostLib(_build.lib_path())), enable_results(HostLib(REF_LIB))


def _recording_filter(log, salt):
    """A filter refusing about a third of the tokens, by a hash of the call,
    that records every call."""
    def fn(user, batch_index, step, parent, prefix, prefix_len, token):
        pre = tuple(prefix[i] for i in range(prefix_len)) if prefix_len > 0 else ()
        log.append((batch_index, step, parent, pre, token))
        h = (token * 2654435761 + step * 97 + parent * 31 + sum(pre) * 7 + salt) & 0xFFFFFFFF
        return 0 if h % 3 == 0 else 1

    return FILTER_FN(fn)


def _by_example(log):
    out = {}
    for call in log:
        out.setdefault(call[0], []).append(call)
    return out


def _each(libs, opts, fn, extra_eos=None):
    out = []
    for lib in libs:
        h = lib.create(**opts)
        try:
            if extra_eos:
                assert lib.set_extra_eos(h, extra_eos) == 0, lib.error()
            out.append(fn(lib, h))
        finally:
            lib.destroy(h)
    return out


def _filtered_batch(libs, case, *, forced=None, validate=0, pool_m=0, salt=0):
    kw = case["kw"]
    K = case["K"]
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], validate_inputs=validate, relaxed_pool_multiplier=pool_m)

    def fn(lib, h):
        log = []
        filt = _recording_filter(log, salt)
        keep = {}
        cons = HostLib.constraints(banned=kw.get("banned"), repetition_penalty=float(kw.get("repetition_penalty", 1.0)),
                                   no_repeat_ngram_size=int(kw.get("no_repeat_ngram_size") or 0), forced=forced,
                                   keep=keep)
        cons.token_filter = C.cast(filt, C.c_void_p)
        st, out = lib.decode(h, case["xin"], K, dtype=case["dtype"], from_logits=kw["from_logits"], steps=kw["steps"],
                             constraints=cons, pool=K * pool_m)
        return st, out, lib.error(), _by_example(log)

    return _each(libs, opts, fn, kw.get("extra_eos"))


def _check(libs, case, **more):
    (s0, o0, e0, l0), (s1, o1, e1, l1) = _filtered_batch(libs, case, **more)
    tag = f"seed {case['seed']} {case['dtype']} B{case['B']} T{case['T']} K{case['K']} V{case['V']}"
    assert (s0, e0) == (s1, e1), tag
    assert l0 == l1, f"{tag}: the filter's calls differ"
    if s0 == 0:
        keys = OUT_KEYS + (POOL_KEYS if more.get("pool_m") else ())
        diff = first_difference(o0, o1, keys)
        assert diff is None, f"{tag}: {diff}"
    return s0, l0


@pytest.mark.parametrize("seed", range(24))
def test_filtered_batch_decodes(libs, seed):
    case = make_case(51000 + seed, vocabs=[3, 7, 40, 257], allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    rng = np.random.default_rng(seed)
    T, V = case["T"], case["V"]
    forced = np.where(rng.random(T) < 0.25, rng.integers(0, V, T), -1).astype(np.int32) if seed % 3 == 0 else None
    st, log = _check(libs, case, forced=forced, pool_m=[0, 0, 2][seed % 3], salt=seed)
    assert st == 0
    assert sum(len(v) for v in log.values()) > 0


@pytest.mark.parametrize("seed", range(6))
def test_filtered_long_constrained(libs, seed):
    """Longer decodes over small vocabularies with n-gram blocking and a
    repetition penalty: the prefixes handed to the filter grow, blocked
    tokens are not offered."""
    rng = np.random.default_rng(52000 + seed)
    B, T, K, V = 2, int(rng.integers(8, 16)), int(rng.choice([2, 3, 4])), int(rng.choice([5, 9, 20]))
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    from_logits = seed % 2 == 1
    if not from_logits:
        x = log_softmax(x)
    dtype = ["f32", "bf16", "f16"][seed % 3]
    kw = dict(from_logits=from_logits, eos_token=int(rng.integers(0, V)) if seed % 2 else -1, extra_eos=[],
              min_length=int(rng.integers(0, 4)), alpha=0.6, no_repeat_ngram_size=int(rng.choice([1, 2, 3])),
              repetition_penalty=float(rng.choice([1.0, 1.5])), steps=[T, max(1, T - 3)], banned=None)
    case = dict(seed=52000 + seed, B=B, T=T, K=K, V=V, dtype=dtype, x=x, xin=to_bits(x, dtype), kw=kw)
    _check(libs, case, salt=seed)


@pytest.mark.parametrize("from_logits", [False, True])
def test_filtered_validate_inputs(libs, from_logits):
    """A NaN in a read row with validate_inputs: the same error, after the
    same filter calls (from logits before the row's calls, from log-probs
    after them)."""
    rng = np.random.default_rng(3)
    B, T, K, V = 2, 4, 3, 30
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    if not from_logits:
        x = log_softmax(x)
    x[1, 2, :, 7] = np.nan
    kw = dict(from_logits=from_logits, eos_token=-1, extra_eos=[], min_length=0, alpha=0.0, steps=None, banned=None,
              no_repeat_ngram_size=0, repetition_penalty=1.0)
    case = dict(seed=3, B=B, T=T, K=K, V=V, dtype="f32", x=x, xin=x, kw=kw)
    st, _ = _check(libs, case, validate=1)
    assert st == -1


@pytest.mark.parametrize("seed", range(8))
def test_filtered_result_and_model_step_decodes(libs, seed):
    """dbs_decode_constrained_ex and dbs_decode_model_steps_ex with a
    filter: the results and the filter's calls (with the call's batch index)."""
    from tests.test_gpu_host_results import _logs_equal, _recorder, same

    case = make_case(53000 + seed, dtypes=["f32"], logits=False, vocabs=[7, 40, 257], allow_invalid=False)
    kw = case["kw"]
    K, T, V = case["K"], case["T"], case["V"]
    x = np.ascontiguousarray(case["xin"][0])
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], relaxed_pool_multiplier=seed % 2)

    def run(lib, h):
        L = lib.lib
        out, logs = {}, {}
        for mode in ("constrained_ex", "model_steps"):
            flog, slog = [], []
            filt = _recording_filter(flog, seed)
            keep = {}
            c = HostLib.constraints(banned=kw["banned"], repetition_penalty=1.3 if seed % 2 else 1.0,
                                    no_repeat_ngram_size=2 if seed % 3 == 0 else 0, keep=keep)
            c.token_filter = C.cast(filt, C.c_void_p)
            c.batch_index = 5
            r = C.c_void_p()
            if mode == "constrained_ex":
                st = L.dbs_decode_constrained_ex(h, x.ctypes.data_as(C.POINTER(C.c_float)), T, V, C.byref(c),
                                                 C.byref(r))
            else:
                _, ex = _recorder(x, slog)
                st = L.dbs_decode_model_steps_ex(h, ex, None, 2, T, V, C.byref(c), C.byref(r))
            out[mode] = (st, lib.error(), read_result(L, r) if st == 0 else None)
            logs[mode] = (flog, slog)
            L.dbs_free_result(r)
        return out, logs

    (ours, our_logs), (theirs, their_logs) = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed}")
    for mode in our_logs:
        assert our_logs[mode][0] == their_logs[mode][0], f"{mode}: the filter's calls differ"
        _logs_equal(our_logs[mode][1], their_logs[mode][1])
    assert our_logs["constrained_ex"][0] and our_logs["constrained_ex"][0][0][0] == 5
    assert our_logs["model_steps"][0] and our_logs["model_steps"][0][0][0] == 2
