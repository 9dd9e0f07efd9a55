# SPDX-License-Identifier: MIT
"""The result-object half of the libdbs host C ABI (include/dbs.h) of
libdbs_hip.so, computed on the GPU, against the reference's own CPU library
(oracle/_ref/libdbs_ref.so) called with identical arguments: decodes into
result handles (one example, typed, constrained, a batch, a batch with
per-example steps, beams, EOS tokens, minimum lengths and banned masks),
model-in-the-loop decodes whose callbacks record what they are shown, the
dense and sparse backward of a result (selected-weight and final-score
gradients), statistics, and the errors of calls that fail. Every array is
compared bit for bit, every status and message as text."""

import ctypes as C
import json
import os

import numpy as np
import pytest

from beamgrad_amd import _build
from tests.cases import log_softmax, make_case
from tests.host_abi import (STEP_EX_FN, STEP_FN, ConstraintsC, HostLib, StatsC, enable_results, read_backward,
                            read_result)

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libdbs_ref.so")
_f32p, _i32p, _u8p = C.POINTER(C.c_float), C.POINTER(C.c_int32), C.POINTER(C.c_uint8)


@pytest.fixture(scope="module")
def libs():
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref is not built")
    return enable_results(HostLib(_build.lib_path())), enable_results(HostLib(REF_LIB))


def _p(a, ct):
    return None if a is None else a.ctypes.data_as(C.POINTER(ct))


def same(a, b, what=""):
    """Two read-outs equal, floats compared as bit patterns."""
    if isinstance(a, dict):
        assert a.keys() == b.keys(), what
        for k in a:
            same(a[k], b[k], f"{what}.{k}")
    elif isinstance(a, (tuple, list)):
        assert isinstance(b, (tuple, list)) and len(a) == len(b), what
        for i, (u, v) in enumerate(zip(a, b)):
            same(u, v, f"{what}[{i}]")
    elif isinstance(a, np.ndarray) or isinstance(b, np.ndarray):
        assert (a is None) == (b is None), what
        if a is not None:
            assert a.shape == b.shape and a.dtype == b.dtype, what
            x, y = (a.view(np.uint32), b.view(np.uint32)) if a.dtype == np.float32 else (a, b)
            assert np.array_equal(x, y), f"{what}: first difference at {np.argwhere(x != y)[:1]}"
    else:
        assert a == b, f"{what}: {a!r} vs {b!r}"


def _options(K, eos=-1, alpha=0.0, min_length=0, validate=0, temperature=0.0, max_dense=0):
    return dict(beam_size=K, eos_token=eos, length_penalty_alpha=alpha, min_length=min_length,
                validate_inputs=validate, selected_temperature=temperature, max_dense_gradient_elements=max_dense)


def _each(libs, opts, fn, extra_eos=None):
    """fn(lib, handle) on both libraries, each with its own handle."""
    out = []
    for lib in libs:
        h = lib.create(**opts)
        try:
            if extra_eos:
                a = np.asarray(extra_eos, np.int32)
                assert lib.lib.dbs_set_extra_eos_tokens(h, _p(a, C.c_int32), len(a)) == 0, lib.error()
            out.append(fn(lib, h))
        finally:
            lib.destroy(h)
    return out


def _summary(L, r, eos):
    buf = C.create_string_buffer(1024)
    st = L.dbs_result_summary_json(r, eos, buf, 1024)
    return st, buf.value.decode(), L.dbs_result_eos_count(r, eos)


def _single(seed, dtype="f32"):
    case = make_case(seed, dtypes=[dtype], logits=False, allow_invalid=False)
    kw = case["kw"]
    x = case["xin"][0]  # [T, K, V]
    return case, kw, np.ascontiguousarray(x)


@pytest.mark.parametrize("seed", range(12))
def test_single_decodes_match_the_reference(libs, seed):
    case, kw, x = _single(5100 + seed)
    K, T, V = case["K"], case["T"], case["V"]
    opts = _options(K, kw["eos_token"], kw["alpha"], kw["min_length"], temperature=[0.0, 0.5, 2.0][seed % 3])
    extra = kw["extra_eos"]
    banned = kw["banned"]

    def run(lib, h):
        L = lib.lib
        res = {}
        r = C.c_void_p()
        st = L.dbs_decode(h, _p(x, C.c_float), T, V, C.byref(r))
        res["decode"] = (st, lib.error(), read_result(L, r) if st == 0 else None,
                         _summary(L, r, kw["eos_token"]) if st == 0 else None)
        L.dbs_free_result(r)
        forced = np.full(T, -1, np.int32)
        st = L.dbs_decode_constrained(h, _p(x, C.c_float), T, V, _p(banned, C.c_uint8), _p(forced, C.c_int32),
                                      kw["min_length"] + 1, C.byref(r))
        res["constrained"] = (st, lib.error(), read_result(L, r) if st == 0 else None)
        L.dbs_free_result(r)
        keep = {}
        c = HostLib.constraints(banned=banned, min_length=-1, repetition_penalty=kw["repetition_penalty"],
                                no_repeat_ngram_size=kw["no_repeat_ngram_size"], keep=keep)
        st = L.dbs_decode_constrained_ex(h, _p(x, C.c_float), T, V, C.byref(c), C.byref(r))
        res["constrained_ex"] = (st, lib.error(), read_result(L, r) if st == 0 else None)
        L.dbs_free_result(r)
        return res

    ours, theirs = _each(libs, opts, run, extra)
    same(ours, theirs, f"seed {seed}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("seed", range(4))
def test_typed_decodes_match_the_reference(libs, dtype, seed):
    case, kw, x = _single(5200 + seed, dtype)
    K, T, V = case["K"], case["T"], case["V"]
    opts = _options(K, kw["eos_token"], kw["alpha"], kw["min_length"])

    def run(lib, h):
        L = lib.lib
        r = C.c_void_p()
        st = L.dbs_decode_typed(h, x.ctypes.data_as(C.c_void_p), {"f16": 1, "bf16": 2}[dtype], T, V, C.byref(r))
        out = (st, lib.error(), read_result(L, r) if st == 0 else None)
        L.dbs_free_result(r)
        br = C.c_void_p()
        xb = np.ascontiguousarray(case["xin"])
        st = L.dbs_decode_batch_typed(h, xb.ctypes.data_as(C.c_void_p), {"f16": 1, "bf16": 2}[dtype], case["B"], T,
                                      V, 1, C.byref(br))
        batch = [read_result(L, L.dbs_batch_result_at(br, b)) for b in range(L.dbs_batch_result_size(br))]
        L.dbs_free_batch_result(br)
        return out, st, lib.error(), batch

    ours, theirs = _each(libs, opts, run, kw["extra_eos"])
    same(ours[0], theirs[0], "typed")
    assert ours[1:3] == theirs[1:3]
    assert len(ours[3]) == len(theirs[3]) == case["B"]
    for b, (a, c) in enumerate(zip(ours[3], theirs[3])):
        same(a, c, f"example {b}")


@pytest.mark.parametrize("seed", range(6))
def test_batch_decodes_match_the_reference(libs, seed):
    case = make_case(5300 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    kw = case["kw"]
    B, T, K, V = case["B"], case["T"], case["K"], case["V"]
    x = np.ascontiguousarray(case["xin"])
    opts = _options(K, kw["eos_token"], kw["alpha"], kw["min_length"])

    def run(lib, h):
        L = lib.lib
        br = C.c_void_p()
        st = L.dbs_decode_batch(h, _p(x, C.c_float), B, T, V, 1, C.byref(br))
        out = [read_result(L, L.dbs_batch_result_at(br, b)) for b in range(L.dbs_batch_result_size(br))]
        assert L.dbs_batch_result_at(br, B) is None and L.dbs_batch_result_at(br, -1) is None
        L.dbs_free_batch_result(br)
        return st, lib.error(), out

    ours, theirs = _each(libs, opts, run, kw["extra_eos"])
    assert ours[:2] == theirs[:2]
    for b, (a, c) in enumerate(zip(ours[2], theirs[2])):
        same(a, c, f"example {b}")


@pytest.mark.parametrize("seed", range(10))
def test_variable_batch_matches_the_reference(libs, seed):
    """Per-example steps, beam sizes, EOS tokens, minimum lengths and banned
    masks (reference dbs_decode_batch_variable: each example decoded alone
    with its own options on the first beams of each step's rows)."""
    rng = np.random.default_rng(5400 + seed)
    B, T, Kmax, V = int(rng.integers(1, 6)), int(rng.integers(1, 8)), int(rng.choice([2, 4, 8, 16])), \
        int(rng.choice([7, 50, 300, 1001]))
    x = log_softmax(rng.normal(0, 2.0, (B, T, Kmax, V)).astype(np.float32))
    if rng.random() < 0.5:
        pool = rng.choice(x.reshape(-1), 6)
        m = rng.random(x.shape) < 0.05
        x[m] = rng.choice(pool, int(m.sum()))
    x = np.ascontiguousarray(x)
    steps = rng.integers(1, T + 1, B).astype(np.int32)
    beams = rng.integers(1, Kmax + 1, B).astype(np.int32)
    eos = rng.integers(-1, V, B).astype(np.int32)
    mins = rng.integers(-1, 4, B).astype(np.int32)
    banned = (rng.random((B, V)) < 0.1).astype(np.uint8)
    forced = np.full((B, T), -1, np.int32)
    use = [rng.random() < 0.7 for _ in range(5)]
    args = [a if u else None for a, u in zip((steps, beams, eos, mins, banned), use)]
    opts = _options(int(rng.integers(1, Kmax + 1)), int(rng.integers(-1, V)), float(rng.choice([0.0, 0.6])))

    def run(lib, h):
        L = lib.lib
        br = C.c_void_p()
        st = L.dbs_decode_batch_variable(h, _p(x, C.c_float), B, T, Kmax, V, _p(args[0], C.c_int32),
                                         _p(args[1], C.c_int32), _p(args[2], C.c_int32), _p(args[3], C.c_int32),
                                         _p(args[4], C.c_uint8), _p(forced, C.c_int32), 1, C.byref(br))
        out = [read_result(L, L.dbs_batch_result_at(br, b)) for b in range(L.dbs_batch_result_size(br))]
        L.dbs_free_batch_result(br)
        return st, lib.error(), out

    ours, theirs = _each(libs, opts, run)
    assert ours[:2] == theirs[:2], (ours[:2], theirs[:2])
    for b, (a, c) in enumerate(zip(ours[2], theirs[2])):
        same(a, c, f"example {b}")


@pytest.mark.parametrize("seed", range(10))
def test_backward_handles_match_the_reference(libs, seed):
    """dbs_backward_dense / _sparse / _default / dbs_backward of a decoded
    result: the gradient w.r.t. the log-probabilities and the initial scores
    from selected-weight and final-score gradients (each alone, both,
    neither)."""
    case, kw, x = _single(5500 + seed)
    K, T, V = case["K"], case["T"], case["V"]
    rng = np.random.default_rng(seed)
    gw = rng.normal(0, 1, T * K).astype(np.float32)
    gf = rng.normal(0, 1, K).astype(np.float32)
    which = [(gw, gf), (None, gf), (gw, None), (None, None)][seed % 4]
    opts = _options(K, kw["eos_token"], kw["alpha"], kw["min_length"], temperature=[0.0, 0.7][seed % 2])

    def run(lib, h):
        L = lib.lib
        r = C.c_void_p()
        assert L.dbs_decode(h, _p(x, C.c_float), T, V, C.byref(r)) == 0, lib.error()
        out = {}
        for name in ("dbs_backward_dense", "dbs_backward_sparse", "dbs_backward_default", "dbs_backward"):
            b = C.c_void_p()
            st = getattr(L, name)(h, r, _p(which[0], C.c_float), None, _p(which[1], C.c_float), C.byref(b))
            out[name] = (st, lib.error(), read_backward(L, b, T * K * V, K) if st == 0 else None)
            L.dbs_free_backward(b)
        L.dbs_free_result(r)
        return out

    ours, theirs = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed}")


def _recorder(x, log):
    """Model-step callbacks that fill each step's rows from x [T, K, V]
    (every beam's row shifted by a function of the token it emitted last, so
    the rows depend on the beams) and record what each call is shown."""
    T, K, V = x.shape

    def rows_for(step, tokens, out):
        rows = np.ctypeslib.as_array(out, shape=(K * V,))
        tok = np.ctypeslib.as_array(tokens, shape=(K,)).copy()
        r = x[step].copy()
        r += (0.01 * (tok[:, None] % 7)).astype(np.float32)
        rows[:] = r.reshape(-1)

    def simple(user, batch_index, step, tokens, scores, beam, vocab, out):
        log.append(("simple", batch_index, step, beam, vocab, np.ctypeslib.as_array(tokens, shape=(K,)).copy(),
                    np.ctypeslib.as_array(scores, shape=(K,)).copy().view(np.uint32)))
        rows_for(step, tokens, out)
        return 0

    def ex(user, info_p, out):
        info = info_p.contents
        t = info.step
        prefixes = np.ctypeslib.as_array(info.prefixes, shape=(K * t,)).copy() if t > 0 else np.zeros(0, np.int32)
        log.append(("ex", info.batch_index, t, info.beam_size, info.vocab_size,
                    np.ctypeslib.as_array(info.parents, shape=(K,)).copy(),
                    np.ctypeslib.as_array(info.tokens, shape=(K,)).copy(),
                    np.ctypeslib.as_array(info.lengths, shape=(K,)).copy(),
                    np.ctypeslib.as_array(info.scores, shape=(K,)).copy().view(np.uint32),
                    np.ctypeslib.as_array(info.raw_scores, shape=(K,)).copy().view(np.uint32),
                    np.ctypeslib.as_array(info.finished, shape=(K,)).copy(), prefixes))
        rows_for(t, info.tokens, out)
        return 0

    return STEP_FN(simple), STEP_EX_FN(ex)


def _logs_equal(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert len(x) == len(y)
        for u, v in zip(x, y):
            if isinstance(u, np.ndarray):
                assert np.array_equal(u, v)
            else:
                assert u == v


@pytest.mark.parametrize("seed", range(8))
def test_model_step_decodes_match_the_reference(libs, seed):
    case, kw, x = _single(5600 + seed)
    K, T, V = case["K"], case["T"], case["V"]
    opts = _options(K, kw["eos_token"], kw["alpha"], kw["min_length"])
    banned = kw["banned"]

    def run(lib, h):
        L = lib.lib
        out, logs = {}, {}
        for mode in ("simple", "workspace", "ex", "ex_constrained"):
            log = []
            simple, ex = _recorder(x, log)
            r = C.c_void_p()
            if mode == "simple":
                st = L.dbs_decode_model_steps(h, simple, None, 3, T, V, C.byref(r))
            elif mode == "workspace":
                ws = C.c_void_p()
                assert L.dbs_workspace_create(C.byref(ws)) == 0
                assert L.dbs_workspace_reserve(ws, 100, 10) == 0
                assert L.dbs_workspace_allocated_bytes(ws) >= 440
                st = L.dbs_decode_model_steps_with_workspace(h, ws, simple, None, 1, T, V, C.byref(r))
                L.dbs_workspace_destroy(ws)
            else:
                keep = {}
                c = HostLib.constraints(banned=banned if mode == "ex_constrained" else None,
                                        min_length=kw["min_length"] + 1 if mode == "ex_constrained" else -1,
                                        repetition_penalty=1.3 if mode == "ex_constrained" else 1.0,
                                        no_repeat_ngram_size=2 if mode == "ex_constrained" else 0, keep=keep)
                st = L.dbs_decode_model_steps_ex(h, ex, None, 2, T, V, C.byref(c), C.byref(r))
            out[mode] = (st, lib.error(), read_result(L, r) if st == 0 else None)
            logs[mode] = log
            L.dbs_free_result(r)
        return out, logs

    (ours, our_logs), (theirs, their_logs) = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed}")
    for mode in our_logs:
        _logs_equal(our_logs[mode], their_logs[mode])


def test_model_step_callback_failure(libs):
    def fail(*_a):
        return 1

    K, T, V = 2, 3, 5

    def run(lib, h):
        r = C.c_void_p()
        st = lib.lib.dbs_decode_model_steps(h, STEP_FN(fail), None, 0, T, V, C.byref(r))
        return st, lib.error(), r.value

    ours, theirs = _each(libs, _options(K), run)
    assert ours == theirs and ours[0] == -2 and ours[2] is None


@pytest.mark.parametrize("validate", [0, 1])
def test_invalid_rows_match_the_reference(libs, validate):
    """NaN/+inf in a row the search reads: the error text names the step and
    beam (no example prefix for one example, "example b: " for a batch)."""
    rng = np.random.default_rng(3)
    B, T, K, V = 3, 4, 3, 20
    x = log_softmax(rng.normal(0, 1, (B, T, K, V)).astype(np.float32))
    x[1, 2, 0, 5] = np.nan
    x[2, 1, 0, 7] = np.inf
    x = np.ascontiguousarray(x)

    def run(lib, h):
        L = lib.lib
        r, br = C.c_void_p(), C.c_void_p()
        one = np.ascontiguousarray(x[1])
        st1 = L.dbs_decode(h, _p(one, C.c_float), T, V, C.byref(r))
        e1 = lib.error()
        L.dbs_free_result(r)
        st2 = L.dbs_decode_batch(h, _p(x, C.c_float), B, T, V, 1, C.byref(br))
        e2 = lib.error()
        L.dbs_free_batch_result(br)

        def fill(user, batch_index, step, tokens, scores, beam, vocab, out):
            np.ctypeslib.as_array(out, shape=(K * V,))[:] = x[1, step].reshape(-1)
            return 0
        st3 = L.dbs_decode_model_steps(h, STEP_FN(fill), None, 0, T, V, C.byref(r))
        e3 = lib.error()
        L.dbs_free_result(r)
        return st1, e1, st2, e2, st3, e3

    ours, theirs = _each(libs, _options(K, validate=validate), run)
    assert ours == theirs


def test_result_errors_match_the_reference(libs):
    rng = np.random.default_rng(8)
    T, K, V = 3, 2, 10
    x = np.ascontiguousarray(log_softmax(rng.normal(0, 1, (2, T, K, V)).astype(np.float32)))
    g = np.ones(T * K, np.float32)

    def run(lib, h):
        L = lib.lib
        out = []
        r, br, b = C.c_void_p(), C.c_void_p(), C.c_void_p()
        out.append((L.dbs_decode(h, _p(x, C.c_float), T, V, None), lib.error()))
        out.append((L.dbs_decode(h, None, T, V, C.byref(r)), lib.error()))
        out.append((L.dbs_decode(h, _p(x, C.c_float), 0, V, C.byref(r)), lib.error()))
        out.append((L.dbs_decode(h, _p(x, C.c_float), T, 0, C.byref(r)), lib.error()))
        out.append((L.dbs_decode(None, _p(x, C.c_float), T, V, C.byref(r)), lib.error()))
        out.append((L.dbs_decode_typed(h, x.ctypes.data_as(C.c_void_p), 7, T, V, C.byref(r)), lib.error()))
        out.append((L.dbs_decode_batch(h, _p(x, C.c_float), 0, T, V, 1, C.byref(br)), lib.error()))
        forced = np.array([1, 20, -1], np.int32)
        out.append((L.dbs_decode_constrained(h, _p(x, C.c_float), T, V, None, _p(forced, C.c_int32), 0,
                                             C.byref(r)), lib.error()))
        keep = {}
        c = HostLib.constraints(repetition_penalty=float("inf"), keep=keep)
        out.append((L.dbs_decode_constrained_ex(h, _p(x, C.c_float), T, V, C.byref(c), C.byref(r)), lib.error()))
        for steps, beams, eos in (([1, 4], None, None), ([1, 2], [0, 1], None), (None, [1, 3], None),
                                  (None, None, [-2, 1]), (None, None, [1, 10])):
            s = None if steps is None else np.asarray(steps, np.int32)
            bm = None if beams is None else np.asarray(beams, np.int32)
            e = None if eos is None else np.asarray(eos, np.int32)
            out.append((L.dbs_decode_batch_variable(h, _p(x, C.c_float), 2, T, K, V, _p(s, C.c_int32),
                                                    _p(bm, C.c_int32), _p(e, C.c_int32), None, None, None, 1,
                                                    C.byref(br)), lib.error()))
        # backward: a NULL result, relaxed-pool gradients without a pool, a
        # dense gradient above max_dense_gradient_elements
        out.append((L.dbs_backward_dense(h, None, None, None, None, C.byref(b)), lib.error()))
        assert L.dbs_decode(h, _p(x, C.c_float), T, V, C.byref(r)) == 0, lib.error()
        out.append((L.dbs_backward_sparse(h, r, None, _p(g, C.c_float), None, C.byref(b)), lib.error()))
        out.append((L.dbs_backward(h, r, None, None, None, None), lib.error()))
        out.append((L.dbs_backward_dense(h, r, None, None, None, C.byref(b)), lib.error()))
        L.dbs_free_result(r)
        return out

    ours, theirs = _each(libs, _options(K, eos=1, max_dense=40), run)
    assert ours == theirs


def test_refusals_name_what_is_not_served(libs):
    """What the HIP engine does not serve is refused with a message naming
    it (the reference computes these): a relaxed pool of more than 1024
    candidates."""
    ours = libs[0]
    L = ours.lib
    T, K, V = 2, 300, 10
    x = np.ascontiguousarray(log_softmax(np.zeros((T, K, V), np.float32)))
    r = C.c_void_p()
    h = ours.create(beam_size=K, relaxed_pool_multiplier=4)
    assert L.dbs_decode(h, _p(x, C.c_float), T, V, C.byref(r)) == -1
    assert "relaxed pool of 1200 candidates" in ours.error()
    ours.destroy(h)


def test_statistics_match_the_reference(libs):
    rng = np.random.default_rng(9)
    T, K, V = 4, 3, 30
    x = np.ascontiguousarray(log_softmax(rng.normal(0, 1, (T, K, V)).astype(np.float32)))

    def run(lib, h):
        L = lib.lib
        r, b = C.c_void_p(), C.c_void_p()
        assert L.dbs_decode(h, _p(x, C.c_float), T, V, C.byref(r)) == 0
        s = StatsC()
        assert L.dbs_get_stats(h, C.byref(s)) == 0
        after_decode = (s.abi_version, s.last_selected_count, s.last_pool_count, s.last_logprob_count,
                        s.used_model_step_callback, s.last_error_category)
        gf = np.ones(K, np.float32)
        assert L.dbs_backward_sparse(h, r, None, None, _p(gf, C.c_float), C.byref(b)) == 0
        assert L.dbs_get_stats(h, C.byref(s)) == 0
        after_backward = (s.used_sparse_backward, s.used_dense_backward, s.last_sparse_grad_count)
        L.dbs_free_backward(b)
        st_bad = L.dbs_decode(h, None, T, V, C.byref(r))
        assert L.dbs_get_stats(h, C.byref(s)) == 0
        after_error = (st_bad, s.last_error_category)
        buf = C.create_string_buffer(2048)
        assert L.dbs_get_stats_json(h, buf, 2048) == 0
        keys = sorted(json.loads(buf.value.decode()))
        L.dbs_reset_stats(h)
        assert L.dbs_get_stats(h, C.byref(s)) == 0
        reset = (s.abi_version, s.last_selected_count, s.last_error_category)
        assert L.dbs_set_deterministic_seed(h, 12345) == 0
        seed = (L.dbs_get_deterministic_seed(h), L.dbs_is_deterministic())
        small = C.create_string_buffer(8)
        short = L.dbs_get_stats_json(h, small, 8)
        L.dbs_free_result(r)
        return after_decode, after_backward, after_error, keys, reset, seed, short

    ours, theirs = _each(libs, _options(K), run)
    assert ours == theirs
