# SPDX-License-Identifier: MIT
"""The relaxed pool (relaxed_pool_multiplier m >= 1) in libdbs_hip.so,
computed on the GPU, against the reference's own CPU library
(oracle/_ref/libdbs_ref.so) called with identical arguments.

With a pool each step keeps the best m * K candidates of an example, the
selection first (reference src/decoder.cpp:40, 294-350). The batch decodes
into caller arrays write them to the pool outputs of DBSDecodeOutputsExC
([B, T, m * K]; dead entries past the candidates and past an example's
steps); asking for no pool output decodes without one. Cases: random decodes
(f32/f16/bf16, logits, EOS and extra EOS, min_length, banned tokens, n-gram
blocking, repetition penalty, per-example steps, forced tokens), pools wider
than a row's shortlist (every row rescanned), wide beams, the overlapped
decode. Result handles keep each example's pool and its soft top-k
inclusion weights (one example, batches, variable batches with per-example
beams, model-step decodes; several temperatures, tolerances and iteration
caps). The pool's gradients: relaxed-weight gradients of the result-handle
backward (dense and sparse, with the initial scores'), pool score and
raw-score gradients of the batch backward (log-probs and logits), and the
pool trace's errors. Outputs are compared bit for bit, statuses and
messages as text."""

import os

import numpy as np
import pytest

from beamgrad_amd import _build
from tests.cases import first_difference, log_softmax, make_case, to_bits
from tests.host_abi import HostLib, enable_results

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libdbs_ref.so")
OUT_KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
            "raw_scores", "from_logprob", "row_lse")
POOL_KEYS = ("pool_parents", "pool_tokens", "pool_lengths", "pool_scores", "pool_raw_scores", "pool_from_logprob")


@pytest.fixture(scope="module")
def libs():
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref is not built")
    return enable_results(HostLib(_build.lib_path())), enable_results(HostLib(REF_LIB))


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


def _pool_decode(libs, case, m, *, forced=None, pool=True):
    kw = case["kw"]
    K = case["K"]
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], relaxed_pool_multiplier=m)
    constrained = forced is not None or kw.get("banned") is not None or kw.get("no_repeat_ngram_size") or \
        kw.get("repetition_penalty", 1.0) > 1.0

    def fn(lib, h):
        keep = {}
        cons = None
        if constrained:
            cons = HostLib.constraints(banned=kw.get("banned"), repetition_penalty=float(kw.get("repetition_penalty", 1.0)),
                                       no_repeat_ngram_size=int(kw.get("no_repeat_ngram_size") or 0), forced=forced,
                                       keep=keep)
        st, out = lib.decode(h, case["xin"], K, dtype=case["dtype"], from_logits=kw["from_logits"], steps=kw["steps"],
                             constraints=cons, pool=K * m if pool else 0)
        return st, out, lib.error()

    return _each(libs, opts, fn, kw.get("extra_eos"))


def _check(libs, case, m, **more):
    (s0, o0, e0), (s1, o1, e1) = _pool_decode(libs, case, m, **more)
    tag = f"seed {case['seed']} {case['dtype']} B{case['B']} T{case['T']} K{case['K']} V{case['V']} m{m}"
    assert (s0, e0) == (s1, e1), tag
    assert s0 == 0, (tag, e0)
    keys = OUT_KEYS + (POOL_KEYS if more.get("pool", True) else ())
    diff = first_difference(o0, o1, keys)
    assert diff is None, f"{tag}: {diff}"
    return o0


@pytest.mark.parametrize("seed", range(40))
def test_pool_batch_decodes_match_the_reference(libs, seed):
    case = make_case(41000 + seed, allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    m = [1, 2, 3, 4, 8][seed % 5]
    if case["K"] * m > 1024:
        m = 1
    _check(libs, case, m)


@pytest.mark.parametrize("seed", range(10))
def test_pool_with_forced_tokens(libs, seed):
    case = make_case(42000 + seed, allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    rng = np.random.default_rng(seed)
    T, V = case["T"], case["V"]
    forced = np.where(rng.random(T) < 0.5, rng.integers(0, V, T), -1).astype(np.int32)
    _check(libs, case, 2, forced=forced)


@pytest.mark.parametrize("overlap", [1, 0])
@pytest.mark.parametrize("shape", [(4, 1000, 4), (16, 4104, 2), (8, 32000, 3), (20, 3000, 2), (64, 2048, 16),
                                   (5, 257, 13)])
def test_pool_wide_and_long_rows(libs, shape, overlap):
    """Pools from 8 to 1024 candidates: within a row's shortlist, and wider
    (every row read in full), with the select pass beside the row pass and
    after it."""
    K, V, m = shape
    rng = np.random.default_rng(K * 7 + m)
    B, T = 3, 6
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    if m % 2:
        x = log_softmax(x)
    dtype = "bf16" if K >= 16 else "f32"
    kw = dict(from_logits=m % 2 == 0, eos_token=int(rng.integers(0, V)), extra_eos=[], min_length=1, alpha=0.6,
              no_repeat_ngram_size=0, repetition_penalty=1.0, steps=[6, 3, 5], banned=None, banned_per_example=None)
    case = dict(seed=K, B=B, T=T, K=K, V=V, dtype=dtype, x=x, xin=to_bits(x, dtype), kw=kw)
    ours = libs[0].lib
    prev = ours.dbs_hip_set_decode_overlap(overlap)
    try:
        _check(libs, case, m)
    finally:
        ours.dbs_hip_set_decode_overlap(prev)


def test_pool_multiplier_without_pool_outputs(libs):
    """A multiplier with no pool output asked for: the plain decode."""
    case = make_case(43000, allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    _check(libs, case, 3, pool=False)



# ---------------------------------------------------------------------------
# Result handles: the pool of every step and its soft top-k inclusion weights
# ---------------------------------------------------------------------------

def _soft(seed):
    """Soft top-k options: temperature, tolerance and iteration cap."""
    return [dict(), dict(soft_topk_temperature=1.0), dict(soft_topk_temperature=0.05, soft_topk_tolerance=1e-2),
            dict(soft_topk_max_iters=5)][seed % 4]


@pytest.mark.parametrize("seed", range(12))
def test_pool_result_decodes(libs, seed):
    """dbs_decode, dbs_decode_constrained_ex (with forced tokens, n-gram
    blocking, a repetition penalty) and dbs_decode_batch with a pool: the
    pool arrays, relaxed weights, counts and statistics."""
    import ctypes as C

    from tests.host_abi import StatsC, read_result

    case = make_case(44000 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    kw = case["kw"]
    B, K, T, V = case["B"], case["K"], case["T"], case["V"]
    m = [1, 2, 3, 4][seed % 4]
    x1 = np.ascontiguousarray(case["xin"][0])
    xb = np.ascontiguousarray(case["xin"])
    rng = np.random.default_rng(seed)
    forced = np.where(rng.random(T) < 0.3, rng.integers(0, V, T), -1).astype(np.int32)
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], relaxed_pool_multiplier=m, selected_temperature=0.5, **_soft(seed))

    def run(lib, h):
        L = lib.lib
        f32p = C.POINTER(C.c_float)
        res = {}
        r, br = C.c_void_p(), C.c_void_p()
        st = L.dbs_decode(h, x1.ctypes.data_as(f32p), T, V, C.byref(r))
        s = StatsC()
        assert L.dbs_get_stats(h, C.byref(s)) == 0
        res["decode"] = (st, lib.error(), read_result(L, r) if st == 0 else None, s.last_pool_count)
        L.dbs_free_result(r)
        keep = {}
        c = HostLib.constraints(banned=kw["banned"], repetition_penalty=1.3, no_repeat_ngram_size=2, forced=forced,
                                keep=keep)
        st = L.dbs_decode_constrained_ex(h, x1.ctypes.data_as(f32p), T, V, C.byref(c), C.byref(r))
        res["constrained_ex"] = (st, lib.error(), read_result(L, r) if st == 0 else None)
        L.dbs_free_result(r)
        st = L.dbs_decode_batch(h, xb.ctypes.data_as(f32p), B, T, V, 1, C.byref(br))
        res["batch"] = (st, lib.error(),
                        [read_result(L, L.dbs_batch_result_at(br, b)) for b in range(L.dbs_batch_result_size(br))])
        L.dbs_free_batch_result(br)
        return res

    from tests.test_gpu_host_results import same

    ours, theirs = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed} m {m}")
    assert ours["decode"][0] == 0 and ours["decode"][2]["pool_size"] == K * m


@pytest.mark.parametrize("seed", range(6))
def test_pool_variable_batches(libs, seed):
    """dbs_decode_batch_variable with a pool: each example's pool is
    beams_b * m candidates."""
    import ctypes as C

    from tests.host_abi import read_result
    from tests.test_gpu_host_results import same

    rng = np.random.default_rng(45000 + seed)
    B, T, Kmax, V = int(rng.integers(1, 5)), int(rng.integers(1, 7)), int(rng.choice([2, 4, 8])), \
        int(rng.choice([7, 50, 300]))
    x = np.ascontiguousarray(log_softmax(rng.normal(0, 2.0, (B, T, Kmax, V)).astype(np.float32)))
    steps = rng.integers(1, T + 1, B).astype(np.int32)
    beams = rng.integers(1, Kmax + 1, B).astype(np.int32)
    eos = rng.integers(-1, V, B).astype(np.int32)
    opts = dict(beam_size=Kmax, eos_token=int(rng.integers(-1, V)), length_penalty_alpha=0.6,
                relaxed_pool_multiplier=int(rng.integers(1, 4)), **_soft(seed))

    def run(lib, h):
        L = lib.lib
        br = C.c_void_p()
        i32 = C.POINTER(C.c_int32)
        st = L.dbs_decode_batch_variable(h, x.ctypes.data_as(C.POINTER(C.c_float)), B, T, Kmax, V,
                                         steps.ctypes.data_as(i32), beams.ctypes.data_as(i32),
                                         eos.ctypes.data_as(i32), None, None, None, 1, C.byref(br))
        out = [read_result(L, L.dbs_batch_result_at(br, b)) for b in range(L.dbs_batch_result_size(br))]
        L.dbs_free_batch_result(br)
        return st, lib.error(), out

    ours, theirs = _each(libs, opts, run)
    assert ours[:2] == theirs[:2] and ours[0] == 0, (ours[:2], theirs[:2])
    for b, (a, c) in enumerate(zip(ours[2], theirs[2])):
        same(a, c, f"example {b}")


@pytest.mark.parametrize("seed", range(6))
def test_pool_model_step_decodes(libs, seed):
    """Model-step decodes keep a pool each step (the device step API)."""
    import ctypes as C

    from tests.host_abi import read_result
    from tests.test_gpu_host_results import _logs_equal, _recorder, same

    case = make_case(46000 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    kw = case["kw"]
    K, T, V = case["K"], case["T"], case["V"]
    x = np.ascontiguousarray(case["xin"][0])
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], relaxed_pool_multiplier=[1, 2, 4][seed % 3], **_soft(seed))

    def run(lib, h):
        L = lib.lib
        out, logs = {}, {}
        for mode in ("plain", "constrained"):
            log = []
            simple, ex = _recorder(x, log)
            r = C.c_void_p()
            if mode == "plain":
                st = L.dbs_decode_model_steps(h, simple, None, 0, T, V, C.byref(r))
            else:
                keep = {}
                c = HostLib.constraints(banned=kw["banned"], repetition_penalty=1.3, no_repeat_ngram_size=2, keep=keep)
                st = L.dbs_decode_model_steps_ex(h, ex, None, 1, T, V, C.byref(c), C.byref(r))
            out[mode] = (st, lib.error(), read_result(L, r) if st == 0 else None)
            logs[mode] = log
            L.dbs_free_result(r)
        return out, logs

    (ours, our_logs), (theirs, their_logs) = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed}")
    for mode in our_logs:
        _logs_equal(our_logs[mode], their_logs[mode])


# ---------------------------------------------------------------------------
# Pool gradients: each pool entry's raw-score gradient joins its parent's
# path after the step's selected children, and its log-prob entry
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seed", range(12))
def test_pool_result_backward(libs, seed):
    """dbs_backward_dense / _sparse / _default / dbs_backward of a pooled
    result with relaxed-weight gradients (alone, with selected-weight and
    final-score gradients): the gradients and the initial scores'."""
    import ctypes as C

    from tests.host_abi import read_backward
    from tests.test_gpu_host_results import same

    case = make_case(47000 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    kw = case["kw"]
    K, T, V = case["K"], case["T"], case["V"]
    m = [1, 2, 3][seed % 3]
    x = np.ascontiguousarray(case["xin"][0])
    rng = np.random.default_rng(seed)
    P = K * m
    grw = rng.normal(0, 1, T * P).astype(np.float32)
    gw = rng.normal(0, 1, T * K).astype(np.float32)
    gf = rng.normal(0, 1, K).astype(np.float32)
    which = [(None, grw, None), (gw, grw, gf), (None, grw, gf), (gw, grw, None)][seed % 4]
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], relaxed_pool_multiplier=m, selected_temperature=0.7, **_soft(seed))

    def run(lib, h):
        L = lib.lib
        r = C.c_void_p()
        assert L.dbs_decode(h, x.ctypes.data_as(C.POINTER(C.c_float)), T, V, C.byref(r)) == 0, lib.error()
        out = {}
        f32 = C.POINTER(C.c_float)
        ptr = [None if a is None else a.ctypes.data_as(f32) for a in which]
        for name in ("dbs_backward_dense", "dbs_backward_sparse", "dbs_backward_default", "dbs_backward"):
            b = C.c_void_p()
            st = getattr(L, name)(h, r, ptr[0], ptr[1], ptr[2], C.byref(b))
            out[name] = (st, lib.error(), read_backward(L, b, T * K * V, K) if st == 0 else None)
            L.dbs_free_backward(b)
        L.dbs_free_result(r)
        return out

    ours, theirs = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed} m {m}")
    assert ours["dbs_backward_dense"][0] == 0


def _pool_trace_case(libs, seed, logits, dtype):
    case = make_case(48000 + seed, dtypes=[dtype], logits=logits, allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    m = [1, 2, 4][seed % 3]
    out = _check(libs, case, m)
    return case, m, out


@pytest.mark.parametrize("seed", range(12))
def test_pool_batch_backward(libs, seed):
    """dbs_backward_batch_into_ex with pool score and raw-score gradients
    on a pooled decode's trace (log-probs, and logits with row_lse),
    accumulating into a buffer with values; with and without the selected
    slots' gradients."""
    logits = seed % 2 == 1
    dtype = ["f32", "bf16", "f16"][seed % 3]
    case, m, out = _pool_trace_case(libs, seed, logits, dtype)
    kw = case["kw"]
    B, T, K, V = case["B"], case["T"], case["K"], case["V"]
    P = K * m
    rng = np.random.default_rng(seed)
    init = rng.normal(size=(B, T, K, V)).astype(np.float32)
    init[rng.random(init.shape) < 0.1] = -0.0
    gps = rng.normal(size=(B, T, P)).astype(np.float32)
    gpr = rng.normal(size=(B, T, P)).astype(np.float32)
    gps[rng.random(gps.shape) < 0.2] = 0.0
    runs = [dict(grad_pool_scores=gps), dict(grad_pool_raw=gpr, grad_final=rng.normal(size=(B, K)).astype(np.float32)),
            dict(grad_pool_scores=gps, grad_pool_raw=gpr, grad_scores=rng.normal(size=(B, T, K)).astype(np.float32))]
    pool = {k: out[k] for k in ("pool_parents", "pool_tokens", "pool_lengths", "pool_from_logprob")}
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], relaxed_pool_multiplier=m)
    for run in runs:
        extra = dict(logits=case["xin"], logits_dtype=dtype, row_lse=out["row_lse"]) if logits else {}

        def fn(lib, h):
            st, g = lib.backward(h, out, V, init, steps=kw["steps"], pool=pool, **extra, **run)
            return st, g, lib.error()

        (s0, g0, e0), (s1, g1, e1) = _each(libs, opts, fn)
        assert (s0, e0) == (s1, e1), (sorted(run), e0, e1)
        assert s0 == 0, e0
        bad = np.argwhere(g0.view(np.uint32) != g1.view(np.uint32))
        assert bad.size == 0, (sorted(run), tuple(bad[0]), g0[tuple(bad[0])], g1[tuple(bad[0])])


def test_pool_trace_errors_match(libs):
    """A pool trace out of range, and pool gradients without a pool trace,
    give the reference's status and text."""
    case, m, out = _pool_trace_case(libs, 3, False, "f32")
    kw = case["kw"]
    B, T, K, V = case["B"], case["T"], case["K"], case["V"]
    init = np.zeros((B, T, K, V), np.float32)
    pool = {k: np.array(out[k]) for k in ("pool_parents", "pool_tokens", "pool_lengths", "pool_from_logprob")}
    bad_pool = dict(pool)
    bad_pool["pool_tokens"] = pool["pool_tokens"].copy()
    bad_pool["pool_tokens"][B - 1, 0, 0] = V
    gps = np.ones((B, T, K * m), np.float32)
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"], relaxed_pool_multiplier=m)

    def fn(lib, h):
        got = [lib.backward(h, out, V, init, steps=kw["steps"], pool=bad_pool, grad_pool_scores=gps)[0], lib.error()]
        got += [lib.backward(h, out, V, init, steps=kw["steps"], grad_pool_scores=gps)[0], lib.error()]
        return got

    ours, theirs = _each(libs, opts, fn)
    assert ours == theirs and ours[0] == -1, (ours, theirs)
