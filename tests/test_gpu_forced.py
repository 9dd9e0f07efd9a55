# SPDX-License-Identifier: MIT
"""Forced tokens (DBSAdvancedConstraintsC.forced_tokens, the per-example
forced_tokens_per_example of dbs_decode_batch_variable) in libdbs_hip.so,
computed on the GPU, against the reference's own CPU library
(oracle/_ref/libdbs_ref.so) called with identical arguments.

At a step whose entry is >= 0 a read beam's only candidate is the forced
token, under the checks any candidate meets: a finite log-prob, banned
tokens, the EOS mask below min_length, n-gram blocking and the repetition
penalty (reference src/decoder.cpp:125-167, src/kernels_scalar.cpp:16-26);
finished beams still compete carried. The cases force likely tokens, EOS
(ending beams, or masked below min_length), banned tokens (no candidate:
the search dies), random tokens, and negative entries other than -1 (not
forced); over the batch decodes into caller arrays (f32/f16/bf16, logits,
per-example steps, wide beams, long rows with shortlists, the overlapped
decode), with validate_inputs, the result-handle decodes (one example, the
variable batch with per-example arrays whose entries past an example's
steps are out of the vocabulary and must not be read) and the model-step
decodes. Outputs are compared bit for bit, statuses and messages as text."""

import ctypes as C
import os

import numpy as np
import pytest

from beamgrad_amd import _build
from tests.cases import first_difference, log_softmax, make_case, to_bits
from tests.host_abi import HostLib, enable_results, read_backward, read_result
from tests.test_gpu_host_results import _logs_equal, _recorder, same

pytestmark = pytest.mark.gpu

REF_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libdbs_ref.so")
OUT_KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
            "raw_scores", "from_logprob", "row_lse")


@pytest.fixture(scope="module")
def libs():
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref is not built")
    return enable_results(HostLib(_build.lib_path())), enable_results(HostLib(REF_LIB))


def _p(a, ct):
    return None if a is None else a.ctypes.data_as(C.POINTER(ct))


def _forced(rng, T, V, x, eos=-1, banned=None, density=0.6):
    """A [T] forced-token array: likely tokens (the argmax of a row of the
    step), EOS, banned tokens, random tokens; -1 and other negative entries
    leave a step free."""
    f = np.full(T, -1, np.int32)
    for t in range(T):
        if rng.random() >= density:
            continue
        r = rng.random()
        if r < 0.25 and eos >= 0:
            f[t] = eos
        elif r < 0.6:
            f[t] = int(np.argmax(x[int(rng.integers(0, x.shape[0])), t, 0]))
        elif r < 0.7 and banned is not None and banned.any():
            f[t] = int(rng.choice(np.flatnonzero(banned)))
        else:
            f[t] = int(rng.integers(0, V))
    if T > 1 and rng.random() < 0.3:
        f[int(rng.integers(0, T))] = -7
    return f


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


def _batch_decode(libs, case, forced, *, validate=0, ml=-1):
    kw = case["kw"]
    opts = dict(beam_size=case["K"], eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], validate_inputs=validate)

    def fn(lib, h):
        keep = {}
        cons = HostLib.constraints(banned=kw.get("banned"), min_length=ml,
                                   repetition_penalty=float(kw.get("repetition_penalty", 1.0)),
                                   no_repeat_ngram_size=int(kw.get("no_repeat_ngram_size") or 0), forced=forced,
                                   keep=keep)
        st, out = lib.decode(h, case["xin"], case["K"], dtype=case["dtype"], from_logits=kw["from_logits"],
                             steps=kw["steps"], constraints=cons)
        return st, out, lib.error()

    return _each(libs, opts, fn, kw.get("extra_eos"))


def _check(libs, case, forced, **more):
    (s0, o0, e0), (s1, o1, e1) = _batch_decode(libs, case, forced, **more)
    tag = f"seed {case['seed']} {case['dtype']} B{case['B']} T{case['T']} K{case['K']} V{case['V']} forced {forced}"
    assert (s0, e0) == (s1, e1), tag
    assert s0 == 0, (tag, e0)
    diff = first_difference(o0, o1, OUT_KEYS)
    assert diff is None, f"{tag}: {diff}"
    return o0


@pytest.mark.parametrize("seed", range(40))
def test_forced_batch_decodes_match_the_reference(libs, seed):
    case = make_case(31000 + seed, allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    rng = np.random.default_rng(seed)
    kw = case["kw"]
    forced = _forced(rng, case["T"], case["V"], case["x"], kw["eos_token"], kw["banned"],
                     density=[0.3, 0.6, 1.0][seed % 3])
    _check(libs, case, forced, ml=-1 if seed % 4 else int(seed % 5))


@pytest.mark.parametrize("seed", range(12))
def test_forced_constrained_decodes(libs, seed):
    """n-gram blocking and the repetition penalty over longer decodes and
    small vocabularies: forced tokens are often blocked or penalised."""
    rng = np.random.default_rng(32000 + seed)
    B, T, K, V = int(rng.integers(1, 4)), int(rng.integers(8, 25)), int(rng.choice([1, 2, 4, 8, 16, 20])), \
        int(rng.choice([5, 12, 40, 300]))
    dtype = str(rng.choice(["f32", "f16", "bf16"]))
    case = make_case(32000 + seed, dtypes=[dtype], vocabs=[V], allow_invalid=False)
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    from_logits = bool(seed % 2)
    if not from_logits:
        x = log_softmax(x)
    kw = dict(case["kw"], from_logits=from_logits, no_repeat_ngram_size=int(rng.choice([1, 2, 3])),
              repetition_penalty=float(rng.choice([1.0, 1.5])), banned_per_example=None,
              steps=[int(s) for s in rng.integers(1, T + 1, size=B)] if seed % 3 == 0 else None)
    case.update(B=B, T=T, K=K, V=V, dtype=dtype, x=x, xin=to_bits(x, dtype), kw=kw)
    # force tokens the beams have already taken (the argmax of earlier steps)
    forced = _forced(rng, T, V, x, kw["eos_token"], kw["banned"], density=0.5)
    _check(libs, case, forced)


@pytest.mark.parametrize("overlap", [1, 0])
@pytest.mark.parametrize("seed", range(6))
def test_forced_wide_beams_and_long_rows(libs, seed, overlap):
    """Wide beams (the workgroup pass's one-pass and rescan paths are
    skipped at forced steps), rows long enough for shortlists, with the
    select pass alongside the row pass and after it."""
    rng = np.random.default_rng(33000 + seed)
    B, T = int(rng.integers(1, 9)), int(rng.integers(4, 10))
    K, V = [(20, 1000), (64, 4104), (4, 32000), (33, 3000), (8, 50257), (16, 8201)][seed]
    dtype = ["f32", "bf16", "f16"][seed % 3]
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    from_logits = seed % 2 == 1
    if not from_logits:
        x = log_softmax(x)
    eos = int(rng.integers(0, V)) if seed % 3 else -1
    kw = dict(from_logits=from_logits, eos_token=eos, extra_eos=[], min_length=int(rng.integers(0, 3)),
              alpha=0.6, no_repeat_ngram_size=2 if seed == 5 else 0,
              repetition_penalty=1.2 if seed == 4 else 1.0,
              steps=[int(s) for s in rng.integers(1, T + 1, size=B)] if seed % 2 else None,
              banned=(rng.random(V) < 0.05).astype(np.uint8) if seed in (1, 3) else None, banned_per_example=None)
    case = dict(seed=33000 + seed, B=B, T=T, K=K, V=V, dtype=dtype, x=x, xin=to_bits(x, dtype), kw=kw)
    forced = _forced(rng, T, V, x, eos, kw["banned"], density=0.5)
    ours = libs[0].lib
    prev = ours.dbs_hip_set_decode_overlap(overlap)
    try:
        _check(libs, case, forced)
    finally:
        ours.dbs_hip_set_decode_overlap(prev)


@pytest.mark.parametrize("from_logits", [False, True])
def test_forced_steps_still_validate_whole_rows(libs, from_logits):
    """validate_inputs checks every element of a row a forced step reads,
    not only the forced one."""
    rng = np.random.default_rng(7)
    B, T, K, V = 3, 4, 3, 50
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    if not from_logits:
        x = log_softmax(x)
    x[1, 2, :, 7] = np.nan
    case = dict(seed=7, B=B, T=T, K=K, V=V, dtype="f32", x=x, xin=x,
                kw=dict(from_logits=from_logits, eos_token=-1, extra_eos=[], min_length=0, alpha=0.0, steps=None,
                        banned=None, no_repeat_ngram_size=0, repetition_penalty=1.0))
    forced = np.array([3, -1, 11, 4], np.int32)
    (s0, _, e0), (s1, _, e1) = _batch_decode(libs, case, forced, validate=1)
    assert s0 == s1 == -1
    assert e0 == e1 and "NaN or +inf" in e0 and e0.startswith("example 1:"), (e0, e1)
    _check(libs, case, forced)


@pytest.mark.parametrize("seed", range(8))
def test_forced_backward_of_forced_traces(libs, seed):
    """The backward of a forced trace (its selected entries are the forced
    log-probs) into caller arrays."""
    case = make_case(34000 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    case["kw"]["banned_per_example"] = None
    rng = np.random.default_rng(seed)
    forced = _forced(rng, case["T"], case["V"], case["x"], case["kw"]["eos_token"], case["kw"]["banned"])
    out = _check(libs, case, forced)
    B, T, K, V = case["B"], case["T"], case["K"], case["V"]
    init = rng.normal(size=(B, T, K, V)).astype(np.float32)
    gf = rng.normal(size=(B, K)).astype(np.float32)
    gs = rng.normal(size=(B, T, K)).astype(np.float32)
    kw = case["kw"]
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"])

    def fn(lib, h):
        st, g = lib.backward(h, out, V, init, steps=kw["steps"], grad_final=gf, grad_scores=gs)
        return st, g, lib.error()

    (s0, g0, e0), (s1, g1, e1) = _each(libs, opts, fn)
    assert (s0, e0) == (s1, e1) and s0 == 0, e0
    assert np.array_equal(g0.view(np.uint32), g1.view(np.uint32))


@pytest.mark.parametrize("seed", range(10))
def test_forced_result_decodes(libs, seed):
    """dbs_decode_constrained and dbs_decode_constrained_ex with forced
    tokens (one example), the dense backward of the result."""
    case = make_case(35000 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    kw = case["kw"]
    K, T, V = case["K"], case["T"], case["V"]
    x = np.ascontiguousarray(case["xin"][0])
    rng = np.random.default_rng(seed)
    forced = _forced(rng, T, V, case["x"][:1], kw["eos_token"], kw["banned"])
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"], selected_temperature=[0.0, 0.5][seed % 2])
    gw = rng.normal(0, 1, T * K).astype(np.float32)

    def run(lib, h):
        L = lib.lib
        res = {}
        r = C.c_void_p()
        st = L.dbs_decode_constrained(h, _p(x, C.c_float), T, V, _p(kw["banned"], C.c_uint8),
                                      _p(forced, C.c_int32), kw["min_length"], C.byref(r))
        res["constrained"] = (st, lib.error(), read_result(L, r) if st == 0 else None)
        if st == 0:
            b = C.c_void_p()
            st2 = L.dbs_backward_dense(h, r, _p(gw, C.c_float), None, None, C.byref(b))
            res["backward"] = (st2, lib.error(), read_backward(L, b, T * K * V, K) if st2 == 0 else None)
            L.dbs_free_backward(b)
        L.dbs_free_result(r)
        keep = {}
        c = HostLib.constraints(banned=kw["banned"], repetition_penalty=1.3, no_repeat_ngram_size=2, forced=forced,
                                keep=keep)
        st = L.dbs_decode_constrained_ex(h, _p(x, C.c_float), T, V, C.byref(c), C.byref(r))
        res["constrained_ex"] = (st, lib.error(), read_result(L, r) if st == 0 else None)
        L.dbs_free_result(r)
        return res

    ours, theirs = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed}")


@pytest.mark.parametrize("seed", range(8))
def test_forced_variable_batches(libs, seed):
    """dbs_decode_batch_variable with forced_tokens_per_example [B,
    max_steps]: each example reads its own row as far as its own steps
    (entries past them are outside the vocabulary and must not be read)."""
    rng = np.random.default_rng(36000 + seed)
    B, T, Kmax, V = int(rng.integers(1, 6)), int(rng.integers(2, 9)), int(rng.choice([2, 4, 8, 16])), \
        int(rng.choice([7, 50, 300, 1001]))
    x = np.ascontiguousarray(log_softmax(rng.normal(0, 2.0, (B, T, Kmax, V)).astype(np.float32)))
    steps = rng.integers(1, T + 1, B).astype(np.int32)
    beams = rng.integers(1, Kmax + 1, B).astype(np.int32)
    eos = rng.integers(-1, V, B).astype(np.int32)
    mins = rng.integers(-1, 4, B).astype(np.int32)
    banned = (rng.random((B, V)) < 0.1).astype(np.uint8)
    forced = np.stack([_forced(rng, T, V, x[b:b + 1], int(eos[b]), banned[b]) for b in range(B)])
    for b in range(B):
        forced[b, steps[b]:] = V + 3
    use = [rng.random() < 0.7 for _ in range(4)]
    args = [a if u else None for a, u in zip((beams, eos, mins, banned), use)]
    opts = dict(beam_size=int(rng.integers(1, Kmax + 1)), eos_token=int(rng.integers(-1, V)),
                length_penalty_alpha=float(rng.choice([0.0, 0.6])))

    def run(lib, h):
        L = lib.lib
        br = C.c_void_p()
        st = L.dbs_decode_batch_variable(h, _p(x, C.c_float), B, T, Kmax, V, _p(steps, C.c_int32),
                                         _p(args[0], C.c_int32), _p(args[1], C.c_int32), _p(args[2], C.c_int32),
                                         _p(args[3], C.c_uint8), _p(np.ascontiguousarray(forced), C.c_int32), 1,
                                         C.byref(br))
        out = [read_result(L, L.dbs_batch_result_at(br, b)) for b in range(L.dbs_batch_result_size(br))]
        L.dbs_free_batch_result(br)
        return st, lib.error(), out

    ours, theirs = _each(libs, opts, run)
    assert ours[:2] == theirs[:2], (ours[:2], theirs[:2])
    assert ours[0] == 0, ours[1]
    for b, (a, c) in enumerate(zip(ours[2], theirs[2])):
        same(a, c, f"example {b}")


@pytest.mark.parametrize("seed", range(6))
def test_forced_model_step_decodes(libs, seed):
    """dbs_decode_model_steps_ex with forced tokens: each step's selection
    on the GPU step API with that step's forced token; the callbacks see the
    same beams."""
    case = make_case(37000 + seed, dtypes=["f32"], logits=False, allow_invalid=False)
    kw = case["kw"]
    K, T, V = case["K"], case["T"], case["V"]
    x = np.ascontiguousarray(case["xin"][0])
    rng = np.random.default_rng(seed)
    forced = _forced(rng, T, V, case["x"][:1], kw["eos_token"], kw["banned"])
    opts = dict(beam_size=K, eos_token=kw["eos_token"], length_penalty_alpha=kw["alpha"],
                min_length=kw["min_length"])

    def run(lib, h):
        L = lib.lib
        out, logs = {}, {}
        for mode in ("plain", "constrained"):
            log = []
            _, ex = _recorder(x, log)
            keep = {}
            c = HostLib.constraints(banned=kw["banned"] if mode == "constrained" else None,
                                    repetition_penalty=1.3 if mode == "constrained" else 1.0,
                                    no_repeat_ngram_size=2 if mode == "constrained" else 0, forced=forced, keep=keep)
            r = C.c_void_p()
            st = L.dbs_decode_model_steps_ex(h, ex, None, 1, T, V, C.byref(c), C.byref(r))
            out[mode] = (st, lib.error(), read_result(L, r) if st == 0 else None)
            logs[mode] = log
            L.dbs_free_result(r)
        return out, logs

    (ours, our_logs), (theirs, their_logs) = _each(libs, opts, run, kw["extra_eos"])
    same(ours, theirs, f"seed {seed}")
    for mode in our_logs:
        _logs_equal(our_logs[mode], their_logs[mode])
