# SPDX-License-Identifier: MIT
"""CPU checks that pin the oracle (oracle/dbs_oracle.c) before it is trusted
as the checker of the HIP engine:

* against the reference's own CPU library (oracle/_ref, where it is built) on
  random cases, bit for bit;
* against the committed fixtures written by that library (tests/golden);
* against the reference's known-answer tests (ties, the two-step golden
  case, the C API example, finite differences);
* against what the mathematics fixes: closed forms for the penalty, exp,
  logsumexp and the 16-bit conversions, exhaustive enumeration for beam
  search wide enough to keep every path, and greedy search for one beam.
"""

import itertools
import math

import numpy as np
import pytest

from oracle.oracle import Oracle, Reference, reference_available
from tests.cases import first_difference, load_golden, log_softmax, make_case

KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
        "raw_scores", "from_logprob", "row_lse")


# ---------------------------------------------------------------------------
# against the reference library
# ---------------------------------------------------------------------------

needs_ref = pytest.mark.skipif(not reference_available(), reason="oracle/_ref not built (reference not mounted)")


@needs_ref
@pytest.mark.parametrize("seed", range(0, 80))
def test_decode_matches_reference_library(oracle, seed):
    case = make_case(100 + seed, allow_invalid=False)
    kw = dict(case["kw"])
    bpe = kw.pop("banned_per_example")
    want_kw = dict(kw)
    ref = Reference()
    if bpe is not None:
        banned = want_kw.pop("banned")
        merged = bpe if banned is None else (bpe | banned[None, :])
        want = ref.decode_per_example_banned(case["xin"], merged, dtype=case["dtype"], **want_kw)
    else:
        want = ref.decode(case["xin"], dtype=case["dtype"], **want_kw)
    got = oracle.decode(case["xin"], dtype=case["dtype"], banned_per_example=bpe, **kw)
    assert first_difference(got, want, KEYS) is None


@needs_ref
@pytest.mark.parametrize("seed", range(0, 24))
def test_per_example_options_match_reference_variable_batch(oracle, seed):
    """Oracle.decode_per_example (each example alone on its first beams[b]
    rows, slots past them empty) against the reference library's
    dbs_decode_batch_variable (float32 rows, per-example steps, beams, EOS
    tokens, minimum lengths)."""
    rng = np.random.default_rng(seed)
    B, T = int(rng.integers(1, 6)), int(rng.integers(1, 8))
    K, V = int(rng.choice([1, 2, 4, 7])), int(rng.choice([3, 13, 40, 300]))
    x = log_softmax(rng.normal(0, 2.0, (B, T, K, V)).astype(np.float32))
    if rng.random() < 0.5:
        x[rng.random(x.shape) < 0.05] = x.reshape(-1)[0]  # ties
    beams = [int(v) for v in rng.integers(1, K + 1, B)]
    eos = [int(v) for v in rng.integers(0, V, B)] if rng.random() < 0.7 else [int(v) for v in rng.integers(-1, V, B)]
    mins = [int(v) for v in rng.integers(0, 5, B)]
    steps = [int(v) for v in rng.integers(1, T + 1, B)] if rng.random() < 0.5 else None
    # the reference library's extra EOS tokens need an EOS token for every example
    extra = tuple(int(v) for v in rng.integers(0, V, 2)) if min(eos) >= 0 and rng.random() < 0.5 else ()
    alpha = float(rng.choice([0.0, 0.6, 1.0]))
    want = Reference().decode_variable(x, beam_size=K, beams=beams, eos_tokens=eos, min_lengths=mins, steps=steps,
                                       eos_token=0, extra_eos=extra, alpha=alpha)
    got = oracle.decode_per_example(x, dtype="f32", beams=beams, eos_tokens=eos, min_lengths=mins, steps=steps,
                                    extra_eos=extra, alpha=alpha)
    keys = ("final_scores", "final_raw_scores", "tokens", "parents", "lengths", "scores", "raw_scores")
    assert first_difference(got, want, keys) is None


@needs_ref
@pytest.mark.parametrize("seed", range(0, 30))
def test_invalid_flags_match_reference_validation(oracle, seed):
    """The reference rejects (validate_inputs) exactly the examples the oracle flags."""
    case = make_case(600 + seed)
    kw = dict(case["kw"])
    kw.pop("banned_per_example")
    got = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    ref = Reference()
    for b in range(case["B"]):
        steps = None if kw["steps"] is None else [kw["steps"][b]]
        kwb = dict(kw, steps=steps)
        try:
            ref.decode(case["xin"][b:b + 1], dtype=case["dtype"], validate=True, **kwb)
            rejected = False
        except Exception:
            rejected = True
        assert rejected == bool(got["invalid"][b])


@needs_ref
@pytest.mark.parametrize("seed", range(0, 30))
def test_backward_matches_reference_library(oracle, seed):
    case = make_case(800 + seed, allow_invalid=False)
    kw = dict(case["kw"])
    kw.pop("banned_per_example")
    tr = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    rng = np.random.default_rng(seed)
    B, T, K = tr["parents"].shape
    grads = dict(grad_final=rng.normal(size=(B, K)).astype(np.float32),
                 grad_final_raw=rng.normal(size=(B, K)).astype(np.float32),
                 grad_scores=rng.normal(size=(B, T, K)).astype(np.float32),
                 grad_raw=rng.normal(size=(B, T, K)).astype(np.float32))
    logits = case["xin"] if kw["from_logits"] else None
    row_lse = tr["row_lse"] if kw["from_logits"] else None
    a = oracle.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits,
                        logits_dtype=case["dtype"], row_lse=row_lse, **grads)
    b = Reference().backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits,
                             logits_dtype=case["dtype"], row_lse=row_lse, **grads)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------------------
# against the committed fixtures
# ---------------------------------------------------------------------------

GOLDEN = load_golden()


@pytest.mark.parametrize("index", range(len(GOLDEN)))
def test_decode_matches_golden(oracle, index):
    g = GOLDEN[index]
    got = oracle.decode(g["xin"], dtype=g["dtype"], **g["kw"])
    assert first_difference(got, g["out"], KEYS) is None


@pytest.mark.parametrize("index", range(len(GOLDEN)))
def test_backward_matches_golden(oracle, index):
    g = GOLDEN[index]
    kw = g["kw"]
    logits = g["xin"] if kw["from_logits"] else None
    grad = oracle.backward(g["out"], g["V"], alpha=kw["alpha"], steps=kw["steps"], grad_final=g["grad_final"],
                           grad_scores=g["grad_scores"], logits=logits, logits_dtype=g["dtype"],
                           row_lse=g["out"]["row_lse"] if kw["from_logits"] else None)
    assert np.array_equal(grad.view(np.uint32), g["grad"].view(np.uint32))


# ---------------------------------------------------------------------------
# known answers from the reference's tests
# ---------------------------------------------------------------------------


def test_ties_pick_lowest_tokens(oracle):
    # reference tests/dbs_tests.cpp:128-142
    out = oracle.decode(np.full((1, 1, 2, 5), -1.0, np.float32))
    assert out["tokens"][0, 0].tolist() == [0, 1]


def test_golden_two_step(oracle):
    # reference tests/dbs_tests.cpp:489-508
    x = np.array([0.0, -1.0, -2.0, -3.0, -4.0, -5.0, -0.5, -0.1, -2.0, -0.2, -0.3, -2.0], np.float32)
    out = oracle.decode(x.reshape(1, 2, 2, 3))
    assert out["tokens"][0, 0, 0] == 0 and out["tokens"][0, 1, 0] == 1


def test_c_api_example(oracle):
    # reference examples/c_api.c: "best beam: tokens 0 1, score -0.300" and a
    # gradient of 1.000 at flattened [T, K, V] indices 0 and 7
    x = np.array([-0.1, -1.0, -2.0, -9.0, -9.0, -9.0, -0.5, -0.2, -2.0, -0.3, -0.9, -2.0], np.float32)
    out = oracle.decode(x.reshape(1, 2, 2, 3))
    assert out["tokens"][0, 0, 0] == 0 and out["tokens"][0, 1, 0] == 1
    assert f"{out['final_scores'][0, 0]:.3f}" == "-0.300"
    grad = oracle.backward(out, 3, grad_final=np.array([[1.0, 0.0]], np.float32)).reshape(-1)
    assert np.nonzero(grad)[0].tolist() == [0, 7] and np.allclose(grad[[0, 7]], 1.0)


def test_finite_differences(oracle):
    # reference tests/dbs_tests.cpp:175-214
    x = np.array([-0.10, -0.40, -1.00, -2.00, -3.00, -3.20, -3.40, -3.60,
                  -0.20, -0.50, -1.10, -2.10, -0.30, -1.00, -1.20, -2.20], np.float32).reshape(1, 2, 2, 4)
    out = oracle.decode(x)
    grad = oracle.backward(out, 4, grad_final=np.array([[1.0, 0.0]], np.float32))
    eps = 1e-3
    assert (grad != 0).sum() == 2
    for i in np.argwhere(grad != 0):
        xp, xm = x.copy(), x.copy()
        xp[tuple(i)] += eps
        xm[tuple(i)] -= eps
        fd = (oracle.decode(xp)["final_scores"][0, 0] - oracle.decode(xm)["final_scores"][0, 0]) / (2 * eps)
        assert abs(fd - grad[tuple(i)]) < 5e-2


def test_logits_finite_differences(oracle):
    """Through the log-softmax: d final / d logits vs central differences in float64 terms."""
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, size=(1, 3, 2, 6)).astype(np.float32)
    out = oracle.decode(x, from_logits=True, alpha=0.6)
    grad = oracle.backward(out, 6, alpha=0.6, grad_final=np.array([[1.0, 0.0]], np.float32), logits=x,
                           row_lse=out["row_lse"])
    eps = 1e-2
    for i in itertools.product(range(1), range(3), range(2), range(6)):
        xp, xm = x.copy(), x.copy()
        xp[i] += eps
        xm[i] -= eps
        op, om = oracle.decode(xp, from_logits=True, alpha=0.6), oracle.decode(xm, from_logits=True, alpha=0.6)
        if not (np.array_equal(op["tokens"], out["tokens"]) and np.array_equal(om["tokens"], out["tokens"])):
            continue  # the selection changed: the surrogate holds it fixed
        fd = (op["final_scores"][0, 0] - om["final_scores"][0, 0]) / (2 * eps)
        assert abs(fd - grad[i]) < 2e-2, (i, fd, grad[i])


# ---------------------------------------------------------------------------
# closed forms and brute force
# ---------------------------------------------------------------------------


def test_length_penalty_closed_form(oracle):
    # within 1 ulp of pow (reference tests/internal_tests.cpp:1246-1269); integer
    # exponents exact
    lengths = np.arange(0, 2001)
    for alpha in (0.0, 0.1, 0.25, 0.5, 0.6, 0.7, 1.0, 1.3, 2.0, 3.0, 3.7):
        a32 = float(np.float32(alpha))  # the penalty takes alpha as float32
        got = oracle.length_penalty(lengths, a32)
        base = (5.0 + np.maximum(lengths, 1).astype(np.float64)) / 6.0
        want = np.power(base, a32).astype(np.float32)
        gap = np.abs(got.view(np.uint32).astype(np.int64) - want.view(np.uint32).astype(np.int64))
        assert gap.max() <= 1
        if alpha == int(alpha):
            assert np.array_equal(got, want)
    # exponents far beyond int range saturate (reference tests/internal_tests.cpp:1257-1262)
    for alpha in (64.5, 1.0e4, 3.0e9, 1.0e30, float(np.finfo(np.float32).max)):
        assert oracle.length_penalty([1, 100], alpha).tolist() == [1.0, np.inf]


def test_log_and_exp_series(oracle):
    lib = oracle.lib
    for x in (1.0, 1.0000001, 1.5, 2.0, 10.0, 151936.0, 1e30):
        assert abs(lib.orc_log_ge1(x) - math.log(x)) <= 4e-16 * max(1.0, math.log(x))
    for y in (0.0, 0.1, 1.0, 5.5, 40.0, 300.0):
        assert abs(lib.orc_exp_ge0(y) - math.exp(y)) <= 4e-16 * math.exp(y)


def test_exp_nonpositive_closed_form(oracle):
    x = -np.concatenate([np.linspace(0, 87, 20001), np.geomspace(1e-30, 1, 2001)]).astype(np.float32)
    got = oracle.exp_nonpositive(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    assert np.all(np.abs(got - want) <= 2.0 * np.spacing(want.astype(np.float32)))
    assert oracle.exp_nonpositive(np.array([0.0, -87.5, -np.inf, np.nan], np.float32)).tolist() == [1.0, 0.0, 0.0, 0.0]


def test_half_conversions_exhaustive(oracle):
    lib = oracle.lib
    # every 16-bit pattern; NaN payloads are not compared (ctypes returns
    # floats through a double, which quiets signaling NaNs)
    bits = np.arange(65536, dtype=np.uint32)
    f16 = np.array([lib.orc_f16_to_f32(int(h)) for h in bits], np.float32)
    want16 = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want16)
    assert np.array_equal(f16.view(np.uint32)[~nan], want16.view(np.uint32)[~nan])
    assert np.all(np.isnan(f16[nan]))
    bf = np.array([lib.orc_bf16_to_f32(int(h)) for h in bits], np.float32)
    want_bf = (bits << 16).astype(np.uint32).view(np.float32)
    nan = np.isnan(want_bf)
    assert np.array_equal(bf.view(np.uint32)[~nan], want_bf.view(np.uint32)[~nan])
    assert np.all(np.isnan(bf[nan]))


def test_row_stats_against_float64(oracle):
    rng = np.random.default_rng(11)
    for V in (1, 2, 255, 256, 257, 5000, 151936):
        row = rng.normal(0, 3, size=V).astype(np.float32)
        mx, lse, bad = oracle.row_stats(row)
        want = float(np.log(np.exp(row.astype(np.float64) - row.max()).sum()) + row.max())
        assert mx == row.max() and not bad
        assert abs(lse - want) <= 1e-5 * max(1.0, abs(mx))
    _, lse, bad = oracle.row_stats(np.array([-np.inf, np.nan, np.inf], np.float32))
    assert lse == -np.inf and bad


def _path_sum(x, path):
    raw = np.float32(0.0)
    for t, (k, v) in enumerate(path):
        raw = np.float32(raw + x[t, k, v])
    return raw


def test_beam_wider_than_all_paths_is_exhaustive(oracle):
    """With K >= V^T every path survives: the final raw scores are all path
    sums (accumulated in float32 in step order), best first."""
    rng = np.random.default_rng(21)
    V, T = 3, 3
    K = V ** T
    x = rng.normal(0, 1, size=(T, K, V)).astype(np.float32)
    out = oracle.decode(x[None])
    sums = []
    for seq in itertools.product(range(V), repeat=T):
        # the row a path reads at step t is that of the slot holding its prefix
        sums.append(seq)
    # follow the decode's own slots to find each path's rows, then recompute
    finals = out["final_raw_scores"][0]
    tokens, parents = out["tokens"][0], out["parents"][0]
    got_paths = set()
    for k in range(K):
        beam, seq, raw = k, [], np.float32(0.0)
        path = []
        for t in range(T - 1, -1, -1):
            path.append((int(parents[t, beam]), int(tokens[t, beam])))
            beam = int(parents[t, beam])
        path.reverse()
        got_paths.add(tuple(v for _, v in path))
        assert _path_sum(x, path) == finals[k]
    assert len(got_paths) == V ** T  # every sequence is a final beam
    assert np.all(np.diff(finals) <= 0)


def test_single_beam_is_greedy(oracle):
    rng = np.random.default_rng(4)
    x = rng.normal(0, 1, size=(1, 6, 1, 50)).astype(np.float32)
    x[0, 2, 0, 7] = x[0, 2, 0, 3] = 9.0  # tie: the lower token wins
    out = oracle.decode(x)
    assert out["tokens"][0, :, 0].tolist() == [int(np.argmax(x[0, t, 0])) for t in range(6)]
    assert out["tokens"][0, 2, 0] == 3


# ---------------------------------------------------------------------------
# path gradient and backtrack, pinned by the reference library and by the
# reference's own property test
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("seed", range(0, 20))
def test_path_gradient_scatters_to_reference_dense_backward(oracle, seed):
    """The per-slot draws, scattered to (t, parent, token) of the slots that
    took a log-prob, are the reference library's dense final-scores gradient
    (at a step the log-prob slots have distinct (parent, token) pairs)."""
    if not reference_available():
        pytest.skip("reference library not built")
    case = make_case(2300 + seed, allow_invalid=False)
    kw = dict(case["kw"])
    kw.pop("banned_per_example")
    tr = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    B, T, K = tr["parents"].shape
    V = case["V"]
    gf = np.random.default_rng(seed).normal(size=(B, K)).astype(np.float32)
    draws = oracle.path_gradient(tr, V, gf, alpha=kw["alpha"], steps=kw["steps"])
    dense = np.zeros((B, T, K, V), np.float32)
    b_i, t_i, k_i = np.nonzero(draws)
    assert np.all(tr["from_logprob"][b_i, t_i, k_i] == 1)
    dense[b_i, t_i, tr["parents"][b_i, t_i, k_i], tr["tokens"][b_i, t_i, k_i]] += draws[b_i, t_i, k_i]
    want = Reference().backward(tr, V, alpha=kw["alpha"], steps=kw["steps"], grad_final=gf)
    assert np.array_equal(dense.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", range(0, 10))
def test_backtracked_paths_reproduce_raw_scores(oracle, seed):
    """Restates the reference's python/tests/test_api.py:118-133 on the
    oracle: following parents back from each final beam gives the tokens of
    the backtracked sequence, the log-probs taken on the way sum to the final
    raw score, and every path starts from beam 0; steps past an example's
    length hold -1 (python/beamgrad/_torch.py:582-606)."""
    rng = np.random.default_rng(4100 + seed)
    B, T, K, V = 3, 6, 4, 13
    x = log_softmax(rng.normal(size=(B, T, K, V)).astype(np.float32))
    steps = [6, 4, 1] if seed % 2 else None
    out = oracle.decode(x, eos_token=3, alpha=0.5, steps=steps)
    paths = oracle.backtrack(out["tokens"], out["parents"], steps)
    for b in range(B):
        n = T if steps is None else steps[b]
        for k in range(K):
            total, beam = 0.0, k
            for t in range(T - 1, -1, -1):
                if t >= n:
                    assert paths[b, k, t] == -1
                    continue
                if out["from_logprob"][b, t, beam]:
                    total += float(x[b, t, out["parents"][b, t, beam], out["tokens"][b, t, beam]])
                assert paths[b, k, t] == out["tokens"][b, t, beam]
                beam = int(out["parents"][b, t, beam])
            assert abs(total - float(out["final_raw_scores"][b, k])) <= 1e-5 * max(1.0, abs(total))
            assert beam == 0


def _forward_paths(tokens, parents, steps):
    """The backtrack's result built forwards, independently of its backward
    walk: after step t, slot k holds its parent slot's sequence (every entry
    -1 when the parent is -1, i.e. the slot is dead or descends from nothing)
    with tokens[t, k] appended; the final beams are the slots after the
    example's last step, padded with -1."""
    B, T, K = tokens.shape
    out = np.full((B, K, T), -1, np.int64)
    for b in range(B):
        n = T if steps is None else int(steps[b])
        seqs = [[] for _ in range(K)]
        for t in range(n):
            seqs = [([-1] * t if parents[b, t, k] < 0 else list(seqs[parents[b, t, k]])) + [int(tokens[b, t, k])]
                    for k in range(K)]
        for k in range(K):
            out[b, k, :n] = seqs[k]
    return out


@pytest.mark.parametrize("seed", range(0, 12))
def test_backtrack_dead_beams_against_forward_construction(oracle, seed):
    """The backtrack's dead-beam branch (a parent of -1 ends the walk; every
    earlier step of that beam holds -1) pinned by brute force: the sequences
    built forwards from the parent pointers. Traces come from decodes where
    beams die (K above the number of paths: V^t < K at early steps, and rows
    that are all -inf) and from arbitrary pointer tables with -1 anywhere."""
    rng = np.random.default_rng(6100 + seed)
    B, T = 3, 5
    K = int(rng.choice([4, 8, 16]))
    V = int(rng.choice([2, 3]))
    x = log_softmax(rng.normal(size=(B, T, K, V)).astype(np.float32))
    x[rng.random((B, T, K)) < 0.15] = -np.inf  # whole rows with no finite entry
    steps = [T, 3, 1] if seed % 2 else None
    out = oracle.decode(x, eos_token=int(rng.integers(-1, V)), alpha=0.5, steps=steps)
    assert (out["parents"] < 0).any()  # dead beams occur
    got = oracle.backtrack(out["tokens"], out["parents"], steps)
    assert np.array_equal(got, _forward_paths(out["tokens"], out["parents"], steps))
    dead = ~np.isfinite(out["final_raw_scores"])
    assert (got[dead] == -1).all()
    # arbitrary pointers: a walk may end at any step
    tokens = rng.integers(0, 100, size=(B, T, K))
    parents = rng.integers(-1, K, size=(B, T, K))
    for st in (None, [T, 2, 1]):
        assert np.array_equal(oracle.backtrack(tokens, parents, st), _forward_paths(tokens, parents, st))
