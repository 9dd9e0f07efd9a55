# SPDX-License-Identifier: MIT
"""GPU parity of the surrogate backward through the C ABI
(dbs_cuda_backward_ex, dbs_cuda_backward, dbs_hip_backward_dense,
dbs_cuda_path_gradient), of the length penalty and of the backtrack, against
the CPU oracle. Gradients are compared bit for bit (the north star allows 1e-6
relative; the engine reproduces the reference's operation order)."""

import numpy as np
import pytest
import torch

from tests.cases import make_case, to_bits

pytestmark = pytest.mark.gpu


def _trace_and_grads(oracle, case, rng):
    kw = dict(case["kw"])
    kw.pop("banned_per_example", None)
    tr = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    B, T, K = tr["parents"].shape
    grads = {"grad_final": rng.normal(size=(B, K)).astype(np.float32)}
    if rng.random() < 0.5:
        grads["grad_final_raw"] = rng.normal(size=(B, K)).astype(np.float32)
    if rng.random() < 0.4:
        grads["grad_scores"] = rng.normal(size=(B, T, K)).astype(np.float32)
    if rng.random() < 0.4:
        grads["grad_raw"] = rng.normal(size=(B, T, K)).astype(np.float32)
    return tr, grads, kw


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


@pytest.mark.parametrize("seed", range(0, 40))
def test_backward_matches_oracle(hip, oracle, seed):
    case = make_case(2000 + seed, allow_invalid=False)
    rng = np.random.default_rng(seed)
    tr, grads, kw = _trace_and_grads(oracle, case, rng)
    logits = case["xin"] if kw["from_logits"] else None
    row_lse = tr["row_lse"] if kw["from_logits"] else None
    want = oracle.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits,
                           logits_dtype=case["dtype"], row_lse=row_lse, **grads)
    got = hip.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits, dtype=case["dtype"],
                       row_lse=row_lse, mode="accumulate", **grads)
    assert np.array_equal(_bits(got), _bits(want)), f"seed {seed}: max |diff| {np.abs(got - want).max()}"
    dense = hip.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits, dtype=case["dtype"],
                         row_lse=row_lse, mode="dense", out_type="f32", **grads)
    assert np.array_equal(_bits(dense), _bits(want))
    for out_type in ("bf16", "f16"):
        dense16 = hip.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits,
                               dtype=case["dtype"], row_lse=row_lse, mode="dense", out_type=out_type, **grads)
        assert np.array_equal(dense16, to_bits(want, out_type)), out_type


# bfloat16 logits with whole 16-byte blocks per row take the table-driven,
# vectorized dense gradient (rows whose logsumexp is below 1 fall back to the
# Cephes evaluation); every output type against the oracle, bit for bit.
@pytest.mark.parametrize("seed", range(0, 12))
def test_dense_gradient_bf16_logits(hip, oracle, seed):
    case = make_case(2600 + seed, allow_invalid=False, dtypes=["bf16"], vocabs=[8, 1000, 4104, 8200],
                     scales=[0.05, 0.5, 3.0, 8.0], logits=True)
    rng = np.random.default_rng(seed + 100)
    tr, grads, kw = _trace_and_grads(oracle, case, rng)
    want = oracle.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=case["xin"],
                           logits_dtype="bf16", row_lse=tr["row_lse"], **grads)
    for out_type in ("bf16", "f16", "f32"):
        got = hip.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=case["xin"], dtype="bf16",
                           row_lse=tr["row_lse"], mode="dense", out_type=out_type, **grads)
        expect = _bits(want) if out_type == "f32" else to_bits(want, out_type)
        assert np.array_equal(_bits(got), expect), f"seed {seed} {out_type} V{case['V']}"


def test_backward_accumulates(hip, oracle):
    case = make_case(77, allow_invalid=False)
    rng = np.random.default_rng(7)
    tr, grads, kw = _trace_and_grads(oracle, case, rng)
    init = rng.normal(size=(case["B"], case["T"], case["K"], case["V"])).astype(np.float32)
    logits = case["xin"] if kw["from_logits"] else None
    row_lse = tr["row_lse"] if kw["from_logits"] else None
    want = oracle.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits,
                           logits_dtype=case["dtype"], row_lse=row_lse, out=init.copy(), **grads)
    got = hip.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], logits=logits, dtype=case["dtype"],
                       row_lse=row_lse, mode="accumulate", initial=init.copy(), **grads)
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("seed", range(0, 10))
def test_final_scores_backward_and_path_gradient(hip, oracle, seed):
    case = make_case(3000 + seed, allow_invalid=False)
    case["kw"]["from_logits"] = False
    case["xin"] = to_bits(case["x"], case["dtype"])
    rng = np.random.default_rng(seed)
    tr, grads, kw = _trace_and_grads(oracle, case, rng)
    gf = grads["grad_final"]
    want = oracle.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], grad_final=gf)
    got = hip.backward(tr, case["V"], alpha=kw["alpha"], steps=kw["steps"], mode="final", grad_final=gf)
    assert np.array_equal(_bits(got), _bits(want))
    draws = hip.path_gradient(tr, case["V"], gf, alpha=kw["alpha"], steps=kw["steps"])
    want_draws = oracle.path_gradient(tr, case["V"], gf, alpha=kw["alpha"], steps=kw["steps"])
    assert np.array_equal(_bits(draws), _bits(want_draws))


def test_finite_differences(hip):
    # reference tests/dbs_tests.cpp:175-214: analytic gradient of the best
    # final score vs central differences of the decode
    x = np.array([-0.10, -0.40, -1.00, -2.00, -3.00, -3.20, -3.40, -3.60,
                  -0.20, -0.50, -1.10, -2.10, -0.30, -1.00, -1.20, -2.20], np.float32).reshape(1, 2, 2, 4)
    tr = hip.decode(x, "f32")
    grad = hip.backward(tr, 4, mode="final", grad_final=np.array([[1.0, 0.0]], np.float32))
    eps = 1e-3
    for i in np.argwhere(grad != 0):
        xp, xm = x.copy(), x.copy()
        xp[tuple(i)] += eps
        xm[tuple(i)] -= eps
        fd = (hip.decode(xp, "f32")["final_scores"][0, 0] - hip.decode(xm, "f32")["final_scores"][0, 0]) / (2 * eps)
        assert abs(fd - grad[tuple(i)]) < 5e-2


@pytest.mark.parametrize("alpha", [0.0, 0.6, 1.0, 2.0, 2.5, 64.0, 65.0, 0.001])
def test_length_penalty_matches_oracle(hip, oracle, alpha):
    lengths = np.concatenate([np.arange(-3, 400), [2**31 - 1, 10**6]]).astype(np.int64)
    got = hip.length_penalty(np.clip(lengths, 0, 2**31 - 1), alpha)
    want = oracle.length_penalty(lengths, alpha)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", range(0, 6))
def test_backtrack_matches_oracle(hip, oracle, seed):
    case = make_case(4000 + seed)
    kw = dict(case["kw"])
    tr = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    got = hip.backtrack(tr["tokens"], tr["parents"], kw["steps"])
    want = oracle.backtrack(tr["tokens"], tr["parents"], kw["steps"])
    assert np.array_equal(got, want)
    assert np.array_equal(hip.backtrack_i64(tr["tokens"], tr["parents"], kw["steps"]), want)
    # the path of every live final beam reproduces its raw score (reference
    # python/tests/test_api.py:118-133), checked in float64 on expanded slots
    assert got.shape == (case["B"], case["K"], case["T"])


@pytest.mark.parametrize("T", [5, 700])  # the trace staged in LDS, and too long for it
def test_backtrack_random_traces(hip, oracle, T):
    """Arbitrary parent pointers (dead ones -1) and per-example steps: the
    int32 and int64 entry points follow them as the oracle does."""
    rng = np.random.default_rng(77 + T)
    B, K = 3, 8
    tokens = rng.integers(0, 50000, size=(B, T, K))
    parents = rng.integers(-1, K, size=(B, T, K))
    steps = np.array([T, max(1, T // 2), 1])
    for st in (None, steps):
        want = oracle.backtrack(tokens, parents, st)
        assert np.array_equal(hip.backtrack(tokens, parents, st), want)
        assert np.array_equal(hip.backtrack_i64(tokens, parents, st), want)
