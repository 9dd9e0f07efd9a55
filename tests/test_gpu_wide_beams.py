# SPDX-License-Identifier: MIT
"""Beams up to DBS_CUDA_MAX_BEAM = 1024 on the GPU (the reference tests
K = 1024 itself: python/tests/test_cuda.py:32, tests/cuda_device_tests.cpp:201,
:545), against the CPU oracle bit for bit: decode (every output), the dense
backward and both backtrack entry points.

Small vocabularies make the wide beams meet their edge cases: at step 0 only
V candidates exist, so K > V leaves dead slots (parent and token -1, score
-inf) that later steps and the backtrack must carry; K > 256 exceeds one
workgroup's thread count in the select pass's rank compaction and in the
backtrack's beam loop."""

import numpy as np
import pytest

from tests.cases import first_difference, log_softmax, to_bits

pytestmark = pytest.mark.gpu


def _rows(seed, B, T, K, V, *, logits, ties):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 2.0, size=(B, T, K, V)).astype(np.float32)
    if not logits:
        x = log_softmax(x)
    if ties:  # many exact ties across rows and beams (ranked by token, then beam)
        pool = rng.choice(x.reshape(-1), size=5)
        mask = rng.random(x.shape) < 0.3
        x[mask] = rng.choice(pool, size=int(mask.sum()))
    x[rng.random(x.shape) < 0.02] = -np.inf
    return x


CASES = [
    # K, V, dtype, logits, options
    (128, 9, "f32", False, dict(eos_token=2, min_length=2, alpha=0.6)),
    (128, 300, "bf16", True, dict(eos_token=17, extra_eos=[4], alpha=1.0)),
    (257, 40, "f16", False, dict(eos_token=-1, alpha=0.0, no_repeat_ngram_size=2)),
    (512, 3, "f32", False, dict(eos_token=1, alpha=2.5, repetition_penalty=1.5)),
    (512, 700, "bf16", True, dict(eos_token=5, min_length=3, alpha=0.6)),
    (1024, 7, "f32", False, dict(eos_token=0, alpha=1.0)),
    (1024, 64, "bf16", True, dict(eos_token=63, extra_eos=[1, 2], min_length=1, alpha=0.6)),
    (1024, 1031, "f32", False, dict(eos_token=-1, alpha=0.0)),
]


def _case(i):
    K, V, dtype, logits, opts = CASES[i]
    B, T = 2, 4
    x = _rows(900 + i, B, T, K, V, logits=logits, ties=i % 2 == 0)
    kw = dict(from_logits=logits, eos_token=opts.get("eos_token", -1), extra_eos=opts.get("extra_eos", []),
              min_length=opts.get("min_length", 0), alpha=opts["alpha"],
              no_repeat_ngram_size=opts.get("no_repeat_ngram_size", 0),
              repetition_penalty=opts.get("repetition_penalty", 1.0),
              steps=[T, T - 1] if i % 3 == 0 else None)
    return x, to_bits(x, dtype), dtype, kw


@pytest.mark.parametrize("i", range(len(CASES)))
def test_wide_beam_decode(hip, oracle, i):
    x, xin, dtype, kw = _case(i)
    want = oracle.decode(xin, dtype=dtype, **kw)
    got = hip.decode(xin, dtype, **kw)
    diff = first_difference(got, want)
    assert diff is None, f"K={x.shape[2]} V={x.shape[3]} {dtype}: {diff}"
    if x.shape[2] > x.shape[3]:
        # step 0 offers V candidates: the other slots are dead
        assert (want["parents"][:, 0, x.shape[3]:] == -1).all()


@pytest.mark.parametrize("i", range(len(CASES)))
def test_wide_beam_backward_and_backtrack(hip, oracle, i):
    x, xin, dtype, kw = _case(i)
    tr = oracle.decode(xin, dtype=dtype, **kw)
    B, T, K = tr["parents"].shape
    V = x.shape[3]
    rng = np.random.default_rng(i)
    grads = dict(grad_final=rng.normal(size=(B, K)).astype(np.float32),
                 grad_scores=rng.normal(size=(B, T, K)).astype(np.float32))
    logits = xin if kw["from_logits"] else None
    row_lse = tr["row_lse"] if kw["from_logits"] else None
    want = oracle.backward(tr, V, alpha=kw["alpha"], steps=kw["steps"], logits=logits, logits_dtype=dtype,
                           row_lse=row_lse, **grads)
    got = hip.backward(tr, V, alpha=kw["alpha"], steps=kw["steps"], logits=logits, dtype=dtype, row_lse=row_lse,
                       mode="dense", out_type="f32", **grads)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    draws = hip.path_gradient(tr, V, grads["grad_final"], alpha=kw["alpha"], steps=kw["steps"])
    want_draws = oracle.path_gradient(tr, V, grads["grad_final"], alpha=kw["alpha"], steps=kw["steps"])
    assert np.array_equal(draws.view(np.uint32), want_draws.view(np.uint32))
    paths = oracle.backtrack(tr["tokens"], tr["parents"], kw["steps"])
    assert np.array_equal(hip.backtrack(tr["tokens"], tr["parents"], kw["steps"]), paths)
    assert np.array_equal(hip.backtrack_i64(tr["tokens"], tr["parents"], kw["steps"]), paths)
    if K > V:  # dead final beams exist only when fewer than K hypotheses survive
        dead = ~np.isfinite(tr["final_raw_scores"])
        assert (paths[dead] == -1).all()
