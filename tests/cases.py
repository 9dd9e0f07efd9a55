# SPDX-License-Identifier: MIT
"""Seeded decode cases shared by the CPU oracle tests and the GPU parity tests.

Each case is a dict: ``x`` (numpy float32 [B, T, K, V] values before the cast
to ``dtype``), ``xin`` (the bytes both paths read: float32, or uint16 bit
patterns for f16/bf16) and the decode options. The generator covers what the
reference's tests exercise: ties, -inf, NaN/+inf, banned tokens (shared and per
example), EOS with extra EOS tokens, min_length, length penalty, n-gram
blocking, repetition penalty, per-example steps, logits and 16-bit rows.
"""

from __future__ import annotations

import numpy as np


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "f16":
        return np.ascontiguousarray(x.astype(np.float16).view(np.uint16))
    import torch

    return np.ascontiguousarray(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16)
                                .view(torch.int16).numpy().view(np.uint16))


def log_softmax(x: np.ndarray) -> np.ndarray:
    m = x.max(-1, keepdims=True)
    return (x - m - np.log(np.exp(x - m).sum(-1, keepdims=True))).astype(np.float32)


def make_case(seed: int, *, big: bool = False, allow_invalid: bool = True, dtypes=None, vocabs=None,
              scales=None, logits=None) -> dict:
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 5))
    T = int(rng.integers(1, 9))
    K = int(rng.choice([1, 2, 3, 4, 5, 8, 9, 16] + ([33, 64, 100] if big else [])))
    vocab_pool = vocabs if vocabs is not None else [2, 3, 7, 40, 255, 256, 257, 1000, 1001, 3000] + (
        [32000, 50257] if big else [])
    V = int(rng.choice(vocab_pool))
    dtype = str(rng.choice(dtypes if dtypes is not None else ["f32", "f16", "bf16"]))
    from_logits = bool(rng.integers(0, 2))
    if logits is not None:
        from_logits = bool(logits)
    scale = float(rng.choice(scales if scales is not None else [0.5, 2.0, 3.0]))
    x = rng.normal(0.0, scale, size=(B, T, K, V)).astype(np.float32)
    if not from_logits:
        x = log_softmax(x)
    # exact ties inside rows and across rows
    if rng.random() < 0.6:
        pool = rng.choice(x.reshape(-1), size=8)
        mask = rng.random(x.shape) < 0.05
        x[mask] = rng.choice(pool, size=int(mask.sum()))
    if rng.random() < 0.3:
        x[..., int(rng.integers(0, V))] = x[..., 0]
    if rng.random() < 0.3:
        x[rng.random(x.shape) < 0.02] = -np.inf
    if rng.random() < 0.05:
        x[...] = -np.inf  # no finite entry anywhere
    invalid = False
    if allow_invalid and rng.random() < 0.15:
        bad = rng.random(x.shape) < 0.001
        x[bad] = np.nan if rng.random() < 0.5 else np.inf
        invalid = bool(bad.any())
    eos = int(rng.integers(-1, V)) if rng.random() < 0.7 else -1
    extra = [int(v) for v in rng.integers(0, V, size=int(rng.integers(0, 3)))] if eos >= 0 else []
    kw = dict(
        from_logits=from_logits,
        eos_token=eos,
        extra_eos=extra,
        min_length=int(rng.integers(0, 5)),
        alpha=float(rng.choice([0.0, 0.6, 1.0, 2.5])),
        no_repeat_ngram_size=int(rng.choice([0, 0, 0, 1, 2, 3])),
        repetition_penalty=float(rng.choice([1.0, 1.0, 1.2, 2.0])),
        steps=[int(s) for s in rng.integers(1, T + 1, size=B)] if rng.random() < 0.4 else None,
        banned=(rng.random(V) < 0.1).astype(np.uint8) if rng.random() < 0.3 else None,
        banned_per_example=(rng.random((B, V)) < 0.05).astype(np.uint8) if rng.random() < 0.2 else None,
    )
    return dict(seed=seed, B=B, T=T, K=K, V=V, dtype=dtype, x=x, xin=to_bits(x, dtype), kw=kw, invalid=invalid)


def load_golden() -> list[dict]:
    """The committed fixtures of tests/golden/cases.npz (reference outputs)."""
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cases.npz")
    z = np.load(path, allow_pickle=False)
    cases = []
    for n in range(int(z["n_cases"][0])):
        p = f"c{n}_"
        B, T, K, V, fl, eos, minlen, ngram, dt = (int(v) for v in z[p + "meta"])
        alpha, rep = (float(v) for v in z[p + "fmeta"])
        kw = dict(from_logits=bool(fl), eos_token=eos, extra_eos=[int(v) for v in z[p + "extra_eos"]],
                  min_length=minlen, alpha=alpha, no_repeat_ngram_size=ngram, repetition_penalty=rep,
                  steps=z[p + "steps"].tolist() if p + "steps" in z else None,
                  banned=z[p + "banned"] if p + "banned" in z else None,
                  banned_per_example=z[p + "banned_per_example"] if p + "banned_per_example" in z else None)
        out = {k[len(p) + 4:]: z[k] for k in z.files if k.startswith(p + "out_")}
        cases.append(dict(index=n, B=B, T=T, K=K, V=V, dtype=["f32", "f16", "bf16"][dt], xin=z[p + "x"], kw=kw,
                          out=out, grad_final=z[p + "grad_final"], grad_scores=z[p + "grad_scores"],
                          grad=z[p + "grad"]))
    return cases


TRACE_KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
              "raw_scores", "from_logprob", "row_lse", "invalid")


def first_difference(a: dict, b: dict, keys=TRACE_KEYS) -> str | None:
    """Name of the first field whose bits differ, or None."""
    for k in keys:
        x, y = np.asarray(a[k]), np.asarray(b[k])
        if x.shape != y.shape:
            return f"{k} (shape {x.shape} vs {y.shape})"
        if x.dtype.kind == "f":
            x, y = x.view(np.uint32 if x.itemsize == 4 else np.uint16), y.view(np.uint32 if y.itemsize == 4 else np.uint16)
        if not np.array_equal(x, y):
            idx = np.argwhere(x != y)[0]
            return f"{k} at {tuple(idx)}: {np.asarray(a[k])[tuple(idx)]} vs {np.asarray(b[k])[tuple(idx)]}"
    return None
