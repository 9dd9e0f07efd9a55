# SPDX-License-Identifier: MIT
"""Writes tests/golden/cases.npz: small decode and backward cases with the
outputs of the reference's own CPU library (oracle/_ref/libdbs_ref.so, built
from /root/reference by oracle/Makefile) through its public C ABI
(dbs_decode_batch_into_ex / dbs_backward_batch_into_ex).

The fixtures pin the oracle (tests/test_oracle.py) and the HIP engine
(tests/test_gpu_golden.py) on machines where the reference is absent.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.oracle import Reference  # noqa: E402
from tests.cases import make_case  # noqa: E402

DECODE_KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
               "raw_scores", "from_logprob", "row_lse")
N_CASES = 40


def main() -> None:
    ref = Reference()
    store: dict[str, np.ndarray] = {}
    n = 0
    seed = 90000
    while n < N_CASES:
        case = make_case(seed, allow_invalid=False)
        seed += 1
        if case["B"] * case["T"] * case["K"] * case["V"] > 20000:
            continue  # keep the fixture file small
        kw = dict(case["kw"])
        bpe = kw.pop("banned_per_example")
        common = dict(dtype=case["dtype"], **kw)
        if bpe is not None:
            banned = kw["banned"]
            merged = bpe if banned is None else (bpe | banned[None, :])
            common.pop("banned")
            out = ref.decode_per_example_banned(case["xin"], merged, **common)
        else:
            out = ref.decode(case["xin"], **common)
        p = f"c{n}_"
        store[p + "x"] = case["xin"]
        store[p + "meta"] = np.array([case["B"], case["T"], case["K"], case["V"], int(kw["from_logits"]),
                                      kw["eos_token"], kw["min_length"], kw["no_repeat_ngram_size"],
                                      ["f32", "f16", "bf16"].index(case["dtype"])], np.int64)
        store[p + "fmeta"] = np.array([kw["alpha"], kw["repetition_penalty"]], np.float32)
        store[p + "extra_eos"] = np.array(kw["extra_eos"], np.int32)
        if kw["steps"] is not None:
            store[p + "steps"] = np.array(kw["steps"], np.int32)
        if kw["banned"] is not None:
            store[p + "banned"] = kw["banned"]
        if bpe is not None:
            store[p + "banned_per_example"] = bpe
        for k in DECODE_KEYS:
            store[p + "out_" + k] = out[k]
        # backward of the final and per-step scores through the reference
        rng = np.random.default_rng(seed)
        gf = rng.normal(size=(case["B"], case["K"])).astype(np.float32)
        gs = rng.normal(size=(case["B"], case["T"], case["K"])).astype(np.float32)
        store[p + "grad_final"] = gf
        store[p + "grad_scores"] = gs
        logits = case["xin"] if kw["from_logits"] else None
        grad = ref.backward(out, case["V"], alpha=kw["alpha"], steps=kw["steps"], grad_final=gf, grad_scores=gs,
                            logits=logits, logits_dtype=case["dtype"],
                            row_lse=out["row_lse"] if kw["from_logits"] else None)
        store[p + "grad"] = grad
        n += 1
    store["n_cases"] = np.array([n])
    np.savez_compressed(os.path.join(HERE, "cases.npz"), **store)
    print(f"wrote {n} cases to tests/golden/cases.npz")


if __name__ == "__main__":
    main()
