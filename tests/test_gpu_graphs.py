# SPDX-License-Identifier: MIT
"""decode and final_scores captured in a HIP graph and replayed (reference
docs/cuda.md:253-257: with validate_inputs=False and no per-example steps the
operators read nothing back, so they can be captured).

Each replay runs on new inputs copied into the captured input tensor, with
eager decodes and host synchronisations between the replays, and every
replay's outputs are compared with the CPU oracle bit for bit (not only with
the eager results). The 16-bit case takes the persistent row pass, whose
overlapped select pass the engine turns off under capture."""

import numpy as np
import pytest
import torch

import beamgrad_amd as bg
from tests.cases import TRACE_KEYS, first_difference, log_softmax, to_bits

pytestmark = pytest.mark.gpu

_TORCH = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
_KEYS = tuple(k for k in TRACE_KEYS if k not in ("row_lse", "invalid"))


def _inputs(seed, shape, dtype, logits):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, size=shape).astype(np.float32)
    if not logits:
        x = log_softmax(x)
    x[rng.random(shape) < 0.01] = -np.inf
    xin = to_bits(x, dtype)
    t = torch.from_numpy(xin.view(np.int16) if xin.dtype == np.uint16 else xin).cuda()
    return xin, (t.view(_TORCH[dtype]) if dtype != "f32" else t)


def _as_numpy(out: bg.BeamSearchOutput) -> dict:
    return {k: getattr(out, k).cpu().numpy() for k in _KEYS}


@pytest.mark.parametrize("dtype, V, logits", [("bf16", 4096, True), ("f16", 1000, False), ("f32", 300, False)])
def test_captured_decode_and_final_scores_replay(oracle, dtype, V, logits):
    B, T, K = 3, 5, 4
    opts = bg.BeamOptions(beam_size=K, eos_token=3, min_length=2, length_penalty_alpha=0.6, validate_inputs=False)
    oracle_kw = dict(dtype=dtype, from_logits=logits, eos_token=3, min_length=2, alpha=0.6)
    _, first = _inputs(0, (B, T, K, V), dtype, logits)
    static_x = first.clone()

    side = torch.cuda.Stream()  # capture (and its warm-up) off the default stream
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            bg.decode(static_x, opts, from_logits=logits)
            bg.final_scores(static_x, opts, from_logits=logits)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = bg.decode(static_x, opts, from_logits=logits)
        captured_scores = bg.final_scores(static_x, opts, from_logits=logits)

    for seed in range(1, 6):
        xin, xt = _inputs(seed, (B, T, K, V), dtype, logits)
        static_x.copy_(xt)
        graph.replay()
        torch.cuda.synchronize()
        want = oracle.decode(xin, **oracle_kw)
        got = _as_numpy(captured)
        diff = first_difference(got, want, keys=_KEYS)
        assert diff is None, f"replay {seed}: {diff}"
        assert np.array_equal(captured_scores.cpu().numpy().view(np.uint32), want["final_scores"].view(np.uint32))
        # eager work between replays, on the same input
        eager = bg.decode(static_x, opts, from_logits=logits)
        assert first_difference(_as_numpy(eager), want, keys=_KEYS) is None
        torch.cuda.synchronize()
