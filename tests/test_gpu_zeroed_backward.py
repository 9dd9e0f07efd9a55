# SPDX-License-Identifier: MIT
"""The rows' gradient written into zeros stored ahead.

The decode's autograd node stores the zeros of the rows' gradient right after
the forward, while the host runs the loss and autograd; its backward then
writes only the rows that receive an entry (beamgrad::decode_backward_into,
dbs_hip_backward_dense with DBS_HIP_GRAD_ZEROED). Checked here:

* the first backward of a graph (zeros stored ahead) equals, bit for bit, a
  second backward of the same graph (retain_graph; it writes the whole
  gradient) for logits in f32/f16/bf16 and log-probs, with per-example steps;
* decode_backward_into writes only rows that a selected slot descends from
  and leaves every other row as it was (a sentinel value there survives);
  the rows it skips are all zero in decode_backward_as's gradient, and the
  rows it writes equal that gradient's.

The whole gradient's parity with the oracle is pinned by the autograd tests
of the API (tests/test_gpu_api.py, tests/test_gpu_torch.py), which now take
this path."""

import pytest
import torch

import beamgrad_amd as bg

pytestmark = pytest.mark.gpu

_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _case(seed, dtype, from_logits, B=3, T=6, K=4, V=700):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, K, V, generator=g) * 3.0
    if not from_logits:
        x = x.log_softmax(-1)
    x = x.to(_DT[dtype]).cuda()
    steps = torch.randint(1, T + 1, (B,), generator=g)
    opts = bg.BeamOptions(beam_size=K, eos_token=int(torch.randint(0, V, (1,), generator=g)), min_length=1,
                          length_penalty_alpha=0.6)
    return x, steps, opts


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("dtype,from_logits", [("bf16", True), ("f16", True), ("f32", True), ("f32", False),
                                               ("bf16", False)])
def test_first_backward_equals_a_second_one(seed, dtype, from_logits):
    x, steps, opts = _case(9100 + seed, dtype, from_logits)
    x.requires_grad_(True)
    result = bg.search(x, opts, steps, from_logits=from_logits)
    costs = torch.rand(result.scores.shape, generator=torch.Generator().manual_seed(seed)).cuda()
    loss = bg.losses.minimum_risk(result, costs)
    (g1,) = torch.autograd.grad(loss, x, retain_graph=True)
    (g2,) = torch.autograd.grad(loss, x)
    assert g1.dtype == x.dtype and g1.shape == x.shape
    assert torch.equal(g1.view(torch.int16 if g1.element_size() == 2 else torch.int32),
                       g2.view(torch.int16 if g2.element_size() == 2 else torch.int32))
    assert g1.abs().sum() > 0


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_into_writes_only_the_rows_with_an_entry(seed, dtype):
    from beamgrad_amd._torch import _engine_decode

    x, steps, opts = _case(9200 + seed, dtype, True)
    B, T, K, V = x.shape
    out = _engine_decode(x, True, steps.cuda(), None, opts)
    parents, tokens, lengths, flp, row_lse = out[11], out[12], out[13], out[14], out[9]
    g = torch.randn(B, K, generator=torch.Generator().manual_seed(seed)).cuda()
    args = (g, None, None, None, parents, tokens, lengths, flp, steps.cuda(), V, 0.6, x, row_lse)
    full = torch.ops.beamgrad.decode_backward_as(*args, x.dtype)
    sentinel = torch.full_like(x, 7.0)
    torch.ops.beamgrad.decode_backward_into(*args, sentinel)
    torch.cuda.synchronize()
    written = (sentinel != 7.0).any(-1)  # rows the call wrote
    # a row with an entry is [b, t, q] with some slot k of step t whose parent is q
    has_entry = torch.zeros(B, T, K, dtype=torch.bool, device=x.device)
    for b in range(B):
        for t in range(int(steps[b])):
            for k in range(K):
                q = int(parents[b, t, k])
                if q >= 0:
                    has_entry[b, t, q] = True
    # written: only rows some slot descends from, and every row whose
    # gradient is not all zero, each exactly as the whole gradient has it
    assert not (written & ~has_entry).any()
    assert written.any()
    assert torch.equal(sentinel[written].float(), full[written].float())
    assert (sentinel[~written] == 7.0).all()
    assert (full[~written] == 0).all()
