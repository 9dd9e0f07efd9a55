# SPDX-License-Identifier: MIT
"""torch integration of the HIP operators: torch.compile(fullgraph), vmap
batching rules and torch.func transforms, restating the reference's checks
(python/tests/test_api.py:457-517). Every result is compared bit for bit with
the eager, batched call (the engine is deterministic)."""

import pytest
import torch

import beamgrad_amd as bg

pytestmark = pytest.mark.gpu

DEV = "cuda"


def random_log_probs(*shape, seed, dtype=torch.float32, logits=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * 2.0
    x = x if logits else x.log_softmax(-1)
    return x.to(dtype).to(DEV)


def test_compile_fullgraph_forward_and_backward():
    options = bg.BeamOptions(beam_size=3, eos_token=2, length_penalty_alpha=0.6)
    weights = torch.tensor([1.0, -0.5, 0.25], device=DEV)

    def loss(x):
        return (bg.final_scores(x, options) * weights).sum()

    compiled = torch.compile(loss, fullgraph=True, backend="aot_eager")
    x = random_log_probs(2, 6, 3, 11, seed=13)
    a = x.clone().requires_grad_(True)
    b = x.clone().requires_grad_(True)
    loss(a).backward()
    compiled(b).backward()
    assert torch.equal(a.grad, b.grad)


def test_compile_fullgraph_decode_and_search():
    options = bg.BeamOptions(beam_size=3, eos_token=2, length_penalty_alpha=0.6)
    x = random_log_probs(2, 6, 3, 11, seed=14)
    trace = torch.compile(lambda y: bg.decode(y, options), fullgraph=True, backend="aot_eager")(x)
    expected = bg.decode(x, options)
    for name in expected._fields:
        assert torch.equal(getattr(trace, name), getattr(expected, name)), name
    result = torch.compile(lambda y: bg.search(y, options), fullgraph=True, backend="aot_eager")(x)
    reference = bg.search(x, options)
    assert torch.equal(result.scores, reference.scores) and torch.equal(result.sequences, reference.sequences)


def test_compile_fullgraph_from_logits_bf16():
    options = bg.BeamOptions(beam_size=4, eos_token=1, min_length=2, length_penalty_alpha=1.0)
    x = random_log_probs(3, 5, 4, 64, seed=15, dtype=torch.bfloat16, logits=True)

    def loss(y):
        return bg.final_scores(y, options, from_logits=True)[:, 0].sum()

    a = x.clone().requires_grad_(True)
    b = x.clone().requires_grad_(True)
    loss(a).backward()
    torch.compile(loss, fullgraph=True, backend="aot_eager")(b).backward()
    assert a.grad.dtype == torch.bfloat16 and torch.equal(a.grad, b.grad)


def test_vmap_matches_a_batched_call():
    options = bg.BeamOptions(beam_size=2, eos_token=1)
    x = random_log_probs(4, 3, 5, 2, 9, seed=17)  # [N, B, T, K, V]
    expected = bg.final_scores(x.reshape(12, 5, 2, 9), options).reshape(4, 3, 2)
    assert torch.equal(torch.vmap(lambda y: bg.final_scores(y, options))(x), expected)
    unbatched = torch.vmap(lambda y: bg.final_scores(y, options))(x[:, 0])
    assert torch.equal(unbatched, expected[:, 0])


def test_vmap_of_decode_and_backtrack():
    options = bg.BeamOptions(beam_size=3, eos_token=2, length_penalty_alpha=0.6)
    x = random_log_probs(2, 3, 6, 3, 10, seed=18)
    traces = torch.vmap(lambda y: tuple(bg.decode(y, options)))(x)
    paths = torch.vmap(lambda y: bg.backtrack(bg.decode(y, options)))(x)
    flat = bg.decode(x.reshape(6, 6, 3, 10), options)
    for name, got in zip(flat._fields, traces, strict=True):
        want = getattr(flat, name)
        assert torch.equal(got, want.reshape(2, 3, *want.shape[1:])), name
    assert torch.equal(paths, bg.backtrack(flat).reshape(2, 3, 3, 6))


def test_torch_func_transforms():
    options = bg.BeamOptions(beam_size=3, eos_token=2, length_penalty_alpha=0.6)
    x = random_log_probs(2, 5, 3, 13, seed=19)
    weights = torch.tensor([1.0, -0.5, 0.25], device=DEV)
    reference = x.clone().requires_grad_(True)
    (bg.final_scores(reference, options) * weights).sum().backward()

    assert torch.equal(torch.func.grad(lambda y: (bg.final_scores(y, options) * weights).sum())(x), reference.grad)
    _, vjp = torch.func.vjp(lambda y: bg.final_scores(y, options), x)
    assert torch.equal(vjp(weights.expand(2, 3))[0], reference.grad)
    jacobian = torch.func.jacrev(lambda y: bg.final_scores(y, options))(x[0])
    assert jacobian.shape == (3, 5, 3, 13)
    combined = (weights.view(3, 1, 1, 1) * jacobian).sum(0)
    torch.testing.assert_close(combined, reference.grad[0])


def test_per_example_gradients_with_vmap_of_grad():
    options = bg.BeamOptions(beam_size=3, eos_token=2)
    x = random_log_probs(4, 6, 3, 11, seed=23)
    reference = x.clone().requires_grad_(True)
    bg.final_scores(reference, options).sum().backward()
    per_example = torch.vmap(torch.func.grad(lambda y: bg.final_scores(y, options).sum()))(x)
    assert torch.equal(per_example, reference.grad)


def test_per_example_logits_gradients_with_vmap_of_grad():
    options = bg.BeamOptions(beam_size=2, eos_token=3, length_penalty_alpha=0.6)
    x = random_log_probs(3, 4, 2, 40, seed=24, dtype=torch.bfloat16, logits=True)
    reference = x.clone().requires_grad_(True)
    bg.final_scores(reference, options, from_logits=True).sum().backward()
    per_example = torch.vmap(torch.func.grad(lambda y: bg.final_scores(y, options, from_logits=True).sum()))(x)
    assert per_example.dtype == torch.bfloat16 and torch.equal(per_example, reference.grad)


def test_vmap_over_banned_masks_is_per_example_banning():
    """A banned mask that varies over the vmapped dimension folds into the
    engine's per-example masks (an addition: the reference refuses it)."""
    options = bg.BeamOptions(beam_size=3, eos_token=2)
    x = random_log_probs(2, 3, 4, 3, 12, seed=25)  # [N, B, T, K, V]
    masks = torch.zeros(2, 12, dtype=torch.uint8, device=DEV)
    masks[0, [0, 5, 7]] = 1
    masks[1, [1, 2, 9]] = 1
    got = torch.vmap(lambda y, m: bg.final_scores(y, options, banned_mask=m))(x, masks)
    for n in range(2):
        want = bg.final_scores(x[n], options, banned_mask=masks[n])
        assert torch.equal(got[n], want)
    per_example = torch.zeros(2, 3, 12, dtype=torch.uint8, device=DEV)
    per_example[:, 1, 4] = 1
    got = torch.vmap(lambda y, m: bg.final_scores(y, options, banned_mask=m))(x, per_example)
    for n in range(2):
        assert torch.equal(got[n], bg.final_scores(x[n], options, banned_mask=per_example[n]))


def test_length_penalty_batching_rule():
    lengths = torch.tensor([[0, 1, 7], [3, 4, 5]], device=DEV)
    got = torch.vmap(lambda n: bg.length_penalty(n, 0.6))(lengths)
    assert torch.equal(got, bg.length_penalty(lengths, 0.6))
