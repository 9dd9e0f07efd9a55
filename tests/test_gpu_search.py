# SPDX-License-Identifier: MIT
"""beam_search with a model in the loop, on the HIP engine (one decode_step per
step). The reference's checks (python/tests/test_search.py:54-205) restated:
the stepped search equals the full decode of the rows it produced, which in
turn is compared bit for bit with the CPU oracle; gradients equal
final_scores's gradient of the stacked rows bit for bit."""

import numpy as np
import pytest
import torch
from torch import nn

import beamgrad_amd as bg

pytestmark = pytest.mark.gpu

DEV = "cuda"


class TinyLM(nn.Module):
    """A GRU language model on the GPU: each step's rows depend on the beams' prefixes."""

    def __init__(self, vocab: int = 13, hidden: int = 16, seed: int = 0):
        super().__init__()
        torch.manual_seed(seed)
        self.embed = nn.Embedding(vocab + 1, hidden)  # the last id is BOS
        self.gru = nn.GRUCell(hidden, hidden)
        self.out = nn.Linear(hidden, vocab)
        self.bos = vocab
        self.to(DEV)

    def step_fn(self):
        def step(beams: bg.BeamState) -> torch.Tensor:
            B, K, t = beams.sequences.shape
            w = self.out.weight
            h = torch.zeros(B * K, self.gru.hidden_size, dtype=w.dtype, device=w.device)
            tokens = beams.sequences.reshape(B * K, t).clamp(min=0).to(w.device)
            h = self.gru(self.embed(torch.full((B * K,), self.bos, device=w.device)), h)
            for i in range(t):
                h = self.gru(self.embed(tokens[:, i]), h)
            return self.out(h).log_softmax(-1).view(B, K, -1)

        return step


def _expected_paths(trace):
    paths = bg.backtrack(trace)
    positions = torch.arange(paths.shape[-1], device=paths.device)
    return torch.where(positions < trace.final_lengths[..., None], paths, -1)


OPTIONS = [
    bg.BeamOptions(beam_size=3),
    bg.BeamOptions(beam_size=4, eos_token=2, min_length=2, length_penalty_alpha=0.6),
    bg.BeamOptions(beam_size=3, eos_token=1, banned_tokens=[4, 5], no_repeat_ngram_size=2, repetition_penalty=1.5),
    bg.BeamOptions(beam_size=4, eos_token=(2, 7, 9), min_length=2, length_penalty_alpha=0.6),
]


@pytest.mark.parametrize("options", OPTIONS)
def test_matches_decode_of_its_rows_and_the_oracle(oracle, options):
    result = bg.beam_search(TinyLM().step_fn(), options, max_steps=6, batch_size=2)
    rows = torch.stack(result.step_log_probs, 1).detach()
    expected = bg.decode(rows, options)
    for name in ("tokens", "parents", "lengths", "scores", "raw_scores", "from_logprob"):
        assert torch.equal(getattr(result.trace, name), getattr(expected, name)), name
    assert torch.equal(result.scores.detach(), expected.final_scores)
    assert torch.equal(result.scores.detach(), bg.final_scores(rows, options))
    assert torch.equal(result.raw_scores, expected.final_raw_scores)
    assert torch.equal(result.lengths, expected.final_lengths)
    T = rows.shape[1]
    assert result.sequences.shape == (2, options.beam_size, 6)
    assert torch.equal(result.sequences[..., :T], _expected_paths(expected))
    assert bool((result.sequences[..., T:] == -1).all())

    eos, extra = options.native_eos()
    banned = None if options.banned_tokens is None else np.asarray(options.banned_mask(rows.shape[-1]), np.uint8)
    want = oracle.decode(rows.cpu().numpy(), dtype="f32", eos_token=eos, extra_eos=extra,
                         min_length=options.min_length, alpha=options.length_penalty_alpha,
                         no_repeat_ngram_size=options.no_repeat_ngram_size,
                         repetition_penalty=options.repetition_penalty, banned=banned)
    for name in ("tokens", "parents", "lengths", "from_logprob"):
        assert np.array_equal(getattr(result.trace, name).cpu().numpy().astype(want[name].dtype), want[name]), name
    for name in ("scores", "raw_scores"):
        assert np.array_equal(getattr(result.trace, name).cpu().numpy().view(np.uint32),
                              want[name].view(np.uint32)), name
    assert np.array_equal(result.scores.detach().cpu().numpy().view(np.uint32), want["final_scores"].view(np.uint32))


def test_step_function_sees_each_beams_prefix():
    model = TinyLM(seed=1)
    options = bg.BeamOptions(beam_size=3, eos_token=0, length_penalty_alpha=0.5)
    seen = []
    inner = model.step_fn()

    def step(beams):
        seen.append(beams)
        return inner(beams)

    result = bg.beam_search(step, options, max_steps=5, batch_size=2)
    trace = result.trace
    assert seen[0].step == 0 and seen[0].sequences.shape == (2, 3, 0)
    assert torch.equal(seen[0].active.cpu(), torch.tensor([[True, False, False]] * 2))
    for beams in seen[1:]:
        t = beams.step
        prefix = bg.decode(torch.stack(result.step_log_probs[:t], 1).detach(), options)
        assert torch.equal(beams.sequences, _expected_paths(prefix))
        assert torch.equal(beams.parents, trace.parents[:, t - 1])
        assert torch.equal(beams.tokens, trace.tokens[:, t - 1])
        assert torch.equal(beams.lengths, trace.lengths[:, t - 1])
        assert torch.equal(beams.scores, trace.scores[:, t - 1])


def test_gradients_reach_the_model():
    model = TinyLM(seed=2)
    options = bg.BeamOptions(beam_size=3, eos_token=3, length_penalty_alpha=0.7)
    weights = torch.tensor([[1.0, -0.5, 0.25]], device=DEV)
    result = bg.beam_search(model.step_fn(), options, max_steps=5)
    (result.scores * weights).sum().backward(retain_graph=True)
    got = [p.grad.clone() for p in model.parameters()]

    # the same loss written out: each final beam's path through the rows
    model.zero_grad()
    rows = torch.stack(result.step_log_probs, 1)
    trace = result.trace
    penalty = ((5.0 + trace.final_lengths.clamp(min=1).double()) / 6.0) ** 0.7
    parents, tokens, flp = (trace.parents.cpu(), trace.tokens.cpu(), trace.from_logprob.cpu())
    loss = rows.new_zeros(())
    for k in range(3):
        beam, total = k, rows.new_zeros(())
        for t in range(rows.shape[1] - 1, -1, -1):
            parent, token = int(parents[0, t, beam]), int(tokens[0, t, beam])
            if flp[0, t, beam]:
                total = total + rows[0, t, parent, token]
            beam = parent
        loss = loss + weights[0, k] * total / penalty[0, k].float()
    loss.backward()
    for g, p in zip(got, model.parameters(), strict=True):
        torch.testing.assert_close(g, p.grad, rtol=1e-5, atol=1e-6)
    assert any(g.abs().sum() > 0 for g in got)


def test_stops_once_every_beam_has_finished():
    options = bg.BeamOptions(beam_size=2, eos_token=0)
    calls = []

    def step(beams):
        calls.append(beams.step)
        lp = torch.full((1, 2, 5), -5.0, device=DEV)
        lp[..., 0] = -0.01  # EOS dominates
        return lp.log_softmax(-1)

    result = bg.beam_search(step, options, max_steps=10)
    assert len(result.step_log_probs) == len(calls) < 10
    assert result.sequences.shape == (1, 2, 10)
    assert bool(result.trace.lengths[:, -1].gt(0).all())
    assert torch.equal(result.scores, bg.final_scores(torch.stack(result.step_log_probs, 1), options))


def test_gradient_equals_final_scores_of_the_stacked_rows():
    model = TinyLM(seed=3)
    options = bg.BeamOptions(beam_size=4, eos_token=1, length_penalty_alpha=0.6, no_repeat_ngram_size=2)
    result = bg.beam_search(model.step_fn(), options, max_steps=6, batch_size=3)
    rows = result.step_log_probs
    weights = torch.randn(3, 4, generator=torch.Generator().manual_seed(0)).to(DEV)
    got = torch.autograd.grad((result.scores * weights).sum(), rows, retain_graph=True)
    expected = torch.autograd.grad((bg.final_scores(torch.stack(rows, 1), options) * weights).sum(), rows)
    for g, e in zip(got, expected, strict=True):
        assert torch.equal(g, e)


def test_no_grad_keeps_no_graph_and_no_rows():
    model = TinyLM(seed=4)
    with torch.no_grad():
        result = bg.beam_search(model.step_fn(), bg.BeamOptions(beam_size=3), max_steps=4, batch_size=2)
        kept = bg.beam_search(model.step_fn(), bg.BeamOptions(beam_size=3), max_steps=4, batch_size=2,
                              return_log_probs=True)
    assert not result.scores.requires_grad
    assert result.step_log_probs == ()
    assert torch.equal(result.scores, kept.scores)
    assert torch.equal(kept.scores, bg.final_scores(torch.stack(kept.step_log_probs, 1), bg.BeamOptions(beam_size=3)))


class TinyLMRescorer:
    """Teacher-forced token log-probabilities of TinyLM (a rescore_fn)."""

    def __init__(self, model):
        self.model = model

    def __call__(self, sequences, lengths):
        m = self.model
        B, K, T = sequences.shape
        tokens = sequences.reshape(B * K, T).clamp(min=0)
        h = torch.zeros(B * K, 16, dtype=m.out.weight.dtype, device=DEV)
        h = m.gru(m.embed(torch.full((B * K,), m.bos, device=DEV)), h)
        out = []
        for t in range(T):
            out.append(m.out(h).log_softmax(-1).gather(1, tokens[:, t:t + 1])[:, 0])
            h = m.gru(m.embed(tokens[:, t]), h)
        return torch.stack(out, 1).view(B, K, T)


@pytest.mark.parametrize("options", [bg.BeamOptions(beam_size=3),
                                     bg.BeamOptions(beam_size=4, eos_token=1, length_penalty_alpha=0.8)])
def test_rescoring_gives_the_same_gradient(options):
    model = TinyLM(seed=5).double()
    step = model.step_fn()
    through_steps = bg.beam_search(step, options, max_steps=6, batch_size=2)
    rescored = bg.beam_search(step, options, max_steps=6, batch_size=2, rescore_fn=TinyLMRescorer(model))
    assert rescored.step_log_probs == ()
    assert torch.equal(rescored.scores.detach(), through_steps.scores.detach())
    assert torch.equal(rescored.sequences, through_steps.sequences)
    weights = torch.linspace(-1.0, 1.0, options.beam_size, device=DEV).double()
    live = torch.isfinite(through_steps.scores)
    params = list(model.parameters())
    a = torch.autograd.grad((through_steps.scores[live] * weights.expand(2, -1)[live]).sum(), params)
    b = torch.autograd.grad((rescored.scores[live] * weights.expand(2, -1)[live]).sum(), params)
    # through the steps the engine computes each entry's gradient in float32
    for x, y in zip(a, b, strict=True):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6)


def test_rescore_fn_shape_is_checked():
    with pytest.raises(ValueError, match="rescore_fn"):
        bg.beam_search(TinyLM(seed=6).step_fn(), bg.BeamOptions(beam_size=2), max_steps=3,
                       rescore_fn=lambda s, n: torch.zeros(1, 2))


def test_vocabulary_change_between_steps_is_rejected():
    opts = bg.BeamOptions(beam_size=2)
    with pytest.raises(ValueError, match="vocabulary"):
        bg.beam_search(lambda beams: torch.zeros(1, 2, 4 + beams.step, device=DEV).log_softmax(-1), opts,
                       max_steps=3)


def test_bf16_rows_decode_as_their_float32_values():
    """16-bit rows go through decode_step as exact float32 conversions, and the
    gradient comes back in the rows' dtype."""
    g = torch.Generator(device=DEV).manual_seed(7)
    table = torch.randn(5, 2, 3, 11, generator=g, device=DEV).log_softmax(-1).bfloat16().requires_grad_()
    options = bg.BeamOptions(beam_size=3, eos_token=2, length_penalty_alpha=0.6)
    result = bg.beam_search(lambda beams: table[beams.step], options, max_steps=5, batch_size=2)
    rows = table.detach().float().transpose(0, 1)
    assert torch.equal(result.scores.detach(), bg.final_scores(rows.contiguous(), options))
    (grad,) = torch.autograd.grad(result.scores[:, 0].sum(), table)
    assert grad.dtype == torch.bfloat16
    ref = rows.clone().requires_grad_()
    (want,) = torch.autograd.grad(bg.final_scores(ref, options)[:, 0].sum(), ref)
    assert torch.equal(grad.float(), want.transpose(0, 1).bfloat16().float())
