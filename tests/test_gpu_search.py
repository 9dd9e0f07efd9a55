# SPDX-License-Identifier: MIT
"""beam_search with a model in the loop (one decode_step per step) and
search over precomputed rows, on the HIP engine.

The model here (``DecayBagLM``) turns a beam's prefix into the next token's
log-probabilities through an exponentially decayed bag of its token
embeddings, so every step's rows depend on which prefixes survived. Its
teacher-forced scorer computes every position at once from a cumulative
decayed sum, a different computation from the step-by-step one.

Properties pinned (the ones the reference's own search tests pin,
python/tests/test_search.py): the stepped search selects what the full decode
of its stacked rows selects, and that decode matches the CPU oracle bit for
bit; every step sees each beam's true prefix; the sequences are the parent
walk of the trace (walked here on the CPU); the gradient equals
final_scores's gradient of the stacked rows bit for bit, reaches the model's
parameters as the hand-written path loss does, and equals the re-scoring
gradient up to float32 rounding; the loop stops once every beam has
finished; no graph and no rows are kept under no_grad; bfloat16 rows decode
as their float32 values with the gradient in bfloat16."""

import numpy as np
import pytest
import torch
from torch import nn

import beamgrad_amd as bg

pytestmark = pytest.mark.gpu

DEV = "cuda"


class DecayBagLM(nn.Module):
    """log_softmax(W_out tanh(W_in s + b)), s = sum over the prefix of
    decay^(age) * E[token] (age 0 for the last token; s = E[BOS] when empty)."""

    def __init__(self, vocab: int = 12, width: int = 10, decay: float = 0.7, seed: int = 0,
                 dtype=torch.float32):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.vocab, self.decay = vocab, decay
        self.embed = nn.Parameter(torch.randn(vocab + 1, width, generator=gen, dtype=dtype))  # row vocab: BOS
        self.w_in = nn.Parameter(torch.randn(width, width, generator=gen, dtype=dtype) / width ** 0.5)
        self.b_in = nn.Parameter(torch.randn(width, generator=gen, dtype=dtype) * 0.1)
        self.w_out = nn.Parameter(torch.randn(vocab, width, generator=gen, dtype=dtype))
        self.to(DEV)

    def _logp(self, bag: torch.Tensor) -> torch.Tensor:
        h = torch.tanh(bag @ self.w_in.T + self.b_in)
        return (h @ self.w_out.T).log_softmax(-1)

    def step(self, beams: bg.BeamState) -> torch.Tensor:
        B, K, t = beams.sequences.shape
        bag = self.embed[self.vocab].expand(B, K, -1)
        if t:
            ages = torch.arange(t - 1, -1, -1, device=DEV, dtype=self.embed.dtype)
            weights = self.decay ** ages  # [t]
            tokens = beams.sequences.clamp(min=0).to(DEV)
            bag = (self.embed[tokens] * weights[:, None]).sum(2)
        return self._logp(bag)

    def teacher_forced(self, sequences: torch.Tensor, lengths: torch.Tensor) -> torch.Tensor:
        """[B, K, T] log-probability of token t given tokens before it, all
        positions from one cumulative sum."""
        B, K, T = sequences.shape
        tokens = sequences.clamp(min=0)
        emb = self.embed[tokens]  # [B, K, T, W]
        # bag before position t: sum_{i < t} decay^(t-1-i) E[i], by a
        # lower-triangular matrix of decay powers
        i = torch.arange(T, device=DEV)
        powers = (i[:, None] - 1 - i[None, :]).clamp(min=0).to(self.embed.dtype)
        zero = torch.zeros((), dtype=self.embed.dtype, device=DEV)
        mix = torch.where(i[None, :] < i[:, None], self.decay ** powers, zero)  # [T, T]
        bags = torch.matmul(mix, emb)  # [B, K, T, W]
        bags[:, :, 0] = self.embed[self.vocab]
        return self._logp(bags).gather(-1, tokens[..., None])[..., 0]


def _walked_paths(trace: bg.BeamSearchOutput) -> torch.Tensor:
    """[B, K, T] tokens of each final beam by walking parents on the CPU (-1
    where no token was emitted and past the beam's length)."""
    tokens, parents, flp = (trace.tokens.cpu().numpy(), trace.parents.cpu().numpy(),
                            trace.from_logprob.cpu().numpy())
    lengths = trace.final_lengths.cpu().numpy()
    B, T, K = tokens.shape
    out = np.full((B, K, T), -1, np.int64)
    for b in range(B):
        for k in range(K):
            beam, emitted = k, []
            for t in range(T - 1, -1, -1):
                if beam < 0:
                    break
                if flp[b, t, beam]:
                    emitted.append(int(tokens[b, t, beam]))
                beam = int(parents[b, t, beam])
            emitted.reverse()
            n = min(len(emitted), int(lengths[b, k]))
            out[b, k, :n] = emitted[:n]
    return torch.from_numpy(out)


CASES = [
    bg.BeamOptions(beam_size=3),
    bg.BeamOptions(beam_size=4, eos_token=2, min_length=2, length_penalty_alpha=0.6),
    bg.BeamOptions(beam_size=3, eos_token=1, banned_tokens=[4, 5], no_repeat_ngram_size=2, repetition_penalty=1.5),
    bg.BeamOptions(beam_size=4, eos_token=(2, 7, 9), min_length=2, length_penalty_alpha=0.6),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_stepped_search_is_the_decode_of_its_rows(oracle, case):
    options = CASES[case]
    model = DecayBagLM(seed=case)
    result = bg.beam_search(model.step, options, max_steps=6, batch_size=2)
    rows = torch.stack(result.step_log_probs, 1).detach()
    T = rows.shape[1]
    eos, extra = options.native_eos()
    banned = None if options.banned_tokens is None else np.asarray(options.banned_mask(rows.shape[-1]), np.uint8)
    want = oracle.decode(rows.cpu().numpy(), dtype="f32", eos_token=eos, extra_eos=extra,
                         min_length=options.min_length, alpha=options.length_penalty_alpha,
                         no_repeat_ngram_size=options.no_repeat_ngram_size,
                         repetition_penalty=options.repetition_penalty, banned=banned)
    for name in ("tokens", "parents", "lengths", "from_logprob"):
        got = getattr(result.trace, name).cpu().numpy()
        assert np.array_equal(got.astype(want[name].dtype), want[name]), name
    for name in ("scores", "raw_scores"):
        got = getattr(result.trace, name).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want[name].view(np.uint32)), name
    assert np.array_equal(result.scores.detach().cpu().numpy().view(np.uint32), want["final_scores"].view(np.uint32))
    assert np.array_equal(result.raw_scores.cpu().numpy().view(np.uint32), want["final_raw_scores"].view(np.uint32))
    assert np.array_equal(result.lengths.cpu().numpy(), want["final_lengths"].astype(np.int64))
    # the decode of the stacked rows is the same search
    assert torch.equal(result.scores.detach(), bg.final_scores(rows, options))
    assert result.sequences.shape == (2, options.beam_size, 6)
    assert torch.equal(result.sequences[..., :T].cpu(), _walked_paths(result.trace))
    assert bool(result.sequences[..., T:].eq(-1).all())


def test_each_step_sees_the_beams_prefixes():
    model = DecayBagLM(seed=11)
    options = bg.BeamOptions(beam_size=3, eos_token=0, length_penalty_alpha=0.5)
    seen: list[bg.BeamState] = []

    def step(beams):
        seen.append(beams)
        return model.step(beams)

    result = bg.beam_search(step, options, max_steps=5, batch_size=2)
    trace = result.trace
    first = seen[0]
    assert first.step == 0 and tuple(first.sequences.shape) == (2, 3, 0)
    assert first.active.cpu().tolist() == [[True, False, False]] * 2
    assert bool(first.parents.eq(-1).all()) and bool(first.tokens.eq(-1).all())
    for beams in seen[1:]:
        t = beams.step
        head = bg.decode(torch.stack(result.step_log_probs[:t], 1).detach(), options)
        assert torch.equal(beams.sequences.cpu(), _walked_paths(head))
        for name in ("parents", "tokens", "lengths", "scores"):
            assert torch.equal(getattr(beams, name), getattr(trace, name)[:, t - 1]), name
        live = torch.isfinite(beams.scores) & ~beams.finished
        assert torch.equal(beams.active, live)


def test_stacked_rows_gradient_is_bit_exact():
    model = DecayBagLM(seed=12)
    options = bg.BeamOptions(beam_size=4, eos_token=1, length_penalty_alpha=0.6, no_repeat_ngram_size=2)
    result = bg.beam_search(model.step, options, max_steps=6, batch_size=3)
    rows = result.step_log_probs
    w = torch.linspace(-2.0, 1.5, 12, device=DEV).view(3, 4)
    got = torch.autograd.grad((result.scores * w).sum(), rows, retain_graph=True)
    want = torch.autograd.grad((bg.final_scores(torch.stack(rows, 1), options) * w).sum(), rows)
    for g, e in zip(got, want, strict=True):
        assert torch.equal(g, e)


def test_gradient_reaches_the_model_as_the_path_loss_does():
    model = DecayBagLM(seed=13)
    options = bg.BeamOptions(beam_size=3, eos_token=3, length_penalty_alpha=0.7)
    w = torch.tensor([[0.5, -1.0, 2.0]], device=DEV)
    result = bg.beam_search(model.step, options, max_steps=5)
    got = torch.autograd.grad((result.scores * w).sum(), list(model.parameters()), retain_graph=True)

    # the same loss spelled out: sum over each final beam's emitted entries
    rows = torch.stack(result.step_log_probs, 1)
    trace = result.trace
    parents, tokens, flp = (trace.parents[0].cpu(), trace.tokens[0].cpu(), trace.from_logprob[0].cpu())
    penalty = bg.length_penalty(trace.final_lengths, 0.7)
    loss = rows.new_zeros(())
    for k in range(3):
        beam, path = k, rows.new_zeros(())
        for t in reversed(range(rows.shape[1])):
            parent = int(parents[t, beam])
            if flp[t, beam]:
                path = path + rows[0, t, parent, int(tokens[t, beam])]
            beam = parent
        loss = loss + w[0, k] * path / penalty[0, k]
    want = torch.autograd.grad(loss, list(model.parameters()))
    for g, e in zip(got, want, strict=True):
        torch.testing.assert_close(g, e, rtol=1e-5, atol=1e-6)
    assert any(bool(g.ne(0).any()) for g in got)


def test_loop_ends_once_every_beam_has_finished():
    options = bg.BeamOptions(beam_size=2, eos_token=0)
    steps_called = []

    def step(beams):
        steps_called.append(beams.step)
        rows = torch.full((1, 2, 6), -4.0, device=DEV)
        rows[..., 0] = 0.0  # EOS is by far the likeliest
        return rows.log_softmax(-1)

    result = bg.beam_search(step, options, max_steps=9)
    assert steps_called == list(range(len(steps_called))) and len(steps_called) < 9
    assert len(result.step_log_probs) == len(steps_called)
    assert tuple(result.sequences.shape) == (1, 2, 9)
    # every final beam ended with the EOS token
    ends = result.sequences.gather(2, (result.lengths - 1).clamp(min=0)[..., None])[..., 0]
    assert bool(result.lengths.gt(0).all()) and bool(ends.eq(0).all())
    assert torch.equal(result.scores, bg.final_scores(torch.stack(result.step_log_probs, 1), options))


def test_no_grad_keeps_neither_graph_nor_rows():
    model = DecayBagLM(seed=14)
    options = bg.BeamOptions(beam_size=3)
    with torch.no_grad():
        plain = bg.beam_search(model.step, options, max_steps=4, batch_size=2)
        kept = bg.beam_search(model.step, options, max_steps=4, batch_size=2, return_log_probs=True)
    assert not plain.scores.requires_grad and plain.step_log_probs == ()
    assert len(kept.step_log_probs) == kept.trace.tokens.shape[1]
    assert torch.equal(plain.scores, kept.scores)
    assert torch.equal(kept.scores, bg.final_scores(torch.stack(kept.step_log_probs, 1), options))


@pytest.mark.parametrize("options", [bg.BeamOptions(beam_size=3),
                                     bg.BeamOptions(beam_size=4, eos_token=1, length_penalty_alpha=0.8)])
def test_rescoring_gradient_matches_the_stepped_one(options):
    model = DecayBagLM(seed=15, dtype=torch.float64)
    stepped = bg.beam_search(model.step, options, max_steps=6, batch_size=2)
    rescored = bg.beam_search(model.step, options, max_steps=6, batch_size=2, rescore_fn=model.teacher_forced)
    assert rescored.step_log_probs == ()
    assert torch.equal(rescored.scores.detach(), stepped.scores.detach())
    assert torch.equal(rescored.sequences, stepped.sequences)
    live = torch.isfinite(stepped.scores)
    w = torch.linspace(-1.0, 1.0, options.beam_size, device=DEV, dtype=torch.float64).expand(2, -1)
    params = list(model.parameters())
    a = torch.autograd.grad((stepped.scores[live] * w[live]).sum(), params)
    b = torch.autograd.grad((rescored.scores[live] * w[live]).sum(), params)
    # through the steps each entry's gradient is formed in float32
    for x, y in zip(a, b, strict=True):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6)


def test_rescore_fn_result_shape_is_checked():
    model = DecayBagLM(seed=16)
    with pytest.raises(ValueError, match=r"rescore_fn must return \[B, K, T\]"):
        bg.beam_search(model.step, bg.BeamOptions(beam_size=2), max_steps=3, rescore_fn=lambda s, n: s.float()[:, :1])
    with pytest.raises(ValueError, match="got list"):
        bg.beam_search(model.step, bg.BeamOptions(beam_size=2), max_steps=3, rescore_fn=lambda s, n: [])


def test_rows_must_keep_their_vocabulary():
    def growing(beams):
        return torch.zeros(1, 2, 5 + beams.step, device=DEV).log_softmax(-1)

    with pytest.raises(ValueError, match="vocabulary entries at step 1"):
        bg.beam_search(growing, bg.BeamOptions(beam_size=2), max_steps=3)


def test_bfloat16_rows_decode_as_float32_with_bfloat16_gradient():
    gen = torch.Generator(device=DEV).manual_seed(17)
    table = torch.randn(5, 2, 3, 11, generator=gen, device=DEV).log_softmax(-1).bfloat16().requires_grad_()
    options = bg.BeamOptions(beam_size=3, eos_token=2, length_penalty_alpha=0.6)
    result = bg.beam_search(lambda beams: table[beams.step], options, max_steps=5, batch_size=2)
    rows = table.detach().float().transpose(0, 1).contiguous()
    assert torch.equal(result.scores.detach(), bg.final_scores(rows, options))
    (grad,) = torch.autograd.grad(result.scores[:, 0].sum(), table)
    assert grad.dtype == torch.bfloat16
    ref = rows.clone().requires_grad_()
    (want,) = torch.autograd.grad(bg.final_scores(ref, options)[:, 0].sum(), ref)
    assert torch.equal(grad.float(), want.transpose(0, 1).bfloat16().float())


def test_search_over_precomputed_rows(oracle):
    """search(): one decode; sequences are the parent walk; unbatched input
    gives unbatched results; the step rows are views of the input."""
    gen = torch.Generator(device=DEV).manual_seed(18)
    x = torch.randn(2, 5, 3, 9, generator=gen, device=DEV).log_softmax(-1).requires_grad_()
    options = bg.BeamOptions(beam_size=3, eos_token=4, min_length=2, length_penalty_alpha=0.5)
    res = bg.search(x, options)
    full = bg.decode(x.detach(), options)
    assert torch.equal(res.scores.detach(), full.final_scores)
    assert torch.equal(res.sequences.cpu(), _walked_paths(full))
    assert all(r.data_ptr() == x[:, t].data_ptr() for t, r in enumerate(res.step_log_probs))
    (g,) = torch.autograd.grad(res.scores.sum() + res.raw_scores.sum(), x)
    assert g.shape == x.shape and bool(g.ne(0).any())
    one = bg.search(x[1].detach(), options)
    assert torch.equal(one.scores, res.scores[1].detach()) and torch.equal(one.sequences, res.sequences[1])
    assert one.trace.tokens.shape == (5, 3) and len(one.step_log_probs) == 5
    logits = bg.search(x.detach() * 3.0, options, from_logits=True)
    assert logits.step_log_probs == ()
