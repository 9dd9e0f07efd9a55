# SPDX-License-Identifier: MIT
"""CPU-side behaviour of the Python front end: option validation (the
reference's rules, python/beamgrad/_options.py), the loud failure on CPU
tensors, and the operators' fake implementations (shapes and dtypes)."""

import numpy as np
import pytest
import torch

import beamgrad_amd as bg


def test_options_validation():
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=0)
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=True)
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=2, eos_token=-2)
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=2, length_penalty_alpha=-1.0)
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=2, length_penalty_alpha=float("inf"))
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=2, repetition_penalty=0.0)
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=2, banned_tokens=[-1])
    with pytest.raises(ValueError):
        bg.BeamOptions(beam_size=2, validate_inputs=1)
    o = bg.BeamOptions(beam_size=np.int64(3), eos_token=[5, 7, 5], banned_tokens=np.array([1, 2]))
    assert o.beam_size == 3 and o.eos_token == (5, 7) and o.banned_tokens == (1, 2)
    assert o.native_eos() == (5, [7])
    assert bg.BeamOptions(beam_size=2, eos_token=[4]).eos_token == 4
    with pytest.raises(ValueError):
        o.eos_ids(6)
    assert o.banned_mask(4) == [0, 1, 1, 0]


@pytest.mark.parametrize("kw, message", [
    (dict(beam_size=2**31), "beam_size must be a positive int (at most 2**31 - 1), got 2147483648"),
    (dict(beam_size=2.0), "beam_size must be a positive int (at most 2**31 - 1), got 2.0"),
    (dict(beam_size=2, eos_token=2**31), "eos_token must be -1 (disabled) or a token id, got 2147483648"),
    (dict(beam_size=2, eos_token="3"),
     "eos_token must be -1 (disabled), a token id or a sequence of token ids, got '3'"),
    (dict(beam_size=2, eos_token=[]), "eos_token must be a non-empty sequence of token ids, got []"),
    (dict(beam_size=2, eos_token=[1, -1]), "eos_token must be a non-empty sequence of token ids, got [1, -1]"),
    (dict(beam_size=2, min_length=-1), "min_length must be a non-negative int (at most 2**31 - 1), got -1"),
    (dict(beam_size=2, length_penalty_alpha=10**400),
     "length_penalty_alpha must be a finite, non-negative number, got " + repr(10**400)),
    (dict(beam_size=2, length_penalty_alpha=True),
     "length_penalty_alpha must be a finite, non-negative number, got True"),
    (dict(beam_size=2, validate_inputs=None), "validate_inputs must be a bool, got None"),
    (dict(beam_size=2, banned_tokens=5), "banned_tokens must be a sequence of token ids, got 5"),
    (dict(beam_size=2, banned_tokens=[1, 2.0]), "banned_tokens must hold non-negative int token ids, got (1, 2.0)"),
    (dict(beam_size=2, no_repeat_ngram_size=-3),
     "no_repeat_ngram_size must be a non-negative int (at most 2**31 - 1), got -3"),
    (dict(beam_size=2, repetition_penalty=float("nan")), "repetition_penalty must be a finite, positive number, got nan"),
    # the first bad field in field order is the one reported
    (dict(beam_size=0, min_length=-1), "beam_size must be a positive int"),
    (dict(beam_size=1, min_length=-1, repetition_penalty=0), "min_length must be a non-negative int"),
])
def test_options_error_messages(kw, message):
    with pytest.raises(ValueError) as err:
        bg.BeamOptions(**kw)
    assert str(err.value).startswith(message)


def test_options_normalized_values():
    o = bg.BeamOptions(beam_size=np.int32(4), eos_token=torch.tensor([9, 9]), min_length=np.int16(2),
                       length_penalty_alpha=np.float32(0.5), banned_tokens=[], no_repeat_ngram_size=np.uint8(3),
                       repetition_penalty=2)
    assert (o.beam_size, o.eos_token, o.min_length, o.banned_tokens, o.no_repeat_ngram_size) == (4, 9, 2, None, 3)
    assert all(type(v) is int for v in (o.beam_size, o.eos_token, o.min_length, o.no_repeat_ngram_size))
    assert type(o.length_penalty_alpha) is float and type(o.repetition_penalty) is float
    assert o.eos_tokens == (9,) and o.native_eos() == (9, [])
    off = bg.BeamOptions(beam_size=1)
    assert off.eos_tokens == () and off.native_eos() == (-1, []) and off.eos_ids(3) == ()
    assert off.banned_ids(3) is None and off.banned_mask(3) is None
    many = bg.BeamOptions(beam_size=1, eos_token=(3, 1, 3, 2), banned_tokens=(0, 4))
    assert many.eos_token == (3, 1, 2) and many.native_eos() == (3, [1, 2]) and many.eos_ids(4) == (3, 1, 2)
    with pytest.raises(ValueError, match=r"eos_token 3 is outside the vocabulary \(size 3\)"):
        many.eos_ids(3)
    with pytest.raises(ValueError, match=r"include ids outside the vocabulary \(size 4\)"):
        many.banned_ids(4)
    assert many.banned_ids(5) == (0, 4) and many.banned_mask(5) == [1, 0, 0, 0, 1]
    with pytest.raises(Exception):
        many.beam_size = 3  # frozen


def test_cpu_tensors_fail_loudly():
    opts = bg.BeamOptions(beam_size=2)
    with pytest.raises(RuntimeError, match="GPU"):
        bg.decode(torch.zeros(1, 3, 2, 5), opts)
    with pytest.raises(RuntimeError, match="GPU"):
        bg.final_scores(torch.zeros(3, 2, 5), opts)
    with pytest.raises(NotImplementedError):
        # no CPU kernel is registered for the operators
        torch.ops.beamgrad.decode_ex(torch.zeros(1, 3, 2, 5), False, None, -1, 0, 0.0, None, 0, 1.0, True, [])


def test_shape_checks():
    opts = bg.BeamOptions(beam_size=2)
    with pytest.raises(ValueError, match="beams"):
        bg.decode(torch.zeros(1, 3, 4, 5), opts)
    with pytest.raises(ValueError, match="shape"):
        bg.decode(torch.zeros(3, 5), opts)
    with pytest.raises(TypeError):
        bg.decode(torch.zeros(1, 3, 2, 5, dtype=torch.int32), opts)


def test_fake_implementations_give_shapes():
    x = torch.empty(2, 3, 4, 7, device="meta", dtype=torch.bfloat16)
    out = torch.ops.beamgrad.decode_ex(x, True, None, -1, 0, 0.0, None, 0, 1.0, True, [])
    assert [tuple(t.shape) for t in out] == [(2, 4), (2, 4), (2, 4)] + [(2, 3, 4)] * 7
    assert out[0].dtype == torch.float32 and out[3].dtype == torch.int32 and out[8].dtype == torch.uint8
    p = torch.empty(2, 3, 4, device="meta", dtype=torch.int32)
    g = torch.ops.beamgrad.decode_backward_as(None, None, None, None, p, p, p, p.to(torch.uint8), None, 7, 0.0, None,
                                              None, torch.bfloat16)
    assert g.shape == (2, 3, 4, 7) and g.dtype == torch.bfloat16
    seq = torch.ops.beamgrad.backtrack(p, p, None)
    assert seq.shape == (2, 4, 3) and seq.dtype == torch.int64


def test_beam_search_argument_errors():
    """beam_search's checks that run before any step reaches the engine
    (reference python/tests/test_search.py:223-238)."""
    opts = bg.BeamOptions(beam_size=2)
    good = lambda beams: torch.zeros(1, 2, 4).log_softmax(-1)  # noqa: E731
    with pytest.raises(TypeError):
        bg.beam_search(good, object(), max_steps=2)
    with pytest.raises(ValueError, match="max_steps"):
        bg.beam_search(good, opts, max_steps=0)
    with pytest.raises(ValueError, match="max_steps"):
        bg.beam_search(good, opts, max_steps=True)
    with pytest.raises(ValueError, match="batch_size"):
        bg.beam_search(good, opts, max_steps=2, batch_size=2**32 + 1)
    with pytest.raises(ValueError, match=r"\[B, K, V\]"):
        bg.beam_search(lambda beams: torch.zeros(1, 3, 4), opts, max_steps=2)
    with pytest.raises(TypeError):
        bg.beam_search(lambda beams: torch.zeros(1, 2, 4, dtype=torch.long), opts, max_steps=2)
    with pytest.raises(ValueError, match="outside the vocabulary"):
        bg.beam_search(good, bg.BeamOptions(beam_size=2, eos_token=4), max_steps=2)
    # the product has no CPU engine: host rows are refused before any decode
    with pytest.raises(ValueError, match="GPU"):
        bg.beam_search(good, opts, max_steps=2)
    with pytest.raises(ValueError, match="rescore_fn|GPU"):
        bg.beam_search(good, opts, max_steps=2, rescore_fn=lambda s, n: torch.zeros(1, 2))


def test_beam_search_state_on_a_fixed_device_checks_the_rows_device():
    opts = bg.BeamOptions(beam_size=2)
    with pytest.raises(ValueError, match="beam state is on meta"):
        bg.beam_search(lambda beams: torch.zeros(1, 2, 4).log_softmax(-1), opts, max_steps=2, device="meta")


def test_sequence_scores_rejects_lengths_outside_the_sequences():
    lp = torch.zeros(2, 3)
    with pytest.raises(ValueError, match=r"lengths must be in \[0, 3\]"):
        bg.sequence_scores(lp, torch.tensor([1, 4]), bg.BeamOptions(beam_size=1))
    with pytest.raises(ValueError, match="shape"):
        bg.sequence_scores(lp, torch.tensor([1]), bg.BeamOptions(beam_size=1))


def test_fake_and_meta_tensors_trace_without_the_engine():
    """Shape-only tensors go through the operators' fake implementations
    (reference python/tests/test_api.py:446-454), so torch.compile and export
    can trace the API without a GPU."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        out = bg.decode(torch.empty(3, 5, 4, 17), bg.BeamOptions(beam_size=4))
        assert out.final_scores.shape == (3, 4)
        assert out.tokens.shape == (3, 5, 4) and out.tokens.dtype == torch.int64
        assert out.from_logprob.dtype == torch.bool
        scores = bg.final_scores(torch.empty(2, 3, 4, 9, dtype=torch.bfloat16), bg.BeamOptions(beam_size=4),
                                 from_logits=True)
        assert scores.shape == (2, 4) and scores.dtype == torch.float32
    meta = bg.decode(torch.empty(2, 6, 3, 11, device="meta"), bg.BeamOptions(beam_size=3))
    assert meta.parents.shape == (2, 6, 3) and meta.parents.device.type == "meta"


def test_batching_rules_are_registered():
    import torch._C as C

    for op in ("decode", "decode_ex", "decode_backward", "decode_backward_as", "final_scores_backward",
               "final_scores_path_gradient", "length_penalty", "backtrack"):
        assert C._dispatch_has_kernel_for_dispatch_key(f"beamgrad::{op}", "FuncTorchBatched"), op


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("temperature", [1.0, 0.25, 3.0])
def test_minimum_risk_closed_form(reduction, temperature):
    """minimum_risk and its gradient against the closed form in float64
    (reference python/beamgrad/losses.py:139-169 defines the objective):
    risk_b = sum_k p_k c_k with p = softmax(s_b / t) over live beams, and
    d risk_b / d s_k = p_k (c_k - risk_b) / t; dead beams (-inf) get no
    probability and their costs (even NaN) are never read; an example with
    no live beam has risk 0 and no gradient."""
    from collections import namedtuple

    rng = np.random.default_rng(17)
    B, K = 6, 5
    s = rng.normal(0.0, 2.0, (B, K))
    s[1, [0, 3]] = -np.inf
    s[4, :] = -np.inf
    c = rng.random((B, K))
    c[1, 3] = np.nan
    c[4, :] = np.nan
    want_risk = np.zeros(B)
    want_grad = np.zeros((B, K))
    for b in range(B):
        live = np.isfinite(s[b])
        if not live.any():
            continue
        z = s[b, live] / temperature
        p = np.exp(z - z.max())
        p /= p.sum()
        want_risk[b] = (p * c[b, live]).sum()
        want_grad[b, live] = p * (c[b, live] - want_risk[b]) / temperature
    scale = {"mean": 1.0 / B, "sum": 1.0, "none": 1.0}[reduction]
    R = namedtuple("R", "scores")
    st = torch.tensor(s, requires_grad=True)
    loss = bg.losses.minimum_risk(R(st), torch.tensor(c), temperature, reduction)
    want_loss = {"mean": want_risk.mean(), "sum": want_risk.sum(), "none": want_risk}[reduction]
    np.testing.assert_allclose(loss.detach().numpy(), want_loss, rtol=1e-12, atol=1e-15)
    loss.sum().backward()
    np.testing.assert_allclose(st.grad.numpy(), want_grad * scale, rtol=1e-10, atol=1e-15)


def test_minimum_risk_errors():
    from collections import namedtuple

    R = namedtuple("R", "scores")
    s = torch.zeros(2, 3)
    with pytest.raises(ValueError, match="temperature must be positive, got 0"):
        bg.losses.minimum_risk(R(s), torch.zeros(2, 3), 0)
    with pytest.raises(ValueError, match=r"costs must have the scores' shape \(2, 3\), got \(3, 2\)"):
        bg.losses.minimum_risk(R(s), torch.zeros(3, 2), reduction="bad")
    with pytest.raises(ValueError, match="reduction must be 'mean', 'sum' or 'none', got 'bad'"):
        bg.losses.minimum_risk(R(s), torch.zeros(2, 3), reduction="bad")
    assert bg.losses.minimum_risk(R(torch.zeros(3)), torch.zeros(1, 3), reduction="none").shape == (1,)
