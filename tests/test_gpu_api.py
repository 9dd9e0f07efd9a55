# SPDX-License-Identifier: MIT
"""GPU tests of the Python API and the torch.ops.beamgrad operators on the
HIP engine, against the CPU oracle (bit for bit) and the reference's API
semantics (python/tests/test_api.py, test_cuda.py, test_training.py)."""

import numpy as np
import pytest
import torch

import beamgrad_amd as bg
from tests.cases import first_difference, make_case, to_bits

pytestmark = pytest.mark.gpu


def _tensor(case):
    xin = case["xin"]
    if case["dtype"] == "f32":
        return torch.from_numpy(xin).cuda()
    t = torch.from_numpy(xin.view(np.int16)).cuda()
    return t.view(torch.bfloat16 if case["dtype"] == "bf16" else torch.float16)


def _options(kw, K):
    eos = kw["eos_token"]
    if eos >= 0 and kw["extra_eos"]:
        eos = [eos] + [t for t in kw["extra_eos"]]
    return bg.BeamOptions(beam_size=K, eos_token=eos, min_length=kw["min_length"],
                          length_penalty_alpha=kw["alpha"], validate_inputs=False,
                          banned_tokens=None if kw["banned"] is None else np.nonzero(kw["banned"])[0].tolist(),
                          no_repeat_ngram_size=kw["no_repeat_ngram_size"],
                          repetition_penalty=kw["repetition_penalty"])


def _oracle_kw(kw):
    # BeamOptions keeps EOS tokens distinct in the order given; the engine and
    # the oracle sort them, so the same set results
    return dict(kw)


@pytest.mark.parametrize("seed", range(0, 24))
def test_decode_api_matches_oracle(oracle, seed):
    case = make_case(9000 + seed, allow_invalid=False)
    kw = case["kw"]
    opts = _options(kw, case["K"])
    x = _tensor(case)
    out = bg.decode(x, opts, kw["steps"], from_logits=kw["from_logits"], banned_mask=None if kw[
        "banned_per_example"] is None else torch.from_numpy(kw["banned_per_example"]))
    want = oracle.decode(case["xin"], dtype=case["dtype"], **_oracle_kw(kw))
    got = {k: getattr(out, k).cpu().numpy() for k in ("final_scores", "final_raw_scores", "scores", "raw_scores")}
    for k in ("final_lengths", "tokens", "parents", "lengths"):
        got[k] = getattr(out, k).cpu().numpy().astype(np.int32)
    got["from_logprob"] = out.from_logprob.cpu().numpy().astype(np.uint8)
    assert first_difference(got, want, tuple(got)) is None
    seq = bg.backtrack(out).cpu().numpy()
    assert np.array_equal(seq, oracle.backtrack(want["tokens"], want["parents"], kw["steps"]))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("from_logits", [False, True])
def test_final_scores_gradient_matches_oracle(oracle, dtype, from_logits):
    rng = np.random.default_rng(11)
    B, T, K, V = 3, 7, 4, 300
    xf = rng.normal(0, 2, size=(B, T, K, V)).astype(np.float32)
    case = dict(dtype=dtype, xin=to_bits(xf, dtype))
    x = _tensor(case).requires_grad_(True)
    opts = bg.BeamOptions(beam_size=K, eos_token=3, min_length=2, length_penalty_alpha=0.6)
    scores = bg.final_scores(x, opts, from_logits=from_logits)
    w = torch.from_numpy(rng.normal(size=(B, K)).astype(np.float32)).cuda()
    (scores * w).sum().backward()
    tr = oracle.decode(case["xin"], dtype=dtype, from_logits=from_logits, eos_token=3, min_length=2, alpha=0.6)
    assert np.array_equal(scores.detach().cpu().numpy().view(np.uint32), tr["final_scores"].view(np.uint32))
    want = oracle.backward(tr, V, alpha=0.6, grad_final=w.cpu().numpy(), logits=case["xin"] if from_logits else None,
                           logits_dtype=dtype, row_lse=tr["row_lse"] if from_logits else None)
    assert x.grad.dtype == x.dtype
    if dtype == "f32":
        assert np.array_equal(x.grad.cpu().numpy().view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(x.grad.view(torch.int16).cpu().numpy().view(np.uint16), to_bits(want, dtype))


def test_search_minimum_risk_gradient(oracle):
    """Config 5's path at a small size: search from bf16 logits, minimum-risk
    loss, backward into the logits; the loss gradient w.r.t. the scores has the
    closed form p_k (c_k - sum_j p_j c_j) / B (reference python/tests/test_training.py:116-128)."""
    rng = np.random.default_rng(5)
    B, T, K, V = 4, 9, 8, 500
    xf = rng.normal(0, 3, size=(B, T, K, V)).astype(np.float32)
    bits = to_bits(xf, "bf16")
    x = torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16).requires_grad_(True)
    opts = bg.BeamOptions(beam_size=K)
    result = bg.search(x, opts, from_logits=True)
    costs = torch.from_numpy(rng.random((B, K)).astype(np.float32)).cuda()
    loss = bg.losses.minimum_risk(result, costs)
    loss.backward()
    s = result.scores.detach().double()
    p = torch.softmax(s, -1)
    c = costs.double()
    g_closed = p * (c - (p * c).sum(-1, keepdim=True)) / B
    s32 = result.scores.detach().clone().requires_grad_(True)
    g_final = torch.autograd.grad(bg.losses.minimum_risk(result._replace(scores=s32), costs), s32)[0]
    assert torch.allclose(g_final.double(), g_closed, rtol=1e-5, atol=1e-7)
    tr = oracle.decode(bits, dtype="bf16", from_logits=True)
    want = oracle.backward(tr, V, grad_final=g_final.cpu().numpy(), logits=bits, logits_dtype="bf16",
                           row_lse=tr["row_lse"])
    assert np.array_equal(x.grad.view(torch.int16).cpu().numpy().view(np.uint16), to_bits(want, "bf16"))
    # sequences: the backtracked paths, -1 past each beam's length
    seq = result.sequences.cpu().numpy()
    paths = oracle.backtrack(tr["tokens"], tr["parents"])
    lens = tr["final_lengths"]
    assert np.array_equal(seq, np.where(np.arange(T) < lens[..., None], paths, -1))


def test_validation_raises_on_nan():
    x = torch.full((2, 3, 2, 10), -1.0, device="cuda")
    x[1, 1, 0, 4] = float("nan")
    with pytest.raises(ValueError, match="example 1"):
        bg.decode(x, bg.BeamOptions(beam_size=2))
    out = bg.decode(x, bg.BeamOptions(beam_size=2, validate_inputs=False))
    assert torch.isfinite(out.final_scores).all()


def test_steps_out_of_range_raise():
    x = torch.full((2, 3, 2, 10), -1.0, device="cuda")
    with pytest.raises(ValueError, match="steps"):
        bg.decode(x, bg.BeamOptions(beam_size=2), steps=[1, 4])


def test_length_penalty_op(oracle):
    lengths = torch.arange(-2, 300, device="cuda")
    got = bg.length_penalty(lengths, 0.6).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.length_penalty(np.arange(-2, 300), 0.6).view(np.uint32))


def _step_through(x, opts):
    """Runs decode_step over the T steps of x [B, T, K, V] from the initial
    state, keeping the prefix matrix as the reference's beam_search does."""
    B, T, K, V = x.shape
    raw = torch.full((B, K), float("-inf"), device="cuda")
    raw[:, 0] = 0
    lengths = torch.zeros(B, K, dtype=torch.int32, device="cuda")
    finished = torch.zeros(B, K, dtype=torch.uint8, device="cuda")
    prefixes = torch.full((B, K, T), -1, dtype=torch.int32, device="cuda")
    eos, extra = opts.native_eos()
    toks, pars, scores = [], [], []
    for t in range(T):
        out = torch.ops.beamgrad.decode_step(
            x[:, t].contiguous(), raw, lengths, finished, prefixes,
            eos, opts.min_length, opts.length_penalty_alpha, None, opts.no_repeat_ngram_size,
            opts.repetition_penalty, False, extra)
        tok, par, lengths, sc, raw, flp, finished, final = out
        toks.append(tok)
        pars.append(par)
        scores.append(sc)
        # new prefixes: the parent's row plus the token when it was expanded
        pidx = par.clamp(min=0).long()
        newp = torch.gather(prefixes, 1, pidx[..., None].expand(B, K, T))
        pos = (lengths - 1).clamp(min=0).long()
        put = (flp > 0) & (par >= 0)
        newp.scatter_(2, pos[..., None], torch.where(put, tok, newp.gather(2, pos[..., None])[..., 0])[..., None])
        prefixes = torch.where((par >= 0)[..., None], newp, torch.full_like(newp, -1))
    return torch.stack(toks, 1), torch.stack(pars, 1), torch.stack(scores, 1), final, raw, lengths


@pytest.mark.parametrize("constrained", [False, True])
@pytest.mark.parametrize("seed", range(0, 4))
def test_step_api_equals_decode(oracle, seed, constrained):
    rng = np.random.default_rng(seed)
    B, T, K, V = 3, 8, 4, 60
    x = torch.from_numpy(np.log(rng.dirichlet(np.ones(V) * 0.3, size=(B, T, K))).astype(np.float32)).cuda()
    opts = bg.BeamOptions(beam_size=K, eos_token=[5, 9], min_length=3, length_penalty_alpha=0.6,
                          no_repeat_ngram_size=2 if constrained else 0,
                          repetition_penalty=1.5 if constrained else 1.0)
    toks, pars, scores, final, raw, lengths = _step_through(x, opts)
    want = bg.decode(x, opts)
    assert torch.equal(toks, want.tokens.int()) and torch.equal(pars, want.parents.int())
    assert torch.equal(scores, want.scores)
    assert torch.equal(final, want.final_scores) and torch.equal(raw, want.final_raw_scores)
    assert torch.equal(lengths, want.final_lengths.int())


@pytest.mark.parametrize("K", [1, 8, 300])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_minimum_risk_kernel_closed_form(K, reduction):
    """The GPU loss (one HIP launch, beamgrad::minimum_risk) against the
    closed form in float64: risk_b = sum_k p_k c_k over the live beams with
    p = softmax(s / t), gradient p_k (c_k - risk_b) / t (times 1 / B for the
    mean); dead beams (-inf) get no probability and their costs (NaN here)
    are not read; an example without a live beam has risk 0. K = 300 takes
    more beams than the kernel has threads."""
    from collections import namedtuple

    rng = np.random.default_rng(K)
    B, t = 5, 0.7
    s = rng.normal(0, 3, (B, K))
    dead = rng.random((B, K)) < 0.2
    dead[3, :] = True
    s[dead] = -np.inf
    c = rng.random((B, K))
    c[dead] = np.nan
    want_risk = np.zeros(B)
    want_grad = np.zeros((B, K))
    for b in range(B):
        live = ~dead[b]
        if not live.any():
            continue
        z = s[b, live] / t
        p = np.exp(z - z.max())
        p /= p.sum()
        want_risk[b] = (p * c[b, live]).sum()
        want_grad[b, live] = p * (c[b, live] - want_risk[b]) / t
    scale = 1.0 / B if reduction == "mean" else 1.0
    R = namedtuple("R", "scores")
    st = torch.tensor(s, dtype=torch.float32, device="cuda", requires_grad=True)
    loss = bg.losses.minimum_risk(R(st), torch.tensor(c, dtype=torch.float32, device="cuda"), t, reduction)
    want_loss = {"mean": want_risk.mean(), "sum": want_risk.sum(), "none": want_risk}[reduction]
    np.testing.assert_allclose(loss.detach().double().cpu().numpy(), want_loss, rtol=2e-6, atol=1e-7)
    loss.sum().backward()
    np.testing.assert_allclose(st.grad.double().cpu().numpy(), want_grad * scale, rtol=2e-5, atol=1e-7)
    assert torch.isfinite(st.grad).all()


def test_minimum_risk_paths_agree():
    """The one-workgroup kernel (B <= 1024, K <= 64; the reduction fused)
    and the per-example kernel (larger batches; the reduction a second
    launch) give each example the same risk and gradient factor, bit for
    bit; the fused mean and sum add the risks in index order; the vmap rule
    gives each slice the unbatched call's bits."""
    from beamgrad_amd import _torch  # noqa: F401  (registers the operators)

    rng = np.random.default_rng(11)
    B, K = 1100, 8
    s = rng.normal(0, 3, (B, K)).astype(np.float32)
    s[rng.random((B, K)) < 0.1] = -np.inf
    c = rng.random((B, K)).astype(np.float32)
    st, ct = torch.tensor(s, device="cuda"), torch.tensor(c, device="cuda")
    risk_big, f_big = torch.ops.beamgrad.minimum_risk(st, ct, 0.8, 0)
    risk_small, f_small = torch.ops.beamgrad.minimum_risk(st[:1000].contiguous(), ct[:1000].contiguous(), 0.8, 0)
    assert torch.equal(risk_big[:1000], risk_small) and torch.equal(f_big[:1000], f_small)
    total, f_sum = torch.ops.beamgrad.minimum_risk(st[:1000].contiguous(), ct[:1000].contiguous(), 0.8, 2)
    assert torch.equal(f_sum, f_small)
    acc = np.float32(0.0)
    for v in risk_small.cpu().numpy():
        acc = np.float32(acc + v)
    assert total.item() == acc
    mean, f_mean = torch.ops.beamgrad.minimum_risk(st[:1000].contiguous(), ct[:1000].contiguous(), 0.8, 1)
    assert mean.item() == np.float32(acc / np.float32(1000))
    sl = st[:12].reshape(3, 4, K).contiguous()
    cl = ct[:12].reshape(3, 4, K).contiguous()
    got = torch.func.vmap(lambda a, b: torch.ops.beamgrad.minimum_risk(a, b, 0.8, 1))(sl, cl)
    for i in range(3):
        want = torch.ops.beamgrad.minimum_risk(sl[i], cl[i], 0.8, 1)
        assert torch.equal(got[0][i], want[0]) and torch.equal(got[1][i], want[1])


def test_decode_trace_engine_outputs():
    """decode_trace's widened trace and its engine trace (outputs 11-14, what
    the backward reads) against decode_ex's own outputs, bit for bit."""
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.normal(0, 2, (3, 6, 4, 257)).astype(np.float32)).cuda()
    args = (x, True, None, 5, 1, 0.6, None, 0, 1.0, True, [])
    ex = torch.ops.beamgrad.decode_ex(*args)
    tr = torch.ops.beamgrad.decode_trace(*args)
    for i in (0, 1, 6, 7, 9):
        assert torch.equal(ex[i].view(torch.int32), tr[i].view(torch.int32)), i
    for i, j in ((2, 2), (3, 3), (4, 4), (5, 5)):
        assert torch.equal(ex[i].long(), tr[j]), i
    assert torch.equal(ex[8].bool(), tr[8])
    assert torch.equal(tr[10], torch.full((3,), 6, dtype=torch.long, device="cuda"))
    for i, j in ((4, 11), (3, 12), (5, 13), (8, 14)):
        assert tr[j].dtype == ex[i].dtype and torch.equal(ex[i], tr[j]), j
