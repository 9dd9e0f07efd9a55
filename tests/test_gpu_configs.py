# SPDX-License-Identifier: MIT
"""The five BASELINE configurations at their full sizes on the GPU, checked
against the reference's own CPU library (oracle/_ref, where it is built; the
oracle otherwise) on identical seeded inputs: every trace field and the final
scores bit for bit, the logsumexp of every row (row_lse: the rows the search
read, 0 elsewhere), the backtracked sequences exactly, and for config 5 the
gradient of the minimum-risk loss w.r.t. the bf16 logits (bf16 bits equal to
the reference's float32 gradient rounded to bf16).

Size-independent properties are checked on the way: the traces are in the
candidate order, every final beam's path re-sums to its raw score, the rows
the search read carry their logsumexp and the others 0."""

import numpy as np
import pytest
import torch

import beamgrad_amd as bg
from bench import CONFIGS, workload
from oracle.oracle import Oracle, Reference, reference_available
from tests.cases import first_difference

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(1200)]

KEYS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores", "raw_scores",
        "from_logprob")


def _host(x: torch.Tensor) -> np.ndarray:
    x = x.detach()
    return x.cpu().numpy() if x.dtype == torch.float32 else x.view(torch.int16).cpu().numpy().view(np.uint16)


def _cpu_decode(name, wl, host):
    cfg = CONFIGS[name]
    kw = dict(dtype=cfg["dtype"], from_logits=cfg["from_logits"], eos_token=cfg["eos"], min_length=cfg["min_length"],
              alpha=cfg["alpha"], no_repeat_ngram_size=cfg.get("ngram", 0), repetition_penalty=cfg.get("rep", 1.0),
              steps=None if wl["steps"] is None else wl["steps"].cpu().numpy(), num_threads=16)
    if reference_available():
        ref = Reference()
        if wl["banned"] is not None:
            return ref.decode_per_example_banned(host, wl["banned"].cpu().numpy(), **kw), ref
        return ref.decode(host, **kw), ref
    orc = Oracle()
    bpe = None if wl["banned"] is None else wl["banned"].cpu().numpy()
    return orc.decode(host, banned_per_example=bpe, **kw), orc


def _gpu_row_lse(name, wl):
    """row_lse [B, T, K] of the config's decode on the GPU (the operator the
    Python API calls, which returns it as its tenth output)."""
    cfg = CONFIGS[name]
    out = torch.ops.beamgrad.decode_ex(wl["x"].detach(), cfg["from_logits"], wl["steps"], cfg["eos"],
                                       cfg["min_length"], cfg["alpha"], wl["banned"], cfg.get("ngram", 0),
                                       cfg.get("rep", 1.0), True, [])
    return out[9].cpu().numpy()


def _gpu_trace(out):
    got = {k: getattr(out, k).detach().cpu().numpy() for k in ("final_scores", "final_raw_scores", "scores",
                                                               "raw_scores")}
    for k in ("final_lengths", "tokens", "parents", "lengths"):
        got[k] = getattr(out, k).cpu().numpy().astype(np.int32)
    got["from_logprob"] = out.from_logprob.cpu().numpy().astype(np.uint8)
    return got


def _properties(got, want, seq, host, cfg):
    # rows read carry their logsumexp, the others 0 (from logits)
    B, T, K = got["tokens"].shape
    # order: per step, slots are sorted by (score desc, raw desc)
    s, r = got["scores"], got["raw_scores"]
    ok = (s[..., :-1] > s[..., 1:]) | ((s[..., :-1] == s[..., 1:]) & (r[..., :-1] >= r[..., 1:]))
    ok |= ~np.isfinite(s[..., 1:])
    assert ok.all()
    # each final beam's path re-sums to its raw score when every step was an expansion
    # (checked where the config reads log-probs, so the entries are the inputs themselves)
    if not cfg["from_logits"] and cfg.get("rep", 1.0) <= 1.0 and cfg["dtype"] == "f32":
        for b in range(min(B, 4)):
            for k in range(K):
                if not np.isfinite(got["final_raw_scores"][b, k]):
                    continue
                beam, raw = k, []
                for t in range(T - 1, -1, -1):
                    p = got["parents"][b, t, beam]
                    if got["from_logprob"][b, t, beam]:
                        raw.append((t, p, got["tokens"][b, t, beam]))
                    beam = p
                acc = np.float32(0.0)
                for t, p, v in reversed(raw):
                    acc = np.float32(acc + host[b, t, p, v])
                assert acc == got["final_raw_scores"][b, k]


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4"])
def test_config_decode_matches_reference(name):
    cfg = CONFIGS[name]
    wl = workload(name)
    opts = bg.BeamOptions(beam_size=cfg["K"], eos_token=cfg["eos"], min_length=cfg["min_length"],
                          length_penalty_alpha=cfg["alpha"], no_repeat_ngram_size=cfg.get("ngram", 0),
                          repetition_penalty=cfg.get("rep", 1.0))
    print(f"[config {name}] decode on the GPU", flush=True)
    out = bg.decode(wl["x"], opts, wl["steps"], from_logits=cfg["from_logits"], banned_mask=wl["banned"])
    seq = bg.backtrack(out).cpu().numpy()
    got = _gpu_trace(out)
    got["row_lse"] = _gpu_row_lse(name, wl)
    host = _host(wl["x"])
    print(f"[config {name}] CPU reference", flush=True)
    want, _ = _cpu_decode(name, wl, host)
    diff = first_difference(got, want, KEYS + ("row_lse",))
    assert diff is None, f"config {name}: {diff}"
    steps = None if wl["steps"] is None else wl["steps"].cpu().numpy()
    assert np.array_equal(seq, Oracle().backtrack(want["tokens"], want["parents"], steps))
    _properties(got, want, seq, host, cfg)
    del host


def test_config5_forward_backward_matches_reference():
    name = "c5"
    cfg = CONFIGS[name]
    wl = workload(name)
    x = wl["x"].requires_grad_(True)
    opts = bg.BeamOptions(beam_size=cfg["K"])
    print("[config c5] search + minimum_risk + backward on the GPU", flush=True)
    result = bg.search(x, opts, from_logits=True)
    loss = bg.losses.minimum_risk(result, wl["costs"])
    loss.backward()
    s = result.scores.detach().clone().requires_grad_(True)
    g_final = torch.autograd.grad(bg.losses.minimum_risk(result._replace(scores=s), wl["costs"]), s)[0]
    got = _gpu_trace(result.trace)
    got["final_scores"] = result.scores.detach().cpu().numpy()
    got["row_lse"] = _gpu_row_lse(name, wl)
    grad_got = x.grad.view(torch.int16).cpu().numpy()
    host = _host(x)
    print("[config c5] CPU reference decode", flush=True)
    want, impl = _cpu_decode(name, wl, host)
    diff = first_difference(got, want, KEYS + ("row_lse",))
    assert diff is None, f"config c5: {diff}"
    print("[config c5] CPU reference backward", flush=True)
    grad_want = impl.backward(want, cfg["V"], grad_final=g_final.cpu().numpy(), logits=host, logits_dtype="bf16",
                              row_lse=want["row_lse"], num_threads=16)
    want_bf16 = torch.from_numpy(grad_want).to(torch.bfloat16).view(torch.int16).numpy()
    del grad_want
    mism = np.count_nonzero(grad_got != want_bf16)
    assert mism == 0, f"config c5: {mism} gradient elements differ"
