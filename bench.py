# SPDX-License-Identifier: MIT
"""Benchmark of the beam-search hot path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input already
resident in HBM: for the headline workload (config C2) that is
``beamgrad_amd.decode(logits, from_logits=True)`` (final scores + trace) and
``backtrack`` on bf16 logits [B=32, T=64, K=8, V=151936] with EOS 151643,
length penalty 1.0 and min_length 4. ``value`` is candidate elements per
second over the timed steps (rows read by the search x V, the reference's
count). Beside it: the row pass's HBM roofline fraction (kernel time from the
engine's HIP events on its own stream), the reference CPU library on the same
batch (num_threads = 0, median of 5 runs), and under ``c5`` the second half
of the metric: the C5 forward + minimum-risk loss + backward step latency with
the forward's and the backward's (dense gradient's: the rows with a path
gradient, written into zeros the forward stores) roofline, and the
reference CPU library's decode + backward of the same batch fed the same
final-score gradient. Every roofline also states the box's measured device
copy bandwidth (``copy_gbs``) and the fraction of it reached.

    python bench.py [--steps K] [--warmup W] [--config c1..c5] [--no-cpu-baseline] [--no-c5]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak, GB/s
METRIC = "decode candidate elements/sec & % of HBM peak BW; fwd+bwd step latency (1 GPU)"

CONFIGS = {
    "c1": dict(B=8, T=32, K=4, V=32000, dtype="f32", from_logits=False, eos=2, alpha=0.6, min_length=0, seed=1001,
               desc="decode()+backtrack() fp32 log-probs [8,32,4,32000], eos 2, alpha 0.6"),
    "c2": dict(B=32, T=64, K=8, V=151936, dtype="bf16", from_logits=True, eos=151643, alpha=1.0, min_length=4,
               seed=1002, desc="from_logits bf16 [32,64,8,151936] N(0,3^2)+Zipf(1.1) bias, eos 151643, "
                               "length_penalty 1.0, min_length 4; final_scores+decode+backtrack"),
    "c3": dict(B=64, T=128, K=5, V=50257, dtype="f16", from_logits=False, eos=50256, alpha=0.0, min_length=8,
               seed=1003, ngram=3, rep=1.2,
               desc="constrained fp16 log-probs [64,128,5,50257], per-example 1% banned, no_repeat_ngram 3, "
                    "repetition_penalty 1.2, min_length 8, steps U[64,128], eos 50256; decode"),
    "c4": dict(B=16, T=64, K=64, V=32000, dtype="f32", from_logits=False, eos=2, alpha=0.6, min_length=0, seed=1004,
               desc="wide-beam fp32 log-probs [16,64,64,32000] with 5% exact ties, eos 2, alpha 0.6; decode"),
    "c5": dict(B=16, T=128, K=8, V=128256, dtype="bf16", from_logits=True, eos=-1, alpha=0.0, min_length=0,
               seed=1005, desc="from_logits bf16 [16,128,8,128256] N(0,3^2); search + minimum_risk(costs U(0,1)) "
                               "forward and backward into the logits"),
}


def workload(name: str) -> dict:
    """Seeded inputs of a config, generated on the GPU: the rows, and the
    per-example steps, banned mask and costs where the config has them."""
    cfg = CONFIGS[name]
    B, V = cfg["B"], cfg["V"]
    gen = torch.Generator(device="cuda").manual_seed(cfg["seed"] + 7)
    out = {"x": make_inputs(cfg), "steps": None, "banned": None, "costs": None}
    if name == "c3":
        out["steps"] = torch.randint(64, 129, (B,), generator=gen, device="cuda")
        banned = torch.zeros(B, V, dtype=torch.uint8, device="cuda")
        n_ban = V // 100
        for b in range(B):
            banned[b, torch.randperm(V, generator=gen, device="cuda")[:n_ban]] = 1
        out["banned"] = banned
    if name == "c5":
        out["costs"] = torch.rand(B, cfg["K"], generator=gen, device="cuda")
    return out


def make_inputs(cfg: dict) -> torch.Tensor:
    """Seeded synthetic rows generated on the GPU, one example at a time."""
    B, T, K, V = cfg["B"], cfg["T"], cfg["K"], cfg["V"]
    gen = torch.Generator(device="cuda").manual_seed(cfg["seed"])
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[cfg["dtype"]]
    x = torch.empty(B, T, K, V, dtype=tdt, device="cuda")
    if cfg is CONFIGS["c3"]:
        for b in range(B):
            x[b] = torch.log_softmax(torch.randn(T, K, V, generator=gen, device="cuda") * 2.5, dim=-1).to(tdt)
    elif cfg is CONFIGS["c5"]:
        for b in range(B):
            x[b] = (torch.randn(T, K, V, generator=gen, device="cuda") * 3.0).to(tdt)
    elif cfg is CONFIGS["c2"]:
        rank = torch.randperm(V, generator=gen, device="cuda").to(torch.float32) + 1.0
        bias = -1.1 * torch.log(rank)  # Zipf(s=1.1) bias shared across rows
        for b in range(B):
            x[b] = (torch.randn(T, K, V, generator=gen, device="cuda") * 3.0 + bias).to(tdt)
    elif cfg is CONFIGS["c4"]:
        for b in range(B):
            lp = torch.log_softmax(torch.randn(T, K, V, generator=gen, device="cuda") * 1.5, dim=-1)
            pool = lp.reshape(T, -1)[:, :64].clone()  # per-step pool of exact values
            tie = torch.rand(T, K, V, generator=gen, device="cuda") < 0.05
            pick = torch.randint(0, 64, (T, K, V), generator=gen, device="cuda")
            lp = torch.where(tie, torch.gather(pool, 1, pick.reshape(T, -1)).reshape(T, K, V), lp)
            x[b] = lp.to(tdt)
    else:
        for b in range(B):
            x[b] = torch.log_softmax(torch.randn(T, K, V, generator=gen, device="cuda") * 2.0, dim=-1).to(tdt)
    return x


def rows_read(out, eos_set: tuple[int, ...]) -> int:
    """Rows the reference reads: beam 0 at step 0, then every live beam that
    has not emitted EOS, for t < steps (decoder.cpp:127-131)."""
    raw = out.raw_scores  # [B, T, K]
    live = torch.isfinite(raw[:, :-1])
    if eos_set:
        finished = torch.isin(out.tokens[:, :-1], torch.tensor(eos_set, device=raw.device))
        live = live & ~finished
    return int(raw.shape[0] + live.sum().item())


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(name: str, wl: dict, rows_per_example: float, runs: int = 5) -> dict | None:
    """The reference's CPU library (oracle/_ref) or, without it, the oracle,
    on this host's cores over the same batch (C5: decode + backward with the
    same final-score gradient): num_threads = 0 (one thread per hardware
    thread), one warm-up, then the median of ``runs`` timed runs."""
    from oracle import oracle as orc

    cfg = CONFIGS[name]
    x = wl["x"].detach()
    host = x.cpu().numpy() if x.dtype == torch.float32 else x.view(torch.int16).cpu().numpy().view(np.uint16)
    kw = dict(dtype=cfg["dtype"], from_logits=cfg["from_logits"], eos_token=cfg["eos"], min_length=cfg["min_length"],
              alpha=cfg["alpha"], no_repeat_ngram_size=cfg.get("ngram", 0), repetition_penalty=cfg.get("rep", 1.0),
              steps=None if wl["steps"] is None else wl["steps"].cpu().numpy(), num_threads=0)
    if orc.reference_available():
        impl, kind = orc.Reference(), "reference"
        kernel_name = impl.kernel_name()
    else:
        impl, kind = orc.Oracle(), "port"
        kernel_name = None
    if wl["banned"] is not None:
        banned = wl["banned"].cpu().numpy()
        if kind == "reference":
            run = lambda: impl.decode_per_example_banned(host, banned, **kw)  # noqa: E731
        else:
            run = lambda: impl.decode(host, banned_per_example=banned, **kw)  # noqa: E731
        what = "per-example dbs_decode_batch_into_ex calls (one banned mask each)"
    elif wl["costs"] is not None:
        # the loss's gradient w.r.t. the final scores, as the GPU computed it
        g_final = np.ascontiguousarray(wl["g_final"].cpu().numpy(), np.float32)

        def run():
            tr = impl.decode(host, **kw)
            impl.backward(tr, cfg["V"], alpha=cfg["alpha"], grad_final=g_final, logits=host, logits_dtype=cfg["dtype"],
                          row_lse=tr["row_lse"], num_threads=0)
        what = "dbs_decode_batch_into_ex + dbs_backward_batch_into_ex"
    else:
        run = lambda: impl.decode(host, **kw)  # noqa: E731
        what = "dbs_decode_batch_into_ex"
    run()  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    cand = rows_per_example * cfg["B"] * cfg["V"]
    nproc = os.cpu_count() or 1
    return {"value": cand / med, "unit": "candidate elements/s", "cores": nproc, "kind": kind,
            "ms_per_step": med * 1e3, "num_threads": 0, "nproc": nproc,
            "cpu_affinity": len(os.sched_getaffinity(0)), "cpu_model": _cpu_model(),
            "dbs_selected_kernel_name": kernel_name,
            "sample": f"the whole batch ({cfg['B']} examples, T={cfg['T']}) through {what} with num_threads=0 "
                      f"(one thread per hardware thread), median of {runs} runs after a warm-up "
                      f"(runs: {', '.join(f'{1e3 * t:.1f}' for t in times)} ms)"}


def _read_kernels(lib, steps: int) -> tuple[dict, float]:
    """Per-kind kernel averages the engine timed with HIP events on its own
    streams (dbs_hip_profile_read), and rescanned rows per step."""
    import ctypes as C

    kernels = {}
    for kind, name in enumerate(("row_pass", "select", "path_walk", "dense_gradient", "backtrack")):
        ms, n = C.c_double(), C.c_int64()
        lib.dbs_hip_profile_read(kind, C.byref(ms), C.byref(n))
        if n.value:
            kernels[name] = {"avg_ms": ms.value / n.value, "launches": n.value}
    ms, n = C.c_double(), C.c_int64()
    lib.dbs_hip_profile_read(5, C.byref(ms), C.byref(n))
    return kernels, n.value / steps


def _traffic(config: str, kernel: str = "row_pass") -> float | None:
    """HBM bytes per launch of a kernel from the committed PMC summary."""
    tfile = os.path.join(ROOT, "profiles", f"{kernel}_{config}_traffic.txt")
    if not os.path.exists(tfile):
        return None
    for line in open(tfile):
        if line.startswith("traffic_bytes_per_launch"):
            return float(line.split("=")[1])
    return None


def measure(name: str, steps: int, warmup: int, copy_probe: bool = False) -> dict:
    """W untimed and K timed steps of one config on the current stream,
    bracketed by synchronisations; the engine's kernel timers run only over
    the timed steps."""
    import beamgrad_amd as bg
    from beamgrad_amd import _abi

    cfg = CONFIGS[name]
    B, T, K, V = cfg["B"], cfg["T"], cfg["K"], cfg["V"]
    wl = workload(name)
    x = wl["x"]
    opts = bg.BeamOptions(beam_size=K, eos_token=cfg["eos"], min_length=cfg["min_length"],
                          length_penalty_alpha=cfg["alpha"], no_repeat_ngram_size=cfg.get("ngram", 0),
                          repetition_penalty=cfg.get("rep", 1.0))
    torch.cuda.synchronize()

    if name == "c5":
        x.requires_grad_(True)

        def step():
            # forward + minimum-risk loss + backward into the logits
            x.grad = None
            result = bg.search(x, opts, from_logits=True)
            loss = bg.losses.minimum_risk(result, wl["costs"])
            loss.backward()
            return result.trace
    else:
        def step():
            out = bg.decode(x, opts, wl["steps"], from_logits=cfg["from_logits"], banned_mask=wl["banned"])
            bg.backtrack(out)
            return out

    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    n_rows = rows_read(out, opts.eos_tokens)
    if name == "c5":
        # grad_final of this batch (the CPU baseline's backward gets the same)
        result = bg.search(x.detach(), opts, from_logits=True)
        s = result.scores.detach().clone().requires_grad_(True)
        wl["g_final"] = torch.autograd.grad(bg.losses.minimum_risk(result._replace(scores=s), wl["costs"]), s)[0]

    if copy_probe:
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # the timed steps run uninstrumented; a second loop of as many steps
    # records each kernel's launches with HIP events (kernels_ms, roofline)
    lib = _abi.load()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        out = step()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    lib.dbs_hip_profile_enable(1)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kernels, rescans = _read_kernels(lib, steps)
    lib.dbs_hip_profile_enable(0)

    ms_per_step = start.elapsed_time(stop) / steps
    elem = 4 if cfg["dtype"] == "f32" else 2
    alg_bytes = n_rows * V * elem
    m = {"name": name, "cfg": cfg, "wl": wl, "out": out, "ms_per_step": ms_per_step, "kernels": kernels,
         "rows_read": n_rows, "alg_bytes": alg_bytes, "value": n_rows * V / (ms_per_step / 1e3),
         "rescans": rescans, "wall_s": wall}
    if name == "c5":
        m["rows_with_gradient"] = rows_with_gradient(out, V, cfg["alpha"])
    return m


def rows_with_gradient(trace, V: int, alpha: float) -> int:
    """R_g: the logits rows (b, t, parent) some final beam's path takes a
    token from, i.e. the rows whose softmax the backward reads."""
    ones = torch.ones(trace.final_scores.shape, dtype=torch.float32, device=trace.tokens.device)
    draws = torch.ops.beamgrad.final_scores_path_gradient(
        ones, trace.parents.int(), trace.tokens.int(), trace.lengths.int(), trace.from_logprob.to(torch.uint8), None,
        V, float(alpha))
    b, t, k = torch.nonzero(draws, as_tuple=True)
    parents = trace.parents[b, t, k]
    keys = (b * trace.parents.shape[1] + t) * trace.parents.shape[2] + parents
    return int(torch.unique(keys).numel())


_COPY_GBS: float | None = None


def copy_bandwidth(gib: int = 2, reps: int = 10) -> float:
    """The box's measured device copy bandwidth (GB/s, bytes read + bytes
    written): a device-to-device copy of ``gib`` GiB on the current stream,
    2 warm-ups, the median of ``reps`` HIP-event timings. Measured once per
    process."""
    global _COPY_GBS
    if _COPY_GBS is None:
        n = gib << 28  # float32 elements
        src = torch.empty(n, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        times = []
        for i in range(2 + reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            dst.copy_(src)
            b.record()
            b.synchronize()
            if i >= 2:
                times.append(a.elapsed_time(b))
        _COPY_GBS = 2 * 4 * n / (float(np.median(times)) / 1e3) / 1e9
        del src, dst
        torch.cuda.empty_cache()
    return _COPY_GBS


def hbm_roofline(bytes_per_launch: float, avg_ms: float, kernel: str, traffic=None) -> dict:
    achieved = bytes_per_launch / (avg_ms / 1e3) / 1e9
    copy_gbs = copy_bandwidth()
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic, "kernel": kernel, "algorithmic_bytes": bytes_per_launch, "copy_gbs": copy_gbs,
            "frac_of_copy": achieved / copy_gbs}


def c5_summary(m: dict) -> dict:
    """The fwd+bwd half of the metric on C5: step latency and the backward's
    (dense gradient's) roofline. The zeros of the bf16 gradient are stored by
    a fill the forward queues (while the host runs the loss and autograd);
    the dense gradient launch reads each logits row with a path gradient once
    and writes that row of the gradient once."""
    cfg = m["cfg"]
    V = cfg["V"]
    bwd_bytes = 2 * m["rows_with_gradient"] * V * 2
    out = {"workload": f"C5: {cfg['desc']}", "ms_per_step": m["ms_per_step"],
           "kernels_ms": {k: round(v["avg_ms"], 4) for k, v in m["kernels"].items()},
           "rows_read": m["rows_read"], "rows_with_gradient": m["rows_with_gradient"]}
    if "row_pass" in m["kernels"]:
        out["forward_roofline"] = hbm_roofline(m["alg_bytes"], m["kernels"]["row_pass"]["avg_ms"], "row_pass",
                                               _traffic("c5"))
    if "dense_gradient" in m["kernels"]:
        out["backward_roofline"] = hbm_roofline(bwd_bytes, m["kernels"]["dense_gradient"]["avg_ms"], "dense_gradient",
                                                _traffic("c5", "dense_gradient"))
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-c5", action="store_true", help="skip the C5 fwd+bwd fields of the default C2 line")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain device copy of 1 GiB (the PMC byte-counter calibration)")
    ap.add_argument("--serial", action="store_true",
                    help="run the select pass after the row pass, not beside it (for PMC counter passes, "
                         "which serialize kernels)")
    args = ap.parse_args()
    if args.serial:
        from beamgrad_amd import _abi
        _abi.load().dbs_hip_set_decode_overlap(0)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build's hot path runs on a single MI355X "
              "(examples are independent and would shard over GPUs with no exchange). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    m = measure(args.config, args.steps, args.warmup, args.copy_probe)
    cfg = m["cfg"]
    B, T, K, V = cfg["B"], cfg["T"], cfg["K"], cfg["V"]
    kernels = m["kernels"]
    ms_per_step = m["ms_per_step"]
    result = {
        "metric": METRIC,
        "value": m["value"],
        "unit": "candidate elements/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded, generated on the GPU)",
        "config": {"workload": f"{args.config.upper()}: {cfg['desc']}", "B": B, "T": T, "K": K, "V": V,
                   "from_logits": cfg["from_logits"], "rows_read_per_step": m["rows_read"],
                   "step_hbm_gbs": m["alg_bytes"] / (ms_per_step / 1e3) / 1e9,
                   "step_hbm_frac": m["alg_bytes"] / (ms_per_step / 1e3) / 1e9 / HBM_PEAK_GBS,
                   "kernels_ms": {k: round(v["avg_ms"], 4) for k, v in kernels.items()},
                   "rescanned_rows_per_step": m["rescans"],
                   "wall_s": round(m["wall_s"], 3)},
        "roofline": hbm_roofline(m["alg_bytes"], kernels["row_pass"]["avg_ms"], "row_pass", _traffic(args.config)),
        "cpu_baseline": None,
    }
    if args.config == "c5":
        result["c5"] = c5_summary(m)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.config, m["wl"], m["rows_read"] / B)
    if args.config == "c2" and not args.no_c5:
        del m
        torch.cuda.empty_cache()
        m5 = measure("c5", max(3, args.steps // 2), 2)
        result["c5"] = c5_summary(m5)
        if not args.no_cpu_baseline:
            result["c5"]["cpu_baseline"] = cpu_baseline("c5", m5["wl"], m5["rows_read"] / m5["cfg"]["B"])
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
