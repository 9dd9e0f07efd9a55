# SPDX-License-Identifier: MIT
"""Calls libdbs_hip through its C ABI (beamgrad_amd._abi) with device memory
from torch, on torch's current HIP stream, and returns numpy results."""

from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from beamgrad_amd import _abi


def _dev(a: np.ndarray | None, dtype=None) -> torch.Tensor | None:
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


class HipEngine:
    def __init__(self):
        self.lib = _abi.load()
        assert self.lib.dbs_cuda_available() == 1

    def stream(self) -> C.c_void_p:
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)

    # ------------------------------------------------------------------
    def decode(self, xin: np.ndarray, dtype: str, *, from_logits=False, eos_token=-1, extra_eos=(), min_length=0,
               alpha=0.0, no_repeat_ngram_size=0, repetition_penalty=1.0, steps=None, banned=None,
               banned_per_example=None, use_ex3: bool | None = None, workspace: bool = True,
               x_offset: int = 0, beams=None, eos_tokens=None, min_lengths=None, expect_status=None,
               with_status: bool = False, noalloc: bool = False, read_back: bool = False) -> dict:
        B, T, K, V = xin.shape
        x = _dev(xin.view(np.int16) if xin.dtype == np.uint16 else xin)
        if x_offset:
            # the rows at an element offset from the allocation (any alignment)
            flat = torch.empty(x.numel() + x_offset, dtype=x.dtype, device=x.device)
            flat[x_offset:] = x.reshape(-1)
            x = flat[x_offset:].view(B, T, K, V)
        dev = x.device
        f32 = dict(dtype=torch.float32, device=dev)
        i32 = dict(dtype=torch.int32, device=dev)
        u8 = dict(dtype=torch.uint8, device=dev)
        out = {
            "final_scores": torch.empty(B, K, **f32), "final_raw_scores": torch.empty(B, K, **f32),
            "final_lengths": torch.empty(B, K, **i32), "tokens": torch.empty(B, T, K, **i32),
            "parents": torch.empty(B, T, K, **i32), "lengths": torch.empty(B, T, K, **i32),
            "scores": torch.empty(B, T, K, **f32), "raw_scores": torch.empty(B, T, K, **f32),
            "from_logprob": torch.empty(B, T, K, **u8), "invalid": torch.empty(B, **u8),
            "row_lse": torch.full((B, T, K), 7.0, **f32),
        }
        steps_d = _dev(None if steps is None else np.asarray(steps, np.int32))
        banned_d = _dev(None if banned is None else np.asarray(banned, np.uint8))
        bpe_d = _dev(None if banned_per_example is None else np.asarray(banned_per_example, np.uint8))
        args = _abi.DecodeArgs()
        args.batch_size, args.steps, args.beam_size, args.vocab_size = B, T, K, V
        args.eos_token, args.min_length, args.length_penalty_alpha = eos_token, min_length, alpha
        args.no_repeat_ngram_size, args.repetition_penalty = no_repeat_ngram_size, repetition_penalty
        args.steps_per_example = _abi.ptr(steps_d)
        args.banned_tokens = _abi.ptr(banned_d)
        per_example = {name: _dev(None if a is None else np.asarray(a, np.int32))
                       for name, a in (("beams", beams), ("eos", eos_tokens), ("min", min_lengths))}
        args.beam_sizes_per_example = _abi.ptr(per_example["beams"])
        args.eos_tokens_per_example = _abi.ptr(per_example["eos"])
        args.min_lengths_per_example = _abi.ptr(per_example["min"])
        o = _abi.DecodeOutputs(*(_abi.ptr(out[k]) for k in (
            "final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
            "raw_scores", "from_logprob", "invalid")))
        opts = _abi.SearchOptions()
        opts.extra_eos_count = len(extra_eos)
        for i, v in enumerate(extra_eos):
            opts.extra_eos_tokens[i] = int(v)
        ws_bytes = self.lib.dbs_cuda_decode_workspace_size(C.byref(args))
        assert ws_bytes > 0
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if workspace else None
        if use_ex3 is None:
            use_ex3 = bpe_d is not None
        fault = C.c_void_p()
        if read_back:
            # dbs_hip_decode_ex4, then the flags and the fault word read back
            # by dbs_hip_decode_read_back before anything else waits
            status = self.lib.dbs_hip_decode_ex4(
                _abi.ptr(x), _abi.DTYPE[dtype], int(from_logits), C.byref(args), C.byref(opts), _abi.ptr(bpe_d),
                C.byref(o), _abi.ptr(out["row_lse"]), _abi.ptr(ws), ws_bytes, C.byref(fault), self.stream())
            assert status == _abi.STATUS_OK, self.lib.dbs_cuda_status_string(status)
            flags = np.full(B, 0xAB, np.uint8)
            word = np.full(1, -7, np.int32)
            st = self.lib.dbs_hip_decode_read_back(_abi.ptr(out["invalid"]), B, flags.ctypes.data, fault, self.stream())
            assert st == _abi.STATUS_OK, self.lib.dbs_cuda_status_string(st)
            if fault.value:
                st = self.lib.dbs_hip_decode_read_back(fault, 4, word.ctypes.data, fault, self.stream())
                assert st == _abi.STATUS_OK, self.lib.dbs_cuda_status_string(st)
            torch.cuda.current_stream().synchronize()
            res = {k: v.cpu().numpy() for k, v in out.items()}
            res["read_back_flags"], res["read_back_fault"] = flags, (int(word[0]) if fault.value else None)
            res["fault_word"] = None
            if fault.value:
                # the word read by a plain copy, from its place in the workspace
                at = fault.value - ws.data_ptr()
                assert 0 <= at <= ws_bytes - 4
                res["fault_word"] = int(ws[at:at + 4].cpu().numpy().view(np.int32)[0])
            return res
        if noalloc:
            status = self.lib.dbs_hip_decode_noalloc(
                _abi.ptr(x), _abi.DTYPE[dtype], int(from_logits), C.byref(args), C.byref(opts), _abi.ptr(bpe_d),
                C.byref(o), _abi.ptr(out["row_lse"]), self.stream())
        elif use_ex3:
            status = self.lib.dbs_hip_decode_ex3(
                _abi.ptr(x), _abi.DTYPE[dtype], int(from_logits), C.byref(args), C.byref(opts), _abi.ptr(bpe_d),
                C.byref(o), _abi.ptr(out["row_lse"]), _abi.ptr(ws), ws_bytes if ws is not None else 0, self.stream())
        else:
            assert bpe_d is None
            status = self.lib.dbs_cuda_decode_ex2(
                _abi.ptr(x), _abi.DTYPE[dtype], int(from_logits), C.byref(args), C.byref(opts), C.byref(o),
                _abi.ptr(out["row_lse"]), _abi.ptr(ws), ws_bytes if ws is not None else 0, self.stream())
        if expect_status is not None:
            torch.cuda.current_stream().synchronize()
            return status
        if not with_status:
            assert status == _abi.STATUS_OK, self.lib.dbs_cuda_status_string(status)
        torch.cuda.current_stream().synchronize()
        res = {k: v.cpu().numpy() for k, v in out.items()}
        return (status, res) if with_status else res

    # ------------------------------------------------------------------
    def _bwd_inputs(self, trace, grads, logits, dtype, row_lse, keep):
        inp = _abi.BackwardInputs()
        for name in ("parents", "tokens", "lengths"):
            keep[name] = _dev(np.asarray(trace[name], np.int32))
            setattr(inp, name, _abi.ptr(keep[name]))
        keep["from_logprob"] = _dev(np.asarray(trace["from_logprob"], np.uint8))
        inp.from_logprob = _abi.ptr(keep["from_logprob"])
        for key, field in (("grad_final", "grad_final_scores"), ("grad_final_raw", "grad_final_raw_scores"),
                           ("grad_scores", "grad_scores"), ("grad_raw", "grad_raw_scores")):
            g = grads.get(key)
            keep[key] = _dev(None if g is None else np.asarray(g, np.float32))
            setattr(inp, field, _abi.ptr(keep[key]))
        if logits is not None:
            keep["logits"] = _dev(logits.view(np.int16) if logits.dtype == np.uint16 else logits)
            keep["row_lse"] = _dev(np.asarray(row_lse, np.float32))
            inp.logits = _abi.ptr(keep["logits"])
            inp.logits_type = _abi.DTYPE[dtype]
            inp.row_lse = _abi.ptr(keep["row_lse"])
        return inp

    def _args(self, B, T, K, V, alpha, steps, keep, beams=None):
        args = _abi.DecodeArgs()
        args.batch_size, args.steps, args.beam_size, args.vocab_size = B, T, K, V
        args.eos_token = -1
        args.length_penalty_alpha = alpha
        args.repetition_penalty = 1.0
        keep["steps"] = _dev(None if steps is None else np.asarray(steps, np.int32))
        args.steps_per_example = _abi.ptr(keep["steps"])
        keep["beams"] = _dev(None if beams is None else np.asarray(beams, np.int32))
        args.beam_sizes_per_example = _abi.ptr(keep["beams"])
        return args

    def backward(self, trace: dict, V: int, *, alpha=0.0, steps=None, logits=None, dtype="f32", row_lse=None,
                 mode="accumulate", out_type="f32", initial: np.ndarray | None = None, beams=None,
                 **grads) -> np.ndarray:
        """mode 'accumulate': dbs_cuda_backward_ex into `initial` (zeros by
        default); 'dense': dbs_hip_backward_dense in out_type; 'final': dbs_cuda_backward."""
        B, T, K = np.asarray(trace["parents"]).shape
        keep = {}
        args = self._args(B, T, K, V, alpha, steps, keep, beams)
        inp = self._bwd_inputs(trace, grads, logits, dtype, row_lse, keep)
        ws_bytes = self.lib.dbs_cuda_backward_workspace_size(C.byref(args))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        if mode == "dense":
            tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[out_type]
            grad = torch.full((B, T, K, V), 3.0, dtype=tdt, device="cuda")  # every element must be written
            status = self.lib.dbs_hip_backward_dense(C.byref(args), C.byref(inp), _abi.ptr(grad),
                                                     _abi.GRAD_TYPE[out_type], _abi.ptr(ws), ws_bytes, self.stream())
        else:
            grad = _dev(np.zeros((B, T, K, V), np.float32) if initial is None else initial)
            if mode == "final":
                status = self.lib.dbs_cuda_backward(C.byref(args), inp.parents, inp.tokens, inp.lengths,
                                                    inp.from_logprob, inp.grad_final_scores, _abi.ptr(grad),
                                                    _abi.ptr(ws), ws_bytes, self.stream())
            else:
                status = self.lib.dbs_cuda_backward_ex(C.byref(args), C.byref(inp), _abi.ptr(grad), _abi.ptr(ws),
                                                       ws_bytes, self.stream())
        assert status == _abi.STATUS_OK, self.lib.dbs_cuda_status_string(status)
        torch.cuda.synchronize()
        if grad.dtype == torch.float32:
            return grad.cpu().numpy()
        return grad.view(torch.int16).cpu().numpy().view(np.uint16)

    def path_gradient(self, trace: dict, V: int, grad_final: np.ndarray, *, alpha=0.0, steps=None,
                      beams=None) -> np.ndarray:
        B, T, K = np.asarray(trace["parents"]).shape
        keep = {}
        args = self._args(B, T, K, V, alpha, steps, keep, beams)
        inp = self._bwd_inputs(trace, {"grad_final": grad_final}, None, "f32", None, keep)
        draws = torch.full((B, T, K), 5.0, dtype=torch.float32, device="cuda")
        status = self.lib.dbs_cuda_path_gradient(C.byref(args), inp.parents, inp.tokens, inp.lengths,
                                                 inp.from_logprob, inp.grad_final_scores, _abi.ptr(draws),
                                                 self.stream())
        assert status == _abi.STATUS_OK
        torch.cuda.synchronize()
        return draws.cpu().numpy()

    def length_penalty(self, lengths: np.ndarray, alpha: float) -> np.ndarray:
        d = _dev(np.asarray(lengths, np.int32))
        out = torch.empty(d.shape, dtype=torch.float32, device="cuda")
        status = self.lib.dbs_cuda_length_penalty(_abi.ptr(d), d.numel(), alpha, _abi.ptr(out), self.stream())
        assert status == _abi.STATUS_OK
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def backtrack(self, tokens, parents, steps=None) -> np.ndarray:
        tok = _dev(np.asarray(tokens, np.int32))
        par = _dev(np.asarray(parents, np.int32))
        st = _dev(None if steps is None else np.asarray(steps, np.int32))
        B, T, K = tok.shape
        out = torch.full((B, K, T), 9, dtype=torch.int64, device="cuda")
        status = self.lib.dbs_hip_backtrack(_abi.ptr(tok), _abi.ptr(par), _abi.ptr(st), B, T, K, _abi.ptr(out),
                                            self.stream())
        assert status == _abi.STATUS_OK
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def backtrack_i64(self, tokens, parents, steps=None) -> np.ndarray:
        tok = _dev(np.asarray(tokens, np.int64))
        par = _dev(np.asarray(parents, np.int64))
        st = _dev(None if steps is None else np.asarray(steps, np.int64))
        B, T, K = tok.shape
        out = torch.full((B, K, T), 9, dtype=torch.int64, device="cuda")
        status = self.lib.dbs_hip_backtrack_i64(_abi.ptr(tok), _abi.ptr(par), _abi.ptr(st), B, T, K, _abi.ptr(out),
                                                self.stream())
        assert status == _abi.STATUS_OK
        torch.cuda.synchronize()
        return out.cpu().numpy()

    # ------------------------------------------------------------------
    def steps(self, xin: np.ndarray, dtype: str, *, from_logits=False, eos_token=-1, extra_eos=(), min_length=0,
              alpha=0.0, beams=None, eos_tokens=None, min_lengths=None) -> dict:
        """The decode of [B, T, K, V] rows run as T calls of
        dbs_cuda_decode_step_ex2 from the initial beam state (unconstrained),
        with the trace collected step by step."""
        B, T, K, V = xin.shape
        x = _dev(xin.view(np.int16) if xin.dtype == np.uint16 else xin)
        dev = x.device
        raw = torch.full((B, K), float("-inf"), dtype=torch.float32, device=dev)
        raw[:, 0] = 0.0
        lengths = torch.zeros(B, K, dtype=torch.int32, device=dev)
        finished = torch.zeros(B, K, dtype=torch.uint8, device=dev)
        per_example = {name: _dev(None if a is None else np.asarray(a, np.int32))
                       for name, a in (("beams", beams), ("eos", eos_tokens), ("min", min_lengths))}
        args = _abi.DecodeArgs()
        args.batch_size, args.steps, args.beam_size, args.vocab_size = B, 1, K, V
        args.eos_token, args.min_length, args.length_penalty_alpha = eos_token, min_length, alpha
        args.repetition_penalty = 1.0
        args.beam_sizes_per_example = _abi.ptr(per_example["beams"])
        args.eos_tokens_per_example = _abi.ptr(per_example["eos"])
        args.min_lengths_per_example = _abi.ptr(per_example["min"])
        opts = _abi.SearchOptions()
        opts.extra_eos_count = len(extra_eos)
        for i, v in enumerate(extra_eos):
            opts.extra_eos_tokens[i] = int(v)
        state = _abi.BeamState(_abi.ptr(raw), _abi.ptr(lengths), _abi.ptr(finished), None, 0, 0)
        ws_bytes = self.lib.dbs_cuda_decode_step_workspace_size(C.byref(args), 0)
        assert ws_bytes > 0
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        names = ("tokens", "parents", "lengths", "scores", "raw_scores", "from_logprob")
        trace = {n: [] for n in names}
        final = torch.empty(B, K, dtype=torch.float32, device=dev)
        for t in range(T):
            out = {"tokens": torch.empty(B, K, dtype=torch.int32, device=dev),
                   "parents": torch.empty(B, K, dtype=torch.int32, device=dev),
                   "lengths": torch.empty(B, K, dtype=torch.int32, device=dev),
                   "scores": torch.empty(B, K, dtype=torch.float32, device=dev),
                   "raw_scores": torch.empty(B, K, dtype=torch.float32, device=dev),
                   "from_logprob": torch.empty(B, K, dtype=torch.uint8, device=dev)}
            o = _abi.DecodeOutputs(_abi.ptr(final), None, None, _abi.ptr(out["tokens"]), _abi.ptr(out["parents"]),
                                   _abi.ptr(out["lengths"]), _abi.ptr(out["scores"]), _abi.ptr(out["raw_scores"]),
                                   _abi.ptr(out["from_logprob"]), None)
            rows = x[:, t].contiguous()
            status = self.lib.dbs_cuda_decode_step_ex2(
                _abi.ptr(rows), _abi.DTYPE[dtype], int(from_logits), C.byref(args), C.byref(opts), C.byref(state),
                C.byref(o), None, _abi.ptr(ws), ws_bytes, self.stream())
            assert status == _abi.STATUS_OK, self.lib.dbs_cuda_status_string(status)
            torch.cuda.synchronize()
            for n in names:
                trace[n].append(out[n].cpu().numpy())
        res = {n: np.stack(v, 1) for n, v in trace.items()}
        res["final_scores"] = final.cpu().numpy()
        res["final_raw_scores"] = raw.cpu().numpy()
        res["final_lengths"] = lengths.cpu().numpy()
        return res
