# SPDX-License-Identifier: MIT
"""ctypes front end of the test oracle (test infrastructure only).

Two CPU implementations of the reference algorithm, both used only as
checkers by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg:

* :class:`Oracle` wraps ``oracle/liboracle.so``, the C restatement in
  ``oracle/dbs_oracle.c``;
* :class:`Reference` wraps ``oracle/_ref/libdbs_ref.so``, the reference's own
  CPU library compiled from its sources by ``oracle/Makefile`` (present where
  it was built; it travels with the tree as a built file).

Inputs are numpy arrays; 16-bit rows are passed as ``uint16`` bit patterns.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DTYPES = {"f32": 0, "f16": 1, "bf16": 2}

_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u8p = C.POINTER(C.c_uint8)
_i64p = C.POINTER(C.c_int64)


def build() -> None:
    """Compile liboracle.so (and _ref where the reference is mounted)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray | None, ctype):
    if a is None:
        return C.cast(None, C.POINTER(ctype))
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data_as(C.POINTER(ctype))


def _vptr(a: np.ndarray | None):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _dtype_of(x: np.ndarray, dtype: str | None) -> str:
    if dtype is not None:
        return dtype
    if x.dtype == np.float32:
        return "f32"
    raise ValueError("16-bit inputs need dtype='f16' or 'bf16' (pass uint16 bit patterns)")


# ---------------------------------------------------------------------------
# C restatement
# ---------------------------------------------------------------------------


class _OrcDecodeArgs(C.Structure):
    _fields_ = [
        ("batch_size", C.c_int), ("steps", C.c_int), ("beam_size", C.c_int), ("vocab_size", C.c_int),
        ("dtype", C.c_int), ("from_logits", C.c_int), ("eos_token", C.c_int),
        ("extra_eos", _i32p), ("extra_eos_count", C.c_int), ("min_length", C.c_int),
        ("length_penalty_alpha", C.c_float), ("no_repeat_ngram_size", C.c_int),
        ("repetition_penalty", C.c_float), ("steps_per_example", _i32p), ("banned", _u8p),
        ("banned_per_example", _u8p), ("num_threads", C.c_int),
    ]


class _OrcDecodeOutputs(C.Structure):
    _fields_ = [
        ("final_scores", _f32p), ("final_raw_scores", _f32p), ("final_lengths", _i32p), ("tokens", _i32p),
        ("parents", _i32p), ("lengths", _i32p), ("scores", _f32p), ("raw_scores", _f32p),
        ("from_logprob", _u8p), ("row_lse", _f32p), ("invalid", _u8p), ("row_read", _u8p),
    ]


class _OrcBackwardArgs(C.Structure):
    _fields_ = [
        ("batch_size", C.c_int), ("steps", C.c_int), ("beam_size", C.c_int), ("vocab_size", C.c_int),
        ("length_penalty_alpha", C.c_float), ("steps_per_example", _i32p), ("parents", _i32p),
        ("tokens", _i32p), ("lengths", _i32p), ("from_logprob", _u8p), ("grad_final_scores", _f32p),
        ("grad_final_raw_scores", _f32p), ("grad_scores", _f32p), ("grad_raw_scores", _f32p),
        ("logits", C.c_void_p), ("logits_dtype", C.c_int), ("row_lse", _f32p), ("num_threads", C.c_int),
    ]


TRACE_FIELDS = ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
                "raw_scores", "from_logprob", "row_lse")


class Oracle:
    """The C restatement (oracle/dbs_oracle.c)."""

    def __init__(self, path: str | None = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        self.lib = C.CDLL(path)
        L = self.lib
        L.orc_decode.argtypes = [C.c_void_p, C.POINTER(_OrcDecodeArgs), C.POINTER(_OrcDecodeOutputs)]
        L.orc_decode.restype = C.c_int
        L.orc_backward.argtypes = [C.POINTER(_OrcBackwardArgs), _f32p]
        L.orc_backward.restype = C.c_int
        L.orc_path_gradient.argtypes = [C.POINTER(_OrcBackwardArgs), _f32p]
        L.orc_path_gradient.restype = C.c_int
        L.orc_length_penalty.argtypes = [C.c_int, C.c_float]
        L.orc_length_penalty.restype = C.c_float
        L.orc_length_penalty_array.argtypes = [_i32p, C.c_int64, C.c_float, _f32p]
        L.orc_exp_nonpositive.argtypes = [C.c_float]
        L.orc_exp_nonpositive.restype = C.c_float
        L.orc_log_ge1.argtypes = [C.c_double]
        L.orc_log_ge1.restype = C.c_double
        L.orc_exp_ge0.argtypes = [C.c_double]
        L.orc_exp_ge0.restype = C.c_double
        L.orc_row_stats.argtypes = [_f32p, C.c_int, _f32p, _f32p, C.POINTER(C.c_int)]
        L.orc_softmax_probability.argtypes = [C.c_float, C.c_float]
        L.orc_softmax_probability.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_backtrack.argtypes = [_i32p, _i32p, _i32p, C.c_int, C.c_int, C.c_int, _i64p]

    # -- numerics ----------------------------------------------------------
    def length_penalty(self, lengths, alpha: float) -> np.ndarray:
        lengths = np.ascontiguousarray(np.clip(np.asarray(lengths, dtype=np.int64), 0, 2**31 - 1), dtype=np.int32)
        out = np.empty(lengths.shape, dtype=np.float32)
        self.lib.orc_length_penalty_array(_ptr(lengths, C.c_int32), lengths.size, float(alpha), _ptr(out, C.c_float))
        return out

    def row_stats(self, row: np.ndarray) -> tuple[float, float, bool]:
        row = np.ascontiguousarray(row, dtype=np.float32)
        mx, lse, bad = C.c_float(), C.c_float(), C.c_int()
        self.lib.orc_row_stats(_ptr(row, C.c_float), row.size, C.byref(mx), C.byref(lse), C.byref(bad))
        return mx.value, lse.value, bool(bad.value)

    def exp_nonpositive(self, x: np.ndarray) -> np.ndarray:
        x = np.asarray(x, dtype=np.float32)
        f = self.lib.orc_exp_nonpositive
        return np.array([f(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)

    # -- decode ------------------------------------------------------------
    def decode(self, x: np.ndarray, *, dtype: str | None = None, from_logits: bool = False, eos_token: int = -1,
               extra_eos=(), min_length: int = 0, alpha: float = 0.0, no_repeat_ngram_size: int = 0,
               repetition_penalty: float = 1.0, steps=None, banned=None, banned_per_example=None,
               num_threads: int = 0) -> dict:
        dtype = _dtype_of(x, dtype)
        x = np.ascontiguousarray(x)
        B, T, K, V = x.shape
        extra = np.ascontiguousarray(np.asarray(list(extra_eos), dtype=np.int32))
        steps_a = None if steps is None else np.ascontiguousarray(np.asarray(steps, dtype=np.int32))
        banned_a = None if banned is None else np.ascontiguousarray(np.asarray(banned, dtype=np.uint8))
        bpe = None if banned_per_example is None else np.ascontiguousarray(np.asarray(banned_per_example, np.uint8))
        args = _OrcDecodeArgs(
            B, T, K, V, DTYPES[dtype], int(bool(from_logits)), int(eos_token), _ptr(extra, C.c_int32), len(extra),
            int(min_length), float(alpha), int(no_repeat_ngram_size), float(repetition_penalty),
            _ptr(steps_a, C.c_int32), _ptr(banned_a, C.c_uint8), _ptr(bpe, C.c_uint8),
            int(num_threads) if num_threads > 0 else (os.cpu_count() or 1),
        )
        out = {
            "final_scores": np.empty((B, K), np.float32), "final_raw_scores": np.empty((B, K), np.float32),
            "final_lengths": np.empty((B, K), np.int32), "tokens": np.empty((B, T, K), np.int32),
            "parents": np.empty((B, T, K), np.int32), "lengths": np.empty((B, T, K), np.int32),
            "scores": np.empty((B, T, K), np.float32), "raw_scores": np.empty((B, T, K), np.float32),
            "from_logprob": np.empty((B, T, K), np.uint8), "row_lse": np.empty((B, T, K), np.float32),
            "invalid": np.empty((B,), np.uint8), "row_read": np.empty((B, T, K), np.uint8),
        }
        o = _OrcDecodeOutputs(*(_ptr(out[name], ct) for name, ct in (
            ("final_scores", C.c_float), ("final_raw_scores", C.c_float), ("final_lengths", C.c_int32),
            ("tokens", C.c_int32), ("parents", C.c_int32), ("lengths", C.c_int32), ("scores", C.c_float),
            ("raw_scores", C.c_float), ("from_logprob", C.c_uint8), ("row_lse", C.c_float),
            ("invalid", C.c_uint8), ("row_read", C.c_uint8))))
        status = self.lib.orc_decode(_vptr(x), C.byref(args), C.byref(o))
        if status != 0:
            raise ValueError("oracle decode: invalid arguments")
        return out

    def decode_per_example(self, x: np.ndarray, *, beams=None, eos_tokens=None, min_lengths=None, steps=None,
                           eos_token: int = -1, extra_eos=(), min_length: int = 0, banned_per_example=None,
                           **kw) -> dict:
        """Per-example beams, EOS tokens and minimum lengths: example b decoded
        alone with its own options on the first beams[b] rows of each step,
        its slots past them empty (reference src/c_api.cpp:638-698, the CUDA
        engine's layout cuda/dbs_cuda.cu:944-955 and :969-980). The extra EOS
        tokens count only for an example with an EOS token."""
        B, T, K, V = x.shape
        empty = {"final_scores": -np.inf, "final_raw_scores": -np.inf, "final_lengths": 0, "tokens": -1,
                 "parents": -1, "lengths": 0, "scores": -np.inf, "raw_scores": -np.inf, "from_logprob": 0,
                 "row_lse": 0.0, "row_read": 0}
        parts = []
        for b in range(B):
            kb = K if beams is None else int(beams[b])
            eb = eos_token if eos_tokens is None else int(eos_tokens[b])
            mb = min_length if min_lengths is None else int(min_lengths[b])
            st = None if steps is None else [int(np.asarray(steps)[b])]
            bpe = None if banned_per_example is None else np.asarray(banned_per_example)[b:b + 1]
            one = self.decode(np.ascontiguousarray(x[b:b + 1, :, :kb]), eos_token=eb,
                              extra_eos=tuple(extra_eos) if eb >= 0 else (), min_length=mb, steps=st,
                              banned_per_example=bpe, **kw)
            full = {}
            for name, a in one.items():
                if name == "invalid":
                    full[name] = a
                    continue
                shape = (1, K) if a.ndim == 2 else (1, T, K)
                f = np.full(shape, empty[name], dtype=a.dtype)
                f[..., :kb] = a
                full[name] = f
            parts.append(full)
        return {k: np.concatenate([q[k] for q in parts], 0) for k in parts[0]}

    # -- backward ----------------------------------------------------------
    def _bwd_args(self, trace: dict, vocab_size: int, alpha: float, steps, grad_final, grad_final_raw, grad_scores,
                  grad_raw, logits, logits_dtype, row_lse, num_threads):
        keep = {}

        def arr(name, a, dt):
            if a is None:
                return None
            keep[name] = np.ascontiguousarray(np.asarray(a, dtype=dt))
            return keep[name]

        par = arr("parents", trace["parents"], np.int32)
        B, T, K = par.shape
        args = _OrcBackwardArgs(
            B, T, K, int(vocab_size), float(alpha), _ptr(arr("steps", steps, np.int32), C.c_int32),
            _ptr(par, C.c_int32), _ptr(arr("tokens", trace["tokens"], np.int32), C.c_int32),
            _ptr(arr("lengths", trace["lengths"], np.int32), C.c_int32),
            _ptr(arr("from_logprob", trace["from_logprob"], np.uint8), C.c_uint8),
            _ptr(arr("gf", grad_final, np.float32), C.c_float), _ptr(arr("gfr", grad_final_raw, np.float32), C.c_float),
            _ptr(arr("gs", grad_scores, np.float32), C.c_float), _ptr(arr("gr", grad_raw, np.float32), C.c_float),
            None, 0, _ptr(arr("lse", row_lse, np.float32), C.c_float),
            int(num_threads) if num_threads > 0 else (os.cpu_count() or 1),
        )
        if logits is not None:
            keep["logits"] = np.ascontiguousarray(logits)
            args.logits = C.c_void_p(keep["logits"].ctypes.data)
            args.logits_dtype = DTYPES[_dtype_of(keep["logits"], logits_dtype)]
        return args, keep, (B, T, K)

    def backward(self, trace: dict, vocab_size: int, *, alpha: float = 0.0, steps=None, grad_final=None,
                 grad_final_raw=None, grad_scores=None, grad_raw=None, logits=None, logits_dtype=None,
                 row_lse=None, num_threads: int = 0, out: np.ndarray | None = None) -> np.ndarray:
        args, keep, (B, T, K) = self._bwd_args(trace, vocab_size, alpha, steps, grad_final, grad_final_raw,
                                               grad_scores, grad_raw, logits, logits_dtype, row_lse, num_threads)
        grad = np.zeros((B, T, K, vocab_size), np.float32) if out is None else out
        if self.lib.orc_backward(C.byref(args), _ptr(grad, C.c_float)) != 0:
            raise ValueError("oracle backward: invalid arguments or trace")
        return grad

    def path_gradient(self, trace: dict, vocab_size: int, grad_final, *, alpha: float = 0.0, steps=None):
        args, keep, (B, T, K) = self._bwd_args(trace, vocab_size, alpha, steps, grad_final, None, None, None, None,
                                               None, None, 1)
        draws = np.empty((B, T, K), np.float32)
        if self.lib.orc_path_gradient(C.byref(args), _ptr(draws, C.c_float)) != 0:
            raise ValueError("oracle path_gradient: invalid arguments or trace")
        return draws

    def backtrack(self, tokens, parents, steps=None) -> np.ndarray:
        tok = np.ascontiguousarray(np.asarray(tokens, np.int32))
        par = np.ascontiguousarray(np.asarray(parents, np.int32))
        B, T, K = tok.shape
        st = None if steps is None else np.ascontiguousarray(np.asarray(steps, np.int32))
        out = np.empty((B, K, T), np.int64)
        self.lib.orc_backtrack(_ptr(tok, C.c_int32), _ptr(par, C.c_int32), _ptr(st, C.c_int32), B, T, K,
                               _ptr(out, C.c_int64))
        return out


# ---------------------------------------------------------------------------
# The reference's own CPU library (oracle/_ref), through its public C ABI
# (include/dbs.h of the reference)
# ---------------------------------------------------------------------------


class _DBSOptionsC(C.Structure):
    _fields_ = [
        ("beam_size", C.c_int), ("eos_token", C.c_int), ("selected_temperature", C.c_float),
        ("soft_topk_temperature", C.c_float), ("relaxed_pool_multiplier", C.c_int), ("vocab_block", C.c_int),
        ("length_penalty_alpha", C.c_float), ("soft_topk_tolerance", C.c_float), ("soft_topk_max_iters", C.c_int),
        ("min_length", C.c_int), ("validate_inputs", C.c_int), ("max_dense_gradient_elements", C.c_int64),
        ("reserved0", C.c_int), ("reserved1", C.c_int),
    ]


class _DBSAdvancedConstraintsC(C.Structure):
    _fields_ = [
        ("banned_tokens", _u8p), ("forced_tokens", _i32p), ("min_length", C.c_int),
        ("repetition_penalty", C.c_float), ("no_repeat_ngram_size", C.c_int), ("token_filter", C.c_void_p),
        ("token_filter_user_data", C.c_void_p), ("batch_index", C.c_int),
    ]


class _DBSDecodeOutputsC(C.Structure):
    _fields_ = [
        ("final_scores", _f32p), ("final_raw_scores", _f32p), ("final_lengths", _i32p), ("tokens", _i32p),
        ("parents", _i32p), ("lengths", _i32p), ("scores", _f32p), ("raw_scores", _f32p), ("from_logprob", _u8p),
    ]


class _DBSDecodeOutputsExC(C.Structure):
    _fields_ = [
        ("base", _DBSDecodeOutputsC), ("pool_parents", _i32p), ("pool_tokens", _i32p), ("pool_lengths", _i32p),
        ("pool_scores", _f32p), ("pool_raw_scores", _f32p), ("pool_from_logprob", _u8p), ("row_lse", _f32p),
        ("reserved", C.c_void_p * 4),
    ]


class _DBSBackwardInputsC(C.Structure):
    _fields_ = [
        ("batch_size", C.c_int), ("steps", C.c_int), ("vocab_size", C.c_int), ("pool_size", C.c_int),
        ("steps_per_example", _i32p), ("parents", _i32p), ("tokens", _i32p), ("lengths", _i32p),
        ("from_logprob", _u8p), ("pool_parents", _i32p), ("pool_tokens", _i32p), ("pool_lengths", _i32p),
        ("pool_from_logprob", _u8p), ("grad_final_scores", _f32p), ("grad_final_raw_scores", _f32p),
        ("grad_scores", _f32p), ("grad_raw_scores", _f32p), ("grad_pool_scores", _f32p),
        ("grad_pool_raw_scores", _f32p), ("logits", C.c_void_p), ("logits_type", C.c_int), ("row_lse", _f32p),
        ("reserved", C.c_void_p * 4),
    ]


def reference_path() -> str:
    return os.path.join(HERE, "_ref", "libdbs_ref.so")


def reference_available() -> bool:
    return os.path.exists(reference_path())


class ReferenceError(RuntimeError):
    pass


class Reference:
    """The reference CPU library (dbs_decode_batch_into_ex / dbs_backward_batch_into_ex)."""

    def __init__(self, path: str | None = None):
        self.lib = C.CDLL(path or reference_path())
        L = self.lib
        L.dbs_create_ex.argtypes = [_DBSOptionsC, C.POINTER(C.c_void_p)]
        L.dbs_create_ex.restype = C.c_int
        L.dbs_destroy.argtypes = [C.c_void_p]
        L.dbs_last_global_error.restype = C.c_char_p
        L.dbs_set_extra_eos_tokens.argtypes = [C.c_void_p, _i32p, C.c_int]
        L.dbs_decode_batch_into_ex.argtypes = [
            C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _i32p,
            C.POINTER(_DBSAdvancedConstraintsC), C.c_int, C.POINTER(_DBSDecodeOutputsExC)]
        L.dbs_decode_batch_into_ex.restype = C.c_int
        L.dbs_backward_batch_into_ex.argtypes = [C.c_void_p, C.POINTER(_DBSBackwardInputsC), C.c_int, _f32p]
        L.dbs_backward_batch_into_ex.restype = C.c_int
        L.dbs_selected_kernel_name.restype = C.c_char_p

    def kernel_name(self) -> str:
        return self.lib.dbs_selected_kernel_name().decode()

    def _handle(self, K, eos_token, extra_eos, min_length, alpha, validate):
        opt = _DBSOptionsC()
        opt.beam_size = K
        opt.eos_token = eos_token
        opt.length_penalty_alpha = alpha
        opt.min_length = min_length
        opt.validate_inputs = 1 if validate else 0
        h = C.c_void_p()
        if self.lib.dbs_create_ex(opt, C.byref(h)) != 0:
            raise ReferenceError(self.lib.dbs_last_global_error().decode())
        if extra_eos:
            e = np.ascontiguousarray(np.asarray(list(extra_eos), np.int32))
            if self.lib.dbs_set_extra_eos_tokens(h, _ptr(e, C.c_int32), len(e)) != 0:
                self.lib.dbs_destroy(h)
                raise ReferenceError(self.lib.dbs_last_global_error().decode())
        return h

    def decode(self, x: np.ndarray, *, dtype: str | None = None, from_logits: bool = False, eos_token: int = -1,
               extra_eos=(), min_length: int = 0, alpha: float = 0.0, no_repeat_ngram_size: int = 0,
               repetition_penalty: float = 1.0, steps=None, banned=None, validate: bool = False,
               num_threads: int = 0) -> dict:
        """dbs_decode_batch_into_ex over the whole batch (one shared banned mask)."""
        dtype = _dtype_of(x, dtype)
        x = np.ascontiguousarray(x)
        B, T, K, V = x.shape
        h = self._handle(K, eos_token, extra_eos, min_length, alpha, validate)
        try:
            out = {
                "final_scores": np.empty((B, K), np.float32), "final_raw_scores": np.empty((B, K), np.float32),
                "final_lengths": np.empty((B, K), np.int32), "tokens": np.empty((B, T, K), np.int32),
                "parents": np.empty((B, T, K), np.int32), "lengths": np.empty((B, T, K), np.int32),
                "scores": np.empty((B, T, K), np.float32), "raw_scores": np.empty((B, T, K), np.float32),
                "from_logprob": np.empty((B, T, K), np.uint8), "row_lse": np.empty((B, T, K), np.float32),
            }
            o = _DBSDecodeOutputsExC()
            o.base = _DBSDecodeOutputsC(*(_ptr(out[n], ct) for n, ct in (
                ("final_scores", C.c_float), ("final_raw_scores", C.c_float), ("final_lengths", C.c_int32),
                ("tokens", C.c_int32), ("parents", C.c_int32), ("lengths", C.c_int32), ("scores", C.c_float),
                ("raw_scores", C.c_float), ("from_logprob", C.c_uint8))))
            o.row_lse = _ptr(out["row_lse"], C.c_float)
            banned_a = None if banned is None else np.ascontiguousarray(np.asarray(banned, np.uint8))
            cons = None
            if banned_a is not None or no_repeat_ngram_size > 0 or repetition_penalty > 1.0:
                cons = _DBSAdvancedConstraintsC()
                cons.banned_tokens = _ptr(banned_a, C.c_uint8)
                cons.min_length = -1
                cons.repetition_penalty = float(repetition_penalty)
                cons.no_repeat_ngram_size = int(no_repeat_ngram_size)
            steps_a = None if steps is None else np.ascontiguousarray(np.asarray(steps, np.int32))
            status = self.lib.dbs_decode_batch_into_ex(
                h, _vptr(x), DTYPES[dtype], int(bool(from_logits)), B, T, V, _ptr(steps_a, C.c_int32),
                None if cons is None else C.byref(cons), int(num_threads), C.byref(o))
            if status != 0:
                raise ReferenceError(self.lib.dbs_last_global_error().decode())
            return out
        finally:
            self.lib.dbs_destroy(h)

    def decode_variable(self, x: np.ndarray, *, beam_size: int, beams=None, eos_tokens=None, min_lengths=None,
                        steps=None, eos_token: int = -1, extra_eos=(), min_length: int = 0, alpha: float = 0.0,
                        num_threads: int = 0) -> dict:
        """dbs_decode_batch_variable (float32 rows [B, T, K, V]): per-example
        steps, beams, EOS tokens and minimum lengths; each example's trace
        comes back [steps_b, beams_b] and is laid out here as [T, K] with
        empty slots past it."""
        x = np.ascontiguousarray(np.asarray(x, np.float32))
        B, T, K, V = x.shape
        L = self.lib
        L.dbs_decode_batch_variable.argtypes = [
            C.c_void_p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p, _i32p, _u8p, _i32p, C.c_int,
            C.POINTER(C.c_void_p)]
        L.dbs_decode_batch_variable.restype = C.c_int
        L.dbs_batch_result_at.argtypes = [C.c_void_p, C.c_int]
        L.dbs_batch_result_at.restype = C.c_void_p
        L.dbs_free_batch_result.argtypes = [C.c_void_p]
        for name, rt in (("steps", C.c_int), ("beam_size", C.c_int)):
            getattr(L, "dbs_result_" + name).argtypes = [C.c_void_p]
            getattr(L, "dbs_result_" + name).restype = rt
        fields = (("tokens", _i32p), ("parents", _i32p), ("lengths", _i32p), ("scores", _f32p),
                  ("raw_scores", _f32p), ("final_scores", _f32p), ("final_raw_scores", _f32p))
        for name, rt in fields:
            getattr(L, "dbs_result_" + name).argtypes = [C.c_void_p]
            getattr(L, "dbs_result_" + name).restype = rt
        h = self._handle(beam_size, eos_token, extra_eos, min_length, alpha, False)
        keep = {}

        def arr(name, a):
            if a is None:
                return None
            keep[name] = np.ascontiguousarray(np.asarray(a, np.int32))
            return _ptr(keep[name], C.c_int32)

        res = C.c_void_p()
        try:
            status = L.dbs_decode_batch_variable(
                h, _ptr(x, C.c_float), B, T, K, V, arr("steps", steps), arr("beams", beams), arr("eos", eos_tokens),
                arr("min", min_lengths), None, None, int(num_threads), C.byref(res))
            if status != 0:
                raise ReferenceError(self.lib.dbs_last_global_error().decode())
            out = {"final_scores": np.full((B, K), -np.inf, np.float32),
                   "final_raw_scores": np.full((B, K), -np.inf, np.float32),
                   "tokens": np.full((B, T, K), -1, np.int32), "parents": np.full((B, T, K), -1, np.int32),
                   "lengths": np.zeros((B, T, K), np.int32), "scores": np.full((B, T, K), -np.inf, np.float32),
                   "raw_scores": np.full((B, T, K), -np.inf, np.float32)}
            for b in range(B):
                r = L.dbs_batch_result_at(res, b)
                st, kb = L.dbs_result_steps(r), L.dbs_result_beam_size(r)
                for name, _ in fields:
                    ptr = getattr(L, "dbs_result_" + name)(r)
                    if name.startswith("final"):
                        out[name][b, :kb] = np.ctypeslib.as_array(ptr, shape=(kb,))
                    else:
                        out[name][b, :st, :kb] = np.ctypeslib.as_array(ptr, shape=(st, kb))
            return out
        finally:
            if res:
                L.dbs_free_batch_result(res)
            self.lib.dbs_destroy(h)

    def decode_per_example_banned(self, x: np.ndarray, banned_per_example: np.ndarray, *, steps=None, **kw) -> dict:
        """B single-example calls, each with its own banned mask (the reference
        has no batched form for this), spread over a pool of `num_threads`
        host threads (ctypes releases the GIL during each call)."""
        from concurrent.futures import ThreadPoolExecutor

        B = x.shape[0]
        threads = kw.pop("num_threads", 0) or (os.cpu_count() or 1)

        def one(b):
            st = None if steps is None else [int(np.asarray(steps)[b])]
            return self.decode(x[b:b + 1], banned=banned_per_example[b], steps=st, num_threads=1, **kw)

        with ThreadPoolExecutor(max_workers=max(1, min(threads, B))) as pool:
            parts = list(pool.map(one, range(B)))
        return {k: np.concatenate([p[k] for p in parts], 0) for k in parts[0]}

    def backward(self, trace: dict, vocab_size: int, *, alpha: float = 0.0, steps=None, grad_final=None,
                 grad_final_raw=None, grad_scores=None, grad_raw=None, logits=None, logits_dtype=None,
                 row_lse=None, num_threads: int = 0) -> np.ndarray:
        keep = {}

        def arr(name, a, dt):
            if a is None:
                return None
            keep[name] = np.ascontiguousarray(np.asarray(a, dtype=dt))
            return keep[name]

        par = arr("parents", trace["parents"], np.int32)
        B, T, K = par.shape
        h = self._handle(K, -1, (), 0, alpha, False)
        try:
            inp = _DBSBackwardInputsC()
            inp.batch_size, inp.steps, inp.vocab_size, inp.pool_size = B, T, int(vocab_size), 0
            inp.steps_per_example = _ptr(arr("steps", steps, np.int32), C.c_int32)
            inp.parents = _ptr(par, C.c_int32)
            inp.tokens = _ptr(arr("tokens", trace["tokens"], np.int32), C.c_int32)
            inp.lengths = _ptr(arr("lengths", trace["lengths"], np.int32), C.c_int32)
            inp.from_logprob = _ptr(arr("flp", trace["from_logprob"], np.uint8), C.c_uint8)
            inp.grad_final_scores = _ptr(arr("gf", grad_final, np.float32), C.c_float)
            inp.grad_final_raw_scores = _ptr(arr("gfr", grad_final_raw, np.float32), C.c_float)
            inp.grad_scores = _ptr(arr("gs", grad_scores, np.float32), C.c_float)
            inp.grad_raw_scores = _ptr(arr("gr", grad_raw, np.float32), C.c_float)
            if logits is not None:
                keep["logits"] = np.ascontiguousarray(logits)
                inp.logits = C.c_void_p(keep["logits"].ctypes.data)
                inp.logits_type = DTYPES[_dtype_of(keep["logits"], logits_dtype)]
                inp.row_lse = _ptr(arr("lse", row_lse, np.float32), C.c_float)
            grad = np.zeros((B, T, K, vocab_size), np.float32)
            status = self.lib.dbs_backward_batch_into_ex(h, C.byref(inp), int(num_threads), _ptr(grad, C.c_float))
            if status != 0:
                raise ReferenceError(self.lib.dbs_last_global_error().decode())
            return grad
        finally:
            self.lib.dbs_destroy(h)
