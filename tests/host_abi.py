# SPDX-License-Identifier: MIT
"""ctypes driver of the libdbs host C ABI (include/dbs.h) for any library that
exports it: libdbs_hip.so (this build, on the GPU) or the reference's own CPU
library (oracle/_ref/libdbs_ref.so). Both are called with identical arguments
and host arrays, so a test can compare their outputs bit for bit."""

from __future__ import annotations

import ctypes as C

import numpy as np

DTYPES = {"f32": 0, "f16": 1, "bf16": 2}
_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)


class OptionsC(C.Structure):
    _fields_ = [("beam_size", C.c_int), ("eos_token", C.c_int), ("selected_temperature", C.c_float),
                ("soft_topk_temperature", C.c_float), ("relaxed_pool_multiplier", C.c_int), ("vocab_block", C.c_int),
                ("length_penalty_alpha", C.c_float), ("soft_topk_tolerance", C.c_float),
                ("soft_topk_max_iters", C.c_int), ("min_length", C.c_int), ("validate_inputs", C.c_int),
                ("max_dense_gradient_elements", C.c_int64), ("reserved0", C.c_int), ("reserved1", C.c_int)]


class ConstraintsC(C.Structure):
    _fields_ = [("banned_tokens", _u8p), ("forced_tokens", _i32p), ("min_length", C.c_int),
                ("repetition_penalty", C.c_float), ("no_repeat_ngram_size", C.c_int), ("token_filter", C.c_void_p),
                ("token_filter_user_data", C.c_void_p), ("batch_index", C.c_int)]


class OutputsC(C.Structure):
    _fields_ = [("final_scores", _f32p), ("final_raw_scores", _f32p), ("final_lengths", _i32p), ("tokens", _i32p),
                ("parents", _i32p), ("lengths", _i32p), ("scores", _f32p), ("raw_scores", _f32p),
                ("from_logprob", _u8p)]


class OutputsExC(C.Structure):
    _fields_ = [("base", OutputsC), ("pool_parents", _i32p), ("pool_tokens", _i32p), ("pool_lengths", _i32p),
                ("pool_scores", _f32p), ("pool_raw_scores", _f32p), ("pool_from_logprob", _u8p),
                ("row_lse", _f32p), ("reserved", C.c_void_p * 4)]


class BackwardInputsC(C.Structure):
    _fields_ = [("batch_size", C.c_int), ("steps", C.c_int), ("vocab_size", C.c_int), ("pool_size", C.c_int),
                ("steps_per_example", _i32p), ("parents", _i32p), ("tokens", _i32p), ("lengths", _i32p),
                ("from_logprob", _u8p), ("pool_parents", _i32p), ("pool_tokens", _i32p), ("pool_lengths", _i32p),
                ("pool_from_logprob", _u8p), ("grad_final_scores", _f32p), ("grad_final_raw_scores", _f32p),
                ("grad_scores", _f32p), ("grad_raw_scores", _f32p), ("grad_pool_scores", _f32p),
                ("grad_pool_raw_scores", _f32p), ("logits", C.c_void_p), ("logits_type", C.c_int),
                ("row_lse", _f32p), ("reserved", C.c_void_p * 4)]


def _p(a, ct):
    return None if a is None else a.ctypes.data_as(C.POINTER(ct))


class HostError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status
        self.message = message


class HostLib:
    """One library's dbs_* entry points."""

    def __init__(self, path: str):
        self.path = path
        L = self.lib = C.CDLL(path)
        L.dbs_create_ex.argtypes = [OptionsC, C.POINTER(C.c_void_p)]
        L.dbs_create_ex.restype = C.c_int
        L.dbs_destroy.argtypes = [C.c_void_p]
        L.dbs_destroy.restype = None
        L.dbs_last_global_error.restype = C.c_char_p
        L.dbs_last_error.argtypes = [C.c_void_p]
        L.dbs_last_error.restype = C.c_char_p
        L.dbs_set_extra_eos_tokens.argtypes = [C.c_void_p, _i32p, C.c_int]
        L.dbs_set_extra_eos_tokens.restype = C.c_int
        L.dbs_decode_batch_into.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_int, C.c_int, _i32p,
                                            C.POINTER(ConstraintsC), C.c_int, C.POINTER(OutputsC)]
        L.dbs_decode_batch_into.restype = C.c_int
        L.dbs_decode_batch_into_ex.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                               _i32p, C.POINTER(ConstraintsC), C.c_int, C.POINTER(OutputsExC)]
        L.dbs_decode_batch_into_ex.restype = C.c_int
        L.dbs_backward_batch_into.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p, _i32p,
                                              _u8p, _f32p, C.c_int, _f32p]
        L.dbs_backward_batch_into.restype = C.c_int
        L.dbs_backward_batch_into_ex.argtypes = [C.c_void_p, C.POINTER(BackwardInputsC), C.c_int, _f32p]
        L.dbs_backward_batch_into_ex.restype = C.c_int
        L.dbs_abi_version.restype = C.c_int
        L.dbs_version_string.restype = C.c_char_p
        L.dbs_selected_kernel_name.restype = C.c_char_p

    # ------------------------------------------------------------------
    def create(self, **opts) -> C.c_void_p:
        o = OptionsC()
        for k, v in opts.items():
            setattr(o, k, v)
        h = C.c_void_p()
        status = self.lib.dbs_create_ex(o, C.byref(h))
        if status != 0:
            raise HostError(status, self.lib.dbs_last_global_error().decode())
        return h

    def destroy(self, h):
        self.lib.dbs_destroy(h)

    def error(self) -> str:
        return self.lib.dbs_last_global_error().decode()

    def set_extra_eos(self, h, tokens) -> int:
        a = np.ascontiguousarray(np.asarray(tokens, np.int32))
        return self.lib.dbs_set_extra_eos_tokens(h, _p(a, C.c_int32) if len(a) else None, len(a))

    # ------------------------------------------------------------------
    @staticmethod
    def constraints(banned=None, min_length=-1, repetition_penalty=1.0, no_repeat_ngram_size=0, forced=None,
                    keep=None):
        c = ConstraintsC()
        if banned is not None:
            keep["banned"] = np.ascontiguousarray(np.asarray(banned, np.uint8))
            c.banned_tokens = _p(keep["banned"], C.c_uint8)
        if forced is not None:
            keep["forced"] = np.ascontiguousarray(np.asarray(forced, np.int32))
            c.forced_tokens = _p(keep["forced"], C.c_int32)
        c.min_length = min_length
        c.repetition_penalty = repetition_penalty
        c.no_repeat_ngram_size = no_repeat_ngram_size
        return c

    def decode(self, h, x: np.ndarray, K: int, *, dtype="f32", from_logits=False, steps=None, constraints=None,
               ex=True, row_lse=True, fill=None, pool=0) -> tuple[int, dict]:
        """dbs_decode_batch_into_ex (or, ex=False, dbs_decode_batch_into for
        f32 log-probs); pool > 0 asks for the relaxed pool's [B, T, pool]
        outputs. Outputs are pre-filled with random bytes so every written
        element is checked. Returns (status, outputs)."""
        x = np.ascontiguousarray(x)
        B, T, KK, V = x.shape
        assert KK == K
        rng = np.random.default_rng(0)

        def buf(shape, dt):
            a = np.empty(shape, dt)
            a.view(np.uint8)[...] = rng.integers(0, 256, a.nbytes, dtype=np.uint8).reshape(a.view(np.uint8).shape)
            return a

        out = {"final_scores": buf((B, K), np.float32), "final_raw_scores": buf((B, K), np.float32),
               "final_lengths": buf((B, K), np.int32), "tokens": buf((B, T, K), np.int32),
               "parents": buf((B, T, K), np.int32), "lengths": buf((B, T, K), np.int32),
               "scores": buf((B, T, K), np.float32), "raw_scores": buf((B, T, K), np.float32),
               "from_logprob": buf((B, T, K), np.uint8)}
        if ex and row_lse:
            out["row_lse"] = buf((B, T, K), np.float32)
        pool_keys = (("pool_parents", np.int32, C.c_int32), ("pool_tokens", np.int32, C.c_int32),
                     ("pool_lengths", np.int32, C.c_int32), ("pool_scores", np.float32, C.c_float),
                     ("pool_raw_scores", np.float32, C.c_float), ("pool_from_logprob", np.uint8, C.c_uint8))
        if ex and pool:
            for name, dt, _ in pool_keys:
                out[name] = buf((B, T, pool), dt)
        base = OutputsC(*(_p(out[n], ct) for n, ct in (
            ("final_scores", C.c_float), ("final_raw_scores", C.c_float), ("final_lengths", C.c_int32),
            ("tokens", C.c_int32), ("parents", C.c_int32), ("lengths", C.c_int32), ("scores", C.c_float),
            ("raw_scores", C.c_float), ("from_logprob", C.c_uint8))))
        steps_a = None if steps is None else np.ascontiguousarray(np.asarray(steps, np.int32))
        cons = None if constraints is None else C.byref(constraints)
        if ex:
            o = OutputsExC()
            o.base = base
            if row_lse:
                o.row_lse = _p(out["row_lse"], C.c_float)
            if pool:
                for name, _, ct in pool_keys:
                    setattr(o, name, _p(out[name], ct))
            status = self.lib.dbs_decode_batch_into_ex(h, x.ctypes.data_as(C.c_void_p), DTYPES[dtype],
                                                       int(bool(from_logits)), B, T, V, _p(steps_a, C.c_int32), cons,
                                                       0, C.byref(o))
        else:
            assert dtype == "f32" and not from_logits
            status = self.lib.dbs_decode_batch_into(h, _p(x, C.c_float), B, T, V, _p(steps_a, C.c_int32), cons, 0,
                                                    C.byref(base))
        return status, out

    def backward(self, h, trace: dict, V: int, initial: np.ndarray, *, steps=None, ex=True, grad_final=None,
                 grad_final_raw=None, grad_scores=None, grad_raw=None, logits=None, logits_dtype="f32",
                 row_lse=None, pool=None, grad_pool_scores=None, grad_pool_raw=None) -> tuple[int, np.ndarray]:
        """dbs_backward_batch_into_ex (or, ex=False, dbs_backward_batch_into
        with the final-score gradient) accumulating into a copy of
        `initial`; `pool` holds a relaxed pool's trace (pool_parents,
        pool_tokens, pool_lengths, pool_from_logprob [B, T, P]) for the pool
        gradients. Returns (status, gradient)."""
        keep = {}

        def arr(name, a, dt):
            if a is None:
                return None
            keep[name] = np.ascontiguousarray(np.asarray(a, dt))
            return keep[name]

        par = arr("par", trace["parents"], np.int32)
        B, T, K = par.shape
        tok = arr("tok", trace["tokens"], np.int32)
        ln = arr("len", trace["lengths"], np.int32)
        flp = arr("flp", trace["from_logprob"], np.uint8)
        st = arr("steps", steps, np.int32)
        grad = np.ascontiguousarray(np.array(initial, np.float32, copy=True))
        if not ex:
            gf = arr("gf", grad_final, np.float32)
            status = self.lib.dbs_backward_batch_into(h, B, T, V, _p(st, C.c_int32), _p(par, C.c_int32),
                                                      _p(tok, C.c_int32), _p(ln, C.c_int32), _p(flp, C.c_uint8),
                                                      _p(gf, C.c_float), 0, _p(grad, C.c_float))
            return status, grad
        inp = BackwardInputsC()
        inp.batch_size, inp.steps, inp.vocab_size, inp.pool_size = B, T, V, 0
        inp.steps_per_example = _p(st, C.c_int32)
        inp.parents, inp.tokens = _p(par, C.c_int32), _p(tok, C.c_int32)
        inp.lengths, inp.from_logprob = _p(ln, C.c_int32), _p(flp, C.c_uint8)
        for name, field, g in (("gf", "grad_final_scores", grad_final), ("gfr", "grad_final_raw_scores",
                                                                        grad_final_raw),
                               ("gs", "grad_scores", grad_scores), ("gr", "grad_raw_scores", grad_raw),
                               ("gps", "grad_pool_scores", grad_pool_scores),
                               ("gpr", "grad_pool_raw_scores", grad_pool_raw)):
            setattr(inp, field, _p(arr(name, g, np.float32), C.c_float))
        if pool is not None:
            inp.pool_size = int(pool["pool_parents"].shape[-1])
            inp.pool_parents = _p(arr("pp", pool["pool_parents"], np.int32), C.c_int32)
            inp.pool_tokens = _p(arr("pt", pool["pool_tokens"], np.int32), C.c_int32)
            inp.pool_lengths = _p(arr("pl", pool["pool_lengths"], np.int32), C.c_int32)
            inp.pool_from_logprob = _p(arr("pf", pool["pool_from_logprob"], np.uint8), C.c_uint8)
        if logits is not None:
            keep["logits"] = np.ascontiguousarray(logits)
            inp.logits = keep["logits"].ctypes.data_as(C.c_void_p)
            inp.logits_type = DTYPES[logits_dtype]
            inp.row_lse = _p(arr("lse", row_lse, np.float32), C.c_float)
        status = self.lib.dbs_backward_batch_into_ex(h, C.byref(inp), 0, _p(grad, C.c_float))
        return status, grad


# ---------------------------------------------------------------------------
# Result handles, backward handles and model-step decodes
# ---------------------------------------------------------------------------

class StatsC(C.Structure):
    _fields_ = [("abi_version", C.c_int), ("last_kernel", C.c_int), ("used_sparse_backward", C.c_int),
                ("used_dense_backward", C.c_int), ("used_batch_threads", C.c_int),
                ("used_model_step_callback", C.c_int), ("last_error_category", C.c_int),
                ("last_decode_ns", C.c_int64), ("last_backward_ns", C.c_int64), ("last_allocation_bytes", C.c_int64),
                ("last_selected_count", C.c_int64), ("last_pool_count", C.c_int64),
                ("last_logprob_count", C.c_int64), ("last_sparse_grad_count", C.c_int64),
                ("total_allocator_calls", C.c_int64), ("total_allocator_bytes", C.c_int64),
                ("reserved_stats0", C.c_int64), ("reserved_stats1", C.c_int64)]


class StepInfoC(C.Structure):
    _fields_ = [("batch_index", C.c_int), ("step", C.c_int), ("beam_size", C.c_int), ("vocab_size", C.c_int),
                ("parents", _i32p), ("tokens", _i32p), ("lengths", _i32p), ("scores", _f32p),
                ("raw_scores", _f32p), ("finished", _u8p), ("prefixes", _i32p), ("reserved", C.c_void_p * 4)]


STEP_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, _i32p, _f32p, C.c_int, C.c_int, _f32p)
STEP_EX_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(StepInfoC), _f32p)

_RESULT_I32 = ("tokens", "parents", "lengths")
_RESULT_F32 = ("scores", "raw_scores", "weights")


def _declare_results(L):
    vp, i = C.c_void_p, C.c_int
    sig = {
        "dbs_decode": (i, [vp, _f32p, i, i, C.POINTER(vp)]),
        "dbs_decode_typed": (i, [vp, vp, i, i, i, C.POINTER(vp)]),
        "dbs_decode_batch_typed": (i, [vp, vp, i, i, i, i, i, C.POINTER(vp)]),
        "dbs_decode_constrained": (i, [vp, _f32p, i, i, _u8p, _i32p, i, C.POINTER(vp)]),
        "dbs_decode_constrained_ex": (i, [vp, _f32p, i, i, C.POINTER(ConstraintsC), C.POINTER(vp)]),
        "dbs_decode_batch": (i, [vp, _f32p, i, i, i, i, C.POINTER(vp)]),
        "dbs_decode_batch_variable": (i, [vp, _f32p, i, i, i, i, _i32p, _i32p, _i32p, _i32p, _u8p, _i32p, i,
                                          C.POINTER(vp)]),
        "dbs_decode_model_steps": (i, [vp, STEP_FN, vp, i, i, i, C.POINTER(vp)]),
        "dbs_decode_model_steps_with_workspace": (i, [vp, vp, STEP_FN, vp, i, i, i, C.POINTER(vp)]),
        "dbs_decode_model_steps_ex": (i, [vp, STEP_EX_FN, vp, i, i, i, C.POINTER(ConstraintsC), C.POINTER(vp)]),
        "dbs_backward": (i, [vp, vp, _f32p, _f32p, _f32p, C.POINTER(vp)]),
        "dbs_backward_dense": (i, [vp, vp, _f32p, _f32p, _f32p, C.POINTER(vp)]),
        "dbs_backward_sparse": (i, [vp, vp, _f32p, _f32p, _f32p, C.POINTER(vp)]),
        "dbs_backward_default": (i, [vp, vp, _f32p, _f32p, _f32p, C.POINTER(vp)]),
        "dbs_free_result": (None, [vp]),
        "dbs_free_batch_result": (None, [vp]),
        "dbs_free_backward": (None, [vp]),
        "dbs_batch_result_size": (i, [vp]),
        "dbs_batch_result_at": (vp, [vp, i]),
        "dbs_result_steps": (i, [vp]),
        "dbs_result_beam_size": (i, [vp]),
        "dbs_result_vocab_size": (i, [vp]),
        "dbs_result_pool_size": (i, [vp]),
        "dbs_result_final_scores": (_f32p, [vp]),
        "dbs_result_final_raw_scores": (_f32p, [vp]),
        "dbs_result_relaxed_weights": (_f32p, [vp]),
        "dbs_result_pool_tokens": (_i32p, [vp]),
        "dbs_result_pool_parents": (_i32p, [vp]),
        "dbs_result_pool_lengths": (_i32p, [vp]),
        "dbs_result_pool_scores": (_f32p, [vp]),
        "dbs_result_pool_raw_scores": (_f32p, [vp]),
        "dbs_backward_grad_log_probs": (_f32p, [vp]),
        "dbs_backward_grad_initial_scores": (_f32p, [vp]),
        "dbs_backward_sparse_logprob_indices": (C.POINTER(C.c_int64), [vp]),
        "dbs_backward_sparse_logprob_values": (_f32p, [vp]),
        "dbs_backward_sparse_logprob_count": (C.c_int64, [vp]),
        "dbs_backward_is_sparse": (i, [vp]),
        "dbs_result_selected_count": (C.c_int64, [vp]),
        "dbs_result_pool_count": (C.c_int64, [vp]),
        "dbs_result_logprob_count": (C.c_int64, [vp]),
        "dbs_backward_grad_log_probs_count": (C.c_int64, [vp]),
        "dbs_backward_grad_initial_scores_count": (C.c_int64, [vp]),
        "dbs_result_eos_count": (C.c_int64, [vp, i]),
        "dbs_result_validate_deterministic_order": (i, [vp]),
        "dbs_result_summary_json": (i, [vp, i, C.c_char_p, C.c_int64]),
        "dbs_get_stats": (i, [vp, C.POINTER(StatsC)]),
        "dbs_get_stats_json": (i, [vp, C.c_char_p, C.c_int64]),
        "dbs_reset_stats": (None, [vp]),
        "dbs_is_deterministic": (i, []),
        "dbs_set_deterministic_seed": (i, [vp, C.c_uint64]),
        "dbs_get_deterministic_seed": (C.c_uint64, [vp]),
        "dbs_workspace_create": (i, [C.POINTER(vp)]),
        "dbs_workspace_destroy": (None, [vp]),
        "dbs_workspace_reserve": (i, [vp, C.c_int64, C.c_int64]),
        "dbs_workspace_allocated_bytes": (C.c_int64, [vp]),
    }
    for name in _RESULT_I32:
        sig[f"dbs_result_{name}"] = (_i32p, [vp])
    for name in _RESULT_F32:
        sig[f"dbs_result_{name}"] = (_f32p, [vp])
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _copy(ptr, n, dt):
    if not ptr or n == 0:
        return None
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dt, copy=True)


def read_result(L, r) -> dict:
    """Every accessor of a result handle, copied out."""
    T, K, V = L.dbs_result_steps(r), L.dbs_result_beam_size(r), L.dbs_result_vocab_size(r)
    out = {"steps": T, "beam_size": K, "vocab_size": V, "pool_size": L.dbs_result_pool_size(r)}
    for name in _RESULT_I32:
        out[name] = _copy(getattr(L, f"dbs_result_{name}")(r), T * K, np.int32)
    for name in _RESULT_F32:
        out[name] = _copy(getattr(L, f"dbs_result_{name}")(r), T * K, np.float32)
    out["final_scores"] = _copy(L.dbs_result_final_scores(r), K, np.float32)
    out["final_raw_scores"] = _copy(L.dbs_result_final_raw_scores(r), K, np.float32)
    out["relaxed_weights_null"] = not L.dbs_result_relaxed_weights(r)
    out["pool_tokens_null"] = not L.dbs_result_pool_tokens(r)
    P = out["pool_size"]
    if P > 0:
        for name in ("pool_tokens", "pool_parents", "pool_lengths"):
            out[name] = _copy(getattr(L, f"dbs_result_{name}")(r), T * P, np.int32)
        for name in ("pool_scores", "pool_raw_scores", "relaxed_weights"):
            out[name] = _copy(getattr(L, f"dbs_result_{name}")(r), T * P, np.float32)
    out["counts"] = (L.dbs_result_selected_count(r), L.dbs_result_pool_count(r), L.dbs_result_logprob_count(r),
                     L.dbs_backward_grad_log_probs_count(r), L.dbs_backward_grad_initial_scores_count(r))
    out["order"] = L.dbs_result_validate_deterministic_order(r)
    return out


def read_backward(L, b, n_dense: int, K: int) -> dict:
    """Every accessor of a backward handle, copied out."""
    count = L.dbs_backward_sparse_logprob_count(b)
    return {"is_sparse": L.dbs_backward_is_sparse(b),
            "dense": _copy(L.dbs_backward_grad_log_probs(b), n_dense, np.float32),
            "initial": _copy(L.dbs_backward_grad_initial_scores(b), K, np.float32),
            "count": count,
            "indices": _copy(L.dbs_backward_sparse_logprob_indices(b), count, np.int64),
            "values": _copy(L.dbs_backward_sparse_logprob_values(b), count, np.float32)}


def enable_results(host: "HostLib") -> "HostLib":
    _declare_results(host.lib)
    return host
