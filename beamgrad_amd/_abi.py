# SPDX-License-Identifier: MIT
"""ctypes declarations of libdbs_hip's C ABI (include/dbs_cuda.h and
include/dbs_hip.h), for callers that drive the engine without the torch
operators: the C-ABI parity tests and the benchmark use it with device
pointers from torch tensors and torch's current HIP stream.

The structures mirror the reference's device ABI field for field (reference
include/dbs_cuda.h:69-100, 145-154, 239-253, 274-284).
"""

from __future__ import annotations

import ctypes as C
import os

from . import _build

_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)

STATUS_OK = 0
STATUS_UNAVAILABLE = 1
STATUS_INVALID_ARGUMENT = 2
STATUS_LAUNCH_FAILED = 3
STATUS_OUT_OF_MEMORY = 4
STATUS_SCRATCH_LIMIT = 5  # dbs_hip_decode_noalloc: the decode needs more than its static scratch
NOALLOC_SCRATCH_BYTES = 64 * 1024 * 1024
MAX_BEAM = 1024
MAX_EXTRA_EOS = 16
DTYPE = {"f32": 0, "f16": 1, "bf16": 2}
GRAD_TYPE = {"f32": 0, "f16": 1, "bf16": 2}


class DecodeArgs(C.Structure):
    _fields_ = [
        ("batch_size", C.c_int), ("steps", C.c_int), ("beam_size", C.c_int), ("vocab_size", C.c_int),
        ("eos_token", C.c_int), ("min_length", C.c_int), ("length_penalty_alpha", C.c_float),
        ("no_repeat_ngram_size", C.c_int), ("repetition_penalty", C.c_float), ("reserved0", C.c_int),
        ("steps_per_example", C.c_void_p), ("beam_sizes_per_example", C.c_void_p),
        ("eos_tokens_per_example", C.c_void_p), ("min_lengths_per_example", C.c_void_p),
        ("banned_tokens", C.c_void_p),
    ]


class DecodeOutputs(C.Structure):
    _fields_ = [
        ("final_scores", C.c_void_p), ("final_raw_scores", C.c_void_p), ("final_lengths", C.c_void_p),
        ("tokens", C.c_void_p), ("parents", C.c_void_p), ("lengths", C.c_void_p), ("scores", C.c_void_p),
        ("raw_scores", C.c_void_p), ("from_logprob", C.c_void_p), ("invalid_input", C.c_void_p),
    ]


class BeamState(C.Structure):
    _fields_ = [
        ("raw_scores", C.c_void_p), ("lengths", C.c_void_p), ("finished", C.c_void_p), ("prefixes", C.c_void_p),
        ("prefix_stride", C.c_int), ("reserved0", C.c_int),
    ]


class BackwardInputs(C.Structure):
    _fields_ = [
        ("parents", C.c_void_p), ("tokens", C.c_void_p), ("lengths", C.c_void_p), ("from_logprob", C.c_void_p),
        ("grad_final_scores", C.c_void_p), ("grad_final_raw_scores", C.c_void_p), ("grad_scores", C.c_void_p),
        ("grad_raw_scores", C.c_void_p), ("logits", C.c_void_p), ("logits_type", C.c_int), ("reserved0", C.c_int),
        ("row_lse", C.c_void_p), ("reserved", C.c_void_p * 4),
    ]


class SearchOptions(C.Structure):
    _fields_ = [
        ("extra_eos_count", C.c_int), ("extra_eos_tokens", C.c_int32 * MAX_EXTRA_EOS), ("reserved0", C.c_int),
        ("reserved", C.c_void_p * 4),
    ]


# name -> (restype, argtypes) for every entry point of include/dbs_cuda.h and include/dbs_hip.h
SIGNATURES = {
    "dbs_cuda_available": (C.c_int, []),
    "dbs_cuda_status_string": (C.c_char_p, [C.c_int]),
    "dbs_cuda_set_synchronization": (C.c_int, [C.c_int]),
    "dbs_cuda_get_synchronization": (C.c_int, []),
    "dbs_cuda_decode_workspace_size": (C.c_int64, [C.POINTER(DecodeArgs)]),
    "dbs_cuda_backward_workspace_size": (C.c_int64, [C.POINTER(DecodeArgs)]),
    "dbs_cuda_decode": (C.c_int, [C.c_void_p, C.POINTER(DecodeArgs), C.POINTER(DecodeOutputs), C.c_void_p,
                                  C.c_int64, C.c_void_p]),
    "dbs_cuda_decode_step_workspace_size": (C.c_int64, [C.POINTER(DecodeArgs), C.c_int]),
    "dbs_cuda_decode_step": (C.c_int, [C.c_void_p, C.POINTER(DecodeArgs), C.POINTER(BeamState),
                                       C.POINTER(DecodeOutputs), C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_cuda_backward": (C.c_int, [C.POINTER(DecodeArgs), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                    C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_cuda_decode_ex": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs), C.POINTER(DecodeOutputs),
                                     C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_cuda_decode_step_ex": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs), C.POINTER(BeamState),
                                          C.POINTER(DecodeOutputs), C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_cuda_backward_ex": (C.c_int, [C.POINTER(DecodeArgs), C.POINTER(BackwardInputs), C.c_void_p, C.c_void_p,
                                       C.c_int64, C.c_void_p]),
    "dbs_cuda_decode_ex2": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs), C.POINTER(SearchOptions),
                                      C.POINTER(DecodeOutputs), C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_cuda_decode_step_ex2": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs),
                                           C.POINTER(SearchOptions), C.POINTER(BeamState), C.POINTER(DecodeOutputs),
                                           C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_cuda_length_penalty": (C.c_int, [C.c_void_p, C.c_int64, C.c_float, C.c_void_p, C.c_void_p]),
    "dbs_cuda_path_gradient": (C.c_int, [C.POINTER(DecodeArgs), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_void_p, C.c_void_p]),
    "dbs_hip_decode_ex3": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs), C.POINTER(SearchOptions),
                                     C.c_void_p, C.POINTER(DecodeOutputs), C.c_void_p, C.c_void_p, C.c_int64,
                                     C.c_void_p]),
    "dbs_hip_decode_ex4": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs), C.POINTER(SearchOptions),
                                     C.c_void_p, C.POINTER(DecodeOutputs), C.c_void_p, C.c_void_p, C.c_int64,
                                     C.POINTER(C.c_void_p), C.c_void_p]),
    "dbs_hip_decode_read_back": (C.c_int, [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p]),
    "dbs_hip_search_sequences": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                           C.c_void_p, C.c_void_p]),
    "dbs_hip_minimum_risk": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float, C.c_int, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p]),
    "dbs_hip_decode_noalloc": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.POINTER(DecodeArgs),
                                         C.POINTER(SearchOptions), C.c_void_p, C.POINTER(DecodeOutputs), C.c_void_p,
                                         C.c_void_p]),
    "dbs_hip_backward_dense": (C.c_int, [C.POINTER(DecodeArgs), C.POINTER(BackwardInputs), C.c_void_p, C.c_int,
                                         C.c_void_p, C.c_int64, C.c_void_p]),
    "dbs_hip_backtrack": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                    C.c_void_p]),
    "dbs_hip_widen_trace": (C.c_int, [C.c_void_p] * 6 + [C.c_int] * 3 + [C.c_void_p] * 7),
    "dbs_hip_backtrack_i64": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                        C.c_void_p]),
    "dbs_hip_profile_enable": (C.c_int, [C.c_int]),
    "dbs_hip_profile_read": (C.c_int, [C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    "dbs_hip_set_row_pass": (C.c_int, [C.c_int]),
    "dbs_hip_set_decode_overlap": (C.c_int, [C.c_int]),
    "dbs_hip_set_select_pass": (C.c_int, [C.c_int]),
}


def load(path: str | None = None) -> C.CDLL:
    """Loads libdbs_hip.so with typed entry points. Import torch first in a
    process that uses both, so that one HIP runtime serves them."""
    path = path or _build.lib_path()
    if not os.path.exists(path):
        raise OSError(f"{path} is not built; run `python -m beamgrad_amd._build`")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def ptr(t) -> C.c_void_p | None:
    """Device (or host) address of a torch tensor, or None."""
    return None if t is None else C.c_void_p(t.data_ptr())
