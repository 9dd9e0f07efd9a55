# SPDX-License-Identifier: MIT
"""dbs_hip_decode_noalloc: the decode of dbs_hip_decode_ex3 with its
workspace in a static device array instead of an allocation. Checked bit for
bit against dbs_hip_decode_ex3 (and the oracle) on calls in a row that reuse
the same array, each smaller than the one before, and its size limit."""

import ctypes as C

import numpy as np
import pytest
import torch

from beamgrad_amd import _abi
from tests.cases import first_difference, make_case, to_bits

pytestmark = pytest.mark.gpu


def _same(hip, oracle, xin, dtype, **kw):
    want = hip.decode(xin, dtype, use_ex3=True, **kw)
    got = hip.decode(xin, dtype, noalloc=True, **kw)
    assert first_difference(got, want) is None
    assert first_difference(got, oracle.decode(xin, dtype=dtype, **kw)) is None


def test_noalloc_matches_ex3_twice_second_smaller(hip, oracle):
    rng = np.random.default_rng(2024)
    V = 151936
    x = rng.normal(0.0, 3.0, size=(3, 6, 8, V)).astype(np.float32)
    x += (-1.1 * np.log(rng.permutation(V) + 1.0)).astype(np.float32)
    _same(hip, oracle, to_bits(x, "bf16"), "bf16", from_logits=True, eos_token=V - 9, min_length=2, alpha=1.0)
    # second call, smaller, on the array the first one left behind
    y = rng.normal(0.0, 2.0, size=(2, 4, 3, 1000)).astype(np.float32)
    _same(hip, oracle, y, "f32", from_logits=True, eos_token=5, alpha=0.6)


@pytest.mark.parametrize("seed", range(6))
def test_noalloc_matches_ex3_random(hip, oracle, seed):
    """Random options (constraints, banned masks, per-example steps) on
    consecutive calls of shrinking size."""
    for i, big in enumerate((True, False)):
        case = make_case(8800 + 10 * seed + i, big=big)
        _same(hip, oracle, case["xin"], case["dtype"], **case["kw"])


def test_noalloc_per_example_arrays(hip, oracle):
    case = make_case(8900, allow_invalid=False)
    B, K = case["B"], case["K"]
    beams = [max(1, K - b) for b in range(B)]
    kw = dict(case["kw"])
    want = hip.decode(case["xin"], case["dtype"], use_ex3=True, beams=beams, **kw)
    got = hip.decode(case["xin"], case["dtype"], noalloc=True, beams=beams, **kw)
    assert first_difference(got, want) is None


def test_noalloc_rejects_beyond_its_scratch(hip):
    lib = hip.lib
    args = _abi.DecodeArgs()
    args.batch_size, args.steps, args.beam_size, args.vocab_size = 32, 64, 64, 32000
    args.eos_token, args.repetition_penalty = -1, 1.0
    need = lib.dbs_cuda_decode_workspace_size(C.byref(args))
    assert need > _abi.NOALLOC_SCRATCH_BYTES
    dummy = torch.zeros(16, dtype=torch.float32, device="cuda")  # never read: nothing is launched
    out = _abi.DecodeOutputs(_abi.ptr(dummy), None, None, None, None, None, None, None, None, None)
    status = lib.dbs_hip_decode_noalloc(_abi.ptr(dummy), _abi.DTYPE["f32"], 0, C.byref(args), None, None,
                                        C.byref(out), None, hip.stream())
    assert status == _abi.STATUS_SCRATCH_LIMIT
    assert b"static scratch" in lib.dbs_cuda_status_string(status)
    # and a decode within the limit still runs afterwards
    case = make_case(8950)
    got = hip.decode(case["xin"], case["dtype"], noalloc=True, **case["kw"])
    want = hip.decode(case["xin"], case["dtype"], use_ex3=True, **case["kw"])
    assert first_difference(got, want) is None
