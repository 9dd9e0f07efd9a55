# SPDX-License-Identifier: MIT
"""CPU checks of the drop-in boundary: libdbs_hip.so loads and exports every
entry point include/*.h declares; the structures keep the reference's layout
(compiled from the headers with gcc, and from the reference's own header when
it is mounted); host-only entry points (statuses, synchronization flag,
workspace sizes, argument validation) behave as the reference's do. No kernel
is launched."""

import ctypes as C
import os
import re
import subprocess

import pytest

from beamgrad_amd import _abi, _build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
REF_HEADER = "/root/reference/include/dbs_cuda.h"


def declared_symbols() -> list[str]:
    names = []
    for header in ("dbs_cuda.h", "dbs_hip.h"):
        text = open(os.path.join(INCLUDE, header)).read()
        names += re.findall(r"DBS_CUDA_EXPORT\s+[\w\s\*]+?\b(dbs_\w+)\s*\(", text)
    return names


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_build.lib_path()):
        pytest.skip("libdbs_hip.so is not built (run __graft_entry__.build())")
    return _abi.load()


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) == 32  # 17 reference entry points + 15 additions
    out = subprocess.run(["nm", "-D", "--defined-only", _build.lib_path()], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (dbs_\w+)", out))
    host = re.findall(r"DBS_EXPORT\s+[\w\s\*]+?\b(dbs_\w+)\s*\(", open(os.path.join(INCLUDE, "dbs.h")).read())
    assert set(names) | set(host) == exported  # the device ABI, its additions and the host ABI
    for name in names:
        assert hasattr(lib, name)
    assert set(_abi.SIGNATURES) == set(names)


def test_reference_entry_points_all_present():
    # the 17 functions of the reference's device ABI (reference include/dbs_cuda.h:102-334)
    ref17 = {"dbs_cuda_available", "dbs_cuda_status_string", "dbs_cuda_set_synchronization",
             "dbs_cuda_get_synchronization", "dbs_cuda_decode_workspace_size", "dbs_cuda_backward_workspace_size",
             "dbs_cuda_decode", "dbs_cuda_decode_step_workspace_size", "dbs_cuda_decode_step", "dbs_cuda_backward",
             "dbs_cuda_decode_ex", "dbs_cuda_decode_step_ex", "dbs_cuda_backward_ex", "dbs_cuda_decode_ex2",
             "dbs_cuda_decode_step_ex2", "dbs_cuda_length_penalty", "dbs_cuda_path_gradient"}
    assert ref17 <= set(declared_symbols())


LAYOUT_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "dbs_cuda.h"
#define F(s, f) printf(#s "." #f " %zu\n", offsetof(s, f));
int main(void) {
  printf("DBSCudaDecodeArgs %zu\n", sizeof(DBSCudaDecodeArgs));
  F(DBSCudaDecodeArgs, repetition_penalty) F(DBSCudaDecodeArgs, steps_per_example) F(DBSCudaDecodeArgs, banned_tokens)
  printf("DBSCudaDecodeOutputs %zu\n", sizeof(DBSCudaDecodeOutputs));
  F(DBSCudaDecodeOutputs, invalid_input)
  printf("DBSCudaBeamState %zu\n", sizeof(DBSCudaBeamState));
  F(DBSCudaBeamState, prefix_stride)
  printf("DBSCudaBackwardInputs %zu\n", sizeof(DBSCudaBackwardInputs));
  F(DBSCudaBackwardInputs, logits_type) F(DBSCudaBackwardInputs, row_lse) F(DBSCudaBackwardInputs, reserved)
  printf("DBSCudaSearchOptions %zu\n", sizeof(DBSCudaSearchOptions));
  F(DBSCudaSearchOptions, reserved0) F(DBSCudaSearchOptions, reserved)
  printf("consts %d %d %d %d\n", DBS_CUDA_MAX_BEAM, DBS_CUDA_MAX_EXTRA_EOS, DBS_CUDA_DTYPE_BF16, DBS_CUDA_STATUS_OUT_OF_MEMORY);
  return 0;
}
"""


def _layout(include_dir: str, tmp_path) -> dict:
    src = tmp_path / "probe.c"
    src.write_text(LAYOUT_PROBE)
    exe = tmp_path / f"probe_{abs(hash(include_dir))}"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{include_dir}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) if not line.startswith("consts") else ("consts", line[7:])
                for line in out.strip().splitlines())


def test_layout_matches_ctypes_mirror(tmp_path):
    lay = _layout(INCLUDE, tmp_path)
    assert int(lay["DBSCudaDecodeArgs"]) == C.sizeof(_abi.DecodeArgs)
    assert int(lay["DBSCudaDecodeOutputs"]) == C.sizeof(_abi.DecodeOutputs)
    assert int(lay["DBSCudaBeamState"]) == C.sizeof(_abi.BeamState)
    assert int(lay["DBSCudaBackwardInputs"]) == C.sizeof(_abi.BackwardInputs)
    assert int(lay["DBSCudaSearchOptions"]) == C.sizeof(_abi.SearchOptions)
    assert int(lay["DBSCudaDecodeArgs.banned_tokens"]) == _abi.DecodeArgs.banned_tokens.offset
    assert int(lay["DBSCudaBackwardInputs.row_lse"]) == _abi.BackwardInputs.row_lse.offset
    assert lay["consts"] == "1024 16 2 4"


@pytest.mark.skipif(not os.path.exists(REF_HEADER), reason="reference not mounted")
def test_layout_matches_reference_header(tmp_path):
    ours = _layout(INCLUDE, tmp_path)
    theirs = _layout(os.path.dirname(REF_HEADER), tmp_path)
    assert ours == theirs


def test_host_entry_points(lib):
    assert lib.dbs_cuda_status_string(0) == b"ok"
    assert lib.dbs_cuda_status_string(2) == b"invalid argument"
    assert lib.dbs_cuda_set_synchronization(2) == _abi.STATUS_INVALID_ARGUMENT
    assert lib.dbs_cuda_set_synchronization(1) == 0 and lib.dbs_cuda_get_synchronization() == 1
    assert lib.dbs_cuda_set_synchronization(0) == 0 and lib.dbs_cuda_get_synchronization() == 0

    args = _abi.DecodeArgs()
    args.batch_size, args.steps, args.beam_size, args.vocab_size = 32, 64, 8, 151936
    args.eos_token, args.repetition_penalty = 151643, 1.0
    assert lib.dbs_cuda_decode_workspace_size(C.byref(args)) > 0
    assert lib.dbs_cuda_backward_workspace_size(C.byref(args)) > 0
    bad = _abi.DecodeArgs.from_buffer_copy(args)
    bad.beam_size = 1025  # above DBS_CUDA_MAX_BEAM
    assert lib.dbs_cuda_decode_workspace_size(C.byref(bad)) < 0
    bad = _abi.DecodeArgs.from_buffer_copy(args)
    bad.eos_token = 151936  # outside the vocabulary
    assert lib.dbs_cuda_decode_workspace_size(C.byref(bad)) < 0
    bad = _abi.DecodeArgs.from_buffer_copy(args)
    bad.reserved0 = 1
    assert lib.dbs_cuda_decode_workspace_size(C.byref(bad)) < 0
    # step workspace needs steps == 1
    assert lib.dbs_cuda_decode_step_workspace_size(C.byref(args), 0) < 0
    one = _abi.DecodeArgs.from_buffer_copy(args)
    one.steps = 1
    assert lib.dbs_cuda_decode_step_workspace_size(C.byref(one), 16) > 0
    # null inputs and outputs are rejected before any device work
    out = _abi.DecodeOutputs()
    assert lib.dbs_cuda_decode_ex2(None, 2, 1, C.byref(args), None, C.byref(out), None, None, 0, None) == 2
    assert lib.dbs_cuda_decode_ex2(C.c_void_p(1), 7, 1, C.byref(args), None, C.byref(out), None, None, 0, None) == 2
    assert lib.dbs_cuda_backward_ex(C.byref(args), None, None, None, 0, None) == 2
    assert lib.dbs_cuda_length_penalty(None, -1, 1.0, None, None) == 2
    assert lib.dbs_hip_profile_enable(3) == 2
    assert lib.dbs_hip_set_row_pass(6) == -2
    assert lib.dbs_hip_set_row_pass(4) == -2  # no longer a kernel
    assert lib.dbs_hip_set_row_pass(-1) == -1  # automatic is the default
    assert lib.dbs_hip_set_row_pass(-1) == -1
    assert lib.dbs_hip_set_decode_overlap(2) == -2
    assert lib.dbs_hip_set_decode_overlap(-1) == -1  # automatic by default
