# SPDX-License-Identifier: MIT
"""CPU checks of the libdbs host C ABI (include/dbs.h) served by
libdbs_hip.so: every declared function is exported, the structures keep the
reference header's layout (gcc probes), and every argument error that is
decided before any device work gives the reference library's status and
message (oracle/_ref/libdbs_ref.so, called with identical arguments). No
kernel is launched."""

import os
import re
import subprocess

import numpy as np
import pytest

from beamgrad_amd import _build
from tests.host_abi import ConstraintsC, HostLib, OptionsC, OutputsC, OutputsExC, BackwardInputsC

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
REF_INCLUDE = "/root/reference/include"
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libdbs_ref.so")


def declared() -> list[str]:
    text = open(os.path.join(INCLUDE, "dbs.h")).read()
    return re.findall(r"DBS_EXPORT\s+[\w\s\*]+?\b(dbs_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def ours():
    if not os.path.exists(_build.lib_path()):
        pytest.skip("libdbs_hip.so is not built (run __graft_entry__.build())")
    import torch  # noqa: F401  (one HIP runtime for torch and the library)

    return HostLib(_build.lib_path())


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref is not built")
    return HostLib(REF_LIB)


def test_declared_host_functions_are_exported(ours):
    names = declared()
    assert {"dbs_decode_batch_into", "dbs_decode_batch_into_ex", "dbs_backward_batch_into",
            "dbs_backward_batch_into_ex", "dbs_create_ex", "dbs_destroy"} <= set(names)
    out = subprocess.run(["nm", "-D", "--defined-only", _build.lib_path()], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (dbs_\w+)", out))
    assert set(names) <= exported


@pytest.mark.skipif(not os.path.exists(REF_INCLUDE), reason="reference not mounted")
def test_declarations_match_the_reference_header():
    """Each declaration of include/dbs.h names a function of the reference's
    header with the same parameter list (whitespace aside)."""
    def decls(path):
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        found = {}
        for m in re.finditer(r"DBS_EXPORT\s+([\w\s\*]+?)\b(dbs_\w+)\s*\(([^;]*?)\)\s*;", text, re.S):
            found[m.group(2)] = (" ".join(m.group(1).split()), " ".join(m.group(3).replace("\n", " ").split()))
        return found

    theirs = decls(os.path.join(REF_INCLUDE, "dbs.h"))
    for name, sig in decls(os.path.join(INCLUDE, "dbs.h")).items():
        assert name in theirs, name
        assert sig == theirs[name], name


PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "dbs.h"
#define S(s) printf(#s " %zu\n", sizeof(s));
#define F(s, f) printf(#s "." #f " %zu\n", offsetof(s, f));
int main(void) {
  S(DBSOptionsC) F(DBSOptionsC, eos_token) F(DBSOptionsC, length_penalty_alpha) F(DBSOptionsC, min_length)
  F(DBSOptionsC, validate_inputs) F(DBSOptionsC, max_dense_gradient_elements) F(DBSOptionsC, reserved1)
  S(DBSAdvancedConstraintsC) F(DBSAdvancedConstraintsC, forced_tokens) F(DBSAdvancedConstraintsC, min_length)
  F(DBSAdvancedConstraintsC, repetition_penalty) F(DBSAdvancedConstraintsC, no_repeat_ngram_size)
  F(DBSAdvancedConstraintsC, token_filter) F(DBSAdvancedConstraintsC, batch_index)
  S(DBSDecodeOutputsC) F(DBSDecodeOutputsC, tokens) F(DBSDecodeOutputsC, from_logprob)
  S(DBSDecodeOutputsExC) F(DBSDecodeOutputsExC, pool_parents) F(DBSDecodeOutputsExC, row_lse)
  F(DBSDecodeOutputsExC, reserved)
  S(DBSBackwardInputsC) F(DBSBackwardInputsC, steps_per_example) F(DBSBackwardInputsC, grad_final_scores)
  F(DBSBackwardInputsC, logits) F(DBSBackwardInputsC, logits_type) F(DBSBackwardInputsC, row_lse)
  F(DBSBackwardInputsC, reserved)
  printf("consts %d %d %d %d %d %d\n", DBS_ABI_VERSION, DBS_OK, DBS_ERROR_INVALID_ARGUMENT, DBS_ERROR_RUNTIME,
         DBS_ERROR_UNKNOWN, (int)DBS_DTYPE_BF16);
  return 0;
}
"""


def _probe(include_dir, tmp_path):
    src = tmp_path / "probe_dbs.c"
    src.write_text(PROBE)
    exe = tmp_path / f"probe_dbs_{abs(hash(include_dir))}"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{include_dir}", str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout


def test_layout_matches_ctypes_mirror(tmp_path):
    import ctypes as C

    lines = dict(line.rsplit(" ", 1) for line in _probe(INCLUDE, tmp_path).strip().splitlines()
                 if not line.startswith("consts"))
    for name, cls in (("DBSOptionsC", OptionsC), ("DBSAdvancedConstraintsC", ConstraintsC),
                      ("DBSDecodeOutputsC", OutputsC), ("DBSDecodeOutputsExC", OutputsExC),
                      ("DBSBackwardInputsC", BackwardInputsC)):
        assert int(lines[name]) == C.sizeof(cls), name
    assert int(lines["DBSBackwardInputsC.row_lse"]) == BackwardInputsC.row_lse.offset
    assert int(lines["DBSOptionsC.max_dense_gradient_elements"]) == OptionsC.max_dense_gradient_elements.offset


@pytest.mark.skipif(not os.path.exists(REF_INCLUDE), reason="reference not mounted")
def test_layout_matches_reference_header(tmp_path):
    assert _probe(INCLUDE, tmp_path) == _probe(REF_INCLUDE, tmp_path)


def test_versions(ours, ref):
    assert ours.lib.dbs_abi_version() == ref.lib.dbs_abi_version() == 10
    assert ours.lib.dbs_version_string() == ref.lib.dbs_version_string()
    assert ours.lib.dbs_selected_kernel_name() == b"hip-gfx950"


BAD_OPTIONS = [dict(beam_size=-1), dict(eos_token=-2), dict(selected_temperature=-1.0),
               dict(soft_topk_temperature=float("nan")), dict(relaxed_pool_multiplier=-1), dict(vocab_block=-3),
               dict(length_penalty_alpha=-0.5), dict(length_penalty_alpha=float("inf")),
               dict(soft_topk_tolerance=-1.0), dict(soft_topk_max_iters=-1), dict(min_length=-1),
               dict(max_dense_gradient_elements=-5)]


@pytest.mark.parametrize("opts", BAD_OPTIONS)
def test_create_rejects_what_the_reference_rejects(ours, ref, opts):
    from tests.host_abi import HostError

    errs = []
    for lib in (ours, ref):
        with pytest.raises(HostError) as e:
            lib.create(**opts)
        errs.append((e.value.status, e.value.message))
    assert errs[0] == errs[1]


def test_extra_eos_errors_match(ours, ref):
    for lib in (ours, ref):
        h = lib.create(beam_size=2, eos_token=-1)
        try:
            assert lib.set_extra_eos(h, [3]) == -1
            assert "need EOS handling" in lib.error()
        finally:
            lib.destroy(h)
    msgs = []
    for lib in (ours, ref):
        h = lib.create(beam_size=2, eos_token=1)
        try:
            msgs.append((lib.set_extra_eos(h, [-4]), lib.error()))
            msgs.append((lib.set_extra_eos(h, [2, 5]), lib.error()))
            msgs.append((lib.set_extra_eos(h, []), lib.error()))
        finally:
            lib.destroy(h)
    assert msgs[:3] == msgs[3:]


def _both(ours, ref, call, **opts):
    """The same failing call on both libraries: (status, message) pairs."""
    res = []
    for lib in (ours, ref):
        h = lib.create(**opts)
        try:
            status = call(lib, h)
            res.append((status, lib.error()))
        finally:
            lib.destroy(h)
    return res


DECODE_ERRORS = {
    "eos outside vocabulary": (dict(beam_size=2, eos_token=9), dict()),
    "steps_per_example out of range": (dict(beam_size=2), dict(steps=[1, 4])),
    "steps_per_example zero": (dict(beam_size=2), dict(steps=[0, 1])),
    "infinite repetition penalty": (dict(beam_size=2), dict(rep=float("inf"))),
    "bad dtype": (dict(beam_size=2), dict(dtype=5)),
    "forced token outside vocabulary": (dict(beam_size=2), dict(forced=[9, -1, -1])),
    # the shared array as far as each example's steps read it: example 1 fails
    "forced token outside vocabulary, second example": (dict(beam_size=2), dict(forced=[1, -1, 9], steps=[2, 3])),
}


@pytest.mark.parametrize("case", sorted(DECODE_ERRORS))
def test_decode_argument_errors_match(ours, ref, case):
    import ctypes as C

    opts, kw = DECODE_ERRORS[case]
    x = np.zeros((2, 3, 2, 9), np.float32)

    def call(lib, h):
        keep = {}
        cons = None
        if "rep" in kw or "forced" in kw:
            cons = HostLib.constraints(repetition_penalty=kw.get("rep", 1.0), forced=kw.get("forced"), keep=keep)
        if "dtype" in kw:
            o = OutputsExC()
            fs = np.zeros((2, 2), np.float32)
            o.base.final_scores = fs.ctypes.data_as(C.POINTER(C.c_float))
            return lib.lib.dbs_decode_batch_into_ex(h, x.ctypes.data_as(C.c_void_p), kw["dtype"], 0, 2, 3, 9, None,
                                                    None, 0, C.byref(o))
        status, _ = lib.decode(h, x, 2, steps=kw.get("steps"), constraints=cons)
        return status

    a, b = _both(ours, ref, call, **opts)
    assert a == b
    assert a[0] == -1


def test_decode_null_and_shape_errors_match(ours, ref):
    import ctypes as C

    x = np.zeros((1, 2, 2, 5), np.float32)
    fs = np.zeros((1, 2), np.float32)
    results = []
    for lib in (ours, ref):
        h = lib.create(beam_size=2)
        try:
            L = lib.lib
            base = OutputsC()
            base.final_scores = fs.ctypes.data_as(C.POINTER(C.c_float))
            got = []
            got.append((L.dbs_decode_batch_into(None, x.ctypes.data_as(C.POINTER(C.c_float)), 1, 2, 5, None, None, 0,
                                                C.byref(base)), lib.error()))
            got.append((L.dbs_decode_batch_into(h, None, 1, 2, 5, None, None, 0, C.byref(base)), lib.error()))
            got.append((L.dbs_decode_batch_into(h, x.ctypes.data_as(C.POINTER(C.c_float)), 1, 2, 5, None, None, 0,
                                                None), lib.error()))
            got.append((L.dbs_decode_batch_into(h, x.ctypes.data_as(C.POINTER(C.c_float)), 0, 2, 5, None, None, 0,
                                                C.byref(base)), lib.error()))
            got.append((L.dbs_decode_batch_into_ex(h, x.ctypes.data_as(C.c_void_p), 0, 0, 1, 2, 5, None, None, 0,
                                                   None), lib.error()))
            o = OutputsExC()
            o.base = base
            o.reserved[1] = 1
            got.append((L.dbs_decode_batch_into_ex(h, x.ctypes.data_as(C.c_void_p), 0, 0, 1, 2, 5, None, None, 0,
                                                   C.byref(o)), lib.error()))
            o = OutputsExC()
            o.base = base
            pool = np.zeros(8, np.int32)
            o.pool_tokens = pool.ctypes.data_as(C.POINTER(C.c_int32))
            got.append((L.dbs_decode_batch_into_ex(h, x.ctypes.data_as(C.c_void_p), 0, 0, 1, 2, 5, None, None, 0,
                                                   C.byref(o)), lib.error()))
            results.append(got)
        finally:
            lib.destroy(h)
    assert results[0] == results[1]
    assert all(s == -1 for s, _ in results[0])


def test_backward_argument_errors_match(ours, ref):
    import ctypes as C

    B, T, K, V = 2, 3, 2, 7
    good = dict(parents=np.zeros((B, T, K), np.int32), tokens=np.zeros((B, T, K), np.int32),
                lengths=np.ones((B, T, K), np.int32), from_logprob=np.ones((B, T, K), np.uint8))
    bad_tok = dict(good, tokens=np.full((B, T, K), V, np.int32))
    bad_par = dict(good, parents=np.full((B, T, K), K, np.int32))
    gf = np.ones((B, K), np.float32)
    init = np.zeros((B, T, K, V), np.float32)

    def calls(lib, h):
        got = []
        for trace, steps in ((bad_tok, None), (bad_par, None), (good, [0, 2]), (good, [1, 9])):
            got.append((lib.backward(h, trace, V, init, steps=steps, grad_final=gf, ex=False)[0], lib.error()))
            got.append((lib.backward(h, trace, V, init, steps=steps, grad_final=gf)[0], lib.error()))
        inp = BackwardInputsC()
        got.append((lib.lib.dbs_backward_batch_into_ex(h, C.byref(inp), 0, None), lib.error()))
        inp.batch_size, inp.steps, inp.vocab_size = B, T, V
        got.append((lib.lib.dbs_backward_batch_into_ex(h, C.byref(inp), 0, init.ctypes.data_as(
            C.POINTER(C.c_float))), lib.error()))
        # logits without row_lse
        keep = {k: np.ascontiguousarray(v) for k, v in good.items()}
        inp.parents = keep["parents"].ctypes.data_as(C.POINTER(C.c_int32))
        inp.tokens = keep["tokens"].ctypes.data_as(C.POINTER(C.c_int32))
        inp.lengths = keep["lengths"].ctypes.data_as(C.POINTER(C.c_int32))
        inp.from_logprob = keep["from_logprob"].ctypes.data_as(C.POINTER(C.c_uint8))
        inp.logits = init.ctypes.data_as(C.c_void_p)
        got.append((lib.lib.dbs_backward_batch_into_ex(h, C.byref(inp), 0, init.ctypes.data_as(
            C.POINTER(C.c_float))), lib.error()))
        inp.logits_type = 9
        got.append((lib.lib.dbs_backward_batch_into_ex(h, C.byref(inp), 0, init.ctypes.data_as(
            C.POINTER(C.c_float))), lib.error()))
        return got

    res = []
    for lib in (ours, ref):
        h = lib.create(beam_size=K)
        try:
            res.append(calls(lib, h))
        finally:
            lib.destroy(h)
    assert res[0] == res[1]
    assert all(s == -1 for s, _ in res[0])


def test_features_the_engine_does_not_serve_are_refused(ours):
    """Relaxed pools and beams beyond the device ABI's limits are refused
    with INVALID_ARGUMENT before any device work (the reference's CPU
    library serves them)."""
    h = ours.create(beam_size=300, relaxed_pool_multiplier=4)
    try:
        st, _ = ours.decode(h, np.zeros((1, 1, 300, 3), np.float32), 300, pool=1200)
        assert st == -1 and "relaxed pool of 1200 candidates" in ours.error()
    finally:
        ours.destroy(h)
    h = ours.create(beam_size=1025)
    try:
        st, _ = ours.decode(h, np.zeros((1, 1, 1025, 3), np.float32), 1025)
        assert st == -1 and "beyond the HIP engine" in ours.error()
    finally:
        ours.destroy(h)


REF_SYMBOLS = "/root/reference/abi/libdbs.symbols"


@pytest.mark.skipif(not os.path.exists(REF_SYMBOLS), reason="reference not mounted")
def test_exported_host_symbols_are_the_references():
    """The host functions libdbs_hip.so exports are exactly the reference's
    81 (its abi/libdbs.symbols, the list its scripts/check_abi.sh checks);
    the device ABI (dbs_cuda_*) and its additions (dbs_hip_*) come on top."""
    out = subprocess.run(["nm", "-D", "--defined-only", _build.lib_path()], capture_output=True, text=True,
                         check=True).stdout
    host = {n for n in re.findall(r" T (dbs_\w+)", out) if not n.startswith(("dbs_cuda_", "dbs_hip_"))}
    want = set(open(REF_SYMBOLS).read().split())
    assert len(want) == 81
    assert host == want
    assert set(declared()) == want


STATS_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "dbs.h"
#define S(s) printf(#s " %zu\n", sizeof(s));
#define F(s, f) printf(#s "." #f " %zu\n", offsetof(s, f));
int main(void) {
  S(DBSStatsC) F(DBSStatsC, last_error_category) F(DBSStatsC, last_decode_ns) F(DBSStatsC, total_allocator_bytes)
  F(DBSStatsC, reserved_stats1)
  S(DBSModelStepInfoC) F(DBSModelStepInfoC, parents) F(DBSModelStepInfoC, finished) F(DBSModelStepInfoC, prefixes)
  F(DBSModelStepInfoC, reserved)
  return 0;
}
"""


def test_result_structs_layout(tmp_path):
    """DBSStatsC and DBSModelStepInfoC: our header against the ctypes
    mirror, and against the reference header where it is mounted."""
    import ctypes as C

    from tests.host_abi import StatsC, StepInfoC

    def probe(include_dir):
        src = tmp_path / "probe_stats.c"
        src.write_text(STATS_PROBE)
        exe = tmp_path / f"probe_stats_{abs(hash(include_dir))}"
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{include_dir}", str(src), "-o", str(exe)],
                       check=True)
        return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout

    ours = probe(INCLUDE)
    lines = dict(line.rsplit(" ", 1) for line in ours.strip().splitlines())
    assert int(lines["DBSStatsC"]) == C.sizeof(StatsC)
    assert int(lines["DBSModelStepInfoC"]) == C.sizeof(StepInfoC)
    assert int(lines["DBSModelStepInfoC.prefixes"]) == StepInfoC.prefixes.offset
    if os.path.exists(REF_INCLUDE):
        assert ours == probe(REF_INCLUDE)
