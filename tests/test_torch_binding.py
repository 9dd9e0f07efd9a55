# SPDX-License-Identifier: MIT
"""The torch binding as a drop-in for the reference's operator modules.

The reference splits its operators in two: ``_C`` owns the namespace
(``TORCH_LIBRARY(beamgrad)``, python/csrc/cpu_ops.cpp:582-608) and
``_C_cuda`` only registers CUDA-key kernels
(``TORCH_LIBRARY_IMPL(beamgrad, CUDA)``, python/csrc/cuda_ops.cpp:484-492),
loaded in that order by python/beamgrad/_torch.py:53-64. Ours mirrors it:
``beamgrad_amd._C`` defines the same seven schemas and ``beamgrad_amd._C_hip``
adds the HIP kernels plus a fragment with this build's own operators, so it
loads beside any definition of the namespace. torch ends the process when a
namespace is defined twice, so the load-order checks run in subprocesses.
"""

import os
import re
import subprocess
import sys
import textwrap

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_OPS = "/root/reference/python/csrc/cpu_ops.cpp"
OUR_SCHEMAS = os.path.join(ROOT, "beamgrad_amd", "csrc", "torch_schemas.cpp")
REFERENCE_OPS = ("decode", "final_scores_backward", "length_penalty", "final_scores_path_gradient", "decode_step",
                 "decode_ex", "decode_backward")


def schema_texts(path):
    """The schema strings of every ``m.def(...)`` in a C++ source (adjacent
    string literals joined), in order."""
    src = open(path).read()
    out = []
    for call in re.finditer(r"m\.def\(\s*((?:\"(?:[^\"\\]|\\.)*\"\s*)+)\)", src):
        out.append("".join(re.findall(r"\"((?:[^\"\\]|\\.)*)\"", call.group(1))))
    return out


def run_python(code, timeout=180):
    env = dict(os.environ, PYTHONPATH=ROOT + os.pathsep + os.environ.get("PYTHONPATH", ""))
    return subprocess.run([sys.executable, "-c", textwrap.dedent(code)], capture_output=True, text=True,
                          timeout=timeout, cwd=ROOT, env=env)


# defines the namespace from Python with the given schemas, as the
# reference's _C does from C++ (both are a Library of kind DEF)
_FOREIGN_DEF = """
import torch
_owner = torch.library.Library("beamgrad", "DEF")
for _s in {schemas!r}:
    _owner.define(_s)
"""


def test_our_schemas_are_the_references_text():
    ours = schema_texts(OUR_SCHEMAS)
    assert [s.split("(")[0] for s in ours] == list(REFERENCE_OPS)
    if not os.path.exists(REF_OPS):
        pytest.skip("the reference is not mounted here")
    theirs = schema_texts(REF_OPS)
    assert ours == theirs


def test_registered_schemas_parse_to_the_references():
    import torch

    import beamgrad_amd as bg

    bg.decode  # noqa: B018  loads the operators
    texts = schema_texts(REF_OPS) if os.path.exists(REF_OPS) else schema_texts(OUR_SCHEMAS)
    for text in texts:
        name = text.split("(")[0]
        want = torch._C.parse_schema("beamgrad::" + text)
        got = getattr(torch.ops.beamgrad, name).default._schema
        assert str(got) == str(want), name
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"beamgrad::{name}", "CUDA"), name
    for name in ("decode_trace", "decode_backward_as", "backtrack"):
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"beamgrad::{name}", "CUDA"), name


def test_impl_module_loads_beside_a_foreign_definition():
    code = _FOREIGN_DEF.format(schemas=schema_texts(OUR_SCHEMAS)) + """
import sys
import beamgrad_amd._C_hip as hip_ops
assert "beamgrad_amd._torch" not in sys.modules  # the package's registrations stayed out
assert hip_ops.device_available() in (False, True)
for name in {ops!r} + ("decode_trace", "decode_backward_as", "backtrack"):
    assert torch._C._dispatch_has_kernel_for_dispatch_key("beamgrad::" + name, "CUDA"), name
print("LOADED")
""".format(ops=REFERENCE_OPS)
    res = run_python(code)
    assert res.returncode == 0 and "LOADED" in res.stdout, res.stderr[-2000:]


def test_package_uses_a_foreign_definition():
    """The Python front end finds the namespace defined and loads only the
    kernels; its fake implementations then serve shape-only tracing."""
    code = _FOREIGN_DEF.format(schemas=schema_texts(OUR_SCHEMAS)) + """
import beamgrad_amd as bg
bg.decode  # the front end: kernels, fakes, autograd
from torch._subclasses.fake_tensor import FakeTensorMode
with FakeTensorMode():
    x = torch.empty(2, 3, 4, 50, dtype=torch.bfloat16)
    out = torch.ops.beamgrad.decode_ex(x, True, None, -1, 0, 0.0, None, 0, 1.0, True, [])
assert tuple(out[3].shape) == (2, 3, 4) and out[3].dtype == torch.int32
print("FAKE_OK", bg.cuda_available() in (False, True))
"""
    res = run_python(code)
    assert res.returncode == 0 and "FAKE_OK" in res.stdout, res.stderr[-2000:]


def test_second_definition_still_aborts():
    """Control for the two tests above: loading our schema owner after a
    foreign definition is the abort they guard against (the package's
    loader therefore skips it)."""
    code = _FOREIGN_DEF.format(schemas=schema_texts(OUR_SCHEMAS)) + """
import beamgrad_amd._C
print("SHOULD_NOT_PRINT")
"""
    res = run_python(code)
    assert res.returncode != 0 and "SHOULD_NOT_PRINT" not in res.stdout
    assert "Only a single TORCH_LIBRARY" in res.stderr


@pytest.mark.gpu
def test_impl_kernels_beside_a_foreign_definition_match_the_oracle():
    """The seven reference operators dispatched to _C_hip's kernels while
    another library owns the namespace, checked bit for bit against the CPU
    oracle (decode_ex from bf16 logits, the dense backward, the path
    gradient)."""
    out_path = os.path.join(ROOT, "gpurun_out", "binding_check.npz")
    os.makedirs(os.path.dirname(out_path), exist_ok=True)
    code = _FOREIGN_DEF.format(schemas=schema_texts(OUR_SCHEMAS)) + f"""
import numpy as np
import beamgrad_amd._C_hip  # the kernels only
gen = torch.Generator(device="cuda").manual_seed(11)
B, T, K, V = 3, 5, 4, 777
x = (torch.randn(B, T, K, V, device="cuda", generator=gen) * 3.0).to(torch.bfloat16)
out = torch.ops.beamgrad.decode_ex(x, True, None, 7, 1, 0.5, None, 0, 1.0, True, [])
g = torch.rand(B, K, device="cuda", generator=gen)
par, tok, ln, flp = out[4], out[3], out[5], out[8]
grad = torch.ops.beamgrad.decode_backward(g, None, None, None, par, tok, ln, flp, None, V, 0.5, x, out[9])
draws = torch.ops.beamgrad.final_scores_path_gradient(g, par, tok, ln, flp, None, V, 0.5)
np.savez({out_path!r}, x=x.view(torch.int16).cpu().numpy(), g=g.cpu().numpy(),
         **{{k: v.cpu().numpy() for k, v in zip(("final_scores", "final_raw_scores", "final_lengths", "tokens",
                                                "parents", "lengths", "scores", "raw_scores", "from_logprob",
                                                "row_lse"), out)}},
         grad=grad.cpu().numpy(), draws=draws.cpu().numpy())
print("RAN")
"""
    res = run_python(code)
    assert res.returncode == 0 and "RAN" in res.stdout, res.stderr[-2000:]
    from oracle.oracle import Oracle

    got = np.load(out_path)
    bits = got["x"].view(np.uint16)
    orc = Oracle()
    want = orc.decode(bits, dtype="bf16", from_logits=True, eos_token=7, min_length=1, alpha=0.5)
    for key in ("final_scores", "final_raw_scores", "final_lengths", "tokens", "parents", "lengths", "scores",
                "raw_scores", "from_logprob", "row_lse"):
        a, b = got[key], want[key]
        if a.dtype.kind == "f":
            assert np.array_equal(a.view(np.uint32), b.astype(np.float32).view(np.uint32)), key
        else:
            assert np.array_equal(a.astype(np.int64), b.astype(np.int64)), key
    grad_want = orc.backward(want, 777, alpha=0.5, grad_final=got["g"], logits=bits, logits_dtype="bf16",
                             row_lse=want["row_lse"])
    assert np.array_equal(got["grad"].view(np.uint32), grad_want.view(np.uint32))
    draws_want = orc.path_gradient(want, 777, got["g"], alpha=0.5)
    assert np.array_equal(got["draws"].view(np.uint32), draws_want.view(np.uint32))
