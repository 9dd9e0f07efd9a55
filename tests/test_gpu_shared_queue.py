# SPDX-License-Identifier: MIT
"""The overlapped decode on streams that share one hardware queue.

HIP maps its streams onto a few hardware queues per process
(GPU_MAX_HW_QUEUES, 4 by default) and shares a queue between streams once
there are more of them; two streams on one queue run their launches in
submission order. The overlapped decode puts its select pass on a second
stream, and with a row pass of one workgroup per row the select pass is
submitted first: its waits must never depend on a launch queued behind it.
It is split in two launches around the row pass (an early one that takes an
example only once its first row is counted, a late one that takes the rest).

A child process with GPU_MAX_HW_QUEUES=1 (every stream on one queue) runs
overlapped decodes of both row-pass kinds (one workgroup per row and
persistent), constrained and not, against the oracle, and checks that no
wait gave up."""

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import ctypes as C
import sys
import numpy as np
import torch
sys.path.insert(0, ROOT)
from tests.hip_abi import HipEngine
from tests.cases import first_difference, make_case
from oracle.oracle import Oracle

hip, oracle = HipEngine(), Oracle()
lib = hip.lib
lib.dbs_hip_set_decode_overlap(1)
lib.dbs_hip_profile_enable(1)
cases = [make_case(8100 + i, vocabs=[1000, 3000], allow_invalid=False) for i in range(4)]
cases += [make_case(8200 + i, vocabs=[4096, 20000], dtypes=["bf16", "f16"], logits=True, allow_invalid=False)
          for i in range(3)]
for i, case in enumerate(cases):
    kw = dict(case["kw"])
    if i % 2:
        kw["no_repeat_ngram_size"], kw["repetition_penalty"] = 2, 1.2
    print("case", case["seed"], case["B"], case["T"], case["K"], case["V"], case["dtype"], flush=True)
    got = hip.decode(case["xin"], case["dtype"], **kw)
    want = oracle.decode(case["xin"], dtype=case["dtype"], **kw)
    diff = first_difference(got, want)
    assert diff is None, (case["seed"], diff)
ms, n = C.c_double(), C.c_int64()
assert lib.dbs_hip_profile_read(6, C.byref(ms), C.byref(n)) == 0
assert n.value == 0, f"{n.value} waits of the overlapped decode gave up"
print("ok", flush=True)
"""


def test_overlapped_decode_on_one_hardware_queue():
    env = dict(os.environ, GPU_MAX_HW_QUEUES="1")
    proc = subprocess.run([sys.executable, "-c", f"ROOT = {ROOT!r}\n" + CHILD], env=env, cwd=ROOT,
                          capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0 and proc.stdout.rstrip().endswith("ok"), (proc.stdout[-2000:], proc.stderr[-3000:])
