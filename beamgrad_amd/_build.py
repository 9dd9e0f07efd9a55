# SPDX-License-Identifier: MIT
"""In-tree build of the native parts of beamgrad_amd for gfx950.

* ``_lib/libdbs_hip.so``: the HIP engine and its C ABIs (include/dbs_cuda.h,
  include/dbs_hip.h, and the host ABI include/dbs.h), compiled by hipcc for
  gfx950 only;
* ``_C*.so``: defines the torch.ops.beamgrad operator schemas (the
  namespace's owner, no kernels);
* ``_C_hip*.so``: the operators' HIP kernels (CUDA dispatch key) and this
  build's additional operators, linked against libdbs_hip.

Run ``python -m beamgrad_amd._build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# Device numerics must be the reference's bit for bit: no FMA contraction, no
# fast math, IEEE f32 division, denormals kept; packed FP32 instructions off.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

LIB_SOURCES = ["csrc/api.hip", "csrc/host_abi.cpp", "csrc/host_results.cpp", "csrc/decode.hip", "csrc/row_pass.hip", "csrc/row_resident.hip",
               "csrc/row_pipe.hip", "csrc/row_logprob.hip", "csrc/row_relay.hip", "csrc/select.hip", "csrc/backward.hip"]


def lib_path() -> str:
    return os.path.join(HERE, "_lib", "libdbs_hip.so")


def ext_path(name: str = "_C_hip") -> str:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return os.path.join(HERE, name + suffix)


def _run(cmd: list[str]) -> None:
    print("[beamgrad_amd build]", " ".join(cmd[:3]), "...", flush=True)
    subprocess.run(cmd, check=True, cwd=HERE)


def build_lib() -> str:
    """Compiles each source to an object in parallel (one hipcc per source),
    then links the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = os.path.join(HERE, "_lib", "obj")
    os.makedirs(objdir, exist_ok=True)
    out = lib_path()
    objs = [os.path.join(objdir, os.path.splitext(os.path.basename(src))[0] + ".o") for src in LIB_SOURCES]

    def compile_one(src_obj):
        src, obj = src_obj
        _run([HIPCC, *HIP_FLAGS, "-fvisibility=hidden", f"-I{ROOT}/include", f"-I{HERE}/csrc", "-c", src,
              "-o", obj])

    jobs = max(1, min(len(LIB_SOURCES), int(os.environ.get("MAX_JOBS", "0") or 0) or (os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(compile_one, zip(LIB_SOURCES, objs)))
    # -Bsymbolic: the library's own calls stay inside it even where another
    # library exporting the same dbs_* names is loaded first
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-Bsymbolic", *objs, "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def _torch_module(name: str, source: str, hip: bool) -> str:
    """One torch extension module compiled by g++: ``name`` from ``source``;
    with ``hip`` it links libdbs_hip and torch's HIP libraries."""
    import torch
    from torch.utils import cpp_extension as ce

    incs = ce.include_paths(device_type="cuda")
    libdirs = ce.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    py_inc = sysconfig.get_paths()["include"]
    out = ext_path(name)
    libs = ["-lc10", "-ltorch", "-ltorch_cpu"]
    if hip:
        libs = [f"-L{os.path.join(HERE, '_lib')}", "-ldbs_hip", *[f"-L{p}" for p in libdirs], *libs, "-lc10_hip",
                "-ltorch_hip", "-Wl,-rpath,$ORIGIN/_lib"]
    else:
        libs = [*[f"-L{p}" for p in libdirs], *libs]
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM=1", "-D__HIP_PLATFORM_AMD__=1",
        f"-DTORCH_EXTENSION_NAME={name}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        *[f"-I{p}" for p in incs], f"-I{py_inc}", f"-I{ROOT}/include", f"-I{ROCM}/include",
        source, *libs, "-o", out + ".tmp",
    ]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build_ext() -> list[str]:
    """The schema owner ``_C`` and the HIP kernels ``_C_hip``."""
    return [_torch_module("_C", "csrc/torch_schemas.cpp", hip=False),
            _torch_module("_C_hip", "csrc/torch_ops.cpp", hip=True)]


def build() -> None:
    build_lib()
    build_ext()


if __name__ == "__main__":
    build()
    sys.exit(0)
