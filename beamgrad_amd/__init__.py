# SPDX-License-Identifier: MIT
"""beamgrad_amd: differentiable beam search on AMD Instinct MI355X (gfx950).

A drop-in for beamgrad's GPU path: the same Python API (``decode``,
``final_scores``, ``backtrack``, ``search``, ``beam_search``,
``length_penalty``, ``losses``) and the same ``torch.ops.beamgrad`` operators,
served by hand-written HIP kernels in ``libdbs_hip`` (whose C ABI is the
reference's ``dbs_cuda.h``).

The public names load on first use. Importing the package itself loads
nothing, so ``beamgrad_amd._C_hip`` (the operators' HIP kernels) can be
imported on its own beside another package that owns the operators and
their Python registrations (the reference's ``_C`` and ``_torch.py``).
"""

from __future__ import annotations

import importlib

__version__ = "0.1.0"

# public name -> the module that defines it
_PUBLIC = {
    "BeamOptions": "._options",
    "CUDA_MAX_BEAM": "._options",
    "BeamSearchResult": "._search",
    "BeamState": "._search",
    "beam_search": "._search",
    "search": "._search",
    "sequence_scores": "._search",
    "BeamSearchOutput": "._torch",
    "backtrack": "._torch",
    "cuda_available": "._torch",
    "decode": "._torch",
    "final_scores": "._torch",
    "length_penalty": "._torch",
}

__all__ = sorted([*_PUBLIC, "losses", "__version__"])


def __getattr__(name: str):
    if name == "losses":
        value = importlib.import_module(".losses", __name__)
    elif name in _PUBLIC:
        value = getattr(importlib.import_module(_PUBLIC[name], __name__), name)
    else:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    globals()[name] = value
    return value


def __dir__():
    return sorted(set(globals()) | set(__all__))
