# SPDX-License-Identifier: MIT
"""beamgrad_amd: differentiable beam search on AMD Instinct MI355X (gfx950).

A drop-in for beamgrad's GPU path: the same Python API (``decode``,
``final_scores``, ``backtrack``, ``search``, ``beam_search``,
``length_penalty``, ``losses``) and the same ``torch.ops.beamgrad`` operators,
served by hand-written HIP kernels in ``libdbs_hip`` (whose C ABI is the
reference's ``dbs_cuda.h``).
"""

from . import losses
from ._options import CUDA_MAX_BEAM, BeamOptions
from ._search import BeamSearchResult, BeamState, beam_search, search, sequence_scores
from ._torch import BeamSearchOutput, backtrack, cuda_available, decode, final_scores, length_penalty

__version__ = "0.1.0"

__all__ = [
    "BeamOptions",
    "BeamSearchOutput",
    "BeamSearchResult",
    "BeamState",
    "CUDA_MAX_BEAM",
    "__version__",
    "backtrack",
    "beam_search",
    "cuda_available",
    "decode",
    "final_scores",
    "length_penalty",
    "losses",
    "search",
    "sequence_scores",
]
