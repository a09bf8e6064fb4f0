"""scao_amd -- the SCAO optimizer step on AMD Instinct MI355X (gfx950).

A drop-in for ``scao`` (whispering3/scao): ``scao_amd.SCAO`` has the
reference optimizer's constructor, param-group keys, state layout and
phase behaviour; its step runs as batched hand-written HIP kernels
(``scao_amd/csrc``) behind the C ABI in ``include/scao_amd.h``.
"""

from .optimizer import SCAO, scao_sub1b, scao_1b, scao_3b, scao_7b, scao_40b, scao_125b
from .preconditioner import SparsePreconditioner
from .utils import matrix_power_neg_quarter, adaptive_rank
from . import logging as scao_logging

__version__ = "0.2.0"

__all__ = [
    "SCAO",
    "scao_sub1b", "scao_1b", "scao_3b", "scao_7b", "scao_40b", "scao_125b",
    "SparsePreconditioner",
    "matrix_power_neg_quarter",
    "adaptive_rank",
    "scao_logging",
    "__version__",
]
