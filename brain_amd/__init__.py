"""brain_amd — MI355X (gfx950) int8 W8A8 matmul backend for swedishembedded/brain.

The product is the C-ABI library libbrain_hip.so (include/brain_hip.h):
hand-written HIP kernels for per-token activation quantization, the decode
GEMV and the prefill GEMM on the int8 matrix cores, plus a C mirror of brain's
`backend_api::Backend` dispatch trait. This package loads that library
(`_lib`), offers torch-tensor wrappers of the typed calls (`ops`) and a thin
object wrapper of the Backend mirror (`backend`).
"""
from ._lib import BrainHipError, load  # noqa: F401

__all__ = ["BrainHipError", "load"]
