"""hybrid_attention_cuda -- the module name the CSAHCA reference imports for its
native ops (hybrid_attention/extension.py:19-23), served by the gfx950 HIP
library through csahca_amd.native.

Put this directory on sys.path (or PYTHONPATH) and the reference's
`load_cuda_extension()` returns this module; its five ops keep the pybind
signatures of csrc/bindings.cpp:54-164.  Importing fails loudly (RuntimeError from the native
loader) when libcsahca.so has not been built: there is no CPU fallback.
"""
from csahca_amd.native import (  # noqa: F401
    csa_chunk_summary,
    csa_decode_forward,
    csa_decode_forward_tiled,
    csa_decode_step,
    csa_select_topk,
    dsv4_decode_forward_tiled,
    dsv4_sparse_decode_forward,
    dsv4_swa_decode_forward,
    hca_decode_forward,
    hybrid_decode_forward,
    lib as _lib,
)

_lib()

__all__ = [
    "csa_decode_forward",
    "csa_decode_forward_tiled",
    "dsv4_swa_decode_forward",
    "dsv4_sparse_decode_forward",
    "dsv4_decode_forward_tiled",
    "csa_chunk_summary",
    "csa_select_topk",
    "csa_decode_step",
    "hca_decode_forward",
    "hybrid_decode_forward",
]
