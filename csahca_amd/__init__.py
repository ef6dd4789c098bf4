"""csahca_amd -- MI355X-native (gfx950) compressed-sparse-attention decode.

Drop-in replacement for the CSAHCA reference's native op surface
(``hybrid_attention_cuda`` behind ``hybrid_attention.extension``): hand-written
HIP kernels behind a C ABI (``include/csahca.h``, ``libcsahca.so``), bound to
PyTorch tensors by :mod:`csahca_amd.native` and wrapped with the reference's
Python signatures in :mod:`csahca_amd.extension`.
"""
from __future__ import annotations

__version__ = "0.1.0"
