"""Python op wrappers with the reference's signatures (hybrid_attention/extension.py).

Same function names, argument order, defaults and environment flags as the
reference module, backed by the gfx950 library instead of the CUDA extension:

* ``load_cuda_extension()`` returns the native op module (:mod:`csahca_amd.native`),
  building it with hipcc first only when ``HYBRID_ATTENTION_JIT=1``
  (hybrid_attention/extension.py:13-45); otherwise a missing library raises.
* ``csa_decode_forward`` / ``csa_decode_forward_tiled`` make every tensor
  contiguous (:48-81).
* ``dsv4_swa_decode_forward`` / ``dsv4_sparse_decode_forward`` view caches as
  uint8, cast indices/lengths to int32 and the sink to fp32, substitute empty
  tensors for None and route to the tiled op unless ``CSAHCA_DSV4_TILED`` is
  falsey, with ``CSAHCA_DSV4_TILE_SIZE`` (0 = automatic) (:84-197).
"""
from __future__ import annotations

import os
from types import ModuleType

import torch

_CUDA_MODULE: ModuleType | None = None


def load_cuda_extension() -> ModuleType:
    """Return the native op module (loading libcsahca.so)."""
    global _CUDA_MODULE
    if _CUDA_MODULE is not None:
        return _CUDA_MODULE
    from . import native

    if not native.library_path().exists():
        if os.environ.get("HYBRID_ATTENTION_JIT", "0") != "1":
            raise RuntimeError(
                "HIP extension is not built. Run `python -m csahca_amd.build` "
                "on the MI355X machine, or set HYBRID_ATTENTION_JIT=1 for a local build.")
        from .build import build

        build()
    native.lib()
    _CUDA_MODULE = native
    return _CUDA_MODULE


def csa_decode_forward(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                       selected_chunks: torch.Tensor, chunk_size: int) -> torch.Tensor:
    module = load_cuda_extension()
    return module.csa_decode_forward(q.contiguous(), k_cache.contiguous(), v_cache.contiguous(),
                                     selected_chunks.contiguous(), int(chunk_size))


def csa_decode_forward_tiled(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             selected_chunks: torch.Tensor, chunk_size: int, tile_size: int = 8) -> torch.Tensor:
    module = load_cuda_extension()
    return module.csa_decode_forward_tiled(q.contiguous(), k_cache.contiguous(), v_cache.contiguous(),
                                           selected_chunks.contiguous(), int(chunk_size), int(tile_size))


def _dsv4_tiled_enabled(module: ModuleType) -> bool:
    if os.environ.get("CSAHCA_DSV4_TILED", "1").strip().lower() in {"", "0", "false", "no", "off"}:
        return False
    return hasattr(module, "dsv4_decode_forward_tiled")


def _dsv4_tile_size() -> int:
    try:
        return int(os.environ.get("CSAHCA_DSV4_TILE_SIZE", "0"))
    except ValueError:
        return 0


def dsv4_swa_decode_forward(q: torch.Tensor, paged_k_cache: torch.Tensor, token_indices: torch.Tensor,
                            topk_lengths: torch.Tensor | None, attn_sink: torch.Tensor | None, page_size: int,
                            softmax_scale: float) -> torch.Tensor:
    """DSV4 decode over the SWA paged FP8 cache (compress_ratio 0).  The cache may
    be a uint8 tensor or a float8 view of the same bytes."""
    module = load_cuda_extension()
    cache_u8 = paged_k_cache.contiguous().view(torch.uint8)
    if topk_lengths is None:
        topk_lengths = torch.empty(0, dtype=torch.int32, device=q.device)
    if attn_sink is None:
        attn_sink = torch.empty(0, dtype=torch.float32, device=q.device)
    if _dsv4_tiled_enabled(module):
        return module.dsv4_decode_forward_tiled(
            q.contiguous(), cache_u8, token_indices.contiguous().to(torch.int32),
            topk_lengths.contiguous().to(torch.int32),
            torch.empty((0, 0), dtype=torch.uint8, device=q.device),
            torch.empty((0, 0), dtype=torch.int32, device=q.device),
            torch.empty(0, dtype=torch.int32, device=q.device),
            attn_sink.contiguous().to(torch.float32), int(page_size), 1, _dsv4_tile_size(), float(softmax_scale))
    return module.dsv4_swa_decode_forward(
        q.contiguous(), cache_u8, token_indices.contiguous().to(torch.int32),
        topk_lengths.contiguous().to(torch.int32), attn_sink.contiguous().to(torch.float32), int(page_size),
        float(softmax_scale))


def dsv4_sparse_decode_forward(q: torch.Tensor, paged_k_cache: torch.Tensor, token_indices: torch.Tensor,
                               topk_lengths: torch.Tensor | None, extra_paged_k_cache: torch.Tensor,
                               extra_token_indices: torch.Tensor, extra_topk_lengths: torch.Tensor | None,
                               attn_sink: torch.Tensor | None, page_size: int, extra_page_size: int,
                               softmax_scale: float) -> torch.Tensor:
    """DSV4 decode over the SWA cache plus C4/C128 compressed cache pages."""
    module = load_cuda_extension()
    cache_u8 = paged_k_cache.contiguous().view(torch.uint8)
    extra_cache_u8 = extra_paged_k_cache.contiguous().view(torch.uint8)
    if topk_lengths is None:
        topk_lengths = torch.empty(0, dtype=torch.int32, device=q.device)
    if extra_topk_lengths is None:
        extra_topk_lengths = torch.empty(0, dtype=torch.int32, device=q.device)
    if attn_sink is None:
        attn_sink = torch.empty(0, dtype=torch.float32, device=q.device)
    args = (q.contiguous(), cache_u8, token_indices.contiguous().to(torch.int32),
            topk_lengths.contiguous().to(torch.int32), extra_cache_u8,
            extra_token_indices.contiguous().to(torch.int32), extra_topk_lengths.contiguous().to(torch.int32),
            attn_sink.contiguous().to(torch.float32), int(page_size), int(extra_page_size))
    if _dsv4_tiled_enabled(module):
        return module.dsv4_decode_forward_tiled(*args, _dsv4_tile_size(), float(softmax_scale))
    return module.dsv4_sparse_decode_forward(*args, float(softmax_scale))


# New ops (no reference counterpart): the selection kernels and the fused step.
def csa_chunk_summary(k_cache: torch.Tensor, chunk_size: int) -> torch.Tensor:
    return load_cuda_extension().csa_chunk_summary(k_cache.contiguous(), int(chunk_size))


def csa_select_topk(q: torch.Tensor, summary: torch.Tensor, top_k: int) -> torch.Tensor:
    return load_cuda_extension().csa_select_topk(q.contiguous(), summary.contiguous(), int(top_k))


def csa_decode_step(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, summary: torch.Tensor,
                    chunk_size: int, top_k: int, tile_size: int = 0):
    return load_cuda_extension().csa_decode_step(q.contiguous(), k_cache.contiguous(), v_cache.contiguous(),
                                                 summary.contiguous(), int(chunk_size), int(top_k), int(tile_size))


def hca_decode_forward(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """hca_reference (hybrid_attention/reference.py:87-92) on the GPU."""
    return load_cuda_extension().hca_decode_forward(q.contiguous(), k_cache.contiguous(), v_cache.contiguous(),
                                                    int(chunk_size))


def hybrid_decode_forward(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, *, csa_chunk_size: int,
                          csa_top_k: int, hca_chunk_size: int, csa_weight: float = 0.7) -> torch.Tensor:
    """hybrid_reference (hybrid_attention/reference.py:95-108) on the GPU."""
    return load_cuda_extension().hybrid_decode_forward(
        q.contiguous(), k_cache.contiguous(), v_cache.contiguous(), csa_chunk_size=int(csa_chunk_size),
        csa_top_k=int(csa_top_k), hca_chunk_size=int(hca_chunk_size), csa_weight=float(csa_weight))
