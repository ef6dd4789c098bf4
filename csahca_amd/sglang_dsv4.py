"""SGLang DeepSeek-V4 decode entry point over the gfx950 DSV4 kernels.

The serving stack (SGLang) builds the decode metadata and keeps tensor
addresses stable for graph replay; this module only maps the tensors it hands
over onto the DSV4 ops of ``csahca_amd.extension``.  It keeps the caller
contract of the reference's adapter
(integrations/sglang_dsv4/csahca_sglang_dsv4_native.py:28-157 and the index
preparation of csahca_sglang_dsv4_patch/patch.py:300-357):

* ``maybe_dsv4_decode_forward(**metadata)`` returns the attention output, or
  ``None`` to let SGLang run its own kernel.  It acts only when
  ``CSAHCA_DSV4_NATIVE`` is set, the batch is in a decode/idle forward mode
  listed in ``CSAHCA_DSV4_NATIVE_FORWARD_MODES`` (default ``DECODE,IDLE``), the
  compress ratio is 0, 4 or 128 and an attention sink is given.  With
  ``CSAHCA_DSV4_NATIVE_STRICT`` set, an unsupported input raises RuntimeError
  instead of delegating.
* FlashMLA views are flattened: caches ``[pages, page_size, 1, bytes]`` ->
  ``[pages, page_size * bytes]``; ``q [T, 1, H, D]`` -> ``[T, H, D]``; index
  tensors ``[T, 1, K]`` -> ``[T, K]``.
* ``match_num_queries`` pads or truncates per-query metadata to the query
  count (SWA indices pad with 0, extra indices with -1, lengths with 1).
"""
from __future__ import annotations

import os
from typing import Any

import torch

_FALSE = {"", "0", "false", "no", "off"}


def _flag(name: str, default: str = "0") -> bool:
    return os.getenv(name, default).strip().lower() not in _FALSE


def _reject(message: str) -> None:
    """Unsupported input: raise in strict mode, else the caller delegates."""
    if _flag("CSAHCA_DSV4_NATIVE_STRICT"):
        raise RuntimeError(message)


def _as_queries(q: torch.Tensor) -> torch.Tensor | None:
    if q.ndim == 3:
        return q
    if q.ndim == 4 and q.shape[1] == 1:
        return q.squeeze(1)
    _reject(f"unsupported q shape for native CSAHCA DSV4 decode: {tuple(q.shape)}")
    return None


def _as_slots(name: str, x: torch.Tensor | None) -> torch.Tensor | None:
    if x is None:
        _reject(f"missing {name} for native CSAHCA DSV4 decode")
        return None
    if x.ndim == 2:
        return x
    if x.ndim == 3 and x.shape[1] == 1:
        return x.squeeze(1)
    _reject(f"unsupported {name} shape for native CSAHCA DSV4 decode: {tuple(x.shape)}")
    return None


def _as_lengths(name: str, x: torch.Tensor | None) -> torch.Tensor | None:
    if x is None:
        _reject(f"missing {name} for native CSAHCA DSV4 decode")
        return None
    if x.ndim == 1:
        return x
    _reject(f"unsupported {name} shape for native CSAHCA DSV4 decode: {tuple(x.shape)}")
    return None


def flatten_flashmla_cache(name: str, x: torch.Tensor | None) -> torch.Tensor | None:
    """[pages, page_size, 1, bytes] (FlashMLA paging) -> [pages, page_size * bytes]."""
    if x is None:
        _reject(f"missing {name} for native CSAHCA DSV4 decode")
        return None
    if x.ndim == 2:
        return x
    if x.ndim == 4 and x.shape[2] == 1:
        return x.reshape(x.shape[0], x.shape[1] * x.shape[3])
    _reject(f"unsupported {name} shape for native CSAHCA DSV4 decode: {tuple(x.shape)}")
    return None


def match_num_queries(x: torch.Tensor | None, num_queries: int, value: int) -> torch.Tensor | None:
    """Per-query metadata cut or padded (with ``value``) to ``num_queries`` rows."""
    if x is None or x.shape[0] == num_queries:
        return x
    if x.shape[0] > num_queries:
        return x[:num_queries]
    tail = torch.full((num_queries - x.shape[0], *x.shape[1:]), value, dtype=x.dtype, device=x.device)
    return torch.cat((x, tail), dim=0)


def _normalise_slots(token_indices, topk_lengths, what: str):
    if token_indices is None or topk_lengths is None:
        raise RuntimeError(f"missing DSV4 {what} indices/topk lengths")
    if token_indices.ndim == 3:
        if token_indices.shape[1] != 1:
            raise RuntimeError(f"unsupported DSV4 {what} index shape {tuple(token_indices.shape)}")
        token_indices = token_indices.squeeze(1)
    if token_indices.ndim != 2:
        raise RuntimeError(f"unsupported DSV4 {what} index rank {token_indices.ndim}")
    if topk_lengths.ndim != 1:
        topk_lengths = topk_lengths.reshape(-1)
    return token_indices, topk_lengths


def prepare_swa_indices(*, core: Any, q: torch.Tensor):
    """SWA slot ids and lengths of the decode metadata (patch.py:310-326)."""
    nq = q.shape[0]
    return _normalise_slots(match_num_queries(core.swa_page_indices, nq, value=0),
                            match_num_queries(core.swa_topk_lengths, nq, value=1), "SWA")


def prepare_extra_indices(*, core: Any, q: torch.Tensor, compress_ratio: int):
    """C4 / C128 slot ids and lengths of the decode metadata (patch.py:329-357)."""
    if compress_ratio == 4:
        ids, lens = getattr(core, "c4_sparse_page_indices", None), getattr(core, "c4_sparse_topk_lengths", None)
    elif compress_ratio == 128:
        ids, lens = getattr(core, "c128_page_indices", None), getattr(core, "c128_topk_lengths_clamp1", None)
    else:
        raise RuntimeError(f"extra indices requested for compress_ratio={compress_ratio}")
    nq = q.shape[0]
    return _normalise_slots(match_num_queries(ids, nq, value=-1), match_num_queries(lens, nq, value=1),
                            f"C{compress_ratio}")


def _mode_allowed(forward_batch: Any) -> bool:
    mode = getattr(forward_batch, "forward_mode", None)
    if mode is None or not mode.is_decode_or_idle():
        return False
    allowed = {m.strip().upper() for m in os.getenv("CSAHCA_DSV4_NATIVE_FORWARD_MODES", "DECODE,IDLE").split(",")
               if m.strip()}
    name = getattr(mode, "name", str(mode)).upper()
    return name in allowed or "DECODE_OR_IDLE" in allowed


def maybe_dsv4_decode_forward(*, q: torch.Tensor, layer_id: int, compress_ratio: int, forward_batch: Any,
                              token_to_kv_pool: Any, swa_k_cache: torch.Tensor, swa_page_indices: torch.Tensor,
                              swa_topk_lengths: torch.Tensor, extra_k_cache: torch.Tensor | None,
                              extra_indices: torch.Tensor | None, extra_topk_lengths: torch.Tensor | None,
                              attn_sink: torch.Tensor | None, page_size: int,
                              softmax_scale: float) -> torch.Tensor | None:
    """DSV4 decode attention for SGLang, or None to delegate (see module doc)."""
    if not _flag("CSAHCA_DSV4_NATIVE"):
        return None
    if not _mode_allowed(forward_batch):
        return None
    if compress_ratio not in (0, 4, 128):
        _reject(f"unsupported native CSAHCA DSV4 compress_ratio={compress_ratio}")
        return None
    if attn_sink is None:
        _reject("native CSAHCA DSV4 decode requires attn_sink")
        return None
    q3 = _as_queries(q)
    cache = flatten_flashmla_cache("swa_k_cache", swa_k_cache)
    ids = _as_slots("swa_page_indices", swa_page_indices)
    lens = _as_lengths("swa_topk_lengths", swa_topk_lengths)
    if q3 is None or cache is None or ids is None or lens is None:
        return None

    from . import extension

    if compress_ratio == 0:
        return extension.dsv4_swa_decode_forward(q3, cache, ids, lens, attn_sink, int(page_size), float(softmax_scale))
    if extra_k_cache is None:
        _reject(f"missing extra_k_cache for native CSAHCA DSV4 ratio={compress_ratio}")
        return None
    ecache = flatten_flashmla_cache("extra_k_cache", extra_k_cache)
    eids = _as_slots("extra_indices", extra_indices)
    elens = _as_lengths("extra_topk_lengths", extra_topk_lengths)
    if ecache is None or eids is None or elens is None:
        return None
    return extension.dsv4_sparse_decode_forward(q3, cache, ids, lens, ecache, eids, elens, attn_sink, int(page_size),
                                                int(token_to_kv_pool.get_extra_key_page_size(layer_id)),
                                                float(softmax_scale))
