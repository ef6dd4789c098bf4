"""SGLang DeepSeek-V4 decode hook over the gfx950 DSV4 kernels.

SGLang's DSV4 attention backend offers every decode step to
``maybe_dsv4_decode_forward(**metadata)`` and runs its own kernel when the hook
returns ``None``.  The keyword signature, the environment switches
(``CSAHCA_DSV4_NATIVE``, ``CSAHCA_DSV4_NATIVE_STRICT``,
``CSAHCA_DSV4_NATIVE_FORWARD_MODES``) and the strict-mode error texts are the
caller contract of the reference hook
(integrations/sglang_dsv4/csahca_sglang_dsv4_native.py:17-157); the index
preparation texts follow csahca_sglang_dsv4_patch/patch.py:300-357.

How this module is organised:

* Every tensor argument is described by one :class:`ArgSpec` row: the rank the
  op takes, the rank of the FlashMLA view SGLang may hand over instead, the
  axis of that view that must have extent 1, and how the view folds into the
  op's layout.  One function, :func:`conform`, applies a row to a tensor.
* A decode route (:data:`ROUTES`) is the list of argument rows a compress
  ratio needs plus the op that runs it; the hook conforms the rows in order
  and calls the op.
* An unusable input raises :class:`Decline` internally.  The hook catches it
  once, at the top, and either delegates (returns ``None``) or, in strict
  mode, raises ``RuntimeError`` with the decline's text.
* The decode-metadata index preparation (:func:`slots_from_metadata`) is
  driven by a second table, :data:`METADATA_SOURCES`, that names the metadata
  fields of each compress ratio and the value short rows are padded with.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Callable, Optional, Sequence

import torch

_OFF_WORDS = frozenset({"", "0", "false", "no", "off"})
_TAG = "native CSAHCA DSV4 decode"


def env_on(name: str, default: str = "0") -> bool:
    """An environment switch: anything but an 'off' word (case-insensitive) is on."""
    return os.getenv(name, default).strip().lower() not in _OFF_WORDS


class Decline(Exception):
    """An input the native path does not take.  The hook delegates on it, or
    raises RuntimeError with the same text when CSAHCA_DSV4_NATIVE_STRICT is on."""


# ---------------------------------------------------------------------------
# argument rows


@dataclass(frozen=True)
class ArgSpec:
    """One tensor argument of the hook.

    ``rank`` is the rank the op takes.  ``view_rank`` is the rank of the
    FlashMLA-shaped view SGLang may pass instead, accepted only when its axis
    ``unit_axis`` has extent 1; ``fold`` turns that view into the op's layout.
    ``missing`` overrides the text used when the argument is None (it may
    name ``{ratio}``)."""

    name: str
    rank: int
    view_rank: Optional[int] = None
    unit_axis: Optional[int] = None
    fold: Optional[Callable[[torch.Tensor], torch.Tensor]] = None
    missing: Optional[str] = None


def _drop_axis1(t: torch.Tensor) -> torch.Tensor:
    return t.squeeze(1)


def _join_page_rows(t: torch.Tensor) -> torch.Tensor:
    # [pages, page_size, 1, bytes_per_row] -> [pages, page_size * bytes_per_row]
    return t.flatten(1)


def queries(name: str) -> ArgSpec:
    """q: [T, H, D], or SGLang's [T, 1, H, D]."""
    return ArgSpec(name, 3, 4, 1, _drop_axis1)


def paged_cache(name: str, missing: Optional[str] = None) -> ArgSpec:
    """A paged cache: [pages, page_bytes], or FlashMLA's [pages, page_size, 1, row_bytes]."""
    return ArgSpec(name, 2, 4, 2, _join_page_rows, missing)


def slot_ids(name: str) -> ArgSpec:
    """Per-query slot ids: [T, K], or [T, 1, K]."""
    return ArgSpec(name, 2, 3, 1, _drop_axis1)


def lengths(name: str) -> ArgSpec:
    """Per-query valid-slot counts: [T] only."""
    return ArgSpec(name, 1)


def conform(spec: ArgSpec, x: Optional[torch.Tensor], ratio: int = 0) -> torch.Tensor:
    """``x`` in the op's layout under ``spec``, or :class:`Decline`."""
    if x is None:
        raise Decline((spec.missing or f"missing {spec.name} for {_TAG}").format(ratio=ratio))
    if x.ndim == spec.rank:
        return x
    if spec.view_rank is not None and x.ndim == spec.view_rank and x.shape[spec.unit_axis] == 1:
        return spec.fold(x)
    raise Decline(f"unsupported {spec.name} shape for {_TAG}: {tuple(x.shape)}")


# ---------------------------------------------------------------------------
# routes


@dataclass(frozen=True)
class Route:
    """The argument rows one compress ratio needs and the op that runs it.
    ``run(ext, tensors, md)`` gets the conformed tensors in ``args`` order."""

    args: Sequence[ArgSpec]
    run: Callable[[Any, list, dict], torch.Tensor]


_WINDOW = (queries("q"), paged_cache("swa_k_cache"), slot_ids("swa_page_indices"), lengths("swa_topk_lengths"))
_EXTRA = (paged_cache("extra_k_cache", "missing extra_k_cache for native CSAHCA DSV4 ratio={ratio}"),
          slot_ids("extra_indices"), lengths("extra_topk_lengths"))


def _run_window(ext, t, md):
    return ext.dsv4_swa_decode_forward(*t, md["attn_sink"], int(md["page_size"]), float(md["softmax_scale"]))


def _run_sparse(ext, t, md):
    extra_page = int(md["token_to_kv_pool"].get_extra_key_page_size(md["layer_id"]))
    return ext.dsv4_sparse_decode_forward(*t, md["attn_sink"], int(md["page_size"]), extra_page,
                                          float(md["softmax_scale"]))


ROUTES = {
    0: Route(_WINDOW, _run_window),
    4: Route(_WINDOW + _EXTRA, _run_sparse),
    128: Route(_WINDOW + _EXTRA, _run_sparse),
}


def _mode_admitted(forward_batch: Any) -> bool:
    """Decode/idle batches whose mode name CSAHCA_DSV4_NATIVE_FORWARD_MODES lists
    (default DECODE,IDLE; the entry DECODE_OR_IDLE admits every such batch)."""
    mode = getattr(forward_batch, "forward_mode", None)
    if mode is None or not mode.is_decode_or_idle():
        return False
    listed = {w.strip().upper() for w in os.getenv("CSAHCA_DSV4_NATIVE_FORWARD_MODES", "DECODE,IDLE").split(",")}
    listed.discard("")
    return "DECODE_OR_IDLE" in listed or getattr(mode, "name", str(mode)).upper() in listed


def _route_for(md: dict) -> Route:
    ratio = md["compress_ratio"]
    if ratio not in ROUTES:
        raise Decline(f"unsupported native CSAHCA DSV4 compress_ratio={ratio}")
    if md["attn_sink"] is None:
        raise Decline("native CSAHCA DSV4 decode requires attn_sink")
    return ROUTES[ratio]


def maybe_dsv4_decode_forward(*, q: torch.Tensor, layer_id: int, compress_ratio: int, forward_batch: Any,
                              token_to_kv_pool: Any, swa_k_cache: torch.Tensor, swa_page_indices: torch.Tensor,
                              swa_topk_lengths: torch.Tensor, extra_k_cache: torch.Tensor | None,
                              extra_indices: torch.Tensor | None, extra_topk_lengths: torch.Tensor | None,
                              attn_sink: torch.Tensor | None, page_size: int,
                              softmax_scale: float) -> torch.Tensor | None:
    """DSV4 decode attention for SGLang's decode metadata, or None to let SGLang
    run its own kernel.  The hook acts only when CSAHCA_DSV4_NATIVE is on and the
    batch's forward mode is admitted; then an unusable input delegates, or raises
    RuntimeError under CSAHCA_DSV4_NATIVE_STRICT."""
    if not env_on("CSAHCA_DSV4_NATIVE") or not _mode_admitted(forward_batch):
        return None
    md = dict(q=q, layer_id=layer_id, compress_ratio=compress_ratio, token_to_kv_pool=token_to_kv_pool,
              swa_k_cache=swa_k_cache, swa_page_indices=swa_page_indices, swa_topk_lengths=swa_topk_lengths,
              extra_k_cache=extra_k_cache, extra_indices=extra_indices, extra_topk_lengths=extra_topk_lengths,
              attn_sink=attn_sink, page_size=page_size, softmax_scale=softmax_scale)
    try:
        route = _route_for(md)
        tensors = [conform(spec, md[spec.name], compress_ratio) for spec in route.args]
    except Decline as why:
        if env_on("CSAHCA_DSV4_NATIVE_STRICT"):
            raise RuntimeError(str(why)) from None
        return None

    from . import extension

    return route.run(extension, tensors, md)


# ---------------------------------------------------------------------------
# index preparation from SGLang's decode metadata


def match_num_queries(x: torch.Tensor | None, num_queries: int, value: int) -> torch.Tensor | None:
    """``x`` with exactly ``num_queries`` rows: longer metadata is cut (a view),
    shorter metadata gains rows filled with ``value``."""
    if x is None or x.shape[0] == num_queries:
        return x
    if x.shape[0] > num_queries:
        return x[:num_queries]
    out = x.new_full((num_queries, *x.shape[1:]), value)
    out[: x.shape[0]].copy_(x)
    return out


@dataclass(frozen=True)
class MetadataSource:
    """Where one compress ratio's slot ids and lengths live in the decode
    metadata, what short id rows are padded with, and the word its errors use."""

    ids: str
    lengths: str
    id_fill: int
    label: str
    missing: str


METADATA_SOURCES = {
    0: MetadataSource("swa_page_indices", "swa_topk_lengths", 0, "SWA", "missing DSV4 SWA indices/topk lengths"),
    4: MetadataSource("c4_sparse_page_indices", "c4_sparse_topk_lengths", -1, "extra",
                      "missing DSV4 extra indices/topk lengths for compress_ratio=4"),
    128: MetadataSource("c128_page_indices", "c128_topk_lengths_clamp1", -1, "extra",
                        "missing DSV4 extra indices/topk lengths for compress_ratio=128"),
}


def slots_from_metadata(core: Any, num_queries: int, ratio: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(slot ids [T, K], lengths [T]) of compress ratio ``ratio`` (0 = the SWA
    window) from SGLang's decode metadata ``core``, fitted to ``num_queries``
    rows (lengths pad with 1)."""
    src = METADATA_SOURCES[ratio]
    ids = match_num_queries(getattr(core, src.ids, None), num_queries, src.id_fill)
    lens = match_num_queries(getattr(core, src.lengths, None), num_queries, 1)
    if ids is None or lens is None:
        raise RuntimeError(src.missing)
    if ids.ndim == 3 and ids.shape[1] != 1:
        raise RuntimeError(f"unsupported DSV4 {src.label} index shape {tuple(ids.shape)}")
    ids = ids.flatten(1, 2) if ids.ndim == 3 else ids
    if ids.ndim != 2:
        raise RuntimeError(f"unsupported DSV4 {src.label} index rank {ids.ndim}")
    return ids, lens.reshape(-1)


def prepare_swa_indices(*, core: Any, q: torch.Tensor):
    """SWA slot ids and lengths for the queries of ``q``."""
    return slots_from_metadata(core, q.shape[0], 0)


def prepare_extra_indices(*, core: Any, q: torch.Tensor, compress_ratio: int):
    """C4 / C128 slot ids and lengths for the queries of ``q``."""
    if compress_ratio not in (4, 128):
        raise RuntimeError(f"extra indices requested for compress_ratio={compress_ratio}")
    return slots_from_metadata(core, q.shape[0], compress_ratio)
