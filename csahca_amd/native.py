"""Torch-tensor binding of libcsahca.so -- the replacement for the reference's
pybind module ``hybrid_attention_cuda`` (csrc/bindings.cpp:54-163).

The five reference ops keep their names, argument order and error texts:
``csa_decode_forward``, ``csa_decode_forward_tiled``, ``dsv4_swa_decode_forward``,
``dsv4_sparse_decode_forward`` and ``dsv4_decode_forward_tiled``.  Structural
checks (device, contiguity, rank, dtype, shape agreement) run here with the
reference's TORCH_CHECK messages (csrc/csa_attention.cu:336-363,394-422,
csrc/dsv4_attention.cu:593-625,671-728,775-848) and raise RuntimeError; value
checks run in the C library.  Outputs and workspaces come from torch's caching
allocator on the current stream; kernels run on torch's current HIP stream,
so calls are graph-capturable.

New ops next to them: ``csa_chunk_summary``, ``csa_select_topk``,
``csa_decode_step`` (summary scoring + top-k + sparse attention in one call),
``hca_decode_forward`` and ``hybrid_decode_forward``.

There is no CPU fallback: without the built library every op raises.
With CSAHCA_ROCTX=1 at import every op runs inside a roctx range named after
it (csahca_amd.tracing).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

from .tracing import traced

# CSAHCA_LIBRARY names another build of the library to load (the host-sanitized
# variant for the sanitizer tests); by default the in-tree libcsahca.so.
_LIB_PATH = Path(os.environ.get("CSAHCA_LIBRARY") or Path(__file__).resolve().parent / "libcsahca.so")
_LIB = None

_DTYPES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}
_FLOATING = (torch.float32, torch.float16, torch.bfloat16, torch.float64)

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
_dbl = ctypes.c_double

_SIGNATURES = {
    "csahca_last_error": (ctypes.c_char_p, []),
    "csahca_abi_version": (_int, []),
    "csahca_csa_decode_workspace_bytes": (_sz, [_i64] * 6),
    "csahca_csa_auto_tile_size": (_i64, [_i64] * 4),
    "csahca_csa_decode_forward": (_int, [_vp] * 5 + [_int, _int] + [_i64] * 6 + [_vp, _sz, _vp]),
    "csahca_csa_decode_forward_tiled": (_int, [_vp] * 5 + [_int, _int] + [_i64] * 7 + [_vp, _sz, _vp]),
    "csahca_csa_chunk_summary": (_int, [_vp, _vp, _int] + [_i64] * 8 + [_vp]),
    "csahca_csa_chunk_summary_at": (_int, [_vp, _vp, _int] + [_i64] * 6 + [_vp, _vp]),
    "csahca_csa_select_workspace_bytes": (_sz, [_i64] * 3),
    "csahca_csa_select_topk": (_int, [_vp, _vp, _vp, _int] + [_i64] * 5 + [_vp, _sz, _vp]),
    "csahca_dsv4_decode_workspace_bytes": (_sz, [_i64] * 5),
    "csahca_dsv4_decode_forward_tiled": (
        _int, [_vp, _int, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp,
               _i64, _vp, _vp, _dbl, _i64, _vp, _vp, _sz, _vp]),
    "csahca_dsv4_swa_decode_forward": (
        _int, [_vp, _int, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _dbl, _vp, _vp, _sz, _vp]),
    "csahca_dsv4_sparse_decode_forward": (
        _int, [_vp, _int, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp,
               _i64, _vp, _vp, _dbl, _vp, _vp, _sz, _vp]),
    "csahca_csa_step_workspace_bytes": (_sz, [_i64] * 6),
    "csahca_csa_decode_step": (_int, [_vp] * 6 + [_int] + [_i64] * 7 + [_vp, _sz, _vp]),
    "csahca_csa_decode_step_dev": (_int, [_vp] * 7 + [_int] + [_i64] * 7 + [_vp, _sz, _vp]),
    "csahca_csa_decode_step_at": (_int, [_vp] * 7 + [_int] + [_i64] * 7 + [_vp, _sz, _vp]),
    "csahca_csa_step_status": (_int, [_vp, ctypes.POINTER(ctypes.c_uint32), _vp]),
    "csahca_csa_decode_step_noalloc": (_int, [_vp] * 6 + [_int] + [_i64] * 7 + [_vp]),
    "csahca_csa_step_noalloc_reset": (_int, [_vp]),
    "csahca_hca_decode_workspace_bytes": (_sz, [_i64] * 5),
    "csahca_dsv4_pack_tokens": (_int, [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "csahca_hca_decode_forward": (_int, [_vp, _vp, _vp, _vp, _dbl, _vp, _int] + [_i64] * 5 + [_vp, _sz, _vp]),
    "csahca_hybrid_decode_forward": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _int] + [_i64] * 8 + [_dbl] +
                                     [_vp, _sz, _vp, _sz, _vp]),
    "csahca_block_linear": (_int, [_vp, _vp, _dbl, _vp, _int, _vp, _vp, _dbl, _vp, _int, _i64, _i64, _i64, _vp,
                                   _vp]),
    "csahca_block_qkv": (_int, [_vp, _vp, _dbl, _vp, _vp, _vp, _vp, _vp, _vp, _int] + [_i64] * 5 + [_vp]),
    "csahca_profile_begin": (_int, []),
    "csahca_profile_end": (_int, []),
    "csahca_device_clock_stamp": (_int, [_vp, _vp]),
    "csahca_device_clock_khz": (_i64, []),
    "csahca_profile_result": (_int, [_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i64),
                                     ctypes.POINTER(_dbl), ctypes.POINTER(_dbl), ctypes.POINTER(_dbl)]),
}

EXPORTED = tuple(_SIGNATURES)


# ABI revision of include/csahca.h that these signatures follow.
ABI_VERSION = 1


def library_path() -> Path:
    return _LIB_PATH


def lib():
    """Load libcsahca.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            raise RuntimeError(
                f"{_LIB_PATH} is not built; run `python -m csahca_amd.build` (hipcc, gfx950)")
        handle = ctypes.CDLL(str(_LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        got = handle.csahca_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{_LIB_PATH} has ABI revision {got}, this binding expects {ABI_VERSION}; rebuild it")
        _LIB = handle
    return _LIB


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _rc(code: int) -> None:
    if code != 0:
        raise RuntimeError(lib().csahca_last_error().decode())


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


# torch's current-device and raw current-stream queries (one C call each; the
# Stream object that torch.cuda.current_stream() builds costs several us).
_current_device = torch._C._cuda_getDevice
_raw_stream = torch._C._cuda_getCurrentRawStream


def _stream() -> int:
    return _raw_stream(_current_device())


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


_SCRATCH_WS: dict = {}
_WS_BYTES: dict = {}


def _ws_bytes(fn_name: str, *args) -> int:
    """A workspace-size query of the library, memoised per (function, shape):
    the sizes are pure functions of their arguments."""
    key = (fn_name,) + args
    n = _WS_BYTES.get(key)
    if n is None:
        n = int(getattr(lib(), fn_name)(*args))
        _WS_BYTES[key] = n
    return n


def _scratch_workspace(nbytes: int, dev: int, stream: int) -> torch.Tensor:
    """A workspace whose contents do not outlive one call (split partials),
    kept per (device, stream, size) instead of allocated per call.  Calls on
    one stream run in order, so they can share it; calls on different streams
    get different buffers.  Never freed while the process runs
    (release_step_workspaces() drops them), because a captured graph keeps
    the address it recorded."""
    key = (dev, stream, nbytes)
    ws = _SCRATCH_WS.get(key)
    if ws is None:
        ws = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=torch.device("cuda", dev))
        _SCRATCH_WS[key] = ws
    return ws


def _defined(t) -> bool:
    return t is not None


def _present(t) -> bool:
    """A tensor that carries values (None and empty tensors mean "absent")."""
    return t is not None and t.numel() > 0


# ---------------------------------------------------------------------------
# CSA
# ---------------------------------------------------------------------------

# With one visible device every CUDA tensor is on it, so the device check
# below runs only where there are several (device_count does not initialise
# the GPU).
_MULTI_DEVICE = torch.cuda.device_count() > 1


def _same_device(dev: int, *tensors) -> None:
    """Every given CUDA tensor (None skipped; a CPU tensor is left to the
    caller's own is_cuda check and its message) lives on device ``dev``: the
    library addresses them all from the one device it launches on."""
    for t in tensors:
        if t is not None and t.is_cuda and t.get_device() != dev:
            raise RuntimeError("all tensors must be on the same device")


def _csa_checks(q, k_cache, v_cache, chunk_indices, chunk_size, tiled: bool, tile_size=None):
    """The reference's TORCH_CHECKs of the CSA ops, in their order (the first
    that fails raises its text); ``chunk_indices`` None (the fused step, which
    selects its own) skips the checks of that tensor.  Each check is an inline
    test, not a call: they run on every eager call."""
    msg = _csa_check_error(q, k_cache, v_cache, chunk_indices, chunk_size, tiled, tile_size)
    if msg is not None:
        raise RuntimeError(msg)
    if _MULTI_DEVICE:
        _same_device(q.get_device(), k_cache, v_cache, chunk_indices)


def _csa_check_error(q, k_cache, v_cache, chunk_indices, chunk_size, tiled, tile_size):
    have_idx = chunk_indices is not None
    if not (q.is_cuda and k_cache.is_cuda and v_cache.is_cuda and (not have_idx or chunk_indices.is_cuda)):
        return "all tensors must be CUDA tensors"
    if not q.is_contiguous():
        return "q must be contiguous"
    if not k_cache.is_contiguous():
        return "k_cache must be contiguous"
    if not v_cache.is_contiguous():
        return "v_cache must be contiguous"
    if have_idx and not chunk_indices.is_contiguous():
        return "chunk_indices must be contiguous"
    if q.dim() != 3:
        return "q must be [batch, heads, head_dim]"
    if k_cache.dim() != 4:
        return "k_cache must be [batch, heads, seq, head_dim]"
    if v_cache.shape != k_cache.shape:
        return "v_cache must match k_cache shape"
    if have_idx and chunk_indices.dim() != 3:
        return "chunk_indices must be [batch, heads, top_k]"
    if q.dtype != k_cache.dtype:
        return "q and k_cache dtype must match"
    if q.dtype != v_cache.dtype:
        return "q and v_cache dtype must match"
    if have_idx and chunk_indices.dtype not in (torch.int32, torch.int64):
        return "chunk_indices must be int32 or int64"
    B, H, D = q.shape
    if not (k_cache.shape[0] == B and k_cache.shape[1] == H and k_cache.shape[3] == D):
        return "KV cache shape must match q"
    if have_idx and not (chunk_indices.shape[0] == B and chunk_indices.shape[1] == H):
        return "chunk_indices batch/head dimensions must match q"
    if not chunk_size > 0:
        return "chunk_size must be positive"
    if tiled:
        if not tile_size > 0:
            return "tile_size must be positive"
        if D > 1024:
            return "head_dim > 1024 is not supported by the tiled kernel"
    elif D > 1024:
        return "head_dim > 1024 is not supported by the v1 kernel"
    if q.dtype not in _FLOATING:
        return f"unsupported dtype {q.dtype}"
    return None


@traced
def csa_decode_forward(q, k_cache, v_cache, chunk_indices, chunk_size):
    """Sparse decode over explicit chunk ids (reference op csa_decode_forward)."""
    chunk_size = int(chunk_size)
    _csa_checks(q, k_cache, v_cache, chunk_indices, chunk_size, tiled=False)
    B, H, D = q.shape
    S, top_k = k_cache.shape[2], chunk_indices.shape[2]
    with torch.cuda.device(q.device):
        out = torch.empty_like(q)
        nbytes = lib().csahca_csa_decode_workspace_bytes(B, H, D, top_k, chunk_size, 0)
        ws = _workspace(nbytes, q.device)
        _rc(lib().csahca_csa_decode_forward(
            _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(chunk_indices), _ptr(out), _DTYPES[q.dtype],
            0 if chunk_indices.dtype == torch.int32 else 1, B, H, S, D, top_k, chunk_size,
            _ptr(ws), ws.numel(), _stream()))
    return out


@traced
def csa_decode_forward_tiled(q, k_cache, v_cache, chunk_indices, chunk_size, tile_size):
    """Split-KV sparse decode (reference op csa_decode_forward_tiled)."""
    chunk_size, tile_size = int(chunk_size), int(tile_size)
    _csa_checks(q, k_cache, v_cache, chunk_indices, chunk_size, tiled=True, tile_size=tile_size)
    B, H, D = q.shape
    S, top_k = k_cache.shape[2], chunk_indices.shape[2]
    dev = q.get_device()
    if dev != _current_device():
        with torch.cuda.device(dev):
            return csa_decode_forward_tiled(q, k_cache, v_cache, chunk_indices, chunk_size, tile_size)
    stream = _raw_stream(dev)
    out = torch.empty_like(q)
    nbytes = _ws_bytes("csahca_csa_decode_workspace_bytes", B, H, D, top_k, chunk_size, tile_size)
    ws = _scratch_workspace(nbytes, dev, stream)
    _rc(lib().csahca_csa_decode_forward_tiled(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), chunk_indices.data_ptr(), out.data_ptr(),
        _DTYPES[q.dtype], 0 if chunk_indices.dtype == torch.int32 else 1, B, H, S, D, top_k, chunk_size, tile_size,
        ws.data_ptr(), ws.numel(), stream))
    return out


def csa_auto_tile_size(batch: int, heads: int, top_k: int, chunk_size: int) -> int:
    return int(lib().csahca_csa_auto_tile_size(batch, heads, top_k, chunk_size))


@traced
def csa_chunk_summary(k_cache, chunk_size, *, out=None, chunk_begin: int = 0, num_chunks: int | None = None):
    """fp32 chunk means of K (chunk_mean, hybrid_attention/reference.py:40-45).

    Returns ``[B, H, S // chunk_size, D]`` fp32.  With ``out`` given, only chunks
    ``[chunk_begin, chunk_begin + num_chunks)`` are (re)computed in place -- the
    incremental update when the cache grows by a chunk.
    """
    chunk_size = int(chunk_size)
    _check(k_cache.is_cuda, "k_cache must be CUDA")
    _check(k_cache.is_contiguous(), "k_cache must be contiguous")
    _check(k_cache.dim() == 4, "k_cache must be [batch, heads, seq, head_dim]")
    _check(k_cache.dtype in _FLOATING, f"unsupported dtype {k_cache.dtype}")
    _check(chunk_size > 0, "chunk_size must be positive")
    B, H, S, D = k_cache.shape
    C = S // chunk_size
    if num_chunks is None:
        num_chunks = C - chunk_begin
    with torch.cuda.device(k_cache.device):
        if out is None:
            out = torch.empty((B, H, C, D), dtype=torch.float32, device=k_cache.device)
        _check(out.is_cuda and out.is_contiguous() and out.dtype == torch.float32 and out.dim() == 4
               and tuple(out.shape[:2]) == (B, H) and out.shape[3] == D,
               "summary must be a contiguous fp32 [batch, heads, chunks, head_dim] CUDA tensor")
        if _MULTI_DEVICE:
            _same_device(k_cache.get_device(), out)
        _rc(lib().csahca_csa_chunk_summary(_ptr(k_cache), _ptr(out), _DTYPES[k_cache.dtype], B, H, S, D,
                                           chunk_size, out.shape[2], int(chunk_begin), int(num_chunks),
                                           _stream()))
    return out


@traced
def csa_chunk_summary_at(k_cache, summary, chunk_size, token_pos):
    """Recompute in place the summary of the chunk that the token at
    ``token_pos`` (a one-element int64 CUDA tensor, read on the device)
    completes; nothing happens when that token completes no chunk.  The
    graph-capturable form of the incremental update: ``summary`` is a
    preallocated ``[B, H, max_chunks, D]`` fp32 tensor and only ever receives
    complete chunks."""
    chunk_size = int(chunk_size)
    _check(k_cache.is_cuda and summary.is_cuda and token_pos.is_cuda, "tensors must be CUDA tensors")
    if _MULTI_DEVICE:
        _same_device(k_cache.get_device(), summary, token_pos)
    _check(k_cache.is_contiguous() and k_cache.dim() == 4, "k_cache must be a contiguous [batch, heads, seq, head_dim]")
    _check(k_cache.dtype in _FLOATING, f"unsupported dtype {k_cache.dtype}")
    _check(chunk_size > 0, "chunk_size must be positive")
    B, H, S, D = k_cache.shape
    _check(summary.is_contiguous() and summary.dtype == torch.float32 and summary.dim() == 4
           and tuple(summary.shape[:2]) == (B, H) and summary.shape[3] == D,
           "summary must be a contiguous fp32 [batch, heads, chunks, head_dim] CUDA tensor")
    _check(token_pos.dtype == torch.int64 and token_pos.numel() == 1, "token_pos must be a one-element int64 tensor")
    with torch.cuda.device(k_cache.device):
        _rc(lib().csahca_csa_chunk_summary_at(_ptr(k_cache), _ptr(summary), _DTYPES[k_cache.dtype], B, H, S, D,
                                              chunk_size, summary.shape[2], _ptr(token_pos), _stream()))
    return summary


@traced
def csa_select_topk(q, summary, top_k):
    """Top-k chunk ids by q . summary / sqrt(D) (select_topk_chunks scoring,
    hybrid_attention/reference.py:51-56).  int32 ``[B, H, min(top_k, C)]``, best
    first; equal scores are ordered by ascending chunk id."""
    top_k = int(top_k)
    _check(q.is_cuda and summary.is_cuda, "q and summary must be CUDA tensors")
    if _MULTI_DEVICE:
        _same_device(q.get_device(), summary)
    _check(q.is_contiguous() and summary.is_contiguous(), "q and summary must be contiguous")
    _check(q.dim() == 3, "q must be [batch, heads, head_dim]")
    _check(summary.dim() == 4 and summary.dtype == torch.float32,
           "summary must be fp32 [batch, heads, chunks, head_dim]")
    B, H, D = q.shape
    _check(tuple(summary.shape[:2]) == (B, H) and summary.shape[3] == D, "summary shape must match q")
    _check(q.dtype in _FLOATING, f"unsupported dtype {q.dtype}")
    _check(top_k >= 0, "top_k must be non-negative")
    C = summary.shape[2]
    k = min(top_k, C)
    with torch.cuda.device(q.device):
        out = torch.empty((B, H, k), dtype=torch.int32, device=q.device)
        ws = _workspace(lib().csahca_csa_select_workspace_bytes(B, H, C), q.device)
        _rc(lib().csahca_csa_select_topk(_ptr(q), _ptr(summary), _ptr(out), _DTYPES[q.dtype], B, H, C, D,
                                         top_k, _ptr(ws), ws.numel(), _stream()))
    return out


_STEP_WS: dict = {}


def _step_workspace(nbytes: int, device, signature: tuple) -> torch.Tensor:
    """Step workspace for one (device, stream, problem shape).

    The fused step keeps per-head launch epochs and tagged exchange words in it,
    laid out by the shape (B*H, chunks, head_dim, top_k, chunk), so each shape
    gets a buffer of its own, zero-filled once (a fill kernel, on the calling
    stream) and then reused by every call of that shape on that stream -- eager
    calls and replays of graphs captured on it alike.  Buffers live until
    release_step_workspaces(): a captured graph keeps their addresses."""
    return _step_ws_get(nbytes, torch.device(device).index, _stream(), signature)[0]


def _step_ws_get(nbytes, dev: int, stream: int, signature: tuple):
    """(workspace, its size in bytes) for (device index, raw stream, shape);
    ``nbytes`` may be a callable, evaluated only when the buffer is created."""
    key = (dev, stream, signature)
    hit = _STEP_WS.get(key)
    if hit is None:
        n = max(int(nbytes() if callable(nbytes) else nbytes), 256)
        ws = torch.zeros(n, dtype=torch.uint8, device=torch.device("cuda", dev))
        hit = (ws, n)
        _STEP_WS[key] = hit
    return hit


def step_workspace_ready(device, stream, signature: tuple) -> bool:
    """Whether a step workspace exists for (device, stream, shape signature)."""
    d = torch.device(device)
    index = d.index if d.index is not None else torch.cuda.current_device()
    return (index, int(stream), tuple(signature)) in _STEP_WS


def release_step_workspaces() -> None:
    """Drop every cached step workspace and per-stream scratch workspace (only
    when no captured graph that used one will be replayed again)."""
    _STEP_WS.clear()
    _SCRATCH_WS.clear()


@traced
def csa_decode_step(q, k_cache, v_cache, summary, chunk_size, top_k, tile_size: int = 0):
    """One CSA decode step from cached summaries in one launch: select the top-k
    chunks (as csa_select_topk), then attend over their tokens (as
    csa_decode_forward).  Returns ``(out, chunk_indices)``.

    ``tile_size`` > 0 runs the two-pass route instead (selection kernels, then
    the split-KV op with that split size)."""
    chunk_size, top_k = int(chunk_size), int(top_k)
    if tile_size and tile_size > 0:
        idx = csa_select_topk(q, summary, top_k)
        return csa_decode_forward_tiled(q, k_cache, v_cache, idx, chunk_size, int(tile_size)), idx
    _csa_checks(q, k_cache, v_cache, None, chunk_size, tiled=False)
    if not (summary.is_cuda and summary.is_contiguous() and summary.dtype == torch.float32 and summary.dim() == 4):
        raise RuntimeError("summary must be a contiguous fp32 [batch, heads, chunks, head_dim] CUDA tensor")
    B, H, D = q.shape
    S = k_cache.shape[2]
    if not (summary.shape[0] == B and summary.shape[1] == H and summary.shape[3] == D):
        raise RuntimeError("summary shape must match q")
    C = summary.shape[2]
    if top_k < 0:
        raise RuntimeError("top_k must be non-negative")
    k = min(top_k, C)
    dev = q.get_device()
    if _MULTI_DEVICE:
        _same_device(dev, summary)
    if dev != _current_device():
        with torch.cuda.device(dev):
            return csa_decode_step(q, k_cache, v_cache, summary, chunk_size, top_k)
    stream = _raw_stream(dev)
    out = torch.empty_like(q)
    idx = q.new_empty((B, H, k), dtype=torch.int32)
    ws, nbytes = _step_ws_get(lambda: lib().csahca_csa_step_workspace_bytes(B, H, C, D, top_k, chunk_size), dev,
                              stream, (B * H, C, D, k, chunk_size))
    _rc((_LIB or lib()).csahca_csa_decode_step(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), summary.data_ptr(),
                                    out.data_ptr(), idx.data_ptr(), _DTYPES[q.dtype], B, H, S, D, C, chunk_size,
                                    top_k, ws.data_ptr(), nbytes, stream))
    return out, idx


NOALLOC_MAX_HEADS = 256      # batch * heads
NOALLOC_MAX_CHUNKS = 2048    # summary rows per head
NOALLOC_MAX_HEAD_DIM = 256


@traced
def csa_decode_step_noalloc(q, k_cache, v_cache, summary, chunk_size, top_k, *, out, indices):
    """csa_decode_step through the library's allocation-free entry point: the
    exchange state lives in a static per-device array, so neither the library
    nor this wrapper allocates anything (``out`` like q, ``indices`` int32
    [B, H, min(top_k, C)] are the caller's).  For callers that cannot allocate
    (graph capture, tight serving loops).  Limits: B*H <= 256, C <= 2048,
    head_dim 64/128/256, bf16/f16/f32, 0 < top_k <= 1024.  Calls that overlap
    on one device race on the shared array.  Returns ``(out, indices)``."""
    chunk_size, top_k = int(chunk_size), int(top_k)
    _check(all(t.is_cuda for t in (q, k_cache, v_cache, summary, out, indices)), "all tensors must be CUDA tensors")
    if _MULTI_DEVICE:
        _same_device(q.get_device(), k_cache, v_cache, summary, out, indices)
    _check(all(t.is_contiguous() for t in (q, k_cache, v_cache, summary, out, indices)), "tensors must be contiguous")
    _check(q.dim() == 3 and k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "q [B, H, D], caches [B, H, S, D]")
    B, H, S, D = k_cache.shape
    _check(tuple(q.shape) == (B, H, D) and q.dtype == k_cache.dtype == v_cache.dtype, "q must match the caches")
    _check(q.dtype in _DTYPES, f"unsupported dtype {q.dtype}")
    _check(summary.dtype == torch.float32 and summary.dim() == 4 and tuple(summary.shape[:2]) == (B, H)
           and summary.shape[3] == D, "summary must be fp32 [batch, heads, chunks, head_dim]")
    C = summary.shape[2]
    _check(out.shape == q.shape and out.dtype == q.dtype, "out must match q")
    _check(tuple(indices.shape) == (B, H, min(top_k, C)) and indices.dtype == torch.int32,
           "indices must be int32 [batch, heads, min(top_k, chunks)]")
    with torch.cuda.device(q.device):
        _rc(lib().csahca_csa_decode_step_noalloc(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(summary), _ptr(out),
                                                 _ptr(indices), _DTYPES[q.dtype], B, H, S, D, C, chunk_size, top_k,
                                                 _stream()))
    return out, indices


@traced
def csa_decode_step_dev(q, k_cache, v_cache, summary, num_chunks, chunk_size, top_k, *, out=None, indices=None):
    """csa_decode_step with the chunk count in device memory: ``summary`` holds
    ``max_chunks`` rows per head and the step selects among the first
    ``clamp(num_chunks, 0, max_chunks)`` of them (``num_chunks``: one-element
    int32 CUDA tensor, read on the device).  Index slots past that count are
    -1.  No host synchronisation and fixed shapes, so a decode loop over a
    growing cache can be captured in one HIP graph.  ``out`` / ``indices``
    may be given to write in place.  Returns ``(out, chunk_indices)``."""
    chunk_size, top_k = int(chunk_size), int(top_k)
    _csa_checks(q, k_cache, v_cache, None, chunk_size, tiled=False)
    _check(summary.is_cuda and summary.is_contiguous() and summary.dtype == torch.float32 and summary.dim() == 4,
           "summary must be a contiguous fp32 [batch, heads, chunks, head_dim] CUDA tensor")
    _check(num_chunks.is_cuda and num_chunks.dtype == torch.int32 and num_chunks.numel() == 1,
           "num_chunks must be a one-element int32 CUDA tensor")
    B, H, D = q.shape
    S = k_cache.shape[2]
    _check(tuple(summary.shape[:2]) == (B, H) and summary.shape[3] == D, "summary shape must match q")
    Cs = summary.shape[2]
    _check(top_k >= 0, "top_k must be non-negative")
    k = min(top_k, Cs)
    if _MULTI_DEVICE:
        _same_device(q.get_device(), summary, num_chunks, out, indices)
    with torch.cuda.device(q.device):
        if out is None:
            out = torch.empty_like(q)
        if indices is None:
            indices = torch.empty((B, H, k), dtype=torch.int32, device=q.device)
        _check(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "out must match q")
        _check(tuple(indices.shape) == (B, H, k) and indices.dtype == torch.int32 and indices.is_contiguous(),
               "indices must be a contiguous int32 [batch, heads, min(top_k, max_chunks)] tensor")
        ws = _step_workspace(lib().csahca_csa_step_workspace_bytes(B, H, Cs, D, top_k, chunk_size), q.device,
                             (B * H, Cs, D, k, chunk_size))
        _rc(lib().csahca_csa_decode_step_dev(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(summary), _ptr(num_chunks),
                                             _ptr(out), _ptr(indices), _DTYPES[q.dtype], B, H, S, D, Cs, chunk_size,
                                             top_k, _ptr(ws), ws.numel(), _stream()))
    return out, indices


_ACTIVATIONS = {None: 0, "silu": 1, "gelu": 2}
_BLOCK_DTYPES = (torch.bfloat16, torch.float16)


def _overlaps(a: torch.Tensor, b: torch.Tensor) -> bool:
    a0, b0 = a.data_ptr(), b.data_ptr()
    return a.device == b.device and a0 < b0 + b.numel() * b.element_size() and b0 < a0 + a.numel() * a.element_size()


def block_linear_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Shapes and types block_linear takes (others use torch's linear)."""
    B, K = x.shape
    return (x.is_cuda and x.dtype in _BLOCK_DTYPES and weight.dtype == x.dtype and x.is_contiguous()
            and weight.is_contiguous() and 0 < B <= 4 and K % 8 == 0 and K <= (4096 if B == 1 else 2048)
            and x.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0)


@traced
def block_linear(x, weight, *, norm_weight=None, eps: float = 1e-6, activation=None, residual=None, base=None,
                 alpha: float = 1.0, out=None, advance_pos=None):
    """Decode-step product ``base + alpha * (act(x' @ weight.T) + residual)`` for
    x [batch <= 4, in_features] (bf16/f16), rounded like the torch ops it
    replaces: x' = x or RMSNorm(x; norm_weight, eps); activation None, "silu"
    or "gelu" (exact); residual and base [batch, out_features], each optional.
    ``out`` may be ``residual`` or ``base`` itself, never ``x``.
    ``advance_pos`` (int64 CUDA tensor) is incremented by one after the
    product.  Returns ``out`` [batch, out_features]."""
    _check(x.is_cuda and weight.is_cuda, "x and weight must be CUDA tensors")
    if _MULTI_DEVICE:
        _same_device(x.get_device(), weight, norm_weight, residual, base, advance_pos, out)
    _check(x.dim() == 2 and weight.dim() == 2 and weight.shape[1] == x.shape[1],
           "x must be [batch, in_features] and weight [out_features, in_features]")
    _check(x.dtype in _BLOCK_DTYPES and weight.dtype == x.dtype, "x and weight must both be bfloat16 or float16")
    _check(x.is_contiguous() and weight.is_contiguous(), "x and weight must be contiguous")
    _check(activation in _ACTIVATIONS, "activation must be None, 'silu' or 'gelu'")
    B, K = x.shape
    N = weight.shape[0]
    if norm_weight is not None:
        _check(norm_weight.is_cuda and norm_weight.dtype == x.dtype and norm_weight.is_contiguous()
               and norm_weight.numel() == K, "norm_weight must be a contiguous [in_features] tensor of x's dtype")
    for name, t in (("residual", residual), ("base", base)):
        if t is not None:
            _check(t.is_cuda and t.dtype == x.dtype and t.is_contiguous() and tuple(t.shape) == (B, N),
                   f"{name} must be a contiguous [batch, out_features] tensor of x's dtype")
    if advance_pos is not None:
        _check(advance_pos.is_cuda and advance_pos.dtype == torch.int64 and advance_pos.numel() == 1,
               "advance_pos must be a one-element int64 CUDA tensor")
    with torch.cuda.device(x.device):
        if out is None:
            out = torch.empty((B, N), dtype=x.dtype, device=x.device)
        _check(out.dtype == x.dtype and out.is_contiguous() and tuple(out.shape) == (B, N),
               "out must be a contiguous [batch, out_features] tensor of x's dtype")
        _check(not _overlaps(out, x), "out must not overlap x")
        _rc(lib().csahca_block_linear(_ptr(x), _ptr(norm_weight), float(eps), _ptr(weight), _ACTIVATIONS[activation],
                                      _ptr(residual), _ptr(base), float(alpha), _ptr(out), _DTYPES[x.dtype], B, N,
                                      K, _ptr(advance_pos), _stream()))
    return out


@traced
def block_qkv(hidden, w_qkv, q, k_cache, v_cache, token_pos, *, norm_weight=None, eps: float = 1e-6,
              num_chunks=None, chunk_size: int = 64):
    """QKV projection of a decode step over a growing cache: RMSNorm(hidden)
    @ w_qkv.T split into q (written to ``q`` [batch, H, D]) and the new token's
    K and V (written to row ``token_pos`` of ``k_cache`` / ``v_cache``
    [batch, H, capacity, D]); ``num_chunks`` (int32, optional) receives
    (token_pos + 1) // chunk_size.  Positions are read on the device."""
    _check(all(t.is_cuda for t in (hidden, w_qkv, q, k_cache, v_cache, token_pos)), "all tensors must be CUDA tensors")
    if _MULTI_DEVICE:
        _same_device(hidden.get_device(), w_qkv, q, k_cache, v_cache, token_pos, num_chunks, norm_weight)
    _check(hidden.dtype in _BLOCK_DTYPES and all(t.dtype == hidden.dtype for t in (w_qkv, q, k_cache, v_cache)),
           "hidden, w_qkv, q and the caches must share a bfloat16 or float16 dtype")
    _check(all(t.is_contiguous() for t in (hidden, w_qkv, q, k_cache, v_cache)), "tensors must be contiguous")
    _check(k_cache.dim() == 4 and k_cache.shape == v_cache.shape, "caches must be [batch, heads, capacity, head_dim]")
    B, H, cap, D = k_cache.shape
    _check(tuple(hidden.shape) == (B, H * D) and tuple(w_qkv.shape) == (3 * H * D, H * D)
           and tuple(q.shape) == (B, H, D), "hidden [batch, H*D], w_qkv [3*H*D, H*D], q [batch, H, D]")
    _check(token_pos.dtype == torch.int64 and token_pos.numel() == 1, "token_pos must be a one-element int64 tensor")
    if num_chunks is not None:
        _check(num_chunks.is_cuda and num_chunks.dtype == torch.int32 and num_chunks.numel() == 1,
               "num_chunks must be a one-element int32 CUDA tensor")
    if norm_weight is not None:
        _check(norm_weight.is_cuda and norm_weight.dtype == hidden.dtype and norm_weight.numel() == H * D,
               "norm_weight must be a [H*D] tensor of hidden's dtype")
    with torch.cuda.device(hidden.device):
        _rc(lib().csahca_block_qkv(_ptr(hidden), _ptr(norm_weight), float(eps), _ptr(w_qkv), _ptr(q), _ptr(k_cache),
                                   _ptr(v_cache), _ptr(token_pos), _ptr(num_chunks), _DTYPES[hidden.dtype], B, H, D,
                                   cap, int(chunk_size), _stream()))
    return q


@traced
def csa_decode_step_at(q, k_cache, v_cache, summary, token_pos, chunk_size, top_k, *, out=None, indices=None):
    """The decode step of the token at ``token_pos`` (one-element int64 CUDA
    tensor, read on the device) just appended to a growing cache: the chunks in
    play are min((pos + 1) // chunk_size, max_chunks); if the token completes a
    chunk, its summary row (``summary``: fp32 [batch, heads, max_chunks, D],
    updated in place) is built first, bit-identical to csa_chunk_summary.  One
    launch in place of csa_chunk_summary_at + csa_decode_step_dev.  Returns
    ``(out, chunk_indices)``."""
    chunk_size, top_k = int(chunk_size), int(top_k)
    _csa_checks(q, k_cache, v_cache, None, chunk_size, tiled=False)
    _check(summary.is_cuda and summary.is_contiguous() and summary.dtype == torch.float32 and summary.dim() == 4,
           "summary must be a contiguous fp32 [batch, heads, chunks, head_dim] CUDA tensor")
    _check(token_pos.is_cuda and token_pos.dtype == torch.int64 and token_pos.numel() == 1,
           "token_pos must be a one-element int64 CUDA tensor")
    B, H, D = q.shape
    S = k_cache.shape[2]
    _check(tuple(summary.shape[:2]) == (B, H) and summary.shape[3] == D, "summary shape must match q")
    Cs = summary.shape[2]
    _check(top_k >= 0, "top_k must be non-negative")
    k = min(top_k, Cs)
    if _MULTI_DEVICE:
        _same_device(q.get_device(), summary, token_pos, out, indices)
    with torch.cuda.device(q.device):
        if out is None:
            out = torch.empty_like(q)
        if indices is None:
            indices = torch.empty((B, H, k), dtype=torch.int32, device=q.device)
        _check(out.shape == q.shape and out.dtype == q.dtype and out.is_contiguous(), "out must match q")
        _check(tuple(indices.shape) == (B, H, k) and indices.dtype == torch.int32 and indices.is_contiguous(),
               "indices must be a contiguous int32 [batch, heads, min(top_k, max_chunks)] tensor")
        ws = _step_workspace(lib().csahca_csa_step_workspace_bytes(B, H, Cs, D, top_k, chunk_size), q.device,
                             (B * H, Cs, D, k, chunk_size))
        _rc(lib().csahca_csa_decode_step_at(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(summary), _ptr(token_pos),
                                            _ptr(out), _ptr(indices), _DTYPES[q.dtype], B, H, S, D, Cs, chunk_size,
                                            top_k, _ptr(ws), ws.numel(), _stream()))
    return out, indices


def csa_step_status(device=None) -> dict:
    """Sticky status words of this process's step workspaces (0 = healthy; bit 0:
    an exchange wait timed out, the affected heads returned NaN and stay poisoned
    until their workspace is released).  Synchronises the calling stream."""
    out = {}
    for key, (ws, _) in _STEP_WS.items():
        if device is not None and key[0] != torch.device(device).index:
            continue
        val = ctypes.c_uint32(0)
        with torch.cuda.device(ws.device):
            _rc(lib().csahca_csa_step_status(_ptr(ws), ctypes.byref(val), _stream()))
        out[key] = val.value
    return out


def csa_step_noalloc_status(device=None) -> int:
    """Sticky status word of csa_decode_step_noalloc's static state on
    ``device`` (default: the current one): 0 = healthy, bit 0 = an exchange
    wait timed out and the affected head slots stay poisoned until
    csa_step_noalloc_reset().  Synchronises the calling stream."""
    val = ctypes.c_uint32(0)
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        _rc(lib().csahca_csa_step_status(None, ctypes.byref(val), _stream()))
    return val.value


def csa_step_noalloc_reset(device=None) -> None:
    """Zero csa_decode_step_noalloc's static state on ``device`` (a fill kernel
    on the current stream; allocates nothing), clearing poisoned head slots."""
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        _rc(lib().csahca_csa_step_noalloc_reset(_stream()))


@traced
def hca_decode_forward(q, k_cache, v_cache, chunk_size, *, blend=None, csa_weight: float = 0.7):
    """hca_reference (hybrid_attention/reference.py:87-92) on the GPU: dense
    attention over the chunk means of K and V, both rounded to the storage
    type.  With ``blend`` (a [B,H,D] tensor of q's dtype) the result is
    ``csa_weight*blend + (1-csa_weight)*hca`` rounded as in hybrid_reference
    (reference.py:95-108)."""
    chunk_size = int(chunk_size)
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _check(t.is_cuda, f"{name} must be a CUDA tensor")
        _check(t.is_contiguous(), f"{name} must be contiguous")
    _check(q.dim() == 3, "q must be [batch, heads, head_dim]")
    _check(k_cache.dim() == 4 and v_cache.shape == k_cache.shape, "k_cache and v_cache must be [batch, heads, seq_len, head_dim]")
    _check(q.dtype in _DTYPES and k_cache.dtype == q.dtype and v_cache.dtype == q.dtype,
           "q, k_cache and v_cache must have the same floating dtype")
    B, H, S, D = k_cache.shape
    _check(tuple(q.shape) == (B, H, D), "q shape must match k_cache")
    if blend is not None:
        _check(blend.is_cuda and blend.is_contiguous() and blend.dtype == q.dtype and blend.shape == q.shape,
               "blend must be a contiguous CUDA tensor shaped and typed like q")
    if _MULTI_DEVICE:
        _same_device(q.get_device(), k_cache, v_cache, blend)
    with torch.cuda.device(q.device):
        out = torch.empty_like(q)
        ws = _workspace(lib().csahca_hca_decode_workspace_bytes(B, H, S, D, chunk_size), q.device)
        _rc(lib().csahca_hca_decode_forward(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(blend), float(csa_weight),
                                            _ptr(out), _DTYPES[q.dtype], B, H, S, D, chunk_size, _ptr(ws),
                                            ws.numel(), _stream()))
    return out


@traced
def hybrid_decode_forward(q, k_cache, v_cache, *, csa_chunk_size: int, csa_top_k: int, hca_chunk_size: int,
                          csa_weight: float = 0.7, summary=None):
    """hybrid_reference (hybrid_attention/reference.py:95-108) on the GPU: the
    CSA decode step (selection from the chunk summaries of K, built here when
    ``summary`` is None) blended with HCA at ``csa_weight``.  Building the
    summary here needs whole chunks, as chunk_mean does (reference.py:40-42)."""
    if summary is None:
        _check(int(csa_chunk_size) > 0, "chunk_size must be positive")
        _check(k_cache.dim() == 4 and k_cache.shape[2] % int(csa_chunk_size) == 0,
               "seq length must be divisible by chunk_size")
        summary = csa_chunk_summary(k_cache, csa_chunk_size)
    csa_chunk_size, csa_top_k, hca_chunk_size = int(csa_chunk_size), int(csa_top_k), int(hca_chunk_size)
    _csa_checks(q, k_cache, v_cache, None, csa_chunk_size, tiled=False)
    _check(summary.is_cuda and summary.is_contiguous() and summary.dtype == torch.float32 and summary.dim() == 4,
           "summary must be a contiguous fp32 [batch, heads, chunks, head_dim] CUDA tensor")
    B, H, S, D = k_cache.shape
    _check(tuple(summary.shape[:2]) == (B, H) and summary.shape[3] == D, "summary shape must match q")
    C = summary.shape[2]
    _check(csa_top_k >= 0, "top_k must be non-negative")
    k = min(csa_top_k, C)
    if _MULTI_DEVICE:
        _same_device(q.get_device(), summary)
    with torch.cuda.device(q.device):
        out = torch.empty_like(q)
        csa_out = torch.empty_like(q)
        idx = torch.empty((B, H, k), dtype=torch.int32, device=q.device)
        sws = _step_workspace(lib().csahca_csa_step_workspace_bytes(B, H, C, D, csa_top_k, csa_chunk_size), q.device,
                              (B * H, C, D, k, csa_chunk_size))
        hws = _workspace(lib().csahca_hca_decode_workspace_bytes(B, H, S, D, hca_chunk_size), q.device)
        _rc(lib().csahca_hybrid_decode_forward(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(summary), _ptr(csa_out),
                                               _ptr(idx), _ptr(out), _DTYPES[q.dtype], B, H, S, D, C, csa_chunk_size,
                                               csa_top_k, hca_chunk_size, float(csa_weight), _ptr(sws), sws.numel(),
                                               _ptr(hws), hws.numel(), _stream()))
    return out


# ---------------------------------------------------------------------------
# DSV4
# ---------------------------------------------------------------------------
_DSV4_HEAD_DIM = 512


def _dsv4_common(q, cache, token_indices, topk_lengths, attn_sink, page_size, allow_empty: bool):
    """The reference's TORCH_CHECKs of the DSV4 ops, in their order (inline
    tests: they run on every eager call)."""
    msg = _dsv4_common_error(q, cache, token_indices, topk_lengths, attn_sink, page_size)
    if msg is not None:
        raise RuntimeError(msg)
    if _MULTI_DEVICE:
        _same_device(q.get_device(), cache, token_indices, topk_lengths, attn_sink)


def _dsv4_common_error(q, cache, token_indices, topk_lengths, attn_sink, page_size):
    has_len, has_sink = topk_lengths is not None, attn_sink is not None
    if has_len and not topk_lengths.is_cuda:
        return "topk_lengths must be CUDA when defined"
    if has_sink and not attn_sink.is_cuda:
        return "attn_sink must be CUDA when defined"
    if not q.is_contiguous():
        return "q must be contiguous"
    if not cache.is_contiguous():
        return "paged_k_cache_u8 must be contiguous"
    if not token_indices.is_contiguous():
        return "token_indices must be contiguous"
    if has_len and not topk_lengths.is_contiguous():
        return "topk_lengths must be contiguous"
    if has_sink and not attn_sink.is_contiguous():
        return "attn_sink must be contiguous"
    if q.dim() != 3:
        return "q must be [num_queries, heads, 512]"
    if q.shape[2] != _DSV4_HEAD_DIM:
        return "q head_dim must be 512 for DSV4"
    if cache.dim() != 2:
        return "paged_k_cache_u8 must be [num_pages, bytes_per_page]"
    if cache.dtype != torch.uint8:
        return "paged_k_cache_u8 must be uint8"
    if token_indices.dim() != 2:
        return "token_indices must be [num_queries, topk_slots]"
    if token_indices.dtype != torch.int32:
        return "token_indices must be int32"
    if has_len and topk_lengths.dtype != torch.int32:
        return "topk_lengths must be int32 when defined"
    if has_sink and attn_sink.dtype != torch.float32:
        return "attn_sink must be float32 when defined"
    if not page_size > 0:
        return "page_size must be positive"
    if q.dtype not in _FLOATING:
        return f"unsupported dtype {q.dtype}"
    nq, heads = q.shape[0], q.shape[1]
    if token_indices.shape[0] != nq:
        return "token_indices query dimension must match q"
    # None and empty tensors both mean "absent" on every route (the reference's
    # untiled ops reject the empty tensors its own wrappers pass for None).
    if has_len and topk_lengths.numel() > 0 and topk_lengths.numel() != nq:
        return "topk_lengths must have one value per query"
    if has_sink and attn_sink.numel() > 0 and attn_sink.numel() != heads:
        return "attn_sink must have one value per head"
    if cache.shape[1] < page_size * (576 + 8):
        return "bytes_per_page is too small for DSV4 page layout"
    return None


def _dsv4_extra_checks(extra_cache, extra_token_indices, extra_topk_lengths, nq, dev: int):
    msg = _dsv4_extra_error(extra_cache, extra_token_indices, extra_topk_lengths, nq)
    if msg is not None:
        raise RuntimeError(msg)
    if _MULTI_DEVICE:
        _same_device(dev, extra_cache, extra_token_indices, extra_topk_lengths)


def _dsv4_extra_error(extra_cache, extra_token_indices, extra_topk_lengths, nq):
    has_len = extra_topk_lengths is not None
    if not extra_cache.is_cuda:
        return "extra_paged_k_cache_u8 must be CUDA"
    if not extra_token_indices.is_cuda:
        return "extra_token_indices must be CUDA"
    if has_len and not extra_topk_lengths.is_cuda:
        return "extra_topk_lengths must be CUDA when defined"
    if not extra_cache.is_contiguous():
        return "extra_paged_k_cache_u8 must be contiguous"
    if not extra_token_indices.is_contiguous():
        return "extra_token_indices must be contiguous"
    if has_len and not extra_topk_lengths.is_contiguous():
        return "extra_topk_lengths must be contiguous"
    if extra_cache.dim() != 2:
        return "extra_paged_k_cache_u8 must be [num_pages, bytes_per_page]"
    if extra_cache.dtype != torch.uint8:
        return "extra_paged_k_cache_u8 must be uint8"
    if extra_token_indices.dim() != 2:
        return "extra_token_indices must be [num_queries, extra_topk_slots]"
    if extra_token_indices.dtype != torch.int32:
        return "extra_token_indices must be int32"
    len_present = has_len and extra_topk_lengths.numel() > 0
    if len_present and extra_topk_lengths.dtype != torch.int32:
        return "extra_topk_lengths must be int32 when defined"
    if extra_token_indices.shape[0] != nq:
        return "extra_token_indices query dimension must match q"
    if len_present and extra_topk_lengths.numel() != nq:
        return "extra_topk_lengths must have one value per query"
    return None


def _opt(t):
    return t if _present(t) else None


@traced
def dsv4_decode_forward_tiled(q, paged_k_cache_u8, token_indices, topk_lengths, extra_paged_k_cache_u8,
                              extra_token_indices, extra_topk_lengths, attn_sink, page_size, extra_page_size,
                              tile_size, softmax_scale):
    """Reference op dsv4_decode_forward_tiled (tile_size 0 = automatic)."""
    page_size, extra_page_size, tile_size = int(page_size), int(extra_page_size), int(tile_size)
    if not (q.is_cuda and paged_k_cache_u8.is_cuda and token_indices.is_cuda):
        raise RuntimeError("q, paged_k_cache_u8, and token_indices must be CUDA tensors")
    _dsv4_common(q, paged_k_cache_u8, token_indices, topk_lengths, attn_sink, page_size, allow_empty=True)
    if paged_k_cache_u8.shape[1] % 4 != 0:
        raise RuntimeError("tiled DSV4 kernel requires bytes_per_page divisible by 4 for vectorized loads")
    nq, heads = q.shape[0], q.shape[1]
    has_extra = (extra_paged_k_cache_u8 is not None and extra_paged_k_cache_u8.numel() > 0
                 and extra_token_indices is not None and extra_token_indices.numel() > 0)
    extra_slots = 0
    if has_extra:
        _dsv4_extra_checks(extra_paged_k_cache_u8, extra_token_indices, extra_topk_lengths, nq, q.get_device())
        if extra_page_size <= 0:
            raise RuntimeError("extra_page_size must be positive")
        ebpp = extra_paged_k_cache_u8.shape[1]
        if ebpp < extra_page_size * (576 + 8):
            raise RuntimeError("extra_bytes_per_page is too small for DSV4 page layout")
        if ebpp % 4 != 0:
            raise RuntimeError("tiled DSV4 kernel requires extra_bytes_per_page divisible by 4 for vectorized loads")
        extra_slots = extra_token_indices.shape[1]
    dev = q.get_device()
    if dev != _current_device():
        with torch.cuda.device(dev):
            return dsv4_decode_forward_tiled(q, paged_k_cache_u8, token_indices, topk_lengths, extra_paged_k_cache_u8,
                                             extra_token_indices, extra_topk_lengths, attn_sink, page_size,
                                             extra_page_size, tile_size, softmax_scale)
    out = torch.empty_like(q)
    if nq == 0 or heads == 0:
        return out
    stream = _raw_stream(dev)
    ws = _scratch_workspace(_ws_bytes("csahca_dsv4_decode_workspace_bytes", nq, heads, token_indices.shape[1],
                                      extra_slots, tile_size), dev, stream)
    ec = extra_paged_k_cache_u8 if has_extra else None
    _rc(lib().csahca_dsv4_decode_forward_tiled(
        q.data_ptr(), _DTYPES[q.dtype], nq, heads, paged_k_cache_u8.data_ptr(), paged_k_cache_u8.shape[0],
        paged_k_cache_u8.shape[1], page_size, token_indices.data_ptr(), token_indices.shape[1],
        _ptr(_opt(topk_lengths)), _ptr(ec), ec.shape[0] if has_extra else 0,
        ec.shape[1] if has_extra else 0, extra_page_size if has_extra else 1,
        _ptr(extra_token_indices) if has_extra else None, extra_slots,
        _ptr(_opt(extra_topk_lengths)) if has_extra else None, _ptr(_opt(attn_sink)), float(softmax_scale),
        tile_size, out.data_ptr(), ws.data_ptr(), ws.numel(), stream))
    return out


@traced
def dsv4_swa_decode_forward(q, paged_k_cache_u8, token_indices, topk_lengths, attn_sink, page_size,
                            softmax_scale):
    """Reference op dsv4_swa_decode_forward (SWA slots only)."""
    page_size = int(page_size)
    if not (q.is_cuda and paged_k_cache_u8.is_cuda and token_indices.is_cuda):
        raise RuntimeError("q, paged_k_cache_u8, and token_indices must be CUDA tensors")
    _dsv4_common(q, paged_k_cache_u8, token_indices, topk_lengths, attn_sink, page_size, allow_empty=True)
    nq, heads = q.shape[0], q.shape[1]
    dev = q.get_device()
    if dev != _current_device():
        with torch.cuda.device(dev):
            return dsv4_swa_decode_forward(q, paged_k_cache_u8, token_indices, topk_lengths, attn_sink, page_size,
                                           softmax_scale)
    out = torch.empty_like(q)
    if nq == 0 or heads == 0:
        return out
    stream = _raw_stream(dev)
    ws = _scratch_workspace(_ws_bytes("csahca_dsv4_decode_workspace_bytes", nq, heads, token_indices.shape[1], 0, 0),
                            dev, stream)
    _rc(lib().csahca_dsv4_swa_decode_forward(
        q.data_ptr(), _DTYPES[q.dtype], nq, heads, paged_k_cache_u8.data_ptr(), paged_k_cache_u8.shape[0],
        paged_k_cache_u8.shape[1], page_size, token_indices.data_ptr(), token_indices.shape[1],
        _ptr(_opt(topk_lengths)), _ptr(_opt(attn_sink)), float(softmax_scale), out.data_ptr(), ws.data_ptr(),
        ws.numel(), stream))
    return out


@traced
def dsv4_sparse_decode_forward(q, paged_k_cache_u8, token_indices, topk_lengths, extra_paged_k_cache_u8,
                               extra_token_indices, extra_topk_lengths, attn_sink, page_size, extra_page_size,
                               softmax_scale):
    """Reference op dsv4_sparse_decode_forward (SWA + C4/C128 extra slots)."""
    page_size, extra_page_size = int(page_size), int(extra_page_size)
    if not (q.is_cuda and paged_k_cache_u8.is_cuda and token_indices.is_cuda
            and extra_paged_k_cache_u8.is_cuda and extra_token_indices.is_cuda):
        raise RuntimeError("q, paged_k_cache_u8, token_indices, extra_paged_k_cache_u8, and extra_token_indices "
                           "must be CUDA tensors")
    _dsv4_common(q, paged_k_cache_u8, token_indices, topk_lengths, attn_sink, page_size, allow_empty=True)
    nq, heads = q.shape[0], q.shape[1]
    _dsv4_extra_checks(extra_paged_k_cache_u8, extra_token_indices, extra_topk_lengths, nq, q.get_device())
    _check(extra_page_size > 0, "extra_page_size must be positive")
    _check(extra_paged_k_cache_u8.shape[1] >= extra_page_size * (576 + 8),
           "extra_bytes_per_page is too small for DSV4 page layout")
    dev = q.get_device()
    if dev != _current_device():
        with torch.cuda.device(dev):
            return dsv4_sparse_decode_forward(q, paged_k_cache_u8, token_indices, topk_lengths,
                                              extra_paged_k_cache_u8, extra_token_indices, extra_topk_lengths,
                                              attn_sink, page_size, extra_page_size, softmax_scale)
    out = torch.empty_like(q)
    if nq == 0 or heads == 0:
        return out
    stream = _raw_stream(dev)
    ws = _scratch_workspace(_ws_bytes("csahca_dsv4_decode_workspace_bytes", nq, heads, token_indices.shape[1],
                                      extra_token_indices.shape[1], 0), dev, stream)
    _rc(lib().csahca_dsv4_sparse_decode_forward(
        q.data_ptr(), _DTYPES[q.dtype], nq, heads, paged_k_cache_u8.data_ptr(), paged_k_cache_u8.shape[0],
        paged_k_cache_u8.shape[1], page_size, token_indices.data_ptr(), token_indices.shape[1],
        _ptr(_opt(topk_lengths)), extra_paged_k_cache_u8.data_ptr(), extra_paged_k_cache_u8.shape[0],
        extra_paged_k_cache_u8.shape[1], extra_page_size, extra_token_indices.data_ptr(),
        extra_token_indices.shape[1], _ptr(_opt(extra_topk_lengths)), _ptr(_opt(attn_sink)),
        float(softmax_scale), out.data_ptr(), ws.data_ptr(), ws.numel(), stream))
    return out


# ---------------------------------------------------------------------------
# Device clock stamps (timing inside captured graphs)
# ---------------------------------------------------------------------------
def device_clock_stamp(stamps: torch.Tensor, index: int) -> None:
    """Store the device wall clock at stamps[index] (int64, on the device) when
    the current stream reaches this point; capturable into a HIP graph."""
    _check(stamps.is_cuda and stamps.dtype == torch.int64 and stamps.is_contiguous(),
           "stamps must be a contiguous int64 CUDA tensor")
    _check(0 <= index < stamps.numel(), "stamp index out of range")
    _rc(lib().csahca_device_clock_stamp(stamps.data_ptr() + 8 * index, _stream()))


def device_clock_khz() -> int:
    """Rate of the device wall clock in kHz."""
    khz = lib().csahca_device_clock_khz()
    if khz <= 0:
        raise RuntimeError("the device wall clock rate query failed")
    return int(khz)


# ---------------------------------------------------------------------------
# Launch profiler
# ---------------------------------------------------------------------------
class profile_launches:
    """Context manager: per-kernel device durations of the library's launches on
    this thread (hipExtLaunchKernel start/stop events).  After the block,
    ``.results`` maps kernel name -> dict(launches, total_ms, min_ms, max_ms,
    avg_us)."""

    def __enter__(self):
        _rc(lib().csahca_profile_begin())
        self.results = {}
        return self

    def __exit__(self, *exc):
        n = lib().csahca_profile_end()
        if n < 0:
            raise RuntimeError(lib().csahca_last_error().decode())
        for i in range(n):
            name = ctypes.c_char_p()
            cnt = _i64()
            tot, mn, mx = _dbl(), _dbl(), _dbl()
            _rc(lib().csahca_profile_result(i, ctypes.byref(name), ctypes.byref(cnt), ctypes.byref(tot),
                                            ctypes.byref(mn), ctypes.byref(mx)))
            self.results[name.value.decode()] = dict(launches=cnt.value, total_ms=tot.value, min_ms=mn.value,
                                                     max_ms=mx.value, avg_us=1e3 * tot.value / max(cnt.value, 1))
        return False


@traced
def dsv4_pack_tokens(k_tokens, page_size, *, cache=None, locs=None):
    """pack_dsv4_cache (hybrid_attention/dsv4_correctness.py:24-59) on the GPU:
    quantise [T, 512] bf16 tokens into the paged FP8 layout.  Without ``cache``
    a zeroed [ceil(T/page_size), bytes_per_page] uint8 cache is allocated and
    token t written at location t, exactly as the reference does; with
    ``cache`` (and optionally int32 ``locs``) tokens are written in place at
    their locations -- the quantize-on-write of a serving cache."""
    page_size = int(page_size)
    _check(k_tokens.is_cuda and k_tokens.dtype == torch.bfloat16, "k_tokens must be bfloat16")
    _check(k_tokens.dim() == 2 and k_tokens.shape[1] == _DSV4_HEAD_DIM, "k_tokens must be [tokens, 512]")
    _check(page_size > 0, "page_size must be positive")
    k_tokens = k_tokens.contiguous()
    T = k_tokens.shape[0]
    lib()  # fail before allocating when the library is missing
    with torch.cuda.device(k_tokens.device):
        if cache is None:
            from .dsv4_layout import bytes_per_page
            cache = torch.zeros(((T + page_size - 1) // page_size, bytes_per_page(page_size)), dtype=torch.uint8,
                                device=k_tokens.device)
        _check(cache.is_cuda and cache.dim() == 2 and cache.is_contiguous(),
               "paged_k_cache_u8 must be [num_pages, bytes_per_page]")
        cache_u8 = cache.view(torch.uint8)
        if locs is not None:
            _check(locs.is_cuda and locs.dtype == torch.int32 and locs.numel() == T, "locs must be int32 [tokens]")
            locs = locs.contiguous()
        if _MULTI_DEVICE:
            _same_device(k_tokens.get_device(), cache, locs)
        _rc(lib().csahca_dsv4_pack_tokens(_ptr(k_tokens), _ptr(locs), T, _ptr(cache_u8), cache_u8.shape[0],
                                          cache_u8.shape[1], page_size, _stream()))
    return cache
