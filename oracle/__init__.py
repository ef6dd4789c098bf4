"""CPU oracle for the CSAHCA decode path -- TEST INFRASTRUCTURE ONLY.

A plain-C restatement (``csahca_oracle.c``) of the reference's CSA and DSV4
algorithms, loaded through ctypes.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only as
the checker (or the timed CPU baseline); the product package ``csahca_amd``
never imports it and has no CPU fallback.

Each wrapper names the reference function it restates; the C file carries the
file:line citations.  Inputs may be numpy arrays or CPU torch tensors; floating
inputs are converted to exact fp32 copies, results come back as float64 numpy
arrays (unrounded) unless stated otherwise.

Parity pins (see the C header): format helpers against torch casts, everything
else against golden vectors written by the reference's own functions
(tests/golden/), closed forms and planted-chunk known answers.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_LIB = None

F32, F16, BF16, F64 = 0, 1, 2, 3

DIM_NOPE = 448
DIM_ROPE = 64
HEAD_DIM = DIM_NOPE + DIM_ROPE
TILE_SIZE = 64
NUM_SCALE_TILES = DIM_NOPE // TILE_SIZE
NOPE_ROPE_BYTES = DIM_NOPE + DIM_ROPE * 2
SCALE_BYTES_PER_TOKEN = NUM_SCALE_TILES + 1

_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_f64p = ctypes.POINTER(ctypes.c_double)
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_i64p = ctypes.POINTER(ctypes.c_int64)
_c_u8p = ctypes.POINTER(ctypes.c_uint8)
_c_u16p = ctypes.POINTER(ctypes.c_uint16)
_i64 = ctypes.c_int64


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB_PATH


def lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build()
        _LIB = ctypes.CDLL(str(_LIB_PATH))
        _declare(_LIB)
    return _LIB


def _declare(L) -> None:
    L.orc_e4m3fn_decode.restype = ctypes.c_float
    L.orc_e4m3fn_decode.argtypes = [ctypes.c_uint8]
    L.orc_e4m3fn_encode.restype = ctypes.c_uint8
    L.orc_e4m3fn_encode.argtypes = [ctypes.c_float]
    L.orc_e4m3fn_encode_array.argtypes = [_c_f32p, _c_u8p, _i64]
    L.orc_round_array.argtypes = [_c_f32p, _c_f32p, _i64, ctypes.c_int]
    L.orc_chunk_mean.argtypes = [_c_f32p, _i64, _i64, _i64, _i64, _i64, _c_f32p]
    L.orc_select_topk.argtypes = [_c_f32p, _c_f32p, _i64, _i64, _i64, _i64, _i64, _c_i32p, _c_f64p]
    L.orc_csa_attend.argtypes = [_c_f32p, _c_f32p, _c_f32p, _c_i64p, _i64, _i64, _i64, _i64, _i64,
                                 _i64, ctypes.c_int, _c_f64p, ctypes.c_int]
    L.orc_full_attend.argtypes = [_c_f32p, _c_f32p, _c_f32p, _i64, _i64, _i64, _i64, ctypes.c_int,
                                  _c_f64p]
    L.orc_hca.argtypes = [_c_f32p, _c_f32p, _c_f32p, _i64, _i64, _i64, _i64, _i64, ctypes.c_int,
                          _c_f64p]
    L.orc_csa_decode_step.argtypes = [_c_f32p, _c_f32p, _c_f32p, _c_f32p, _i64, _i64, _i64, _i64,
                                      _i64, _i64, ctypes.c_int, _c_i32p, _c_i64p, _c_f64p,
                                      ctypes.c_int]
    L.orc_dsv4_bytes_per_page.restype = ctypes.c_int64
    L.orc_dsv4_bytes_per_page.argtypes = [_i64]
    L.orc_dsv4_pack.argtypes = [_c_u16p, _i64, _i64, _c_u8p]
    L.orc_dsv4_dequant.argtypes = [_c_u8p, _i64, _c_i32p, _i64, _i64, _c_f32p]
    L.orc_dsv4_attention.argtypes = [_c_f32p, _i64, _i64, _c_u8p, _i64, _i64, _c_i32p, _i64,
                                     _c_i32p, _c_f32p, _i64, ctypes.c_double, _c_u8p, _i64, _i64,
                                     _c_i32p, _i64, _c_i32p, _i64, _c_f64p]


# --------------------------------------------------------------------------
# conversion helpers
# --------------------------------------------------------------------------

def _np(x) -> np.ndarray:
    if hasattr(x, "detach"):  # torch tensor
        import torch

        t = x.detach().cpu()
        if t.dtype in (torch.bfloat16, torch.float16):
            t = t.float()
        return t.numpy()
    return np.asarray(x)


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(_np(x), dtype=np.float32)


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctype)


def dtype_code(dtype) -> int:
    """Map a torch dtype (or name) to the oracle's storage-type code."""
    name = str(dtype).replace("torch.", "")
    return {"float32": F32, "float16": F16, "bfloat16": BF16, "float64": F64}[name]


def round_to(x, dtype) -> np.ndarray:
    """Round an array to a storage dtype (bf16/f16 ties-to-even), returned as fp32."""
    a = _f32(x)
    out = np.empty_like(a)
    lib().orc_round_array(_ptr(a, _c_f32p), _ptr(out, _c_f32p), a.size, dtype_code(dtype))
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3fn_decode(b: int) -> float:
    return float(lib().orc_e4m3fn_decode(int(b)))


def e4m3fn_encode(x: float) -> int:
    return int(lib().orc_e4m3fn_encode(float(x)))


def e4m3fn_encode_array(x) -> np.ndarray:
    a = _f32(x).reshape(-1)
    out = np.empty(a.size, dtype=np.uint8)
    lib().orc_e4m3fn_encode_array(_ptr(a, _c_f32p), _ptr(out, _c_u8p), a.size)
    return out


# --------------------------------------------------------------------------
# CSA (hybrid_attention/reference.py, csrc/csa_attention.cu)
# --------------------------------------------------------------------------

def chunk_mean(k, chunk_size: int) -> np.ndarray:
    """reference.py:40-45 -> fp32 [B,H,S//chunk,D]."""
    a = _f32(k)
    B, H, S, D = a.shape
    out = np.empty((B, H, S // chunk_size, D), dtype=np.float32)
    lib().orc_chunk_mean(_ptr(a, _c_f32p), B, H, S, D, chunk_size, _ptr(out, _c_f32p))
    return out


def select_topk(q, summary, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """reference.py:48-56 scoring + top-k from summaries.

    Returns (indices int32 [B,H,min(k,C)], scores float64 [B,H,C]); order is
    score descending, equal scores by ascending chunk index.
    """
    qa = _f32(q)
    sa = _f32(summary)
    B, H, C, D = sa.shape
    k = min(int(top_k), C)
    idx = np.empty((B, H, k), dtype=np.int32)
    scores = np.empty((B, H, C), dtype=np.float64)
    lib().orc_select_topk(_ptr(qa, _c_f32p), _ptr(sa, _c_f32p), B, H, C, D, k,
                          _ptr(idx, _c_i32p), _ptr(scores, _c_f64p))
    return idx, scores


def select_topk_chunks(q, k_cache, chunk_size: int, top_k: int) -> np.ndarray:
    """reference.py:48-56 end to end (chunk_mean then scoring + top-k)."""
    return select_topk(q, chunk_mean(k_cache, chunk_size), top_k)[0]


def csa_attend(q, k, v, indices, chunk_size: int, prob_dtype=F32, nthreads: int = 1) -> np.ndarray:
    """Sparse decode over chunk ids; float64 [B,H,D] (unrounded).

    prob_dtype=F32: the cuda-csa / cuda-csa-tiled op math (csa_attention.cu);
    prob_dtype=<value dtype>: torch-csa (reference.py:69-84), which rounds the
    softmax probabilities to the value dtype before the weighted sum.
    """
    qa, ka, va = _f32(q), _f32(k), _f32(v)
    ia = np.ascontiguousarray(_np(indices), dtype=np.int64)
    B, H, S, D = ka.shape
    top_k = ia.shape[-1]
    out = np.empty((B, H, D), dtype=np.float64)
    code = prob_dtype if isinstance(prob_dtype, int) else dtype_code(prob_dtype)
    lib().orc_csa_attend(_ptr(qa, _c_f32p), _ptr(ka, _c_f32p), _ptr(va, _c_f32p), _ptr(ia, _c_i64p),
                         B, H, S, D, top_k, chunk_size, code, _ptr(out, _c_f64p), nthreads)
    return out


def csa_reference(q, k, v, *, chunk_size: int, top_k: int, selected_chunks=None, dtype=None):
    """torch-csa (reference.py:69-84); probabilities rounded to ``dtype``
    (default: bfloat16, the value dtype of the headline config)."""
    if selected_chunks is None:
        selected_chunks = select_topk_chunks(q, k, chunk_size, top_k)
    pd = BF16 if dtype is None else (dtype if isinstance(dtype, int) else dtype_code(dtype))
    return csa_attend(q, k, v, selected_chunks, chunk_size, prob_dtype=pd)


def full_decode_attention(q, k, v, prob_dtype=F32) -> np.ndarray:
    """reference.py:31-37 over every token."""
    qa, ka, va = _f32(q), _f32(k), _f32(v)
    B, H, S, D = ka.shape
    out = np.empty((B, H, D), dtype=np.float64)
    code = prob_dtype if isinstance(prob_dtype, int) else dtype_code(prob_dtype)
    lib().orc_full_attend(_ptr(qa, _c_f32p), _ptr(ka, _c_f32p), _ptr(va, _c_f32p), B, H, S, D, code,
                          _ptr(out, _c_f64p))
    return out


def hca_reference(q, k, v, *, chunk_size: int, dtype=BF16) -> np.ndarray:
    """reference.py:87-92."""
    qa, ka, va = _f32(q), _f32(k), _f32(v)
    B, H, S, D = ka.shape
    out = np.empty((B, H, D), dtype=np.float64)
    code = dtype if isinstance(dtype, int) else dtype_code(dtype)
    lib().orc_hca(_ptr(qa, _c_f32p), _ptr(ka, _c_f32p), _ptr(va, _c_f32p), B, H, S, D, chunk_size,
                  code, _ptr(out, _c_f64p))
    return out


class DecodeStepTimer:
    """Holds fp32 copies of one CSA decode workload for repeated CPU-baseline steps
    (selection from cached summaries + torch-csa attention, reference.py:51-84)."""

    def __init__(self, q, k, v, summary, chunk_size: int, top_k: int, prob_dtype=BF16):
        self.q, self.k, self.v, self.s = _f32(q), _f32(k), _f32(v), _f32(summary)
        self.B, self.H, self.S, self.D = self.k.shape
        self.chunk, self.top_k = int(chunk_size), int(top_k)
        kk = min(self.top_k, self.S // self.chunk)
        self.idx32 = np.empty((self.B, self.H, kk), dtype=np.int32)
        self.idx64 = np.empty((self.B, self.H, kk), dtype=np.int64)
        self.out = np.empty((self.B, self.H, self.D), dtype=np.float64)
        self.prob_dtype = prob_dtype

    def step(self, nthreads: int = 1) -> np.ndarray:
        lib().orc_csa_decode_step(_ptr(self.q, _c_f32p), _ptr(self.k, _c_f32p), _ptr(self.v, _c_f32p),
                                  _ptr(self.s, _c_f32p), self.B, self.H, self.S, self.D, self.chunk,
                                  self.top_k, self.prob_dtype, _ptr(self.idx32, _c_i32p),
                                  _ptr(self.idx64, _c_i64p), _ptr(self.out, _c_f64p), nthreads)
        return self.out

    def attend(self, nthreads: int = 1) -> np.ndarray:
        """torch-csa attention alone over the selection of the last step() (the
        reference's attend-only mode with precomputed chunk ids)."""
        lib().orc_csa_attend(_ptr(self.q, _c_f32p), _ptr(self.k, _c_f32p), _ptr(self.v, _c_f32p),
                             _ptr(self.idx64, _c_i64p), self.B, self.H, self.S, self.D, self.idx64.shape[-1],
                             self.chunk, self.prob_dtype, _ptr(self.out, _c_f64p), nthreads)
        return self.out


# --------------------------------------------------------------------------
# DSV4 (hybrid_attention/dsv4_correctness.py, csrc/dsv4_attention.cu)
# --------------------------------------------------------------------------

def bytes_per_page(page_size: int) -> int:
    """dsv4_correctness.py:19-21."""
    return int(lib().orc_dsv4_bytes_per_page(int(page_size)))


def _bf16_bits(x) -> np.ndarray:
    if hasattr(x, "detach"):
        import torch

        t = x.detach().cpu().contiguous()
        if t.dtype != torch.bfloat16:
            raise ValueError("k_tokens must be bfloat16")
        return t.view(torch.int16).numpy().view(np.uint16)
    a = np.asarray(x)
    if a.dtype != np.uint16:
        raise ValueError("expected bf16 bit patterns (uint16)")
    return a


def pack_dsv4_cache(k_tokens, *, page_size: int) -> np.ndarray:
    """dsv4_correctness.py:24-59: [T,512] bf16 -> uint8 [pages, bytes_per_page]."""
    bits = np.ascontiguousarray(_bf16_bits(k_tokens))
    T = bits.shape[0]
    pages = (T + page_size - 1) // page_size
    cache = np.zeros((pages, bytes_per_page(page_size)), dtype=np.uint8)
    lib().orc_dsv4_pack(_ptr(bits, _c_u16p), T, page_size, _ptr(cache, _c_u8p))
    return cache


def dequant_dsv4_cache(cache, token_indices, *, page_size: int) -> np.ndarray:
    """dsv4_correctness.py:62-88 -> fp32 [..., 512] holding bf16 values."""
    c = np.ascontiguousarray(_np(cache)).view(np.uint8)
    idx = np.ascontiguousarray(_np(token_indices), dtype=np.int32)
    flat = idx.reshape(-1)
    out = np.empty((flat.size, HEAD_DIM), dtype=np.float32)
    lib().orc_dsv4_dequant(_ptr(c, _c_u8p), c.shape[1], _ptr(flat, _c_i32p), flat.size, page_size,
                           _ptr(out, _c_f32p))
    return out.reshape(*idx.shape, HEAD_DIM)


def _opt_i32(x):
    if x is None:
        return None
    a = np.ascontiguousarray(_np(x), dtype=np.int32)
    return a if a.size else None


def dsv4_reference_attention(q, cache, token_indices, topk_lengths, attn_sink, *, page_size: int,
                             softmax_scale: float, extra_cache=None, extra_token_indices=None,
                             extra_topk_lengths=None, extra_page_size=None) -> np.ndarray:
    """dsv4_correctness.py:91-141 -> float64 [nq,H,512] (unrounded)."""
    qa = _f32(q)
    nq, H, _ = qa.shape
    c = np.ascontiguousarray(_np(cache)).view(np.uint8)
    idx = np.ascontiguousarray(_np(token_indices), dtype=np.int32).reshape(nq, -1)
    lens = _opt_i32(topk_lengths)
    sink = None if attn_sink is None else _f32(attn_sink)
    if sink is not None and sink.size == 0:
        sink = None
    has_extra = extra_cache is not None and extra_token_indices is not None
    if has_extra:
        if extra_page_size is None:
            raise ValueError("extra_page_size is required with extra_cache")
        ec = np.ascontiguousarray(_np(extra_cache)).view(np.uint8)
        eidx = np.ascontiguousarray(_np(extra_token_indices), dtype=np.int32).reshape(nq, -1)
        elens = _opt_i32(extra_topk_lengths)
        has_extra = eidx.shape[1] > 0 and ec.size > 0
    out = np.empty((nq, H, HEAD_DIM), dtype=np.float64)
    null_u8 = ctypes.cast(None, _c_u8p)
    null_i32 = ctypes.cast(None, _c_i32p)
    lib().orc_dsv4_attention(
        _ptr(qa, _c_f32p), nq, H, _ptr(c, _c_u8p), c.shape[0], c.shape[1], _ptr(idx, _c_i32p),
        idx.shape[1], null_i32 if lens is None else _ptr(lens, _c_i32p),
        ctypes.cast(None, _c_f32p) if sink is None else _ptr(sink, _c_f32p), page_size,
        float(softmax_scale),
        _ptr(ec, _c_u8p) if has_extra else null_u8, ec.shape[0] if has_extra else 0,
        ec.shape[1] if has_extra else 0, _ptr(eidx, _c_i32p) if has_extra else null_i32,
        eidx.shape[1] if has_extra else 0,
        (null_i32 if (not has_extra or elens is None) else _ptr(elens, _c_i32p)),
        int(extra_page_size) if has_extra else 1, _ptr(out, _c_f64p))
    return out


def ncores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
