"""Seeded synthetic inputs for the CSA and DSV4 decode paths.

Every tensor is drawn on the CPU generator, in the reference's draw order, and
only then moved to the requested device, so CPU checkers and the GPU kernels
see identical bytes.  (The reference draws with a generator on its target
device -- hybrid_attention/reference.py:126-130 -- whose CUDA stream of numbers
cannot be reproduced here; the CPU generator stream can, and its digests are
pinned by tests/golden/synthetic_hash.json.)
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .dsv4_layout import HEAD_DIM, pack_dsv4_cache


@dataclass(frozen=True)
class SyntheticCase:
    q: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    chunk_size: int
    top_k: int


def make_synthetic_case(*, batch: int = 1, heads: int = 8, seq_len: int = 4096, head_dim: int = 128,
                        chunk_size: int = 64, top_k: int = 8, dtype: torch.dtype = torch.bfloat16,
                        device: str | torch.device = "cpu", seed: int = 0) -> SyntheticCase:
    """Same draws as hybrid_attention/reference.py:111-131 (q, then K, then V, all
    ``randn`` in ``dtype``), taken from a CPU generator seeded with ``seed``."""
    if seq_len % chunk_size != 0:
        raise ValueError("seq_len must be divisible by chunk_size")
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    q = torch.randn(batch, heads, head_dim, dtype=dtype, generator=g)
    k = torch.randn(batch, heads, seq_len, head_dim, dtype=dtype, generator=g)
    v = torch.randn(batch, heads, seq_len, head_dim, dtype=dtype, generator=g)
    return SyntheticCase(q=q.to(device), k_cache=k.to(device), v_cache=v.to(device),
                         chunk_size=chunk_size, top_k=top_k)


def plant_chunks(q: torch.Tensor, k_cache: torch.Tensor, chunks: torch.Tensor, chunk_size: int,
                 alpha: float, *, inplace: bool = False) -> torch.Tensor:
    """Bias the listed chunks of ``k_cache`` towards ``q``.

    ``chunks`` is ``[B, H, n]`` (distinct ids per head); every token of chunk
    ``chunks[b,h,j]`` gets ``(alpha * (n - j)) * q_hat`` added in fp32
    (``q_hat`` = unit ``q[b,h]``) and is rounded back to the cache dtype, so the
    selected set AND its score order are known in advance when ``alpha`` dwarfs
    the spread of the unbiased chunk scores.  Only the planted rows are read and
    written (on whatever device the tensors live); returns a copy unless
    ``inplace``.
    """
    k = k_cache if inplace else k_cache.clone()
    B, H, S, D = k.shape
    n = chunks.shape[-1]
    C = S // chunk_size
    qf = q.float()
    q_hat = qf / qf.norm(dim=-1, keepdim=True)                                      # [B, H, D]
    weight = alpha * (n - torch.arange(n, dtype=torch.float32, device=k.device))     # [n]
    bias = weight[None, None, :, None] * q_hat.to(k.device)[:, :, None, :]           # [B, H, n, D]
    kv = k[:, :, :C * chunk_size].view(B, H, C, chunk_size, D)
    bi = torch.arange(B, device=k.device)[:, None, None]
    hi = torch.arange(H, device=k.device)[None, :, None]
    ci = chunks.to(device=k.device, dtype=torch.long)
    rows = kv[bi, hi, ci].float()                                                   # [B, H, n, chunk, D]
    kv[bi, hi, ci] = (rows + bias[:, :, :, None, :]).to(k.dtype)
    return k


def scattered_chunks(batch: int, heads: int, num_chunks: int, top_k: int) -> torch.Tensor:
    """Chunk ids ``i * num_chunks // top_k`` (uniformly scattered), same for all heads."""
    ids = torch.tensor([i * num_chunks // top_k for i in range(top_k)], dtype=torch.int32)
    return ids.expand(batch, heads, top_k).contiguous()


def clustered_chunks(batch: int, heads: int, num_chunks: int, top_k: int, start: int | None = None) -> torch.Tensor:
    """A contiguous run of ``top_k`` chunk ids starting at ``start`` (default: the middle)."""
    s = (num_chunks - top_k) // 2 if start is None else start
    ids = torch.arange(s, s + top_k, dtype=torch.int32)
    return ids.expand(batch, heads, top_k).contiguous()


@dataclass
class Dsv4Case:
    q: torch.Tensor
    k_tokens: torch.Tensor
    cache: torch.Tensor
    token_indices: torch.Tensor
    topk_lengths: torch.Tensor
    attn_sink: torch.Tensor
    page_size: int
    extra_tokens: torch.Tensor | None = None
    extra_cache: torch.Tensor | None = None
    extra_token_indices: torch.Tensor | None = None
    extra_topk_lengths: torch.Tensor | None = None
    extra_page_size: int | None = None


def make_dsv4_case(*, compress_ratio: int, num_queries: int = 7, heads: int = 8, num_tokens: int = 1024,
                   top_k: int = 128, page_size: int = 256, extra_tokens: int = 1024, extra_top_k: int = 0,
                   extra_page_size: int | None = None, q_dtype: torch.dtype = torch.bfloat16,
                   full_lengths: bool = False, seed: int = 0, device: str | torch.device = "cpu",
                   pack: bool = True) -> Dsv4Case:
    """The draw sequence of hybrid_attention/dsv4_correctness.py:168-227 on a CPU
    generator: q, k_tokens, token_indices, topk_lengths, attn_sink, then for
    compress_ratio 4/128 extra_tokens, extra_token_indices (last two slots -1 when
    extra_top_k >= 4) and extra_topk_lengths.

    ``extra_page_size`` defaults to ``page_size // compress_ratio`` like the
    reference; when that is 0 (e.g. page 64, ratio 128, where the reference
    harness raises) pass it explicitly.  ``full_lengths`` replaces the drawn
    lengths by full ones after the draws (dsv4_benchmark.py:48,74).
    """
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    q = torch.randn(num_queries, heads, HEAD_DIM, dtype=q_dtype, generator=g)
    k_tokens = torch.randn(num_tokens, HEAD_DIM, dtype=torch.bfloat16, generator=g)
    token_indices = torch.randint(0, num_tokens, (num_queries, top_k), dtype=torch.int32, generator=g)
    topk_lengths = torch.randint(max(1, top_k // 2), top_k + 1, (num_queries,), dtype=torch.int32, generator=g)
    attn_sink = torch.randn(heads, dtype=torch.float32, generator=g)
    case = Dsv4Case(q=q, k_tokens=k_tokens, cache=None, token_indices=token_indices, topk_lengths=topk_lengths,
                    attn_sink=attn_sink, page_size=page_size)
    if compress_ratio:
        eps = extra_page_size if extra_page_size is not None else page_size // compress_ratio
        if eps <= 0:
            raise ValueError("extra_page_size must be positive")
        etop = extra_top_k or (512 if compress_ratio == 4 else 128)
        case.extra_tokens = torch.randn(extra_tokens, HEAD_DIM, dtype=torch.bfloat16, generator=g)
        ei = torch.randint(0, extra_tokens, (num_queries, etop), dtype=torch.int32, generator=g)
        if etop >= 4:
            ei[:, -2:] = -1
        case.extra_token_indices = ei
        case.extra_topk_lengths = torch.randint(max(1, etop // 2), etop + 1, (num_queries,), dtype=torch.int32,
                                                generator=g)
        case.extra_page_size = eps
    if full_lengths:
        case.topk_lengths = torch.full((num_queries,), top_k, dtype=torch.int32)
        if compress_ratio:
            case.extra_topk_lengths = torch.full((num_queries,), case.extra_token_indices.shape[1],
                                                 dtype=torch.int32)
    if pack:
        case.cache = pack_dsv4_cache(case.k_tokens.to(device), page_size=page_size)
        if compress_ratio:
            case.extra_cache = pack_dsv4_cache(case.extra_tokens.to(device), page_size=case.extra_page_size)
    for name in ("q", "k_tokens", "token_indices", "topk_lengths", "attn_sink", "extra_tokens",
                 "extra_token_indices", "extra_topk_lengths"):
        t = getattr(case, name)
        if t is not None:
            setattr(case, name, t.to(device))
    return case


def make_dsv4_bench_case(*, compress_ratio: int, num_queries: int = 1, heads: int = 8, num_tokens: int = 4096,
                         top_k: int = 64, page_size: int = 256, extra_tokens: int = 4096, extra_top_k: int = 0,
                         extra_page_size: int | None = None, q_dtype: torch.dtype = torch.bfloat16, seed: int = 0,
                         device: str | torch.device = "cpu") -> Dsv4Case:
    """The inputs of the reference DSV4 benchmark harness
    (hybrid_attention/dsv4_benchmark.py:30-76) on a CPU generator: q, k_tokens,
    token_indices (uniform over the pool), full lengths, sink, then for
    compress_ratio 4/128 extra_tokens and extra_token_indices; extra page size
    ``page_size // compress_ratio`` unless ``extra_page_size`` is given;
    extra_top_k defaults to 512 (C4) / 128 (C128).  Every query draws its own
    slots, independently of the others (a batch of independent sequences).
    Its published H100 cases are nq 1, H 8, top_k 64, page 256 with extra_top_k
    128 (C4) and 64 (C128) (docs/dsv4_abi_status.md:64-65)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    q = torch.randn(num_queries, heads, HEAD_DIM, dtype=q_dtype, generator=g)
    k_tokens = torch.randn(num_tokens, HEAD_DIM, dtype=torch.bfloat16, generator=g)
    token_indices = torch.randint(0, num_tokens, (num_queries, top_k), dtype=torch.int32, generator=g)
    topk_lengths = torch.full((num_queries,), top_k, dtype=torch.int32)
    attn_sink = torch.randn(heads, dtype=torch.float32, generator=g)
    case = Dsv4Case(q=q, k_tokens=k_tokens, cache=None, token_indices=token_indices, topk_lengths=topk_lengths,
                    attn_sink=attn_sink, page_size=page_size)
    if compress_ratio:
        eps = extra_page_size if extra_page_size is not None else page_size // compress_ratio
        if eps <= 0:
            raise ValueError("page_size // compress_ratio must be positive")
        etop = extra_top_k or (512 if compress_ratio == 4 else 128)
        case.extra_tokens = torch.randn(extra_tokens, HEAD_DIM, dtype=torch.bfloat16, generator=g)
        case.extra_token_indices = torch.randint(0, extra_tokens, (num_queries, etop), dtype=torch.int32,
                                                 generator=g)
        case.extra_topk_lengths = torch.full((num_queries,), etop, dtype=torch.int32)
        case.extra_page_size = eps
    case.cache = pack_dsv4_cache(case.k_tokens.to(device), page_size=page_size)
    if compress_ratio:
        case.extra_cache = pack_dsv4_cache(case.extra_tokens.to(device), page_size=case.extra_page_size)
    for name in ("q", "k_tokens", "token_indices", "topk_lengths", "attn_sink", "extra_tokens",
                 "extra_token_indices", "extra_topk_lengths"):
        t = getattr(case, name)
        if t is not None:
            setattr(case, name, t.to(device))
    return case


def make_dsv4_window_case(*, compress_ratio: int, num_queries: int, heads: int, context: int = 65536,
                          page_size: int = 64, window: int = 128, extra_top_k: int = 64,
                          extra_page_size: int | None = None, q_dtype: torch.dtype = torch.bfloat16,
                          seed: int = 0, device: str | torch.device = "cpu") -> Dsv4Case:
    """A serving-shaped DSV4 decode workload (SWA windows over a paged pool, C4/C128 extra slots).

    ``context`` latent rows are stored in pages of ``page_size`` whose physical
    order is a seeded random permutation (the page table).  Query ``i`` attends
    the ``window`` most recent tokens ending at logical position
    ``context - 1 - i`` (SWA slots), plus -- for compress_ratio 4 / 128 --
    ``extra_top_k`` distinct compressed entries drawn at random from the
    ``context // compress_ratio`` entries its position can see, stored in their
    own permuted pages of ``extra_page_size`` (default ``page_size //
    compress_ratio``, at least 1).  All lengths are full.  Draw order: q, SWA
    rows, SWA page permutation, sink, then extra rows, extra permutation and the
    per-query extra selections.
    """
    if context % page_size:
        raise ValueError("context must be a multiple of page_size")
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    q = torch.randn(num_queries, heads, HEAD_DIM, dtype=q_dtype, generator=g)
    rows = torch.randn(context, HEAD_DIM, dtype=torch.bfloat16, generator=g)
    pages = context // page_size
    perm = torch.randperm(pages, generator=g)
    sink = torch.randn(heads, dtype=torch.float32, generator=g)
    phys = torch.empty_like(rows)
    phys.view(pages, page_size, HEAD_DIM)[perm] = rows.view(pages, page_size, HEAD_DIM)
    end = context - 1 - torch.arange(num_queries)
    pos = end[:, None] - torch.arange(window - 1, -1, -1)[None, :]
    pos = pos.clamp_min(0)
    token_indices = (perm[pos // page_size] * page_size + pos % page_size).to(torch.int32)
    lengths = torch.full((num_queries,), window, dtype=torch.int32)
    case = Dsv4Case(q=q, k_tokens=phys, cache=None, token_indices=token_indices, topk_lengths=lengths,
                    attn_sink=sink, page_size=page_size)
    if compress_ratio:
        eps = extra_page_size if extra_page_size is not None else max(1, page_size // compress_ratio)
        n_extra = context // compress_ratio
        if n_extra % eps:
            raise ValueError("compressed entries must fill whole pages")
        erows = torch.randn(n_extra, HEAD_DIM, dtype=torch.bfloat16, generator=g)
        epages = n_extra // eps
        eperm = torch.randperm(epages, generator=g)
        ephys = torch.empty_like(erows)
        ephys.view(epages, eps, HEAD_DIM)[eperm] = erows.view(epages, eps, HEAD_DIM)
        sel = torch.empty((num_queries, extra_top_k), dtype=torch.int64)
        for i in range(num_queries):
            visible = max(extra_top_k, (int(end[i]) + 1) // compress_ratio)
            sel[i] = torch.randperm(visible, generator=g)[:extra_top_k]
        case.extra_tokens = ephys
        case.extra_token_indices = (eperm[sel // eps] * eps + sel % eps).to(torch.int32)
        case.extra_topk_lengths = torch.full((num_queries,), extra_top_k, dtype=torch.int32)
        case.extra_page_size = eps
    case.cache = pack_dsv4_cache(case.k_tokens.to(device), page_size=page_size)
    if compress_ratio:
        case.extra_cache = pack_dsv4_cache(case.extra_tokens.to(device), page_size=case.extra_page_size)
    for name in ("q", "k_tokens", "token_indices", "topk_lengths", "attn_sink", "extra_tokens",
                 "extra_token_indices", "extra_topk_lengths"):
        t = getattr(case, name)
        if t is not None:
            setattr(case, name, t.to(device))
    return case
