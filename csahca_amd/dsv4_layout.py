"""DSV4 paged FP8 latent-cache byte layout (the cache format the DSV4 decode reads).

Layout (hybrid_attention/dsv4_correctness.py:10-21, csrc/dsv4_attention.cu:13-19):
page ``p`` starts at byte ``p * bytes_per_page``.  It holds ``page_size`` token rows
of 576 bytes -- 448 OCP e4m3 "nope" values followed by 64 bf16 "rope" values --
then ``page_size`` scale rows of 8 bytes (7 UE8M0 exponents, one per 64 nope
values, and one pad byte), then zero padding up to
``bytes_per_page = ceil(page_size * 584 / 576) * 576``.  Token ``loc`` lives on
page ``loc // page_size`` at row ``loc % page_size``.  A nope value decodes as
``e4m3(byte) * 2**(scale_byte - 127)``; rope values are stored raw.

``pack_dsv4_cache`` is a vectorised torch restatement of the reference's
per-token packing loop (dsv4_correctness.py:24-59) that runs on CPU or GPU
tensors and produces the same bytes (the input builder of tests and bench;
the decode kernels read the format directly, and the checker's decoder of it
lives with the oracle).
"""
from __future__ import annotations

import torch

DIM_NOPE = 448
DIM_ROPE = 64
HEAD_DIM = DIM_NOPE + DIM_ROPE
TILE_SIZE = 64
NUM_SCALE_TILES = DIM_NOPE // TILE_SIZE
NOPE_ROPE_BYTES = DIM_NOPE + DIM_ROPE * 2
SCALE_BYTES_PER_TOKEN = NUM_SCALE_TILES + 1
FP8_MAX = 448.0


def bytes_per_page(page_size: int) -> int:
    """dsv4_correctness.py:19-21."""
    raw = page_size * (NOPE_ROPE_BYTES + SCALE_BYTES_PER_TOKEN)
    return ((raw + NOPE_ROPE_BYTES - 1) // NOPE_ROPE_BYTES) * NOPE_ROPE_BYTES


def _ceil_log2_exact(x: torch.Tensor) -> torch.Tensor:
    """ceil(log2(x)) for positive normal fp32 x, computed exactly from the bits.

    The reference evaluates ``math.ceil(math.log2(float(x)))`` in double
    (dsv4_correctness.py:49); for an fp32 input that is the binary exponent,
    plus one unless x is an exact power of two.
    """
    mant, exp = torch.frexp(x)  # x = mant * 2**exp, mant in [0.5, 1)
    return torch.where(mant == 0.5, exp - 1, exp).to(torch.int32)


def pack_dsv4_cache(k_tokens: torch.Tensor, *, page_size: int) -> torch.Tensor:
    """Pack ``[tokens, 512]`` bf16 latent rows into the paged byte layout.

    Per 64-value nope tile: ``scale = 2**ceil(log2(max(max_abs, 1e-8) / 448))``,
    exponent byte ``clamp(log2(scale) + 127, 0, 255)``, values divided by the
    scale, clamped to +-448 and cast to e4m3 (dsv4_correctness.py:44-54).
    """
    if k_tokens.dtype != torch.bfloat16:
        raise ValueError("k_tokens must be bfloat16")
    if k_tokens.dim() != 2 or k_tokens.shape[1] != HEAD_DIM:
        raise ValueError(f"k_tokens must be [tokens, {HEAD_DIM}]")
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    device = k_tokens.device
    tokens = k_tokens.shape[0]
    pages = (tokens + page_size - 1) // page_size
    bpp = bytes_per_page(page_size)
    cache = torch.zeros((pages, bpp), dtype=torch.uint8, device=device)
    if tokens == 0:
        return cache

    nope = k_tokens[:, :DIM_NOPE].float().reshape(tokens, NUM_SCALE_TILES, TILE_SIZE)
    max_abs = nope.abs().amax(dim=-1).clamp_min(1e-8)
    exponent = _ceil_log2_exact(max_abs / FP8_MAX)
    scale = torch.ldexp(torch.ones_like(max_abs), exponent)
    quant = (nope / scale[..., None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    scale_u8 = (exponent + 127).clamp(0, 255).to(torch.uint8)

    padded = pages * page_size
    rows = torch.zeros((padded, NOPE_ROPE_BYTES), dtype=torch.uint8, device=device)
    rows[:tokens, :DIM_NOPE] = quant.reshape(tokens, DIM_NOPE).view(torch.uint8)
    rows[:tokens, DIM_NOPE:] = k_tokens[:, DIM_NOPE:].contiguous().view(torch.uint8)
    srows = torch.zeros((padded, SCALE_BYTES_PER_TOKEN), dtype=torch.uint8, device=device)
    srows[:tokens, :NUM_SCALE_TILES] = scale_u8

    data_end = page_size * NOPE_ROPE_BYTES
    cache[:, :data_end] = rows.reshape(pages, data_end)
    cache[:, data_end:data_end + page_size * SCALE_BYTES_PER_TOKEN] = srows.reshape(pages, -1)
    return cache
