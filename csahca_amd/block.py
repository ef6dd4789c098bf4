"""Decode blocks that route their attention through the gfx950 CSA kernels.

Two blocks:

* ``MiniCSADecodeBlock`` -- the reference's benchmark block
  (hybrid_attention/model_inference.py:14-76): q = q_proj(hidden); CSA
  attention of q over a static [B,H,S,D] cache; out_proj; optional GELU MLP on
  the block input; ``hidden + 0.01 * out``.  Selection modes:

  - ``precomputed``: chunk ids handed in (model_inference.py:140-162 with
    ``--selection precomputed``), attention by ``csa_decode_forward_tiled``;
  - ``dynamic``: top-k recomputed every step (model_inference.py:52-53) by the
    fused ``csa_decode_step`` from chunk summaries.  The cache is static, so the
    summaries are built once (``summary_cache=True``) or, to mirror the
    reference's per-step ``chunk_mean`` exactly, rebuilt every step
    (``summary_cache=False``).

* ``HybridDecodeBlock`` -- the BASELINE config-3 block: RMSNorm -> QKV
  projection -> the new token's K/V appended to a growing cache -> the chunk
  summary of a chunk that just completed -> CSA over the complete chunks (fused
  step) -> out projection -> residual -> RMSNorm -> SiLU MLP -> residual.

Matrix products use torch (the vendor BLAS); the attention path is the HIP
library, which raises if it is not built.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import native


def _linear_weight(out_f: int, in_f: int, *, std: float | None, generator, dtype, device) -> torch.Tensor:
    """nn.Linear's default init (uniform +-1/sqrt(in)) or N(0, std^2)."""
    if std is None:
        bound = 1.0 / math.sqrt(in_f)
        w = torch.empty(out_f, in_f).uniform_(-bound, bound, generator=generator)
    else:
        w = torch.empty(out_f, in_f).normal_(0.0, std, generator=generator)
    return w.to(dtype=dtype, device=device)


class MiniCSADecodeBlock:
    """The reference benchmark block (hybrid_attention/model_inference.py:14-76)."""

    def __init__(self, *, heads: int, head_dim: int, dtype: torch.dtype, device, mlp_ratio: float,
                 seed: int = 0, init_std: float | None = None):
        self.heads, self.head_dim = heads, head_dim
        self.hidden_dim = heads * head_dim
        g = torch.Generator().manual_seed(seed)
        kw = dict(std=init_std, generator=g, dtype=dtype, device=device)
        self.w_q = _linear_weight(self.hidden_dim, self.hidden_dim, **kw)
        self.w_out = _linear_weight(self.hidden_dim, self.hidden_dim, **kw)
        mlp_dim = int(self.hidden_dim * mlp_ratio)
        self.use_mlp = mlp_dim > 0
        if self.use_mlp:
            self.w_up = _linear_weight(mlp_dim, self.hidden_dim, **kw)
            self.w_down = _linear_weight(self.hidden_dim, mlp_dim, **kw)

    def attention(self, q, k_cache, v_cache, *, selection: str, selected_chunks=None, summary=None,
                  chunk_size: int, top_k: int, tile_size: int = 8):
        if selection == "precomputed":
            return native.csa_decode_forward_tiled(q, k_cache, v_cache, selected_chunks, chunk_size, tile_size)
        if selection == "dynamic":
            if summary is None:  # the reference's per-step chunk_mean
                summary = native.csa_chunk_summary(k_cache, chunk_size)
            out, _idx = native.csa_decode_step(q, k_cache, v_cache, summary, chunk_size, top_k)
            return out
        raise ValueError(f"unknown selection: {selection}")

    def forward(self, hidden, k_cache, v_cache, *, selection: str = "precomputed", selected_chunks=None,
                summary=None, chunk_size: int = 64, top_k: int = 8, tile_size: int = 8):
        batch = hidden.shape[0]
        q = F.linear(hidden, self.w_q).view(batch, self.heads, self.head_dim)
        attn = self.attention(q, k_cache, v_cache, selection=selection, selected_chunks=selected_chunks,
                              summary=summary, chunk_size=chunk_size, top_k=top_k, tile_size=tile_size)
        out = F.linear(attn.reshape(batch, self.hidden_dim), self.w_out)
        if self.use_mlp:
            out = out + F.linear(F.gelu(F.linear(hidden, self.w_up)), self.w_down)
        return hidden + 0.01 * out

    __call__ = forward


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


class HybridDecodeBlock:
    """RMSNorm -> QKV -> CSA over a growing cache -> out
    projection -> SiLU MLP, weights N(0, 0.02^2).

    The cache is preallocated with ``capacity`` token slots; ``prefill`` fills
    the first ``S`` and builds the summaries of its complete chunks.  Each
    ``step`` appends one token's K/V at position ``length``, extends the
    summaries when that token completes a chunk, and selects the top-k among
    the complete chunks only (the open chunk has no summary yet)."""

    def __init__(self, *, batch: int, heads: int, head_dim: int, capacity: int, chunk_size: int = 64,
                 top_k: int = 8, mlp_ratio: float = 2.0, dtype=torch.bfloat16, device="cuda", seed: int = 0,
                 init_std: float = 0.02):
        self.batch, self.heads, self.head_dim = batch, heads, head_dim
        self.hidden_dim = heads * head_dim
        self.chunk_size, self.top_k = chunk_size, top_k
        self.capacity = capacity
        g = torch.Generator().manual_seed(seed)
        kw = dict(std=init_std, generator=g, dtype=dtype, device=device)
        self.w_qkv = _linear_weight(3 * self.hidden_dim, self.hidden_dim, **kw)
        self.w_out = _linear_weight(self.hidden_dim, self.hidden_dim, **kw)
        mlp_dim = int(self.hidden_dim * mlp_ratio)
        self.use_mlp = mlp_dim > 0
        if self.use_mlp:
            self.w_up = _linear_weight(mlp_dim, self.hidden_dim, **kw)
            self.w_down = _linear_weight(self.hidden_dim, mlp_dim, **kw)
        self.norm1 = torch.ones(self.hidden_dim, dtype=dtype, device=device)
        self.norm2 = torch.ones(self.hidden_dim, dtype=dtype, device=device)
        self.k_cache = torch.zeros(batch, heads, capacity, head_dim, dtype=dtype, device=device)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.length = 0
        self.summary = torch.empty(batch, heads, 0, head_dim, dtype=torch.float32, device=device)

    def prefill(self, k: torch.Tensor, v: torch.Tensor) -> None:
        S = k.shape[2]
        if S > self.capacity:
            raise ValueError("prefill longer than the cache capacity")
        self.k_cache[:, :, :S].copy_(k)
        self.v_cache[:, :, :S].copy_(v)
        self.length = S
        C = S // self.chunk_size
        self.summary = torch.empty(self.batch, self.heads, C, self.head_dim, dtype=torch.float32,
                                   device=self.k_cache.device)
        if C:
            native.csa_chunk_summary(self.k_cache, self.chunk_size, out=self.summary, chunk_begin=0, num_chunks=C)

    def _extend_summary(self) -> None:
        C = self.length // self.chunk_size
        if C == self.summary.shape[2]:
            return
        grown = torch.empty(self.batch, self.heads, C, self.head_dim, dtype=torch.float32, device=self.summary.device)
        grown[:, :, : self.summary.shape[2]].copy_(self.summary)
        native.csa_chunk_summary(self.k_cache, self.chunk_size, out=grown, chunk_begin=C - 1, num_chunks=1)
        self.summary = grown

    def step(self, hidden: torch.Tensor) -> torch.Tensor:
        if self.length >= self.capacity:
            raise RuntimeError("cache capacity exhausted")
        B, H, D = self.batch, self.heads, self.head_dim
        x = rms_norm(hidden, self.norm1)
        qkv = F.linear(x, self.w_qkv).view(B, 3, H, D)
        q = qkv[:, 0].contiguous()
        self.k_cache[:, :, self.length].copy_(qkv[:, 1])
        self.v_cache[:, :, self.length].copy_(qkv[:, 2])
        self.length += 1
        self._extend_summary()
        if self.summary.shape[2] == 0:
            raise RuntimeError("no complete chunk to attend to")
        attn, _idx = native.csa_decode_step(q, self.k_cache, self.v_cache, self.summary, self.chunk_size, self.top_k)
        h = hidden + F.linear(attn.reshape(B, self.hidden_dim), self.w_out)
        if self.use_mlp:
            h = h + F.linear(F.silu(F.linear(rms_norm(h, self.norm2), self.w_up)), self.w_down)
        return h

    __call__ = step
