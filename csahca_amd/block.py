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

* ``HybridDecodeBlock`` -- a hybrid decode block: RMSNorm -> QKV
  projection -> the new token's K/V appended to a growing cache -> the chunk
  summary of a chunk that just completed -> CSA over the complete chunks (fused
  step) -> out projection -> residual -> RMSNorm -> SiLU MLP -> residual.
  Where the shapes allow (bf16/f16, batch <= 4, 16-byte aligned rows) its
  products run as the library's decode-step GEMV kernels with the norms, the
  cache append, the activation and the residuals fused in, and the chunk
  summary built inside the CSA step: four or five launches per step.
  Otherwise, or with ``fused=False``, the products are torch's.

The mini block likewise runs its products (q, out, GELU MLP and the
``hidden + 0.01 * out`` tail) as library kernels where the shapes allow.  The
attention path is always the HIP library, which raises if it is not built.
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
                 seed: int = 0, init_std: float | None = None, fused: bool | None = None):
        self.heads, self.head_dim = heads, head_dim
        self.hidden_dim = heads * head_dim
        self.fused = fused  # None: the library's products whenever a call's shapes allow
        g = torch.Generator().manual_seed(seed)
        kw = dict(std=init_std, generator=g, dtype=dtype, device=device)
        self.w_q = _linear_weight(self.hidden_dim, self.hidden_dim, **kw)
        self.w_out = _linear_weight(self.hidden_dim, self.hidden_dim, **kw)
        mlp_dim = int(self.hidden_dim * mlp_ratio)
        self.mlp_dim = mlp_dim
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

    def can_fuse(self, hidden: torch.Tensor) -> bool:
        """Whether the library's decode-step products take this call's shapes."""
        B = hidden.shape[0]
        widest = max(self.hidden_dim, self.mlp_dim)
        return (hidden.is_cuda and hidden.dtype in (torch.bfloat16, torch.float16) and self.w_q.dtype == hidden.dtype
                and 0 < B <= 4 and self.hidden_dim % 8 == 0 and self.mlp_dim % 8 == 0
                and widest <= (4096 if B == 1 else 2048))

    def forward(self, hidden, k_cache, v_cache, *, selection: str = "precomputed", selected_chunks=None,
                summary=None, chunk_size: int = 64, top_k: int = 8, tile_size: int = 8, out=None):
        """One decode step; the result goes to ``out`` when given (it may be
        ``hidden`` itself: the step's last kernel reads each hidden value
        before overwriting it)."""
        fuse = self.can_fuse(hidden) if self.fused is None else self.fused
        if fuse:
            if not self.can_fuse(hidden):
                raise ValueError("the fused block products need bf16/f16, batch <= 4 and feature sizes that are "
                                 "multiples of 8 (at most 4096, or 2048 for batch > 1)")
            return self._forward_fused(hidden, k_cache, v_cache, out, selection=selection,
                                       selected_chunks=selected_chunks, summary=summary, chunk_size=chunk_size,
                                       top_k=top_k, tile_size=tile_size)
        res = self._forward_torch(hidden, k_cache, v_cache, selection=selection, selected_chunks=selected_chunks,
                                  summary=summary, chunk_size=chunk_size, top_k=top_k, tile_size=tile_size)
        if out is None:
            return res
        out.copy_(res)
        return out

    def _forward_torch(self, hidden, k_cache, v_cache, *, selection, selected_chunks, summary, chunk_size, top_k,
                       tile_size):
        batch = hidden.shape[0]
        q = F.linear(hidden, self.w_q).view(batch, self.heads, self.head_dim)
        attn = self.attention(q, k_cache, v_cache, selection=selection, selected_chunks=selected_chunks,
                              summary=summary, chunk_size=chunk_size, top_k=top_k, tile_size=tile_size)
        out = F.linear(attn.reshape(batch, self.hidden_dim), self.w_out)
        if self.use_mlp:
            out = out + F.linear(F.gelu(F.linear(hidden, self.w_up)), self.w_down)
        return hidden + 0.01 * out

    def _forward_fused(self, hidden, k_cache, v_cache, out, **attn_kw):
        """The same block through the library's decode-step products: q
        projection, attention, out projection, and for the MLP the GELU up
        projection and the down projection whose epilogue adds the out
        projection and forms ``hidden + 0.01 * out``: four or two products,
        each one launch."""
        B = hidden.shape[0]
        if not hidden.is_contiguous() or hidden.data_ptr() % 16:
            hidden = hidden.contiguous().clone()
        q = native.block_linear(hidden, self.w_q).view(B, self.heads, self.head_dim)
        attn = self.attention(q, k_cache, v_cache, **attn_kw).reshape(B, self.hidden_dim)
        if self.use_mlp:
            o = native.block_linear(attn, self.w_out)
            u = native.block_linear(hidden, self.w_up, activation="gelu")
            return native.block_linear(u, self.w_down, residual=o, base=hidden, alpha=0.01, out=out)
        return native.block_linear(attn, self.w_out, base=hidden, alpha=0.01, out=out)

    __call__ = forward


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


class HybridDecodeBlock:
    """Hybrid decode block: RMSNorm -> QKV -> CSA over a growing cache -> out
    projection -> SiLU MLP, weights N(0, 0.02^2).

    The cache is preallocated with ``capacity`` token slots and the chunk
    summaries with ``capacity // chunk_size`` rows; ``prefill`` fills the first
    ``S`` tokens and builds the summaries of their complete chunks.  Each
    ``step`` appends one token's K/V at the next position, builds the summary of
    the chunk that token completes (if any), and selects the top-k among the
    complete chunks only (the open chunk has no summary yet).

    The position and the chunk count live in device memory and every tensor
    keeps its shape, so a step has no host synchronisation: ``capture`` records
    one step as a HIP graph whose replays advance the cache token by token.
    ``length`` mirrors the position on the host (for the capacity check)."""

    def __init__(self, *, batch: int, heads: int, head_dim: int, capacity: int, chunk_size: int = 64,
                 top_k: int = 8, mlp_ratio: float = 2.0, dtype=torch.bfloat16, device="cuda", seed: int = 0,
                 init_std: float = 0.02, fused: bool | None = None):
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
        self.summary_buf = torch.zeros(batch, heads, capacity // chunk_size, head_dim, dtype=torch.float32,
                                       device=device)
        self.pos = torch.zeros(1, dtype=torch.int64, device=device)       # next token position
        self.nchunks = torch.zeros(1, dtype=torch.int32, device=device)   # complete chunks
        self.attn = torch.empty(batch, heads, head_dim, dtype=dtype, device=device)
        self.indices = torch.empty(batch, heads, min(top_k, capacity // chunk_size), dtype=torch.int32,
                                   device=device)
        self.q = torch.empty(batch, heads, head_dim, dtype=dtype, device=device)
        self.length = 0
        widest = max(self.hidden_dim, mlp_dim)
        can_fuse = (dtype in (torch.bfloat16, torch.float16) and 0 < batch <= 4 and self.hidden_dim % 8 == 0
                    and mlp_dim % 8 == 0 and widest <= (4096 if batch == 1 else 2048))
        if fused and not can_fuse:
            raise ValueError("the fused decode step needs bf16/f16, batch <= 4 and feature sizes "
                             "that are multiples of 8 (at most 4096, or 2048 for batch > 1)")
        self.fused = can_fuse if fused is None else bool(fused)

    @property
    def summary(self) -> torch.Tensor:
        """Summaries of the complete chunks (a view of the preallocated rows)."""
        return self.summary_buf[:, :, : self.length // self.chunk_size]

    def prefill(self, k: torch.Tensor, v: torch.Tensor) -> None:
        S = k.shape[2]
        if S > self.capacity:
            raise ValueError("prefill longer than the cache capacity")
        self.k_cache[:, :, :S].copy_(k)
        self.v_cache[:, :, :S].copy_(v)
        self.length = S
        C = S // self.chunk_size
        if C:
            native.csa_chunk_summary(self.k_cache, self.chunk_size, out=self.summary_buf, chunk_begin=0,
                                     num_chunks=C)
        self.pos.fill_(S)
        self.nchunks.fill_(C)

    def _step(self, hidden: torch.Tensor, out=None) -> torch.Tensor:
        return self._step_fused(hidden, out) if self.fused else self._step_torch(hidden, out)

    def _step_fused(self, hidden: torch.Tensor, out=None) -> torch.Tensor:
        """The step as library kernels: RMSNorm + QKV + cache append (and the
        complete-chunk count), the CSA step (which first builds the summary of a
        chunk the token completes), out projection + residual, then RMSNorm + up
        projection + SiLU and down projection + residual; the last one advances
        the position."""
        B, D = self.batch, self.hidden_dim
        if not hidden.is_contiguous() or hidden.data_ptr() % 16:
            hidden = hidden.contiguous().clone()
        native.block_qkv(hidden, self.w_qkv, self.q, self.k_cache, self.v_cache, self.pos, norm_weight=self.norm1,
                         num_chunks=self.nchunks, chunk_size=self.chunk_size)
        native.csa_decode_step_at(self.q, self.k_cache, self.v_cache, self.summary_buf, self.pos, self.chunk_size,
                                  self.top_k, out=self.attn, indices=self.indices)
        if not self.use_mlp:
            return native.block_linear(self.attn.view(B, D), self.w_out, residual=hidden, advance_pos=self.pos,
                                       out=out)
        h = native.block_linear(self.attn.view(B, D), self.w_out, residual=hidden)
        u = native.block_linear(h, self.w_up, norm_weight=self.norm2, activation="silu")
        return native.block_linear(u, self.w_down, residual=h, advance_pos=self.pos, out=out)

    def _step_torch(self, hidden: torch.Tensor, out=None) -> torch.Tensor:
        B, H, D = self.batch, self.heads, self.head_dim
        x = rms_norm(hidden, self.norm1)
        qkv = F.linear(x, self.w_qkv).view(B, 3, H, D)
        q = qkv[:, 0].contiguous()
        self.k_cache.index_copy_(2, self.pos, qkv[:, 1].unsqueeze(2))
        self.v_cache.index_copy_(2, self.pos, qkv[:, 2].unsqueeze(2))
        native.csa_chunk_summary_at(self.k_cache, self.summary_buf, self.chunk_size, self.pos)
        self.pos.add_(1)
        self.nchunks.copy_(torch.div(self.pos, self.chunk_size, rounding_mode="floor"))
        native.csa_decode_step_dev(q, self.k_cache, self.v_cache, self.summary_buf, self.nchunks, self.chunk_size,
                                   self.top_k, out=self.attn, indices=self.indices)
        h = hidden + F.linear(self.attn.reshape(B, self.hidden_dim), self.w_out)
        if self.use_mlp:
            h = h + F.linear(F.silu(F.linear(rms_norm(h, self.norm2), self.w_up)), self.w_down)
        if out is None:
            return h
        out.copy_(h)
        return out

    def _advance(self) -> None:
        if self.length >= self.capacity:
            raise RuntimeError("cache capacity exhausted")
        if (self.length + 1) // self.chunk_size == 0:
            raise RuntimeError("no complete chunk to attend to")
        self.length += 1

    def step(self, hidden: torch.Tensor, out=None) -> torch.Tensor:
        """One decode step; the result goes to ``out`` when given (it may be
        ``hidden`` itself, which the fused step's last kernel reads before
        overwriting)."""
        self._advance()
        return self._step(hidden, out)

    __call__ = step

    def capture(self, hidden: torch.Tensor, steps: int = 1, feedback: bool = False):
        """Record ``steps`` consecutive steps on the static input ``hidden`` as
        one HIP graph.

        Returns ``(replay, out)``: each ``replay()`` runs the steps (each
        appending one token) and leaves the last result in ``out``.  With
        ``feedback`` every step writes its result into ``hidden``, which the
        next step (and the next replay) consumes, as a decode loop feeds its
        hidden state back; ``out`` is then ``hidden``.  Without it every step
        reads the same ``hidden``.  A warm-up step on the capture stream creates
        that stream's library state first; its position advance is undone, and
        the K/V slot it wrote is overwritten by the next step."""
        steps = int(steps)
        if steps < 1:
            raise ValueError("steps must be positive")
        s = torch.cuda.Stream(device=hidden.device)
        s.wait_stream(torch.cuda.current_stream(hidden.device))
        with torch.cuda.stream(s):
            self._step(hidden)
            self.pos.sub_(1)
            self.nchunks.copy_(torch.div(self.pos, self.chunk_size, rounding_mode="floor"))
        torch.cuda.current_stream(hidden.device).wait_stream(s)
        torch.cuda.synchronize(hidden.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for _ in range(steps):
                out = self._step(hidden, hidden if feedback else None)

        def replay():
            for _ in range(steps):
                self._advance()
            graph.replay()
            return out

        replay.graph = graph
        return replay, out
