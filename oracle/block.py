"""Decode-block restatements on the CPU -- TEST INFRASTRUCTURE ONLY.

Two blocks, each written from its specification with torch CPU ops around the
C oracle's CSA.  Only tests/ imports this module, as the checker.

* :func:`mini_block` -- the reference benchmark block,
  hybrid_attention/model_inference.py:48-76: ``q = hidden W_q^T`` (bf16
  linear), top-k chunk selection from chunk means, CSA attention, ``out =
  attn W_out^T`` plus, when the block has an MLP, ``W_down gelu(W_up hidden)``
  on the block INPUT, then ``hidden + 0.01 * out``, every op in the weights'
  dtype.  Pinned bit for bit, on outputs and selected chunks, by
  tests/golden/block_mini.npz, which the reference block itself wrote
  (tests/test_oracle_block.py).
* :func:`baseline_block_steps` -- the BASELINE config-2 block (RMSNorm ->
  fused QKV -> append the token's K/V -> CSA over the complete chunks of the
  grown cache -> out projection + residual -> RMSNorm -> SiLU MLP + residual).
  The reference has no such block, so no fixture exists; the restatement is
  pinned by closed forms at special weights instead (zero QKV weights make the
  attention an exact mean of value rows; zero out-projection weights leave the
  MLP alone; tests/test_oracle_block.py).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import BF16, F32, chunk_mean, csa_attend, select_topk


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * weight in fp32, rounded to x's dtype."""
    xf = x.float()
    inv = 1.0 / torch.sqrt((xf * xf).mean(dim=-1, keepdim=True) + eps)
    return (xf * inv * weight.float()).to(x.dtype)


def _csa(q, k, v, selected, chunk, prob_dtype) -> torch.Tensor:
    out = csa_attend(q, k, v, selected, chunk, prob_dtype=prob_dtype)
    return torch.from_numpy(out).to(torch.float32).to(q.dtype)


def mini_block(hidden, w_q, w_out, k, v, *, chunk: int, top_k: int, w_up=None, w_down=None, selected=None,
               prob_dtype=BF16):
    """One step of the reference block (model_inference.py:48-76).

    ``prob_dtype`` BF16 is the torch-csa backend (probabilities rounded to the
    value dtype before PV); F32 is the cuda-csa op math.  ``selected`` None lets
    the block select its chunks (reference.py:48-56).  Returns (output,
    selected chunk ids int32 numpy)."""
    B = hidden.shape[0]
    _, H, _, D = k.shape
    q = F.linear(hidden, w_q).view(B, H, D)
    if selected is None:
        selected = select_topk(q, chunk_mean(k, chunk), top_k)[0]
    attn = _csa(q, k, v, selected, chunk, prob_dtype)
    out = F.linear(attn.reshape(B, H * D), w_out)
    if w_up is not None:
        out = out + F.linear(F.gelu(F.linear(hidden, w_up)), w_down)
    return hidden + 0.01 * out, np.asarray(selected)


def baseline_block_steps(w: dict, k0: torch.Tensor, v0: torch.Tensor, hiddens, *, heads: int, head_dim: int,
                         chunk: int, top_k: int, prob_dtype=F32):
    """Consecutive steps of the BASELINE block over a cache that grows by one
    token per step, from the prefilled ``k0``/``v0`` [B, H, S0, D].

    ``w`` holds ``w_qkv`` [3 H D, H D], ``w_out``, ``norm1``, ``norm2`` and,
    with an MLP, ``w_up`` / ``w_down``.  Values are rounded to the weights'
    dtype wherever the block stores them (q, the appended K/V, every linear
    output).  Selection scores the summaries of the complete chunks of the grown
    cache, the appended token included.  Returns the list of step outputs."""
    B = k0.shape[0]
    H, D = heads, head_dim
    k, v = k0.clone(), v0.clone()
    outs = []
    for hidden in hiddens:
        qkv = F.linear(rms_norm(hidden, w["norm1"]), w["w_qkv"]).view(B, 3, H, D)
        q = qkv[:, 0].contiguous()
        k = torch.cat([k, qkv[:, 1].unsqueeze(2)], dim=2)
        v = torch.cat([v, qkv[:, 2].unsqueeze(2)], dim=2)
        C = k.shape[2] // chunk
        ids, _ = select_topk(q, chunk_mean(k[:, :, : C * chunk].contiguous(), chunk), top_k)
        h = hidden + F.linear(_csa(q, k, v, ids, chunk, prob_dtype).reshape(B, H * D), w["w_out"])
        if "w_up" in w:
            h = h + F.linear(F.silu(F.linear(rms_norm(h, w["norm2"]), w["w_up"])), w["w_down"])
        outs.append(h)
    return outs
