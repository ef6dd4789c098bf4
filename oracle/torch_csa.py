"""torch-csa restated with torch CPU ops -- TEST INFRASTRUCTURE ONLY.

The CPU baseline bench.py times beside the C restatement: the torch-csa decode
step of hybrid_attention/reference.py written here from the algorithm (not the
reference file, which never travels to the GPU box).
  * selection from cached fp32 chunk summaries: scores = q . summary / sqrt(D)
    in fp32, top-k ids best first (select_topk_chunks, reference.py:48-56, with
    chunk_mean's output given);
  * gather of the selected chunks' tokens (gather_chunk_tokens, :59-66);
  * fp32 scores over the gathered keys, fp32 softmax, probabilities rounded to
    the value dtype, PV in that dtype (full_decode_attention, :31-37).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  Its outputs are checked against the C oracle in
tests/test_oracle_csa.py.
"""
from __future__ import annotations

import math

import torch


def select_topk(q: torch.Tensor, summary: torch.Tensor, top_k: int) -> torch.Tensor:
    """int32 [B, H, min(top_k, C)] chunk ids by q . summary / sqrt(D), best first."""
    B, H, C, D = summary.shape
    scores = torch.matmul(summary, q.float().unsqueeze(-1)).squeeze(-1) * (1.0 / math.sqrt(D))
    return scores.topk(min(top_k, C), dim=-1).indices.to(torch.int32)


def attend(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, chunk_ids: torch.Tensor,
           chunk_size: int) -> torch.Tensor:
    """Softmax attention of q over the tokens of the selected chunks, [B, H, D] in q's dtype."""
    B, H, S, D = k_cache.shape
    offs = torch.arange(chunk_size, dtype=torch.long)
    tok = (chunk_ids.long().unsqueeze(-1) * chunk_size + offs).reshape(B, H, -1)   # [B, H, k * chunk]
    idx = tok.unsqueeze(-1).expand(-1, -1, -1, D)
    keys = torch.gather(k_cache, 2, idx)
    vals = torch.gather(v_cache, 2, idx)
    scores = torch.matmul(keys.float(), q.float().unsqueeze(-1)).squeeze(-1) * (1.0 / math.sqrt(D))
    probs = torch.softmax(scores, dim=-1).to(v_cache.dtype)
    return torch.matmul(probs.unsqueeze(2), vals).squeeze(2).to(q.dtype)


def decode_step(q, k_cache, v_cache, summary, chunk_size: int, top_k: int) -> torch.Tensor:
    """One decode step: selection from cached summaries, then attention."""
    return attend(q, k_cache, v_cache, select_topk(q, summary, top_k), chunk_size)
