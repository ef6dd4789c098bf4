"""Write golden input/output vectors from the reference's own Python functions.

Run once, in the build container where the reference checkout exists:

    python tests/golden/make_golden.py --reference /root/reference

It imports ``hybrid_attention.reference``, ``hybrid_attention.dsv4_correctness``
and ``hybrid_attention.model_inference`` from the reference checkout (CPU only; the CUDA extension is never loaded) and
saves small ``.npz`` fixtures next to this script.  The fixtures are data only:
inputs, the reference's outputs, and SHA-256 digests of inputs regenerated from
a seed.  Nothing under tests/ imports the reference at test time.

What each fixture pins (functions no closed form fixes bit for bit):
  csa_small.npz      chunk_mean, select_topk_chunks, csa_reference (probability
                     cast to bf16), full_decode_attention, hca_reference and
                     hybrid_reference on B1 H2 S512 D64, chunk 64, k 4.
  csa_default.npz    the reference correctness CLI's default case (B1 H2 S1024
                     D128, chunk 64, k 4; hybrid_attention/correctness.py:13-25)
                     with inputs regenerated from seed 0 on the CPU generator.
  csa_ties.npz       torch.topk order on exactly tied chunk scores (recorded,
                     not relied on: the build declares its own tie-break).
  synthetic_hash.json  SHA-256 of make_synthetic_case(device="cpu") inputs at the
                     headline shape and of the DSV4 CLI's draw sequence.
  dsv4_c{0,4,128}.npz  pack_dsv4_cache bytes, dequant and reference_attention
                     for the three compress ratios (nq 3, H 8, page 64).
  dsv4_pack_edges.npz  pack bytes at power-of-two scale boundaries, tiny tiles,
                     values needing the +-448 clamp and a rope passthrough.
  block_mini.npz     MiniCSADecodeBlock.forward (hybrid_attention/model_inference.py:14-76)
                     with the torch-csa backend and the block's own top-k
                     selection, MLP ratio 0.0 and 2.0, B2 H2 D64 S512, chunk 64,
                     k 4: its weights, inputs, selected chunks and output
                     (odd hidden features zero, so the output there is the
                     block's update alone).

``--only NAME`` (repeatable: csa, hashes, dsv4, block) rewrites just those fixtures.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def csa_fixtures(R) -> None:
    case = R.make_synthetic_case(batch=1, heads=2, seq_len=512, head_dim=64, chunk_size=64, top_k=4,
                                 dtype=torch.bfloat16, device="cpu", seed=0)
    q, k, v = case.q, case.k_cache, case.v_cache
    sel = R.select_topk_chunks(q, k, 64, 4)
    np.savez_compressed(
        HERE / "csa_small.npz",
        q=bits16(q), k=bits16(k), v=bits16(v), chunk_size=64, top_k=4,
        chunk_mean=R.chunk_mean(k, 64).numpy(),
        selected=sel.numpy(),
        csa_out=bits16(R.csa_reference(q, k, v, chunk_size=64, top_k=4, selected_chunks=sel)),
        full_out=bits16(R.full_decode_attention(q, k, v)),
        hca_chunk=128,
        hca_out=bits16(R.hca_reference(q, k, v, chunk_size=128)),
        hybrid_out=bits16(R.hybrid_reference(q, k, v, csa_chunk_size=64, csa_top_k=4, hca_chunk_size=128)),
    )

    case = R.make_synthetic_case(batch=1, heads=2, seq_len=1024, head_dim=128, chunk_size=64, top_k=4,
                                 dtype=torch.bfloat16, device="cpu", seed=0)
    q, k, v = case.q, case.k_cache, case.v_cache
    sel = R.select_topk_chunks(q, k, 64, 4)
    np.savez_compressed(
        HERE / "csa_default.npz",
        seed=0, shape=np.array([1, 2, 1024, 128]), chunk_size=64, top_k=4,
        sha_q=sha(q), sha_k=sha(k), sha_v=sha(v),
        chunk_mean=R.chunk_mean(k, 64).numpy(),
        selected=sel.numpy(),
        csa_out=bits16(R.csa_reference(q, k, v, chunk_size=64, top_k=4, selected_chunks=sel)),
    )

    # Exact ties: constant keys make every chunk score equal.
    qt = torch.ones(1, 1, 64, dtype=torch.bfloat16)
    kt = torch.ones(1, 1, 64 * 16, 64, dtype=torch.bfloat16)
    np.savez_compressed(HERE / "csa_ties.npz", torch_topk_order=R.select_topk_chunks(qt, kt, 64, 5).numpy(),
                        torch_version=torch.__version__)


def synthetic_hashes(R, DC) -> None:
    case = R.make_synthetic_case(batch=1, heads=8, seq_len=32768, head_dim=128, chunk_size=64, top_k=8,
                                 dtype=torch.bfloat16, device="cpu", seed=0)
    meta = {
        "torch_version": torch.__version__,
        "csa_headline": {"shape": [1, 8, 32768, 128], "seed": 0, "sha_q": sha(case.q),
                         "sha_k": sha(case.k_cache), "sha_v": sha(case.v_cache)},
    }
    # DSV4 CLI draw sequence (dsv4_correctness.py:168-227) at the fixture sizes.
    for ratio in (0, 4, 128):
        d = dsv4_draw(ratio, nq=3, heads=8, tokens=128, top_k=32, page=64, extra_tokens=128, extra_top_k=32,
                      seed=0, DC=DC, pack=False)
        meta[f"dsv4_c{ratio}"] = {k: sha(v) for k, v in d.items() if isinstance(v, torch.Tensor)}
    (HERE / "synthetic_hash.json").write_text(json.dumps(meta, indent=1, sort_keys=True) + "\n")


def dsv4_draw(ratio, *, nq, heads, tokens, top_k, page, extra_tokens, extra_top_k, seed, DC, pack=True):
    """The draw order of dsv4_correctness.main (dsv4_correctness.py:168-227), on CPU."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    out = {}
    out["q"] = torch.randn(nq, heads, DC.HEAD_DIM, dtype=torch.bfloat16, generator=g)
    out["k_tokens"] = torch.randn(tokens, DC.HEAD_DIM, dtype=torch.bfloat16, generator=g)
    out["token_indices"] = torch.randint(0, tokens, (nq, top_k), dtype=torch.int32, generator=g)
    out["topk_lengths"] = torch.randint(max(1, top_k // 2), top_k + 1, (nq,), dtype=torch.int32, generator=g)
    out["attn_sink"] = torch.randn(heads, dtype=torch.float32, generator=g)
    if ratio:
        extra_page = page // ratio if page // ratio > 0 else 1
        out["extra_tokens"] = torch.randn(extra_tokens, DC.HEAD_DIM, dtype=torch.bfloat16, generator=g)
        ei = torch.randint(0, extra_tokens, (nq, extra_top_k), dtype=torch.int32, generator=g)
        if extra_top_k >= 4:
            ei[:, -2:] = -1
        out["extra_token_indices"] = ei
        out["extra_topk_lengths"] = torch.randint(max(1, extra_top_k // 2), extra_top_k + 1, (nq,),
                                                  dtype=torch.int32, generator=g)
        out["extra_page_size"] = extra_page
    if pack:
        out["cache"] = DC.pack_dsv4_cache(out["k_tokens"], page_size=page)
        if ratio:
            out["extra_cache"] = DC.pack_dsv4_cache(out["extra_tokens"], page_size=out["extra_page_size"])
    return out


def dsv4_fixtures(DC) -> None:
    page = 64
    for ratio in (0, 4, 128):
        d = dsv4_draw(ratio, nq=3, heads=8, tokens=128, top_k=32, page=page, extra_tokens=128, extra_top_k=32,
                      seed=0, DC=DC)
        scale = 1.0 / math.sqrt(DC.HEAD_DIM)
        kw = {}
        if ratio:
            kw = dict(extra_cache=d["extra_cache"], extra_token_indices=d["extra_token_indices"],
                      extra_topk_lengths=d["extra_topk_lengths"], extra_page_size=d["extra_page_size"])
        out = DC.reference_attention(d["q"], d["cache"], d["token_indices"], d["topk_lengths"], d["attn_sink"],
                                     page_size=page, softmax_scale=scale, **kw)
        out_nosink = DC.reference_attention(d["q"], d["cache"], d["token_indices"], d["topk_lengths"], None,
                                            page_size=page, softmax_scale=scale, **kw)
        deq = DC.dequant_dsv4_cache(d["cache"], d["token_indices"][:1], page_size=page)
        payload = dict(
            ratio=ratio, page_size=page, softmax_scale=scale,
            q=bits16(d["q"]), k_tokens=bits16(d["k_tokens"]), cache=d["cache"].numpy(),
            token_indices=d["token_indices"].numpy(), topk_lengths=d["topk_lengths"].numpy(),
            attn_sink=d["attn_sink"].numpy(), dequant_q0=bits16(deq),
            out=bits16(out), out_nosink=bits16(out_nosink),
        )
        if ratio:
            payload.update(extra_tokens=bits16(d["extra_tokens"]), extra_cache=d["extra_cache"].numpy(),
                           extra_token_indices=d["extra_token_indices"].numpy(),
                           extra_topk_lengths=d["extra_topk_lengths"].numpy(), extra_page_size=d["extra_page_size"])
        np.savez_compressed(HERE / f"dsv4_c{ratio}.npz", **payload)

    # Pack edge cases: one token per row pattern, page_size 4.
    rows = []
    base = torch.zeros(DC.HEAD_DIM, dtype=torch.float32)
    r = base.clone(); r[:64] = 448.0; r[64:128] = 224.0; r[128:192] = 896.0; r[192] = 1.0; rows.append(r)
    r = base.clone(); r[0] = 1e-9; r[64] = 3.0e-8; r[128] = -5.0; r[192:256] = torch.linspace(-2, 2, 64); rows.append(r)
    r = base.clone(); r[:448] = torch.linspace(-1000, 1000, 448); r[448:] = torch.linspace(-3, 3, 64); rows.append(r)
    r = base.clone(); r[:448] = 2.0 ** torch.arange(-20, 428).float().clamp(max=20) / 7.0; rows.append(r)
    r = base.clone(); r[:448:7] = 0.0137; r[1:448:5] = -448.0 * 2 ** -10; rows.append(r)
    k_tokens = torch.stack(rows).to(torch.bfloat16)
    np.savez_compressed(HERE / "dsv4_pack_edges.npz", k_tokens=bits16(k_tokens), page_size=4,
                        cache=DC.pack_dsv4_cache(k_tokens, page_size=4).numpy(),
                        bpp={ps: DC.bytes_per_page(ps) for ps in (1, 2, 4, 16, 64, 256)}.__repr__())


def block_fixtures(MI, R) -> None:
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(8)
    hidden = torch.randn(2, 128, generator=g).to(bf)
    # Odd features are zero: there the output is 0.01 * (attention + MLP) alone,
    # so the block's composition shows above the residual's bf16 rounding.
    hidden[:, 1::2] = 0
    k = torch.randn(2, 2, 512, 64, generator=g).to(bf)
    v = torch.randn(2, 2, 512, 64, generator=g).to(bf)
    fx = dict(hidden=bits16(hidden), k=bits16(k), v=bits16(v), heads=2, head_dim=64, chunk_size=64, top_k=4)
    for ratio in (0.0, 2.0):
        tag = f"mlp{int(ratio)}"
        torch.manual_seed(7)  # default nn.Linear init, as the reference benchmark seeds it
        blk = MI.MiniCSADecodeBlock(heads=2, head_dim=64, dtype=bf, device=torch.device("cpu"), mlp_ratio=ratio)
        with torch.no_grad():
            out = blk(hidden, k, v, None, backend="torch-csa", chunk_size=64, top_k=4, tile_size=8)
            sel = R.select_topk_chunks(blk.q_proj(hidden).view(2, 2, 64), k, 64, 4)
        fx[f"{tag}_w_q"] = bits16(blk.q_proj.weight)
        fx[f"{tag}_w_out"] = bits16(blk.out_proj.weight)
        if blk.use_mlp:
            fx[f"{tag}_w_up"] = bits16(blk.up_proj.weight)
            fx[f"{tag}_w_down"] = bits16(blk.down_proj.weight)
        fx[f"{tag}_selected"] = sel.numpy()
        fx[f"{tag}_out"] = bits16(out)
    np.savez_compressed(HERE / "block_mini.npz", **fx)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", action="append", choices=["csa", "hashes", "dsv4", "block"])
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    from hybrid_attention import dsv4_correctness as DC  # noqa: E402
    from hybrid_attention import model_inference as MI  # noqa: E402
    from hybrid_attention import reference as R  # noqa: E402

    torch.set_num_threads(4)
    todo = set(args.only or ["csa", "hashes", "dsv4", "block"])
    if "csa" in todo:
        csa_fixtures(R)
    if "hashes" in todo:
        synthetic_hashes(R, DC)
    if "dsv4" in todo:
        dsv4_fixtures(DC)
    if "block" in todo:
        block_fixtures(MI, R)
    for p in sorted(HERE.glob("*.npz")) + [HERE / "synthetic_hash.json"]:
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
