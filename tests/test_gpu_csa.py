"""GPU parity of the CSA kernels against the CPU oracle (and golden vectors).

Tolerances (the parity bar of this path): outputs |got - ref| <= 2e-2 + 1e-2 |ref| for
16-bit storage (1e-4 + 1e-4 |ref| for fp32/fp64 storage); selected chunk ids
bit-exact under the declared tie-break (score desc, chunk id asc), where a
mismatch is accepted only between chunks whose oracle scores agree to 1e-5
(fp32 summation-order noise).
"""
import numpy as np
import pytest
import torch

import oracle
from csahca_amd import extension, native
from csahca_amd.synthetic import clustered_chunks, make_synthetic_case, plant_chunks, scattered_chunks

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    native.lib()


def tol_for(dtype):
    return (2e-2, 1e-2) if dtype in (torch.bfloat16, torch.float16) else (1e-4, 1e-4)


def assert_close(got: torch.Tensor, ref: np.ndarray, atol: float, rtol: float, what: str = ""):
    g = got.detach().float().cpu().numpy().astype(np.float64)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    diff = np.abs(g - ref)
    bad = diff > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{what} max_abs={diff.max():.3e} bad={int(bad.sum())}/{bad.size}"


def assert_indices(got: torch.Tensor, want: np.ndarray, scores: np.ndarray, eps: float = 1e-5):
    g = got.cpu().numpy()
    assert g.shape == want.shape
    if np.array_equal(g, want):
        return
    B, H, k = want.shape
    for b in range(B):
        for h in range(H):
            if np.array_equal(g[b, h], want[b, h]):
                continue
            assert len(set(g[b, h].tolist())) == k
            s = scores[b, h]
            for j in range(k):
                a, w = s[g[b, h, j]], s[want[b, h, j]]
                assert abs(a - w) <= eps * max(1.0, abs(w)), (b, h, j, g[b, h], want[b, h])


def run_tiled(case, idx, tile):
    return extension.csa_decode_forward_tiled(case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV),
                                              idx.to(DEV), case.chunk_size, tile)


# ---------------------------------------------------------------------------

def test_headline_decode_step():
    """B1 H8 S32768 D128 chunk64 k8 bf16: summaries, selection, attention."""
    case = make_synthetic_case(batch=1, heads=8, seq_len=32768, head_dim=128, chunk_size=64, top_k=8, seed=0)
    q, k, v = case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV)
    summ = extension.csa_chunk_summary(k, 64)
    summ_ref = oracle.chunk_mean(case.k_cache, 64)
    np.testing.assert_allclose(summ.cpu().numpy(), summ_ref, rtol=0, atol=2e-6)
    idx = extension.csa_select_topk(q, summ, 8)
    want, scores = oracle.select_topk(case.q, summ_ref, 8)
    assert_indices(idx, want, scores)
    ref32 = oracle.csa_attend(case.q, case.k_cache, case.v_cache, want, 64, prob_dtype=oracle.F32)
    ref_torch_csa = oracle.csa_reference(case.q, case.k_cache, case.v_cache, chunk_size=64, top_k=8,
                                         selected_chunks=want, dtype=torch.bfloat16)
    for tile in (8, 16, 64, native.csa_auto_tile_size(1, 8, 8, 64)):
        out = extension.csa_decode_forward_tiled(q, k, v, idx, 64, tile)
        assert_close(out, ref32, 2e-2, 1e-2, f"tile={tile}")
        assert_close(out, ref_torch_csa, 2e-2, 1e-2, f"vs torch-csa tile={tile}")
    out, idx2 = native.csa_decode_step(q, k, v, summ, 64, 8)
    assert torch.equal(idx2, idx)
    assert_close(out, ref32, 2e-2, 1e-2, "fused step")
    out1 = extension.csa_decode_forward(q, k, v, idx.long(), 64)
    assert_close(out1, ref32, 2e-2, 1e-2, "v1 op")


def test_golden_small_fixture(golden_dir):
    g = np.load(golden_dir / "csa_small.npz")
    to_t = lambda bits: torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    q, k, v = to_t(g["q"]), to_t(g["k"]), to_t(g["v"])
    summ = extension.csa_chunk_summary(k, 64)
    np.testing.assert_allclose(summ.cpu().numpy(), g["chunk_mean"], rtol=0, atol=2e-6)
    idx = extension.csa_select_topk(q, summ, 4)
    assert np.array_equal(idx.cpu().numpy(), g["selected"])
    out = extension.csa_decode_forward_tiled(q, k, v, idx, 64)
    want = oracle.bf16_bits_to_f32(g["csa_out"]).astype(np.float64)
    assert_close(out, want, 2e-2, 1e-2, "golden csa_out")


SWEEP = [
    # B, H, S, D, chunk, k, dtype
    (1, 8, 8192, 128, 64, 8, torch.bfloat16),
    (1, 8, 8192, 128, 64, 32, torch.bfloat16),
    (3, 2, 4096, 128, 64, 5, torch.bfloat16),
    (2, 3, 2048, 64, 64, 4, torch.bfloat16),
    (2, 2, 2048, 256, 32, 6, torch.bfloat16),
    (1, 2, 1024, 512, 64, 4, torch.bfloat16),
    (2, 2, 2048, 128, 64, 8, torch.float16),
    (2, 2, 2048, 128, 64, 8, torch.float32),
    (1, 2, 1024, 64, 64, 4, torch.float64),
    (1, 3, 1000, 96, 50, 4, torch.bfloat16),   # generic path: D not a vector width, chunk not a power of 2
    (1, 2, 512, 1024, 64, 2, torch.bfloat16),  # generic path, widest head
    (1, 2, 512, 32, 16, 7, torch.float32),
]


@pytest.mark.parametrize("B,H,S,D,chunk,k,dtype", SWEEP)
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_sweep_parity(B, H, S, D, chunk, k, dtype, index_dtype):
    g = torch.Generator().manual_seed(B * 1000 + S + D + k)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    kc = torch.randn(B, H, S, D, generator=g).to(dtype)
    vc = torch.randn(B, H, S, D, generator=g).to(dtype)
    C = S // chunk
    idx = torch.stack([torch.randperm(C, generator=g)[:k] for _ in range(B * H)]).view(B, H, k).to(index_dtype)
    ref = oracle.csa_attend(q, kc, vc, idx, chunk, prob_dtype=oracle.F32)
    atol, rtol = tol_for(dtype)
    qd, kd, vd, idd = q.to(DEV), kc.to(DEV), vc.to(DEV), idx.to(DEV)
    for tile in (1, 7, 8, 64, k * chunk):
        out = extension.csa_decode_forward_tiled(qd, kd, vd, idd, chunk, tile)
        assert out.dtype == dtype and out.shape == q.shape
        assert_close(out, ref, atol, rtol, f"tile={tile}")
    assert_close(extension.csa_decode_forward(qd, kd, vd, idd, chunk), ref, atol, rtol, "v1")
    # selection parity on the same inputs
    summ = extension.csa_chunk_summary(kd, chunk)
    summ_ref = oracle.chunk_mean(kc, chunk)
    np.testing.assert_allclose(summ.cpu().numpy(), summ_ref, rtol=1e-6, atol=2e-6)
    want, scores = oracle.select_topk(q, summ_ref, k)
    assert_indices(extension.csa_select_topk(qd, summ, k), want, scores)


def test_edge_indices():
    B, H, S, D, chunk = 1, 4, 1000, 128, 64  # last chunk (id 15) is partial: tokens 960..999
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, H, D, generator=g).bfloat16()
    kc = torch.randn(B, H, S, D, generator=g).bfloat16()
    vc = torch.randn(B, H, S, D, generator=g).bfloat16()
    idx = torch.tensor([[[3, -1, 15, 9],        # negative id skipped, partial chunk
                         [-1, -1, -1, -1],      # nothing valid -> zeros
                         [40, 15, -5, 15],      # id past the cache skipped, duplicate counted twice
                         [0, 1, 2, 3]]], dtype=torch.int32)
    ref = oracle.csa_attend(q, kc, vc, idx, chunk)
    for tile in (1, 8, 33, 256):
        out = extension.csa_decode_forward_tiled(q.to(DEV), kc.to(DEV), vc.to(DEV), idx.to(DEV), chunk, tile)
        assert_close(out, ref, 2e-2, 1e-2, f"tile={tile}")
        assert torch.all(out[0, 1] == 0)
    # top_k = 0 -> zeros
    out = extension.csa_decode_forward_tiled(q.to(DEV), kc.to(DEV), vc.to(DEV),
                                             torch.empty(B, H, 0, dtype=torch.int32, device=DEV), chunk, 8)
    assert torch.all(out == 0)


@pytest.mark.parametrize("kind", ["scattered", "clustered"])
@pytest.mark.parametrize("S,k", [(32768, 8), (131072, 32)])
def test_planted_selection_bit_exact(kind, S, k):
    B, H, D, chunk = 1, 8, 128, 64
    C = S // chunk
    case = make_synthetic_case(batch=B, heads=H, seq_len=S, head_dim=D, chunk_size=chunk, top_k=k, seed=2)
    ids = scattered_chunks(B, H, C, k) if kind == "scattered" else clustered_chunks(B, H, C, k)
    kp = plant_chunks(case.q, case.k_cache, ids, chunk, alpha=1.0).to(DEV)
    summ = extension.csa_chunk_summary(kp, chunk)
    idx = extension.csa_select_topk(case.q.to(DEV), summ, k)
    assert torch.equal(idx.cpu(), ids)


def test_tie_break_lowest_index_first():
    q = torch.ones(2, 3, 64, dtype=torch.bfloat16, device=DEV)
    k = torch.ones(2, 3, 64 * 40, 64, dtype=torch.bfloat16, device=DEV)
    summ = extension.csa_chunk_summary(k, 64)
    idx = extension.csa_select_topk(q, summ, 7)
    assert torch.equal(idx.cpu(), torch.arange(7, dtype=torch.int32).expand(2, 3, 7))
    # ties below distinct winners: chunk 30 best, then equal rest in index order
    k[:, :, 30 * 64:31 * 64] = 2.0
    idx = extension.csa_select_topk(q, extension.csa_chunk_summary(k, 64), 4)
    assert torch.equal(idx.cpu(), torch.tensor([30, 0, 1, 2], dtype=torch.int32).expand(2, 3, 4))


def test_select_top_k_larger_than_chunks_and_wide():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 2, 128, generator=g).bfloat16()
    summ = torch.randn(2, 2, 3000, 128, generator=g) * 0.1
    want, scores = oracle.select_topk(q, summ, 300)
    got = extension.csa_select_topk(q.to(DEV), summ.to(DEV), 300)
    assert_indices(got, want, scores)
    want, scores = oracle.select_topk(q, summ[:, :, :5], 9)
    got = extension.csa_select_topk(q.to(DEV), summ[:, :, :5].contiguous().to(DEV), 9)
    assert got.shape == (2, 2, 5)
    assert_indices(got, want, scores)


def test_summary_incremental_update():
    case = make_synthetic_case(batch=1, heads=2, seq_len=4096, head_dim=128, chunk_size=64, top_k=4, seed=9)
    k = case.k_cache.to(DEV)
    full = extension.csa_chunk_summary(k, 64)
    part = torch.zeros_like(full)
    native.csa_chunk_summary(k, 64, out=part, chunk_begin=10, num_chunks=5)
    assert torch.equal(part[:, :, 10:15], full[:, :, 10:15])
    assert torch.all(part[:, :, :10] == 0) and torch.all(part[:, :, 15:] == 0)


def test_deterministic_and_tile_invariant():
    case = make_synthetic_case(batch=2, heads=8, seq_len=16384, head_dim=128, chunk_size=64, top_k=16, seed=4)
    q, k, v = case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV)
    summ = extension.csa_chunk_summary(k, 64)
    idx = extension.csa_select_topk(q, summ, 16)
    a = extension.csa_decode_forward_tiled(q, k, v, idx, 64, 16)
    b = extension.csa_decode_forward_tiled(q, k, v, idx, 64, 16)
    assert torch.equal(a, b)
    assert torch.equal(idx, extension.csa_select_topk(q, summ, 16))
    outs = [extension.csa_decode_forward_tiled(q, k, v, idx, 64, t).float() for t in (1, 8, 64, 1024)]
    for o in outs[1:]:
        assert torch.allclose(o, outs[0], atol=1e-2, rtol=1e-2)


def test_large_offsets_beyond_2_to_32_elements():
    """B32 H8 S131072 D128: K and V each hold 2^32 elements, so the last heads sit
    past every 32-bit offset.  Heads (0,0) and (31,7) are checked on the CPU."""
    B, H, S, D, chunk, k = 32, 8, 131072, 128, 64, 8
    g = torch.Generator(device=DEV).manual_seed(0)
    kc = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=DEV).normal_(generator=g)
    vc = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=DEV).normal_(generator=g)
    q = torch.randn(B, H, D, dtype=torch.bfloat16, device=DEV, generator=g)
    C = S // chunk
    idx = torch.arange(C - k, C, dtype=torch.int32, device=DEV).flip(0).expand(B, H, k).contiguous()
    out = extension.csa_decode_forward_tiled(q, kc, vc, idx, chunk, 64)
    summ = extension.csa_chunk_summary(kc, chunk)
    sel = extension.csa_select_topk(q, summ, k)
    for b, h in ((0, 0), (31, 7)):
        ks, vs = kc[b:b + 1, h:h + 1].cpu(), vc[b:b + 1, h:h + 1].cpu()
        qs = q[b:b + 1, h:h + 1].cpu()
        ref = oracle.csa_attend(qs, ks, vs, idx[b:b + 1, h:h + 1].cpu(), chunk)
        assert_close(out[b:b + 1, h:h + 1], ref, 2e-2, 1e-2, f"bh=({b},{h})")
        sref = oracle.chunk_mean(ks, chunk)
        np.testing.assert_allclose(summ[b:b + 1, h:h + 1].cpu().numpy(), sref, rtol=0, atol=2e-6)
        want, scores = oracle.select_topk(qs, sref, k)
        assert_indices(sel[b:b + 1, h:h + 1], want, scores)
    del kc, vc
    torch.cuda.empty_cache()


def test_cuda_graph_replays_match_eager():
    """A step captured on stream s shares s's workspace for its shape with eager
    calls on s, so launch epochs carry across replays and interleaved eager calls;
    eager calls of smaller and larger shapes on s (workspaces of their own) leave
    the captured graph intact.  Every replay and every eager call must equal its
    eager reference bit for bit, with the status word clean."""
    case = make_synthetic_case(batch=1, heads=8, seq_len=32768, head_dim=128, chunk_size=64, top_k=8, seed=0)
    q, k, v = case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV)
    summ = extension.csa_chunk_summary(k, 64)
    g = torch.Generator().manual_seed(11)
    qs, ks, vs = (torch.randn(*shape, generator=g).to(torch.bfloat16).to(DEV)
                  for shape in ((1, 4, 128), (1, 4, 8192, 128), (1, 4, 8192, 128)))
    ql, kl, vl = (torch.randn(*shape, generator=g).to(torch.bfloat16).to(DEV)
                  for shape in ((4, 8, 128), (4, 8, 16384, 128), (4, 8, 16384, 128)))
    summ_s, summ_l = extension.csa_chunk_summary(ks, 64), extension.csa_chunk_summary(kl, 64)
    eager_out, eager_idx = native.csa_decode_step(q, k, v, summ, 64, 8)
    small_out, small_idx = native.csa_decode_step(qs, ks, vs, summ_s, 64, 8)
    large_out, large_idx = native.csa_decode_step(ql, kl, vl, summ_l, 64, 8)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        native.csa_decode_step(q, k, v, summ, 64, 8)  # creates s's workspace for this shape
    assert native.step_workspace_ready(DEV, s.cuda_stream, (8, 512, 128, 8, 64))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        gout, gidx = native.csa_decode_step(q, k, v, summ, 64, 8)
    for r in range(4):
        with torch.cuda.stream(s):
            gout.zero_()
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gidx, eager_idx), r
        assert torch.equal(gout, eager_out), r
        with torch.cuda.stream(s):  # eager work on the capture stream between replays
            o, i = native.csa_decode_step(q, k, v, summ, 64, 8)
            so, si = native.csa_decode_step(qs, ks, vs, summ_s, 64, 8)
            lo, li = native.csa_decode_step(ql, kl, vl, summ_l, 64, 8)
        torch.cuda.synchronize()
        assert torch.equal(o, eager_out) and torch.equal(i, eager_idx), r
        assert torch.equal(so, small_out) and torch.equal(si, small_idx), r
        assert torch.equal(lo, large_out) and torch.equal(li, large_idx), r
    assert all(v == 0 for v in native.csa_step_status().values())


FUSED = [
    # B, H, S, D, chunk, k, dtype      (P = workgroups per head follows from B*H)
    (1, 8, 32768, 128, 64, 8, torch.bfloat16),     # headline: P = 8
    (1, 8, 32768, 128, 64, 32, torch.bfloat16),
    (2, 8, 8192, 128, 64, 8, torch.bfloat16),
    (8, 8, 8192, 128, 64, 16, torch.bfloat16),     # P = 8
    (32, 8, 4096, 128, 64, 8, torch.bfloat16),     # P = 2
    (64, 8, 2048, 128, 64, 4, torch.bfloat16),     # P = 1: one workgroup per head
    # P = 1 on 256 heads: the double-buffered kernel; 70 chunks and 7 x 48 rows
    # walk in ragged batches of 64
    (32, 8, 3360, 128, 48, 7, torch.bfloat16),
    (32, 8, 3360, 128, 48, 7, torch.float16),
    (1, 4, 8192, 64, 64, 8, torch.float16),
    (1, 2, 8192, 256, 32, 12, torch.float32),
    (1, 1, 1048576, 64, 64, 8, torch.bfloat16),    # 16384 chunks: keys stay in global memory
    (1, 2, 4096, 96, 64, 4, torch.bfloat16),       # head_dim 96: two-pass fallback inside the op
    (1, 2, 4096, 128, 64, 4, torch.float64),       # fp64: two-pass fallback
    (1, 2, 32768, 128, 16, 2000, torch.bfloat16),  # k > 1024: two-pass fallback
    (1, 2, 2048, 128, 64, 50, torch.bfloat16),     # k > C clamps to C
]


@pytest.mark.parametrize("B,H,S,D,chunk,k,dtype", FUSED)
def test_fused_step_matches_oracle_and_two_pass(B, H, S, D, chunk, k, dtype):
    g = torch.Generator().manual_seed(B * 7 + H * 3 + k + D)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    kc = torch.randn(B, H, S, D, generator=g).to(dtype)
    vc = torch.randn(B, H, S, D, generator=g).to(dtype)
    qd, kd, vd = q.to(DEV), kc.to(DEV), vc.to(DEV)
    summ = extension.csa_chunk_summary(kd, chunk)
    out, idx = native.csa_decode_step(qd, kd, vd, summ, chunk, k)
    idx2 = extension.csa_select_topk(qd, summ, k)
    assert torch.equal(idx, idx2)
    want, scores = oracle.select_topk(q, summ.cpu(), k)
    assert_indices(idx, want, scores)
    atol, rtol = tol_for(dtype)
    if B * H * S * D <= 64 * 8 * 2048 * 128:
        ref = oracle.csa_attend(q, kc, vc, idx.cpu(), chunk, prob_dtype=oracle.F32)
        assert_close(out, ref, atol, rtol, "fused vs oracle")
    two = extension.csa_decode_forward_tiled(qd, kd, vd, idx, chunk, 16)
    assert torch.allclose(out.float(), two.float(), atol=atol, rtol=rtol)
    assert all(v == 0 for v in native.csa_step_status().values())


WIDE = [
    # B, H, S, D, chunk, k, dtype: the 8-wavefront instantiation forced
    # (CSAHCA_STEP_WIDE=1); phase A batches of 128 summary rows, phase C of 128
    # selected rows, double-buffered
    (1, 8, 32768, 128, 64, 8, torch.bfloat16),   # 512 chunks, 512 rows: four batches each
    (4, 8, 8192, 128, 48, 7, torch.float16),     # 170 chunks, 336 rows: ragged last batches
    (2, 4, 16384, 128, 64, 40, torch.bfloat16),  # 256 chunks, 2560 rows: twenty batches of attention
    (1, 2, 99968, 128, 64, 8, torch.bfloat16),   # 1562 chunks: thirteen batches, the last ragged
    (32, 8, 2048, 128, 64, 20, torch.bfloat16),  # 256 heads, 32 chunks (one short batch), 1280 rows: the default rule's choice
]


@pytest.mark.parametrize("B,H,S,D,chunk,k,dtype", WIDE)
def test_wide_step_matches_oracle_and_split_step(B, H, S, D, chunk, k, dtype, monkeypatch):
    """One workgroup of 8 wavefronts per head against the oracle (ids bit-exact
    up to 1e-5 score ties, outputs within the bf16 bar) and against the split
    kernel on the same inputs (identical ids)."""
    g = torch.Generator().manual_seed(B * 5 + H + k + S // 1024)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    kc = torch.randn(B, H, S, D, generator=g).to(dtype)
    vc = torch.randn(B, H, S, D, generator=g).to(dtype)
    qd, kd, vd = q.to(DEV), kc.to(DEV), vc.to(DEV)
    summ = extension.csa_chunk_summary(kd, chunk)
    monkeypatch.setenv("CSAHCA_STEP_WIDE", "1")
    out, idx = native.csa_decode_step(qd, kd, vd, summ, chunk, k)
    monkeypatch.setenv("CSAHCA_STEP_WIDE", "0")
    out_split, idx_split = native.csa_decode_step(qd, kd, vd, summ, chunk, k)
    assert torch.equal(idx, idx_split)
    want, scores = oracle.select_topk(q, summ.cpu(), k)
    assert_indices(idx, want, scores)
    atol, rtol = tol_for(dtype)
    ref = oracle.csa_attend(q, kc, vc, idx.cpu(), chunk, prob_dtype=oracle.F32)
    assert_close(out, ref, atol, rtol, "wide step vs oracle")
    assert torch.allclose(out.float(), out_split.float(), atol=atol, rtol=rtol)
    assert all(v == 0 for v in native.csa_step_status().values())


def test_fused_step_ties_and_planted_selections():
    B, H, S, D, chunk, k = 1, 8, 32768, 128, 64, 8  # P = 8 workgroups per head exchange keys
    q = torch.ones(B, H, D, dtype=torch.bfloat16, device=DEV)
    kc = torch.ones(B, H, S, D, dtype=torch.bfloat16, device=DEV)
    v = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    _, idx = native.csa_decode_step(q, kc, v, extension.csa_chunk_summary(kc, chunk), chunk, k)
    assert torch.equal(idx.cpu(), torch.arange(k, dtype=torch.int32).expand(B, H, k))  # all tie: lowest ids
    kc[:, :, 300 * chunk:301 * chunk] = 2.0  # one winner above 511 tied chunks
    _, idx = native.csa_decode_step(q, kc, v, extension.csa_chunk_summary(kc, chunk), chunk, k)
    want = torch.tensor([300] + list(range(k - 1)), dtype=torch.int32).expand(B, H, k)
    assert torch.equal(idx.cpu(), want)
    C = S // chunk
    case = make_synthetic_case(batch=B, heads=H, seq_len=S, head_dim=D, chunk_size=chunk, top_k=k, seed=4)
    for ids in (scattered_chunks(B, H, C, k), clustered_chunks(B, H, C, k)):
        kp = plant_chunks(case.q, case.k_cache, ids, chunk, alpha=1.0).to(DEV)
        _, idx = native.csa_decode_step(case.q.to(DEV), kp, case.v_cache.to(DEV),
                                        extension.csa_chunk_summary(kp, chunk), chunk, k)
        assert torch.equal(idx.cpu(), ids)
    assert all(v == 0 for v in native.csa_step_status().values())


def test_pipelined_step_first_batch_follows_the_tie_break():
    """At B32 H8 S8192 top-8 each head is one workgroup (P = 1, the
    double-buffered instantiation), which requests the rows of its first slots
    from a scan for the best chunk while the selection still runs.  With values
    constant per chunk (every row of chunk c holds c) the output is the
    softmax-weighted mean of the attended chunk ids, so a first batch read from
    any chunk but the selection's first shows: all keys tied (ids 0..7, the
    first chunk 0 and not the last tied one), then two planted chunks tied above
    the rest (the lower id first)."""
    B, H, S, D, chunk, k = 32, 8, 8192, 128, 64, 8
    q = torch.ones(B, H, D, dtype=torch.bfloat16, device=DEV)
    kc = torch.ones(B, H, S, D, dtype=torch.bfloat16, device=DEV)
    ids = (torch.arange(S, device=DEV) // chunk).to(torch.bfloat16)
    vc = ids[None, None, :, None].expand(B, H, S, D).contiguous()
    for planted, first in ((), list(range(k))), ((77, 5), [5, 77, 0, 1, 2, 3, 4, 6]):
        for c in planted:
            kc[:, :, c * chunk:(c + 1) * chunk] = 2.0
        out, idx = native.csa_decode_step(q, kc, vc, extension.csa_chunk_summary(kc, chunk), chunk, k)
        want = torch.tensor(first, dtype=torch.int32).expand(B, H, k)
        assert torch.equal(idx.cpu(), want)
        tok = (idx.long().unsqueeze(-1) * chunk + torch.arange(chunk, device=DEV)).reshape(B, H, k * chunk, 1)
        kg = torch.gather(kc, 2, tok.expand(-1, -1, -1, D)).cpu()
        vg = torch.gather(vc, 2, tok.expand(-1, -1, -1, D)).cpu()
        local = torch.arange(k, dtype=torch.int32).expand(B, H, k).contiguous()
        ref = oracle.csa_attend(q.cpu(), kg, vg, local, chunk, prob_dtype=oracle.F32)
        assert_close(out, ref, 2e-2, 1e-2, f"planted {planted}")
    assert all(v == 0 for v in native.csa_step_status().values())
    del q, kc, vc, out
    torch.cuda.empty_cache()


def test_fused_step_device_count_matches_oracle():
    B, H, S, D, chunk, k = 1, 8, 32768, 128, 64, 8
    case = make_synthetic_case(batch=B, heads=H, seq_len=S, head_dim=D, chunk_size=chunk, top_k=k, seed=6)
    q, kd, vd = case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV)
    summ = extension.csa_chunk_summary(kd, chunk)
    summ_ref = oracle.chunk_mean(case.k_cache, chunk)
    n = torch.zeros(1, dtype=torch.int32, device=DEV)
    for count in (1, 5, 37, 100, 512):  # few chunks leave most workgroups without local candidates
        n.fill_(count)
        out, idx = native.csa_decode_step_dev(q, kd, vd, summ, n, chunk, k)
        want, scores = oracle.select_topk(case.q, summ_ref[:, :, :count], k)
        kk = want.shape[-1]
        assert_indices(idx[:, :, :kk], want, scores)
        assert torch.all(idx[:, :, kk:] == -1)
        ref = oracle.csa_attend(case.q, case.k_cache, case.v_cache, idx.cpu(), chunk, prob_dtype=oracle.F32)
        assert_close(out, ref, 2e-2, 1e-2, f"count {count}")
    assert all(v == 0 for v in native.csa_step_status().values())


def test_fused_step_repeated_calls_rearm_counters():
    case = make_synthetic_case(batch=1, heads=8, seq_len=32768, head_dim=128, chunk_size=64, top_k=8, seed=1)
    q, k, v = case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV)
    summ = extension.csa_chunk_summary(k, 64)
    first, idx = native.csa_decode_step(q, k, v, summ, 64, 8)
    for _ in range(50):
        out, idx2 = native.csa_decode_step(q, k, v, summ, 64, 8)
    torch.cuda.synchronize()
    assert torch.equal(out, first) and torch.equal(idx2, idx)
    assert all(v == 0 for v in native.csa_step_status().values())


def test_exchange_timeout_poisons_the_head_until_the_workspace_is_zeroed(monkeypatch):
    """The fused step's time-out path, forced from the host: with
    CSAHCA_STEP_TEST_TIMEOUT=n the last workgroup of head 0 publishes neither
    keys nor partial and every bounded wait gives up after n polls, so every
    workgroup still exits.  Head 0's output is NaN and the sticky status bit
    is set, while the other heads keep the oracle's ids and outputs.  Later
    calls on that workspace (switch off) keep head 0 NaN and the bit set; a
    zero-filled workspace recovers."""
    B, H, S, D, chunk, k = 1, 8, 32768, 128, 64, 8  # P = 8 workgroups per head
    case = make_synthetic_case(batch=B, heads=H, seq_len=S, head_dim=D, chunk_size=chunk, top_k=k, seed=11)
    q, kd, vd = case.q.to(DEV), case.k_cache.to(DEV), case.v_cache.to(DEV)
    summ = extension.csa_chunk_summary(kd, chunk)
    want, scores = oracle.select_topk(case.q, summ.cpu(), k)
    ref = oracle.csa_attend(case.q, case.k_cache, case.v_cache, want, chunk, prob_dtype=oracle.F32)
    native.release_step_workspaces()
    monkeypatch.setenv("CSAHCA_STEP_TEST_TIMEOUT", "4096")
    out, idx = native.csa_decode_step(q, kd, vd, summ, chunk, k)
    torch.cuda.synchronize()
    monkeypatch.delenv("CSAHCA_STEP_TEST_TIMEOUT")

    def healthy_heads_match(o, i):
        assert_indices(i[:, 1:], want[:, 1:], scores[:, 1:])
        assert_close(o[:, 1:], ref[:, 1:], 2e-2, 1e-2, "heads 1..7")

    assert torch.isnan(out[0, 0].float()).all()
    healthy_heads_match(out, idx)
    assert all(v & 1 for v in native.csa_step_status().values())
    for _ in range(2):  # the head stays poisoned on this workspace
        out2, idx2 = native.csa_decode_step(q, kd, vd, summ, chunk, k)
        torch.cuda.synchronize()
        assert torch.isnan(out2[0, 0].float()).all()
        healthy_heads_match(out2, idx2)
    assert all(v & 1 for v in native.csa_step_status().values())
    native.release_step_workspaces()  # the next call zero-fills a new workspace
    out3, idx3 = native.csa_decode_step(q, kd, vd, summ, chunk, k)
    assert_indices(idx3, want, scores)
    assert_close(out3, ref, 2e-2, 1e-2, "after a zero-filled workspace")
    assert all(v == 0 for v in native.csa_step_status().values())


def test_workgroups_per_head_override_is_bounded_by_residency(monkeypatch):
    """CSAHCA_STEP_WGS_PER_HEAD=64 at B32 H8 asks for 16384 workgroups that wait
    on each other, far more than the device holds at once; the library shrinks P
    to what the kernel's occupancy allows, and the result matches the default
    launch (same ids; outputs within fp32 reordering)."""
    B, H, S, D, chunk, k = 32, 8, 8192, 128, 64, 8
    g = torch.Generator().manual_seed(29)
    q, kc, vc = (torch.randn(*sh, generator=g).to(torch.bfloat16).to(DEV)
                 for sh in ((B, H, D), (B, H, S, D), (B, H, S, D)))
    summ = extension.csa_chunk_summary(kc, chunk)
    want, want_idx = native.csa_decode_step(q, kc, vc, summ, chunk, k)
    monkeypatch.setenv("CSAHCA_STEP_WGS_PER_HEAD", "64")
    for _ in range(3):
        got, idx = native.csa_decode_step(q, kc, vc, summ, chunk, k)
    torch.cuda.synchronize()
    assert torch.equal(idx, want_idx)
    assert torch.allclose(got.float(), want.float(), atol=2e-2, rtol=1e-2)
    assert all(v == 0 for v in native.csa_step_status().values())


GRID = [  # every point of the sweep B {1, 8, 32} x S {8192, 32768, 131072} x top-k {8, 32}
    (B, S, k) for B in (1, 8, 32) for S in (8192, 32768, 131072) for k in (8, 32)
]


def _check_step_against_oracle(B, S, k, H=8, D=128, chunk=64):
    """The fused decode step on N(0,1) bf16 inputs drawn on the device against
    the oracle: chunk summaries on the first and last head, selections of
    every head (bit-exact up to 1e-5 score ties), and the attention of every
    head over the selected chunks' tokens, gathered on the device so the
    oracle works on [B, H, k*chunk, D] copies."""
    g = torch.Generator(device=DEV).manual_seed(B * 31 + S // 1024 + k)
    q = torch.randn(B, H, D, device=DEV, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, H, S, D, device=DEV, generator=g, dtype=torch.bfloat16)
    vc = torch.randn(B, H, S, D, device=DEV, generator=g, dtype=torch.bfloat16)
    summ = extension.csa_chunk_summary(kc, chunk)
    out, idx = native.csa_decode_step(q, kc, vc, summ, chunk, k)
    for b, h in ((0, 0), (B - 1, H - 1)):
        np.testing.assert_allclose(summ[b:b + 1, h:h + 1].cpu().numpy(),
                                   oracle.chunk_mean(kc[b:b + 1, h:h + 1].cpu(), chunk), rtol=1e-6, atol=2e-6)
    want, scores = oracle.select_topk(q.cpu(), summ.cpu(), k)
    assert_indices(idx, want, scores)
    tok = (idx.long().unsqueeze(-1) * chunk + torch.arange(chunk, device=DEV)).reshape(B, H, k * chunk, 1)
    kg = torch.gather(kc, 2, tok.expand(-1, -1, -1, D)).cpu()
    vg = torch.gather(vc, 2, tok.expand(-1, -1, -1, D)).cpu()
    local = torch.arange(k, dtype=torch.int32).expand(B, H, k).contiguous()
    ref = oracle.csa_attend(q.cpu(), kg, vg, local, chunk, prob_dtype=oracle.F32)
    assert_close(out, ref, 2e-2, 1e-2, f"B{B} S{S} k{k}")
    assert all(v == 0 for v in native.csa_step_status().values())
    del q, kc, vc, summ, out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B,S,k", GRID)
def test_sweep_grid_point_matches_oracle(B, S, k):
    """The fused decode step at a config-1 grid point (H8 D128 chunk 64, bf16
    N(0,1) drawn on the device) against the oracle: chunk summaries on the
    first and last head, selection from the device summaries (ids bit-exact up
    to 1e-5 score ties), and attention over the selected chunks' tokens, which
    are gathered on the device so the oracle works on [B, H, k*64, D] copies.

    The launch shape the host picks differs across the grid: P = 8 workgroups
    per head with a head's workgroups on one XCD at B1 S32768 top-8; P = 1 and
    the double-buffered instantiation at B32 top-8 (at S131072 over K and V of
    2^32 elements, 8 GiB, each, so the byte offsets of the last heads pass
    2^32); the 8-wavefront instantiation at B32 top-32."""
    _check_step_against_oracle(B, S, k)



@pytest.mark.parametrize("B,S,k", [
    (32, 12288, 5),  # 192 chunks: 3 summary batches; 320 slots: 5 attention batches, the first requested early
    (32, 20480, 3),  # 320 chunks: 5 summary batches; 192 slots: 3 attention batches
    (32, 16384, 1),  # 64 slots: one attention batch per wavefront (batch by batch)
])
def test_double_buffered_walks_end_in_either_buffer(B, S, k):
    """At B32 H8 each head is one workgroup on the double-buffered
    instantiation, whose walks consume their last batch in a tail of their own:
    in the second buffer after an even number of batches (every config-1
    point) and in the first after an odd number, which these shapes give to
    both the summary walk and the attention walk."""
    _check_step_against_oracle(B, S, k)


def test_largest_sweep_point_properties():
    """B32 H8 S131072 D128 top-32 (17 GiB of K/V) is too large for the CPU
    oracle, so parity rests on size-independent properties: planted chunks are
    selected exactly and in their planted order, the fused step's ids equal the
    selection kernels', and its output equals the two-pass split-KV route over
    those ids."""
    B, H, S, D, chunk, k = 32, 8, 131072, 128, 64, 32
    g = torch.Generator(device=DEV).manual_seed(123)
    q = torch.randn(B, H, D, device=DEV, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, H, S, D, device=DEV, generator=g, dtype=torch.bfloat16)
    vc = torch.randn(B, H, S, D, device=DEV, generator=g, dtype=torch.bfloat16)
    ids = scattered_chunks(B, H, S // chunk, k).to(DEV)
    q_hat = q.float() / q.float().norm(dim=-1, keepdim=True)
    for j, c in enumerate(ids[0, 0].tolist()):  # the same chunks in every head; bias k - j orders them
        kc[:, :, c * chunk:(c + 1) * chunk] += ((k - j) * q_hat)[:, :, None, :].to(torch.bfloat16)
    summ = extension.csa_chunk_summary(kc, chunk)
    out, idx = native.csa_decode_step(q, kc, vc, summ, chunk, k)
    assert torch.equal(idx, ids)
    assert torch.equal(idx, extension.csa_select_topk(q, summ, k))
    two = extension.csa_decode_forward_tiled(q, kc, vc, idx, chunk, 16)
    assert_close(out, two.float().cpu().numpy(), 2e-2, 1e-2, "fused vs two-pass at B32 S131072 k32")
    assert all(v == 0 for v in native.csa_step_status().values())
    del q, kc, vc, summ, out, two
    torch.cuda.empty_cache()


def test_device_clock_stamps_time_a_captured_run():
    """Two clock stamps captured into one graph around decode steps: every
    replay writes a later pair, the interval is positive and below the host's
    wall time for the replay, and it grows with the number of steps inside."""
    import time

    B, H, S, D, chunk, k = 1, 8, 32768, 128, 64, 8
    g = torch.Generator(device=DEV).manual_seed(7)
    q = torch.randn(B, H, D, device=DEV, generator=g).to(torch.bfloat16)
    kc = torch.randn(B, H, S, D, device=DEV, generator=g, dtype=torch.bfloat16)
    vc = torch.randn(B, H, S, D, device=DEV, generator=g, dtype=torch.bfloat16)
    summ = extension.csa_chunk_summary(kc, chunk)
    khz = native.device_clock_khz()
    assert khz > 0
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        native.csa_decode_step(q, kc, vc, summ, chunk, k)
    torch.cuda.synchronize()
    spans = {}
    for n in (1, 8):
        stamps = torch.zeros(2, dtype=torch.int64, device=DEV)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            native.device_clock_stamp(stamps, 0)
            for _ in range(n):
                native.csa_decode_step(q, kc, vc, summ, chunk, k)
            native.device_clock_stamp(stamps, 1)
        prev = None
        for _ in range(3):
            t0 = time.perf_counter()
            with torch.cuda.stream(s):
                graph.replay()
            torch.cuda.synchronize()
            wall_ms = (time.perf_counter() - t0) * 1e3
            a, b = stamps.cpu().tolist()
            assert b > a
            assert (b - a) / khz < wall_ms
            if prev is not None:
                assert a > prev
            prev = b
        spans[n] = (b - a) / khz
    assert spans[8] > 4 * spans[1]
    assert all(v == 0 for v in native.csa_step_status().values())


def test_phase_timeline_tool_runs_the_stamped_build():
    """python -m csahca_amd.timeline (libcsahca_timeline.so, in a child process
    of its own) reports every phase boundary of the decode step in order."""
    import re
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, "-m", "csahca_amd.timeline", "--seq", "8192", "--steps", "5", "--copies", "2"],
                       cwd=root, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    rows = [ln for ln in r.stdout.splitlines() if ln.startswith("| ") and not ln.startswith("| boundary")]
    times = {}
    for ln in rows:
        cells = [c.strip() for c in ln.strip("|").split("|")]
        times[cells[0]] = float(cells[1])
    names = [n for n in times if not n.startswith("last workgroup")]
    assert any(n.startswith("A:") for n in names) and any(n.startswith("D: output") for n in names)
    seq = [times[n] for n in names]
    assert all(b >= a for a, b in zip(seq, seq[1:])) and seq[0] > 0
    assert re.search(r"clock \d+ kHz", r.stdout)



COLOCATE = [
    # B, H, S, D, chunk, k, dtype: the placement of a head's P workgroups
    (1, 8, 32768, 128, 64, 8, torch.bfloat16),   # headline: P = 8, one head per XCD
    (1, 8, 32768, 128, 64, 32, torch.float16),   # 2048 slots
    (1, 2, 4096, 128, 48, 5, torch.bfloat16),    # 2 heads (not a multiple of 8), ragged split
    (8, 8, 8192, 128, 64, 8, torch.bfloat16),    # 64 heads
    (32, 8, 4096, 128, 64, 8, torch.bfloat16),   # 256 heads, P = 2
    (1, 4, 8192, 64, 64, 8, torch.float16),
]


@pytest.mark.parametrize("B,H,S,D,chunk,k,dtype", COLOCATE)
def test_colocated_workgroups_give_the_same_bits(B, H, S, D, chunk, k, dtype, monkeypatch):
    """Block b serving head b % (B*H) (a head's workgroups on one XCD,
    CSAHCA_STEP_COLOCATE=1) or head b / P (=0) changes only where each
    (head, workgroup) runs: ids and outputs are identical, and both match the
    oracle."""
    g = torch.Generator().manual_seed(B * 11 + H + k + S // 1024)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    kc = torch.randn(B, H, S, D, generator=g).to(dtype)
    vc = torch.randn(B, H, S, D, generator=g).to(dtype)
    qd, kd, vd = q.to(DEV), kc.to(DEV), vc.to(DEV)
    summ = extension.csa_chunk_summary(kd, chunk)
    outs = {}
    for colo in ("1", "0"):
        monkeypatch.setenv("CSAHCA_STEP_COLOCATE", colo)
        outs[colo] = native.csa_decode_step(qd, kd, vd, summ, chunk, k)
    assert torch.equal(outs["1"][1], outs["0"][1])
    assert torch.equal(outs["1"][0], outs["0"][0])
    want, scores = oracle.select_topk(q, summ.cpu(), k)
    assert_indices(outs["1"][1], want, scores)
    atol, rtol = tol_for(dtype)
    ref = oracle.csa_attend(q, kc, vc, outs["1"][1].cpu(), chunk, prob_dtype=oracle.F32)
    assert_close(outs["1"][0], ref, atol, rtol, "colocated")
    assert all(v == 0 for v in native.csa_step_status().values())
