"""GPU parity of the decode blocks (csahca_amd/block.py).

MiniCSADecodeBlock restates hybrid_attention/model_inference.py:14-76.  It is
checked against the reference block's own outputs (tests/golden/block_mini.npz,
torch-csa backend) and against oracle.block.mini_block, the CPU restatement
that fixture pins bit for bit, with cuda-csa math (fp32 probabilities).
HybridDecodeBlock (the BASELINE config-2 block over a growing cache) is checked
step by step against oracle.block.baseline_block_steps, pinned by closed forms,
which rounds exactly where the GPU block stores bf16 (q, the appended K/V, every
linear output) -- also at the stated shape: hidden 1024 (H8 D128), a 32768-token
cache, std-0.02 weights, MLP ratio 2.0 and 0.0, across a chunk boundary.
Tolerance: |got - ref| <= 2e-2 + 1e-2 |ref| on block outputs.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from csahca_amd import native
from oracle import block as OB
from csahca_amd.block import HybridDecodeBlock, MiniCSADecodeBlock, rms_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    native.lib()


def assert_close(got, ref, atol=2e-2, rtol=1e-2, what=""):
    g = got.detach().double().cpu().numpy()
    r = ref.detach().double().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref, np.float64)
    diff = np.abs(g - r)
    bad = diff > atol + rtol * np.abs(r)
    assert not bad.any(), f"{what} max_abs={diff.max():.3e} bad={int(bad.sum())}/{bad.size}"


def cpu_csa(q, k, v, selected, chunk):
    """cuda-csa semantics (fp32 probabilities) from the oracle, rounded to bf16."""
    out = oracle.csa_attend(q, k, v, selected, chunk, prob_dtype=oracle.F32)
    return torch.from_numpy(out).to(torch.float32).to(BF)


def make_static(B=1, H=8, S=4096, D=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(B, H * D, generator=g).to(BF)
    k = torch.randn(B, H, S, D, generator=g).to(BF)
    v = torch.randn(B, H, S, D, generator=g).to(BF)
    return hidden, k, v


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("mlp_ratio", [0.0, 2.0])
def test_mini_block_matches_cpu_restatement(mlp_ratio, fused):
    hidden, k, v = make_static()
    blk = MiniCSADecodeBlock(heads=8, head_dim=128, dtype=BF, device=DEV, mlp_ratio=mlp_ratio, seed=1, fused=fused)
    mlp = dict(w_up=blk.w_up.cpu(), w_down=blk.w_down.cpu()) if mlp_ratio else {}
    want, sel = OB.mini_block(hidden, blk.w_q.cpu(), blk.w_out.cpu(), k, v, chunk=64, top_k=8, prob_dtype=oracle.F32,
                              **mlp)
    sel_t = torch.from_numpy(sel).to(torch.int32).to(DEV)
    got = blk(hidden.to(DEV), k.to(DEV), v.to(DEV), selection="precomputed", selected_chunks=sel_t)
    assert_close(got, want, what="precomputed")
    # dynamic selection (fused step) from cached or per-step summaries selects the same chunks here
    summ = native.csa_chunk_summary(k.to(DEV), 64)
    got_dyn = blk(hidden.to(DEV), k.to(DEV), v.to(DEV), selection="dynamic", summary=summ)
    got_dyn2 = blk(hidden.to(DEV), k.to(DEV), v.to(DEV), selection="dynamic", summary=None)
    assert torch.equal(got_dyn, got_dyn2)
    assert_close(got_dyn, want, what="dynamic")


@pytest.mark.parametrize("fused", [True, False])
def test_mini_block_graph_replays_match_eager(fused):
    hidden, k, v = (t.to(DEV) for t in make_static(seed=3))
    blk = MiniCSADecodeBlock(heads=8, head_dim=128, dtype=BF, device=DEV, mlp_ratio=2.0, seed=2, fused=fused)
    summ = native.csa_chunk_summary(k, 64)
    eager = blk(hidden, k, v, selection="dynamic", summary=summ)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        blk(hidden, k, v, selection="dynamic", summary=summ)  # warm the stream's workspace
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = blk(hidden, k, v, selection="dynamic", summary=summ)
    for _ in range(3):
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        with torch.cuda.stream(s):  # eager work on the capture stream between replays
            again = blk(hidden, k, v, selection="dynamic", summary=summ)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    assert all(x == 0 for x in native.csa_step_status().values())


def cpu_hybrid_reference(blk: HybridDecodeBlock, k0, v0, hiddens):
    """oracle.block.baseline_block_steps with the block's own weights."""
    w = {n: getattr(blk, n).cpu() for n in ("w_qkv", "w_out", "norm1", "norm2")}
    if blk.use_mlp:
        w["w_up"], w["w_down"] = blk.w_up.cpu(), blk.w_down.cpu()
    return OB.baseline_block_steps(w, k0, v0, hiddens, heads=blk.heads, head_dim=blk.head_dim,
                                   chunk=blk.chunk_size, top_k=blk.top_k, prob_dtype=oracle.F32)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("mlp_ratio", [0.0, 2.0])
def test_hybrid_block_steps_match_cpu_across_a_chunk_boundary(mlp_ratio, fused):
    B, H, D, S0, steps = 1, 4, 64, 250, 10  # the 256th token completes chunk 4 during the run
    blk = HybridDecodeBlock(batch=B, heads=H, head_dim=D, capacity=512, chunk_size=64, top_k=3, mlp_ratio=mlp_ratio,
                            device=DEV, seed=5, fused=fused)
    assert blk.fused == fused
    g = torch.Generator().manual_seed(9)
    k0 = torch.randn(B, H, S0, D, generator=g).to(BF)
    v0 = torch.randn(B, H, S0, D, generator=g).to(BF)
    hiddens = [torch.randn(B, H * D, generator=g).to(BF) for _ in range(steps)]
    blk.prefill(k0.to(DEV), v0.to(DEV))
    assert blk.summary.shape[2] == 3
    want = cpu_hybrid_reference(blk, k0, v0, hiddens)
    for i, hdn in enumerate(hiddens):
        got = blk(hdn.to(DEV))
        assert_close(got, want[i], what=f"step {i}")
    assert blk.length == S0 + steps and blk.summary.shape[2] == 4
    # the summary of the chunk completed during decoding equals a fresh build
    fresh = native.csa_chunk_summary(blk.k_cache[:, :, :256].contiguous(), 64)
    torch.testing.assert_close(blk.summary, fresh, rtol=0, atol=0)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("mlp_ratio", [0.0, 2.0])
def test_mini_block_matches_the_reference_blocks_outputs(mlp_ratio, fused, golden_dir):
    """The reference block's own output (torch-csa backend) and selection.
    Odd hidden features are zero in the fixture, so there the output is the
    block's update alone; its tolerance scales with that update's magnitude."""
    z = np.load(golden_dir / "block_mini.npz")
    tag = f"mlp{int(mlp_ratio)}"
    bf = lambda name: torch.from_numpy(z[name].view(np.int16)).view(BF).to(DEV)  # noqa: E731
    hidden, k, v = bf("hidden"), bf("k"), bf("v")
    blk = MiniCSADecodeBlock(heads=2, head_dim=64, dtype=BF, device=DEV, mlp_ratio=mlp_ratio, fused=fused)
    blk.w_q, blk.w_out = bf(f"{tag}_w_q"), bf(f"{tag}_w_out")
    if mlp_ratio:
        blk.w_up, blk.w_down = bf(f"{tag}_w_up"), bf(f"{tag}_w_down")
    ref = torch.from_numpy(z[f"{tag}_out"].view(np.int16)).view(BF).float()
    sel = torch.from_numpy(z[f"{tag}_selected"]).to(DEV)
    summ = native.csa_chunk_summary(k, 64)
    _, idx = native.csa_decode_step(native.block_linear(hidden, blk.w_q).view(2, 2, 64) if fused else
                                    F.linear(hidden, blk.w_q).view(2, 2, 64), k, v, summ, 64, 4)
    assert torch.equal(idx, sel)
    for got in (blk(hidden, k, v, selection="dynamic", summary=summ, chunk_size=64, top_k=4),
                blk(hidden, k, v, selection="precomputed", selected_chunks=sel, chunk_size=64)):
        got = got.float().cpu()
        assert_close(got[:, 0::2], ref[:, 0::2], what="input features")
        scale = ref[:, 1::2].abs().max().item()
        assert_close(got[:, 1::2], ref[:, 1::2], atol=2e-2 * scale, what="update-only features")


@pytest.mark.parametrize("mlp_ratio", [0.0, 2.0])
def test_hybrid_block_at_the_stated_shape_across_a_chunk_boundary(mlp_ratio):
    """BASELINE config 2's block as stated: hidden 1024 (H8 D128), std-0.02
    weights, a 32768-token cache, chunk 64, top 8.  The cache holds 32765
    tokens; the third step's token completes chunk 511.  Every step is checked
    against the CPU restatement; a graph of one step, replayed from the same
    state, equals the eager steps bit for bit."""
    B, H, D, S0, steps = 1, 8, 128, 32765, 6
    mk = lambda: HybridDecodeBlock(batch=B, heads=H, head_dim=D, capacity=S0 + steps + 64, chunk_size=64,  # noqa: E731
                                   top_k=8, mlp_ratio=mlp_ratio, device=DEV, seed=41)
    eager, graphed = mk(), mk()
    assert eager.fused and torch.equal(eager.w_qkv, graphed.w_qkv)
    assert abs(eager.w_qkv.float().std().item() - 0.02) < 1e-3
    g = torch.Generator().manual_seed(42)
    k0 = torch.randn(B, H, S0, D, generator=g).to(BF)
    v0 = torch.randn(B, H, S0, D, generator=g).to(BF)
    hiddens = [torch.randn(B, H * D, generator=g).to(BF) for _ in range(steps)]
    for blk in (eager, graphed):
        blk.prefill(k0.to(DEV), v0.to(DEV))
    want = cpu_hybrid_reference(eager, k0, v0, hiddens)
    hbuf = hiddens[0].to(DEV)
    replay, gout = graphed.capture(hbuf)
    for i, hdn in enumerate(hiddens):
        got = eager(hdn.to(DEV))
        assert_close(got, want[i], what=f"step {i}")
        hbuf.copy_(hdn.to(DEV))
        assert torch.equal(replay(), got), f"graph step {i}"
    assert int(eager.nchunks.item()) == 512 == int(graphed.nchunks.item())
    fresh = native.csa_chunk_summary(eager.k_cache[:, :, :32768].contiguous(), 64)
    torch.testing.assert_close(eager.summary[:, :, 511], fresh[:, :, 511], rtol=0, atol=0)
    assert all(x == 0 for x in native.csa_step_status().values())


def test_fused_hybrid_block_batch_two_matches_cpu():
    B, H, D, S0, steps = 2, 8, 128, 190, 4  # the 192nd token completes chunk 2
    blk = HybridDecodeBlock(batch=B, heads=H, head_dim=D, capacity=256, chunk_size=64, top_k=2, mlp_ratio=2.0,
                            device=DEV, seed=11)
    assert blk.fused
    g = torch.Generator().manual_seed(12)
    k0 = torch.randn(B, H, S0, D, generator=g).to(BF)
    v0 = torch.randn(B, H, S0, D, generator=g).to(BF)
    hiddens = [torch.randn(B, H * D, generator=g).to(BF) for _ in range(steps)]
    blk.prefill(k0.to(DEV), v0.to(DEV))
    want = cpu_hybrid_reference(blk, k0, v0, hiddens)
    for i, hdn in enumerate(hiddens):
        assert_close(blk(hdn.to(DEV)), want[i], what=f"step {i}")
    assert int(blk.pos.item()) == S0 + steps and int(blk.nchunks.item()) == (S0 + steps) // 64


def test_hybrid_block_rejects_unfusable_shapes_when_asked_to_fuse():
    with pytest.raises(ValueError, match="fused decode step"):
        HybridDecodeBlock(batch=5, heads=2, head_dim=64, capacity=128, device=DEV, fused=True)
    blk = HybridDecodeBlock(batch=5, heads=2, head_dim=64, capacity=128, device=DEV)
    assert not blk.fused  # automatic choice falls back to torch products


# ---------------------------------------------------------------------------
# Device-side position / chunk count (graph-capturable growing cache)
# ---------------------------------------------------------------------------

def test_summary_at_writes_only_the_chunk_a_token_completes():
    _, k, _ = make_static(B=1, H=4, S=512, D=64, seed=11)
    k = k.to(DEV)
    fresh = native.csa_chunk_summary(k, 64)
    summ = torch.full((1, 4, 8, 64), -7.0, device=DEV)
    pos = torch.zeros(1, dtype=torch.int64, device=DEV)
    for p in (0, 62, 64, 100, 126):  # completes no chunk
        pos.fill_(p)
        native.csa_chunk_summary_at(k, summ, 64, pos)
    assert torch.all(summ == -7.0)
    for p, c in ((63, 0), (191, 2), (511, 7)):
        pos.fill_(p)
        native.csa_chunk_summary_at(k, summ, 64, pos)
        torch.testing.assert_close(summ[:, :, c], fresh[:, :, c], rtol=0, atol=0)
    untouched = [c for c in range(8) if c not in (0, 2, 7)]
    assert torch.all(summ[:, :, untouched] == -7.0)
    pos.fill_(575)  # chunk 8: past both the summary rows and the cache
    native.csa_chunk_summary_at(k, summ, 64, pos)
    pos.fill_(-1)
    native.csa_chunk_summary_at(k, summ, 64, pos)
    assert torch.all(summ[:, :, untouched] == -7.0)


def test_decode_step_dev_matches_the_host_count_step():
    _, k, v = make_static(B=2, H=4, S=4096, D=128, seed=12)
    q = torch.randn(2, 4, 128, generator=torch.Generator().manual_seed(13)).to(BF).to(DEV)
    k, v = k.to(DEV), v.to(DEV)
    summ = native.csa_chunk_summary(k, 64)  # 64 chunks
    n = torch.tensor([64], dtype=torch.int32, device=DEV)
    want, want_idx = native.csa_decode_step(q, k, v, summ, 64, 8)
    got, got_idx = native.csa_decode_step_dev(q, k, v, summ, n, 64, 8)
    assert torch.equal(got_idx, want_idx) and torch.equal(got, want)
    # fewer chunks in play than summary rows: the first 40 only
    n.fill_(40)
    part, part_idx = native.csa_decode_step(q, k, v, summ[:, :, :40].contiguous(), 64, 8)
    got, got_idx = native.csa_decode_step_dev(q, k, v, summ, n, 64, 8)
    assert torch.equal(got_idx, part_idx)
    assert_close(got, part, atol=1e-3, rtol=1e-3, what="40 of 64 chunks")


@pytest.mark.parametrize("D,dtype", [(128, BF), (64, torch.float16), (256, torch.float32)])
def test_decode_step_at_equals_summary_at_then_step_dev(D, dtype):
    """One launch (summary built inside the step) against the two-launch
    sequence, bit for bit, token by token across chunk boundaries: the summary
    rows, the selected ids and the outputs."""
    B, H, chunk, cap, k = 1, 4, 32, 20 * 32, 3
    g = torch.Generator().manual_seed(D)
    kc = torch.randn(B, H, cap, D, generator=g).to(dtype).to(DEV)
    vc = torch.randn(B, H, cap, D, generator=g).to(dtype).to(DEV)
    q = torch.randn(B, H, D, generator=g).to(dtype).to(DEV)
    Cs = cap // chunk
    s1 = torch.zeros(B, H, Cs, D, dtype=torch.float32, device=DEV)
    s2 = torch.zeros_like(s1)
    start = 3 * chunk - 3
    native.csa_chunk_summary(kc, chunk, out=s1, chunk_begin=0, num_chunks=start // chunk)
    s2.copy_(s1)
    pos = torch.zeros(1, dtype=torch.int64, device=DEV)
    nch = torch.zeros(1, dtype=torch.int32, device=DEV)
    for p in list(range(start, start + 8)) + [cap - 1]:  # completes chunks 2 and 19
        pos.fill_(p)
        native.csa_chunk_summary_at(kc, s1, chunk, pos)
        nch.fill_((p + 1) // chunk)
        o1, i1 = native.csa_decode_step_dev(q, kc, vc, s1, nch, chunk, k)
        o2, i2 = native.csa_decode_step_at(q, kc, vc, s2, pos, chunk, k)
        assert torch.equal(s1, s2), p
        assert torch.equal(i1, i2) and torch.equal(o1, o2), p
    fresh = native.csa_chunk_summary(kc, chunk)
    assert torch.equal(s2[:, :, :3], fresh[:, :, :3]) and torch.equal(s2[:, :, 19], fresh[:, :, 19])


def test_decode_step_dev_with_fewer_chunks_than_top_k():
    _, k, v = make_static(B=1, H=4, S=1024, D=64, seed=14)
    q = torch.randn(1, 4, 64, generator=torch.Generator().manual_seed(15)).to(BF)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    summ = native.csa_chunk_summary(kd, 64)  # 16 rows
    n = torch.tensor([3], dtype=torch.int32, device=DEV)
    got, idx = native.csa_decode_step_dev(qd, kd, vd, summ, n, 64, 8)
    want_idx, _ = oracle.select_topk(q, oracle.chunk_mean(k[:, :, :192].contiguous(), 64), 8)
    assert idx.shape == (1, 4, 8)
    assert np.array_equal(idx[:, :, :3].cpu().numpy(), want_idx) and torch.all(idx[:, :, 3:] == -1)
    assert_close(got, cpu_csa(q, k, v, want_idx, 64), what="3 chunks")
    n.fill_(0)
    got, idx = native.csa_decode_step_dev(qd, kd, vd, summ, n, 64, 8)
    assert torch.all(idx == -1) and torch.all(got == 0)
    n.fill_(1000)  # clamped to the 16 summary rows
    got, idx = native.csa_decode_step_dev(qd, kd, vd, summ, n, 64, 8)
    full, full_idx = native.csa_decode_step(qd, kd, vd, summ, 64, 8)
    assert torch.equal(idx, full_idx) and torch.equal(got, full)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("mlp_ratio", [0.0, 2.0])
def test_hybrid_block_graph_replays_match_eager_steps(mlp_ratio, fused):
    B, H, D, S0, steps = 1, 4, 64, 1000, 100  # tokens 1024 and 1088 complete chunks 15 and 16
    blocks = [HybridDecodeBlock(batch=B, heads=H, head_dim=D, capacity=1200, chunk_size=64, top_k=4,
                                mlp_ratio=mlp_ratio, device=DEV, seed=21, fused=fused) for _ in range(2)]
    g = torch.Generator().manual_seed(22)
    k0 = torch.randn(B, H, S0, D, generator=g).to(BF).to(DEV)
    v0 = torch.randn(B, H, S0, D, generator=g).to(BF).to(DEV)
    hiddens = [torch.randn(B, H * D, generator=g).to(BF).to(DEV) for _ in range(steps)]
    for blk in blocks:
        blk.prefill(k0, v0)
    eager, graphed = blocks
    hbuf = torch.empty(B, H * D, dtype=BF, device=DEV)
    hbuf.copy_(hiddens[0])
    replay, out = graphed.capture(hbuf)
    for i in range(steps):
        want = eager(hiddens[i])
        hbuf.copy_(hiddens[i])
        got = replay()
        assert torch.equal(got, want), f"step {i}"
    assert eager.length == graphed.length == S0 + steps
    assert int(graphed.pos.item()) == S0 + steps and int(graphed.nchunks.item()) == (S0 + steps) // 64
    assert torch.equal(graphed.k_cache, eager.k_cache) and torch.equal(graphed.summary_buf, eager.summary_buf)
    fresh = native.csa_chunk_summary(eager.k_cache[:, :, :1088].contiguous(), 64)
    torch.testing.assert_close(eager.summary, fresh, rtol=0, atol=0)


@pytest.mark.parametrize("fused", [True, False])
def test_mini_block_in_place_output_equals_returned_output(fused):
    hidden, k, v = (t.to(DEV) for t in make_static(seed=4))
    blk = MiniCSADecodeBlock(heads=8, head_dim=128, dtype=BF, device=DEV, mlp_ratio=2.0, seed=3, fused=fused)
    summ = native.csa_chunk_summary(k, 64)
    want = blk(hidden, k, v, selection="dynamic", summary=summ)
    buf = hidden.clone()
    got = blk(buf, k, v, selection="dynamic", summary=summ, out=buf)
    assert got.data_ptr() == buf.data_ptr() and torch.equal(buf, want)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("mlp_ratio", [0.0, 2.0])
def test_hybrid_block_multi_step_graph_with_feedback_matches_eager(mlp_ratio, fused):
    """A graph of 5 consecutive steps whose results feed the next step in place
    equals 5 eager steps with the hidden state fed back, replay after replay,
    across a chunk boundary."""
    B, H, D, S0, G, reps = 1, 4, 64, 118, 5, 4  # token 128 completes chunk 1 during replay 1
    blocks = [HybridDecodeBlock(batch=B, heads=H, head_dim=D, capacity=256, chunk_size=64, top_k=2,
                                mlp_ratio=mlp_ratio, device=DEV, seed=31, fused=fused) for _ in range(2)]
    g = torch.Generator().manual_seed(32)
    k0 = torch.randn(B, H, S0, D, generator=g).to(BF).to(DEV)
    v0 = torch.randn(B, H, S0, D, generator=g).to(BF).to(DEV)
    h0 = torch.randn(B, H * D, generator=g).to(BF).to(DEV)
    for blk in blocks:
        blk.prefill(k0, v0)
    eager, graphed = blocks
    he = h0.clone()
    hg = h0.clone()
    replay, out = graphed.capture(hg, steps=G, feedback=True)
    assert out is hg
    for r in range(reps):
        for _ in range(G):
            eager(he, out=he)
        replay()
        assert torch.equal(hg, he), f"replay {r}"
    assert eager.length == graphed.length == S0 + G * reps
    assert torch.equal(graphed.k_cache, eager.k_cache) and torch.equal(graphed.summary_buf, eager.summary_buf)
