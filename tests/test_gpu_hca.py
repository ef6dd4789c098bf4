"""GPU parity of HCA (hca_reference, hybrid_attention/reference.py:87-92) and the
CSA/HCA hybrid blend (hybrid_reference, reference.py:95-108) against the CPU
oracle and the golden vectors.

Tolerance (the parity bar of this path): |got - ref| <= 2e-2 + 1e-2 |ref| for 16-bit
storage, 1e-4 + 1e-4 |ref| for fp32/fp64 storage.
"""
import numpy as np
import pytest
import torch

import oracle
from csahca_amd import extension, native
from csahca_amd.synthetic import make_synthetic_case

pytestmark = pytest.mark.gpu

DEV = "cuda"
CODE = {torch.bfloat16: oracle.BF16, torch.float16: oracle.F16, torch.float32: oracle.F32,
        torch.float64: oracle.F64}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    native.lib()


def tol_for(dtype):
    return (2e-2, 1e-2) if dtype in (torch.bfloat16, torch.float16) else (1e-4, 1e-4)


def assert_close(got, ref, dtype, what=""):
    atol, rtol = tol_for(dtype)
    g = got.detach().double().cpu().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    assert g.shape == ref.shape, (g.shape, ref.shape)
    diff = np.abs(g - ref)
    bad = diff > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{what} max_abs={diff.max():.3e} bad={int(bad.sum())}/{bad.size}"


def inputs(B, H, S, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, S, D, generator=g).to(dtype)
    v = torch.randn(B, H, S, D, generator=g).to(dtype)
    return q, k, v


def test_golden_small_fixture(golden_dir):
    """The correctness.py default case: hca_out and hybrid_out written by the
    reference's own functions."""
    g = np.load(golden_dir / "csa_small.npz")
    to_t = lambda bits: torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    q, k, v = to_t(g["q"]), to_t(g["k"]), to_t(g["v"])
    chunk = int(g["hca_chunk"])
    hca = native.hca_decode_forward(q, k, v, chunk)
    assert_close(hca, oracle.bf16_bits_to_f32(g["hca_out"]), torch.bfloat16, "hca")
    hyb = native.hybrid_decode_forward(q, k, v, csa_chunk_size=int(g["chunk_size"]), csa_top_k=int(g["top_k"]),
                                       hca_chunk_size=chunk)
    assert_close(hyb, oracle.bf16_bits_to_f32(g["hybrid_out"]), torch.bfloat16, "hybrid")


HCA_CASES = [
    # B, H, S, D, chunk, dtype
    (1, 8, 32768, 128, 256, torch.bfloat16),  # reference benchmark hca_chunk 256 at the target context
    (2, 4, 4096, 64, 64, torch.float16),
    (1, 2, 1024, 128, 64, torch.float32),
    (1, 1, 512, 256, 128, torch.bfloat16),
    (2, 3, 640, 96, 64, torch.bfloat16),     # D/8 = 12 vector columns
    (1, 2, 384, 100, 32, torch.float32),     # D/4 = 25 vector columns
    (1, 2, 256, 99, 16, torch.bfloat16),     # D not a multiple of 8: scalar columns
    (1, 2, 96, 64, 1, torch.bfloat16),       # chunk 1: full attention over every token
    (1, 1, 128, 1024, 64, torch.float64),    # largest head_dim; f64 storage
    (1, 1, 8192, 128, 8192, torch.bfloat16), # one chunk: output = mean of V
    (1, 2, 32768, 64, 64, torch.bfloat16),   # C = 512: merge rows in batches (C > 256)
    (1, 1, 16384, 40, 4, torch.float16),     # C = 4096: two probability passes of 2048 rows
]


@pytest.mark.parametrize("B,H,S,D,chunk,dtype", HCA_CASES)
def test_hca_matches_oracle(B, H, S, D, chunk, dtype):
    q, k, v = inputs(B, H, S, D, dtype, seed=S + D + chunk)
    ref = oracle.hca_reference(q, k, v, chunk_size=chunk, dtype=CODE[dtype])
    got = native.hca_decode_forward(q.to(DEV), k.to(DEV), v.to(DEV), chunk)
    assert_close(got, ref, dtype, f"hca B{B} H{H} S{S} D{D} chunk{chunk} {dtype}")


def test_hca_single_chunk_is_rounded_mean_of_v():
    q, k, v = inputs(1, 2, 256, 128, torch.bfloat16, seed=3)
    got = native.hca_decode_forward(q.to(DEV), k.to(DEV), v.to(DEV), 256)
    mean_v = v.float().mean(dim=2).to(torch.bfloat16).float()  # one summary row, probability 1
    # equal, or one bf16 ulp apart where the fp32 summation order moves the mean across a rounding boundary
    assert torch.all((got.cpu().float() - mean_v).abs() <= mean_v.abs() * 2.0 ** -8 + 1e-30)


def test_hybrid_matches_oracle_blend():
    case = make_synthetic_case(batch=1, heads=8, seq_len=8192, head_dim=128, chunk_size=64, top_k=8, seed=1)
    q, k, v = case.q, case.k_cache, case.v_cache
    got = native.hybrid_decode_forward(q.to(DEV), k.to(DEV), v.to(DEV), csa_chunk_size=64, csa_top_k=8,
                                       hca_chunk_size=256)
    bf = torch.bfloat16
    csa = oracle.round_to(oracle.csa_reference(q, k, v, chunk_size=64, top_k=8, dtype=bf), bf)
    hca = oracle.round_to(oracle.hca_reference(q, k, v, chunk_size=256, dtype=oracle.BF16), bf)
    want = oracle.round_to(oracle.round_to(0.7 * csa, bf) + oracle.round_to(0.3 * hca, bf), bf)
    assert_close(got, want, bf, "hybrid")


def test_hybrid_weight_one_is_csa_and_zero_is_hca():
    q, k, v = (t.to(DEV) for t in inputs(1, 4, 2048, 128, torch.bfloat16, seed=7))
    summ = native.csa_chunk_summary(k, 64)
    csa, _ = native.csa_decode_step(q, k, v, summ, 64, 4)
    hca = native.hca_decode_forward(q, k, v, 128)
    assert torch.equal(native.hybrid_decode_forward(q, k, v, csa_chunk_size=64, csa_top_k=4, hca_chunk_size=128,
                                                    csa_weight=1.0, summary=summ), csa)
    assert torch.equal(native.hybrid_decode_forward(q, k, v, csa_chunk_size=64, csa_top_k=4, hca_chunk_size=128,
                                                    csa_weight=0.0, summary=summ), hca)


@pytest.mark.parametrize("B,H,S,D,dtype,top_k", [
    (1, 8, 8192, 128, torch.bfloat16, 8),    # one launch: step blocks + HCA chunk blocks
    (1, 8, 32768, 128, torch.bfloat16, 8),   # the headline shape
    (4, 8, 8192, 128, torch.bfloat16, 32),   # 32 heads, top-32
    (1, 2, 65536, 128, torch.bfloat16, 8),   # 1024 summary rows (the 32-keys-per-lane top-k)
    (1, 3, 4352, 128, torch.float16, 8),     # one launch, 51 chunk items: the last HCA block takes one
    (1, 2, 4096, 128, torch.float32, 8),     # fp32: the two ops in turn
    (1, 4, 4096, 64, torch.bfloat16, 8),     # head_dim 64: the two ops in turn
])
def test_hybrid_equals_the_two_ops_in_turn(B, H, S, D, dtype, top_k):
    """csahca_hybrid_decode_forward gives exactly the bits of the CSA decode
    step followed by the blended HCA op, fused into one launch or not."""
    q, k, v = (t.to(DEV) for t in inputs(B, H, S, D, dtype, seed=B * 17 + H + D))
    summ = native.csa_chunk_summary(k, 64)
    csa, _ = native.csa_decode_step(q, k, v, summ, 64, top_k)
    hc = 256 if S % 256 == 0 else 128
    want = native.hca_decode_forward(q, k, v, hc, blend=csa, csa_weight=0.7)
    got = native.hybrid_decode_forward(q, k, v, csa_chunk_size=64, csa_top_k=top_k, hca_chunk_size=hc,
                                       summary=summ)
    assert torch.equal(got, want)
    assert all(x == 0 for x in native.csa_step_status().values())


def test_hybrid_graph_replays_match_eager():
    """The hybrid launch captured in a HIP graph: every replay (with eager work
    and synchronisations between replays) equals the eager result."""
    q, k, v = (t.to(DEV) for t in inputs(1, 8, 8192, 128, torch.bfloat16, seed=13))
    summ = native.csa_chunk_summary(k, 64)

    def run():
        return native.hybrid_decode_forward(q, k, v, csa_chunk_size=64, csa_top_k=8, hca_chunk_size=256,
                                            summary=summ)

    want = run()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()  # creates s's step workspace for this shape
    assert native.step_workspace_ready(DEV, s.cuda_stream, (8, 128, 128, 8, 64))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        got = run()
    for i in range(5):
        with torch.cuda.stream(s):
            got.zero_()
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), i
        with torch.cuda.stream(s):  # eager work on the capture stream, same workspace
            again = run()
        torch.cuda.synchronize()
        assert torch.equal(again, want), i
    assert all(x == 0 for x in native.csa_step_status().values())


def test_hca_rejects_ragged_sequence_with_reference_message():
    q, k, v = (t.to(DEV) for t in inputs(1, 1, 100, 64, torch.bfloat16, seed=0))
    with pytest.raises(RuntimeError, match="seq length must be divisible by chunk_size"):
        native.hca_decode_forward(q, k, v, 64)


def test_extension_wrappers_route_to_native():
    q, k, v = (t.to(DEV) for t in inputs(1, 2, 512, 64, torch.bfloat16, seed=5))
    assert torch.equal(extension.hca_decode_forward(q, k, v, 64), native.hca_decode_forward(q, k, v, 64))
