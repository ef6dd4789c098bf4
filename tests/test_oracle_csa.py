"""Pin the CSA oracle (oracle/csahca_oracle.c) against the reference's golden
vectors, closed forms and planted-chunk known answers.

Golden vectors were written by the reference's own functions
(tests/golden/make_golden.py); everything else is fixed by mathematics, so a
dropped scale, a wrong slot/offset index, a transposed operand or a skipped
probability cast fails at least one test below.
"""
import hashlib
import math

import numpy as np
import pytest
import torch

import oracle
from csahca_amd.synthetic import clustered_chunks, make_synthetic_case, plant_chunks, scattered_chunks


def bf16(bits):
    return oracle.bf16_bits_to_f32(bits)


def to_bf16_bits(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def sha(t):
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


@pytest.fixture(scope="module")
def small(golden_dir):
    return np.load(golden_dir / "csa_small.npz")


def test_chunk_mean_golden(small):
    k = bf16(small["k"])
    got = oracle.chunk_mean(k, 64)
    want = small["chunk_mean"]
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-7)


def test_select_topk_golden(small):
    q, k = bf16(small["q"]), bf16(small["k"])
    idx, scores = oracle.select_topk(q, oracle.chunk_mean(k, 64), 4)
    assert np.array_equal(idx, small["selected"])
    # the golden selection is not decided by a near tie
    for bh in range(scores.shape[1]):
        s = np.sort(scores[0, bh])[::-1]
        assert s[3] - s[4] > 1e-4


def test_csa_reference_golden(small):
    q, k, v = bf16(small["q"]), bf16(small["k"]), bf16(small["v"])
    out = oracle.csa_reference(q, k, v, chunk_size=64, top_k=4, selected_chunks=small["selected"],
                               dtype=torch.bfloat16)
    want = bf16(small["csa_out"])
    got = oracle.round_to(out, torch.bfloat16)
    # same bf16 value, or one bf16 ulp apart (fp32 vs double accumulation)
    ulp = np.abs(want) * 2.0 ** -7 + 1e-6
    assert np.all(np.abs(got - want) <= ulp), np.abs(got - want).max()
    # the probability cast matters: fp32 probabilities differ visibly at this tolerance
    out32 = oracle.csa_attend(q, k, v, small["selected"], 64, prob_dtype=oracle.F32)
    assert np.abs(out32 - want).max() > np.abs(out - want).max()


def test_full_hca_hybrid_golden(small):
    q, k, v = bf16(small["q"]), bf16(small["k"]), bf16(small["v"])
    full = oracle.full_decode_attention(q, k, v, prob_dtype=oracle.BF16)
    ulp = lambda w: np.abs(w) * 2.0 ** -7 + 1e-6
    w = bf16(small["full_out"])
    assert np.all(np.abs(oracle.round_to(full, torch.bfloat16) - w) <= ulp(w))
    hca = oracle.hca_reference(q, k, v, chunk_size=int(small["hca_chunk"]), dtype=oracle.BF16)
    w = bf16(small["hca_out"])
    assert np.all(np.abs(oracle.round_to(hca, torch.bfloat16) - w) <= ulp(w))
    # hybrid_reference = 0.7 * csa + 0.3 * hca, each term and the sum rounded to bf16
    csa = oracle.round_to(oracle.csa_reference(q, k, v, chunk_size=64, top_k=4, dtype=torch.bfloat16), torch.bfloat16)
    hb = oracle.round_to(oracle.round_to(0.7 * csa, torch.bfloat16) + oracle.round_to(0.3 * oracle.round_to(hca, torch.bfloat16), torch.bfloat16), torch.bfloat16)
    w = bf16(small["hybrid_out"])
    assert np.all(np.abs(hb - w) <= 2 * ulp(w))


def test_default_case_regenerates_and_matches(golden_dir):
    g = np.load(golden_dir / "csa_default.npz")
    case = make_synthetic_case(batch=1, heads=2, seq_len=1024, head_dim=128, chunk_size=64, top_k=4, seed=0)
    assert sha(case.q) == str(g["sha_q"]) and sha(case.k_cache) == str(g["sha_k"]) and sha(case.v_cache) == str(g["sha_v"])
    summ = oracle.chunk_mean(case.k_cache, 64)
    np.testing.assert_allclose(summ, g["chunk_mean"], rtol=0, atol=2e-7)
    idx, _ = oracle.select_topk(case.q, summ, 4)
    assert np.array_equal(idx, g["selected"])
    out = oracle.round_to(oracle.csa_reference(case.q, case.k_cache, case.v_cache, chunk_size=64, top_k=4,
                                               selected_chunks=idx, dtype=torch.bfloat16), torch.bfloat16)
    want = bf16(g["csa_out"])
    assert np.all(np.abs(out - want) <= np.abs(want) * 2.0 ** -7 + 1e-6)


def test_tie_break_declared_order(golden_dir):
    q = np.ones((1, 1, 64), np.float32)
    k = np.ones((1, 1, 64 * 16, 64), np.float32)
    idx, scores = oracle.select_topk(q, oracle.chunk_mean(k, 64), 5)
    assert np.all(scores == scores[0, 0, 0])
    assert idx.tolist() == [[[0, 1, 2, 3, 4]]]
    # torch's order on the same ties is implementation-defined (recorded for the
    # record only): five distinct chunk ids, not necessarily the lowest ones
    t = np.load(golden_dir / "csa_ties.npz")["torch_topk_order"].ravel().tolist()
    assert len(set(t)) == 5 and all(0 <= c < 16 for c in t)


@pytest.mark.parametrize("kind", ["scattered", "clustered"])
def test_planted_chunks_known_answer(kind):
    B, H, S, D, chunk, k = 2, 3, 4096, 128, 64, 8
    C = S // chunk
    case = make_synthetic_case(batch=B, heads=H, seq_len=S, head_dim=D, chunk_size=chunk, top_k=k, seed=3)
    ids = scattered_chunks(B, H, C, k) if kind == "scattered" else clustered_chunks(B, H, C, k)
    kp = plant_chunks(case.q, case.k_cache, ids, chunk, alpha=1.0)
    idx = oracle.select_topk_chunks(case.q, kp, chunk, k)
    assert np.array_equal(idx, ids.numpy())


def test_top_k_clamped_to_num_chunks():
    case = make_synthetic_case(batch=1, heads=1, seq_len=256, head_dim=32, chunk_size=64, top_k=8, seed=1)
    idx = oracle.select_topk_chunks(case.q, case.k_cache, 64, 8)
    assert idx.shape == (1, 1, 4)
    assert sorted(idx.ravel().tolist()) == [0, 1, 2, 3]


def test_closed_form_single_token_and_uniform():
    rng = np.random.default_rng(0)
    B, H, S, D, chunk = 1, 2, 256, 16, 4
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    k = rng.standard_normal((B, H, S, D)).astype(np.float32)
    v = rng.standard_normal((B, H, S, D)).astype(np.float32)
    # chunk 63 covers tokens 252..255; with seq 253 only token 252 is in range
    idx = np.array([[[-1, 63]], [[-1, 63]]], dtype=np.int64).reshape(B, H, 2)
    out = oracle.csa_attend(q, k[:, :, :253], v[:, :, :253], idx, chunk)
    np.testing.assert_allclose(out, v[:, :, 252], rtol=0, atol=1e-12)
    # identical keys -> uniform weights -> mean of the selected values
    ku = np.broadcast_to(k[:, :, :1], k.shape).copy()
    idx = np.array([[[5, 9, 2]], [[0, 1, 7]]], dtype=np.int64).reshape(B, H, 3)
    out = oracle.csa_attend(q, ku, v, idx, chunk)
    for h in range(H):
        toks = np.concatenate([np.arange(c * chunk, (c + 1) * chunk) for c in idx[0, h]])
        np.testing.assert_allclose(out[0, h], v[0, h, toks].astype(np.float64).mean(0), rtol=0, atol=1e-12)
    # all slots invalid -> zero output
    out = oracle.csa_attend(q, k, v, np.full((B, H, 2), -1, np.int64), chunk)
    assert np.all(out == 0)


def test_closed_form_two_tokens_scale():
    # two tokens whose scores differ by exactly d/sqrt(D): weight = sigmoid(d/sqrt(D))
    D = 64
    q = np.zeros((1, 1, D), np.float32); q[0, 0, 0] = 2.0
    k = np.zeros((1, 1, 2, D), np.float32); k[0, 0, 0, 0] = 1.5; k[0, 0, 1, 0] = -0.5
    v = np.zeros((1, 1, 2, D), np.float32); v[0, 0, 0, 1] = 1.0; v[0, 0, 1, 2] = 1.0
    out = oracle.csa_attend(q, k, v, np.array([[[0]]], np.int64), 2)
    p0 = 1.0 / (1.0 + math.exp(-(2.0 * 1.5 - 2.0 * -0.5) / math.sqrt(D)))
    assert out[0, 0, 1] == pytest.approx(p0, abs=1e-12)
    assert out[0, 0, 2] == pytest.approx(1 - p0, abs=1e-12)


def test_selection_covering_everything_is_full_attention(small):
    # k * chunk = S: torch-csa equals full_decode_attention (golden full_out)
    q, k, v = bf16(small["q"]), bf16(small["k"]), bf16(small["v"])
    idx = np.tile(np.arange(8, dtype=np.int64), (1, 2, 1))
    out = oracle.round_to(oracle.csa_attend(q, k, v, idx, 64, prob_dtype=oracle.BF16), torch.bfloat16)
    w = bf16(small["full_out"])
    assert np.all(np.abs(out - w) <= np.abs(w) * 2.0 ** -7 + 1e-6)


def test_slot_order_is_irrelevant():
    case = make_synthetic_case(batch=1, heads=2, seq_len=1024, head_dim=64, chunk_size=64, top_k=4, seed=5)
    idx = np.array([[[3, 7, 1, 12], [0, 15, 4, 9]]], np.int64)
    a = oracle.csa_attend(case.q, case.k_cache, case.v_cache, idx, 64)
    b = oracle.csa_attend(case.q, case.k_cache, case.v_cache, idx[..., ::-1].copy(), 64)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)


def test_torch_restatement_golden_and_oracle(small):
    """oracle/torch_csa.py (the CPU baseline's torch-ops restatement) reproduces
    the reference's golden selection and output, and the C oracle's step at a
    larger shape (ids exactly; outputs within one bf16 ulp)."""
    from oracle import torch_csa

    def t(bits):
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)

    q, k, v = t(small["q"]), t(small["k"]), t(small["v"])
    summ = torch.from_numpy(oracle.chunk_mean(bf16(small["k"]), 64).astype(np.float32))
    idx = torch_csa.select_topk(q, summ, 4)
    assert np.array_equal(idx.numpy(), small["selected"])
    out = torch_csa.attend(q, k, v, idx, 64).float().numpy()
    want = bf16(small["csa_out"])
    assert np.all(np.abs(out - want) <= np.abs(want) * 2.0 ** -7 + 1e-6)
    case = make_synthetic_case(batch=1, heads=4, seq_len=8192, head_dim=128, chunk_size=64, top_k=8, seed=5)
    summ = torch.from_numpy(oracle.chunk_mean(case.k_cache, 64).astype(np.float32))
    got = torch_csa.decode_step(case.q, case.k_cache, case.v_cache, summ, 64, 8).float().numpy()
    want_idx, _ = oracle.select_topk(case.q, summ.numpy(), 8)
    assert np.array_equal(torch_csa.select_topk(case.q, summ, 8).numpy(), want_idx)
    ref = oracle.round_to(oracle.csa_attend(case.q, case.k_cache, case.v_cache, want_idx, 64,
                                            prob_dtype=oracle.BF16), torch.bfloat16)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -7 + 1e-6), np.abs(got - ref).max()
