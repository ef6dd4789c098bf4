"""Pins of the CPU block restatements (oracle/block.py).

* mini_block against tests/golden/block_mini.npz, written by the reference's
  own MiniCSADecodeBlock (hybrid_attention/model_inference.py:14-76, torch-csa
  backend): bit-exact outputs and selected chunks, and a planted composition
  mistake (the GELU MLP fed the attention output instead of the block input)
  that the fixture rejects.
* baseline_block_steps (the BASELINE block; no reference implementation) by
  closed forms at special weights, computed independently in float64 numpy.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import block as OB

BF = torch.bfloat16


def _bf(bits):
    return torch.from_numpy(np.asarray(bits).view(np.int16)).view(BF)


@pytest.fixture(scope="module")
def fixture(golden_dir):
    return np.load(golden_dir / "block_mini.npz")


def _weights(z, tag):
    w = dict(w_q=_bf(z[f"{tag}_w_q"]), w_out=_bf(z[f"{tag}_w_out"]))
    if f"{tag}_w_up" in z:
        w.update(w_up=_bf(z[f"{tag}_w_up"]), w_down=_bf(z[f"{tag}_w_down"]))
    return w


@pytest.mark.parametrize("tag", ["mlp0", "mlp2"])
def test_mini_block_matches_the_reference_block_bit_for_bit(fixture, tag):
    z = fixture
    hidden, k, v = _bf(z["hidden"]), _bf(z["k"]), _bf(z["v"])
    out, sel = OB.mini_block(hidden, k=k, v=v, chunk=int(z["chunk_size"]), top_k=int(z["top_k"]), **_weights(z, tag))
    assert np.array_equal(sel, z[f"{tag}_selected"])
    assert torch.equal(out, _bf(z[f"{tag}_out"]))
    # with the reference's own selection handed in, the same output
    out2, _ = OB.mini_block(hidden, k=k, v=v, chunk=64, top_k=4, selected=z[f"{tag}_selected"], **_weights(z, tag))
    assert torch.equal(out2, out)


def test_fixture_rejects_a_misplaced_mlp(fixture):
    """The MLP applied to the attention output instead of the block input
    changes the zero-input features by far more than bf16 rounding."""
    z = fixture
    hidden, k, v = _bf(z["hidden"]), _bf(z["k"]), _bf(z["v"])
    w = _weights(z, "mlp2")
    q = F.linear(hidden, w["w_q"]).view(2, 2, 64)
    attn = torch.from_numpy(oracle.csa_attend(q, k, v, z["mlp2_selected"], 64, prob_dtype=oracle.BF16)).float().to(BF)
    a = F.linear(attn.reshape(2, 128), w["w_out"])
    wrong = hidden + 0.01 * (a + F.linear(F.gelu(F.linear(attn.reshape(2, 128), w["w_up"])), w["w_down"]))
    ref = _bf(z["mlp2_out"]).float()
    odd = (wrong.float() - ref)[:, 1::2].abs()
    assert odd.max() > 0.2 * ref[:, 1::2].abs().max()


def _rms64(x, w, eps=1e-6):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def _bf_round(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(BF)


def _cache(B, H, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, H, S, D, generator=g).to(BF), torch.randn(B, H, S, D, generator=g).to(BF))


def test_baseline_block_attention_is_the_value_mean_at_zero_qkv():
    """Zero QKV weights: q = 0 scores every chunk 0, so the lowest k chunk ids
    win, every token weighs the same and the attention is the mean of their
    value rows; the appended token (K = V = 0) sits past them."""
    B, H, D, chunk, k, S0 = 2, 2, 16, 8, 2, 40
    k0, v0 = _cache(B, H, S0, D, 1)
    g = torch.Generator().manual_seed(2)
    w = dict(w_qkv=torch.zeros(3 * H * D, H * D, dtype=BF), w_out=(torch.randn(H * D, H * D, generator=g) * 0.2).to(BF),
             norm1=torch.ones(H * D, dtype=BF), norm2=torch.ones(H * D, dtype=BF))
    hidden = torch.zeros(B, H * D, dtype=BF)
    outs = OB.baseline_block_steps(w, k0, v0, [hidden, hidden], heads=H, head_dim=D, chunk=chunk, top_k=k)
    attn = v0[:, :, : k * chunk].double().mean(dim=2).numpy().reshape(B, H * D)
    want = attn @ w["w_out"].double().numpy().T
    for out in outs:
        np.testing.assert_allclose(out.double().numpy(), want, rtol=2e-2, atol=2e-2 * np.abs(want).max())


def test_baseline_block_mlp_is_silu_over_the_normed_residual():
    """Zero out-projection: h = hidden, and the step adds W_down silu(W_up
    rms_norm(hidden) * norm2) -- SiLU, after the second norm, onto the residual."""
    B, H, D, chunk, k, S0 = 1, 2, 16, 8, 2, 31
    k0, v0 = _cache(B, H, S0, D, 3)
    g = torch.Generator().manual_seed(4)
    HD, M = H * D, 2 * H * D
    w = dict(w_qkv=(torch.randn(3 * HD, HD, generator=g) * 0.1).to(BF), w_out=torch.zeros(HD, HD, dtype=BF),
             norm1=torch.ones(HD, dtype=BF), norm2=(1 + 0.5 * torch.randn(HD, generator=g)).to(BF),
             w_up=(torch.randn(M, HD, generator=g) * 0.3).to(BF), w_down=(torch.randn(HD, M, generator=g) * 0.3).to(BF))
    hidden = torch.randn(B, HD, generator=g).to(BF)
    (out,) = OB.baseline_block_steps(w, k0, v0, [hidden], heads=H, head_dim=D, chunk=chunk, top_k=k)
    up = _rms64(hidden.double().numpy(), w["norm2"].double().numpy()) @ w["w_up"].double().numpy().T
    delta = (up / (1 + np.exp(-up))) @ w["w_down"].double().numpy().T
    got = out.double().numpy() - hidden.double().numpy()
    np.testing.assert_allclose(got, delta, rtol=3e-2, atol=3e-2 * np.abs(delta).max())
    gelu = (0.5 * up * (1 + np.tanh(0.7978845608 * (up + 0.044715 * up ** 3)))) @ w["w_down"].double().numpy().T
    assert np.abs(gelu - delta).max() > 2 * 3e-2 * np.abs(delta).max()  # the tolerance tells SiLU from GELU


def test_baseline_block_appends_before_attending():
    """Only the V block of W_qkv is non-zero (identity), so q = 0 and the new
    token's value row is rms_norm(hidden) * norm1.  With S0 + 1 = k * chunk the
    new token completes chunk k - 1, which the tie selection includes, so the
    attention is the mean over k * chunk rows with that row among them."""
    B, H, D, chunk, k = 1, 2, 16, 8, 3
    S0 = k * chunk - 1
    HD = H * D
    k0, v0 = _cache(B, H, S0, D, 5)
    g = torch.Generator().manual_seed(6)
    w_qkv = torch.zeros(3 * HD, HD)
    w_qkv[2 * HD:] = torch.eye(HD)
    w = dict(w_qkv=w_qkv.to(BF), w_out=torch.eye(HD, dtype=BF), norm1=(1 + 0.5 * torch.randn(HD, generator=g)).to(BF),
             norm2=torch.ones(HD, dtype=BF))
    hidden = torch.randn(B, HD, generator=g).to(BF)
    (out,) = OB.baseline_block_steps(w, k0, v0, [hidden], heads=H, head_dim=D, chunk=chunk, top_k=k)
    v_new = _bf_round(_rms64(hidden.double().numpy(), w["norm1"].double().numpy())).double().numpy()
    attn = (v0.double().numpy().sum(axis=2).reshape(B, HD) + v_new) / (k * chunk)
    want = hidden.double().numpy() + attn
    np.testing.assert_allclose(out.double().numpy(), want, rtol=1e-2, atol=1e-2)
    # without the appended row the mean would differ by v_new / (k * chunk)
    assert np.abs(v_new / (k * chunk)).max() > 5e-2
