"""GPU parity of the decode-step products (csahca_block_linear,
csahca_block_qkv) against a float64 CPU restatement that rounds to the storage
type exactly where the torch ops they replace round: the RMSNorm output, the
F.linear output, F.silu / F.gelu of the rounded product, the residual add, and
`hidden + 0.01 * out`.

Tolerance (the parity bar of this path): |got - ref| <= 2e-2 + 1e-2 |ref|.
"""
import numpy as np
import pytest
import torch

from csahca_amd import native

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    native.lib()


def assert_close(got, ref, what=""):
    g = got.detach().double().cpu().numpy()
    r = ref.detach().double().cpu().numpy()
    assert g.shape == r.shape, (g.shape, r.shape)
    diff = np.abs(g - r)
    bad = diff > 2e-2 + 1e-2 * np.abs(r)
    assert not bad.any(), f"{what} max_abs={diff.max():.3e} bad={int(bad.sum())}/{bad.size}"


def ref_linear(x, w, dtype, *, norm=None, eps=1e-6, residual=None, act=None, base=None, alpha=1.0):
    xf = x.double()
    if norm is not None:
        xf = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * norm.double()).to(dtype).double()
    y = (xf @ w.double().T).to(dtype).double()
    if act == "silu":
        y = (y * torch.sigmoid(y)).to(dtype).double()
    if act == "gelu":
        y = (0.5 * y * (1.0 + torch.erf(y / 2.0 ** 0.5))).to(dtype).double()
    if residual is not None:
        y = (y + residual.double()).to(dtype).double()
    if base is not None:
        y = (base.double() + (alpha * y).to(dtype).double()).to(dtype).double()
    return y


def operands(B, N, K, dtype, seed, norm, residual):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, K, generator=g).to(dtype)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype)
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).to(dtype) if norm else None
    res = torch.randn(B, N, generator=g).to(dtype) if residual else None
    return x, w, nw, res


CASES = [
    # B, N, K, dtype, norm, residual, act
    (1, 3072, 1024, torch.bfloat16, True, False, None),   # the block's QKV shape
    (1, 1024, 1024, torch.bfloat16, False, True, None),   # out projection + residual
    (1, 2048, 1024, torch.bfloat16, True, False, "silu"),  # RMSNorm + up projection + SiLU
    (1, 1024, 2048, torch.bfloat16, False, True, None),   # down projection + residual
    (3, 1000, 520, torch.float16, True, False, None),     # ragged K (65 chunks of 8), N not a multiple of 8
    (4, 7, 8, torch.bfloat16, False, False, "silu"),      # one 16-byte chunk per row, 4 rows
    (1, 64, 4096, torch.bfloat16, True, True, None),      # widest K (8 loads per lane per row)
    (2, 130, 2048, torch.float16, False, True, None),     # widest K with batch > 1
    (1, 2048, 1024, torch.bfloat16, False, False, "gelu"),  # the mini block's up projection
    (3, 96, 256, torch.float16, True, True, "gelu"),      # activation, then residual
]


@pytest.mark.parametrize("B,N,K,dtype,norm,residual,act", CASES)
def test_block_linear_matches_rounded_reference(B, N, K, dtype, norm, residual, act):
    x, w, nw, res = operands(B, N, K, dtype, seed=N + K + B, norm=norm, residual=residual)
    ref = ref_linear(x, w, dtype, norm=nw, residual=res, act=act)
    got = native.block_linear(x.to(DEV), w.to(DEV), norm_weight=None if nw is None else nw.to(DEV),
                              residual=None if res is None else res.to(DEV), activation=act)
    assert got.dtype == dtype
    assert_close(got, ref, f"B{B} N{N} K{K} {dtype} norm={norm} res={residual} act={act}")


@pytest.mark.parametrize("mlp", [False, True])
def test_block_linear_scaled_base_matches_the_mini_block_tail(mlp):
    """`hidden + 0.01 * (out [+ mlp])` (model_inference.py:70-76) as the epilogue
    of the last product."""
    dtype = torch.bfloat16
    x, w, _, out = operands(1, 1024, 2048 if mlp else 1024, dtype, seed=5, norm=False, residual=True)
    hidden = torch.randn(1, 1024, generator=torch.Generator().manual_seed(6)).to(dtype)
    ref = ref_linear(x, w, dtype, residual=out if mlp else None, base=hidden, alpha=0.01)
    got = native.block_linear(x.to(DEV), w.to(DEV), residual=out.to(DEV) if mlp else None, base=hidden.to(DEV),
                              alpha=0.01)
    assert_close(got, ref, f"mlp={mlp}")


def test_block_linear_rows_are_independent_of_batch():
    """Row b of a batch-4 product equals the batch-1 product of that row (the
    4-row kernel and the 1-row kernel agree bit for bit)."""
    x, w, nw, _ = operands(4, 300, 1024, torch.bfloat16, seed=3, norm=True, residual=False)
    x, w, nw = x.to(DEV), w.to(DEV), nw.to(DEV)
    full = native.block_linear(x, w, norm_weight=nw)
    for b in range(4):
        one = native.block_linear(x[b:b + 1].contiguous(), w, norm_weight=nw)
        assert torch.equal(one[0], full[b]), b


def test_block_linear_advances_the_position_once_per_call():
    x, w, _, res = operands(1, 256, 512, torch.bfloat16, seed=4, norm=False, residual=True)
    x, w, res = x.to(DEV), w.to(DEV), res.to(DEV)
    pos = torch.tensor([41], dtype=torch.int64, device=DEV)
    plain = native.block_linear(x, w, residual=res)
    for i in range(3):
        got = native.block_linear(x, w, residual=res, advance_pos=pos)
        assert torch.equal(got, plain)
    assert int(pos.item()) == 44


def test_block_qkv_scatters_q_and_appends_kv_at_the_device_position():
    B, H, D, cap, chunk = 2, 4, 64, 300, 64
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(6)
    hidden = torch.randn(B, H * D, generator=g).to(dtype)
    w = (0.02 * torch.randn(3 * H * D, H * D, generator=g)).to(dtype)
    nw = (1.0 + 0.1 * torch.randn(H * D, generator=g)).to(dtype)
    ref = ref_linear(hidden, w, dtype, norm=nw).view(B, 3, H, D)
    k0 = torch.randn(B, H, cap, D, generator=g).to(dtype).to(DEV)
    v0 = torch.randn(B, H, cap, D, generator=g).to(dtype).to(DEV)
    for p in (0, 127, 299):
        kc, vc = k0.clone(), v0.clone()
        q = torch.empty(B, H, D, dtype=dtype, device=DEV)
        pos = torch.tensor([p], dtype=torch.int64, device=DEV)
        nch = torch.full((1,), -7, dtype=torch.int32, device=DEV)
        native.block_qkv(hidden.to(DEV), w.to(DEV), q, kc, vc, pos, norm_weight=nw.to(DEV), num_chunks=nch,
                         chunk_size=chunk)
        assert_close(q, ref[:, 0], f"q at {p}")
        assert_close(kc[:, :, p], ref[:, 1], f"k at {p}")
        assert_close(vc[:, :, p], ref[:, 2], f"v at {p}")
        others = torch.ones(cap, dtype=torch.bool)
        others[p] = False
        assert torch.equal(kc[:, :, others], k0[:, :, others]) and torch.equal(vc[:, :, others], v0[:, :, others])
        assert int(nch.item()) == (p + 1) // chunk
        assert int(pos.item()) == p  # read, not advanced


def test_block_qkv_position_outside_the_cache_writes_no_kv():
    B, H, D, cap = 1, 2, 64, 96
    dtype = torch.float16
    g = torch.Generator().manual_seed(8)
    hidden = torch.randn(B, H * D, generator=g).to(dtype).to(DEV)
    w = (0.02 * torch.randn(3 * H * D, H * D, generator=g)).to(dtype).to(DEV)
    kc = torch.randn(B, H, cap, D, generator=g).to(dtype).to(DEV)
    vc = torch.randn(B, H, cap, D, generator=g).to(dtype).to(DEV)
    k0, v0 = kc.clone(), vc.clone()
    q = torch.zeros(B, H, D, dtype=dtype, device=DEV)
    for p in (cap, -1):
        native.block_qkv(hidden, w, q, kc, vc, torch.tensor([p], dtype=torch.int64, device=DEV), chunk_size=32)
        assert torch.equal(kc, k0) and torch.equal(vc, v0)
    ref = ref_linear(hidden.cpu(), w.cpu(), dtype).view(B, 3, H, D)
    assert_close(q, ref[:, 0], "q")


def test_block_linear_output_may_alias_residual_but_not_x():
    x, w, _, res = operands(2, 256, 256, torch.bfloat16, seed=9, norm=False, residual=True)
    x, w, res = x.to(DEV), w.to(DEV), res.to(DEV)
    want = native.block_linear(x, w, residual=res)
    buf = res.clone()
    got = native.block_linear(x, w, residual=buf, out=buf)
    assert got.data_ptr() == buf.data_ptr() and torch.equal(buf, want)
    with pytest.raises(RuntimeError, match="must not overlap x"):
        native.block_linear(x, w, out=x)
