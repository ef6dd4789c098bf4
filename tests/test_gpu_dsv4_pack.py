"""GPU quantize-on-write (pack_dsv4_cache, hybrid_attention/dsv4_correctness.py:24-59):
bytes must equal the reference rule bit for bit -- against the golden fixture the
reference's own pack wrote, and against the oracle's C restatement (itself pinned
to those fixtures and to torch's float8_e4m3fn cast)."""
import math

import numpy as np
import pytest
import torch

import oracle
from csahca_amd import dsv4_layout, native

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    native.lib()


def bits_to_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def test_golden_edge_tokens(golden_dir):
    g = np.load(golden_dir / "dsv4_pack_edges.npz")
    tok = bits_to_bf16(g["k_tokens"]).to(DEV)
    got = native.dsv4_pack_tokens(tok, int(g["page_size"]))
    assert np.array_equal(got.cpu().numpy(), g["cache"])


def varied_tokens(T, seed):
    """bf16 tokens whose 64-value tiles span zero, tiny, ordinary and huge magnitudes."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(T, 512, generator=gen)
    tile_scale = torch.pow(2.0, torch.randint(-60, 60, (T, 8), generator=gen).float())
    x[:, :448] *= tile_scale[:, :7].repeat_interleave(64, dim=1)
    x[0, :64] = 0.0                       # all-zero tile: max_abs clamps to 1e-8
    x[1, 64:128] = 448.0 * 2.0 ** -3      # max_abs / 448 exactly a power of two
    x[1, 128:192] = torch.linspace(-896.0, 896.0, 64)
    x[2, :448] = 1e-30                    # far below one quantum
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("page_size", [1, 16, 64, 256])
def test_pack_matches_oracle_bit_exact(page_size):
    tok = varied_tokens(300, seed=page_size)
    want = oracle.pack_dsv4_cache(tok, page_size=page_size)
    got = native.dsv4_pack_tokens(tok.to(DEV), page_size)
    assert got.shape == want.shape
    diff = np.flatnonzero(got.cpu().numpy().ravel() != np.asarray(want).ravel())
    assert diff.size == 0, f"{diff.size} bytes differ, first at {diff[:8]}"


def test_every_bf16_value_in_range_converts_like_the_oracle():
    """Each 64-value tile holds 448 (so max_abs / 448 = 1, E = 0 and the values
    are stored unscaled) and 63 of the finite bf16 values with |v| <= 448 --
    all of them over the tokens, subnormals and both zeros included: every
    value the e4m3 conversion can meet, bit-exact against the oracle."""
    vals = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 448.0)]
    ntiles = -(-vals.size // 63)
    tiles = np.zeros((ntiles, 64), dtype=np.float32)
    tiles[:, 0] = 448.0
    body = np.zeros(ntiles * 63, dtype=np.float32)
    body[:vals.size] = vals
    tiles[:, 1:] = body.reshape(ntiles, 63)
    T = -(-ntiles // 7)
    nope = np.zeros((T * 7, 64), dtype=np.float32)
    nope[:ntiles] = tiles
    x = np.zeros((T, 512), dtype=np.float32)
    x[:, :448] = nope.reshape(T, 448)
    x[:, 448:] = np.random.default_rng(5).standard_normal((T, 64))
    tok = torch.from_numpy(x).to(torch.bfloat16)
    assert np.array_equal(tok[:, :448].float().numpy(), x[:, :448])  # the values are exact bf16
    want = oracle.pack_dsv4_cache(tok, page_size=64)
    got = native.dsv4_pack_tokens(tok.to(DEV), 64)
    assert np.array_equal(got.cpu().numpy(), np.asarray(want))


def test_power_of_two_boundaries_and_rounding_ties():
    # tiles whose max is 448 * 2^k exactly (E = k), one ulp above (E = k + 1), and
    # values on e4m3 rounding ties
    rows = []
    for k in (-8, -1, 0, 1, 5):
        base = 448.0 * 2.0 ** k
        rows.append(torch.full((512,), base))
        rows.append(torch.full((512,), float(torch.tensor(base, dtype=torch.bfloat16).float()) * (1 + 2 ** -7)))
    ties = torch.tensor([1.0625, 1.1875, 3.25, 0.0029296875, -0.0009765625, 17.0, 18.0, 448.0] * 64)
    rows.append(ties)
    tok = torch.stack(rows).to(torch.bfloat16)
    want = oracle.pack_dsv4_cache(tok, page_size=4)
    got = native.dsv4_pack_tokens(tok.to(DEV), 4)
    assert np.array_equal(got.cpu().numpy(), np.asarray(want))


def test_scattered_writes_through_locations():
    ps, pages = 64, 12
    bpp = dsv4_layout.bytes_per_page(ps)
    tok = varied_tokens(200, seed=7)
    perm = torch.randperm(pages * ps, generator=torch.Generator().manual_seed(1))[:200].to(torch.int32)
    locs = perm.clone()
    locs[5] = -1          # skipped
    locs[6] = pages * ps  # page past the cache: skipped
    cache = torch.zeros(pages, bpp, dtype=torch.uint8, device=DEV)
    native.dsv4_pack_tokens(tok.to(DEV), ps, cache=cache, locs=locs.to(DEV))
    got = cache.cpu().numpy()
    # reference bytes of each written token: pack it alone at its in-page row
    for t in range(200):
        loc = int(locs[t])
        if loc < 0 or loc >= pages * ps:
            continue
        page, row = divmod(loc, ps)
        single = np.asarray(oracle.pack_dsv4_cache(tok[t:t + 1].repeat(ps, 1), page_size=ps))[0]
        r0 = row * 576
        assert np.array_equal(got[page, r0:r0 + 576], single[r0:r0 + 576]), t
        s0 = ps * 576 + row * 8
        assert np.array_equal(got[page, s0:s0 + 7], single[s0:s0 + 7]), t
    # skipped tokens wrote nothing: their own rows are still zero unless another token owns them
    owned = {int(l) for l in locs.tolist() if 0 <= l < pages * ps}
    for loc in (int(perm[5]), int(perm[6]) if int(perm[6]) < pages * ps else None):
        if loc is not None and loc not in owned:
            page, row = divmod(loc, ps)
            assert not got[page, row * 576:(row + 1) * 576].any()


def test_gpu_pack_then_decode_matches_oracle_pipeline():
    ps, T, nq, H = 64, 512, 3, 16
    tok = varied_tokens(T, seed=3)
    tok[:, :448] = torch.randn(T, 448, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    cache = native.dsv4_pack_tokens(tok.to(DEV), ps)
    gen = torch.Generator().manual_seed(4)
    q = torch.randn(nq, H, 512, generator=gen).to(torch.bfloat16)
    idx = torch.randint(0, T, (nq, 96), generator=gen, dtype=torch.int32)
    lens = torch.tensor([96, 50, 1], dtype=torch.int32)
    sink = torch.randn(H, generator=gen)
    scale = 1.0 / math.sqrt(512)
    got = native.dsv4_swa_decode_forward(q.to(DEV), cache, idx.to(DEV), lens.to(DEV), sink.to(DEV), ps, scale)
    want = oracle.dsv4_reference_attention(q, oracle.pack_dsv4_cache(tok, page_size=ps), idx, lens, sink,
                                           page_size=ps, softmax_scale=scale)
    g = got.float().cpu().numpy().astype(np.float64)
    assert np.all(np.abs(g - want) <= 5e-2 + 5e-2 * np.abs(want))
