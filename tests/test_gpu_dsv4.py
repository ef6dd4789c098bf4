"""GPU parity of the DSV4 paged-FP8 decode against the CPU oracle and the
reference's golden vectors.  Tolerance for the FP8-cache modes (the parity bar
of this path): |got - ref| <= 5e-2 + 5e-2 |ref| for 16-bit queries; fp32 queries are
held to 1e-4 + 1e-4 |ref|."""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from csahca_amd import dsv4_layout, extension, native
from csahca_amd.synthetic import make_dsv4_case, make_dsv4_window_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = 1.0 / math.sqrt(512)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("no HIP device visible")
    native.lib()


def assert_close(got, ref, atol=5e-2, rtol=5e-2, what=""):
    g = got.detach().float().cpu().numpy().astype(np.float64)
    assert g.shape == ref.shape
    diff = np.abs(g - ref)
    bad = diff > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{what} max_abs={diff.max():.3e} bad={int(bad.sum())}/{bad.size}"


def oracle_out(c, sink=True, scale=SCALE, lengths=True):
    kw = {}
    if c.extra_cache is not None:
        kw = dict(extra_cache=c.extra_cache.cpu(), extra_token_indices=c.extra_token_indices.cpu(),
                  extra_topk_lengths=c.extra_topk_lengths.cpu() if lengths else None,
                  extra_page_size=c.extra_page_size)
    return oracle.dsv4_reference_attention(c.q.cpu(), c.cache.cpu(), c.token_indices.cpu(),
                                           c.topk_lengths.cpu() if lengths else None,
                                           c.attn_sink.cpu() if sink else None, page_size=c.page_size,
                                           softmax_scale=scale, **kw)


def gpu_out(c, sink=True, scale=SCALE, lengths=True):
    s = c.attn_sink.to(DEV) if sink else None
    if c.extra_cache is not None:
        return extension.dsv4_sparse_decode_forward(
            c.q.to(DEV), c.cache.to(DEV), c.token_indices.to(DEV), c.topk_lengths.to(DEV) if lengths else None,
            c.extra_cache.to(DEV), c.extra_token_indices.to(DEV),
            c.extra_topk_lengths.to(DEV) if lengths else None, s, c.page_size, c.extra_page_size, scale)
    return extension.dsv4_swa_decode_forward(c.q.to(DEV), c.cache.to(DEV), c.token_indices.to(DEV),
                                             c.topk_lengths.to(DEV) if lengths else None, s, c.page_size, scale)


@pytest.mark.parametrize("ratio", [0, 4, 128])
def test_golden_fixtures(golden_dir, ratio):
    g = np.load(golden_dir / f"dsv4_c{ratio}.npz")
    bf = lambda bits: torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    q = bf(g["q"])
    cache = torch.from_numpy(g["cache"]).to(DEV)
    idx = torch.from_numpy(g["token_indices"]).to(DEV)
    lens = torch.from_numpy(g["topk_lengths"]).to(DEV)
    sink = torch.from_numpy(g["attn_sink"]).to(DEV)
    ps = int(g["page_size"])
    for key, s in (("out", sink), ("out_nosink", None)):
        if ratio:
            out = extension.dsv4_sparse_decode_forward(
                q, cache, idx, lens, torch.from_numpy(g["extra_cache"]).to(DEV),
                torch.from_numpy(g["extra_token_indices"]).to(DEV),
                torch.from_numpy(g["extra_topk_lengths"]).to(DEV), s, ps, int(g["extra_page_size"]),
                float(g["softmax_scale"]))
        else:
            out = extension.dsv4_swa_decode_forward(q, cache, idx, lens, s, ps, float(g["softmax_scale"]))
        want = oracle.bf16_bits_to_f32(g[key]).astype(np.float64)
        assert_close(out, want, what=key)


@pytest.mark.parametrize("ratio", [0, 4, 128])
@pytest.mark.parametrize("nq,heads", [(1, 8), (1, 64), (32, 8), (32, 64)])
def test_baseline_window_configs(ratio, nq, heads):
    c = make_dsv4_window_case(compress_ratio=ratio, num_queries=nq, heads=heads, seed=ratio + nq + heads,
                              device=DEV)
    ref = oracle_out(c)
    assert_close(gpu_out(c), ref, what="tiled")
    for scale in (1.0 / math.sqrt(576),):
        assert_close(gpu_out(c, scale=scale), oracle_out(c, scale=scale), what="scale 1/sqrt(576)")


@pytest.mark.parametrize("ratio", [0, 4, 128])
def test_reference_harness_shapes_page_256(ratio):
    c = make_dsv4_case(compress_ratio=ratio, num_queries=7, heads=8, num_tokens=1024, top_k=128, page_size=256,
                       extra_tokens=1024, extra_top_k=0, seed=1, device=DEV)
    ref = oracle_out(c)
    assert_close(gpu_out(c), ref)
    assert_close(gpu_out(c, sink=False), oracle_out(c, sink=False), what="no sink")
    assert_close(gpu_out(c, lengths=False), oracle_out(c, lengths=False), what="no lengths")


@pytest.mark.parametrize("route", ["tiled-auto", "tiled-1", "tiled-8", "tiled-1000", "untiled"])
def test_routes_agree(route, monkeypatch):
    if route == "untiled":
        monkeypatch.setenv("CSAHCA_DSV4_TILED", "0")
    else:
        monkeypatch.setenv("CSAHCA_DSV4_TILE_SIZE", "0" if route == "tiled-auto" else route.split("-")[1])
    for ratio in (0, 4):
        c = make_dsv4_case(compress_ratio=ratio, num_queries=5, heads=16, num_tokens=512, top_k=64, page_size=64,
                           extra_tokens=512, extra_top_k=48, seed=3, device=DEV)
        assert_close(gpu_out(c), oracle_out(c), what=route)


@pytest.mark.parametrize("q_dtype", [torch.float32, torch.float16, torch.float64])
def test_query_dtypes(q_dtype):
    c = make_dsv4_case(compress_ratio=4, num_queries=3, heads=8, num_tokens=256, top_k=32, page_size=64,
                       extra_tokens=256, extra_top_k=32, q_dtype=q_dtype, seed=4, device=DEV)
    out = gpu_out(c)
    assert out.dtype == q_dtype
    tol = (5e-2, 5e-2) if q_dtype == torch.float16 else (1e-4, 1e-4)
    assert_close(out, oracle_out(c), *tol)


def test_edges():
    c = make_dsv4_case(compress_ratio=4, num_queries=4, heads=8, num_tokens=256, top_k=16, page_size=64,
                       extra_tokens=256, extra_top_k=16, seed=6, device=DEV)
    c.topk_lengths = torch.tensor([0, 16, 100, -3], dtype=torch.int32, device=DEV)
    c.extra_topk_lengths = torch.tensor([0, 5, 16, 0], dtype=torch.int32, device=DEV)
    c.token_indices[1, :4] = -1
    c.token_indices[2, 3] = 10_000_000  # page past the cache: skipped
    assert_close(gpu_out(c), oracle_out(c))
    # query 0 and 3 have nothing valid: with a sink the output is exactly 0
    out = gpu_out(c)
    assert torch.all(out[0] == 0) and torch.all(out[3] == 0)
    out = gpu_out(c, sink=False)
    assert torch.all(out[0] == 0)
    # every slot -1
    c.token_indices.fill_(-1)
    c.extra_token_indices.fill_(-1)
    assert torch.all(gpu_out(c) == 0)


def _poison_rows(cache, locs, page_size):
    """Rows (and scale bytes) of the given token locations made of NaN codes:
    e4m3 0x7f, bf16 rope 0x7fc0, scale bytes 254 (2^127)."""
    rows = dsv4_layout.NOPE_ROPE_BYTES
    for loc in locs:
        page, slot = divmod(int(loc), page_size)
        base = slot * rows
        cache[page, base:base + dsv4_layout.DIM_NOPE] = 0x7F
        cache[page, base + dsv4_layout.DIM_NOPE:base + rows] = torch.tensor([0xC0, 0x7F], dtype=torch.uint8).repeat(
            dsv4_layout.DIM_ROPE)
        sb = page_size * rows + slot * dsv4_layout.SCALE_BYTES_PER_TOKEN
        cache[page, sb:sb + dsv4_layout.NUM_SCALE_TILES] = 254


def test_onepass_never_reads_the_rows_of_slots_past_the_lengths():
    """The one-pass kernel (bf16 queries, lists of at most 256 slots) loads a
    zero row for every slot past its list's length: the rows those slots
    index are filled with NaN codes here (and are indexed by no counted slot),
    so any read of them would reach the output through the PV product."""
    c = make_dsv4_case(compress_ratio=4, num_queries=4, heads=16, num_tokens=256, top_k=64, page_size=64,
                       extra_tokens=256, extra_top_k=32, seed=9, device="cpu")
    for idx, lens, cache, ps in ((c.token_indices, c.topk_lengths, c.cache, c.page_size),
                                 (c.extra_token_indices, c.extra_topk_lengths, c.extra_cache, c.extra_page_size)):
        counted = {int(v) for q in range(idx.shape[0]) for v in idx[q, :max(int(lens[q]), 0)].tolist()}
        past = {int(v) for q in range(idx.shape[0]) for v in idx[q, max(int(lens[q]), 0):].tolist()}
        poison = sorted(l for l in past - counted if l >= 0)
        assert poison, "the case leaves no row indexed only past a length"
        _poison_rows(cache, poison, ps)
    want = oracle_out(c)
    assert np.isfinite(want).all()
    for name in ("q", "cache", "token_indices", "topk_lengths", "extra_cache", "extra_token_indices",
                 "extra_topk_lengths", "attn_sink"):
        setattr(c, name, getattr(c, name).to(DEV))
    got = gpu_out(c)
    assert torch.isfinite(got.float()).all()
    assert_close(got, want, what="rows past the lengths poisoned")


def test_unaligned_bytes_per_page_scalar_path():
    c = make_dsv4_case(compress_ratio=0, num_queries=3, heads=8, num_tokens=256, top_k=32, page_size=64, seed=7)
    bpp = c.cache.shape[1]
    wide = torch.zeros((c.cache.shape[0], bpp + 4), dtype=torch.uint8)
    wide[:, :bpp] = c.cache  # rows and scales keep their offsets; 4 trailing pad bytes per page
    c.cache = wide
    assert_close(gpu_out(c), oracle_out(c))


@pytest.mark.parametrize("path", ["valu-f32", "onepass-bf16", "query-bf16", "split-bf16"])
def test_e4m3_and_scale_decode_exhaustive(path, monkeypatch):
    """Single valid slot, no sink: out = the dequantised row exactly (softmax
    weight 1).  Rows cover all 256 e4m3 codes (NaN codes excluded) under many
    scale bytes.  fp32 queries take the VALU kernel; bf16 queries the one-pass
    kernel, the per-query MFMA kernel or the split MFMA kernel + merge (all
    round the probability 1.0 and the bf16 row exactly)."""
    codes = np.array([b for b in range(256) if (b & 0x7F) != 0x7F], dtype=np.uint8)
    ps = 4
    bpp = dsv4_layout.bytes_per_page(ps)
    # exponent bytes keep every dequantised value a normal fp32 number
    scale_bytes = [93, 100, 110, 120, 127, 130, 140, 200]
    n = len(scale_bytes)
    cache = np.zeros((math.ceil(n / ps), bpp), dtype=np.uint8)
    rope = torch.randn(n, 64, generator=torch.Generator().manual_seed(0)).bfloat16()
    rope_bytes = rope.view(torch.int16).numpy().view(np.uint8).reshape(n, 128)
    for t, sb in enumerate(scale_bytes):
        page, r = divmod(t, ps)
        row = np.resize(np.roll(codes, 37 * t), 448)
        cache[page, r * 576:r * 576 + 448] = row
        cache[page, r * 576 + 448:r * 576 + 576] = rope_bytes[t]
        cache[page, ps * 576 + r * 8:ps * 576 + r * 8 + 7] = [sb + 3 * j for j in range(7)]
    locs = np.arange(n, dtype=np.int32)
    want = oracle.dequant_dsv4_cache(cache, locs, page_size=ps).astype(np.float64)
    if path in ("query-bf16", "split-bf16"):
        monkeypatch.setenv("CSAHCA_DSV4_QUERY", "1" if path == "query-bf16" else "0")
    q = torch.zeros(n, 1, 512, dtype=torch.float32 if path == "valu-f32" else torch.bfloat16, device=DEV)
    idx = torch.from_numpy(locs.reshape(n, 1)).to(DEV)
    out = extension.dsv4_swa_decode_forward(q, torch.from_numpy(cache).to(DEV), idx, None, None, ps, SCALE)
    got = out[:, 0].float().cpu().numpy().astype(np.float64)
    # the oracle dequant rounds nope values to bf16 (exact for e4m3 * 2^k)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("ratio,nq,heads", [(0, 1, 8), (4, 3, 24), (128, 2, 64), (4, 7, 70), (0, 5, 16)])
def test_mfma_path_matches_valu_path_and_oracle(ratio, nq, heads, monkeypatch):
    """bf16 queries with automatic tiling take the grouped-head MFMA kernel;
    CSAHCA_DSV4_MFMA=0 keeps the VALU kernels.  Both against the oracle, with
    ragged lengths, -1 slots and heads not a multiple of 16."""
    page = 256 if ratio == 128 else 64  # extra pages hold page/ratio tokens (>= 1)
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=512, top_k=96, page_size=page,
                       extra_tokens=512, extra_top_k=40, seed=11 + heads, device=DEV)
    c.token_indices[0, 5] = -1
    ref = oracle_out(c)
    got_mfma = gpu_out(c)
    monkeypatch.setenv("CSAHCA_DSV4_MFMA", "0")
    got_valu = gpu_out(c)
    assert_close(got_mfma, ref, what="mfma")
    assert_close(got_valu, ref, what="valu")


@pytest.mark.parametrize("ratio,nq,heads,top_k,extra_top_k", [
    (0, 1, 8, 128, 0),      # SWA window: 8 sub-tiles, 2 per wavefront
    (4, 1, 8, 128, 64),     # 12 sub-tiles, 3 per wavefront
    (128, 1, 64, 128, 64),  # 4 head groups of one query on one XCD
    (4, 3, 24, 96, 40),     # second head group holds 8 heads
    (4, 7, 70, 96, 40),     # 5 head groups, the last with 6 heads; 7 queries
    (0, 2, 16, 600, 0),     # 38 sub-tiles: the row buffers refill 3 times
    (4, 2, 8, 5, 3),        # 8 slots: one partial sub-tile, three idle wavefronts
    (4, 9, 16, 40, 9),      # 9 queries: the grid's XCD mapping wraps
])
def test_query_kernel_matches_split_kernel_and_oracle(ratio, nq, heads, top_k, extra_top_k, monkeypatch):
    """The per-query MFMA kernel (CSAHCA_DSV4_QUERY=1) and the split MFMA kernel
    + merge (=0) against the oracle, with ragged lengths, -1 slots, a slot whose
    page is past the cache, and with and without the sink."""
    page = 256 if ratio == 128 else 64
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=1024, top_k=top_k,
                       page_size=page, extra_tokens=1024, extra_top_k=extra_top_k, seed=31 + heads + top_k,
                       device=DEV)
    c.token_indices[0, min(5, top_k - 1)] = -1
    c.token_indices[-1, 0] = 10_000_000
    for sink in (True, False):
        ref = oracle_out(c, sink=sink)
        for route in ("1", "0"):
            monkeypatch.setenv("CSAHCA_DSV4_QUERY", route)
            assert_close(gpu_out(c, sink=sink), ref, what=f"query={route} sink={sink}")


@pytest.mark.parametrize("ratio,nq,heads,top_k,extra_top_k", [
    (0, 1, 8, 128, 0),     # one round of 8 sub-tiles, two of 4
    (4, 3, 24, 96, 40),    # 9 sub-tiles: two rounds of 8 (the second nearly empty), three of 4
    (0, 2, 16, 600, 0),    # 38 sub-tiles
])
@pytest.mark.parametrize("waves", ["4", "8"])
@pytest.mark.parametrize("parts", ["1", "2", "4"])
def test_query_kernel_wavefront_counts(ratio, nq, heads, top_k, extra_top_k, waves, parts, monkeypatch):
    """The per-query kernel with 4 and with 8 wavefronts per workgroup
    (CSAHCA_DSV4_QWAVES), and with one or two workgroups per (query, 16 heads)
    each writing its share of the output dims (CSAHCA_DSV4_QPARTS), against
    the oracle, with ragged lengths and a -1 slot."""
    page = 256 if ratio == 128 else 64
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=1024, top_k=top_k,
                       page_size=page, extra_tokens=1024, extra_top_k=extra_top_k, seed=7 + heads + top_k,
                       device=DEV)
    c.token_indices[0, min(5, top_k - 1)] = -1
    monkeypatch.setenv("CSAHCA_DSV4_QUERY", "1")
    monkeypatch.setenv("CSAHCA_DSV4_QWAVES", waves)
    monkeypatch.setenv("CSAHCA_DSV4_QPARTS", parts)
    for sink in (True, False):
        assert_close(gpu_out(c, sink=sink), oracle_out(c, sink=sink), what=f"waves={waves} parts={parts} sink={sink}")


@pytest.mark.parametrize("ratio,nq,heads,top_k,extra_top_k", [
    (4, 7, 70, 96, 40),     # 5 head groups (the last with 6 heads), 7 queries
    (128, 32, 64, 64, 64),  # the benchmark's grouped-head shape class
    (0, 9, 16, 128, 0),     # 9 queries: the grid's XCD mapping wraps
])
def test_query_kernel_dim_parts_give_the_same_bits(ratio, nq, heads, top_k, extra_top_k, monkeypatch):
    """Two workgroups per (query, 16 heads), each writing half the output dims,
    run every output block's MFMA chain exactly as one workgroup does: the
    outputs are identical to the one-workgroup launch."""
    page = 256 if ratio == 128 else 64
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=1024, top_k=top_k,
                       page_size=page, extra_tokens=1024, extra_top_k=extra_top_k, seed=3 + nq + heads,
                       device=DEV)
    c.token_indices[0, 3] = -1
    monkeypatch.setenv("CSAHCA_DSV4_QUERY", "1")
    outs = {}
    for parts in ("1", "2", "4"):
        monkeypatch.setenv("CSAHCA_DSV4_QPARTS", parts)
        outs[parts] = gpu_out(c, sink=True)
    assert torch.equal(outs["1"], outs["2"])
    assert torch.equal(outs["1"], outs["4"])
    assert_close(outs["4"], oracle_out(c, sink=True), what="parts=4")


ONEPASS = [
    # ratio, nq, heads, top_k, extra_top_k
    (0, 1, 8, 128, 0),       # SWA window: 8 sub-tiles, one per wavefront
    (4, 1, 8, 128, 64),      # 12 sub-tiles: wavefronts 0..3 take two
    (128, 1, 64, 128, 64),   # 4 head groups of one query on one XCD
    (4, 3, 24, 96, 40),      # second head group holds 8 heads
    (4, 7, 70, 96, 40),      # 5 head groups, the last with 6 heads; 7 queries
    (4, 2, 8, 5, 3),         # 8 slots: one partial sub-tile, seven idle wavefronts
    (4, 9, 16, 40, 9),       # 9 queries: the grid's XCD mapping wraps
    (0, 2, 16, 256, 0),      # 256 slots: every wavefront takes two full sub-tiles
    (4, 32, 64, 128, 64),    # the benchmark's grouped-head shape class (2 dim parts)
    (128, 32, 8, 128, 64),   # 4 dim parts
]


@pytest.mark.parametrize("ratio,nq,heads,top_k,extra_top_k", ONEPASS)
def test_onepass_kernel_matches_oracle_and_query_kernel(ratio, nq, heads, top_k, extra_top_k, monkeypatch):
    """The one-pass kernel (the default route for bf16 queries with at most
    256 slots) against the oracle and against the per-query kernel
    (CSAHCA_DSV4_QUERY=1), with ragged lengths, a -1 slot, a slot whose page is
    past the cache, and with and without the sink."""
    page = 256 if ratio == 128 else 64
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=1024, top_k=top_k,
                       page_size=page, extra_tokens=1024, extra_top_k=extra_top_k, seed=41 + heads + top_k + nq,
                       device=DEV)
    c.token_indices[0, min(5, top_k - 1)] = -1
    c.token_indices[-1, 0] = 10_000_000
    for sink in (True, False):
        ref = oracle_out(c, sink=sink)
        got = gpu_out(c, sink=sink)
        assert_close(got, ref, what=f"onepass sink={sink}")
        monkeypatch.setenv("CSAHCA_DSV4_QUERY", "1")
        assert_close(got, gpu_out(c, sink=sink).float().cpu().numpy().astype(np.float64), what="vs query kernel")
        monkeypatch.delenv("CSAHCA_DSV4_QUERY")


@pytest.mark.parametrize("ratio,nq,heads,top_k,extra_top_k", [(4, 7, 70, 96, 40), (128, 32, 64, 64, 64),
                                                               (0, 9, 16, 128, 0)])
def test_onepass_dim_parts_give_the_same_bits(ratio, nq, heads, top_k, extra_top_k, monkeypatch):
    """Two or four workgroups per (query, 16 heads) (CSAHCA_DSV4_QPARTS), each
    writing its share of the output dims, run the same scores, softmax and
    output-block MFMA chains: identical outputs."""
    page = 256 if ratio == 128 else 64
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=1024, top_k=top_k,
                       page_size=page, extra_tokens=1024, extra_top_k=extra_top_k, seed=5 + nq + heads,
                       device=DEV)
    c.token_indices[0, 3] = -1
    outs = {}
    for parts in ("2", "4"):
        monkeypatch.setenv("CSAHCA_DSV4_QPARTS", parts)
        outs[parts] = gpu_out(c, sink=True)
    assert torch.equal(outs["2"], outs["4"])
    assert_close(outs["2"], oracle_out(c, sink=True), what="parts=2")


@pytest.mark.parametrize("ratio,nq,heads,top_k,extra_top_k", [(4, 3, 24, 128, 64), (0, 9, 16, 128, 0),
                                                               (4, 2, 8, 5, 3), (128, 32, 64, 128, 64)])
@pytest.mark.parametrize("waves", ["8", "12"])
def test_onepass_shapes_match_the_oracle(ratio, nq, heads, top_k, extra_top_k, waves, monkeypatch):
    """Lists of up to 192 slots run with 12 wavefronts of one sub-tile each by
    default; CSAHCA_DSV4_OPWAVES=8 forces the 8-wavefront shape (two sub-tiles
    each).  Both against the oracle, with ragged lengths and a -1 slot, and with
    two and four dim parts."""
    page = 256 if ratio == 128 else 64
    c = make_dsv4_case(compress_ratio=ratio, num_queries=nq, heads=heads, num_tokens=1024, top_k=top_k,
                       page_size=page, extra_tokens=1024, extra_top_k=extra_top_k, seed=13 + nq + heads,
                       device=DEV)
    c.token_indices[0, min(3, top_k - 1)] = -1
    monkeypatch.setenv("CSAHCA_DSV4_OPWAVES", waves)
    for parts in ("2", "4"):
        monkeypatch.setenv("CSAHCA_DSV4_QPARTS", parts)
        for sink in (True, False):
            assert_close(gpu_out(c, sink=sink), oracle_out(c, sink=sink), what=f"waves={waves} parts={parts}")


def test_onepass_takes_lists_up_to_256_slots(monkeypatch):
    """257 slots leave the one-pass kernel for the per-query kernel; both sides
    of the boundary match the oracle, and CSAHCA_DSV4_ONEPASS=0 routes a
    256-slot list to the per-query kernel with the same result."""
    for top_k in (256, 257):
        c = make_dsv4_case(compress_ratio=0, num_queries=4, heads=16, num_tokens=1024, top_k=top_k, page_size=64,
                           seed=top_k, device=DEV)
        ref = oracle_out(c)
        got = gpu_out(c)
        assert_close(got, ref, what=f"top_k={top_k}")
        monkeypatch.setenv("CSAHCA_DSV4_ONEPASS", "0")
        assert_close(gpu_out(c), ref, what=f"top_k={top_k} onepass off")
        monkeypatch.delenv("CSAHCA_DSV4_ONEPASS")


def test_onepass_with_an_empty_swa_list_and_without_lengths():
    """An empty SWA list with extra slots (the one-pass kernel's index loads
    then read the extra list for their stand-in addresses) and calls without
    length tensors, against the oracle."""
    c = make_dsv4_case(compress_ratio=4, num_queries=3, heads=16, num_tokens=1024, top_k=16, page_size=64,
                       extra_tokens=1024, extra_top_k=64, seed=77, device=DEV)
    c.token_indices = c.token_indices[:, :0].contiguous()
    c.topk_lengths = torch.zeros(3, dtype=torch.int32, device=c.topk_lengths.device)
    for lengths in (True, False):
        for sink in (True, False):
            assert_close(gpu_out(c, sink=sink, lengths=lengths), oracle_out(c, sink=sink, lengths=lengths),
                         what=f"empty SWA list, lengths={lengths} sink={sink}")
    c = make_dsv4_case(compress_ratio=0, num_queries=5, heads=8, num_tokens=1024, top_k=100, page_size=64, seed=78,
                       device=DEV)
    assert_close(gpu_out(c, lengths=False), oracle_out(c, lengths=False), what="SWA only, no lengths")


@pytest.mark.parametrize("route", ["onepass", "1", "0"])
def test_scale_byte_255_gives_nan_like_the_reference(route, monkeypatch):
    """A scale byte of 255 is 2^128 = inf in the reference's fp32 dequant, so
    every score of that query is NaN (q . k meets inf) and so is its output;
    queries whose rows have no such byte stay finite and correct.  The MFMA
    kernels decode such sub-tiles in software."""
    if route != "onepass":
        monkeypatch.setenv("CSAHCA_DSV4_QUERY", route)
    c = make_dsv4_case(compress_ratio=0, num_queries=3, heads=8, num_tokens=256, top_k=32, page_size=64, seed=9)
    cache = c.cache.clone()
    loc = int(c.token_indices[1, 3])
    page, r = divmod(loc, 64)
    cache[page, 64 * 576 + r * 8 + 2] = 255  # one scale byte of one row of query 1
    c.cache = cache
    c.topk_lengths = torch.full((3,), 32, dtype=torch.int32)
    c.token_indices[0].masked_fill_(c.token_indices[0] == loc, (loc + 1) % 256)
    c.token_indices[2].masked_fill_(c.token_indices[2] == loc, (loc + 1) % 256)
    ref = oracle_out(c)
    got = gpu_out(c).float().cpu().numpy()
    assert np.isnan(ref[1]).all() and np.isnan(got[1]).all()
    assert_close(torch.from_numpy(got[[0, 2]]), ref[[0, 2]])


def test_sglang_adapter_end_to_end(monkeypatch):
    """FlashMLA-shaped decode metadata through csahca_amd.sglang_dsv4 equals the
    2-D op call and the oracle."""
    import types

    from csahca_amd import sglang_dsv4

    monkeypatch.setenv("CSAHCA_DSV4_NATIVE", "1")
    c = make_dsv4_case(compress_ratio=4, num_queries=4, heads=16, num_tokens=512, top_k=64, page_size=64,
                       extra_tokens=512, extra_top_k=32, seed=21, device=DEV)
    ps, eps = c.page_size, c.extra_page_size
    pool = types.SimpleNamespace(get_extra_key_page_size=lambda layer: eps)
    mode = types.SimpleNamespace(name="DECODE", is_decode_or_idle=lambda: True)
    out = sglang_dsv4.maybe_dsv4_decode_forward(
        q=c.q.unsqueeze(1), layer_id=0, compress_ratio=4, forward_batch=types.SimpleNamespace(forward_mode=mode),
        token_to_kv_pool=pool, swa_k_cache=c.cache.view(c.cache.shape[0], ps, 1, -1),
        swa_page_indices=c.token_indices.unsqueeze(1), swa_topk_lengths=c.topk_lengths,
        extra_k_cache=c.extra_cache.view(c.extra_cache.shape[0], eps, 1, -1),
        extra_indices=c.extra_token_indices.unsqueeze(1), extra_topk_lengths=c.extra_topk_lengths,
        attn_sink=c.attn_sink, page_size=ps, softmax_scale=SCALE)
    assert torch.equal(out, gpu_out(c))
    assert_close(out, oracle_out(c))
