"""Pin the DSV4 oracle and the product's torch pack against the reference's golden
vectors (tests/golden/dsv4_*.npz) and closed forms."""
import ast
import hashlib
import json
import math

import numpy as np
import pytest
import torch

import oracle
from csahca_amd import dsv4_layout
from csahca_amd.synthetic import make_dsv4_case


def bf16(bits):
    return oracle.bf16_bits_to_f32(bits)


def bits_to_bf16_tensor(bits):
    return torch.from_numpy(np.asarray(bits, np.uint16).view(np.int16).copy()).view(torch.bfloat16)


@pytest.fixture(scope="module", params=[0, 4, 128])
def case(request, golden_dir):
    return np.load(golden_dir / f"dsv4_c{request.param}.npz")


def test_bytes_per_page(golden_dir):
    want = ast.literal_eval(str(np.load(golden_dir / "dsv4_pack_edges.npz")["bpp"]))
    for ps, bpp in want.items():
        assert oracle.bytes_per_page(ps) == bpp
        assert dsv4_layout.bytes_per_page(ps) == bpp
    assert oracle.bytes_per_page(64) == 37440 and oracle.bytes_per_page(256) == 149760


def test_pack_matches_golden(case):
    page = int(case["page_size"])
    assert np.array_equal(oracle.pack_dsv4_cache(case["k_tokens"], page_size=page), case["cache"])
    got = dsv4_layout.pack_dsv4_cache(bits_to_bf16_tensor(case["k_tokens"]), page_size=page)
    assert np.array_equal(got.numpy(), case["cache"])
    if int(case["ratio"]):
        eps = int(case["extra_page_size"])
        assert np.array_equal(oracle.pack_dsv4_cache(case["extra_tokens"], page_size=eps), case["extra_cache"])
        got = dsv4_layout.pack_dsv4_cache(bits_to_bf16_tensor(case["extra_tokens"]), page_size=eps)
        assert np.array_equal(got.numpy(), case["extra_cache"])


def test_pack_edges_golden(golden_dir):
    g = np.load(golden_dir / "dsv4_pack_edges.npz")
    ps = int(g["page_size"])
    assert np.array_equal(oracle.pack_dsv4_cache(g["k_tokens"], page_size=ps), g["cache"])
    got = dsv4_layout.pack_dsv4_cache(bits_to_bf16_tensor(g["k_tokens"]), page_size=ps)
    assert np.array_equal(got.numpy(), g["cache"])


def test_dequant_matches_golden(case):
    page = int(case["page_size"])
    got = oracle.dequant_dsv4_cache(case["cache"], case["token_indices"][:1], page_size=page)
    assert np.array_equal(got, bf16(case["dequant_q0"]))


def _run(case, sink=True):
    kw = {}
    if int(case["ratio"]):
        kw = dict(extra_cache=case["extra_cache"], extra_token_indices=case["extra_token_indices"],
                  extra_topk_lengths=case["extra_topk_lengths"], extra_page_size=int(case["extra_page_size"]))
    return oracle.dsv4_reference_attention(bf16(case["q"]), case["cache"], case["token_indices"],
                                           case["topk_lengths"], case["attn_sink"] if sink else None,
                                           page_size=int(case["page_size"]),
                                           softmax_scale=float(case["softmax_scale"]), **kw)


def test_attention_matches_golden(case):
    for sink, key in ((True, "out"), (False, "out_nosink")):
        got = oracle.round_to(_run(case, sink), torch.bfloat16)
        want = bf16(case[key])
        assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-6), np.abs(got - want).max()


def test_draw_order_hashes(golden_dir):
    meta = json.loads((golden_dir / "synthetic_hash.json").read_text())
    for ratio in (0, 4, 128):
        c = make_dsv4_case(compress_ratio=ratio, num_queries=3, heads=8, num_tokens=128, top_k=32, page_size=64,
                           extra_tokens=128, extra_top_k=32, extra_page_size=max(1, 64 // ratio) if ratio else None,
                           seed=0, pack=False)
        want = meta[f"dsv4_c{ratio}"]
        for name, digest in want.items():
            t = getattr(c, name)
            assert hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest() == digest, name


def _single_token_cache(row_bf16: torch.Tensor, page_size=4):
    return oracle.pack_dsv4_cache(row_bf16.reshape(1, 512), page_size=page_size)


def test_closed_forms():
    rng = np.random.default_rng(0)
    row = torch.from_numpy(rng.standard_normal(512).astype(np.float32)).to(torch.bfloat16)
    cache = _single_token_cache(row)
    k = oracle.dequant_dsv4_cache(cache, np.array([0], np.int32), page_size=4)[0].astype(np.float64)
    q = rng.standard_normal((1, 2, 512)).astype(np.float32)
    scale = 1 / math.sqrt(512)
    idx = np.array([[0, -1, -1]], np.int32)
    sink = np.array([0.3, -1.2], np.float32)
    out = oracle.dsv4_reference_attention(q, cache, idx, None, sink, page_size=4, softmax_scale=scale)
    for h in range(2):
        x = float(np.dot(q[0, h].astype(np.float64), k)) * scale
        w = math.exp(x) / (math.exp(x) + math.exp(float(sink[h])))
        np.testing.assert_allclose(out[0, h], w * k, rtol=1e-12, atol=1e-12)
    # no sink: a single token gets weight 1
    out = oracle.dsv4_reference_attention(q, cache, idx, None, None, page_size=4, softmax_scale=scale)
    np.testing.assert_allclose(out[0, 0], k, rtol=0, atol=1e-12)
    # sink = -inf is the same as no sink
    out2 = oracle.dsv4_reference_attention(q, cache, idx, None, np.full(2, -np.inf, np.float32), page_size=4,
                                           softmax_scale=scale)
    np.testing.assert_allclose(out2, out, rtol=0, atol=0)
    # all slots invalid -> 0, with or without sink; length 0 -> 0
    for s in (None, sink):
        o = oracle.dsv4_reference_attention(q, cache, np.full((1, 3), -1, np.int32), None, s, page_size=4,
                                            softmax_scale=scale)
        assert np.all(o == 0)
        o = oracle.dsv4_reference_attention(q, cache, idx, np.array([0], np.int32), s, page_size=4,
                                            softmax_scale=scale)
        assert np.all(o == 0)


def test_pack_round_trip_error_bound():
    rng = np.random.default_rng(7)
    x = torch.from_numpy((rng.standard_normal((64, 512)) * np.exp(rng.uniform(-6, 6, (64, 1)))).astype(np.float32))
    xb = x.to(torch.bfloat16)
    cache = dsv4_layout.pack_dsv4_cache(xb, page_size=16)
    deq = torch.from_numpy(oracle.dequant_dsv4_cache(cache.numpy(), np.arange(64, dtype=np.int32), page_size=16))
    ref = xb.float()
    assert torch.equal(deq[:, 448:], ref[:, 448:])
    tile_max = ref[:, :448].reshape(64, 7, 64).abs().amax(-1, keepdim=True)
    err = (deq[:, :448] - ref[:, :448]).reshape(64, 7, 64).abs()
    # e4m3 keeps 4 significant bits: relative error <= 2^-4 of the value; subnormal floor 2^-10 of the tile max
    bound = torch.maximum(ref[:, :448].reshape(64, 7, 64).abs() * 2 ** -4, tile_max * 2 ** -10)
    assert torch.all(err <= bound * 1.0001)


def test_scale_byte_255_makes_the_query_nan():
    """A scale byte of 255 decodes to 2^128 = inf in fp32 (dsv4_correctness.py:76),
    so that query's scores meet inf and torch.softmax -- the reference's
    normaliser (:139) -- returns NaN, which the output inherits; other queries
    are untouched.  Checked against torch.softmax on the oracle's own
    dequantised rows, and against the oracle with the byte cleared."""
    import math

    import torch

    from csahca_amd.synthetic import make_dsv4_case

    c = make_dsv4_case(compress_ratio=0, num_queries=3, heads=8, num_tokens=256, top_k=32, page_size=64, seed=9)
    cache = c.cache.clone()
    loc = int(c.token_indices[1, 3])
    page, r = divmod(loc, 64)
    cache[page, 64 * 576 + r * 8 + 2] = 255
    for qi in (0, 2):
        c.token_indices[qi].masked_fill_(c.token_indices[qi] == loc, (loc + 1) % 256)
    lens = torch.full((3,), 32, dtype=torch.int32)
    scale = 1.0 / math.sqrt(512)
    out = oracle.dsv4_reference_attention(c.q, cache, c.token_indices, lens, c.attn_sink, page_size=64,
                                          softmax_scale=scale)
    rows = torch.from_numpy(oracle.dequant_dsv4_cache(cache.numpy(), c.token_indices[1].numpy().astype(np.int32),
                                                      page_size=64).astype(np.float32))
    assert torch.isinf(rows).any()
    scores = torch.cat([c.attn_sink[:1], rows @ c.q[1, 0].float() * scale])
    assert torch.isnan(torch.softmax(scores, dim=0)).all()
    assert np.isnan(out[1]).all()
    clean = oracle.dsv4_reference_attention(c.q, c.cache, c.token_indices, lens, c.attn_sink, page_size=64,
                                            softmax_scale=scale)
    assert np.isfinite(out[[0, 2]]).all() and np.array_equal(out[[0, 2]], clean[[0, 2]])
