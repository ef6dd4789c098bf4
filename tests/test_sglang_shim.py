"""CPU tests of the SGLang DSV4 adapter (csahca_amd/sglang_dsv4.py): gating,
strict-mode errors, FlashMLA view flattening and per-query padding, checked
with fake SGLang metadata objects and a captured op call (the caller contract
of integrations/sglang_dsv4/csahca_sglang_dsv4_native.py:28-157 and
csahca_sglang_dsv4_patch/patch.py:300-357)."""
import types

import pytest
import torch

from csahca_amd import extension, sglang_dsv4


class Mode:
    def __init__(self, name, decode=True):
        self.name = name
        self._decode = decode

    def is_decode_or_idle(self):
        return self._decode


class Pool:
    def __init__(self, extra_page_size):
        self.extra_page_size = extra_page_size
        self.asked = []

    def get_extra_key_page_size(self, layer_id):
        self.asked.append(layer_id)
        return self.extra_page_size


def metadata(ratio=4, T=3, H=8, pages=5, ps=64, K=16, EK=8, q4d=True, cache4d=True):
    bytes_per_row = 585  # 64 * 585 = 37440 = bytes_per_page(64)
    q = torch.zeros(T, 1, H, 512, dtype=torch.bfloat16) if q4d else torch.zeros(T, H, 512, dtype=torch.bfloat16)
    cache = torch.zeros(pages, ps, 1, bytes_per_row, dtype=torch.uint8) if cache4d else torch.zeros(pages, ps * bytes_per_row, dtype=torch.uint8)
    md = dict(q=q, layer_id=7, compress_ratio=ratio, forward_batch=types.SimpleNamespace(forward_mode=Mode("DECODE")),
              token_to_kv_pool=Pool(16), swa_k_cache=cache, swa_page_indices=torch.zeros(T, 1, K, dtype=torch.int32),
              swa_topk_lengths=torch.full((T,), K, dtype=torch.int32), extra_k_cache=None, extra_indices=None,
              extra_topk_lengths=None, attn_sink=torch.zeros(H), page_size=ps, softmax_scale=0.044)
    if ratio:
        md.update(extra_k_cache=torch.zeros(pages, 16, 1, 585, dtype=torch.uint8),
                  extra_indices=torch.zeros(T, 1, EK, dtype=torch.int32),
                  extra_topk_lengths=torch.full((T,), EK, dtype=torch.int32))
    return md


@pytest.fixture
def captured(monkeypatch):
    calls = []
    monkeypatch.setattr(extension, "dsv4_swa_decode_forward", lambda *a: calls.append(("swa", a)) or "swa-out")
    monkeypatch.setattr(extension, "dsv4_sparse_decode_forward", lambda *a: calls.append(("sparse", a)) or "sparse-out")
    monkeypatch.setenv("CSAHCA_DSV4_NATIVE", "1")
    monkeypatch.delenv("CSAHCA_DSV4_NATIVE_STRICT", raising=False)
    monkeypatch.delenv("CSAHCA_DSV4_NATIVE_FORWARD_MODES", raising=False)
    return calls


def test_disabled_by_default(monkeypatch):
    monkeypatch.delenv("CSAHCA_DSV4_NATIVE", raising=False)
    assert sglang_dsv4.maybe_dsv4_decode_forward(**metadata()) is None
    monkeypatch.setenv("CSAHCA_DSV4_NATIVE", "off")
    assert sglang_dsv4.maybe_dsv4_decode_forward(**metadata()) is None


def test_forward_mode_gate(captured, monkeypatch):
    md = metadata()
    md["forward_batch"] = types.SimpleNamespace(forward_mode=Mode("EXTEND", decode=False))
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) is None
    md["forward_batch"] = types.SimpleNamespace(forward_mode=Mode("IDLE"))
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) == "sparse-out"
    monkeypatch.setenv("CSAHCA_DSV4_NATIVE_FORWARD_MODES", "DECODE")
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) is None
    md["forward_batch"] = types.SimpleNamespace()
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) is None


def test_sparse_route_flattens_flashmla_views(captured):
    md = metadata(ratio=4, T=3, H=8, pages=5, ps=64, K=16, EK=8)
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) == "sparse-out"
    kind, args = captured[-1]
    q, cache, ids, lens, ecache, eids, elens, sink, ps, eps, scale = args
    assert kind == "sparse" and q.shape == (3, 8, 512) and cache.shape == (5, 64 * 585)
    assert ids.shape == (3, 16) and lens.shape == (3,) and ecache.shape == (5, 16 * 585) and eids.shape == (3, 8)
    assert (ps, eps, scale) == (64, 16, pytest.approx(0.044)) and md["token_to_kv_pool"].asked == [7]


def test_swa_route(captured):
    md = metadata(ratio=0, q4d=False, cache4d=False)
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) == "swa-out"
    kind, args = captured[-1]
    assert kind == "swa" and args[0].shape == (3, 8, 512) and args[1].shape == (5, 64 * 585)


@pytest.mark.parametrize("change,msg", [
    (dict(compress_ratio=2), "unsupported native CSAHCA DSV4 compress_ratio=2"),
    (dict(attn_sink=None), "requires attn_sink"),
    (dict(q=torch.zeros(3, 2, 8, 512)), "unsupported q shape"),
    (dict(swa_page_indices=None), "missing swa_page_indices"),
    (dict(swa_topk_lengths=torch.zeros(3, 2, dtype=torch.int32)), "unsupported swa_topk_lengths shape"),
    (dict(swa_k_cache=torch.zeros(5, 64, 2, 585, dtype=torch.uint8)), "unsupported swa_k_cache shape"),
    (dict(extra_k_cache=None), "missing extra_k_cache"),
])
def test_strict_mode_raises_and_lenient_mode_delegates(captured, monkeypatch, change, msg):
    md = metadata(ratio=4)
    md.update(change)
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) is None
    monkeypatch.setenv("CSAHCA_DSV4_NATIVE_STRICT", "1")
    with pytest.raises(RuntimeError, match=msg):
        sglang_dsv4.maybe_dsv4_decode_forward(**md)


def test_match_num_queries_pads_and_truncates():
    x = torch.arange(6, dtype=torch.int32).view(2, 3)
    assert sglang_dsv4.match_num_queries(x, 2, -1) is x
    assert sglang_dsv4.match_num_queries(None, 4, 0) is None
    assert torch.equal(sglang_dsv4.match_num_queries(x, 1, -1), x[:1])
    padded = sglang_dsv4.match_num_queries(x, 4, -1)
    assert padded.shape == (4, 3) and torch.equal(padded[:2], x) and torch.all(padded[2:] == -1)


def test_prepare_indices_from_decode_metadata():
    q = torch.zeros(4, 8, 512)
    core = types.SimpleNamespace(
        swa_page_indices=torch.ones(2, 1, 16, dtype=torch.int32), swa_topk_lengths=torch.full((2, 1), 16),
        c4_sparse_page_indices=torch.ones(2, 1, 8, dtype=torch.int32), c4_sparse_topk_lengths=torch.full((2,), 8),
        c128_page_indices=torch.ones(5, 4, dtype=torch.int32), c128_topk_lengths_clamp1=torch.full((5,), 4))
    ids, lens = sglang_dsv4.prepare_swa_indices(core=core, q=q)
    assert ids.shape == (4, 16) and torch.all(ids[2:] == 0) and lens.tolist() == [16, 16, 1, 1]
    ids, lens = sglang_dsv4.prepare_extra_indices(core=core, q=q, compress_ratio=4)
    assert ids.shape == (4, 8) and torch.all(ids[2:] == -1) and lens.tolist() == [8, 8, 1, 1]
    ids, lens = sglang_dsv4.prepare_extra_indices(core=core, q=q, compress_ratio=128)
    assert ids.shape == (4, 4) and lens.tolist() == [4, 4, 4, 4]
    with pytest.raises(RuntimeError, match="compress_ratio=0"):
        sglang_dsv4.prepare_extra_indices(core=core, q=q, compress_ratio=0)
    core.swa_page_indices = torch.ones(4, 2, 16, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="unsupported DSV4 SWA index shape"):
        sglang_dsv4.prepare_swa_indices(core=core, q=q)


@pytest.mark.parametrize("change,msg", [
    (dict(extra_indices=torch.zeros(3, 2, 8, dtype=torch.int32)), "unsupported extra_indices shape"),
    (dict(extra_topk_lengths=None), "missing extra_topk_lengths for native CSAHCA DSV4 decode"),
    (dict(extra_k_cache=torch.zeros(5, 16, 585, dtype=torch.uint8)), "unsupported extra_k_cache shape"),
    # the first unusable argument in route order names the error
    (dict(q=torch.zeros(8, 512), extra_k_cache=None), "unsupported q shape"),
])
def test_strict_mode_extra_arguments(captured, monkeypatch, change, msg):
    md = metadata(ratio=128)
    md.update(change)
    assert sglang_dsv4.maybe_dsv4_decode_forward(**md) is None
    monkeypatch.setenv("CSAHCA_DSV4_NATIVE_STRICT", "yes")
    with pytest.raises(RuntimeError, match=msg):
        sglang_dsv4.maybe_dsv4_decode_forward(**md)
    assert captured == []


def test_routes_cover_the_reference_ratios_only():
    assert sorted(sglang_dsv4.ROUTES) == [0, 4, 128]
    assert [s.name for s in sglang_dsv4.ROUTES[0].args] == ["q", "swa_k_cache", "swa_page_indices",
                                                           "swa_topk_lengths"]
    assert [s.name for s in sglang_dsv4.ROUTES[4].args][4:] == ["extra_k_cache", "extra_indices",
                                                               "extra_topk_lengths"]


def test_conform_folds_only_unit_axes():
    spec = sglang_dsv4.paged_cache("c")
    x = torch.arange(2 * 3 * 4, dtype=torch.uint8).view(2, 3, 1, 4)
    assert torch.equal(sglang_dsv4.conform(spec, x), x.view(2, 12))
    with pytest.raises(sglang_dsv4.Decline, match=r"unsupported c shape .*\(2, 3, 2, 2\)"):
        sglang_dsv4.conform(spec, x.view(2, 3, 2, 2))
    with pytest.raises(sglang_dsv4.Decline, match="unsupported n shape"):
        sglang_dsv4.conform(sglang_dsv4.lengths("n"), torch.zeros(3, 1))


def test_metadata_missing_extra_fields():
    q = torch.zeros(2, 8, 512)
    core = types.SimpleNamespace(c128_page_indices=torch.ones(2, 4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="missing DSV4 extra indices/topk lengths for compress_ratio=128"):
        sglang_dsv4.prepare_extra_indices(core=core, q=q, compress_ratio=128)
    core = types.SimpleNamespace(swa_page_indices=torch.ones(2, 1, 1, 16, dtype=torch.int32),
                                 swa_topk_lengths=torch.ones(2))
    with pytest.raises(RuntimeError, match="unsupported DSV4 SWA index rank 4"):
        sglang_dsv4.prepare_swa_indices(core=core, q=q)
