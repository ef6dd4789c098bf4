"""CPU-only checks of the C ABI and the torch binding: the library loads, exports
every symbol include/csahca.h declares, and rejects bad arguments on the host
with the reference's messages -- before any HIP call, so no GPU is needed."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from csahca_amd import extension, native

ROOT = Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "csahca.h").read_text()
    return sorted(set(re.findall(r"\b(csahca_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not native.library_path().exists():
        pytest.fail("libcsahca.so is not built (run python -m csahca_amd.build)")
    return native.lib()


def test_exports_every_header_symbol(lib):
    syms = header_symbols()
    assert len(syms) >= 19
    raw = ctypes.CDLL(str(native.library_path()))
    for s in syms:
        assert hasattr(raw, s), s
    assert set(syms) == set(native.EXPORTED)
    assert lib.csahca_abi_version() == native.ABI_VERSION == 1


def test_clock_stamp_rejects_a_null_pointer_before_any_launch(lib):
    assert lib.csahca_device_clock_stamp(None, None) == 1
    assert b"null clock stamp pointer" in lib.csahca_last_error()


def test_timeline_build_is_a_separate_library():
    """The phase stamps live only in libcsahca_timeline.so (built beside the
    product library); the product library exports none of their entry points."""
    from csahca_amd import build

    names = ("csahca_step_timeline_read", "csahca_step_timeline_clear", "csahca_step_timeline_rate_khz")
    tl = ctypes.CDLL(str(build.LIB_TIMELINE))
    for n in names:
        assert hasattr(tl, n), n
    prod = ctypes.CDLL(str(native.library_path()))
    for n in names:
        assert not hasattr(prod, n), n


def test_workspace_sizes(lib):
    # B1 H8 D128 k8 chunk64 tile8: 64 tiles per head -> 8*64*(2 + 128) floats (+ alignment)
    n = lib.csahca_csa_decode_workspace_bytes(1, 8, 128, 8, 64, 8)
    assert n >= 8 * 64 * 130 * 4
    assert lib.csahca_csa_select_workspace_bytes(1, 8, 512) == 8 * 512 * 4
    assert lib.csahca_dsv4_decode_workspace_bytes(1, 8, 128, 64, 0) > 0
    assert lib.csahca_csa_auto_tile_size(1, 8, 8, 64) >= 16


def _csa_call(lib, **over):
    args = dict(q=1, k=1, v=1, idx=1, out=1, dtype=2, index_dtype=0, B=1, H=1, S=64, D=128, top_k=1, chunk=64,
                tile=8, ws=None, wsb=0)
    args.update(over)
    return lib.csahca_csa_decode_forward_tiled(args["q"], args["k"], args["v"], args["idx"], args["out"],
                                               args["dtype"], args["index_dtype"], args["B"], args["H"], args["S"],
                                               args["D"], args["top_k"], args["chunk"], args["tile"], args["ws"],
                                               args["wsb"], None)


def test_csa_argument_errors_before_any_launch(lib):
    assert _csa_call(lib, chunk=0) == 1
    assert lib.csahca_last_error().decode() == "chunk_size must be positive"
    assert _csa_call(lib, tile=0) == 1
    assert lib.csahca_last_error().decode() == "tile_size must be positive"
    assert _csa_call(lib, D=2048) == 1
    assert "head_dim > 1024" in lib.csahca_last_error().decode()
    assert _csa_call(lib, dtype=9) == 1
    assert _csa_call(lib, index_dtype=5) == 1
    assert lib.csahca_last_error().decode() == "chunk_indices must be int32 or int64"
    # missing workspace is reported, not dereferenced
    assert _csa_call(lib) == 2
    # empty problems succeed without touching memory
    assert _csa_call(lib, B=0) == 0


def test_dsv4_argument_errors(lib):
    f = lib.csahca_dsv4_decode_forward_tiled
    common = dict(q=1, dtype=2, nq=1, heads=8, cache=1, pages=1, bpp=37440, ps=64, idx=1, slots=4, lens=None,
                  ecache=None, epages=0, ebpp=0, eps=1, eidx=None, eslots=0, elens=None, sink=None, scale=0.04,
                  tile=0, out=1, ws=None, wsb=0)

    def call(**o):
        a = dict(common)
        a.update(o)
        return f(a["q"], a["dtype"], a["nq"], a["heads"], a["cache"], a["pages"], a["bpp"], a["ps"], a["idx"],
                 a["slots"], a["lens"], a["ecache"], a["epages"], a["ebpp"], a["eps"], a["eidx"], a["eslots"],
                 a["elens"], a["sink"], a["scale"], a["tile"], a["out"], a["ws"], a["wsb"], None)

    assert call(ps=0) == 1 and lib.csahca_last_error().decode() == "page_size must be positive"
    assert call(bpp=1000) == 1
    assert lib.csahca_last_error().decode() == "bytes_per_page is too small for DSV4 page layout"
    assert call(bpp=37442) == 1
    assert "divisible by 4" in lib.csahca_last_error().decode()
    assert call(ecache=1, epages=4, ebpp=9792, eps=0, eidx=1, eslots=8) == 1
    assert lib.csahca_last_error().decode() == "extra_page_size must be positive"
    assert call(ecache=1, epages=4, ebpp=100, eps=16, eidx=1, eslots=8) == 1
    assert lib.csahca_last_error().decode() == "extra_bytes_per_page is too small for DSV4 page layout"
    assert call() == 2  # valid arguments, no workspace
    assert call(nq=0) == 0
    g = lib.csahca_dsv4_sparse_decode_forward
    rc = g(1, 2, 1, 8, 1, 1, 37440, 64, 1, 4, None, 1, 1, 9792, 0, 1, 8, None, None, 0.04, 1, None, 0, None)
    assert rc == 1 and lib.csahca_last_error().decode() == "extra_page_size must be positive"


def test_device_state_entry_points_argument_errors(lib):
    """csahca_csa_decode_step_dev / csahca_csa_chunk_summary_at reject bad
    arguments before any HIP call (dummy pointers are never dereferenced)."""
    def step(**o):
        a = dict(q=1, k=1, v=1, summ=1, n=1, out=1, idx=1, dtype=2, B=1, H=1, S=64, D=128, C=1, chunk=64, top_k=1,
                 ws=None, wsb=0)
        a.update(o)
        return lib.csahca_csa_decode_step_dev(a["q"], a["k"], a["v"], a["summ"], a["n"], a["out"], a["idx"], a["dtype"],
                                              a["B"], a["H"], a["S"], a["D"], a["C"], a["chunk"], a["top_k"], a["ws"],
                                              a["wsb"], None)

    assert step(n=None) == 1 and lib.csahca_last_error().decode() == "null num_chunks pointer"
    assert step(chunk=0) == 1 and lib.csahca_last_error().decode() == "chunk_size must be positive"
    assert step(C=2) == 1 and lib.csahca_last_error().decode() == "summaries cover more chunks than the cache holds"
    assert step(top_k=-1) == 1
    assert step() == 2  # valid arguments, no workspace
    assert step(B=0) == 0

    def step_at(**o):
        a = dict(q=1, k=1, v=1, summ=1, pos=1, out=1, idx=1, dtype=2, B=1, H=1, S=64, D=128, C=1, chunk=64, top_k=1,
                 ws=None, wsb=0)
        a.update(o)
        return lib.csahca_csa_decode_step_at(a["q"], a["k"], a["v"], a["summ"], a["pos"], a["out"], a["idx"],
                                             a["dtype"], a["B"], a["H"], a["S"], a["D"], a["C"], a["chunk"],
                                             a["top_k"], a["ws"], a["wsb"], None)

    assert step_at(pos=None) == 1 and lib.csahca_last_error().decode() == "null token_pos pointer"
    assert step_at(C=2) == 1 and lib.csahca_last_error().decode() == "summaries cover more chunks than the cache holds"
    assert step_at() == 2  # valid arguments, no workspace
    assert step_at(B=0) == 0

    def summ_at(**o):
        a = dict(k=1, summ=1, dtype=2, B=1, H=1, S=64, D=128, chunk=64, C=1, pos=1)
        a.update(o)
        return lib.csahca_csa_chunk_summary_at(a["k"], a["summ"], a["dtype"], a["B"], a["H"], a["S"], a["D"],
                                               a["chunk"], a["C"], a["pos"], None)

    assert summ_at(pos=None) == 1 and lib.csahca_last_error().decode() == "null token_pos pointer"
    assert summ_at(chunk=0) == 1 and lib.csahca_last_error().decode() == "chunk_size must be positive"
    assert summ_at(dtype=9) == 1
    assert summ_at(C=0) == 0  # no summary rows: nothing to write


def test_hybrid_argument_errors(lib):
    """csahca_hybrid_decode_forward checks its HCA half before anything runs."""
    def hyb(**o):
        a = dict(q=1, k=1, v=1, summ=1, csa=1, idx=1, out=1, dtype=2, B=1, H=1, S=512, D=128, C=8, cc=64, top_k=4,
                 hc=256, w=0.7, sws=None, swsb=0, hws=None, hwsb=0)
        a.update(o)
        return lib.csahca_hybrid_decode_forward(a["q"], a["k"], a["v"], a["summ"], a["csa"], a["idx"], a["out"],
                                                a["dtype"], a["B"], a["H"], a["S"], a["D"], a["C"], a["cc"],
                                                a["top_k"], a["hc"], a["w"], a["sws"], a["swsb"], a["hws"], a["hwsb"],
                                                None)

    assert hyb(hc=300) == 1 and lib.csahca_last_error().decode() == "seq length must be divisible by chunk_size"
    assert hyb(hc=0) == 1 and lib.csahca_last_error().decode() == "chunk_size must be positive"
    assert hyb(csa=None) == 1 and lib.csahca_last_error().decode() == "null tensor pointer"
    assert hyb() == 2 and lib.csahca_last_error().decode() == "workspace too small for hca decode"
    assert hyb(B=0) == 0


def test_block_product_argument_errors(lib):
    """csahca_block_linear / csahca_block_qkv reject bad arguments before any
    HIP call (dummy pointers are never dereferenced)."""
    def lin(**o):
        a = dict(x=16, norm=None, eps=1e-6, w=16, act=0, res=None, base=None, alpha=1.0, y=16, dtype=2, B=1, N=8,
                 K=64, adv=None)
        a.update(o)
        return lib.csahca_block_linear(a["x"], a["norm"], a["eps"], a["w"], a["act"], a["res"], a["base"], a["alpha"],
                                       a["y"], a["dtype"], a["B"], a["N"], a["K"], a["adv"], None)

    assert lin(dtype=0) == 1 and "bfloat16 and float16" in lib.csahca_last_error().decode()
    assert lin(B=5) == 1 and "at most 4 token rows" in lib.csahca_last_error().decode()
    assert lin(K=12) == 1 and "multiple of 8" in lib.csahca_last_error().decode()
    assert lin(K=4104) == 1
    assert lin(B=2, K=4096) == 1 and "needs batch 1" in lib.csahca_last_error().decode()
    assert lin(act=7) == 1 and lib.csahca_last_error().decode() == "unknown activation"
    assert lin(x=8) == 1 and "16-byte aligned" in lib.csahca_last_error().decode()
    assert lin(w=None) == 1 and lib.csahca_last_error().decode() == "null tensor pointer"
    assert lin(B=0) == 0 and lin(N=0) == 0  # empty products: nothing to do
    assert lin(B=0, adv=16) == 1 and "non-empty product" in lib.csahca_last_error().decode()
    assert lin(K=0) == 1 and lib.csahca_last_error().decode() == "in_features must be positive"

    def qkv(**o):
        a = dict(h=16, norm=None, eps=1e-6, w=16, q=16, k=16, v=16, pos=16, nch=None, dtype=2, B=1, H=2, D=64,
                 cap=128, chunk=64)
        a.update(o)
        return lib.csahca_block_qkv(a["h"], a["norm"], a["eps"], a["w"], a["q"], a["k"], a["v"], a["pos"], a["nch"],
                                    a["dtype"], a["B"], a["H"], a["D"], a["cap"], a["chunk"], None)

    assert qkv(pos=None) == 1 and lib.csahca_last_error().decode() == "null token_pos pointer"
    assert qkv(chunk=0) == 1 and lib.csahca_last_error().decode() == "chunk_size must be positive"
    assert qkv(D=61) == 1 and "multiple of 8" in lib.csahca_last_error().decode()  # H*D = 122
    assert qkv(dtype=3) == 1
    assert qkv(B=0) == 0


def test_binding_rejects_cpu_tensors_with_reference_messages(lib):
    q = torch.zeros(1, 2, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)
    idx = torch.zeros(1, 2, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="all tensors must be CUDA tensors"):
        native.csa_decode_forward(q, k, k, idx, 64)
    with pytest.raises(RuntimeError, match="all tensors must be CUDA tensors"):
        extension.csa_decode_forward_tiled(q, k, k, idx, 64)
    cache = torch.zeros(1, 37440, dtype=torch.uint8)
    tok = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="q, paged_k_cache_u8, and token_indices must be CUDA tensors"):
        extension.dsv4_swa_decode_forward(torch.zeros(1, 8, 512), cache, tok, None, None, 64, 0.04)
    with pytest.raises(RuntimeError, match="extra_token_indices must be CUDA tensors"):
        native.dsv4_sparse_decode_forward(torch.zeros(1, 8, 512), cache, tok, None, cache, tok, None, None, 64, 1,
                                          0.04)


def test_extension_env_flags(monkeypatch):
    monkeypatch.setenv("CSAHCA_DSV4_TILE_SIZE", "17")
    assert extension._dsv4_tile_size() == 17
    monkeypatch.setenv("CSAHCA_DSV4_TILE_SIZE", "x")
    assert extension._dsv4_tile_size() == 0
    monkeypatch.setenv("CSAHCA_DSV4_TILED", "off")
    assert extension._dsv4_tiled_enabled(native) is False
    monkeypatch.setenv("CSAHCA_DSV4_TILED", "1")
    assert extension._dsv4_tiled_enabled(native) is True


def test_product_package_does_not_import_oracle():
    for p in (ROOT / "csahca_amd").rglob("*.py"):
        text = p.read_text()
        assert "import oracle" not in text and "from oracle" not in text, p


def test_reference_module_name_resolves_to_native_ops(monkeypatch):
    """`import hybrid_attention_cuda` (hybrid_attention/extension.py:19-23) finds
    the compat module, whose ops are the native bindings with the pybind names."""
    import importlib
    import sys

    monkeypatch.syspath_prepend(str(ROOT / "csahca_amd" / "compat"))
    sys.modules.pop("hybrid_attention_cuda", None)
    mod = importlib.import_module("hybrid_attention_cuda")
    for name in ("csa_decode_forward", "csa_decode_forward_tiled", "dsv4_swa_decode_forward",
                 "dsv4_sparse_decode_forward", "dsv4_decode_forward_tiled"):
        assert getattr(mod, name) is getattr(native, name)
    sys.modules.pop("hybrid_attention_cuda", None)


def test_workspace_sizes_over_the_shape_range(lib):
    """Every *_workspace_bytes function over ordinary and extreme shapes:
    negative sizes give 0, sizes grow with the shape, and no shape makes the
    host arithmetic misbehave (the sanitized build runs this under UBSan)."""
    big = 1 << 40
    for B, H, C, D, k, chunk in [(1, 8, 512, 128, 8, 64), (32, 8, 2048, 128, 32, 64), (1, 1, 1, 64, 1, 1),
                                 (0, 8, 512, 128, 8, 64), (1, 8, 0, 128, 8, 64), (-1, 8, 512, 128, 8, 64)]:
        n = lib.csahca_csa_step_workspace_bytes(B, H, C, D, k, chunk)
        assert (n == 0) == (B < 0)
        t = lib.csahca_csa_decode_workspace_bytes(B, H, D, k, chunk, 8)
        assert t >= 0
    assert lib.csahca_csa_step_workspace_bytes(1, 8, 512, 128, 8, 0) == 0
    assert lib.csahca_csa_step_workspace_bytes(32, 8, 2048, 128, 32, 64) > \
        lib.csahca_csa_step_workspace_bytes(1, 8, 512, 128, 8, 64)
    for nq, H, T, E, tile in [(1, 8, 128, 0, 0), (32, 64, 128, 64, 0), (32, 64, 600, 64, 16), (0, 8, 128, 0, 0),
                              (-1, 8, 128, 0, 0)]:
        n = lib.csahca_dsv4_decode_workspace_bytes(nq, H, T, E, tile)
        assert (n == 0) == (nq <= 0)  # no query, or a negative size: no workspace
    assert lib.csahca_hca_decode_workspace_bytes(1, 8, 32768, 128, 256) >= 8 * 128 * (1 + 128) * 4
    assert lib.csahca_csa_select_workspace_bytes(32, 8, 2048) == 32 * 8 * 2048 * 4
    for f in (lib.csahca_csa_auto_tile_size,):
        assert f(1, 8, 8, 64) > 0 and f(32, 8, 32, 64) > 0
    # sizes far past any device: the functions still return without faulting
    lib.csahca_csa_select_workspace_bytes(big, 8, 2048)
    lib.csahca_dsv4_decode_workspace_bytes(1 << 20, 64, 1 << 16, 64, 0)


def test_roctx_ranges_only_when_asked():
    """Without CSAHCA_ROCTX the ops are the undecorated functions; with
    CSAHCA_ROCTX=1 at import each op is wrapped in a roctx range named after
    it, and ranges open and close (depth 0 after the pop) without a profiler."""
    import subprocess
    import sys

    from csahca_amd import tracing

    assert not hasattr(native.csa_decode_step, "__wrapped__")
    code = ("from csahca_amd import native, tracing\n"
            "assert tracing.ENABLED and native.csa_decode_step.__wrapped__.__name__ == 'csa_decode_step'\n"
            "assert native.dsv4_decode_forward_tiled.__wrapped__ is not None\n"
            "d = tracing.push('csahca.test'); assert d >= 0, d\n"
            "assert tracing.pop() >= 0\n"
            "with tracing.op_range('csahca.block'): pass\n"
            "print('ok')\n")
    env = dict(__import__("os").environ, CSAHCA_ROCTX="1")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr[-2000:]
    with tracing.op_range("csahca.noop"):  # disabled: no library needed
        pass


def test_tensors_on_another_device_are_rejected():
    """The bindings check that every CUDA tensor of a call is on the launching
    device (the library addresses all of them from that device); CPU tensors
    are left to the ops' own is_cuda checks and messages."""
    from csahca_amd import native

    class Fake:
        def __init__(self, dev):
            self.is_cuda = dev >= 0
            self._dev = dev

        def get_device(self):
            return self._dev

    native._same_device(0, Fake(0), None, Fake(-1))
    with pytest.raises(RuntimeError, match="all tensors must be on the same device"):
        native._same_device(0, Fake(0), Fake(1))
