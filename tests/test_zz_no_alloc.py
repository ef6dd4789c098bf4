"""The allocation-free decode step (csahca_csa_decode_step_noalloc, exchange
state in a static device array) against the workspace entry point
(csahca_csa_decode_step), both called through the C ABI: bit-identical ids and
outputs on consecutive calls whose shapes shrink and grow, eagerly and under a
captured graph."""
from __future__ import annotations

import ctypes

import pytest
import torch

from csahca_amd import extension, native

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(B, H, S, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(*sh, generator=g).to(dtype).to(DEV) for sh in ((B, H, D), (B, H, S, D), (B, H, S, D)))
    return q, k, v, extension.csa_chunk_summary(k, 64)


def _outputs(q, summ, top_k):
    B, H, _ = q.shape
    k = min(top_k, summ.shape[2])
    return torch.empty_like(q), torch.empty((B, H, k), dtype=torch.int32, device=DEV)


def _noalloc(q, k, v, summ, out, idx, top_k, chunk=64):
    B, H, S, D = k.shape
    rc = native.lib().csahca_csa_decode_step_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), summ.data_ptr(), out.data_ptr(), idx.data_ptr(),
        native._DTYPES[q.dtype], B, H, S, D, summ.shape[2], chunk, top_k, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, native.lib().csahca_last_error().decode()


def _with_workspace(q, k, v, summ, top_k, chunk=64):
    B, H, S, D = k.shape
    C = summ.shape[2]
    out, idx = _outputs(q, summ, top_k)
    nbytes = native.lib().csahca_csa_step_workspace_bytes(B, H, C, D, top_k, chunk)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    rc = native.lib().csahca_csa_decode_step(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), summ.data_ptr(), out.data_ptr(), idx.data_ptr(),
        native._DTYPES[q.dtype], B, H, S, D, C, chunk, top_k, ws.data_ptr(), nbytes,
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, native.lib().csahca_last_error().decode()
    status = ctypes.c_uint32(1)
    assert native.lib().csahca_csa_step_status(ws.data_ptr(), ctypes.byref(status),
                                               torch.cuda.current_stream().cuda_stream) == 0
    assert status.value == 0
    return out, idx


CASES = [  # B, H, S, D, dtype, top_k: each call smaller, then larger again
    (4, 8, 32768, 128, torch.bfloat16, 8),
    (1, 4, 8192, 128, torch.bfloat16, 8),
    (32, 8, 131072 // 16, 64, torch.float16, 32),
    (1, 8, 131072, 128, torch.bfloat16, 32),   # 2048 chunks: the largest the scratch takes, P = 32
    (2, 2, 4096, 256, torch.float32, 5),
]


def test_noalloc_step_equals_workspace_step():
    for i, (B, H, S, D, dtype, top_k) in enumerate(CASES):
        q, k, v, summ = _inputs(B, H, S, D, dtype, seed=40 + i)
        want_out, want_idx = _with_workspace(q, k, v, summ, top_k)
        out, idx = _outputs(q, summ, top_k)
        for rep in range(2):  # the second call of a shape starts from the state the first left
            out.fill_(float("nan"))
            idx.fill_(-7)
            _noalloc(q, k, v, summ, out, idx, top_k)
            torch.cuda.synchronize()
            assert torch.equal(idx, want_idx), (i, rep)
            assert torch.equal(out, want_out), (i, rep)


def test_noalloc_step_under_graph_capture():
    q, k, v, summ = _inputs(1, 8, 32768, 128, torch.bfloat16, seed=7)
    qs, ks, vs, summ_s = _inputs(2, 4, 8192, 128, torch.bfloat16, seed=8)
    want_out, want_idx = _with_workspace(q, k, v, summ, 8)
    want_s, want_si = _with_workspace(qs, ks, vs, summ_s, 8)
    out, idx = _outputs(q, summ, 8)
    out_s, idx_s = _outputs(qs, summ_s, 8)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        _noalloc(q, k, v, summ, out, idx, 8)
    for r in range(3):
        with torch.cuda.stream(s):
            out.zero_()
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx, want_idx) and torch.equal(out, want_out), r
        with torch.cuda.stream(s):  # another shape through the same static array between replays
            _noalloc(qs, ks, vs, summ_s, out_s, idx_s, 8)
        torch.cuda.synchronize()
        assert torch.equal(idx_s, want_si) and torch.equal(out_s, want_s), r


def test_noalloc_python_wrapper_matches():
    q, k, v, summ = _inputs(1, 8, 16384, 128, torch.bfloat16, seed=9)
    want_out, want_idx = _with_workspace(q, k, v, summ, 8)
    out, idx = _outputs(q, summ, 8)
    native.csa_decode_step_noalloc(q, k, v, summ, 64, 8, out=out, indices=idx)
    torch.cuda.synchronize()
    assert torch.equal(idx, want_idx) and torch.equal(out, want_out)


def test_noalloc_timeout_poisons_until_reset(monkeypatch):
    """After an exchange time-out (forced from the host with
    CSAHCA_STEP_TEST_TIMEOUT: the last workgroup of head 0 publishes nothing,
    waits give up after 4096 polls) the static state's head slot 0 is
    poisoned: head 0 returns NaN on this and later calls, the status word read
    through csahca_csa_step_status(NULL) keeps bit 0, and the other heads are
    unaffected; csahca_csa_step_noalloc_reset clears it."""
    q, k, v, summ = _inputs(1, 8, 32768, 128, torch.bfloat16, seed=12)
    want_out, want_idx = _with_workspace(q, k, v, summ, 8)
    out, idx = _outputs(q, summ, 8)
    native.csa_step_noalloc_reset()
    assert native.csa_step_noalloc_status() == 0
    monkeypatch.setenv("CSAHCA_STEP_TEST_TIMEOUT", "4096")
    _noalloc(q, k, v, summ, out, idx, 8)
    torch.cuda.synchronize()
    monkeypatch.delenv("CSAHCA_STEP_TEST_TIMEOUT")
    for rep in range(2):
        assert torch.isnan(out[0, 0].float()).all(), rep
        assert torch.equal(out[0, 1:], want_out[0, 1:]) and torch.equal(idx[0, 1:], want_idx[0, 1:]), rep
        assert native.csa_step_noalloc_status() & 1, rep
        _noalloc(q, k, v, summ, out, idx, 8)
        torch.cuda.synchronize()
    native.csa_step_noalloc_reset()
    _noalloc(q, k, v, summ, out, idx, 8)
    torch.cuda.synchronize()
    assert torch.equal(out, want_out) and torch.equal(idx, want_idx)
    assert native.csa_step_noalloc_status() == 0


@pytest.mark.parametrize("B,H,C,D,top_k,msg", [
    (257, 1, 8, 128, 4, "batch \\* heads exceeds 256"),
    (1, 8, 2049, 128, 4, "num_chunks exceeds 2048"),
    (1, 8, 8, 512, 4, "head_dim exceeds 256"),
    (1, 8, 8, 128, 0, "needs top_k > 0"),
])
def test_noalloc_rejects_sizes_beyond_its_limits(B, H, C, D, top_k, msg):
    rc = native.lib().csahca_csa_decode_step_noalloc(None, None, None, None, None, None, native._DTYPES[torch.bfloat16],
                                                     B, H, C * 64, D, C, 64, top_k, None)
    assert rc != 0
    assert __import__("re").search(msg, native.lib().csahca_last_error().decode())
