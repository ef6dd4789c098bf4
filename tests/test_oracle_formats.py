"""Pin the oracle's scalar formats against torch's own casts (library routines).

e4m3fn decode: all 256 codes.  e4m3fn encode: every representable value, every
midpoint between neighbours (ties to even), values just either side of each
midpoint, the overflow boundary (448 / 464 / 480) and a dense log-uniform sweep.
bf16 / f16 rounding: random fp32 patterns including exact ties.
"""
import math

import numpy as np
import torch

import oracle


def torch_e4m3_bytes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3fn_decode_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    want = codes.view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.e4m3fn_decode(b) for b in range(256)], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(nan, np.isnan(got))
    assert nan.sum() == 2  # 0x7F and 0xFF
    assert np.array_equal(got[~nan], want[~nan])
    assert oracle.e4m3fn_decode(0x7E) == 448.0
    assert oracle.e4m3fn_decode(0x01) == 2.0 ** -9


def _finite_values():
    vals = np.array([oracle.e4m3fn_decode(b) for b in range(128)], dtype=np.float64)
    vals = np.sort(vals[~np.isnan(vals)])
    return vals


def test_e4m3fn_encode_matches_torch_on_boundaries():
    vals = _finite_values()
    mids = (vals[:-1] + vals[1:]) / 2.0
    probes = [vals, mids]
    for m in mids:
        probes.append(np.array([np.nextafter(np.float32(m), np.float32(-np.inf)),
                                np.nextafter(np.float32(m), np.float32(np.inf))]))
    probes.append(np.array([447.9, 448.0, 455.0, 463.99, 464.0, 464.01, 470.0, 479.99, 480.0, 500.0, 1e6, 0.0,
                            1e-30, 2.0 ** -10, 2.0 ** -10 + 1e-12, 3 * 2.0 ** -10]))
    x = np.concatenate(probes).astype(np.float32)
    x = np.concatenate([x, -x])
    got = oracle.e4m3fn_encode_array(x)
    want = torch_e4m3_bytes(x)
    assert np.array_equal(got, want), np.nonzero(got != want)


def test_e4m3fn_encode_matches_torch_dense():
    rng = np.random.default_rng(0)
    mag = np.exp(rng.uniform(math.log(1e-5), math.log(600.0), 400_000))
    x = (mag * rng.choice([-1.0, 1.0], mag.size)).astype(np.float32)
    assert np.array_equal(oracle.e4m3fn_encode_array(x), torch_e4m3_bytes(x))


def test_round_bf16_f16_match_torch():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    # exact ties for bf16: low 16 bits == 0x8000
    ties = ((rng.integers(0, 2 ** 16, 4096, dtype=np.uint32) << 16) | 0x8000).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, ties[np.isfinite(ties)], rng.standard_normal(10000).astype(np.float32)])
    got = oracle.round_to(x, torch.bfloat16)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    y = (rng.standard_normal(100_000) * np.exp(rng.uniform(-20, 12, 100_000))).astype(np.float32)
    got = oracle.round_to(y, torch.float16)
    want = torch.from_numpy(y).to(torch.float16).float().numpy()
    assert np.array_equal(got, want)
