"""CPU models of the lane networks of the one-wavefront top-k
(csa_device.hpp): the top-8 network (wave_top8_desc) that gives the k-th
largest of 64 lane maxima for k <= 8, the full bitonic sort (wave_sort_desc)
it replaces there, and the one-pass compaction's per-lane first slots (one
ballot per bit of the lane counts, mbcnt per ballot).  The models follow the
device code's permutes lane by lane (lane_xor d = value of lane ^ d; row
mirror = lane ^ 15; half-row mirror = lane ^ 7) on uint32 lanes, and are
checked against sorting and a plain exclusive prefix sum over random inputs,
heavy ties and zeros."""
import numpy as np
import pytest

LANE = np.arange(64)


def mask(bit):
    return np.where((LANE >> bit) & 1, np.uint32(0xFFFFFFFF), np.uint32(0))


def cx_desc(x, d):
    p = x[LANE ^ d]
    return np.where(LANE & d, np.minimum(x, p), np.maximum(x, p)).astype(np.uint32)


def merge_desc(x, d):
    while d >= 1:
        x = cx_desc(x, d)
        d //= 2
    return x


def wave_sort_desc(x):
    x = x ^ mask(1)
    x = merge_desc(x, 1)
    x = x ^ mask(1) ^ mask(2)
    x = merge_desc(x, 2)
    x = x ^ mask(2) ^ mask(3)
    x = merge_desc(x, 4)
    x = x ^ mask(3) ^ mask(4)
    x = merge_desc(x, 8)
    x = x ^ mask(4) ^ mask(5)
    x = merge_desc(x, 16)
    x = x ^ mask(5)
    return merge_desc(x, 32)


def wave_top8_desc(x):
    x = x ^ mask(1)
    x = merge_desc(x, 1)
    x = x ^ mask(1) ^ mask(2)
    x = merge_desc(x, 2)
    x = x ^ mask(2)
    x = merge_desc(x, 4)
    for partner in (LANE ^ 15, (LANE ^ 7) ^ 16, (LANE ^ 7) ^ 32):
        # (lane_xor<16/32> then the half-row mirror: the value of lane (l ^ 7) ^ d)
        x = np.maximum(x, x[partner]).astype(np.uint32)
        x = merge_desc(x, 4)
    return x


def inputs():
    rng = np.random.default_rng(5)
    yield rng.integers(0, 2 ** 32, 64, dtype=np.uint64).astype(np.uint32)
    yield rng.integers(0, 4, 64).astype(np.uint32)          # heavy ties
    yield np.zeros(64, dtype=np.uint32)
    yield np.arange(64, dtype=np.uint32)                     # ascending
    yield np.arange(64, dtype=np.uint32)[::-1].copy()        # descending
    x = np.zeros(64, dtype=np.uint32)
    x[[3, 17, 40, 63]] = [9, 9, 7, 2 ** 32 - 1]               # fewer than 8 non-zero lanes
    yield x
    for s in range(200):
        r = np.random.default_rng(100 + s)
        yield r.integers(0, r.integers(2, 2 ** 31), 64).astype(np.uint32)


def test_top8_network_gives_the_eight_largest_in_every_block():
    for x in inputs():
        want = np.sort(x)[::-1][:8]
        got = wave_top8_desc(x)
        for b in range(8):
            assert np.array_equal(got[8 * b:8 * b + 8], want), (x, got)


def test_full_sort_model_sorts():
    for x in inputs():
        assert np.array_equal(wave_sort_desc(x), np.sort(x)[::-1])


@pytest.mark.parametrize("M", [8, 32])
def test_bit_sliced_prefix_gives_each_lane_its_first_slot(M):
    rng = np.random.default_rng(M)
    for trial in range(300):
        cnt = rng.integers(0, M + 1, 64) if trial % 3 else rng.integers(0, 2, 64) * M
        slot = np.zeros(64, dtype=np.int64)
        n = 0
        b = 0
        while (1 << b) <= M:
            bal = ((cnt >> b) & 1).astype(bool)
            below = np.array([bal[:l].sum() for l in range(64)])  # mbcnt: set bits of lanes below
            slot += below << b
            n += int(bal.sum()) << b
            b += 1
        assert np.array_equal(slot, np.concatenate(([0], np.cumsum(cnt)[:-1])))
        assert n == cnt.sum()
