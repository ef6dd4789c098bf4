"""CPU models of the two transposed cross-lane reductions of the CSA kernels
(common.hpp transposed_group_sum, csa_device.hpp fold_groups_t): a lane holds N
values; every exchange at distance d sends one half of them to lane ^ d and adds
the partner's half to the other, so the values a lane holds halve per step.
The models follow the device code's exchange schedule on 64 float32 lanes and
check that the sums carry exactly the bits of the butterfly reduction (every
value summed over all its lanes at the same distances, in the same order),
and which row or column each lane ends with -- for every (N, L) and
(VEC, LPR) the kernels instantiate.  Bit identity is what keeps the chunk
scores, and so the selected chunks, the same as the butterfly's."""
import numpy as np
import pytest

LANE = np.arange(64)


def butterfly(v, dists):
    b = v.copy()
    for d in dists:
        b = (b + b[LANE ^ d]).astype(np.float32)
    return b


def halving_step(v, m, d):
    """One exchange at distance d on the first m values of each lane: lanes with
    bit d set keep the upper half and send the lower, the others the reverse."""
    h = m // 2
    up = (LANE & d) != 0
    out = v.copy()
    for i in range(h):
        send = np.where(up, v[:, i], v[:, i + h]).astype(np.float32)
        keep = np.where(up, v[:, i + h], v[:, i]).astype(np.float32)
        out[:, i] = (keep + send[LANE ^ d]).astype(np.float32)
    return out, up


@pytest.mark.parametrize("N,L", [(8, 32), (8, 16), (8, 64), (4, 16), (1, 32), (2, 2), (16, 32)])
def test_transposed_group_sum_matches_the_butterfly(N, L):
    """Rows of L lanes, N rows per lane group: exchanges at L/2, L/4, ... while
    a lane holds more than one value, then plain butterfly steps; lane l ends
    with the sum of row (l % L) / (L / N)."""
    rng = np.random.default_rng(N * 100 + L)
    for _ in range(100):
        v = (rng.standard_normal((64, N)) * 10 ** rng.uniform(-3, 3)).astype(np.float32)
        want = butterfly(v, [L >> s for s in range(1, L.bit_length())])
        t, m, d = v.copy(), N, L // 2
        while m > 1:
            t, _ = halving_step(t, m, d)
            m //= 2
            d //= 2
        s = t[:, 0].copy()
        while d >= 1:
            s = (s + s[LANE ^ d]).astype(np.float32)
            d //= 2
        row = (LANE % L) // (L // N)
        assert np.array_equal(s.view(np.uint32), want[LANE, row].view(np.uint32))


@pytest.mark.parametrize("VEC,LPR", [(8, 16), (8, 8), (8, 32), (4, 32), (4, 16), (4, 64)])
def test_transposed_row_group_fold_matches_the_butterfly(VEC, LPR):
    """The attention state's row groups (64 / LPR groups of LPR lanes, VEC
    columns a lane): exchanges at ascending distances LPR, 2 LPR, ..., 32 halve
    the columns a lane holds while it holds more than one; each lane ends with
    max(1, VEC * LPR / 64) column sums, and every (column, lane-column) pair is
    held by exactly one lane."""
    rng = np.random.default_rng(VEC * 100 + LPR)
    keep_n = max(1, VEC // (64 // LPR))
    for _ in range(100):
        acc = (rng.standard_normal((64, VEC)) * 10 ** rng.uniform(-3, 3)).astype(np.float32)
        want = butterfly(acc, [LPR << s for s in range(0, 64) if (LPR << s) < 64])
        v, base, m, off = acc.copy(), np.zeros(64, int), VEC, LPR
        while off < 64:
            if m > 1:
                v, up = halving_step(v, m, off)
                base += np.where(up, m // 2, 0)
                m //= 2
            else:
                v[:, 0] = (v[:, 0] + v[LANE ^ off, 0]).astype(np.float32)
            off *= 2
        for e in range(keep_n):
            assert np.array_equal(v[:, e].view(np.uint32), want[LANE, base + e].view(np.uint32))
        cover = {}
        for lane in range(64):
            for e in range(keep_n):
                cover.setdefault((lane % LPR, base[lane] + e), []).append(lane)
        assert len(cover) == LPR * VEC and all(len(x) == 1 for x in cover.values())


def test_a_wrong_exchange_order_is_caught():
    """Planted mistake: swapping which half a lane keeps changes the row a lane
    ends with, which the mapping check above would reject."""
    v = np.arange(64 * 8, dtype=np.float32).reshape(64, 8)
    t, m, d = v.copy(), 8, 16
    while m > 1:
        h = m // 2
        up = (LANE & d) == 0  # reversed
        out = t.copy()
        for i in range(h):
            send = np.where(up, t[:, i], t[:, i + h])
            keep = np.where(up, t[:, i + h], t[:, i])
            out[:, i] = keep + send[LANE ^ d]
        t, m, d = out, h, d // 2
    s = t[:, 0]
    while d >= 1:
        s = s + s[LANE ^ d]
        d //= 2
    want = butterfly(v, [16, 8, 4, 2, 1])
    row = (LANE % 32) // 4
    assert not np.array_equal(s, want[LANE, row])
