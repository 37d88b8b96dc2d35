"""Pins the oracle's 2:4 pruning and compressed layout (the 2:4-sparse forward) before they are trusted as checkers.

xo_prune24 restates src/tools/prune24.py:43-56 (score, drop the 2 lowest of every 4 consecutive k). It is checked
against an independent numpy restatement of that script (np.argsort over the same scores, here with a stable sort:
the reference's default sort leaves ties unspecified, so the build fixes "lower k dropped first"). xo_pack24 is checked
by unpacking its output with numpy from the layout's definition and comparing with the pruned dense bytes.
"""
import numpy as np
import pytest


def _codes(rng, shape, few_values=False):
    """Random finite E4M3 codes; few_values draws from 6 magnitudes so ties are frequent."""
    if few_values:
        mags = np.array([0x00, 0x20, 0x30, 0x38, 0x40, 0x48], np.uint8)
        q = mags[rng.integers(0, len(mags), size=shape)]
    else:
        q = rng.integers(0, 0x7F, size=shape).astype(np.uint8)   # 0x00 .. 0x7E: no NaN code
    sign = rng.integers(0, 2, size=shape).astype(np.uint8) << 7
    return q | sign


def _prune_numpy(orc, q, wanda=False):
    """prune24.py:45-54 restated with numpy (stable sort: ties drop the lower k first)."""
    n, k = q.shape
    v = np.abs(orc.E4M3_LUT[q].astype(np.float64))
    score = v * v.max(0, keepdims=True) if wanda else v
    g = score.reshape(n, k // 4, 4)
    drop = np.argsort(g, axis=2, kind="stable")[:, :, :2]
    mask = np.ones_like(g, dtype=bool)
    np.put_along_axis(mask, drop, False, axis=2)
    return np.where(mask.reshape(n, k), q, 0).astype(np.uint8)


@pytest.mark.parametrize("few", [False, True])
@pytest.mark.parametrize("wanda", [False, True])
def test_prune24_matches_numpy(orc, few, wanda):
    rng = np.random.default_rng(11 + few + 2 * wanda)
    q = _codes(rng, (96, 256), few)
    assert (orc.prune24(q, wanda=wanda) == _prune_numpy(orc, q, wanda)).all()


def test_prune24_invariants(orc):
    rng = np.random.default_rng(5)
    q = _codes(rng, (64, 512), few_values=True)
    p = orc.prune24(q)
    g, gq = p.reshape(64, 128, 4), q.reshape(64, 128, 4)
    assert ((g & 0x7F) != 0).sum(2).max() <= 2                   # at most 2 nonzero bytes per group of 4
    kept = (g == gq) & (g != 0)
    v = np.abs(orc.E4M3_LUT[gq])
    dropped_max = np.where(g == 0, v, 0).max(2)
    kept_min = np.where(kept, v, np.inf).min(2)
    assert (dropped_max <= kept_min).all()                       # every kept |value| >= every dropped one
    assert (orc.prune24(p) == p).all()                           # idempotent


def test_prune24_ties_drop_lower_k_first(orc):
    q = np.zeros((1, 128), np.uint8)
    q[0, :4] = [0x38, 0x38, 0x38, 0x38]                          # all equal: k0, k1 dropped
    q[0, 4:8] = [0x40, 0x38, 0x38, 0x40]                         # 1.0 ties at k5, k6 are the two lowest
    q[0, 8:12] = [0x38, 0x40, 0xB8, 0x30]                        # |-1| ties 1.0: k8 (lower) dropped with k11
    p = orc.prune24(q)
    assert list(p[0, :12]) == [0, 0, 0x38, 0x38, 0x40, 0, 0, 0x40, 0, 0x40, 0xB8, 0]


def _unpack_numpy(vals, idx, N, K):
    """Dense [N][K] bytes from the compressed layout, by its definition (xt_oracle.h xo_pack24)."""
    out = np.zeros((N, K), np.uint8)
    for t in range(N // 16):
        for kb in range(K // 128):
            for lane in range(64):
                g, r = lane >> 4, lane & 15
                w = int(idx[t, kb, lane])
                for j in range(8):
                    p0, p1 = (w >> (4 * j)) & 3, (w >> (4 * j + 2)) & 3
                    assert p0 < p1
                    base = 128 * kb + 32 * g + 4 * j
                    out[16 * t + r, base + p0] = vals[t, kb, lane, 2 * j]
                    out[16 * t + r, base + p1] = vals[t, kb, lane, 2 * j + 1]
    return out


def test_pack24_roundtrip(orc):
    rng = np.random.default_rng(3)
    for few in (False, True):
        p = orc.prune24(_codes(rng, (32, 256), few))
        vals, idx = orc.pack24(p)
        assert (_unpack_numpy(vals, idx, 32, 256) == p).all()


def test_pack24_known_answer(orc):
    q = np.zeros((16, 128), np.uint8)
    q[0, 1], q[0, 3] = 0x38, 0x40        # group 0 of row 0 keeps positions 1, 3
    q[0, 36] = 0x30                      # lane group 1 (k 32..63), group 1: one nonzero at position 0 -> (0, 1)
    q[5, 127] = 0xC0                     # row 5, lane group 3, group 7: one nonzero at position 3 -> (0, 3)
    vals, idx = orc.pack24(q)
    assert idx[0, 0, 0] & 0xF == (1 | 3 << 2) and list(vals[0, 0, 0, :2]) == [0x38, 0x40]
    assert (idx[0, 0, 16] >> 4) & 0xF == (0 | 1 << 2) and list(vals[0, 0, 16, 2:4]) == [0x30, 0]
    assert (idx[0, 0, 48 + 5] >> 28) & 0xF == (0 | 3 << 2) and list(vals[0, 0, 48 + 5, 14:16]) == [0, 0xC0]
    assert idx[0, 0, 2] == 0x44444444                             # an all-zero row: every group keeps (0, 1)


def test_pack24_rejects_dense_groups(orc):
    q = np.zeros((16, 128), np.uint8)
    q[3, 8:11] = 0x38
    with pytest.raises(ValueError):
        orc.pack24(q)
