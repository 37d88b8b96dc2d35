"""Comparing block scales that come from a GEMM-fed maximum (fc1's repack, PixAI fc1's repack).

A block scale is the least power of two s with 448 s >= |max| of its 128 values. Where the oracle's block maximum
lies within about 1e-4 of a boundary 448 * 2^k, the matrix core's summation (which differs from fp64 by ~1e-5
relative) can move the kernel's maximum to the other side, and its scale is then exactly 2x or 0.5x the oracle's:
a different, equally valid packing of the same block. These helpers accept exactly that and nothing else."""
import numpy as np


def blocks_agree(got_s, ref_s, ref_amax=None, got_codes=None, ref_codes=None, decode=None, rel=1e-4):
    """got_s, ref_s: scale planes [nblk][M]. A block whose scales differ must differ by exactly 2x, with
    - ref_amax [nblk][M] given: the reference maximum within rel of 448 times the smaller scale, or
    - got_codes / ref_codes [M][128 nblk] and decode given: the larger scale's block maximum decoding to 224 or 240
      (448 s_small / s_big, rounded) and the smaller one's to 416 or 448.
    Returns the mask [nblk][M] of blocks whose scales are equal."""
    got_s = np.asarray(got_s, np.float64)
    ref_s = np.asarray(ref_s, np.float64)
    eq = got_s == ref_s
    if eq.all():
        return eq
    ratio = got_s[~eq] / ref_s[~eq]
    assert np.isin(ratio, (0.5, 2.0)).all(), "block scales differ by more than one binade"
    lo = np.minimum(got_s, ref_s)
    if ref_amax is not None:
        edge = np.abs(np.asarray(ref_amax, np.float64) / (448.0 * lo) - 1.0) <= rel
        assert edge[~eq].all(), "block scales differ away from a power-of-two boundary"
    else:
        M = got_s.shape[1]
        gmax = np.abs(decode(got_codes)).reshape(M, -1, 128).max(2).T
        rmax = np.abs(decode(ref_codes)).reshape(M, -1, 128).max(2).T
        big = np.where(got_s > ref_s, gmax, rmax)[~eq]
        small = np.where(got_s > ref_s, rmax, gmax)[~eq]
        assert np.isin(big, (224.0, 240.0)).all() and np.isin(small, (416.0, 448.0)).all(), \
            "block scales differ away from a power-of-two boundary"
    return eq


def block_amax(h, nblk):
    """|max| of each 128-wide block of h [M][>= 128 nblk], as a plane [nblk][M]."""
    h = np.asarray(h, np.float64)
    return np.abs(h[:, :128 * nblk]).reshape(h.shape[0], nblk, 128).max(2).T


def codes_differing(got_codes, ref_codes, eq):
    """Fraction of E4M3 codes that differ, over the blocks whose scales agree (eq [nblk][M])."""
    nblk = eq.shape[0]
    g = got_codes[:, :128 * nblk]
    r = ref_codes[:, :128 * nblk]
    mask = np.repeat(eq.T, 128, 1)
    return float(np.mean(g[mask] != r[mask])) if mask.any() else 0.0
