"""CPU pins of the oracle's patch-operand producer (oracle/xt_img.c, a restatement of src/core/procimg.h:592-969).

The reference ships no test or fixture for this path. The restatement is pinned here by what fixes it independently:
  - the resample against PIL's own antialiased bicubic (Image.resize(BICUBIC) in float mode "F": the same Keys cubic,
    a = -0.5, with support 2 * max(scale, 1) and centres (i + 0.5) * scale) of the white-padded square, which catches a
    wrong centre, offset, support, axis or channel;
  - the identity path (side == S) in closed form, v / 127.5 - 1 rounded once (one fma) then to fp16;
  - the divide-by-255 of alpha over white exhaustively against round(x / 255);
  - the 2x2 pyramid against its exact mean (|level - mean| < 1, constant images stay constant, sizes per pi_pyramid);
  - the axis weights by their normalisation (taps plus white taps sum to the scale).
"""
import numpy as np
import pytest

S = 448


def _f16(bits):
    return bits.view(np.float16).astype(np.float32)


def _planes(out, S=S):
    """[(S/14)^2][592] -> [3][S][S] (B, G, R) in pixel order (procimg.h:1606-1607 jo[] and the 14-row bands)."""
    n = S // 14
    t = out[:, :588].reshape(n, n, 3, 14, 14)                 # patch row, patch col, plane, ky, kx
    return t.transpose(2, 0, 3, 1, 4).reshape(3, S, S)


def _pil_ref(crop, S=S):
    """PIL float bicubic of the crop centred on a white square of side max(cw, ch), per channel R G B."""
    from PIL import Image
    ch, cw = crop.shape[:2]
    side = max(cw, ch)
    sq = np.full((side, side, 3), 255.0, np.float32)
    oy, ox = (side - ch) >> 1, (side - cw) >> 1
    sq[oy:oy + ch, ox:ox + cw] = crop[..., :3]
    chans = [np.asarray(Image.fromarray(sq[..., c], "F").resize((S, S), Image.BICUBIC)) for c in range(3)]
    return np.stack(chans)                                     # [3][S][S], R G B


def _img(h, w, seed):
    r = np.random.default_rng(seed)
    # smooth content plus noise: both the low and the high frequencies are exercised
    yy, xx = np.mgrid[0:h, 0:w]
    base = 127.5 + 100 * np.sin(xx[..., None] / (7.0 + np.arange(4)) + yy[..., None] / 11.0)
    img = np.clip(base + r.normal(0, 20, (h, w, 4)), 0, 255).astype(np.uint8)
    img[..., 3] = 255
    return img


@pytest.mark.parametrize("h,w,crop", [(900, 1300, (100, 50, 1100, 800)),   # downscale 2.46x, landscape
                                      (700, 520, (10, 20, 500, 660)),       # downscale 1.47x, portrait
                                      (300, 260, (0, 0, 260, 300)),         # upscale 1.49x
                                      (1000, 1000, (0, 0, 999, 1000))])     # downscale just above 2x
def test_resample_matches_pil_bicubic(orc, h, w, crop):
    img = _img(h, w, 3)
    x0, y0, cw, ch = crop
    out, (L, *_) = orc.img_prep([img], x0, y0, cw, ch, S)
    assert L == 0
    got = _planes(_f16(out)) * 127.5 + 127.5                   # B G R in 0..255
    ref = np.clip(_pil_ref(img[y0:y0 + ch, x0:x0 + cw]), 0, 255)[::-1]
    d = np.abs(got - ref)
    # fp16 of values in [-1, 1] is within 2^-11 relative (0.07 of 255 units); PIL sums horizontally first, in double
    assert d.max() < 0.15, d.max()
    assert d.mean() < 0.02
    assert (out[:, 588:] == 0).all()


def test_identity_path_closed_form(orc):
    img = _img(600, 500, 5)
    x0, y0, cw, ch = 30, 40, 300, S                            # side == S: no resample, white padding left and right
    out, (L, x, y, cw2, ch2) = orc.img_prep([img], x0, y0, cw, ch, S)
    assert (L, cw2, ch2) == (0, cw, ch)
    got = _planes(out)
    ox = (S - cw) >> 1
    c = np.float64(np.float32(1.0 / 127.5))
    v = img[y0:y0 + ch, x0:x0 + cw, :3].astype(np.float64)
    exact = np.float32(v * c - 1.0).astype(np.float16).view(np.uint16)   # one fma, then fp16 (both RNE)
    for p in range(3):
        assert (got[p][:, ox:ox + cw] == exact[..., 2 - p]).all()
        assert (got[p][:, :ox] == 0x3C00).all() and (got[p][:, ox + cw:] == 0x3C00).all()


def test_div255_exhaustive(orc):
    x = np.arange(0, 255 * 255 + 1, dtype=np.int64)
    div = (x + 128 + ((x + 128) >> 8)) >> 8                      # the macro as the oracle states it
    assert (div == np.floor(x / 255.0 + 0.5)).all()
    r = np.random.default_rng(1)
    rgba = r.integers(0, 256, (64, 80, 4), dtype=np.uint8)
    rgba[0, :, 3] = 255
    rgba[1, :, 3] = 0
    o = orc.img_over_white(rgba)
    a = rgba[..., 3:4].astype(np.float64)
    ref = np.floor((rgba[..., :3] * a + 255 * (255 - a)) / 255.0 + 0.5)
    assert (o[..., :3] == ref).all() and (o[..., 3] == 255).all()
    assert (o[0, :, :3] == rgba[0, :, :3]).all() and (o[1, :, :3] == 255).all()


def test_pyramid_levels(orc):
    img = _img(2000, 3100, 7)
    lv = orc.img_pyramid(img, S)
    assert [l.shape[:2] for l in lv] == [(2000, 3100), (1000, 1550)]   # the next long side, 775, is under 2 S
    for a, b in zip(lv, lv[1:]):
        h, w = b.shape[:2]
        blk = a[:2 * h, :2 * w].astype(np.float64).reshape(h, 2, w, 2, 4)
        mean = blk.mean(axis=(1, 3))
        assert np.abs(b - mean).max() < 1.0
        assert (b >= blk.min(axis=(1, 3))).all() and (b <= blk.max(axis=(1, 3))).all()
    flat = np.full((1800, 1800, 4), 77, np.uint8)
    assert all((l == 77).all() for l in orc.img_pyramid(flat, S))
    # the level choice leaves a resample factor in [2, 4) once the pyramid reaches that far
    out, (L, x0, y0, cw, ch) = orc.img_prep(lv, 0, 0, 3100, 2000, S)
    assert L == 1 and 2 <= max(cw, ch) / S < 4


@pytest.mark.parametrize("side,off,length", [(1100, 150, 800), (300, 20, 260), (448, 0, 448), (1792, 0, 1792)])
def test_axis_weights_normalised(orc, side, off, length):
    for sc, add in ((1.0, 0.0), (np.float32(1 / 127.5), -1.0)):
        w, s, n, k = orc.img_axis(S, side, off, length, sc, add)
        tot = np.array([w[i, :n[i]].astype(np.float64).sum() for i in range(S)]) + (k - add) / 255.0
        assert np.abs(tot / sc - 1).max() < 1e-5
        assert (s >= 0).all() and (s + n <= length)[n > 0].all()      # taps stay inside the content
