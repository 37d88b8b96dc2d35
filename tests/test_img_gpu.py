"""GPU parity of the patch-operand producer (eva_img_*: src/core/procimg.h:592-969 on the GPU) against the oracle
(oracle/xt_img.c, itself pinned against PIL's bicubic and closed forms in test_img_oracle.py). Bit-exact: the same
integer formulas for alpha over white and the pyramid, the same float operations for the tap tables, one fma per tap in
tap order, fp16 round-to-nearest-even."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

S = 448


def _say(*a):
    print(*a, flush=True)


def _st():
    return torch.cuda.current_stream().cuda_stream


def _img(h, w, seed, alpha=False):
    r = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h, 0:w]
    base = 127.5 + 110 * np.sin(xx[..., None] / (5.0 + np.arange(4)) + yy[..., None] / 9.0)
    img = np.clip(base + r.normal(0, 30, (h, w, 4)), 0, 255).astype(np.uint8)
    if not alpha:
        img[..., 3] = 255
    return img


class DevImage:
    """Level 0 on the device (rows padded to a 64-byte stride, as a decoder would leave them) and its pyramid."""

    def __init__(self, xt, dev, img):
        h, w = img.shape[:2]
        self.stride = (w * 4 + 63) // 64 * 64
        buf = np.zeros((h, self.stride), np.uint8)
        buf[:, :w * 4] = img.reshape(h, w * 4)
        self.l0 = torch.from_numpy(buf).to(dev)
        self.p = xt.EvaPyr()
        self.p.lv[0], self.p.ls[0], self.p.lw[0], self.p.lh[0] = self.l0.data_ptr(), self.stride, w, h
        nb = xt.lib.eva_img_pyramid_bytes(w, h, S)
        self.levels = torch.empty(max(nb, 32), dtype=torch.uint8, device=dev)
        rc = xt.lib.eva_img_pyramid(C.byref(self.p), xt.ptr(self.levels), nb, S, _st())
        assert rc == 0
        torch.cuda.synchronize()

    def level(self, L):
        w, h, ls = self.p.lw[L], self.p.lh[L], self.p.ls[L]
        if L == 0:
            a = self.l0.cpu().numpy()
        else:
            off = self.p.lv[L] - self.levels.data_ptr()
            a = self.levels[off:off + ls * h].cpu().numpy().reshape(h, ls)
        return np.ascontiguousarray(a[:, :w * 4].reshape(h, w, 4))


def test_over_white_bitexact(dev, xt, orc):
    img = _img(37, 301, 1, alpha=True)
    img[0, :, 3] = 0
    img[1, :, 3] = 255
    d = torch.from_numpy(img.copy()).to(dev)
    assert xt.lib.eva_img_over_white(xt.ptr(d), 301 * 4, 301, 37, _st()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), orc.img_over_white(img))


@pytest.mark.parametrize("h,w", [(2000, 3100), (1900, 901), (500, 400)])
def test_pyramid_bitexact(dev, xt, orc, h, w):
    img = _img(h, w, 2)
    di = DevImage(xt, dev, img)
    ref = orc.img_pyramid(img, S)
    assert di.p.nlv == len(ref)
    for L in range(1, len(ref)):
        assert np.array_equal(di.level(L), ref[L]), f"level {L}"


# (image h, w, level-0 crop x0, y0, cw, ch): level 1 downscale, level 0 downscale, upscale, identity (side == S),
# portrait, a crop clipped at the image edge, a thin strip, and a crop that lands exactly on S at level 1
CASES = [(2000, 3100, (0, 0, 3100, 2000)), (2000, 3100, (700, 300, 1500, 1200)), (900, 700, (50, 60, 600, 800)),
         (300, 260, (0, 0, 260, 300)), (600, 500, (30, 40, 300, 448)), (2000, 3100, (2900, 1800, 900, 900)),
         (1200, 1300, (100, 500, 1150, 60)), (2000, 3100, (0, 0, 896, 896))]


@pytest.mark.parametrize("h,w,crop", CASES)
def test_prep_bitexact(dev, xt, orc, h, w, crop):
    img = _img(h, w, 3)
    di = DevImage(xt, dev, img)
    ref, (L, x0, y0, cw, ch) = orc.img_prep(orc.img_pyramid(img, S), *crop, S=S)
    _say(f"crop {crop} -> level {L} rect {x0, y0, cw, ch}")
    nb = xt.lib.eva_img_prep_bytes(S, 4 * S - 1)
    scratch = torch.empty(nb, dtype=torch.uint8, device=dev)
    out = torch.full(((S // 14) ** 2, 592), 0x7E00, dtype=torch.int16, device=dev)   # NaN bits: all must be written
    rc = xt.lib.eva_img_prep(C.byref(di.p), *crop, S, xt.ptr(scratch), nb, xt.ptr(out), _st())
    assert rc == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    diff = got != ref
    assert not diff.any(), f"{diff.sum()} halves differ, first at {np.argwhere(diff)[0]}"


def test_prep_feeds_engine(dev, xt, orc, tmp_path):
    """Crops produced on the GPU straight into the engine's device input buffer (eva_dev_input) give the same scores
    as the same crops produced by the oracle on the CPU and submitted through eva_submit (the reference's path)."""
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path = str(tmp_path / "eva02_synth_v2.bin")
    blob.write_v2(path, blob.synth_model(seed=0, nt=10861))
    img = _img(2000, 3100, 4)
    crops = [(0, 0, 3100, 2000), (900, 400, 1000, 1000)]
    lv = orc.img_pyramid(img, S)
    host = np.stack([orc.img_prep(lv, *c, S=S)[0] for c in crops]).view(np.float16)
    e = Engine(path, device=0, nb=2)
    e.ready()
    e.submit(0, host)
    ref = e.wait(0, 2)
    di = DevImage(xt, dev, img)
    nb = xt.lib.eva_img_prep_bytes(S, 4 * S - 1)
    scratch = torch.empty(nb, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    din, st = e.dev_input(), e.stream()
    for k, c in enumerate(crops):   # on the engine's stream, ahead of its forward
        assert xt.lib.eva_img_prep(C.byref(di.p), *c, S, xt.ptr(scratch), nb, C.c_void_p(din + k * 1024 * 592 * 2), st) == 0
    e.run()
    e.sync()
    hip = C.CDLL("libamdhip64.so")
    got = np.empty((2, e.nt), np.float32)
    assert hip.hipMemcpy(C.c_void_p(got.ctypes.data), C.c_void_p(e.dev_output()), C.c_size_t(got.nbytes), 2) == 0
    e.close()
    assert np.array_equal(got, ref)
