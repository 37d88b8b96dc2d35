"""eva_img_prep_static, the patch-operand producer with no allocation and no scratch argument, against eva_img_prep (the
same kernels with a caller-given scratch) through the C-ABI: two calls in a row, the second on a smaller rect, each
bit-identical to eva_img_prep on the same rect; a rect needing more than EVA_IMG_STATIC_BYTES fails with -1; a rect at
the model side (the identity path, no staging) matches too."""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

S = 448
STATIC_BYTES = 448 * (4 * 448 - 1) * 16


def _st():
    return torch.cuda.current_stream().cuda_stream


def _pyramid(xt, dev, h, w, seed):
    r = np.random.default_rng(seed)
    stride = w * 4
    img = r.integers(0, 256, (h, stride), dtype=np.uint8)
    img.reshape(h, w, 4)[..., 3] = 255
    l0 = torch.from_numpy(img).to(dev)
    p = xt.EvaPyr()
    p.lv[0], p.ls[0], p.lw[0], p.lh[0] = l0.data_ptr(), stride, w, h
    nb = xt.lib.eva_img_pyramid_bytes(w, h, S)
    levels = torch.empty(max(nb, 32), dtype=torch.uint8, device=dev)
    assert xt.lib.eva_img_pyramid(C.byref(p), xt.ptr(levels), nb, S, _st()) == 0
    torch.cuda.synchronize()
    return p, (l0, levels)


def test_img_prep_static_matches_scratch_entry_point(dev, xt):
    p, keep = _pyramid(xt, dev, 2048, 3072, 5)
    scratch = torch.empty(xt.lib.eva_img_prep_bytes(S, 4 * S - 1), dtype=torch.uint8, device=dev)
    out_ref = torch.zeros(1024 * 592, dtype=torch.int16, device=dev)
    out = torch.zeros_like(out_ref)
    # full view (level 1: a 1536 x 1024 rect, 11 MB of staging), then a smaller 900 x 700 crop (level 0)
    for rect in ((0, 0, 3072, 2048), (300, 200, 900, 700)):
        print("rect", rect, flush=True)
        assert xt.lib.eva_img_prep(C.byref(p), *rect, S, xt.ptr(scratch), scratch.numel(), xt.ptr(out_ref), _st()) == 0
        assert xt.lib.eva_img_prep_static(C.byref(p), *rect, S, xt.ptr(out), _st()) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, out_ref), rect
        out.zero_()
    # the identity path (long side S on level 0) stages nothing
    rect = (10, 20, S, 300)
    assert xt.lib.eva_img_prep(C.byref(p), *rect, S, xt.ptr(scratch), scratch.numel(), xt.ptr(out_ref), _st()) == 0
    assert xt.lib.eva_img_prep_static(C.byref(p), *rect, S, xt.ptr(out), _st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref)


def test_img_prep_static_rejects_rects_past_its_maximum(dev, xt):
    # at S = 1008 a 3000-wide rect stays on level 0 (3000 < 2 x 2 x 1008) and needs 1008 x 3000 x 16 bytes of staging
    p, keep = _pyramid(xt, dev, 2000, 3000, 6)
    assert 1008 * 3000 * 16 > STATIC_BYTES
    out = torch.zeros(72 * 72 * 592, dtype=torch.int16, device=dev)
    assert xt.lib.eva_img_prep_static(C.byref(p), 0, 0, 3000, 2000, 1008, xt.ptr(out), _st()) == -1
    torch.cuda.synchronize()
