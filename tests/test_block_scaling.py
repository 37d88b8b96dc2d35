"""Why the build drops the reference's SmoothQuant (export_eva.py:52-58, 100-110). With 1x128 activation and 128x128
weight block scales s = |max| / 448 (the reference's own scale rule, export_eva.py:64-66, applied per block), channel
outliers in the activations cost less accuracy than the reference's production scheme (SmoothQuant with alpha 0.5,
then one E4M3 scale per tensor, the activation scale from the calibrated maximum times HEADROOM 1.25), and smoothing on
top of block scales changes nothing measurable. The test also prices the power-of-two alternative (the least power of
two s with 448 s >= |max|, which a matrix core could apply as an E8M0 exponent): it is never more accurate and up to
1.4x worse where a few outliers carry the energy, which is why the build keeps exact |max| / 448 scales. The real
activation statistics are not available (the calibration file of the reference does not parse), so the test uses
synthetic activations with outlier channels of the kind SmoothQuant targets. E4M3 rounding is torch's
float8_e4m3fn cast after a +-448 clamp."""
import numpy as np
import pytest
import torch


def _q8(x):
    return torch.from_numpy(np.clip(x, -448, 448).astype(np.float32)).to(torch.float8_e4m3fn).to(torch.float32).numpy()


def _per_tensor(x, amax):
    s = amax / 448.0
    return _q8(x / s).astype(np.float64) * s


def _scale(amax, pow2):
    """|max| / 448 (the build's rule), or the least power of two at or above it (exact frexp in float64)"""
    s = np.asarray(amax, np.float64) / 448.0
    if pow2:
        m, e = np.frexp(s)
        s = np.ldexp(1.0, np.where(m == 0.5, e - 1, e))
    s[s == 0] = 1
    return s


def _act_blocks(x, pow2=False):
    M, K = x.shape
    xb = x.reshape(M, K // 128, 128)
    s = _scale(np.abs(xb).max(-1, keepdims=True), pow2)
    return (_q8(xb / s) * s).reshape(M, K).astype(np.float64)


def _w_blocks(w, pow2=False):
    N, K = w.shape
    wb = w.reshape(N // 128, 128, K // 128, 128)
    s = _scale(np.abs(wb).max((1, 3), keepdims=True), pow2)
    return (_q8(wb / s) * s).reshape(N, K).astype(np.float64)


def _smooth(a, w, alpha=0.5):
    """export_eva.py:52-58: s[k] = clip(amax_act[k]^alpha / amax_wcol[k]^(1 - alpha), 1e-3, 1e3)"""
    wa = np.abs(w).max(0)
    s = np.ones_like(a)
    ok = (a > 0) & (wa > 0)
    s[ok] = np.clip(a[ok] ** alpha / wa[ok] ** (1 - alpha), 1e-3, 1e3)
    return s


@pytest.mark.parametrize("n_out,mag", [(0, 1.0), (8, 20.0), (8, 60.0), (32, 30.0), (4, 300.0)])
def test_block_scales_vs_smoothquant(n_out, mag):
    r = np.random.default_rng(int(n_out * 1000 + mag))
    M, K, N = 1024, 1024, 512
    x = r.standard_normal((M, K)).astype(np.float32)
    x[:, r.choice(K, n_out, replace=False)] *= np.float32(mag)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T

    def err(y):
        return np.linalg.norm(y - ref) / np.linalg.norm(ref)
    s = _smooth(np.abs(x).max(0), w)
    xs, ws = x / s, w * s
    e_ref = err(_per_tensor(xs, 1.25 * np.abs(xs).max()) @ _per_tensor(ws, np.abs(ws).max()).T)
    e_blk = err(_act_blocks(x) @ _w_blocks(w).T)
    e_blk_sq = err(_act_blocks(xs) @ _w_blocks(ws).T)
    e_pow2 = err(_act_blocks(x, True) @ _w_blocks(w, True).T)
    print(f"outliers {n_out} x{mag}: SmoothQuant + per-tensor {e_ref:.4f}, |max| / 448 blocks {e_blk:.4f}, "
          f"+ SmoothQuant {e_blk_sq:.4f}, power-of-two blocks {e_pow2:.4f}")
    assert e_blk <= 1.02 * e_ref
    assert abs(e_blk_sq - e_blk) <= 0.05 * e_blk
    assert e_blk <= e_pow2 <= 1.5 * e_blk
