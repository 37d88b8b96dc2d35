"""Full wd forward on the GPU against the oracle, on a synthetic random-init blob in the reference's v2 format.

1. Teacher-forced parity: every kernel of the 24-layer forward (7 per layer, plus embed, pool, final LN, head) is
   recomputed by the oracle from the GPU's own inputs to that step: LayerNorm packing, final LN and pool bit-exact;
   GEMM-fed epilogues within one output rounding unit plus 2e-4 of the terms; attention within 4e-3; the head's
   sigmoid scores within 1e-4 (the contract asks 2e-3) with identical top-50 tag sets.
2. The engine (eva_open .. eva_wait, one HIP graph replay) returns exactly the scores of that validated sequence.
   With 2:4-sparse weights (EVA_SPARSE24) the same holds against the oracle with the same pruned
   weights (its "dense-decoded reference"), and the sparse engine's graph returns that validated sequence's bits.
3. Free running, the GPU and the oracle drift apart through the per-layer E4M3 re-quantization exactly as the oracle
   drifts from itself when only its fp32 summation order changes (tests/golden/forward_self_divergence.json); the
   GPU's drift is held to 2x that envelope, with a top-50 overlap within 6 tags of the oracle's overlap with itself.
   The strict 2e-3 bound cannot hold free running for any implementation
   whose sums are ordered differently from the oracle's: the oracle against itself breaks it (0.053).
"""
import json
import os
from collections import defaultdict

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

T, D, HIDP = 1025, 1024, 2816
HERE = os.path.dirname(os.path.abspath(__file__))


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def synth_blob(tmp_path_factory):
    from xtagger_amd import blob
    path = str(tmp_path_factory.mktemp("blob") / "eva02_synth_v2.bin")
    _say("writing synthetic v2 blob")
    blob.write_v2(path, blob.synth_model(seed=0, nt=10861))
    return path, blob.read_v2(path)


def _f16(u):
    return np.asarray(u).view(np.uint16).view(np.float16).astype(np.float64)


def _bf16(u):
    return (np.asarray(u).view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


class OracleCheck:
    """Recomputes each step with the oracle from the GPU's inputs; records the worst error / bound per step kind."""

    def __init__(self, orc, m, inp, nb, sparse=False):
        self.orc, self.m, self.inp, self.nb, self.sparse = orc, m, inp, nb, sparse
        self.M = nb * T
        self.worst = defaultdict(float)
        self._w = (None, None)

    def weights(self, i):
        if self._w[0] == i:
            return self._w[1]
        orc, L = self.orc, self.m["layers"][i]
        W = {}
        pr = (lambda qs: (orc.prune24(qs[0]), qs[1])) if self.sparse else (lambda qs: qs)
        W["qkv"] = pr(orc.quant_w(L["wqkv"].astype(np.float32)))
        W["wo"] = pr(orc.quant_w(L["wo"].astype(np.float32)))
        w12 = np.zeros((2 * HIDP, D), np.float32)
        w12[:2 * 2736] = L["w12"].astype(np.float32)
        W["w12"] = pr(orc.quant_w(w12))
        wt, dd = orc.fold_w2(L["w2"].view(np.uint16), L["mlnw"], L["mlnb"])
        W["w2"] = pr(orc.quant_w(wt))
        W["c"], W["d"] = orc.fold_c(*W["w2"]), dd
        self._w = (i, W)
        return W

    def close(self, name, got, ref, scale, unit):
        err = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
        bound = unit * np.abs(ref) + 2e-4 * scale
        w = float((err / bound).max())
        self.worst[name] = max(self.worst[name], w)
        assert w <= 1.0, f"{name}: err / bound {w:.3f}"

    def __call__(self, step, i, g):
        orc, m, nb, M = self.orc, self.m, self.nb, self.M
        if step == "pe":
            ref = orc.embed(self.inp.view(np.uint16), m["pe"].view(np.uint16), m["pos"], nb)
            self.close("embed", _f16(g["x"]), _f16(ref), np.abs(_f16(ref)).max(), 2.0 ** -10)
            return
        if step in ("ln1", "ln2"):
            L = m["layers"][i]
            w, b = (L["ln1w"], L["ln1b"]) if step == "ln1" else (L["ln2w"], L["ln2b"])
            q, s, _ = orc.ln_quant(g["x"].view(np.uint16), w, b)
            assert np.array_equal(g["h8"], q) and np.array_equal(g["sh"], s), f"{step} layer {i} packing differs"
            self.worst["ln (bit-exact)"] = 0.0
            return
        W = self.weights(i) if i < 24 else None
        if step == "qkv":
            acc = orc.gemm_f32(g["h8"], g["sh"], *W["qkv"], 3 * D)
            q, k, vt = orc.qkv_epi(acc, nb, m["rope"])
            sc = np.abs(acc).max()
            for nm, got, ref in (("q", g["q"], q), ("k", g["k"], k), ("vt", g["vt"], vt)):
                self.close("qkv+rope " + nm, _bf16(got), _bf16(ref), sc, 2.0 ** -7)
        elif step == "flash":
            ref = orc.attention(g["q"].view(np.uint16), g["k"].view(np.uint16), g["vt"].view(np.uint16), nb)
            err = np.abs(g["o32"] - ref)
            w = float(err.max() / (4e-3 * np.abs(ref).max()))
            self.worst["attention"] = max(self.worst["attention"], w)
            assert w <= 1.0, f"attention layer {i}"
            q8, s8 = orc.quant_act(g["o32"])
            assert np.array_equal(g["h8"], q8) and np.array_equal(g["sh"], s8), f"attention packing layer {i}"
        elif step == "oproj":
            acc = orc.gemm_f32(g["h8"], g["sh"], *W["wo"], D)
            ref = orc.oproj_epi(acc, g["x_in"].view(np.uint16))
            self.close("oproj+residual", _f16(g["x"]), _f16(ref), np.abs(acc).max(), 2.0 ** -10)
        elif step == "fc1":
            acc = orc.gemm_f32(g["h8"], g["sh"], *W["w12"], 2 * HIDP)
            hf, stat = orc.fc1_epi(acc)
            q, s = orc.quant_act(hf)
            frac = float(np.mean(g["m8"] != q))
            self.worst["fc1 codes differing (frac)"] = max(self.worst["fc1 codes differing (frac)"], frac)
            assert frac < 2e-3, f"fc1 layer {i}: {frac:.2e} of codes differ"
            # the block scale is one GEMM-fed maximum over 128 units: the matrix core's sum moves it by ~1e-5
            sdev = float(np.abs(g["sm"] / s - 1).max())
            self.worst["fc1 block scale rel"] = max(self.worst["fc1 block scale rel"], sdev)
            assert sdev < 1e-3
            dq = orc.e4m3_decode(g["m8"]) * np.repeat(g["sm"].T, 128, 1)
            self.close("fc1+swiglu (dequantized)", dq, hf, np.abs(hf).max(), 2.0 ** -3)
            self.close("fc1 row sums", g["stat"][..., 0], stat[..., 0], np.abs(stat[..., 1]).max() ** 0.5, 0.0)
            self.close("fc1 row sums of squares", g["stat"][..., 1], stat[..., 1], np.abs(stat[..., 1]).max(), 0.0)
        elif step == "fc2":
            acc = orc.gemm_f32(g["m8"], g["sm"], *W["w2"], D)
            ref = orc.fc2_epi(acc, g["stat"], W["c"], W["d"], g["x_in"].view(np.uint16))
            S, Q = g["stat"][..., 0].sum(0), g["stat"][..., 1].sum(0)
            mean = S / 2730.0
            rstd = 1.0 / np.sqrt(np.maximum(Q / 2730.0 - mean ** 2, 0) + 1e-6)
            self.close("fc2+folded LN", _f16(g["x"]), _f16(ref), np.abs(rstd[:, None] * acc).max(), 2.0 ** -10)
        elif step == "head":
            p = orc.pool(g["x"].view(np.uint16), nb)
            assert np.array_equal(g["pool"], p), "pool differs"
            pn, pq, ps = orc.lnh(p, m["fnw"], m["fnb"])
            assert np.array_equal(g["pn"].view(np.uint16), pn) and np.array_equal(g["pq"], pq)
            assert np.array_equal(g["ps"], ps), "final LN packing differs"
            nt = m["nt"]
            hq, hs = orc.head_pack(m["hw"][:nt])
            logit = orc.gemm_rr_f64_rows(pq, ps, hq, hs, nt, np.arange(nb))
            ref = 1.0 / (1.0 + np.exp(-(logit + m["hb"][:nt])))
            err = float(np.abs(g["out"] - ref).max())
            self.worst["head sigmoid |err|"] = err
            assert err <= 1e-4
            for b in range(nb):
                a = set(np.argsort(-g["out"][b], kind="stable")[:50])
                r = set(np.argsort(-ref[b], kind="stable")[:50])
                srt = np.sort(ref[b])[::-1]
                _say(f"  image {b}: top-50 identical {a == r}, gap at rank 50/51 {srt[49] - srt[50]:.2e}")
                assert a == r


def test_forward_teacher_forced_and_engine(dev, xt, orc, synth_blob):
    from tests.fwd_driver import StepForward
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path, m = synth_blob
    nb = 1
    inp = blob.synth_inputs(nb, seed=1)
    _say("step driver: packing weights")
    drv = StepForward(xt, m, nb, dev)
    chk = OracleCheck(orc, m, inp, nb)
    last = [-1]

    def check(step, i, g):
        if i != last[0]:
            _say(f"  layer {i}")
            last[0] = i
        chk(step, i, g)

    out = drv.run(inp, check=check)
    for k, v in sorted(chk.worst.items()):
        _say(f"  worst {k}: {v:.3g}")
    _say("engine forward")
    e = Engine(path, device=0, nb=nb)
    e.ready()
    e.submit(0, inp)
    got = e.wait(0, nb)
    e.close()
    assert np.array_equal(got, out), "the engine's graph differs from the validated kernel sequence"
    np.save(os.path.join(os.environ.get("TMPDIR", "/tmp"), "xtag_gpu_forward_seed1.npy"), got)


def test_forward_sparse_teacher_forced_and_engine(dev, xt, orc, synth_blob):
    from tests.fwd_driver import StepForward
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path, m = synth_blob
    nb = 1
    inp = blob.synth_inputs(nb, seed=2)
    _say("sparse step driver: packing, pruning and compressing weights")
    drv = StepForward(xt, m, nb, dev, sparse=True)
    chk = OracleCheck(orc, m, inp, nb, sparse=True)
    out = drv.run(inp, check=chk)
    for k, v in sorted(chk.worst.items()):
        _say(f"  worst {k}: {v:.3g}")
    _say("sparse engine forward")
    e = Engine(path, device=0, nb=nb, sparse=True)
    e.ready()
    e.submit(0, inp)
    got = e.wait(0, nb)
    e.close()
    assert np.array_equal(got, out), "the sparse engine's graph differs from the validated kernel sequence"


def _free_run(path, m, inp, orc):
    """The engine's scores and fp16 head inputs for inp, and the oracle's, both free running over 24 blocks."""
    from xtagger_amd.engine import Engine
    nb, nt = len(inp), m["nt"]
    e = Engine(path, device=0, nb=nb, extra=1)                # extra > 0: the engine keeps hpn, the head inputs
    e.ready()
    e.submit(0, inp)
    got = e.wait(0, nb)[:, :nt]
    hpn = e.hpn(0, nb)
    e.close()
    _say(f"oracle free-running forward (24 layers, {nb} images)")
    ref, pn = orc.forward(m, inp, nl=24)
    return got, hpn, ref, pn


def _rel_l2(a, b):
    a = np.asarray(a).view(np.float16).astype(np.float64)
    b = np.asarray(b).view(np.float16).astype(np.float64)
    return np.linalg.norm(a - b, axis=1) / np.linalg.norm(b, axis=1)


@pytest.fixture(scope="module")
def conditioned_blob(tmp_path_factory):
    from tests.golden.make_forward_divergence import CONDITIONED
    from xtagger_amd import blob
    path = str(tmp_path_factory.mktemp("blob") / "eva02_conditioned_v2.bin")
    _say("writing the conditioned synthetic v2 blob")
    blob.write_v2(path, blob.synth_model(**CONDITIONED))
    return path, blob.read_v2(path)


def test_forward_free_running_conditioned(dev, orc, conditioned_blob):
    """The north star's contract, free running: on a well-conditioned synthetic model (residual branches scaled by
    0.01, smooth inputs, a head whose 50 leading tags have a margin) the GPU engine's sigmoid scores are within 2e-3
    of the oracle's for each image, with identical top-50 sets, and its fp16 head inputs (the pooled, normalised
    features) lie within twice the relative distance that a change of summation order alone puts between two oracle
    runs; planted mistakes (RoPE rotated the wrong way, the MLP LayerNorm's beta dropped, Wo 2% too large, each in
    every block) move those features by more than that bound (recorded in the fixture)."""
    path, m = conditioned_blob
    from xtagger_amd import blob
    inp = blob.synth_smooth_inputs(2, seed=1)
    got, hpn, ref, pn = _free_run(path, m, inp, orc)
    env = json.load(open(os.path.join(HERE, "golden", "forward_self_divergence.json")))["conditioned"]
    bound = 2 * max(env["head_input_rel_l2_per_image"])
    planted = env["planted_mistakes_head_input_rel_l2"]
    assert all(min(v) > bound for v in planted.values()), "the fixture's planted mistakes must exceed the bound"
    rel = _rel_l2(hpn, pn)
    assert np.isfinite(got).all()
    for i in range(len(inp)):
        d = np.abs(got[i] - ref[i])
        a = set(np.argsort(-got[i], kind="stable")[:50])
        r = set(np.argsort(-ref[i], kind="stable")[:50])
        srt = np.sort(ref[i])[::-1]
        _say(f"  image {i}: sigmoid max |diff| {d.max():.2e} mean {d.mean():.2e} (oracle vs itself "
             f"{env['sigmoid_max_abs_diff_per_image'][i]:.2e}), top-50 identical {a == r}, gap at rank 50/51 "
             f"{srt[49] - srt[50]:.2e}; head inputs rel {rel[i]:.2e} (bound {bound:.2e}, planted mistakes "
             + ", ".join(f"{k} {v[i]:.2e}" for k, v in planted.items()) + ")")
        assert d.max() <= 2e-3
        assert a == r
        assert rel[i] <= bound


def test_forward_free_running_chaotic(dev, orc, synth_blob):
    """The default synthetic model (every block weight N(0, 0.02), inputs of uniform noise) is chaotic: every block
    re-quantizes its activations to E4M3, a different fp32 summation order flips a few roundings and the flips cascade,
    so the oracle drifts from itself by a sizeable fraction of the scores. Per image, the GPU's drift from the oracle
    stays within twice the oracle's own, and its top-50 overlap within 6 tags of the oracle's overlap with itself."""
    from xtagger_amd import blob
    path, m = synth_blob
    inp = blob.synth_inputs(2, seed=1)
    got, hpn, ref, pn = _free_run(path, m, inp, orc)
    env = json.load(open(os.path.join(HERE, "golden", "forward_self_divergence.json")))["chaotic"]
    assert np.isfinite(got).all()
    for i in range(len(inp)):
        d = np.abs(got[i] - ref[i])
        top = len(set(np.argsort(-got[i])[:50]) & set(np.argsort(-ref[i])[:50]))
        _say(f"  image {i}: GPU vs oracle max {d.max():.3e} mean {d.mean():.3e} top-50 overlap {top}; oracle vs "
             f"itself max {env['sigmoid_max_abs_diff_per_image'][i]:.3e} mean "
             f"{env['sigmoid_mean_abs_diff_per_image'][i]:.3e} overlap {env['top50_overlap_per_image'][i]}")
        assert d.max() <= 2 * env["sigmoid_max_abs_diff_per_image"][i]
        assert d.mean() <= 2 * env["sigmoid_mean_abs_diff_per_image"][i]
        assert top >= env["top50_overlap_per_image"][i] - 6


def _pin_block_maxima(w):
    """w with one element of every 128 x 128 block (rows padded as the kernels pad them) set to the tensor's |max|, so
    that per-tensor and per-block amax / 448 scales coincide and give the same E4M3 codes."""
    w = w.astype(np.float32).copy()
    mx = np.abs(w).max()
    n, k = w.shape
    for r0 in range(0, n, 128):
        for c0 in range(0, k, 128):
            blk = w[r0:r0 + 128, c0:c0 + 128]
            if np.abs(blk).max() == 0:
                continue
            i = np.unravel_index(np.argmax(np.abs(blk)), blk.shape)
            blk[i] = np.sign(blk[i]) * mx
    return w


def _v3_engine_vs_v2(tmp_path, orc, m, calib, inp, sparse=False):
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    p2, p3 = str(tmp_path / "eq_v2.bin"), str(tmp_path / "eq_v3.bin")
    blob.write_v2(p2, m)
    blob.write_v3(p3, m, calib)
    out = []
    for p in (p2, p3):
        e = Engine(p, device=0, nb=len(inp), extra=1, sparse=sparse)
        e.ready()
        e.submit(0, inp)
        out.append((e.wait(0, len(inp))[:, :m["nt"]], e.hpn(0, len(inp))))
        e.close()
    return out


@pytest.mark.parametrize("sparse", [False, True])
def test_v3_blob_matches_v2_where_its_quantization_does(dev, orc, tmp_path, sparse):
    """The reference's production blob (export_eva.py v3: E4M3 weights with one scale per tensor, SmoothQuant folds,
    the [24][12] scale table, rs | W~2 | c | d) read by the engine. Written here from the conditioned synthetic model
    with every 128 x 128 block's maximum pinned to its tensor's (so per-tensor and block scales give the same codes),
    calibration maxima equal to the weight-column maxima (so every smoothing factor is 1) and the MLP LayerNorm's
    gamma 1 and beta 0: the v3 engine then computes what the v2 engine computes up to the rounding of c (summed by numpy
    in the blob) and of the fc1 multiplier rs = 1 / adq. Per image: sigmoid within 2e-3 of the v2 engine, identical
    top-50, fp16 head inputs within the free-running bound of the conditioned model. sparse: both engines 2:4-prune
    the same codes (EVA_SPARSE24); the v3 engine recomputes c from the pruned W~ with rs."""
    from tests.golden.make_forward_divergence import CONDITIONED
    from xtagger_amd import blob
    m = blob.synth_model(**CONDITIONED)
    calib = {"act": [], "h": [], "qkv": blob.synth_calib(m, seed=2)["qkv"]}
    for L in m["layers"]:
        L["wqkv"] = _pin_block_maxima(L["wqkv"]).astype(np.float16)
        L["wo"] = _pin_block_maxima(L["wo"]).astype(np.float16)
        L["w12"] = _pin_block_maxima(L["w12"]).astype(np.float16)
        L["w2"] = _pin_block_maxima(L["w2"]).astype(np.float16)
        L["mlnw"] = np.where(np.arange(2736) < 2730, 1.0, 0.0).astype(np.float32)
        L["mlnb"] = np.zeros(2736, np.float32)
        cm = lambda w: np.abs(w.astype(np.float32)).max(0)
        calib["act"].append(np.stack([cm(L["wqkv"]), cm(L["wo"]), cm(L["w12"])]))
        calib["h"].append(cm(L["w2"]))
    calib = {k: np.asarray(v, np.float32) for k, v in calib.items()}
    inp = blob.synth_smooth_inputs(2, seed=1)
    (s2, pn2), (s3, pn3) = _v3_engine_vs_v2(tmp_path, orc, m, calib, inp, sparse)
    env = json.load(open(os.path.join(HERE, "golden", "forward_self_divergence.json")))["conditioned"]
    bound = 2 * max(env["head_input_rel_l2_per_image"])
    rel = _rel_l2(pn3, pn2)
    for i in range(len(inp)):
        d = np.abs(s3[i] - s2[i])
        same = set(np.argsort(-s3[i], kind="stable")[:50]) == set(np.argsort(-s2[i], kind="stable")[:50])
        _say(f"  image {i}: v3 vs v2 sigmoid max {d.max():.2e}, top-50 identical {same}, head inputs rel {rel[i]:.2e} "
             f"(bound {bound:.2e})")
        assert d.max() <= 2e-3 and same and rel[i] <= bound


def test_v3_blob_with_smoothing(dev, orc, tmp_path):
    """A v3 blob with real SmoothQuant factors (synthetic calibration maxima spread 16x with 20x outlier channels) and
    per-tensor E4M3 weights: the engine runs the smoothed network, which is the v2 network up to the different weight
    quantization (one scale per tensor instead of per block, on smoothed columns). Per image the head inputs stay
    within 2% of the v2 engine's (a v3 scale or multiplier applied wrongly, such as rs without adq carried back into
    fc2, moves them by far more), and the sigmoid scores within 2e-2."""
    from tests.golden.make_forward_divergence import CONDITIONED
    from xtagger_amd import blob
    m = blob.synth_model(**CONDITIONED)
    inp = blob.synth_smooth_inputs(2, seed=1)
    (s2, pn2), (s3, pn3) = _v3_engine_vs_v2(tmp_path, orc, m, blob.synth_calib(m, seed=5), inp)
    rel = _rel_l2(pn3, pn2)
    for i in range(len(inp)):
        d = np.abs(s3[i] - s2[i])
        top = len(set(np.argsort(-s3[i])[:50]) & set(np.argsort(-s2[i])[:50]))
        _say(f"  image {i}: v3 (smoothed) vs v2 sigmoid max {d.max():.2e} mean {d.mean():.2e}, top-50 overlap {top}, "
             f"head inputs rel {rel[i]:.2e}")
        assert np.isfinite(s3[i]).all() and rel[i] <= 2e-2 and d.max() <= 2e-2


def test_partial_batch_and_head_rows(dev, synth_blob):
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path, m = synth_blob
    nb = 4
    inp = blob.synth_inputs(3, seed=5)
    e = Engine(path, device=0, nb=nb, extra=3)
    e.ready()
    assert e.nt == m["nt"] + 3
    e.submit(1, inp)                                           # n < nb: the extra slots are ignored
    s = e.wait(1, 3)
    assert np.isfinite(s).all()
    # extra rows never fire before they are written (zero weights, bias -16)
    assert np.abs(s[:, m["nt"]:] - 1.0 / (1.0 + np.exp(16.0))).max() < 1e-6
    hpn = e.hpn(1, 3)
    assert hpn is not None and hpn.shape == (3, 1024)
    w, b = e.head_get()
    assert np.array_equal(w, m["hw"][:m["nt"]]) and np.array_equal(b, m["hb"][:m["nt"]])
    # a stolen row (eva_head_put, eva.h:645-650) and an edited file row: the engine keeps the fp16 head as the master
    # and repacks only the written row (every head row carries its own 1x128 scales); its score follows from the
    # oracle packing of that row and the batch's fp16 head inputs (hpn), and no other row's score moves by a bit
    nt0 = m["nt"]
    e.head_put(nt0, m["hw"][7], float(m["hb"][7]))
    e.submit(2, inp)
    s2 = e.wait(2, 3)
    from oracle import oracle as O
    pq, ps = O.quant_act(e.hpn(2, 3).view(np.float16).astype(np.float32))
    hq, hs = O.head_pack(m["hw"][7:8])
    ref = 1.0 / (1.0 + np.exp(-(O.gemm_rr_f64_rows(pq, ps, hq, hs, 1, np.arange(3))[:, 0] + m["hb"][7])))
    assert np.abs(s2[:, nt0] - ref).max() < 1e-4
    assert np.array_equal(s2[:, :nt0], s[:, :nt0]), "file-tag scores changed by an extra-row upload"
    assert np.array_equal(s2[:, nt0 + 1:], s[:, nt0 + 1:])
    # an edited file row next to others of the same 128-row range: only its own column changes
    j = nt0 - 5
    w_new = (m["hw"][j].astype(np.float32) * 40.0).astype(np.float16)   # a much larger row
    e.head_put(j, w_new, 0.25)
    e.submit(3, inp)
    s3 = e.wait(3, 3)
    others = np.ones(e.nt, bool)
    others[j] = False
    assert np.array_equal(s3[:, others], s2[:, others])
    hq, hs = O.head_pack(w_new[None])
    ref = 1.0 / (1.0 + np.exp(-(O.gemm_rr_f64_rows(pq, ps, hq, hs, 1, np.arange(3))[:, 0] + 0.25)))
    assert np.abs(s3[:, j] - ref).max() < 1e-4
    e.head_put(j, m["hw"][j], float(m["hb"][j]))                      # restore: the file row's scores come back
    e.submit(4, inp)
    assert np.array_equal(e.wait(4, 3), s2)
    # resident-input path: one graph replay on the inputs already in the device buffer gives the same scores
    e.run()
    e.sync()
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out_t = torch.empty((nb, e.nt), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    assert hip.hipMemcpy(out_t.data_ptr(), e.dev_output(), out_t.numel() * 4, 3) == 0
    torch.cuda.synchronize()
    assert np.array_equal(out_t.cpu().numpy()[:3], s2)
    e.close()


def test_truncated_blob_fails_at_ready(dev, tmp_path, synth_blob):
    from xtagger_amd.engine import Engine
    path, _ = synth_blob
    bad = str(tmp_path / "trunc.bin")
    with open(path, "rb") as f:
        data = f.read(256 + 4096)
    with open(bad, "wb") as f:
        f.write(data)
    e = Engine(bad, device=0, nb=1)
    with pytest.raises(RuntimeError):
        e.ready()
    e.close()


def test_submit_ring_nonblocking(dev, synth_blob):
    """eva.h:627-680: up to EVA_NBUF batches are in flight at once. Eight eva_submit calls on bufs 0..7 with distinct
    inputs return while the GPU is still busy with the earlier batches (each waits only for its own buf's previous
    batch), and every buf's scores equal those of the same inputs submitted one at a time."""
    import time
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path, m = synth_blob
    nb = 4
    e = Engine(path, device=0, nb=nb)
    e.ready()
    inp = blob.synth_inputs(8 * nb, seed=77).reshape(8, nb, 1024, 592)
    ref = []
    for b in range(8):                                          # one at a time
        e.submit(b, inp[b])
        ref.append(e.wait(b, nb))
    t_batch = []
    for _ in range(2):                                          # the time of one forward, measured here
        t0 = time.perf_counter()
        e.submit(0, inp[0])
        e.wait(0, nb)
        t_batch.append(time.perf_counter() - t0)
    t_one = min(t_batch)
    t0 = time.perf_counter()
    for b in range(8):
        e.submit(b, inp[b])
    t_submit = time.perf_counter() - t0
    pending = [e.query(b) for b in range(8)]
    got = [e.wait(b, nb) for b in range(8)]
    e.close()
    _say(f"  one forward {t_one * 1e3:.2f} ms, 8 submits returned in {t_submit * 1e3:.2f} ms, done right after: {pending}")
    # a submit that waited for the stream would find every earlier batch done and take about 7 forwards in all
    assert sum(pending[:7]) < 7, "every earlier batch was done when the eighth submit returned"
    assert t_submit < 5 * t_one, "the submits waited for the GPU"
    for b in range(8):
        assert np.array_equal(got[b], ref[b]), f"buf {b}"


@pytest.mark.parametrize("sparse", [False, True])
def test_batch_halves(dev, synth_blob, sparse):
    """A batch runs as two halves at once (the first ceil(nb / 2) inputs on the engine stream, the rest on the second
    lane). With nb = 3 (halves of 2 and 1): full, partial (n = 1: the second lane idle, n = 2: exactly the first half)
    and resident batches give every image the scores an nb = 1 engine gives it, bit for bit; dense and 2:4-sparse."""
    import ctypes
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path, m = synth_blob
    inp = blob.synth_inputs(3, seed=93)
    e1 = Engine(path, device=0, nb=1, sparse=sparse)
    e1.ready()
    ref = []
    for i in range(3):
        e1.submit(0, inp[i:i + 1])
        ref.append(e1.wait(0, 1)[0].copy())
    e1.close()
    ref = np.stack(ref)
    e = Engine(path, device=0, nb=3, sparse=sparse)
    e.ready()
    e.submit(0, inp)
    assert np.array_equal(e.wait(0, 3), ref)
    e.submit(1, inp[2:3])
    assert np.array_equal(e.wait(1, 1), ref[2:3])
    e.submit(2, inp[1:3])
    assert np.array_equal(e.wait(2, 2), ref[1:3])
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    d_in = torch.from_numpy(np.ascontiguousarray(inp)).to(dev)
    torch.cuda.synchronize()
    assert hip.hipMemcpy(e.dev_input(), d_in.data_ptr(), d_in.numel() * 2, 3) == 0
    torch.cuda.synchronize()
    e.run()
    e.sync()
    out_t = torch.empty((3, e.nt), dtype=torch.float32, device=dev)
    assert hip.hipMemcpy(out_t.data_ptr(), e.dev_output(), out_t.numel() * 4, 3) == 0
    torch.cuda.synchronize()
    assert np.array_equal(out_t.cpu().numpy(), ref)
    e.close()


def test_profile_per_op(dev, synth_blob):
    """eva.h:312-338: eva_profile runs one direct forward with an event after every op and returns the GPU time per op
    kind. Every kind takes time, the layer kinds dominate the total, the direct forward (the two halves of the batch one
    after the other) takes about as long as a graph replay (the halves at once) up to the factor two of that
    concurrency, and the profile leaves the scores of the next forward unchanged."""
    import time
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    path, _ = synth_blob
    nb = 4
    e = Engine(path, device=0, nb=nb)
    e.ready()
    inp = blob.synth_inputs(nb, seed=3)
    e.submit(0, inp)
    ref = e.wait(0, nb)
    prof = e.profile()
    e.run()
    e.sync()
    reps = 5
    t0 = time.perf_counter()
    for _ in range(reps):
        e.run()
    e.sync()
    t_graph = (time.perf_counter() - t0) / reps * 1e3
    e.submit(0, inp)
    got = e.wait(0, nb)
    e.close()
    tot = sum(prof.values())
    _say("  " + ", ".join(f"{k} {v:.3f}" for k, v in prof.items()) + f"; total {tot:.2f} ms, graph {t_graph:.2f} ms")
    assert list(prof) == ["patch+embed", "ln1", "qkv", "flash", "oproj", "ln2", "fc1", "fc2", "pool+head"]
    assert all(v > 0 for v in prof.values())
    assert prof["qkv"] + prof["flash"] + prof["fc1"] + prof["fc2"] > 0.5 * tot
    assert 0.5 * t_graph < tot < 4.0 * t_graph
    assert np.array_equal(got, ref)
