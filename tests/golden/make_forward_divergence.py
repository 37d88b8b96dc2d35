"""Writes forward_self_divergence.json: how far the oracle's own full wd forward moves when only its fp32 GEMM
summation order changes (scalar fma chain vs 8-lane AVX2), for two synthetic models. CPU only (~15 minutes).

- "chaotic": blob.synth_model(seed=0) (every block weight N(0, 0.02)) on synth_inputs(2, seed=1) (pixels U[0, 1]).
  Each block re-quantizes its activations to E4M3; a different summation order flips a few roundings and the flips
  cascade through the 24 blocks, so the two orders end up a sizeable fraction of the scores apart.
- "conditioned": blob.synth_model(seed=0, layer_scale=0.01, head_std=0.002, lead_tags=50) on
  synth_smooth_inputs(2, seed=1): residual branches scaled as a trained network's layer scale keeps them, inputs whose
  pooled features carry the image. For it the file also records how far three planted mistakes move the fp16 head
  inputs (the pooled, normalised features) of the same forward: RoPE rotated the wrong way, the MLP LayerNorm's beta
  dropped, and Wo 2% too large, each in every block.

Per model and image: sigmoid max / mean |difference|, top-50 overlap, relative L2 distance of the fp16 head inputs,
and the gap between the scores at rank 50 and 51. The GPU free-running tests (tests/test_forward_gpu.py) are held to
these envelopes.

    python tests/golden/make_forward_divergence.py
"""
import copy
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import numpy as np  # noqa: E402

from oracle import oracle as O  # noqa: E402
from xtagger_amd import blob  # noqa: E402

CONDITIONED = dict(seed=0, nt=10861, layer_scale=0.01, head_std=0.002, lead_tags=50)


def _f16(pn):
    return np.asarray(pn).view(np.float16).astype(np.float64)


def _rel(a, b):
    return (np.linalg.norm(_f16(a) - _f16(b), axis=1) / np.linalg.norm(_f16(b), axis=1)).tolist()


def _run(m, x, scalar):
    if scalar:
        os.environ["XO_SCALAR"] = "1"
    else:
        os.environ.pop("XO_SCALAR", None)
    t = time.time()
    out = O.forward(m, x, nl=24)
    print(f"  forward ({'scalar' if scalar else 'AVX2'}) {time.time() - t:.0f} s", flush=True)
    return out


def _envelope(m, x):
    a, pa = _run(m, x, False)
    b, pb = _run(m, x, True)
    d = np.abs(a - b)
    tops = [len(set(np.argsort(-a[i])[:50]) & set(np.argsort(-b[i])[:50])) for i in range(len(a))]
    gaps = [float(np.sort(a[i])[::-1][49] - np.sort(a[i])[::-1][50]) for i in range(len(a))]
    env = {"sigmoid_max_abs_diff_per_image": d.max(1).tolist(), "sigmoid_mean_abs_diff_per_image": d.mean(1).tolist(),
           "top50_overlap_per_image": tops, "head_input_rel_l2_per_image": _rel(pb, pa), "gap_rank50_51": gaps}
    return env, pa


def main():
    out = {}
    print("chaotic model", flush=True)
    m = blob.synth_model(seed=0, nt=10861)
    env, _ = _envelope(m, blob.synth_inputs(2, seed=1))
    out["chaotic"] = {"model": "xtagger_amd.blob.synth_model(seed=0, nt=10861)", "input": "synth_inputs(2, seed=1)",
                      "layers": 24, **env}
    print("conditioned model", flush=True)
    m = blob.synth_model(**CONDITIONED)
    x = blob.synth_smooth_inputs(2, seed=1)
    env, base = _envelope(m, x)
    planted = {}
    mb = copy.deepcopy(m)
    mb["rope"] = mb["rope"].copy()
    mb["rope"][..., 1] *= -1
    planted["rope_rotated_the_wrong_way"] = _rel(_run(mb, x, False)[1], base)
    mb = copy.deepcopy(m)
    for L in mb["layers"]:
        L["mlnb"] = L["mlnb"] * 0
    planted["mlp_layernorm_beta_dropped"] = _rel(_run(mb, x, False)[1], base)
    mb = copy.deepcopy(m)
    for L in mb["layers"]:
        L["wo"] = (L["wo"].astype(np.float32) * 1.02).astype(np.float16)
    planted["wo_2pct_too_large"] = _rel(_run(mb, x, False)[1], base)
    out["conditioned"] = {"model": "xtagger_amd.blob.synth_model(" + ", ".join(f"{k}={v}" for k, v in
                                                                              CONDITIONED.items()) + ")",
                          "input": "synth_smooth_inputs(2, seed=1)", "layers": 24, **env,
                          "planted_mistakes_head_input_rel_l2": planted}
    with open(os.path.join(HERE, "forward_self_divergence.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))


if __name__ == "__main__":
    main()
