"""Writes forward_self_divergence.json: how far the oracle's own full wd forward moves when only its fp32 GEMM
summation order changes (scalar fma chain vs 8-lane AVX2), on the synthetic seed-0 model and two seed-1 images.
The GPU forward is held to a multiple of this envelope (tests/test_forward_gpu.py). CPU only (~2 minutes).

    python tests/golden/make_forward_divergence.py
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import numpy as np  # noqa: E402

from oracle import oracle as O  # noqa: E402
from xtagger_amd import blob  # noqa: E402


def main():
    m = blob.synth_model(seed=0, nt=10861)
    x = blob.synth_inputs(2, seed=1)
    os.environ.pop("XO_SCALAR", None)
    a, _ = O.forward(m, x, nl=24)
    os.environ["XO_SCALAR"] = "1"
    b, _ = O.forward(m, x, nl=24)
    d = np.abs(a - b)
    tops = [len(set(np.argsort(-a[i])[:50]) & set(np.argsort(-b[i])[:50])) for i in range(2)]
    out = {"model": "xtagger_amd.blob.synth_model(seed=0, nt=10861)", "input": "synth_inputs(2, seed=1)",
           "layers": 24, "sigmoid_max_abs_diff": float(d.max()), "sigmoid_mean_abs_diff": float(d.mean()),
           "top50_overlap_per_image": tops, "top50_overlap": float(np.mean(tops))}
    with open(os.path.join(HERE, "forward_self_divergence.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(out)


if __name__ == "__main__":
    main()
