"""Write tests/golden/config0.npz: BASELINE config 0 inputs with float64
oracle outputs, final state and every gradient.

Config 0 (B=2, L=256, H=1, D=P=64, seed 0, floor 1e-2, shifted unit keys,
decay logits N(2,1)) from ``mamba4_amd.inputs``; expected values from the
pinned CPU oracle (``oracle.memread``: dense float64 forward, closed-form
float64 backward).  The reference repository holds no golden vectors for
this path, so these fixtures freeze the pinned oracle's answers.

Run: ``python tests/golden/make_golden.py``.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from mamba4_amd.inputs import workload_inputs  # noqa: E402
from oracle import memread as oracle  # noqa: E402

NAMES = ["keys", "values", "queries", "beta", "log_decay", "floor"]


def main():
    data = workload_inputs("config0", seed=0, cotangents=True)
    args = [data[n].astype(np.float64) for n in NAMES]
    out, var, s, c = oracle.dense_reference(*args)
    _, res = oracle.forward(*args, chunk=64)
    rng = np.random.default_rng(1)
    d_s = rng.normal(size=s.shape) * 0.01
    d_s = 0.5 * (d_s + np.swapaxes(d_s, -1, -2))
    d_c = rng.normal(size=c.shape) * 0.01
    grads = oracle.backward(res, data["d_output"], data["d_variance"], d_s, d_c)
    payload = {f"in_{n}": data[n] for n in NAMES}
    # Expected values are stored in float32: storage rounding (6e-8) is far
    # below the parity tolerances (1e-4 outputs, 1e-3 gradients).
    f32 = np.float32
    payload.update(
        d_output=data["d_output"],
        d_variance=data["d_variance"],
        d_final_evidence=d_s.astype(f32),
        d_final_cross=d_c.astype(f32),
        output=out.astype(f32),
        variance=var.astype(f32),
        evidence=s.astype(f32),
        cross=c.astype(f32),
    )
    payload.update({f"grad_{k}": v.astype(f32) for k, v in grads.items()})
    path = os.path.join(HERE, "config0.npz")
    np.savez_compressed(path, **payload)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
