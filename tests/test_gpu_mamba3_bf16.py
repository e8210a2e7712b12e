"""The bfloat16 Mamba-3 scan (mamba3_fused with bfloat16 c, b, x:
m3s_forward_bf16 / m3s_backward_bf16) against the fused-kernel oracle
(oracle/mamba3_fused.py), which rounds to bfloat16 at the reference's points
(lm/kernels/flashmamba.py:575-786).

What pins the rounding points: the GPU result must sit much closer to the
bfloat16 oracle than the bfloat16 oracle sits to the exact (float64) result
of the same inputs, for y, the final state and every gradient; a kernel
that rounded at other points (or not at all) would land about as far from
the bfloat16 oracle as the exact result does.  What remains between GPU and
oracle is float32 accumulation order, which now and then moves an
intermediate across a bfloat16 rounding boundary.  Errors are relative
2-norms over each array (a single boundary crossing is one element; the
maximum norm would be dominated by it).  Bounds: err(GPU, bf16 oracle)
<= 0.1 err(bf16 oracle, exact) and <= 5e-4 (measured: at most 0.04 and 2e-4).
"""

import numpy as np
import pytest

from oracle import mamba3 as m3
from oracle import mamba3_fused as mf

NAMES = m3.ARGS
pytestmark = pytest.mark.gpu


def _rel(actual, expected):
    """||actual - expected|| / ||expected|| (2-norms over the array)."""
    expected = np.asarray(expected, np.float64)
    return float(np.linalg.norm(np.asarray(actual, np.float64) - expected)
                 / max(np.linalg.norm(expected), 1e-30))


def _host(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _case(batch, length, heads, dim, width, angles, seed):
    import torch

    from mamba4_amd import mamba3_fused

    x = m3.inputs(batch=batch, length=length, heads=heads, dim=dim, width=width,
                  angle_count=angles, seed=seed)
    x = {n: (mf.round_bf16(v) if n in ("c", "b", "x") else np.asarray(v, np.float32))
         .astype(np.float64) for n, v in x.items()}
    rng = np.random.default_rng(seed + 1)
    d_y = mf.round_bf16(rng.normal(size=(batch, length, heads * width))).astype(np.float64)
    d_final = rng.normal(size=(batch, heads, dim, width)).astype(np.float32).astype(np.float64)
    t = {}
    for n in NAMES:
        dtype = torch.bfloat16 if n in ("c", "b", "x") else torch.float32
        t[n] = torch.tensor(x[n], dtype=torch.float32, device="cuda:0").to(dtype)
        t[n].requires_grad_(True)
    y, final = mamba3_fused(*(t[n] for n in NAMES[:7]), q_bias=t["q_bias"], k_bias=t["k_bias"])
    assert y.dtype == torch.bfloat16 and final.dtype == torch.float32
    ((y.float() * torch.tensor(d_y, dtype=torch.float32, device="cuda:0")).sum()
     + (final * torch.tensor(d_final, dtype=torch.float32, device="cuda:0")).sum()).backward()
    args = [x[n] for n in NAMES]
    y16, f16, _, _ = mf.fused_forward(*args, rnd=mf.round_bf16, dtype=np.float32)
    y64, f64, _, _ = mf.fused_forward(*args, rnd=None, dtype=np.float64)
    g16 = mf.fused_backward(*args, d_y=d_y, d_final=d_final, rnd=mf.round_bf16,
                            dtype=np.float32)
    g64 = mf.fused_backward(*args, d_y=d_y, d_final=d_final, rnd=None, dtype=np.float64)
    rows = [("y", _host(y), y16, y64), ("final", _host(final), f16, f64)]
    for n in NAMES:
        if x[n].size:
            assert t[n].grad.dtype == t[n].dtype, n
            rows.append((n, _host(t[n].grad).reshape(g16[n].shape), g16[n], g64[n]))
    for name, got, want, exact in rows:
        near, model = _rel(got, want), _rel(want, exact)
        print(f"{name}: gpu-bf16 oracle {near:.2e}, bf16 oracle-exact {model:.2e}")
        assert near <= 0.1 * model and near <= 5e-4, (name, near, model)


@pytest.mark.parametrize("length", [45, 7])
def test_bf16_reference_test_shapes(gpu_lib, length):
    from gpu_helpers import announce

    announce(f"mamba3 bf16 B2 T{length} H4 N8 P6 A2")
    _case(2, length, 4, 8, 6, 2, seed=length)


@pytest.mark.parametrize("batch,length,heads,dim,width,angles",
                         [(1, 130, 5, 32, 16, 8), (2, 100, 3, 16, 8, 0),
                          (1, 200, 2, 128, 64, 32), (1, 70, 128, 16, 8, 4),
                          (2, 90, 6, 128, 64, 64)])
def test_bf16_matches_fused_oracle(gpu_lib, batch, length, heads, dim, width, angles):
    from gpu_helpers import announce

    announce(f"mamba3 bf16 B{batch} T{length} H{heads} N{dim} P{width} A{angles}")
    _case(batch, length, heads, dim, width, angles, seed=3 * length + heads)
