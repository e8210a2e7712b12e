"""The gfx950 Mamba-3 scan (mamba4_amd.mamba3_fused, m3s_forward /
m3s_backward) against the float64 oracle (oracle/mamba3.py).

Shapes follow the reference's own checks of the fused-layout scan
(lm/tests/test_flashmamba.py:98-160: B=2, H=4, N=8, P=6, A=2 at T = 45, 40,
7), plus chunk edges, the trained widths (N=128, P=64, A=32: d_state 128,
head_dim 64, rope_fraction 0.5 in lm/configs/mamba4-125m.json) and no
angles.  Tolerances: outputs normwise <= 1e-5 and gradients normwise <= 1e-4
against float64 (float32 arithmetic throughout), plus the reference's
elementwise bounds where its test states them (values 2e-5, gradients
5e-5 relative to each array's scale).
"""

import numpy as np
import pytest

from oracle import mamba3 as m3

NAMES = m3.ARGS


def _gpu(x, grad=False):
    import torch

    return {n: torch.tensor(np.asarray(x[n], np.float32), device="cuda:0", requires_grad=grad)
            for n in NAMES}


def _host(t):
    return t.detach().cpu().numpy().astype(np.float64)


def _run(t):
    from mamba4_amd import mamba3_fused

    return mamba3_fused(*(t[n] for n in NAMES[:7]), q_bias=t["q_bias"], k_bias=t["k_bias"])


def _rounded(x):
    """Inputs as the GPU sees them (float32), in float64 for the oracle."""
    return {n: np.asarray(v, np.float32).astype(np.float64) for n, v in x.items()}


def test_mamba3_fused_rejects_host_tensors_and_bad_shapes():
    import torch

    from mamba4_amd import mamba3_fused

    x = m3.inputs(batch=1, length=4, heads=2, dim=8, width=4, angle_count=2)
    t = {n: torch.tensor(np.asarray(v, np.float32)) for n, v in x.items()}
    with pytest.raises(ValueError):
        mamba3_fused(*(t[n] for n in NAMES[:7]), q_bias=t["q_bias"], k_bias=t["k_bias"])


def _check(x, seed, out_tol=1e-5, grad_tol=1e-4):
    import torch

    from gpu_helpers import normwise

    x = _rounded(x)
    t = _gpu(x, grad=True)
    y, final = _run(t)
    rng = np.random.default_rng(seed)
    d_y = rng.normal(size=y.shape)
    d_final = rng.normal(size=final.shape)
    (y * torch.tensor(d_y, dtype=torch.float32, device="cuda:0")).sum().backward(
        retain_graph=True)
    (final * torch.tensor(d_final, dtype=torch.float32, device="cuda:0")).sum().backward()
    y_ref, final_ref = m3.forward(*(x[n] for n in NAMES))
    assert normwise(_host(y), y_ref) <= out_tol
    assert normwise(_host(final), final_ref) <= out_tol
    np.testing.assert_allclose(_host(y), y_ref, rtol=2e-5, atol=2e-5 * np.abs(y_ref).max())
    grads = m3.backward(*(x[n] for n in NAMES), d_y, d_final)
    for n in NAMES:
        if x[n].size == 0:
            continue
        want = grads[n]
        got = _host(t[n].grad).reshape(want.shape)
        err = normwise(got, want)
        assert err <= grad_tol, (n, err)
        np.testing.assert_allclose(got, want, rtol=5e-5, atol=5e-5 * np.abs(want).max(),
                                   err_msg=n)


@pytest.mark.gpu
@pytest.mark.parametrize("length", [45, 40, 7])
def test_reference_test_shapes(gpu_lib, length):
    from gpu_helpers import announce

    announce(f"mamba3 B2 T{length} H4 N8 P6 A2")
    _check(m3.inputs(batch=2, length=length, heads=4, dim=8, width=6, angle_count=2,
                     seed=length), seed=length + 1)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "batch,length,heads,dim,width,angles",
    [(2, 64, 3, 16, 8, 4), (2, 65, 3, 16, 8, 4), (1, 130, 5, 32, 16, 8), (2, 100, 3, 16, 8, 0),
     (1, 200, 2, 128, 64, 32), (3, 129, 7, 64, 33, 32), (1, 70, 128, 16, 8, 4),
     (2, 90, 6, 128, 64, 64)],
)
def test_matches_oracle(gpu_lib, batch, length, heads, dim, width, angles):
    from gpu_helpers import announce

    announce(f"mamba3 B{batch} T{length} H{heads} N{dim} P{width} A{angles}")
    _check(m3.inputs(batch=batch, length=length, heads=heads, dim=dim, width=width,
                     angle_count=angles, seed=7 * length + heads), seed=length)


@pytest.mark.gpu
def test_full_size_row_against_oracle(gpu_lib):
    """The 125M Mamba-3 mixer's shape (B16 T1024 H24 N128 P64 A32): batch row
    3 against the oracle, forward and backward (the cotangent is zero on the
    other rows, so the bias gradients are row 3's alone)."""
    import torch

    from gpu_helpers import announce, normwise

    announce("mamba3 full size B16 T1024 H24 N128 P64 A32")
    x = _rounded(m3.inputs(batch=16, length=1024, heads=24, dim=128, width=64, angle_count=32,
                           seed=11))
    t = _gpu(x, grad=True)
    y, final = _run(t)
    rng = np.random.default_rng(12)
    d_y = np.zeros(y.shape)
    d_y[3] = rng.normal(size=y.shape[1:])
    (y * torch.tensor(d_y, dtype=torch.float32, device="cuda:0")).sum().backward()
    row = {n: (v[3:4] if n not in ("q_bias", "k_bias") else v) for n, v in x.items()}
    y_ref, final_ref = m3.forward(*(row[n] for n in NAMES))
    assert normwise(_host(y[3:4]), y_ref) <= 1e-5
    assert normwise(_host(final[3:4]), final_ref) <= 1e-5
    grads = m3.backward(*(row[n] for n in NAMES), d_y[3:4], None)
    for n in NAMES:
        got = _host(t[n].grad)
        if n not in ("q_bias", "k_bias"):
            assert not got[:3].any() and not got[4:].any(), n
            got = got[3:4]
        err = normwise(got.reshape(grads[n].shape), grads[n])
        assert err <= 1e-4, (n, err)


@pytest.mark.gpu
def test_backward_is_bit_reproducible(gpu_lib):
    """Every reduction of the backward runs in a fixed order (per-wave LDS
    slots, fixed-order sums; no atomics): two backward passes over the same
    inputs give identical gradients for all nine inputs.  Twelve heads per
    group, so every wave of the gradient kernel contributes to each sum."""
    import torch

    from gpu_helpers import announce

    announce("mamba3 backward twice, B2 T300 H12 N128 P64 A32")
    x = _rounded(m3.inputs(batch=2, length=300, heads=12, dim=128, width=64, angle_count=32,
                           seed=21))
    d_y = None
    grads = []
    for _ in range(2):
        t = _gpu(x, grad=True)
        y, final = _run(t)
        if d_y is None:
            rng = np.random.default_rng(22)
            d_y = torch.tensor(rng.normal(size=y.shape), dtype=torch.float32, device="cuda:0")
            d_f = torch.tensor(rng.normal(size=final.shape), dtype=torch.float32,
                               device="cuda:0")
        ((y * d_y).sum() + (final * d_f).sum()).backward()
        torch.cuda.synchronize()
        grads.append({n: t[n].grad.clone() for n in NAMES})
    for n in NAMES:
        assert torch.equal(grads[0][n], grads[1][n]), n


@pytest.mark.gpu
def test_long_sequence_large_phases(gpu_lib):
    """Angle rates offset by 20 over 12288 tokens: the accumulated phases
    reach 1e5, past the 2^16 range of the kernels' sin/cos.  Each chunk's
    stored start phase is kept reduced modulo 2 pi, so every phase a chunk
    rotates by stays below about 2 pi + 64 * max(rate * dt).  What remains is
    float32 rounding of the phases within each chunk and of the carried start
    phases over 192 chunks (about 1e-4 to 1e-3 rad against the float64
    oracle's exact cumulative sums): outputs normwise <= 3e-3, gradients
    <= 1e-2."""
    import torch

    from gpu_helpers import announce, normwise

    announce("mamba3 B1 T12288 H2 N8 P4 A2, phases to 1e5")
    x = m3.inputs(batch=1, length=12288, heads=2, dim=8, width=4, angle_count=2, seed=3)
    x["angles"] = x["angles"] + 20.0
    x = _rounded(x)
    t = _gpu(x, grad=True)
    y, final = _run(t)
    rng = np.random.default_rng(4)
    d_y = rng.normal(size=y.shape)
    (y * torch.tensor(d_y, dtype=torch.float32, device="cuda:0")).sum().backward()
    y_ref, final_ref = m3.forward(*(x[n] for n in NAMES))
    assert normwise(_host(y), y_ref) <= 3e-3
    assert normwise(_host(final), final_ref) <= 3e-3
    grads = m3.backward(*(x[n] for n in NAMES), d_y, None)
    for n in NAMES:
        got = _host(t[n].grad).reshape(grads[n].shape)
        err = normwise(got, grads[n])
        assert err <= 1e-2, (n, err)
