"""Pins the float64 Mamba-3 scan oracle (oracle/mamba3.py) without the
reference: two independent formulations of the forward, the chunk algebra, a
brute-force closed form, causality, and central finite differences for every
gradient.  The reference's own checks of this operator are of the same kind
(lm/tests/test_mamba3_transformer.py:32-75: chunked vs the local-frame
NumPy recurrence and vs the token recurrence, gradients vs the recurrence);
the reference ships no golden vectors for it.
"""

import numpy as np
import pytest

from oracle import mamba3 as m3


def _call(fn, x, **kw):
    return fn(*(x[n] for n in m3.ARGS), **kw)


@pytest.mark.parametrize("angle_count", [0, 2, 8])
def test_cumulative_frame_matches_local_frame(angle_count):
    """The local frame turns the state by minus each phase increment and never
    rotates q or k; agreement pins the rotation's sign, the pairing and the
    phase integration."""
    x = m3.inputs(batch=2, length=23, heads=3, dim=16, width=5, angle_count=angle_count, seed=1)
    y, final = _call(m3.forward, x)
    y_loc, final_loc = _call(m3.local_forward, x)
    np.testing.assert_allclose(y, y_loc, rtol=1e-11, atol=1e-11)
    # The local state lives in the frame of the last token: turn it back.
    theta = m3.phases(x["angles"], x["dt"])[:, -1]
    turned = np.swapaxes(m3.rotate(np.swapaxes(final_loc, -1, -2), theta[:, :, None, :]), -1, -2)
    np.testing.assert_allclose(final, turned, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("chunk", [1, 4, 16, 64])
def test_chunk_form_matches_token_recurrence(chunk):
    x = m3.inputs(batch=2, length=37, heads=2, dim=16, width=8, angle_count=4, seed=2)
    y, final = _call(m3.forward, x)
    y_c, final_c, starts = _call(m3.chunked_forward, x, chunk=chunk)
    np.testing.assert_allclose(y_c, y, rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(final_c, final, rtol=1e-10, atol=1e-11)
    # Each stored start state is the token recurrence's state before the
    # chunk plus the next token's trapezoid term prev_t0 k_{t0-1} v_{t0-1}^T
    # (which the chunk's decay exp(p_t) then turns into exp(adt_t0) * it).
    _, k, _ = m3.frame(x["c"], x["b"], x["dt"], x["angles"], x["q_bias"], x["k_bias"])
    v = x["x"].reshape(2, 37, 2, 8)
    prev = x["dt"] * (1 - m3.sigmoid(x["trap"]))
    for i, t0 in enumerate(range(0, 37, chunk)):
        if t0 == 0:
            assert not starts[:, :, 0].any()
            continue
        cut = {n: (v_[:, :t0] if n not in ("q_bias", "k_bias") else v_) for n, v_ in x.items()}
        _, s = _call(m3.forward, cut)
        s = s + prev[:, t0, :, None, None] * k[:, t0 - 1, :, :, None] * v[:, t0 - 1, :, None, :]
        np.testing.assert_allclose(starts[:, :, i], s, rtol=1e-10, atol=1e-11)


def test_zero_angles_full_trapezoid_is_decayed_linear_attention():
    """angles = 0 and sigma(trap) = 1: y_t = sum_{s<=t} exp(p_t - p_s) dt_s
    (q_t . k_s) v_s with the biases added, by a brute-force double sum."""
    x = m3.inputs(batch=1, length=9, heads=2, dim=6, width=3, angle_count=2, seed=3)
    x["angles"] = np.zeros_like(x["angles"])
    x["trap"] = np.full_like(x["trap"], 60.0)
    y, _ = _call(m3.forward, x)
    q = x["c"][:, :, None, :] + x["q_bias"]
    k = x["b"][:, :, None, :] + x["k_bias"]
    v = x["x"].reshape(1, 9, 2, 3)
    p = np.cumsum(x["adt"], 1)
    expected = np.zeros_like(v)
    for t in range(9):
        for s in range(t + 1):
            w = np.exp(p[:, t] - p[:, s]) * x["dt"][:, s]
            expected[:, t] += (w * np.einsum("bhn,bhn->bh", q[:, t], k[:, s]))[..., None] * v[:, s]
    np.testing.assert_allclose(y, expected.reshape(1, 9, 6), rtol=1e-12, atol=1e-12)


def test_no_future_leakage():
    """Changing every input from token 5 on leaves y[:, :5] unchanged
    (lm/tests/test_mamba3_transformer.py:73-78)."""
    x = m3.inputs(batch=2, length=11, heads=2, dim=8, width=4, angle_count=2, seed=4)
    y, _ = _call(m3.forward, x)
    changed = {n: (v if n in ("q_bias", "k_bias") else np.concatenate(
        [v[:, :5], v[:, 5:] + 0.7], 1)) for n, v in x.items()}
    y2, _ = _call(m3.forward, changed)
    np.testing.assert_allclose(y2[:, :5], y[:, :5], rtol=0, atol=1e-14)


def test_backward_matches_finite_differences():
    x = m3.inputs(batch=2, length=6, heads=2, dim=6, width=3, angle_count=2, seed=5)
    rng = np.random.default_rng(6)
    d_y = rng.normal(size=x["x"].shape)
    d_final = rng.normal(size=(2, 2, 6, 3))
    grads = m3.backward(*(x[n] for n in m3.ARGS), d_y, d_final)

    def loss(arrays):
        y, final = _call(m3.forward, arrays)
        return np.sum(y * d_y) + np.sum(final * d_final)

    eps = 1e-6
    for name in m3.ARGS:
        base = x[name]
        numeric = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            hi, lo = dict(x), dict(x)
            hi[name], lo[name] = base.copy(), base.copy()
            hi[name][idx] += eps
            lo[name][idx] -= eps
            numeric[idx] = (loss(hi) - loss(lo)) / (2 * eps)
        np.testing.assert_allclose(grads[name], numeric, rtol=1e-6, atol=1e-7, err_msg=name)


def test_rotation_is_orthogonal_and_back_is_its_transpose():
    rng = np.random.default_rng(7)
    u, du = rng.normal(size=(3, 10)), rng.normal(size=(3, 10))
    theta = rng.normal(size=(3, 3))
    r = m3.rotate(u, theta)
    np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(u, axis=-1))
    np.testing.assert_allclose(np.sum(r * du), np.sum(u * m3.rotate_back(du, theta)))
    np.testing.assert_array_equal(r[:, 6:], u[:, 6:])


# The fused-kernel restatement with model-dtype rounding (oracle/mamba3_fused.py).

def test_round_bf16_matches_torch_bfloat16():
    """Round-to-nearest-even to bfloat16, ties included, equals torch's
    float32 -> bfloat16 conversion."""
    torch = pytest.importorskip("torch")
    from oracle import mamba3_fused as mf

    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.normal(size=20000).astype(np.float32) * 10.0 ** rng.integers(-6, 6, 20000),
        # exact ties: a bfloat16 value plus half its last place, both parities
        (np.arange(1, 2001, dtype=np.float32) * 2 ** -7 + 2 ** -16).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -3.5, 65504.0, 1e-38], np.float32),
    ])
    want = torch.tensor(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(mf.round_bf16(x), want)


@pytest.mark.parametrize("chunk,length", [(16, 37), (64, 130), (8, 8)])
def test_fused_forward_without_rounding_is_the_chunk_algebra(chunk, length):
    from oracle import mamba3_fused as mf

    x = m3.inputs(batch=2, length=length, heads=3, dim=16, width=8, angle_count=4, seed=4)
    y, final = _call(m3.forward, x)
    _, _, starts = _call(m3.chunked_forward, x, chunk=chunk)
    y_f, final_f, starts_f, phase0 = _call(mf.fused_forward, x, chunk=chunk, rnd=None,
                                           dtype=np.float64)
    np.testing.assert_allclose(y_f, y, rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(final_f, final, rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(starts_f, starts, rtol=1e-10, atol=1e-11)
    # Start phases: the running phase at each chunk's first token minus its own step.
    theta = m3.phases(x["angles"], x["dt"])
    first = np.arange(0, length, chunk)
    inc = x["angles"][:, first, None, :] * x["dt"][:, first, :, None]
    want = np.swapaxes(theta[:, first] - inc, 1, 2)
    np.testing.assert_allclose(phase0[..., 0:8:2], want, rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(phase0[..., 1:8:2], want, rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("chunk,length", [(16, 37), (64, 70)])
def test_fused_backward_without_rounding_matches_the_recurrence(chunk, length):
    """All nine gradients of the chunk-form backward (with the chunk-end
    terms and mamba3_fused's glue) equal the finite-difference-pinned token
    recurrence's."""
    from oracle import mamba3_fused as mf

    x = m3.inputs(batch=2, length=length, heads=3, dim=16, width=8, angle_count=4, seed=6)
    rng = np.random.default_rng(7)
    y, final = _call(m3.forward, x)
    dy, dfin = rng.normal(size=y.shape), rng.normal(size=final.shape)
    want = _call(m3.backward, x, d_y=dy, d_final=dfin)
    got = _call(mf.fused_backward, x, d_y=dy, d_final=dfin, chunk=chunk, rnd=None,
                dtype=np.float64)
    for name in m3.ARGS:
        np.testing.assert_allclose(got[name], want[name], rtol=1e-9, atol=1e-10, err_msg=name)


def test_bfloat16_model_rounding_is_bfloat16_sized():
    """With bfloat16 operands the results move from the exact ones by a few
    bfloat16 places (not zero, not float32-sized, not wrong): normwise
    between 2^-12 and 2^-5, for y and for every gradient."""
    from oracle import mamba3_fused as mf

    x = m3.inputs(batch=1, length=70, heads=2, dim=16, width=8, angle_count=4, seed=8)
    for n in ("c", "b", "x"):
        x[n] = mf.round_bf16(x[n]).astype(np.float64)
    rng = np.random.default_rng(9)
    dy = mf.round_bf16(rng.normal(size=(1, 70, 16))).astype(np.float64)
    y64, _, _, _ = _call(mf.fused_forward, x, rnd=None, dtype=np.float64)
    y16, _, _, _ = _call(mf.fused_forward, x, rnd=mf.round_bf16, dtype=np.float32)
    err = np.linalg.norm(y16 - y64) / np.linalg.norm(y64)
    assert 2.0 ** -12 < err < 2.0 ** -5, err
    g64 = _call(mf.fused_backward, x, d_y=dy, rnd=None, dtype=np.float64)
    g16 = _call(mf.fused_backward, x, d_y=dy, rnd=mf.round_bf16, dtype=np.float32)
    for name in m3.ARGS:
        err = np.linalg.norm(g16[name] - g64[name]) / np.linalg.norm(g64[name])
        assert 2.0 ** -14 < err < 2.0 ** -5, (name, err)
