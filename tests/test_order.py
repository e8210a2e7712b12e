"""The order head's gated vector scan: the float64 oracle pinned on the CPU,
the HIP kernels against it on the GPU.

Oracle pins: closed forms of the scan (constant decay and value, lam = 0,
log lam = 0), the reference's own chunked-vs-sequential test
(lm/tests/test_mamba4.py:301-324) at its shape, central finite differences
and float64 torch autograd of the recurrence for the VJP, and planted
mistakes that each check must catch.

GPU tolerances (fp32 HIP vs float64 oracle): outputs rtol 1e-5 / atol 1e-6
(the reference's own chunked-vs-sequential tolerance), gradients rtol 1e-4 /
atol 1e-5 (:322-324).
"""

import numpy as np
import pytest
import torch

from oracle import order as oracle


def _problem(batch=2, time=37, heads=3, width=5, seed=3, initial=False):
    # The reference test's inputs: N(0,1) values, logits N(0,1) + 2
    # (lm/tests/test_mamba4.py:304-306), lam = sigmoid(logits).
    rng = np.random.default_rng(seed)
    values = rng.normal(size=(batch, time, heads, width))
    logits = rng.normal(size=(batch, time, heads)) + 2
    log_decay = -np.log1p(np.exp(-logits))
    init = rng.normal(size=(batch, heads, width)) if initial else None
    return values, log_decay, init


# ----------------------------------------------------------------- CPU pins


def test_sequential_scan_known_answers():
    t = np.arange(12)
    lam, v, h0 = 0.8, 1.7, -0.6
    values = np.full((1, 12, 1, 2), v)
    decay = np.full((1, 12, 1), lam)
    # Constant decay and value from zero: h_t = v (1 - lam^(t+1)).
    np.testing.assert_allclose(
        oracle.order_memory(values, decay)[0, :, 0, 0], v * (1 - lam ** (t + 1)), rtol=1e-14
    )
    init = np.full((1, 1, 2), h0)
    want = lam ** (t + 1) * h0 + v * (1 - lam ** (t + 1))
    np.testing.assert_allclose(oracle.order_memory(values, decay, init)[0, :, 0, 1], want,
                               rtol=1e-14)
    np.testing.assert_allclose(
        oracle.order_memory_chunked(values, np.log(decay), 5, init)[0, :, 0, 1], want,
        rtol=1e-13)
    # lam = 0 copies the values; log lam = 0 keeps the initial state exactly.
    rng = np.random.default_rng(0)
    x = rng.normal(size=(2, 9, 3, 4))
    np.testing.assert_array_equal(oracle.order_memory(x, np.zeros((2, 9, 3))), x)
    h = oracle.order_memory_chunked(x, np.zeros((2, 9, 3)), 4, rng.normal(size=(2, 3, 4)))
    np.testing.assert_array_equal(h, np.broadcast_to(h[:, :1], h.shape))


@pytest.mark.parametrize("chunk", [1, 4, 8, 37, 64])
def test_chunked_scan_matches_sequential_scan(chunk):
    # lm/tests/test_mamba4.py:301-316 at its shape (2, 37, 3, 5), chunk 8,
    # plus other chunk sizes and an initial state.
    values, log_decay, init = _problem(initial=True)
    seq = oracle.order_memory(values, np.exp(log_decay))
    np.testing.assert_allclose(oracle.order_memory_chunked(values, log_decay, chunk), seq,
                               rtol=1e-12, atol=1e-13)
    seq = oracle.order_memory(values, np.exp(log_decay), init)
    np.testing.assert_allclose(oracle.order_memory_chunked(values, log_decay, chunk, init), seq,
                               rtol=1e-12, atol=1e-13)


def _loss_weights(shape, seed=9):
    return np.random.default_rng(seed).normal(size=shape)


def _check_against_finite_differences(backward):
    values, log_decay, init = _problem(time=11, width=3, initial=True)
    d_out = _loss_weights(values.shape)
    d_values, d_log, d_init = backward(values, log_decay, d_out, init)

    def loss(v, lg, h0):
        return np.sum(d_out * oracle.order_memory_chunked(v, lg, 4, h0))

    eps = 1e-6
    rng = np.random.default_rng(1)
    for _ in range(6):
        i = tuple(rng.integers(0, n) for n in values.shape)
        vp, vm = values.copy(), values.copy()
        vp[i] += eps
        vm[i] -= eps
        assert abs((loss(vp, log_decay, init) - loss(vm, log_decay, init)) / (2 * eps)
                   - d_values[i]) < 1e-6
        j = tuple(rng.integers(0, n) for n in log_decay.shape)
        lp, lm = log_decay.copy(), log_decay.copy()
        lp[j] += eps
        lm[j] -= eps
        assert abs((loss(values, lp, init) - loss(values, lm, init)) / (2 * eps)
                   - d_log[j]) < 1e-6
        k = tuple(rng.integers(0, n) for n in init.shape)
        ip, im = init.copy(), init.copy()
        ip[k] += eps
        im[k] -= eps
        assert abs((loss(values, log_decay, ip) - loss(values, log_decay, im)) / (2 * eps)
                   - d_init[k]) < 1e-6


def test_backward_matches_finite_differences():
    _check_against_finite_differences(oracle.order_memory_backward)


def test_backward_matches_autograd_of_the_recurrence():
    values, log_decay, init = _problem(time=23, width=4, initial=True)
    d_out = _loss_weights(values.shape)
    v = torch.tensor(values, requires_grad=True)
    lg = torch.tensor(log_decay, requires_grad=True)
    h0 = torch.tensor(init, requires_grad=True)
    h, outs = h0, []
    for t in range(values.shape[1]):
        lam = torch.exp(lg[:, t])[..., None]
        h = lam * h - torch.expm1(lg[:, t])[..., None] * v[:, t]
        outs.append(h)
    (torch.stack(outs, 1) * torch.tensor(d_out)).sum().backward()
    d_values, d_log, d_init = oracle.order_memory_backward(values, log_decay, d_out, init)
    np.testing.assert_allclose(d_values, v.grad.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(d_log, lg.grad.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(d_init, h0.grad.numpy(), rtol=1e-12, atol=1e-13)


def _planted(mistake):
    """order_memory_backward with one plausible mistake."""

    def backward(values, log_decay, d_output, initial=None):
        lam = np.exp(log_decay)[..., None]
        inflow = -np.expm1(log_decay)[..., None]
        h = oracle.order_memory_chunked(values, log_decay, 64, initial)
        start = np.zeros_like(h[:, 0]) if initial is None else initial
        previous = np.concatenate([start[:, None], h[:, :-1]], axis=1)
        if mistake == "current state":
            previous = h
        time = values.shape[1]
        g = np.zeros_like(start)
        d_values = np.empty_like(values)
        d_log = np.empty(log_decay.shape)
        for t in reversed(range(time)):
            if t + 1 < time:
                carry = lam[:, t] if mistake == "own decay" else lam[:, t + 1]
                g = d_output[:, t] + carry * g
            else:
                g = d_output[:, t]
            d_values[:, t] = (lam[:, t] if mistake == "decay as inflow" else inflow[:, t]) * g
            scale = 1.0 if mistake == "no chain factor" else lam[:, t, :, 0]
            d_log[:, t] = scale * np.sum(g * (previous[:, t] - values[:, t]), axis=-1)
        return d_values, d_log, lam[:, 0] * g

    return backward


@pytest.mark.parametrize(
    "mistake", ["current state", "own decay", "decay as inflow", "no chain factor"]
)
def test_planted_backward_mistakes_are_caught(mistake):
    with pytest.raises(AssertionError):
        _check_against_finite_differences(_planted(mistake))


# ----------------------------------------------------------------- GPU parity


def _gpu(*arrays):
    return [None if a is None else torch.tensor(np.asarray(a, np.float32), device="cuda:0")
            for a in arrays]


def _host(t):
    return t.detach().cpu().numpy().astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "batch,time,heads,width,chunk,initial",
    [(2, 37, 3, 5, 8, False), (2, 37, 3, 5, 8, True), (3, 200, 4, 64, 64, True),
     (2, 130, 2, 128, 16, False), (1, 70, 2, 200, 64, True), (2, 1, 3, 64, 64, True)],
)
def test_order_scan_matches_oracle(gpu_lib, batch, time, heads, width, chunk, initial):
    from mamba4_amd import order_memory_chunked
    from tests.gpu_helpers import announce

    values, log_decay, init = _problem(batch, time, heads, width, seed=time, initial=initial)
    d_out = _loss_weights(values.shape)
    announce(f"order scan B{batch} T{time} H{heads} W{width} chunk={chunk} init={initial}")
    v, lg, h0, d = _gpu(values, log_decay, init, d_out)
    v.requires_grad_(True)
    lg.requires_grad_(True)
    if h0 is not None:
        h0.requires_grad_(True)
    out = order_memory_chunked(v, lg, chunk, initial=h0)
    (out * d).sum().backward()
    torch.cuda.synchronize()
    want = oracle.order_memory_chunked(values, log_decay, chunk, init)
    np.testing.assert_allclose(_host(out), want, rtol=1e-5, atol=1e-6)
    d_values, d_log, d_init = oracle.order_memory_backward(values, log_decay, d_out, init)
    np.testing.assert_allclose(_host(v.grad), d_values, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_host(lg.grad), d_log, rtol=1e-4, atol=1e-5)
    if h0 is not None:
        np.testing.assert_allclose(_host(h0.grad), d_init, rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
def test_order_cached_step_and_decay_form(gpu_lib):
    """The order head's cached decode step (lm/models/mamba4.py:283-287) is
    the scan over one token from the cache; order_memory takes the decays."""
    from mamba4_amd import order_memory, order_memory_chunked
    from tests.gpu_helpers import announce

    values, log_decay, cache = _problem(4, 1, 6, 64, seed=4, initial=True)
    announce("order scan cached step B4 H6 W64")
    v, lg, c = _gpu(values, log_decay, cache)
    got = _host(order_memory_chunked(v, lg, initial=c))[:, 0]
    lam = np.exp(log_decay)[:, 0, :, None]
    np.testing.assert_allclose(got, lam * cache + (1 - lam) * values[:, 0], rtol=1e-5,
                               atol=1e-6)
    values, log_decay, _ = _problem(2, 37, 3, 5)
    v, decay = _gpu(values, np.exp(log_decay))
    np.testing.assert_allclose(_host(order_memory(v, decay)),
                               oracle.order_memory(values, np.exp(log_decay)), rtol=1e-5,
                               atol=1e-6)


@pytest.mark.gpu
def test_order_scan_full_size(gpu_lib):
    """The 60M shape (B=16, T=1024, H=8, W=64): chunk sizes agree, and a
    batch row matches the oracle."""
    from mamba4_amd import order_memory_chunked
    from tests.gpu_helpers import announce, normwise

    values, log_decay, _ = _problem(16, 1024, 8, 64, seed=11)
    announce("order scan full size B16 T1024 H8 W64")
    v, lg = _gpu(values, log_decay)
    a = _host(order_memory_chunked(v, lg, 64))
    b = _host(order_memory_chunked(v, lg, 16))
    assert normwise(a, b) <= 1e-5
    want = oracle.order_memory_chunked(values[5:6], log_decay[5:6], 64)
    assert normwise(a[5:6], want) <= 1e-5


def test_order_scan_rejects_bad_arguments():
    from mamba4_amd import order_memory_chunked

    with pytest.raises(ValueError):
        order_memory_chunked(torch.zeros(1, 2, 3, 4), torch.zeros(1, 2, 3))
