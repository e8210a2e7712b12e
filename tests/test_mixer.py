"""Mixer prologue and epilogue (the memory read's caller preprocessing and
read gating, lm/models/mamba4.py:183-237, 266-273).

CPU tests pin the float64 oracle (oracle/mixer.py) by known answers taken
from the reference's parameterisation and tests, by the cache-continuation
invariant of the key shift, by central finite differences of the VJPs and by
planted mistakes.  GPU tests compare the HIP kernels with the oracle.
"""

import math

import numpy as np
import pytest

from oracle import mixer as oracle

BETA_MAX = 8.0
FLOOR_MIN = 0.25


def raw_inputs(batch=2, time=9, heads=3, dim=8, value_dim=12, seed=0):
    rng = np.random.default_rng(seed)
    return dict(
        key=rng.normal(size=(batch, time, heads, dim)),
        query=rng.normal(size=(batch, time, heads, dim)),
        beta_raw=rng.normal(size=(batch, time, heads)),
        dt_raw=rng.normal(size=(batch, time, heads)),
        beta_bias=rng.normal(size=heads),
        dt_bias=rng.normal(size=heads) - 2.0,
        a_log=rng.uniform(0.0, math.log(16.0), size=heads),
        floor_raw=rng.normal(size=(heads, dim)),
        previous=rng.normal(size=(batch, heads, dim)),
        read=rng.normal(size=(batch, time, heads, value_dim)),
        variance=rng.uniform(0.0, 30.0, size=(batch, time, heads)),
        value=rng.normal(size=(batch, time, heads, value_dim)),
        confidence_scale=rng.uniform(0.05, 0.5, size=heads),
        skip=rng.normal(size=heads),
    )


PROLOGUE_ARGS = ["key", "query", "beta_raw", "dt_raw", "beta_bias", "dt_bias", "a_log", "floor_raw"]


def _inverse_softplus(x):
    return math.log(math.expm1(x))


def test_prologue_known_answers():
    x = raw_inputs()
    heads, dim = x["floor_raw"].shape
    # Parameterisation of lm/models/mamba4.py:196-237.  beta starts at 1/2
    # whatever beta_max (lm/tests/test_mamba4.py:326-332): with
    # start = 0.5 / max(beta_max, 1) the bias is log(start / (1 - start)).
    start = 0.5 / max(BETA_MAX, 1.0)
    bias = np.full(heads, math.log(start / (1 - start)))
    floor_init = 1.0
    floor_raw = np.full((heads, dim), _inverse_softplus(floor_init - FLOOR_MIN))
    dt = 0.05
    keys, queries, beta, log_decay, floor, shifted = oracle.prologue(
        x["key"], x["query"], np.zeros_like(x["beta_raw"]), np.zeros_like(x["dt_raw"]),
        bias, np.full(heads, _inverse_softplus(dt)), np.zeros(heads), floor_raw,
        beta_max=BETA_MAX, floor_min=FLOOR_MIN)
    np.testing.assert_allclose(beta, 0.5, rtol=1e-12)
    np.testing.assert_allclose(floor, floor_init, rtol=1e-12)
    np.testing.assert_allclose(log_decay, -dt, rtol=1e-12)  # -exp(0) * softplus(inv(dt))
    # Key shift: position 0 writes under a zero key (lm/tests/test_mamba4.py:364-375),
    # position t under the raw key of t - 1, and the cache keeps the last raw key.
    np.testing.assert_array_equal(keys[:, 0], 0.0)
    np.testing.assert_array_equal(shifted, x["key"][:, -1])
    norms = np.linalg.norm(x["key"][:, :-1], axis=-1)
    np.testing.assert_allclose(np.linalg.norm(keys[:, 1:], axis=-1),
                               norms / np.sqrt(norms**2 + 1e-6), rtol=1e-12)
    cosine = np.sum(keys[:, 1:] * x["key"][:, :-1], -1) / np.linalg.norm(keys[:, 1:], axis=-1)
    np.testing.assert_allclose(cosine, norms, rtol=1e-12)
    qn = np.linalg.norm(x["query"], axis=-1)
    np.testing.assert_allclose(np.linalg.norm(queries, axis=-1), qn / np.sqrt(qn**2 + 1e-6),
                               rtol=1e-12)
    # Without the shift the keys are only normalised.
    k2 = oracle.prologue(*(x[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX,
                         floor_min=FLOOR_MIN, key_shift=False)[0]
    kn = np.linalg.norm(x["key"], axis=-1, keepdims=True)
    np.testing.assert_allclose(k2, x["key"] / np.sqrt(kn**2 + 1e-6), rtol=1e-12)
    # beta lies in (0, beta_max); the floor stays above floor_min.
    _, _, beta, log_decay, floor, _ = oracle.prologue(
        *(x[n] * 3 for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN)
    assert np.all((beta > 0) & (beta < BETA_MAX)) and np.all(floor > FLOOR_MIN)
    assert np.all(log_decay < 0)


def test_prologue_shift_and_cache_continuation():
    # The cached decode path (lm/models/mamba4.py:185-195) feeds the last raw
    # key of one call as `previous` of the next: the split run equals the
    # full run.
    x = raw_inputs(time=10)
    args = [x[n] for n in PROLOGUE_ARGS]
    full = oracle.prologue(*args, beta_max=BETA_MAX, floor_min=FLOOR_MIN, previous=x["previous"])
    split = 4
    a = [v[:, :split] if v.ndim >= 3 else v for v in args]
    b = [v[:, split:] if v.ndim >= 3 else v for v in args]
    first = oracle.prologue(*a, beta_max=BETA_MAX, floor_min=FLOOR_MIN, previous=x["previous"])
    second = oracle.prologue(*b, beta_max=BETA_MAX, floor_min=FLOOR_MIN, previous=first[5])
    for i in range(4):
        np.testing.assert_allclose(np.concatenate([first[i], second[i]], axis=1), full[i],
                                   rtol=1e-13)
    np.testing.assert_array_equal(second[5], full[5])
    # previous takes the place of the zero key at position 0.
    pn = np.linalg.norm(x["previous"], axis=-1, keepdims=True)
    np.testing.assert_allclose(full[0][:, 0], x["previous"] / np.sqrt(pn**2 + 1e-6), rtol=1e-12)


def _prologue_loss(x, cot, prologue=oracle.prologue):
    out = prologue(*(x[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN,
                   previous=x["previous"])
    names = ["d_keys", "d_queries", "d_beta", "d_log_decay", "d_floor", "d_shifted"]
    return sum(np.sum(o * cot[n]) for o, n in zip(out, names))


def _prologue_cotangents(x, seed=5):
    rng = np.random.default_rng(seed)
    return dict(
        d_keys=rng.normal(size=x["key"].shape), d_queries=rng.normal(size=x["query"].shape),
        d_beta=rng.normal(size=x["beta_raw"].shape), d_log_decay=rng.normal(size=x["dt_raw"].shape),
        d_floor=rng.normal(size=x["floor_raw"].shape), d_shifted=rng.normal(size=x["previous"].shape),
    )


GRAD_OF = {
    "key": "d_key", "query": "d_query", "beta_raw": "d_beta_raw", "dt_raw": "d_dt_raw",
    "beta_bias": "d_beta_bias", "dt_bias": "d_dt_bias", "a_log": "d_a_log",
    "floor_raw": "d_floor_raw", "previous": "d_previous",
}


def _directional_errors(backward):
    x = raw_inputs(time=6, heads=2, dim=5, seed=3)
    cot = _prologue_cotangents(x)
    grads = backward(*(x[n] for n in PROLOGUE_ARGS), *(cot[n] for n in
                     ["d_keys", "d_queries", "d_beta", "d_log_decay", "d_floor", "d_shifted"]),
                     beta_max=BETA_MAX, previous=x["previous"])
    rng = np.random.default_rng(11)
    errors = {}
    for name, gname in GRAD_OF.items():
        u = rng.normal(size=x[name].shape)
        h = 1e-6
        plus, minus = dict(x), dict(x)
        plus[name] = x[name] + h * u
        minus[name] = x[name] - h * u
        fd = (_prologue_loss(plus, cot) - _prologue_loss(minus, cot)) / (2 * h)
        an = np.sum(grads[gname] * u)
        errors[name] = abs(fd - an) / max(abs(fd), 1e-3)
    return errors


def test_prologue_backward_matches_central_differences():
    errors = _directional_errors(oracle.prologue_backward)
    assert max(errors.values()) < 1e-6, errors


def test_prologue_backward_planted_mistakes_are_caught():
    # Each mistake, planted in a copy of the oracle's VJP, must fail the check.
    def drop_projection(*a, **k):
        g = oracle.prologue_backward(*a, **k)
        x = a[0]
        src = np.concatenate([k["previous"][:, None], x[:, :-1]], axis=1)
        r = 1 / np.sqrt(np.sum(src * src, -1, keepdims=True) + 1e-6)
        g["d_key"][:, :-1] = (r * a[8])[:, 1:]  # d_keys * r without -y (y.dy)
        return g

    def no_shifted_cotangent(*a, **k):
        g = oracle.prologue_backward(*a[:13], None, **k)
        return g

    def wrong_a_log_sign(*a, **k):
        g = oracle.prologue_backward(*a, **k)
        g["d_a_log"] = -g["d_a_log"]
        return g

    def sigmoid_not_derivative(*a, **k):
        g = oracle.prologue_backward(*a, **k)
        s = 1 / (1 + np.exp(-(a[2] + a[4])))
        g["d_beta_raw"] = a[10] * BETA_MAX * s
        g["d_beta_bias"] = np.sum(g["d_beta_raw"], axis=(0, 1))
        return g

    for planted in (drop_projection, no_shifted_cotangent, wrong_a_log_sign,
                    sigmoid_not_derivative):
        errors = _directional_errors(planted)
        assert max(errors.values()) > 1e-3, planted.__name__


def test_epilogue_known_answers():
    x = raw_inputs()
    args = [x[n] for n in ["read", "variance", "value", "confidence_scale", "skip"]]
    # No variance: the gate is sigmoid(1).
    out = oracle.epilogue(args[0], np.zeros_like(args[1]), args[2], args[3], np.zeros_like(args[4]))
    np.testing.assert_allclose(out, args[0] / (1 + math.exp(-1)), rtol=1e-12)
    # Nothing read: the skip passes D * value through.
    out = oracle.epilogue(np.zeros_like(args[0]), args[1], args[2], args[3], args[4])
    np.testing.assert_allclose(out, args[4][:, None] * args[2], rtol=1e-12)
    # gate = sigmoid(1 - s log1p(var)) at var = e - 1 is sigmoid(1 - s).
    var = np.full_like(args[1], math.e - 1)
    out = oracle.epilogue(args[0], var, args[2], args[3], np.zeros_like(args[4]))
    gate = 1 / (1 + np.exp(-(1 - args[3])))
    np.testing.assert_allclose(out, args[0] * gate[:, None], rtol=1e-12)


def test_epilogue_backward_matches_central_differences():
    x = raw_inputs(time=5, heads=2, value_dim=6, seed=4)
    names = ["read", "variance", "value", "confidence_scale", "skip"]
    d_out = np.random.default_rng(9).normal(size=x["read"].shape)
    grads = oracle.epilogue_backward(*(x[n] for n in names), d_out)
    rng = np.random.default_rng(12)
    for name in names:
        u = rng.normal(size=x[name].shape)
        h = 1e-6
        plus, minus = dict(x), dict(x)
        plus[name] = x[name] + h * u
        minus[name] = x[name] - h * u
        fd = (np.sum(d_out * oracle.epilogue(*(plus[n] for n in names)))
              - np.sum(d_out * oracle.epilogue(*(minus[n] for n in names)))) / (2 * h)
        an = np.sum(grads["d_" + name] * u)
        assert abs(fd - an) <= 1e-6 * max(abs(fd), 1e-3), name


# ------------------------------------------------------------------ GPU ----

def _gpu(x, names, grad=False):
    import torch

    return {n: torch.tensor(np.asarray(x[n], np.float32), device="cuda:0", requires_grad=grad)
            for n in names}


def _host(t):
    return t.detach().cpu().numpy().astype(np.float64)


def _close(actual, expected, rtol=2e-5, atol=2e-6, what=""):
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=atol, err_msg=what)


@pytest.mark.gpu
@pytest.mark.parametrize("dim,shift,with_previous", [(64, True, False), (64, True, True),
                                                     (8, False, False), (12, True, True)])
def test_gpu_prologue_matches_oracle(gpu_lib, dim, shift, with_previous):
    from gpu_helpers import announce
    from mamba4_amd import memory_inputs

    announce(f"mixer prologue dim={dim} shift={shift} previous={with_previous}")
    x = raw_inputs(batch=2, time=37, heads=3, dim=dim, seed=7)
    names = PROLOGUE_ARGS + ["previous"]
    t = _gpu(x, names, grad=True)
    prev = t["previous"] if with_previous else None
    out = memory_inputs(*(t[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN,
                        key_shift=shift, previous=prev)
    ref = oracle.prologue(*(x[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX,
                          floor_min=FLOOR_MIN, key_shift=shift,
                          previous=x["previous"] if with_previous else None)
    for name, a, e in zip(out._fields, out, ref):
        if e is None:
            assert a is None
            continue
        _close(_host(a), e, what=name)
    cot = _prologue_cotangents(x)
    cot_names = ["d_keys", "d_queries", "d_beta", "d_log_decay", "d_floor", "d_shifted"]
    loss = sum((o * _gpu(cot, [c])[c]).sum() for o, c in zip(out, cot_names) if o is not None)
    loss.backward()
    grads = oracle.prologue_backward(
        *(x[n] for n in PROLOGUE_ARGS), *(cot[c] for c in cot_names[:5]),
        cot["d_shifted"] if shift else None, beta_max=BETA_MAX, key_shift=shift,
        previous=x["previous"] if with_previous else None)
    for name in PROLOGUE_ARGS:
        _close(_host(t[name].grad), grads[GRAD_OF[name]], rtol=2e-5, atol=2e-5, what=name)
    if with_previous:
        expected = grads["d_previous"] if shift else np.zeros_like(x["previous"])
        _close(_host(t["previous"].grad), expected, rtol=2e-5, atol=2e-5, what="previous")


@pytest.mark.gpu
def test_gpu_prologue_cache_continuation_and_errors(gpu_lib):
    import torch

    from gpu_helpers import announce
    from mamba4_amd import memory_inputs

    announce("mixer prologue cache continuation")
    x = raw_inputs(batch=2, time=12, heads=2, dim=64, seed=8)
    t = _gpu(x, PROLOGUE_ARGS)
    full = memory_inputs(*(t[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN)
    cut = 5
    head = [t[n][:, :cut] if t[n].dim() >= 3 else t[n] for n in PROLOGUE_ARGS]
    tail = [t[n][:, cut:] if t[n].dim() >= 3 else t[n] for n in PROLOGUE_ARGS]
    first = memory_inputs(*head, beta_max=BETA_MAX, floor_min=FLOOR_MIN)
    second = memory_inputs(*tail, beta_max=BETA_MAX, floor_min=FLOOR_MIN, previous=first.shifted)
    for i in range(4):
        torch.testing.assert_close(torch.cat([first[i], second[i]], 1), full[i], rtol=0, atol=0)
    torch.testing.assert_close(second.shifted, full.shifted, rtol=0, atol=0)
    with pytest.raises(ValueError, match="memory_beta_max"):
        memory_inputs(*(t[n] for n in PROLOGUE_ARGS), beta_max=0.0)
    with pytest.raises(ValueError, match="floor"):
        memory_inputs(*(t[n] for n in PROLOGUE_ARGS), floor_min=0.0)


@pytest.mark.gpu
@pytest.mark.parametrize("value_dim", [64, 12, 128])
def test_gpu_epilogue_matches_oracle(gpu_lib, value_dim):
    from gpu_helpers import announce
    from mamba4_amd import gated_read

    announce(f"mixer epilogue value_dim={value_dim}")
    x = raw_inputs(batch=2, time=21, heads=3, value_dim=value_dim, seed=9)
    names = ["read", "variance", "value", "confidence_scale", "skip"]
    t = _gpu(x, names, grad=True)
    out = gated_read(*(t[n] for n in names))
    _close(_host(out), oracle.epilogue(*(x[n] for n in names)), what="out")
    d_out = np.random.default_rng(10).normal(size=x["read"].shape)
    (out * _gpu({"d": d_out}, ["d"])["d"]).sum().backward()
    grads = oracle.epilogue_backward(*(x[n] for n in names), d_out)
    for n in names:
        _close(_host(t[n].grad), grads["d_" + n], rtol=2e-5, atol=2e-5, what=n)


@pytest.mark.gpu
@pytest.mark.parametrize("value_dim", [64, 128])
def test_gpu_mixer_memory_path_end_to_end(gpu_lib, value_dim):
    """memory_inputs -> selective_gaussian_memory -> gated_read, the memory
    path of SelectiveMemoryMixer.__call__ (lm/models/mamba4.py:183-273), with
    gradients for every raw input and parameter against the composed float64
    oracle (oracle.mixer around oracle.memread)."""
    from gpu_helpers import announce, normwise
    from mamba4_amd import gated_read, memory_inputs, selective_gaussian_memory
    from oracle import memread

    announce(f"mixer memory path end to end value_dim={value_dim}")
    x = raw_inputs(batch=2, time=80, heads=2, dim=64, value_dim=value_dim, seed=13)
    names = PROLOGUE_ARGS + ["value", "confidence_scale", "skip"]
    t = _gpu(x, names, grad=True)
    inputs = memory_inputs(*(t[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX,
                           floor_min=FLOOR_MIN)
    result = selective_gaussian_memory(inputs.keys, t["value"], inputs.queries, inputs.beta,
                                       inputs.log_decay, inputs.floor, chunk_size=64)
    out = gated_read(result.output, result.variance, t["value"], t["confidence_scale"],
                     t["skip"])
    d_out = np.random.default_rng(14).normal(size=out.shape)
    (out * _gpu({"d": d_out}, ["d"])["d"]).sum().backward()

    keys, queries, beta, log_decay, floor, _ = oracle.prologue(
        *(x[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN)
    (read, variance, _, _), res = memread.forward(keys, x["value"], queries, beta, log_decay,
                                                  floor, chunk=64)
    expected = oracle.epilogue(read, variance, x["value"], x["confidence_scale"], x["skip"])
    assert normwise(_host(out), expected) <= 1e-4
    ge = oracle.epilogue_backward(read, variance, x["value"], x["confidence_scale"], x["skip"],
                                  d_out)
    gm = memread.backward(res, ge["d_read"], ge["d_variance"])
    gp = oracle.prologue_backward(*(x[n] for n in PROLOGUE_ARGS), gm["keys"], gm["queries"],
                                  gm["beta"], gm["log_decay"], gm["floor"], None,
                                  beta_max=BETA_MAX)
    expected_grads = {GRAD_OF[n][2:]: gp[GRAD_OF[n]] for n in PROLOGUE_ARGS}
    expected_grads["value"] = gm["values"] + ge["d_value"]
    expected_grads["confidence_scale"] = ge["d_confidence_scale"]
    expected_grads["skip"] = ge["d_skip"]
    for n in names:
        err = normwise(_host(t[n].grad), expected_grads[n])
        assert err <= 1e-3, (n, err)
