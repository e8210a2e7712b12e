"""NumPy restatement of the memory mixer's prologue and epilogue -- TEST
INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, as the checker of the HIP
library; the product path never routes through it.

The memory read's caller (``SelectiveMemoryMixer.__call__``,
lm/models/mamba4.py:126-337) turns its projections into the operator's
inputs and gates the operator's reads.  Restated here in float64:

* ``prologue`` (lm/models/mamba4.py:183-237): the key shift (each value is
  written under the previous position's key; position 0 takes the cached key
  or zero, :183-195), unit normalisation ``x * rsqrt(sum x^2 + 1e-6)``
  (``_unit``, :37-39), ``beta = beta_max * sigmoid(beta_raw + beta_bias)``
  (:196-210), ``log_decay = -exp(a_log) * softplus(dt_raw + dt_bias)``
  (:211-221) and ``floor = floor_min + softplus(floor_raw)`` (:231-237).
* ``prologue_backward``: its closed-form VJP for every input and parameter.
* ``epilogue`` (lm/models/mamba4.py:266-273): the confidence gate
  ``read * sigmoid(1 - confidence_scale * log1p(variance))`` and the skip
  ``+ D * value``.
* ``epilogue_backward``: its closed-form VJP.

Shapes: key and query ``[B,T,H,D]``, beta_raw and dt_raw ``[B,T,H]``,
beta_bias, dt_bias, a_log, confidence_scale and D ``[H]``, floor_raw
``[H,D]``, previous (the cached raw key) ``[B,H,D]``, read and value
``[B,T,H,P]``, variance ``[B,T,H]``.

``PINNED`` names the tests that pin each function (known answers from the
reference's own tests and parameterisation, invariants, and central finite
differences for the VJPs).
"""

import numpy as np

EPS = 1e-6  # _unit, lm/models/mamba4.py:37-39

PINNED = {
    "prologue": [
        "tests/test_mixer.py::test_prologue_known_answers",
        "tests/test_mixer.py::test_prologue_shift_and_cache_continuation",
    ],
    "prologue_backward": [
        "tests/test_mixer.py::test_prologue_backward_matches_central_differences",
        "tests/test_mixer.py::test_prologue_backward_planted_mistakes_are_caught",
    ],
    "epilogue": [
        "tests/test_mixer.py::test_epilogue_known_answers",
    ],
    "epilogue_backward": [
        "tests/test_mixer.py::test_epilogue_backward_matches_central_differences",
    ],
}


def _sigmoid(x):
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def _softplus(x):
    return np.logaddexp(0.0, x)


def _shift(key, previous):
    """Keys of the previous position; position 0 takes ``previous`` (or zero)."""
    first = np.zeros_like(key[:, :1]) if previous is None else previous[:, None]
    return np.concatenate([first, key[:, :-1]], axis=1)


def _unit(x):
    """x * rsqrt(sum x^2 + 1e-6) over the last axis (lm/models/mamba4.py:37-39)."""
    return x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + EPS)


def prologue(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, *,
             beta_max=1.0, floor_min=0.25, key_shift=True, previous=None):
    """The memory read's inputs from the mixer's projections.

    Returns ``(keys, queries, beta, log_decay, floor, shifted)``; ``shifted``
    is the raw key of the last position (the cache entry the next call takes
    as ``previous``, lm/models/mamba4.py:191-195), or None without the shift.
    """
    f = np.float64
    key, query = np.asarray(key, f), np.asarray(query, f)
    shifted = None
    if key_shift:
        shifted = key[:, -1].copy()
        key = _shift(key, None if previous is None else np.asarray(previous, f))
    keys, queries = _unit(key), _unit(query)
    beta = beta_max * _sigmoid(np.asarray(beta_raw, f) + np.asarray(beta_bias, f))
    dt = _softplus(np.asarray(dt_raw, f) + np.asarray(dt_bias, f))
    log_decay = -np.exp(np.asarray(a_log, f)) * dt
    floor = floor_min + _softplus(np.asarray(floor_raw, f))
    return keys, queries, beta, log_decay, floor, shifted


def _unit_vjp(x, dy):
    """VJP of _unit: r (dy - y (y . dy)) with r = rsqrt(|x|^2 + eps), y = x r."""
    r = 1.0 / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + EPS)
    y = x * r
    return r * (dy - y * np.sum(y * dy, axis=-1, keepdims=True))


def prologue_backward(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                      d_keys, d_queries, d_beta, d_log_decay, d_floor, d_shifted=None, *,
                      beta_max=1.0, key_shift=True, previous=None):
    """Closed-form VJP of ``prologue``.

    Returns a dict with d_key, d_query, d_beta_raw, d_dt_raw, d_beta_bias,
    d_dt_bias, d_a_log, d_floor_raw and d_previous (None when ``previous`` is
    None or without the shift).
    """
    f = np.float64
    key, query = np.asarray(key, f), np.asarray(query, f)
    d_keys, d_queries = np.asarray(d_keys, f), np.asarray(d_queries, f)
    src = key
    if key_shift:
        src = _shift(key, None if previous is None else np.asarray(previous, f))
    d_src = _unit_vjp(src, d_keys)
    d_query = _unit_vjp(query, d_queries)
    d_previous = None
    if key_shift:
        d_key = np.zeros_like(key)
        d_key[:, :-1] = d_src[:, 1:]
        if d_shifted is not None:
            d_key[:, -1] += np.asarray(d_shifted, f)
        if previous is not None:
            d_previous = d_src[:, 0].copy()
    else:
        d_key = d_src
    z = np.asarray(beta_raw, f) + np.asarray(beta_bias, f)
    s = _sigmoid(z)
    d_beta_raw = np.asarray(d_beta, f) * beta_max * s * (1.0 - s)
    u = np.asarray(dt_raw, f) + np.asarray(dt_bias, f)
    rate = np.exp(np.asarray(a_log, f))
    d_dt_raw = np.asarray(d_log_decay, f) * (-rate) * _sigmoid(u)
    d_a_log = np.sum(np.asarray(d_log_decay, f) * (-rate * _softplus(u)), axis=(0, 1))
    d_floor_raw = np.asarray(d_floor, f) * _sigmoid(np.asarray(floor_raw, f))
    return dict(
        d_key=d_key, d_query=d_query, d_beta_raw=d_beta_raw, d_dt_raw=d_dt_raw,
        d_beta_bias=np.sum(d_beta_raw, axis=(0, 1)), d_dt_bias=np.sum(d_dt_raw, axis=(0, 1)),
        d_a_log=d_a_log, d_floor_raw=d_floor_raw, d_previous=d_previous,
    )


def epilogue(read, variance, value, confidence_scale, skip):
    """read * sigmoid(1 - scale * log1p(variance)) + D * value (lm/models/mamba4.py:266-273)."""
    f = np.float64
    gate = _sigmoid(1.0 - np.asarray(confidence_scale, f) * np.log1p(np.asarray(variance, f)))
    return np.asarray(read, f) * gate[..., None] + np.asarray(skip, f)[:, None] * np.asarray(value, f)


def epilogue_backward(read, variance, value, confidence_scale, skip, d_out):
    """Closed-form VJP of ``epilogue``: d_read, d_variance, d_value,
    d_confidence_scale and d_skip."""
    f = np.float64
    read, value, d_out = np.asarray(read, f), np.asarray(value, f), np.asarray(d_out, f)
    variance, scale = np.asarray(variance, f), np.asarray(confidence_scale, f)
    log_var = np.log1p(variance)
    gate = _sigmoid(1.0 - scale * log_var)
    slope = np.sum(d_out * read, axis=-1) * gate * (1.0 - gate)
    return dict(
        d_read=d_out * gate[..., None],
        d_variance=slope * (-scale / (1.0 + variance)),
        d_value=d_out * np.asarray(skip, f)[:, None],
        d_confidence_scale=np.sum(slope * (-log_var), axis=(0, 1)),
        d_skip=np.sum(d_out * value, axis=(0, 1, 3)),
    )
