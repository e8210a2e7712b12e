"""Seeded synthetic inputs for the memory-read workloads.

One generator, ``numpy.random.default_rng(seed)``, with a fixed draw order:
queries, keys, values, decay logits, beta logits, then (optionally) the
cotangents of output and variance.  The distributions follow the caller's
preprocessing in lm/models/mamba4.py:183-237:

* q, k ~ N(0,1) per element, L2-normalised per token (``_unit``, :37-39);
* keys are shifted so each value is written under the previous position's
  key and the first position writes with a zero key (:183-194);
* v ~ N(0,1); log_decay = log sigmoid(x) = -softplus(-x) with
  x ~ N(decay_mean, 1); beta = sigmoid(N(0,1)); floor = floor_value * 1.

Named workloads mirror the benchmark configurations: ``config0`` (B2 L256
H1), ``config2`` (B16 L1024 H8), ``config3`` (B32 L1024 H12, decay logits
N(4,1), q/k/v rounded to bf16 after normalisation), ``config4`` (decode
states, decay logits N(3,1)).
"""

import numpy as np

WORKLOADS = {
    "config0": dict(batch=2, time=256, heads=1, decay_mean=2.0),
    "config1": dict(batch=16, time=1024, heads=8, decay_mean=2.0),
    "config2": dict(batch=16, time=1024, heads=8, decay_mean=2.0),
    "config3": dict(batch=32, time=1024, heads=12, decay_mean=4.0, bf16=True),
    "config4": dict(batch=2048, time=1024, heads=8, decay_mean=3.0),
}


def _softplus(x):
    return np.logaddexp(0.0, x)


def _unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def round_to_bf16(x):
    """Round float32 values to the nearest bfloat16 (ties to even)."""
    bits = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return rounded.astype(np.uint32).view(np.float32)


def synthetic_inputs(
    batch,
    time,
    heads,
    key_dim=64,
    value_dim=64,
    decay_mean=2.0,
    floor_value=1e-2,
    seed=0,
    cotangents=False,
    shift_keys=True,
    bf16=False,
):
    """Return a dict of float32 arrays: keys, values, queries, beta,
    log_decay, floor and, with ``cotangents``, d_output and d_variance."""
    rng = np.random.default_rng(seed)
    queries = _unit(rng.normal(size=(batch, time, heads, key_dim)))
    keys = _unit(rng.normal(size=(batch, time, heads, key_dim)))
    values = rng.normal(size=(batch, time, heads, value_dim))
    decay_logits = rng.normal(decay_mean, 1.0, size=(batch, time, heads))
    beta_logits = rng.normal(0.0, 1.0, size=(batch, time, heads))
    out = {}
    if cotangents:
        out["d_output"] = rng.normal(size=(batch, time, heads, value_dim)).astype(
            np.float32
        )
        out["d_variance"] = rng.normal(size=(batch, time, heads)).astype(np.float32)
    if shift_keys:
        keys = np.concatenate((np.zeros_like(keys[:, :1]), keys[:, :-1]), axis=1)
    out.update(
        keys=keys.astype(np.float32),
        values=values.astype(np.float32),
        queries=queries.astype(np.float32),
        beta=(1.0 / (1.0 + np.exp(-beta_logits))).astype(np.float32),
        log_decay=(-_softplus(-decay_logits)).astype(np.float32),
        floor=np.full((heads, key_dim), floor_value, np.float32),
    )
    if bf16:
        for name in ("keys", "values", "queries"):
            out[name] = round_to_bf16(out[name])
    return out


def workload_inputs(name, seed=0, cotangents=False, **overrides):
    spec = dict(WORKLOADS[name])
    spec.update(overrides)
    return synthetic_inputs(seed=seed, cotangents=cotangents, **spec)
