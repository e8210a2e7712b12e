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


def device_tokens(gen, shape, shift, decay_mean=3.0):
    """Config-0 distributions drawn on the GPU with a torch generator: q, k
    unit-norm N(0,1), v N(0,1), beta = sigmoid(N(0,1)), log_decay =
    log sigmoid(N(decay_mean, 1)); with ``shift`` the keys move one position
    along axis 1 (a zero key first).  Returns contiguous float32
    (keys, values, queries, beta, log_decay) of shape ``shape + (64,)`` and
    ``shape``."""
    import torch
    import torch.nn.functional as F

    kw = dict(device=gen.device, generator=gen, dtype=torch.float32)
    q = torch.randn(*shape, 64, **kw)
    k = torch.randn(*shape, 64, **kw)
    q = q / q.norm(dim=-1, keepdim=True)
    k = k / k.norm(dim=-1, keepdim=True)
    if shift:
        k = torch.cat([torch.zeros_like(k[:, :1]), k[:, :-1]], dim=1)
    v = torch.randn(*shape, 64, **kw)
    log_decay = -F.softplus(-(torch.randn(*shape, **kw) + decay_mean))
    beta = torch.sigmoid(torch.randn(*shape, **kw))
    return [t.contiguous() for t in (k, v, q, beta, log_decay)]


def decode_states(batch=2048, heads=8, context=1024, seed=0, slice_rows=128, keep_rows=()):
    """BASELINE config 4's resident states on cuda:0: the end states (S, C)
    [batch, heads, 64, 64] of a ``context``-token gated recurrence with
    config-0 distributions and lambda = sigmoid(N(3,1)) (``device_tokens``),
    built slice by slice with this library's forward, which stores no factors
    (no gradient is taken).  Floor 1e-2.  Returns (evidence, cross, floor,
    kept) where ``kept`` maps each row of ``keep_rows`` to its prefill inputs
    as float64 host arrays (for checking its end state)."""
    import torch

    from mamba4_amd import memory

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    f32 = dict(dtype=torch.float32, device=dev)
    evidence = torch.empty(batch, heads, 64, 64, **f32)
    cross = torch.empty(batch, heads, 64, 64, **f32)
    floor = torch.full((heads, 64), 1e-2, **f32)
    kept = {}
    for first in range(0, batch, slice_rows):
        rows = min(slice_rows, batch - first)
        k, v, q, beta, log_decay = device_tokens(gen, (rows, context, heads), shift=True)
        with torch.no_grad():
            out = memory.memread_forward(k, v, q, beta, log_decay, floor, None, None, 64,
                                         store_factors=False)
        evidence[first:first + rows] = out[2]
        cross[first:first + rows] = out[3]
        for r in keep_rows:
            if first <= r < first + rows:
                kept[r] = {n: t[r - first].double().cpu().numpy() for n, t in
                           zip(("keys", "values", "queries", "beta", "log_decay"),
                               (k, v, q, beta, log_decay))}
        del k, v, q, beta, log_decay, out
    torch.cuda.synchronize()
    return evidence, cross, floor, kept


def reference_benchmark_inputs(batch=16, length=1024, heads=12, dim=64, width=128, seed=0):
    """The reference's own memory-read benchmark inputs
    (scripts/kernel_benchmark.py:214-224, the shape its published TPU v4
    timings use, lm/results/speed-125m/bench-kernels.json:284-291): unit
    N(0,1) keys and queries (no key shift), N(0,1) values, beta ~ U(0.05, 1),
    log_decay = log U(0.9, 0.999), floor ~ U(0.25, 1.5) per (head, column),
    drawn in that order from default_rng(seed).  Its fwd+bwd differentiates
    a fixed projection of the outputs (projected_loss, :37-47): the
    cotangents are cos(i * 1.7) on the output and cos(i * 2.7) on the
    variance, i the flat index (in float32, as there).  Returns float32 arrays, cotangents
    included."""
    rng = np.random.default_rng(seed)
    k = rng.normal(size=(batch, length, heads, dim))
    q = rng.normal(size=k.shape)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    v = rng.normal(size=(batch, length, heads, width))
    beta = rng.uniform(0.05, 1.0, size=k.shape[:-1])
    log_decay = np.log(rng.uniform(0.9, 0.999, size=k.shape[:-1]))
    floor = rng.uniform(0.25, 1.5, size=(heads, dim))
    out = {n: a.astype(np.float32) for n, a in
           dict(keys=k, values=v, queries=q, beta=beta, log_decay=log_decay,
                floor=floor).items()}
    # As projected_loss forms them: a float32 index times float32 (index + 1.7).
    for name, like, factor in (("d_output", v, 1.7), ("d_variance", beta, 2.7)):
        phase = np.arange(like.size, dtype=np.float32) * np.float32(factor)
        out[name] = np.cos(phase).astype(np.float32).reshape(like.shape)
    return out


# The Mamba-3 scan's nine inputs, in the order of mamba3_fused's arguments
# (lm/kernels/flashmamba.py:1125-1162) and of m3s_forward.
MAMBA3_ARGS = ["c", "b", "x", "adt", "dt", "trap", "angles", "q_bias", "k_bias"]


def mamba3_inputs(batch=2, length=37, heads=3, dim=16, width=8, angle_count=4, seed=0):
    """Seeded float64 inputs of the Mamba-3 scan in the reference tests'
    ranges (lm/tests/test_flashmamba.py:104-118): standard-normal rows, dt a
    softplus of N(-1, 1), adt = -dt * U(0.5, 2), N(0,1) trap logits and
    angle rates, biases 0.1 N(0,1)."""
    rng = np.random.default_rng(seed)
    c = rng.normal(size=(batch, length, dim))
    b = rng.normal(size=(batch, length, dim))
    x = rng.normal(size=(batch, length, heads * width))
    dt = np.log1p(np.exp(rng.normal(size=(batch, length, heads)) - 1))
    adt = -dt * rng.uniform(0.5, 2.0, size=dt.shape)
    trap = rng.normal(size=dt.shape)
    angles = rng.normal(size=(batch, length, angle_count))
    q_bias = rng.normal(size=(heads, dim)) * 0.1
    k_bias = rng.normal(size=(heads, dim)) * 0.1
    return dict(c=c, b=b, x=x, adt=adt, dt=dt, trap=trap, angles=angles, q_bias=q_bias,
                k_bias=k_bias)
