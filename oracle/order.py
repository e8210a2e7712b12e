"""NumPy restatement of the order head's gated vector scan -- TEST
INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, as the checker of the HIP
library; the product path never routes through it.

The memory mixer's order head (lm/models/mamba4.py:274-289) runs, per batch
row, head and channel, the scan ``h_t = lam_t h_(t-1) + (1 - lam_t) v_t``
from ``h_(-1) = 0``.  Restated here in float64:

* ``order_memory`` (lm/models/mamba4.py:46-56): the scan from the decays
  themselves, as the reference's associative scan computes it.
* ``order_memory_chunked`` (lm/models/mamba4.py:59-95): the same scan from
  log decays, in chunks: within a chunk one masked decay-weighted product
  with inflow ``1 - lam = -expm1(log lam)``, chunk ends combined by the
  decayed carry of lm/kernels/prefix.py:27-44, each chunk's reads taking
  ``exp(prefix)`` times the state it starts from.  ``initial`` (an addition
  of this build) is the state before the first token; the reference's cached
  decode step (lm/models/mamba4.py:283-287) is this scan over one token from
  the cached state.
* ``order_memory_backward``: the closed-form VJP of the chunked scan with
  respect to values, log decays and the initial state.

Shapes: values ``[B,T,H,W]``, decays and log decays ``[B,T,H]``, initial
``[B,H,W]``.

``PINNED`` names the tests that pin each function.
"""

import numpy as np

PINNED = {
    "order_memory": [
        "tests/test_order.py::test_sequential_scan_known_answers",
    ],
    "order_memory_chunked": [
        "tests/test_order.py::test_chunked_scan_matches_sequential_scan",
        "tests/test_order.py::test_sequential_scan_known_answers",
    ],
    "order_memory_backward": [
        "tests/test_order.py::test_backward_matches_finite_differences",
        "tests/test_order.py::test_backward_matches_autograd_of_the_recurrence",
        "tests/test_order.py::test_planted_backward_mistakes_are_caught",
    ],
}


def order_memory(values, decay, initial=None):
    """h_t = decay_t h_(t-1) + (1 - decay_t) v_t, token by token.

    The reference evaluates the same recurrence with lax.associative_scan
    over (decay, (1 - decay) v) pairs (lm/models/mamba4.py:46-56); the
    sequential form is its definition.
    """
    v = np.asarray(values, np.float64)
    lam = np.asarray(decay, np.float64)[..., None]
    batch, time, heads, width = v.shape
    state = (
        np.zeros((batch, heads, width)) if initial is None else np.array(initial, np.float64)
    )
    out = np.empty_like(v)
    for t in range(time):
        state = lam[:, t] * state + (1.0 - lam[:, t]) * v[:, t]
        out[:, t] = state
    return out


def order_memory_chunked(values, log_decay, chunk_size=64, initial=None):
    """Chunked form of the scan (lm/models/mamba4.py:59-95)."""
    x = np.asarray(values, np.float64)
    logs_in = np.asarray(log_decay, np.float64)
    batch, time, heads, width = x.shape
    padding = (-time) % chunk_size
    count = (time + padding) // chunk_size

    def chunks(a):
        a = np.pad(a, [(0, 0), (0, padding)] + [(0, 0)] * (a.ndim - 2))
        a = a.reshape(batch, count, chunk_size, *a.shape[2:])
        return np.swapaxes(a, 2, 3)  # [B, n, H, c, ...]

    value, logs = chunks(x), chunks(logs_in)
    inflow = -np.expm1(logs)
    prefix = np.cumsum(logs, axis=-1)  # cumulative (lm/kernels/prefix.py:17-24)
    position = np.arange(chunk_size)
    causal = position[:, None] >= position[None, :]
    difference = prefix[..., :, None] - prefix[..., None, :]
    weights = np.where(causal, np.exp(np.where(causal, difference, 0.0)), 0.0)
    local = np.einsum("bnhts,bnhsp->bnhtp", weights * inflow[..., None, :], value)
    # chunk_carry (lm/kernels/prefix.py:27-44) restated as its recurrence:
    # end_n = exp(total_n) end_(n-1) + local end_n.
    state = (
        np.zeros((batch, heads, width)) if initial is None else np.array(initial, np.float64)
    )
    starts = np.empty((batch, count, heads, width))
    for n in range(count):
        starts[:, n] = state
        state = np.exp(prefix[:, n, :, -1])[..., None] * state + local[:, n, :, -1]
    output = local + np.exp(prefix)[..., None] * starts[:, :, :, None, :]
    output = np.swapaxes(output, 2, 3).reshape(batch, count * chunk_size, heads, width)
    return output[:, :time]


def order_memory_backward(values, log_decay, d_output, initial=None):
    """VJP of the scan: (d_values, d_log_decay, d_initial).

    With g_t = dout_t + lam_(t+1) g_(t+1) (g past the end is zero), the
    cotangent reaching h_t, and h_t = lam_t h_(t-1) + (1 - lam_t) v_t:
      d v_t = (1 - lam_t) g_t,
      d log lam_t = lam_t sum_c g_t,c (h_(t-1),c - v_t,c),
      d initial = lam_0 g_0.
    """
    v = np.asarray(values, np.float64)
    logs = np.asarray(log_decay, np.float64)
    lam = np.exp(logs)[..., None]
    inflow = -np.expm1(logs)[..., None]
    dout = np.asarray(d_output, np.float64)
    batch, time, heads, width = v.shape
    h = order_memory_chunked(v, logs, chunk_size=max(time, 1), initial=initial)
    start = (
        np.zeros((batch, heads, width)) if initial is None else np.array(initial, np.float64)
    )
    previous = np.concatenate([start[:, None], h[:, :-1]], axis=1)
    g = np.zeros((batch, heads, width))
    d_values = np.empty_like(v)
    d_log = np.empty(logs.shape)
    for t in reversed(range(time)):
        g = dout[:, t] + (lam[:, t + 1] * g if t + 1 < time else 0.0)
        d_values[:, t] = inflow[:, t] * g
        d_log[:, t] = lam[:, t, :, 0] * np.sum(g * (previous[:, t] - v[:, t]), axis=-1)
    d_initial = lam[:, 0] * g if time > 0 else np.zeros_like(start)
    return d_values, d_log, d_initial
