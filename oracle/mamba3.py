"""Float64 restatement of the FlashMamba Mamba-3 SISO scan.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU baseline as the checker; the product path never calls it.

The operator is ``mamba3_fused`` (lm/kernels/flashmamba.py:1125-1162) over
``fused_scan`` (:901-957): one shared query row c_t and key row b_t per token
([B,T,N]), values x_t ([B,T,H*P]), per-head log decays adt, steps dt and
trapezoid logits ([B,T,H]), shared angle rates ([B,T,A], A <= N/2) and
per-head biases q_bias, k_bias ([H,N] or [H,1,N]).  Per head h:

    theta_t = sum_{s<=t} angles_s * dt_s                 (phase, no modulo)
    q_t = rot(c_t + q_bias, theta_t),  k_t = rot(b_t + k_bias, theta_t)
    sigma = sigmoid(trap), gamma = dt sigma, prev = dt (1 - sigma)
    h_t = exp(adt_t) (h_{t-1} + prev_t k_{t-1} v_{t-1}^T) + gamma_t k_t v_t^T
    y_t = q_t^T h_t

rot turns coordinate pair (2i, 2i+1) by theta_i for i < A and keeps the
rest (lm/kernels/mamba3.py:20-40 with pairwise=True).

Functions and what pins them (tests/test_mamba3_oracle.py):
  forward        token recurrence in the cumulative frame
                 (lm/kernels/mamba3.py:258-289, mamba3_sequential).  Pinned
                 against ``local_forward`` (a different formulation: the state
                 is turned by each step's phase increment, q and k are never
                 rotated), against ``chunked_forward`` (the chunk algebra), and
                 against a brute-force double sum for zero angles.
  local_forward  lm/kernels/mamba3.py:292-340 (numpy_reference).
  chunked_forward lm/kernels/mamba3.py:60-126 (mamba3_chunked_serial); also
                 returns each chunk's start state.
  backward       hand-derived reverse mode of ``forward`` for all nine
                 inputs; pinned by central finite differences.
"""

import numpy as np


def _heads(q_bias, heads, dim):
    q = np.zeros((heads, dim)) if q_bias is None else np.asarray(q_bias, np.float64)
    return q.reshape(heads, dim)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def phases(angles, dt):
    """theta [B,T,H,A] = inclusive running sum over t of angles * dt
    (lm/kernels/flashmamba.py:87-89, :1115-1122)."""
    inc = np.asarray(angles, np.float64)[:, :, None, :] * np.asarray(dt, np.float64)[..., None]
    return np.cumsum(inc, axis=1)


def rotate(u, theta):
    """Pairwise rotation of the last axis of u by theta (pairs i < A)."""
    out = np.array(u, np.float64, copy=True)
    a = theta.shape[-1]
    left, right = u[..., 0:2 * a:2], u[..., 1:2 * a:2]
    cos, sin = np.cos(theta), np.sin(theta)
    out[..., 0:2 * a:2] = left * cos - right * sin
    out[..., 1:2 * a:2] = left * sin + right * cos
    return out


def rotate_back(du, theta):
    """Transpose of ``rotate`` applied to a cotangent."""
    out = np.array(du, np.float64, copy=True)
    a = theta.shape[-1]
    dl, dr = du[..., 0:2 * a:2], du[..., 1:2 * a:2]
    cos, sin = np.cos(theta), np.sin(theta)
    out[..., 0:2 * a:2] = dl * cos + dr * sin
    out[..., 1:2 * a:2] = -dl * sin + dr * cos
    return out


def frame(c, b, dt, angles, q_bias, k_bias):
    """Rotated per-head queries and keys [B,T,H,N] and the phases."""
    c, b = np.asarray(c, np.float64), np.asarray(b, np.float64)
    heads, dim = np.shape(dt)[-1], c.shape[-1]
    qb, kb = _heads(q_bias, heads, dim), _heads(k_bias, heads, dim)
    theta = phases(angles, dt)
    q = rotate(c[:, :, None, :] + qb, theta)
    k = rotate(b[:, :, None, :] + kb, theta)
    return q, k, theta


def _weights(dt, trap):
    dt = np.asarray(dt, np.float64)
    s = sigmoid(np.asarray(trap, np.float64))
    return s, dt * s, dt * (1 - s)


def forward(c, b, x, adt, dt, trap, angles, q_bias=None, k_bias=None, initial=None):
    """y [B,T,H*P] and the final state [B,H,N,P] (float64)."""
    batch, length, heads = np.shape(dt)
    q, k, _ = frame(c, b, dt, angles, q_bias, k_bias)
    v = np.asarray(x, np.float64).reshape(batch, length, heads, -1)
    _, gamma, prev = _weights(dt, trap)
    alpha = np.exp(np.asarray(adt, np.float64))
    dim, width = q.shape[-1], v.shape[-1]
    state = np.zeros((batch, heads, dim, width)) if initial is None else \
        np.array(initial, np.float64)
    last = np.zeros_like(state)
    y = np.empty_like(v)
    for t in range(length):
        cur = k[:, t, :, :, None] * v[:, t, :, None, :]
        state = alpha[:, t, :, None, None] * (state + prev[:, t, :, None, None] * last) \
            + gamma[:, t, :, None, None] * cur
        y[:, t] = np.einsum("bhn,bhnp->bhp", q[:, t], state)
        last = cur
    return y.reshape(batch, length, heads * width), state


def local_forward(c, b, x, adt, dt, trap, angles, q_bias=None, k_bias=None):
    """The local-frame recurrence (lm/kernels/mamba3.py:292-340): q and k
    stay unrotated, the state turns by minus each step's phase increment."""
    batch, length, heads = np.shape(dt)
    c, b = np.asarray(c, np.float64), np.asarray(b, np.float64)
    dim = c.shape[-1]
    q = c[:, :, None, :] + _heads(q_bias, heads, dim)
    k = b[:, :, None, :] + _heads(k_bias, heads, dim)
    v = np.asarray(x, np.float64).reshape(batch, length, heads, -1)
    _, gamma, prev = _weights(dt, trap)
    alpha = np.exp(np.asarray(adt, np.float64))
    angles, dt = np.asarray(angles, np.float64), np.asarray(dt, np.float64)
    state = np.zeros((batch, heads, dim, v.shape[-1]))
    last = np.zeros_like(state)
    y = np.empty_like(v)

    def turn(s, delta):  # rotate the state's coordinate axis (axis -2) by delta
        return np.swapaxes(rotate(np.swapaxes(s, -1, -2), delta[:, :, None, :]), -1, -2)

    for t in range(length):
        delta = angles[:, t, None, :] * dt[:, t, :, None]
        cur = k[:, t, :, :, None] * v[:, t, :, None, :]
        a = alpha[:, t, :, None, None]
        state = a * turn(state, -delta) + prev[:, t, :, None, None] * a * turn(last, -delta) \
            + gamma[:, t, :, None, None] * cur
        y[:, t] = np.einsum("bhn,bhnp->bhp", q[:, t], state)
        last = cur
    return y.reshape(batch, length, -1), state


def chunked_forward(c, b, x, adt, dt, trap, angles, q_bias=None, k_bias=None, chunk=16):
    """Chunk form (lm/kernels/mamba3.py:60-126): within-chunk decayed scores
    with source weights scale_s = gamma_s + prev_{s+1}, the diagonal weighted
    by gamma_t, the carried state read through exp(p_t), and the chunk update
    weighted by scale_s exp(p_end - p_s).  Returns y, final, starts
    [B,H,chunks,N,P]."""
    batch, length, heads = np.shape(dt)
    q, k, _ = frame(c, b, dt, angles, q_bias, k_bias)
    v = np.asarray(x, np.float64).reshape(batch, length, heads, -1)
    _, gamma, prev = _weights(dt, trap)
    scale = gamma + np.concatenate([prev[:, 1:], np.zeros_like(prev[:, :1])], axis=1)
    adt = np.asarray(adt, np.float64)
    state = np.zeros((batch, heads, q.shape[-1], v.shape[-1]))
    y = np.empty_like(v)
    starts = []
    for c0 in range(0, length, chunk):
        sl = slice(c0, min(length, c0 + chunk))
        p = np.cumsum(adt[:, sl], axis=1)                      # [B,L,H]
        qc, kc, vc = q[:, sl], k[:, sl], v[:, sl]
        n = p.shape[1]
        lower = np.tril(np.ones((n, n)), -1)
        decay = np.exp(np.minimum(p[:, :, None, :] - p[:, None, :, :], 0.0))  # [B,t,s,H]
        w = decay * lower[None, :, :, None] * scale[:, sl][:, None, :, :]
        w = w + np.eye(n)[None, :, :, None] * gamma[:, sl][:, None, :, :]
        scores = np.einsum("bthn,bshn->btsh", qc, kc)
        within = np.einsum("btsh,bshp->bthp", scores * w, vc)
        inherited = np.einsum("bthn,bhnp->bthp", qc, state) * np.exp(p)[..., None]
        y[:, sl] = within + inherited
        starts.append(state)
        tail = np.exp(p[:, -1:] - p) * scale[:, sl]
        state = np.exp(p[:, -1])[..., None, None] * state + \
            np.einsum("bthn,bthp->bhnp", kc, vc * tail[..., None])
    return y.reshape(batch, length, -1), state, np.stack(starts, axis=2)


def backward(c, b, x, adt, dt, trap, angles, q_bias, k_bias, d_y, d_final=None):
    """Gradients of <y, d_y> + <final, d_final> with respect to all nine
    inputs, by reverse mode through ``forward`` (derived by hand)."""
    batch, length, heads = np.shape(dt)
    c, b = np.asarray(c, np.float64), np.asarray(b, np.float64)
    dim = c.shape[-1]
    qb, kb = _heads(q_bias, heads, dim), _heads(k_bias, heads, dim)
    theta = phases(angles, dt)
    qu, ku = c[:, :, None, :] + qb, b[:, :, None, :] + kb
    q, k = rotate(qu, theta), rotate(ku, theta)
    v = np.asarray(x, np.float64).reshape(batch, length, heads, -1)
    width = v.shape[-1]
    sig, gamma, prev = _weights(dt, trap)
    alpha = np.exp(np.asarray(adt, np.float64))
    dy = np.asarray(d_y, np.float64).reshape(batch, length, heads, width)

    # Forward again, keeping every state.
    states = np.zeros((length + 1, batch, heads, dim, width))
    curs = np.zeros_like(states)          # curs[t+1] = k_t v_t^T, curs[0] = 0
    for t in range(length):
        curs[t + 1] = k[:, t, :, :, None] * v[:, t, :, None, :]
        states[t + 1] = alpha[:, t, :, None, None] * (states[t] + prev[:, t, :, None, None]
                                                      * curs[t]) \
            + gamma[:, t, :, None, None] * curs[t + 1]

    dh = np.zeros((batch, heads, dim, width)) if d_final is None else \
        np.array(d_final, np.float64)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    d_alpha, d_gamma, d_prev = (np.zeros((batch, length, heads)) for _ in range(3))
    dh_next = np.zeros_like(dh)           # gradient of h_{t+1}
    for t in reversed(range(length)):
        dh = dh + q[:, t, :, :, None] * dy[:, t, :, None, :]
        if t + 1 < length:
            dh = dh + alpha[:, t + 1, :, None, None] * dh_next
        dq[:, t] = np.einsum("bhnp,bhp->bhn", states[t + 1], dy[:, t])
        d_cur = gamma[:, t, :, None, None] * dh
        if t + 1 < length:
            d_cur = d_cur + (alpha[:, t + 1] * prev[:, t + 1])[:, :, None, None] * dh_next
        dk[:, t] = np.einsum("bhnp,bhp->bhn", d_cur, v[:, t])
        dv[:, t] = np.einsum("bhnp,bhn->bhp", d_cur, k[:, t])
        d_alpha[:, t] = np.einsum("bhnp,bhnp->bh", dh,
                                  states[t] + prev[:, t, :, None, None] * curs[t])
        d_prev[:, t] = alpha[:, t] * np.einsum("bhnp,bhnp->bh", dh, curs[t])
        d_gamma[:, t] = np.einsum("bhnp,bhnp->bh", dh, curs[t + 1])
        dh_next, dh = dh, np.zeros_like(dh)

    d_adt = d_alpha * alpha
    d_dt = d_gamma * sig + d_prev * (1 - sig)
    d_trap = (d_gamma - d_prev) * np.asarray(dt, np.float64) * sig * (1 - sig)

    # Through the rotations: pair i turns by theta_i.
    a = theta.shape[-1]
    d_theta = (dq[..., 1:2 * a:2] * q[..., 0:2 * a:2] - dq[..., 0:2 * a:2] * q[..., 1:2 * a:2]
               + dk[..., 1:2 * a:2] * k[..., 0:2 * a:2] - dk[..., 0:2 * a:2] * k[..., 1:2 * a:2])
    dqu, dku = rotate_back(dq, theta), rotate_back(dk, theta)
    d_inc = np.flip(np.cumsum(np.flip(d_theta, 1), 1), 1)          # [B,T,H,A]
    angles = np.asarray(angles, np.float64)
    d_angles = np.einsum("btha,bth->bta", d_inc, np.asarray(dt, np.float64))
    d_dt = d_dt + np.einsum("btha,bta->bth", d_inc, angles)
    return {
        "c": dqu.sum(2), "b": dku.sum(2), "x": dv.reshape(batch, length, -1),
        "adt": d_adt, "dt": d_dt, "trap": d_trap, "angles": d_angles,
        "q_bias": dqu.sum((0, 1)), "k_bias": dku.sum((0, 1)),
    }


def inputs(batch=2, length=37, heads=3, dim=16, width=8, angle_count=4, seed=0):
    """Seeded inputs in the reference tests' ranges
    (lm/tests/test_flashmamba.py:104-118); the generator lives with the
    package's other synthetic inputs (mamba4_amd.inputs.mamba3_inputs)."""
    from mamba4_amd.inputs import mamba3_inputs

    return mamba3_inputs(batch, length, heads, dim, width, angle_count, seed)


ARGS = ["c", "b", "x", "adt", "dt", "trap", "angles", "q_bias", "k_bias"]
