"""Chunk-form restatement of FlashMamba's fused Mamba-3 kernels, with the
model-dtype rounding of their matrix operands.

TEST INFRASTRUCTURE ONLY: imported by tests/ and ``bench.py``'s CPU
baseline as the checker; the product path never calls it.

The reference's fused forward and backward kernels
(lm/kernels/flashmamba.py:589-660 and :663-786) multiply matrix operands in
the model dtype with float32 accumulation: for a bfloat16 model the rotated
queries and keys, the values, the masked score mixes, the carried states and
the scaled cotangents are rounded to bfloat16 where the kernels call
``.astype(model dtype)`` (:575-586, :634-659, :721-751); everything else is
float32.  ``fused_forward`` and ``fused_backward`` follow those kernels chunk
by chunk, with ``rnd`` applied at exactly those points, plus the glue around
them: the trapezoid weights and duplicated angle rates of ``mamba3_fused``
(:1113-1162) and the chunk-end terms and reverse prefix of
``_fused_backward`` (:1000-1108).

With ``rnd=None`` (no rounding) in float64 they are the exact chunk algebra,
pinned against the token recurrence of ``oracle.mamba3`` (forward, and the
finite-difference-pinned backward) in tests/test_mamba3_oracle.py;
``round_bf16`` is pinned against torch's bfloat16 conversion there.  With
``rnd=round_bf16`` in float32 they are the bfloat16 model's arithmetic, the
oracle of the library's bfloat16 scan entry points.
"""

import numpy as np

from oracle.mamba3 import _heads, sigmoid


def round_bf16(x):
    """x rounded to the nearest bfloat16 (ties to even), as float32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32)
    bias = ((u >> 16) & 1) + np.uint32(0x7FFF)
    return ((u + bias) & np.uint32(0xFFFF0000)).view(np.float32)


def _partner(x):
    """(-x[2i+1] at 2i, x[2i] at 2i+1) on the last axis (:566-572)."""
    out = np.empty_like(x)
    out[..., 0::2] = -x[..., 1::2]
    out[..., 1::2] = x[..., 0::2]
    return out


def _rates(angles, dim, dtype):
    """[B,T,A] angle rates on both coordinates of their pair (:1113-1122)."""
    a = np.asarray(angles, dtype)
    rates = np.zeros(a.shape[:2] + (dim,), dtype)
    rates[..., 0:2 * a.shape[-1]:2] = a
    rates[..., 1:2 * a.shape[-1]:2] = a
    return rates


def _glue(dt, trap, dtype):
    """gamma, scale and sigma of mamba3_fused (:1146-1150)."""
    s = sigmoid(np.asarray(trap, np.float64)).astype(dtype)
    dt = np.asarray(dt, dtype)
    gamma = dt * s
    prev = dt * (1 - s)
    scale = gamma + np.concatenate([prev[:, 1:], np.zeros_like(prev[:, :1])], axis=1)
    return gamma, scale, s


def _chunks(length, chunk):
    return [(c0, min(length, c0 + chunk)) for c0 in range(0, length, chunk)]


def _frame(cc, bc, qb, kb, theta, rnd):
    """The rotated queries and keys of one chunk and head, before and after
    the model-dtype rounding (_rotated, :575-586, then :634)."""
    q = rnd(cc + qb)
    k = rnd(bc + kb)
    cos, sin = np.cos(theta), np.sin(theta)
    q_rot = q * cos + _partner(q) * sin
    k_rot = k * cos + _partner(k) * sin
    return q_rot, k_rot, rnd(q_rot), rnd(k_rot), cos, sin


def _terms(p, gamma, scale, dtype):
    """_chunk_terms (:114-119) of one chunk and head: decay [t,s] (s < t),
    weights, source = scale * tail and tail."""
    n = p.shape[0]
    lower = np.tril(np.ones((n, n), bool), -1)
    decay = np.where(lower, np.exp(np.where(lower, p[:, None] - p[None, :], 0)), 0).astype(dtype)
    weights = decay * scale[None, :] + np.diag(gamma)
    tail = np.exp(p[-1] - p)
    return lower, decay, weights, scale * tail, tail


def fused_forward(c, b, x, adt, dt, trap, angles, q_bias, k_bias, chunk=64, rnd=None,
                  dtype=np.float32):
    """y [B,T,H*P] (rounded by rnd), final [B,H,N,P], and the residuals:
    starts [B,H,NC,N,P] and the chunks' start phases [B,H,NC,N]."""
    rnd = rnd or (lambda v: v)
    batch, length, heads = np.shape(dt)
    c, b = np.asarray(c, dtype), np.asarray(b, dtype)
    dim = c.shape[-1]
    v_all = np.asarray(x, dtype).reshape(batch, length, heads, -1)
    width = v_all.shape[-1]
    qb, kb = _heads(q_bias, heads, dim).astype(dtype), _heads(k_bias, heads, dim).astype(dtype)
    gamma, scale, _ = _glue(dt, trap, dtype)
    adt = np.asarray(adt, dtype)
    rates = _rates(angles, dim, dtype)
    dtv = np.asarray(dt, dtype)
    spans = _chunks(length, chunk)
    y = np.zeros((batch, length, heads, width), dtype)
    starts = np.zeros((batch, heads, len(spans), dim, width), dtype)
    phase0 = np.zeros((batch, heads, len(spans), dim), dtype)
    final = np.zeros((batch, heads, dim, width), dtype)
    for bi in range(batch):
        for h in range(heads):
            state = np.zeros((dim, width), dtype)
            phase = np.zeros(dim, dtype)
            for ci, (t0, t1) in enumerate(spans):
                theta = phase + np.cumsum(rates[bi, t0:t1] * dtv[bi, t0:t1, h, None], axis=0)
                phase0[bi, h, ci] = phase
                phase = theta[-1]
                _, _, q, k, _, _ = _frame(c[bi, t0:t1], b[bi, t0:t1], qb[h], kb[h], theta, rnd)
                v = v_all[bi, t0:t1, h]
                p = np.cumsum(adt[bi, t0:t1, h])
                _, _, weights, source, _ = _terms(p, gamma[bi, t0:t1, h], scale[bi, t0:t1, h],
                                                 dtype)
                scores = q @ k.T
                within = rnd(scores * weights) @ v
                starts[bi, h, ci] = state
                inherited = q @ rnd(state)
                y[bi, t0:t1, h] = rnd(within + np.exp(p)[:, None] * inherited)
                weighted = rnd(v * source[:, None])
                state = np.exp(p[-1]) * state + k.T @ weighted
            final[bi, h] = state
    return y.reshape(batch, length, -1), final, starts, phase0


def fused_backward(c, b, x, adt, dt, trap, angles, q_bias, k_bias, d_y, d_final=None,
                   chunk=64, rnd=None, dtype=np.float32):
    """Gradients of <y, d_y> + <final, d_final> for all nine inputs, as the
    reference's fused backward kernel computes them (d_y rounded to the model
    dtype first, :1008), then through mamba3_fused's glue."""
    rnd = rnd or (lambda v: v)
    batch, length, heads = np.shape(dt)
    c, b = np.asarray(c, dtype), np.asarray(b, dtype)
    dim = c.shape[-1]
    v_all = np.asarray(x, dtype).reshape(batch, length, heads, -1)
    width = v_all.shape[-1]
    dy_all = rnd(np.asarray(d_y, dtype)).reshape(batch, length, heads, width)
    qb, kb = _heads(q_bias, heads, dim).astype(dtype), _heads(k_bias, heads, dim).astype(dtype)
    gamma, scale, sig = _glue(dt, trap, dtype)
    adt = np.asarray(adt, dtype)
    rates = _rates(angles, dim, dtype)
    dtv = np.asarray(dt, dtype)
    spans = _chunks(length, chunk)
    _, _, starts, phase0 = fused_forward(c, b, x, adt, dt, trap, angles, q_bias, k_bias, chunk,
                                         rnd, dtype)
    dc = np.zeros((batch, length, dim), dtype)
    db = np.zeros_like(dc)
    dx = np.zeros((batch, length, heads, width), dtype)
    d_rate = np.zeros((batch, length, dim), dtype)
    dqb = np.zeros((heads, dim), dtype)
    dkb = np.zeros_like(dqb)
    d_adt = np.zeros((batch, length, heads), dtype)
    d_gam = np.zeros_like(d_adt)
    d_scale = np.zeros_like(d_adt)
    d_dt = np.zeros_like(d_adt)
    for bi in range(batch):
        for h in range(heads):
            carry = np.zeros((dim, width), dtype) if d_final is None else \
                np.asarray(d_final, dtype)[bi, h].copy()
            later = np.zeros(dim, dtype)
            for ci in reversed(range(len(spans))):
                t0, t1 = spans[ci]
                theta = phase0[bi, h, ci] + np.cumsum(rates[bi, t0:t1] * dtv[bi, t0:t1, h, None],
                                                      axis=0)
                q_rot, k_rot, q, k, cos, sin = _frame(c[bi, t0:t1], b[bi, t0:t1], qb[h], kb[h],
                                                      theta, rnd)
                v, dy = v_all[bi, t0:t1, h], dy_all[bi, t0:t1, h]
                p = np.cumsum(adt[bi, t0:t1, h])
                lower, decay, weights, source, tail = _terms(p, gamma[bi, t0:t1, h],
                                                             scale[bi, t0:t1, h], dtype)
                end, start, end_decay = carry, starts[bi, h, ci], np.exp(p[-1])
                scores = q @ k.T
                d_mixed = dy @ v.T
                mixed = scores * weights
                dv = rnd(mixed).T @ dy
                d_scores = d_mixed * weights
                dq = rnd(d_scores) @ k
                dk = rnd(d_scores).T @ q
                d_weights = d_mixed * scores
                carried = np.exp(p)
                scaled_dy = rnd(dy * carried[:, None])
                dq = dq + scaled_dy @ rnd(start).T
                inherited = q @ rnd(start)
                dp = carried * np.sum(dy * inherited, axis=1)
                d_start = q.T @ scaled_dy + end_decay * end
                end_low = rnd(end)
                v_end = v @ end_low.T
                dk = dk + source[:, None] * v_end
                dv = dv + source[:, None] * (k @ end_low)
                d_source = np.sum(k * v_end, axis=1)
                flow = d_source * source
                off = np.where(lower, d_weights * weights, 0)
                dp = dp + np.sum(off, axis=1) - flow - np.sum(off, axis=0)
                d_gam[bi, t0:t1, h] = np.diag(d_weights)
                d_scale[bi, t0:t1, h] = d_source * tail + np.sum(d_weights * decay, axis=0)
                d_end = end_decay * np.sum(end * start)
                dp[-1] += np.sum(flow) + d_end
                d_adt[bi, t0:t1, h] = np.cumsum(dp[::-1])[::-1]
                dx[bi, t0:t1, h] = dv
                carry = d_start
                dq_pre = dq * cos - _partner(dq) * sin
                dk_pre = dk * cos - _partner(dk) * sin
                dc[bi, t0:t1] += dq_pre
                db[bi, t0:t1] += dk_pre
                dqb[h] += dq_pre.sum(0)
                dkb[h] += dk_pre.sum(0)
                d_theta = dq * _partner(q_rot) + dk * _partner(k_rot)
                d_inc = later + np.cumsum(d_theta[::-1], axis=0)[::-1]
                later = later + d_theta.sum(0)
                d_rate[bi, t0:t1] += d_inc * dtv[bi, t0:t1, h, None]
                d_dt[bi, t0:t1, h] += np.sum(d_inc * rates[bi, t0:t1], axis=1)
    # mamba3_fused's glue (:1146-1162): scale_t = gamma_t + prev_{t+1},
    # gamma = dt sigma, prev = dt (1 - sigma), the rates duplicate the angles.
    d_gam_total = d_gam + d_scale
    d_prev = np.concatenate([np.zeros_like(d_scale[:, :1]), d_scale[:, :-1]], axis=1)
    d_dt = d_dt + d_gam_total * sig + d_prev * (1 - sig)
    d_trap = (d_gam_total - d_prev) * dtv * sig * (1 - sig)
    a = np.shape(angles)[-1]
    d_angles = d_rate[..., 0:2 * a:2] + d_rate[..., 1:2 * a:2]
    # The row and value gradients come back in their inputs' model dtype
    # (dx from the kernel, :765; dc, db cast at the end, :1089-1090).
    return {
        "c": rnd(dc), "b": rnd(db), "x": rnd(dx).reshape(batch, length, -1), "adt": d_adt,
        "dt": d_dt,
        "trap": d_trap, "angles": d_angles, "q_bias": dqb, "k_bias": dkb,
    }
