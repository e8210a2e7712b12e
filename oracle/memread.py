"""NumPy restatement of the Mamba 4 memory read -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, as the checker of the HIP
library; the product path never routes through it.

Operator (per batch row b and head h; D = key width, P = value width)::

    S_t = lam_t S_(t-1) + beta_t k_t k_t^T        lam_t = exp(log_decay_t)
    C_t = lam_t C_(t-1) + beta_t v_t k_t^T
    A_t = S_t + diag(floor)                         (the floor is never decayed)
    y_t = A_t^-1 q_t,  output_t = C_t y_t,  variance_t = q_t . y_t

Functions:

* ``dense_reference`` -- sequential float64 recurrence with dense solves
  (lm/kernels/mamba4_reference.py:6-32).
* ``forward`` -- the chunked decomposition of the fused path
  (lm/kernels/mamba4_fused.py:372-454): per-chunk prefix of log decays,
  chunk statistics, decayed carry of chunk-end states, per-token Cholesky
  with reciprocal pivots, and chunk-level reads.  Returns the residuals the
  backward needs (start states, solutions, factors).
* ``backward`` -- closed-form VJP of ``forward`` for every input, the
  initial state and cotangents on output, variance and the final state.
  The solve part restates _chunk_solve_backward
  (lm/kernels/mamba4_fused.py:340-366); the rest is the adjoint of the
  chunk glue that the reference leaves to JAX autodiff.
* ``decode_step`` -- one cached write/read (lm/kernels/mamba4.py:341-355).
* ``cholesky_reciprocal`` / ``factored_solve`` -- the factor and the two
  substitutions with reciprocal pivots (lm/kernels/mamba4_fused.py:45-113).
* ``spd_solve`` / ``spd_solve_backward`` -- the batched SPD solve and its
  VJP (lm/kernels/mamba4.py:164-215).
* ``diagnostics`` -- spectral and finiteness probes of a state
  (lm/kernels/mamba4.py:358-376).

``PINNED`` names, for every function, the tests that pin it against the
reference's known answers, invariants, an independent float64 autodiff and
finite differences.
"""

import numpy as np

PINNED = {
    "dense_reference": [
        "tests/test_oracle.py::test_dense_exact_recall_of_orthonormal_keys",
        "tests/test_oracle.py::test_dense_zero_key_reads_the_floor",
        "tests/test_oracle.py::test_dense_single_write_retention",
        "tests/test_oracle.py::test_dense_floor_bounds_every_precision",
        "tests/test_oracle.py::test_dense_matches_weighted_batch_closed_form",
    ],
    "forward": [
        "tests/test_oracle.py::test_chunked_forward_matches_dense_for_every_chunk",
        "tests/test_oracle.py::test_chunked_continuation_matches_full_run",
        "tests/test_oracle.py::test_factors_reproduce_each_precision",
    ],
    "backward": [
        "tests/test_oracle.py::test_backward_matches_float64_autograd",
        "tests/test_oracle.py::test_backward_matches_central_differences",
        "tests/test_oracle.py::test_planted_backward_mistakes_are_caught",
    ],
    "decode_step": [
        "tests/test_oracle.py::test_decode_matches_prefill",
    ],
    "cholesky_reciprocal": [
        "tests/test_oracle.py::test_reciprocal_cholesky_matches_lapack",
    ],
    "factored_solve": [
        "tests/test_oracle.py::test_factored_solve_matches_dense_solve",
    ],
    "spd_solve": [
        "tests/test_oracle.py::test_spd_solve_matches_dense_solve_and_reads_lower_triangle",
    ],
    "spd_solve_backward": [
        "tests/test_oracle.py::test_spd_solve_backward_matches_float64_autograd",
        "tests/test_oracle.py::test_planted_spd_backward_mistakes_are_caught",
    ],
    "diagnostics": [
        "tests/test_oracle.py::test_diagnostics_on_known_spectra",
        "tests/test_oracle.py::test_diagnostics_symmetrise_and_flag_non_finite_states",
    ],
}


def _shape_inputs(keys, values, queries, beta, log_decay, floor, dtype):
    keys, values, queries = (np.asarray(a, dtype) for a in (keys, values, queries))
    batch, time, heads, dim = keys.shape
    if queries.shape != keys.shape or values.shape[:3] != keys.shape[:3]:
        # Same check and message as lm/kernels/mamba4.py:268-269.
        raise ValueError("Selective memory keys, values and queries disagree")
    shape = (batch, time, heads)
    beta = np.broadcast_to(np.asarray(beta, dtype), shape)
    log_decay = np.broadcast_to(np.asarray(log_decay, dtype), shape)
    floor = np.broadcast_to(np.asarray(floor, dtype), (heads, dim))
    return keys, values, queries, beta, log_decay, floor


def dense_reference(
    keys, values, queries, beta, log_decay, floor, initial=None, dtype=np.float64
):
    """Sequential recurrence with one dense solve per token.

    Restates selective_dense_reference (lm/kernels/mamba4_reference.py:6-32),
    taking log decays like the public op (lm/kernels/mamba4.py:343) and an
    optional (evidence, cross) initial state (lm/kernels/mamba4.py:274-278).
    Returns (output [B,T,H,P], variance [B,T,H], evidence [B,H,D,D],
    cross [B,H,P,D]).
    """
    k, v, q, beta, log_decay, floor = _shape_inputs(
        keys, values, queries, beta, log_decay, floor, dtype
    )
    batch, time, heads, dim = k.shape
    value_dim = v.shape[-1]
    if initial is None:
        evidence = np.zeros((batch, heads, dim, dim), dtype)
        cross = np.zeros((batch, heads, value_dim, dim), dtype)
    else:
        evidence = np.array(initial[0], dtype)
        cross = np.array(initial[1], dtype)
    diagonal = floor[:, :, None] * np.eye(dim, dtype=dtype)
    reads = np.zeros((batch, time, heads, value_dim), dtype)
    variances = np.zeros((batch, time, heads), dtype)
    for t in range(time):
        gate = np.exp(log_decay[:, t])[..., None, None]
        b = beta[:, t][..., None, None]
        evidence = gate * evidence + b * k[:, t, :, :, None] * k[:, t, :, None, :]
        cross = gate * cross + b * v[:, t, :, :, None] * k[:, t, :, None, :]
        solved = np.linalg.solve(evidence + diagonal[None], q[:, t, :, :, None])[..., 0]
        reads[:, t] = np.einsum("bhpd,bhd->bhp", cross, solved)
        variances[:, t] = np.sum(q[:, t] * solved, axis=-1)
    return reads, variances, evidence, cross


def cholesky_reciprocal(matrix):
    """Lower Cholesky factor whose diagonal holds the reciprocal pivots.

    Restates the left-looking column loop of _factor_token
    (lm/kernels/mamba4_fused.py:93-113): column j starts from A[:, j] and
    subtracts every earlier column scaled by its row-j entry; the pivot's
    reciprocal square root scales the entries below the diagonal and is
    itself kept on the diagonal, so no later step divides.
    """
    matrix = np.asarray(matrix)
    dim = matrix.shape[-1]
    lower = np.zeros_like(matrix)
    for j in range(dim):
        column = matrix[..., :, j] - np.einsum(
            "...ik,...k->...i", lower[..., :, :j], lower[..., j, :j]
        )
        reciprocal = 1.0 / np.sqrt(column[..., j])
        below = column * reciprocal[..., None]
        below[..., : j + 1] = 0.0
        lower[..., :, j] = below
        lower[..., j, j] = reciprocal
    return lower


def factored_solve(lower, rhs):
    """Solve L L^T y = rhs from a reciprocal-diagonal factor.

    Restates _substitute (lm/kernels/mamba4_fused.py:45-75): a forward
    substitution L z = rhs and a backward substitution L^T y = z, each
    multiplying by the stored reciprocal pivot instead of dividing.
    """
    lower = np.asarray(lower)
    value = np.array(rhs, dtype=lower.dtype)
    dim = value.shape[-1]
    for j in range(dim):
        value[..., j] = (
            value[..., j]
            - np.einsum("...k,...k->...", lower[..., j, :j], value[..., :j])
        ) * lower[..., j, j]
    for j in reversed(range(dim)):
        value[..., j] = (
            value[..., j]
            - np.einsum("...k,...k->...", lower[..., j + 1 :, j], value[..., j + 1 :])
        ) * lower[..., j, j]
    return value


def spd_solve(precision, rhs):
    """Solve precision y = rhs for SPD [..., d, d] precision, [..., d] rhs.

    Restates spd_solve / _factor_and_solve (lm/kernels/mamba4.py:164-201):
    only the lower triangle is read (``cholesky_reciprocal`` touches column
    entries on and below the diagonal only), then the two substitutions.
    Returns (solution, lower factor).
    """
    precision = np.asarray(precision, np.float64)
    lower = cholesky_reciprocal(precision)
    return factored_solve(lower, np.asarray(rhs, np.float64)), lower


def spd_solve_backward(lower, solution, gradient):
    """VJP of ``spd_solve`` (lm/kernels/mamba4.py:204-215).

    z = A^-1 g from the stored factor; d rhs = z and
    d precision = -(z y^T + y z^T) / 2, the symmetric form.
    """
    z = factored_solve(lower, gradient)
    outer = z[..., :, None] * np.asarray(solution)[..., None, :]
    return -0.5 * (outer + np.swapaxes(outer, -1, -2)), z


def _chunked(x, batch, count, chunk, padding):
    # Padding writes nothing and does not decay: zero beta and log decay
    # (lm/kernels/mamba4_fused.py:402-406).
    x = np.pad(x, [(0, 0), (0, padding)] + [(0, 0)] * (x.ndim - 2))
    x = x.reshape(batch, count, chunk, *x.shape[2:])
    return np.swapaxes(x, 2, 3)


def _unchunked(x, batch, time):
    x = np.swapaxes(x, 2, 3)
    return x.reshape(batch, -1, *x.shape[3:])[:, :time]


def forward(
    keys,
    values,
    queries,
    beta,
    log_decay,
    floor,
    chunk=64,
    initial=None,
    dtype=np.float64,
):
    """Chunked forward; returns ((output, variance, evidence, cross), residuals).

    Follows selective_memory_fused (lm/kernels/mamba4_fused.py:372-454):

    * chunking with beta = log_decay = 0 padding (:399-409);
    * inclusive prefix P of the chunk's log decays (:410, prefix.py:17-24);
    * tail weights beta_s exp(P_last - P_s) and the chunk statistics
      K^T diag(tail) K and V^T diag(tail) K (:411-415);
    * the decayed carry of chunk-end states (prefix.py:27-44), start states
      (:417-425);
    * per-token precisions A_t = exp(P_t) S0 + sum_{s<=t} W_ts k_s k_s^T +
      diag(floor), W_ts = beta_s exp(P_t - P_s) (the decomposition stated in
      the module docstring, lm/kernels/mamba4_fused.py:3-8), each factored by
      ``cholesky_reciprocal`` and solved by ``factored_solve`` (:116-152);
    * reads (Y K^T * W) V + exp(P) Y C0^T and variance q.y (:439-447).
    """
    k, v, q, beta, log_decay, floor = _shape_inputs(
        keys, values, queries, beta, log_decay, floor, dtype
    )
    batch, time, heads, dim = k.shape
    value_dim = v.shape[-1]
    padding = (-time) % chunk
    count = (time + padding) // chunk

    def chunked(x):
        return _chunked(x, batch, count, chunk, padding)

    kc, vc, qc = chunked(k), chunked(v), chunked(q)
    bc, gc = chunked(beta), chunked(log_decay)
    prefix = np.cumsum(gc, axis=-1)
    tail = bc * np.exp(prefix[..., -1:] - prefix)
    chunk_evidence = np.einsum("bnhs,bnhsd,bnhse->bnhde", tail, kc, kc)
    chunk_cross = np.einsum("bnhs,bnhsp,bnhsd->bnhpd", tail, vc, kc)
    if initial is None:
        state_s = np.zeros((batch, heads, dim, dim), dtype)
        state_c = np.zeros((batch, heads, value_dim, dim), dtype)
    else:
        state_s = np.array(initial[0], dtype)
        state_c = np.array(initial[1], dtype)
    starts_s = np.empty((batch, count, heads, dim, dim), dtype)
    starts_c = np.empty((batch, count, heads, value_dim, dim), dtype)
    for i in range(count):
        starts_s[:, i] = state_s
        starts_c[:, i] = state_c
        decay = np.exp(prefix[:, i, :, -1])[..., None, None]
        state_s = decay * state_s + chunk_evidence[:, i]
        state_c = decay * state_c + chunk_cross[:, i]

    position = np.arange(chunk)
    causal = position[:, None] >= position[None, :]
    difference = np.where(causal, prefix[..., :, None] - prefix[..., None, :], 0.0)
    decay_ts = np.where(causal, np.exp(difference), 0.0)
    weights = decay_ts * bc[..., None, :]
    carried = np.exp(prefix)
    outer = (kc[..., :, None] * kc[..., None, :]).reshape(*kc.shape[:-1], dim * dim)
    local = np.matmul(weights, outer).reshape(*kc.shape[:-1], dim, dim)
    diagonal = floor[:, :, None] * np.eye(dim, dtype=dtype)
    precision = (
        local
        + carried[..., None, None] * starts_s[:, :, :, None]
        + diagonal[None, None, :, None]
    )
    lower = cholesky_reciprocal(precision)
    solved = factored_solve(lower, qc)
    scores = np.einsum("bnhtd,bnhsd->bnhts", solved, kc)
    within = np.einsum("bnhts,bnhsp->bnhtp", scores * weights, vc)
    inherited = np.einsum("bnhtd,bnhpd->bnhtp", solved, starts_c)
    output = within + carried[..., None] * inherited
    variance = np.sum(qc * solved, axis=-1)
    residuals = dict(
        shape=(batch, time, heads, dim, value_dim, chunk, count, padding),
        kc=kc,
        vc=vc,
        qc=qc,
        bc=bc,
        prefix=prefix,
        tail=tail,
        decay_ts=decay_ts,
        weights=weights,
        starts_s=starts_s,
        starts_c=starts_c,
        solved=solved,
        lower=lower,
        dtype=dtype,
    )
    result = (
        _unchunked(output, batch, time),
        _unchunked(variance, batch, time),
        state_s,
        state_c,
    )
    return result, residuals


def backward(residuals, d_output, d_variance, d_evidence=None, d_cross=None):
    """Closed-form VJP of ``forward``.

    Returns dict(keys, values, queries, beta, log_decay, floor,
    initial_evidence, initial_cross).  Derivation (per chunk, W_ts =
    beta_s exp(P_t - P_s) for s <= t, S0 / C0 the chunk start states):

    * ybar_t = C_t^T dout_t + dvar_t q_t with C_t = exp(P_t) C0 +
      sum_s W_ts v_s k_s^T; z_t = A_t^-1 ybar_t by the stored factor
      (_factored_kernel, lm/kernels/mamba4_fused.py:155-174);
    * dq_t = z_t + dvar_t y_t; the precision cotangent is the symmetric
      -(z y^T + y z^T)/2 of spd_solve's VJP (lm/kernels/mamba4.py:208-215),
      so d floor = -sum z*y;
    * the contractions gy = Y K^T, gz = Z K^T, dW = gy (gv - gz) with
      gv = dOut V^T give d keys, d beta and the prefix cotangent exactly as
      in _chunk_solve_backward (lm/kernels/mamba4_fused.py:343-366), plus
      the value path of the reads (:443-446);
    * start-state cotangents accumulate in a reverse carry over chunks (the
      transpose of prefix.py:27-44), and the chunk-end terms add
      tail_s-weighted contributions to keys, values, beta and the prefix;
    * d log_decay is the reverse cumulative sum of the prefix cotangent
      (the transpose of prefix.py:17-24).
    """
    batch, time, heads, dim, value_dim, chunk, count, padding = residuals["shape"]
    dtype = residuals["dtype"]
    kc, vc, qc = residuals["kc"], residuals["vc"], residuals["qc"]
    prefix, tail = residuals["prefix"], residuals["tail"]
    decay_ts, weights = residuals["decay_ts"], residuals["weights"]
    starts_s, starts_c = residuals["starts_s"], residuals["starts_c"]
    y, lower = residuals["solved"], residuals["lower"]

    def chunked(x):
        return _chunked(np.asarray(x, dtype), batch, count, chunk, padding)

    dout = chunked(d_output)
    dvar = chunked(np.broadcast_to(np.asarray(d_variance, dtype), (batch, time, heads)))
    carried = np.exp(prefix)

    gv = np.einsum("bnhtp,bnhsp->bnhts", dout, vc)
    ybar = (
        np.einsum("bnhts,bnhsd->bnhtd", weights * gv, kc)
        + carried[..., None] * np.einsum("bnhpd,bnhtp->bnhtd", starts_c, dout)
        + dvar[..., None] * qc
    )
    z = factored_solve(lower, ybar)
    d_queries = z + dvar[..., None] * y

    # Start-state cotangents of each chunk's own reads.
    local_s = -0.5 * (
        np.einsum("bnht,bnhtd,bnhte->bnhde", carried, z, y)
        + np.einsum("bnht,bnhtd,bnhte->bnhde", carried, y, z)
    )
    local_c = np.einsum("bnht,bnhtp,bnhtd->bnhpd", carried, dout, y)

    # Reverse carry: the cotangent of chunk i's end state is the start-state
    # cotangent of chunk i+1 (the final-state cotangent for the last chunk).
    grad_s = (
        np.zeros((batch, heads, dim, dim), dtype)
        if d_evidence is None
        else np.array(d_evidence, dtype)
    )
    grad_c = (
        np.zeros((batch, heads, value_dim, dim), dtype)
        if d_cross is None
        else np.array(d_cross, dtype)
    )
    ends_s = np.empty_like(starts_s)
    ends_c = np.empty_like(starts_c)
    for i in reversed(range(count)):
        ends_s[:, i] = grad_s
        ends_c[:, i] = grad_c
        decay = np.exp(prefix[:, i, :, -1])[..., None, None]
        grad_s = local_s[:, i] + decay * grad_s
        grad_c = local_c[:, i] + decay * grad_c

    gy = np.einsum("bnhtd,bnhsd->bnhts", y, kc)
    gz = np.einsum("bnhtd,bnhsd->bnhts", z, kc)
    mix = gv - gz
    through_y = weights * mix
    through_z = weights * gy
    symmetric_end = ends_s + np.swapaxes(ends_s, -1, -2)
    gk_end = np.einsum("bnhde,bnhse->bnhsd", symmetric_end, kc)
    hv_end = np.einsum("bnhpd,bnhsp->bnhsd", ends_c, vc)
    hk_end = np.einsum("bnhpd,bnhsd->bnhsp", ends_c, kc)
    d_keys = (
        np.einsum("bnhts,bnhtd->bnhsd", through_y, y)
        - np.einsum("bnhts,bnhtd->bnhsd", through_z, z)
        + tail[..., None] * (gk_end + hv_end)
    )
    d_values = (
        np.einsum("bnhts,bnhtp->bnhsp", through_z, dout) + tail[..., None] * hk_end
    )
    quad_end = 0.5 * np.sum(kc * gk_end, axis=-1) + np.sum(vc * hk_end, axis=-1)
    end_decay = np.exp(prefix[..., -1:] - prefix)
    d_beta = np.sum(decay_ts * gy * mix, axis=-2) + end_decay * quad_end
    d_weights = weights * gy * mix
    end_weights = tail * quad_end
    ysz = 0.5 * (
        np.einsum("bnhtd,bnhde,bnhte->bnht", y, starts_s, z)
        + np.einsum("bnhtd,bnhde,bnhte->bnht", z, starts_s, y)
    )
    docy = np.einsum("bnhtp,bnhpd,bnhtd->bnht", dout, starts_c, y)
    d_prefix = (
        np.sum(d_weights, axis=-1)
        - np.sum(d_weights, axis=-2)
        + carried * (docy - ysz)
        - end_weights
    )
    d_prefix[..., -1] += (
        np.exp(prefix[..., -1])
        * (
            np.sum(ends_s * starts_s, axis=(-1, -2))
            + np.sum(ends_c * starts_c, axis=(-1, -2))
        )
        + np.sum(end_weights, axis=-1)
    )
    d_log_decay = np.flip(np.cumsum(np.flip(d_prefix, -1), axis=-1), -1)
    d_floor = -np.sum(z * y, axis=(0, 1, 3))

    def unchunked(x):
        return _unchunked(x, batch, time)

    return dict(
        keys=unchunked(d_keys),
        values=unchunked(d_values),
        queries=unchunked(d_queries),
        beta=unchunked(d_beta),
        log_decay=unchunked(d_log_decay),
        floor=d_floor,
        initial_evidence=grad_s,
        initial_cross=grad_c,
    )


def decode_step(evidence, cross, key, value, query, beta, log_decay, floor, dtype=np.float64):
    """One exact write/read from a cached state.

    Restates selective_decode (lm/kernels/mamba4.py:341-355): decayed rank-one
    writes of S and C, a solve with S + diag(floor), and the two reads.
    Shapes: evidence [...,D,D], cross [...,P,D], key/query [...,D], value
    [...,P], beta/log_decay [...], floor broadcastable to [...,D].
    Returns (output, variance, new_evidence, new_cross).
    """
    evidence, cross = np.asarray(evidence, dtype), np.asarray(cross, dtype)
    key, value, query = (np.asarray(a, dtype) for a in (key, value, query))
    lam = np.exp(np.asarray(log_decay, dtype))[..., None, None]
    b = np.asarray(beta, dtype)[..., None, None]
    evidence = lam * evidence + b * key[..., :, None] * key[..., None, :]
    cross = lam * cross + b * value[..., :, None] * key[..., None, :]
    floor = np.broadcast_to(np.asarray(floor, dtype), key.shape)
    precision = evidence + floor[..., :, None] * np.eye(key.shape[-1], dtype=dtype)
    solved = np.linalg.solve(precision, query[..., None])[..., 0]
    output = np.einsum("...pd,...d->...p", cross, solved)
    variance = np.sum(query * solved, axis=-1)
    return output, variance, evidence, cross


DIAGNOSTIC_KEYS = (
    "precision_min_eigenvalue",
    "precision_max_eigenvalue",
    "precision_max_condition",
    "state_all_finite",
    "cross_max_abs",
    "floor_min",
    "floor_max",
)


def diagnostics(evidence, cross, floor):
    """Spectral and finiteness probes of a state (float64).

    Restates selective_diagnostics (lm/kernels/mamba4.py:358-376): the
    eigenvalues of the symmetrised precision (P + P^T)/2, P = evidence +
    diag(floor), their extremes over every state, the largest ratio of a
    state's largest to its smallest (floored at 1e-30), whether evidence and
    cross are finite, the largest cross magnitude and the floor's range.
    Shapes: evidence [...,D,D], cross [...,P,D], floor broadcastable to
    [...,D].  A state with a non-finite precision entry has NaN eigenvalues
    (the device kernel's convention; LAPACK gives NaN or fails there).
    """
    evidence = np.asarray(evidence, np.float64)
    cross = np.asarray(cross, np.float64)
    floor = np.asarray(floor, np.float64)
    dim = evidence.shape[-1]
    precision = evidence + np.broadcast_to(floor, evidence.shape[:-1])[..., :, None] * np.eye(dim)
    sym = (precision + np.swapaxes(precision, -1, -2)) * 0.5
    flat = sym.reshape(-1, dim, dim)
    eig = np.full((flat.shape[0], dim), np.nan)
    ok = np.isfinite(flat).all(axis=(-1, -2))
    if ok.any():
        eig[ok] = np.linalg.eigvalsh(flat[ok])
    minimum, maximum = eig[:, 0], eig[:, -1]
    return {
        "precision_min_eigenvalue": np.min(minimum),
        "precision_max_eigenvalue": np.max(maximum),
        "precision_max_condition": np.max(maximum / np.maximum(minimum, 1e-30)),
        "state_all_finite": bool(np.all(np.isfinite(evidence)) and np.all(np.isfinite(cross))),
        "cross_max_abs": np.max(np.abs(cross)),
        "floor_min": np.min(floor),
        "floor_max": np.max(floor),
    }
