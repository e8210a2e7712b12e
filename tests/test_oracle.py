"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

The reference holds no golden vectors for the memory read; every oracle
function is pinned here by the reference's own known answers and
invariants (lm/tests/test_mamba4.py, formal/Mamba4/*.lean), by an
independent float64 torch autograd of the dense recurrence, by central
finite differences, and by planted mistakes that these checks must catch.
"""

import importlib.util
import os
import sys

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import memread as oracle


def arrays(time=13, heads=3, dim=4, value_dim=5, seed=0, batch=2):
    """Same distributions as the reference's test fixture
    (lm/tests/test_mamba4.py:19-29)."""
    rng = np.random.default_rng(seed)
    k = rng.normal(size=(batch, time, heads, dim))
    q = rng.normal(size=k.shape)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    v = rng.normal(size=(batch, time, heads, value_dim))
    beta = rng.uniform(0.05, 1.0, size=k.shape[:-1])
    decay = rng.uniform(0.3, 0.999, size=k.shape[:-1])
    floor = rng.uniform(0.25, 1.5, size=(heads, dim))
    return k, v, q, beta, np.log(decay), floor


def test_dense_exact_recall_of_orthonormal_keys():
    # lm/tests/test_mamba4.py:137-152: read(k_i) = v_i / (1 + floor / beta).
    dim, value_dim = 4, 3
    keys = np.eye(dim)[None, :, None, :]
    values = np.random.default_rng(1).normal(size=(1, dim, 1, value_dim))
    beta = np.full((1, dim, 1), 2.0)
    floor = np.full((1, dim), 1e-3)
    out, var, s, c = oracle.dense_reference(
        keys, values, keys, beta, np.zeros_like(beta), floor
    )
    # Each token reads its own just-written value at the same ratio.
    np.testing.assert_allclose(out, values / (1 + 5e-4), rtol=1e-12)
    np.testing.assert_allclose(var, 1 / (2.0 + 1e-3), rtol=1e-12)
    precision = s[0, 0] + 1e-3 * np.eye(dim)
    for i in range(dim):
        read = c[0, 0] @ np.linalg.solve(precision, keys[0, i, 0])
        np.testing.assert_allclose(read, values[0, i, 0] / (1 + 5e-4), rtol=1e-12)


def test_dense_zero_key_reads_the_floor():
    # lm/tests/test_mamba4.py:364-375: a shifted first token has a zero key,
    # so A_0 = diag(floor), variance = sum q^2/floor and nothing is read.
    k, v, q, beta, log_decay, floor = arrays(time=5)
    k[:, 0] = 0.0
    out, var, _, _ = oracle.dense_reference(k, v, q, beta, log_decay, floor)
    np.testing.assert_allclose(var[:, 0], np.sum(q[:, 0] ** 2 / floor, -1), rtol=1e-12)
    np.testing.assert_allclose(out[:, 0], 0.0, atol=1e-15)


def test_dense_single_write_retention():
    # formal/Mamba4/Retention.lean:28-55: one write of weight w under a unit
    # key is read back at w / (w + floor); here w = beta * prod(later decays).
    dim, value_dim, floor = 6, 2, 0.3
    rng = np.random.default_rng(2)
    key = rng.normal(size=dim)
    key /= np.linalg.norm(key)
    time = 5
    keys = np.zeros((1, time, 1, dim))
    keys[0, 0, 0] = key
    queries = np.broadcast_to(key, (1, time, 1, dim))
    values = np.zeros((1, time, 1, value_dim))
    values[0, 0, 0] = rng.normal(size=value_dim)
    beta = np.zeros((1, time, 1))
    beta[0, 0, 0] = 0.7
    log_decay = np.log(rng.uniform(0.5, 0.99, size=(1, time, 1)))
    out, var, _, _ = oracle.dense_reference(
        keys, values, queries, beta, log_decay, np.full((1, dim), floor)
    )
    weight = 0.7 * np.exp(np.cumsum(log_decay[0, :, 0]) - log_decay[0, 0, 0])
    np.testing.assert_allclose(var[0, :, 0], 1 / (weight + floor), rtol=1e-12)
    np.testing.assert_allclose(
        out[0, :, 0], values[0, 0, 0][None] * (weight / (weight + floor))[:, None],
        rtol=1e-12,
    )


def test_dense_floor_bounds_every_precision():
    # lm/tests/test_mamba4.py:46-58 with extreme gates 1e-4 and 1.
    k, v, q, beta, log_decay, floor = arrays(time=40)
    decay = np.exp(log_decay)
    decay[:, ::7] = 1e-4
    decay[:, 3::7] = 1.0
    _, var, s, _ = oracle.dense_reference(k, v, q, beta, np.log(decay), floor)
    precision = s + floor[None, :, :, None] * np.eye(4)
    assert np.all(np.linalg.eigvalsh(precision)[..., 0] >= floor.min(-1)[None] - 1e-12)
    assert np.all(var <= 1 / floor.min() + 1e-12)
    assert np.all(var >= 0)


def test_dense_matches_weighted_batch_closed_form():
    # The recurrence equals one weighted batch write with weights
    # beta_s * prod_{r>s} lam_r (effective_weights, analysis/memory.py:23-32,
    # from_batch :45-54), read by a scipy Cholesky solve (:66-72).
    k, v, q, beta, log_decay, floor = arrays(time=11, dim=5, value_dim=3)
    out, var, s, c = oracle.dense_reference(k, v, q, beta, log_decay, floor)
    for b in range(2):
        for h in range(3):
            later = np.concatenate((np.cumsum(log_decay[b, ::-1, h])[::-1][1:], [0.0]))
            w = beta[b, :, h] * np.exp(later)
            s_batch = k[b, :, h].T @ (w[:, None] * k[b, :, h])
            c_batch = v[b, :, h].T @ (w[:, None] * k[b, :, h])
            np.testing.assert_allclose(s[b, h], s_batch, rtol=1e-12, atol=1e-14)
            np.testing.assert_allclose(c[b, h], c_batch, rtol=1e-12, atol=1e-14)
            factor = scipy.linalg.cho_factor(s_batch + np.diag(floor[h]), lower=True)
            x = scipy.linalg.cho_solve(factor, q[b, -1, h])
            np.testing.assert_allclose(out[b, -1, h], c_batch @ x, rtol=1e-10)
            np.testing.assert_allclose(var[b, -1, h], q[b, -1, h] @ x, rtol=1e-10)


@pytest.mark.parametrize("chunk", [1, 4, 5, 13, 16, 64])
def test_chunked_forward_matches_dense_for_every_chunk(chunk):
    # lm/tests/test_mamba4.py:32-43 (chunk invariance, padding included).
    k, v, q, beta, log_decay, floor = arrays()
    expected = oracle.dense_reference(k, v, q, beta, log_decay, floor)
    actual, _ = oracle.forward(k, v, q, beta, log_decay, floor, chunk=chunk)
    for x, y in zip(actual, expected):
        np.testing.assert_allclose(x, y, rtol=1e-10, atol=1e-12)


def test_chunked_forward_matches_dense_at_key_width_64():
    k, v, q, beta, log_decay, floor = arrays(time=70, heads=2, dim=64, value_dim=64)
    floor = np.full_like(floor, 1e-2)
    expected = oracle.dense_reference(k, v, q, beta, log_decay, floor)
    actual, _ = oracle.forward(k, v, q, beta, log_decay, floor, chunk=32)
    for x, y in zip(actual, expected):
        np.testing.assert_allclose(x, y, rtol=1e-8, atol=1e-10)


def test_chunked_continuation_matches_full_run():
    # lm/tests/test_mamba4.py:107-124.
    k, v, q, beta, log_decay, floor = arrays()
    full, _ = oracle.forward(k, v, q, beta, log_decay, floor, chunk=4)
    first, _ = oracle.forward(
        k[:, :6], v[:, :6], q[:, :6], beta[:, :6], log_decay[:, :6], floor, chunk=4
    )
    second, _ = oracle.forward(
        k[:, 6:], v[:, 6:], q[:, 6:], beta[:, 6:], log_decay[:, 6:], floor,
        chunk=4, initial=(first[2], first[3]),
    )
    np.testing.assert_allclose(second[0], full[0][:, 6:], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(second[1], full[1][:, 6:], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(second[2], full[2], rtol=1e-10, atol=1e-12)


def test_factors_reproduce_each_precision():
    k, v, q, beta, log_decay, floor = arrays(time=9, dim=8)
    _, res = oracle.forward(k, v, q, beta, log_decay, floor, chunk=4)
    lower = res["lower"].copy()
    diag = np.einsum("...ii->...i", lower)
    true_lower = np.tril(lower, -1) + np.einsum("...i,ij->...ij", 1 / diag, np.eye(8))
    rebuilt = true_lower @ np.swapaxes(true_lower, -1, -2)
    # Rebuild the precisions independently from the dense recurrence.
    time = 9
    for t in range(time):
        _, _, s_t, _ = oracle.dense_reference(
            k[:, : t + 1], v[:, : t + 1], q[:, : t + 1], beta[:, : t + 1],
            log_decay[:, : t + 1], floor,
        )
        a_t = s_t + floor[None, :, :, None] * np.eye(8)
        np.testing.assert_allclose(rebuilt[:, t // 4, :, t % 4], a_t, rtol=1e-10, atol=1e-12)


def test_reciprocal_cholesky_matches_lapack():
    rng = np.random.default_rng(3)
    a = rng.normal(size=(5, 64, 64))
    a = a @ np.swapaxes(a, -1, -2) / 64 + 1e-2 * np.eye(64)
    lower = oracle.cholesky_reciprocal(a)
    reference = np.linalg.cholesky(a)
    np.testing.assert_allclose(np.tril(lower, -1), np.tril(reference, -1), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(
        np.einsum("...ii->...i", lower), 1 / np.einsum("...ii->...i", reference), rtol=1e-10
    )


def test_factored_solve_matches_dense_solve():
    rng = np.random.default_rng(4)
    a = rng.normal(size=(7, 16, 16))
    a = a @ np.swapaxes(a, -1, -2) + 0.5 * np.eye(16)
    rhs = rng.normal(size=(7, 16))
    got = oracle.factored_solve(oracle.cholesky_reciprocal(a), rhs)
    np.testing.assert_allclose(got, np.linalg.solve(a, rhs[..., None])[..., 0], rtol=1e-9)


def test_decode_matches_prefill():
    # lm/tests/test_mamba4.py:125-134.
    k, v, q, beta, log_decay, floor = arrays()
    out, var, s_end, c_end = oracle.dense_reference(k, v, q, beta, log_decay, floor)
    s = np.zeros((2, 3, 4, 4))
    c = np.zeros((2, 3, 5, 4))
    for t in range(k.shape[1]):
        o, sv, s, c = oracle.decode_step(
            s, c, k[:, t], v[:, t], q[:, t], beta[:, t], log_decay[:, t], floor
        )
        np.testing.assert_allclose(o, out[:, t], rtol=1e-12, atol=1e-14)
        np.testing.assert_allclose(sv, var[:, t], rtol=1e-12)
    np.testing.assert_allclose(s, s_end, rtol=1e-12)
    np.testing.assert_allclose(c, c_end, rtol=1e-12)


# ---------------------------------------------------------------------------
# Backward: independent float64 autograd, finite differences, planted errors.


def torch_dense(k, v, q, beta, log_decay, floor, s0, c0):
    """float64 torch statement of the dense recurrence, differentiated by
    autograd (an independent mechanism from the closed-form backward)."""
    evidence, cross = s0, c0
    reads, variances = [], []
    dim = k.shape[-1]
    eye = torch.eye(dim, dtype=torch.float64)
    for t in range(k.shape[1]):
        gate = torch.exp(log_decay[:, t])[..., None, None]
        b = beta[:, t][..., None, None]
        evidence = gate * evidence + b * k[:, t, :, :, None] * k[:, t, :, None, :]
        cross = gate * cross + b * v[:, t, :, :, None] * k[:, t, :, None, :]
        precision = evidence + floor[None, :, :, None] * eye
        solved = torch.linalg.solve(precision, q[:, t, :, :, None])[..., 0]
        reads.append(torch.einsum("bhpd,bhd->bhp", cross, solved))
        variances.append(torch.sum(q[:, t] * solved, dim=-1))
    return torch.stack(reads, 1), torch.stack(variances, 1), evidence, cross


def backward_problem(seed=5, time=11, dim=6, value_dim=5, heads=2):
    k, v, q, beta, log_decay, floor = arrays(
        time=time, heads=heads, dim=dim, value_dim=value_dim, seed=seed
    )
    rng = np.random.default_rng(seed + 100)
    root = rng.normal(size=(2, heads, dim, dim)) / dim
    s0 = root @ np.swapaxes(root, -1, -2)
    c0 = rng.normal(size=(2, heads, value_dim, dim)) * 0.3
    d_out = rng.normal(size=v.shape)
    d_var = rng.normal(size=beta.shape)
    d_s = rng.normal(size=s0.shape)  # deliberately not symmetric
    d_c = rng.normal(size=c0.shape)
    return (k, v, q, beta, log_decay, floor, s0, c0), (d_out, d_var, d_s, d_c)


def autograd_gradients(inputs, cotangents):
    tensors = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in inputs]
    out, var, s, c = torch_dense(*tensors)
    d_out, d_var, d_s, d_c = (torch.tensor(x, dtype=torch.float64) for x in cotangents)
    loss = (out * d_out).sum() + (var * d_var).sum() + (s * d_s).sum() + (c * d_c).sum()
    loss.backward()
    return [t.grad.numpy() for t in tensors]


def sym(x):
    return 0.5 * (x + np.swapaxes(x, -1, -2))


def compare_to_autograd(module, chunk):
    inputs, cotangents = backward_problem()
    k, v, q, beta, log_decay, floor, s0, c0 = inputs
    _, res = module.forward(k, v, q, beta, log_decay, floor, chunk=chunk, initial=(s0, c0))
    grads = module.backward(res, *cotangents)
    expected = autograd_gradients(inputs, cotangents)
    names = ["keys", "values", "queries", "beta", "log_decay", "floor"]
    for name, want in zip(names, expected[:6]):
        np.testing.assert_allclose(grads[name], want, rtol=1e-8, atol=1e-10, err_msg=name)
    # Evidence enters only through symmetric contractions; compare the
    # symmetric parts (autograd of a dense solve returns -z y^T).
    np.testing.assert_allclose(
        sym(grads["initial_evidence"]), sym(expected[6]), rtol=1e-8, atol=1e-10
    )
    np.testing.assert_allclose(grads["initial_cross"], expected[7], rtol=1e-8, atol=1e-10)


@pytest.mark.parametrize("chunk", [1, 4, 5, 16])
def test_backward_matches_float64_autograd(chunk):
    compare_to_autograd(oracle, chunk)


def test_backward_matches_central_differences():
    inputs, cotangents = backward_problem(seed=7, time=9, dim=5, value_dim=3)
    k, v, q, beta, log_decay, floor, s0, c0 = inputs
    _, res = oracle.forward(k, v, q, beta, log_decay, floor, chunk=4, initial=(s0, c0))
    grads = oracle.backward(res, *cotangents)
    d_out, d_var, d_s, d_c = cotangents

    def loss(args):
        out, var, s, c = oracle.dense_reference(*args[:6], initial=(args[6], args[7]))
        return (out * d_out).sum() + (var * d_var).sum() + (s * d_s).sum() + (c * d_c).sum()

    rng = np.random.default_rng(11)
    names = ["keys", "values", "queries", "beta", "log_decay", "floor"]
    for index, name in enumerate(names):
        direction = rng.normal(size=np.shape(inputs[index]))
        eps = 1e-6
        plus = list(inputs)
        minus = list(inputs)
        plus[index] = inputs[index] + eps * direction
        minus[index] = inputs[index] - eps * direction
        numeric = (loss(plus) - loss(minus)) / (2 * eps)
        analytic = np.sum(grads[name] * direction)
        assert abs(numeric - analytic) <= 1e-6 * max(1.0, abs(numeric)), name


PLANTS = [
    ("- end_weights\n", "+ end_weights\n"),
    ("+ tail[..., None] * (gk_end + hv_end)", "+ tail[..., None] * (gk_end - hv_end)"),
    ("symmetric_end = ends_s + np.swapaxes(ends_s, -1, -2)", "symmetric_end = 2 * ends_s"),
    ("d_queries = z + dvar[..., None] * y", "d_queries = z"),
    ("mix = gv - gz", "mix = gv + gz"),
    ("+ carried * (docy - ysz)", "+ carried * (docy + ysz)"),
    ("grad_s = local_s[:, i] + decay * grad_s", "grad_s = local_s[:, i] + grad_s"),
    ("end_decay = np.exp(prefix[..., -1:] - prefix)", "end_decay = np.exp(prefix - prefix[..., -1:])"),
]


@pytest.mark.parametrize("plant", PLANTS, ids=[p[1][:30] for p in PLANTS])
def test_planted_backward_mistakes_are_caught(plant, tmp_path):
    """A copy of the oracle with one plausible mistake must fail the check."""
    source = open(oracle.__file__).read()
    assert plant[0] in source, plant[0]
    path = tmp_path / "planted.py"
    path.write_text(source.replace(plant[0], plant[1]))
    spec = importlib.util.spec_from_file_location("planted_oracle", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    with pytest.raises(AssertionError):
        compare_to_autograd(module, chunk=4)


def spd_problem(seed=4, count=7, dim=6):
    """The reference's spd_solve test problem (lm/tests/test_mamba4.py:60-64)."""
    rng = np.random.default_rng(seed)
    a = rng.normal(size=(count, dim, dim))
    a = a @ np.swapaxes(a, -1, -2) + 0.5 * np.eye(dim)
    rhs = rng.normal(size=(count, dim))
    return a, rhs


def test_spd_solve_matches_dense_solve_and_reads_lower_triangle():
    a, rhs = spd_problem()
    got, _ = oracle.spd_solve(a, rhs)
    np.testing.assert_allclose(got, np.linalg.solve(a, rhs[..., None])[..., 0], rtol=1e-10)
    garbage = a + np.triu(np.random.default_rng(1).normal(size=a.shape) * 50, 1)
    again, _ = oracle.spd_solve(garbage, rhs)
    np.testing.assert_array_equal(again, got)


def compare_spd_to_autograd(module):
    a, rhs = spd_problem()
    # The reference's check: d/d(matrix) of sum(sin(solve(sym(matrix), rhs)))
    # against a dense float64 solve (lm/tests/test_mamba4.py:60-81).
    matrix = torch.tensor(a, dtype=torch.float64, requires_grad=True)
    vector = torch.tensor(rhs, dtype=torch.float64, requires_grad=True)
    symmetric = (matrix + matrix.transpose(-1, -2)) / 2
    torch.sin(torch.linalg.solve(symmetric, vector[..., None])[..., 0]).sum().backward()
    solution, lower = module.spd_solve(a, rhs)
    d_a, d_rhs = module.spd_solve_backward(lower, solution, np.cos(solution))
    np.testing.assert_allclose(sym(d_a), matrix.grad.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(d_rhs, vector.grad.numpy(), rtol=1e-9, atol=1e-12)
    # The VJP itself is the symmetric form of -z y^T (autograd of a plain solve).
    plain = torch.tensor(a, dtype=torch.float64, requires_grad=True)
    torch.sin(torch.linalg.solve(plain, vector.detach()[..., None])[..., 0]).sum().backward()
    np.testing.assert_allclose(d_a, sym(plain.grad.numpy()), rtol=1e-9, atol=1e-12)


def test_spd_solve_backward_matches_float64_autograd():
    compare_spd_to_autograd(oracle)


SPD_PLANTS = [
    ("-0.5 * (outer + np.swapaxes", "-1.0 * (outer + np.swapaxes"),
    ("z[..., :, None] * np.asarray(solution)[..., None, :]", "z[..., :, None] * z[..., None, :]"),
    ("z = factored_solve(lower, gradient)", "z = np.asarray(gradient, np.float64)"),
    ("(outer + np.swapaxes(outer, -1, -2))", "(outer - np.swapaxes(outer, -1, -2))"),
]


def _planted_module(plant, tmp_path):
    source = open(oracle.__file__).read()
    assert plant[0] in source, plant[0]
    path = tmp_path / "planted.py"
    path.write_text(source.replace(plant[0], plant[1]))
    spec = importlib.util.spec_from_file_location("planted_oracle", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


@pytest.mark.parametrize("plant", SPD_PLANTS, ids=[p[1][:30] for p in SPD_PLANTS])
def test_planted_spd_backward_mistakes_are_caught(plant, tmp_path):
    with pytest.raises(AssertionError):
        compare_spd_to_autograd(_planted_module(plant, tmp_path))


def test_every_pinning_test_named_by_the_oracle_exists():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for function, tests in oracle.PINNED.items():
        assert hasattr(oracle, function), function
        for name in tests:
            path, test = name.split("::")
            text = open(os.path.join(root, path)).read()
            assert f"def {test}(" in text, name


def _known_spectrum_state(rng, batch, heads, dim, value_dim):
    """States whose precision evidence + diag(floor) has known eigenvalues:
    Q diag(mu) Q^T minus the floor's diagonal, Q a random orthogonal matrix."""
    mu = np.exp(rng.uniform(np.log(1e-3), np.log(50.0), size=(batch, heads, dim)))
    q, _ = np.linalg.qr(rng.normal(size=(batch, heads, dim, dim)))
    precision = np.einsum("bhij,bhj,bhkj->bhik", q, mu, q)
    floor = rng.uniform(0.01, 0.5, size=(heads, dim))
    evidence = precision - floor[None, :, :, None] * np.eye(dim)
    cross = rng.normal(size=(batch, heads, value_dim, dim))
    return mu, evidence, cross, floor


def test_diagnostics_on_known_spectra():
    # lm/kernels/mamba4.py:358-376 on states with planted eigenvalues, cross
    # entries and floors: every statistic has a closed-form answer.
    rng = np.random.default_rng(40)
    for dim in (1, 5, 64):
        mu, evidence, cross, floor = _known_spectrum_state(rng, 2, 3, dim, 4)
        cross[1, 2, 3, 0] = -9.5  # the largest magnitude, planted
        got = oracle.diagnostics(evidence, cross, floor)
        assert set(got) == set(oracle.DIAGNOSTIC_KEYS)
        np.testing.assert_allclose(got["precision_min_eigenvalue"], mu.min(), rtol=1e-9)
        np.testing.assert_allclose(got["precision_max_eigenvalue"], mu.max(), rtol=1e-9)
        cond = (mu.max(axis=-1) / mu.min(axis=-1)).max()
        np.testing.assert_allclose(got["precision_max_condition"], cond, rtol=1e-8)
        assert got["state_all_finite"] is True
        assert got["cross_max_abs"] == max(9.5, np.abs(cross).max())
        assert got["floor_min"] == floor.min() and got["floor_max"] == floor.max()
    # A floor shared by every head ([D]) broadcasts like the reference's.
    mu, evidence, cross, floor = _known_spectrum_state(rng, 1, 2, 3, 2)
    shared = np.array([0.1, 0.2, 0.3])
    evidence = evidence + (floor - shared)[None, :, :, None] * np.eye(3)
    got = oracle.diagnostics(evidence, cross, shared)
    np.testing.assert_allclose(got["precision_min_eigenvalue"], mu.min(), rtol=1e-9)
    assert got["floor_min"] == 0.1 and got["floor_max"] == 0.3


def test_diagnostics_symmetrise_and_flag_non_finite_states():
    rng = np.random.default_rng(41)
    mu, evidence, cross, floor = _known_spectrum_state(rng, 2, 2, 6, 3)
    skew = rng.normal(size=evidence.shape)
    skew = skew - np.swapaxes(skew, -1, -2)
    # An antisymmetric part leaves the symmetrised precision unchanged.
    got = oracle.diagnostics(evidence + skew, cross, floor)
    np.testing.assert_allclose(got["precision_min_eigenvalue"], mu.min(), rtol=1e-9)
    np.testing.assert_allclose(got["precision_max_eigenvalue"], mu.max(), rtol=1e-9)
    # A NaN cross entry: not finite, and the maximum magnitude is NaN.
    bad = cross.copy()
    bad[0, 1, 2, 3] = np.nan
    got = oracle.diagnostics(evidence, bad, floor)
    assert got["state_all_finite"] is False and np.isnan(got["cross_max_abs"])
    assert np.isfinite(got["precision_min_eigenvalue"])
    # An infinite evidence entry: not finite, NaN eigenvalue extremes.
    bad = evidence.copy()
    bad[1, 0, 0, 0] = np.inf
    got = oracle.diagnostics(bad, cross, floor)
    assert got["state_all_finite"] is False
    assert np.isnan(got["precision_min_eigenvalue"]) and np.isnan(got["precision_max_eigenvalue"])
    assert np.isfinite(got["cross_max_abs"])
    # A non-positive-definite precision: the condition uses the 1e-30 floor.
    neg = evidence.copy()
    shift = mu[0, 0].min() + 1e-3
    neg[0, 0] -= shift * np.eye(6)
    got = oracle.diagnostics(neg, cross, floor)
    np.testing.assert_allclose(got["precision_min_eigenvalue"], -1e-3, rtol=1e-6)
    want = (mu[0, 0].max() - shift) / 1e-30
    assert got["precision_max_condition"] == pytest.approx(want, rel=1e-6)
