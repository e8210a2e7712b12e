"""Batched SPD solve (spd_solve, lm/kernels/mamba4.py:190-217) on the GPU.

The HIP solve and its VJP are compared with the float64 oracle
(oracle.memread.spd_solve / spd_solve_backward, pinned against dense
solves and float64 autograd).  The reference's own test problem
(lm/tests/test_mamba4.py:60-81: seven 6x6 systems) uses the reference's
tolerances, rtol 2e-5 on solutions and rtol 2e-4 / atol 2e-5 on gradients;
the 64-wide problems use normwise 1e-4 on solutions and 1e-3 on gradients.
"""

import numpy as np
import pytest
import torch

from oracle import memread as oracle
from tests.gpu_helpers import announce, host, normwise

pytestmark = pytest.mark.gpu


def spd(count, dim, seed, ridge=0.5, garbage_upper=False):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(count, dim, dim))
    a = x @ np.swapaxes(x, -1, -2) / dim + ridge * np.eye(dim)
    rhs = rng.normal(size=(count, dim))
    stored = a.copy()
    if garbage_upper:
        stored += np.triu(rng.normal(size=a.shape) * 100.0, 1)
    return a, stored, rhs


def solve_on_gpu(stored, rhs, cotangent, backend=None):
    from mamba4_amd import spd_solve

    dev = torch.device("cuda:0")
    a = torch.tensor(stored, dtype=torch.float32, device=dev, requires_grad=True)
    b = torch.tensor(rhs, dtype=torch.float32, device=dev, requires_grad=True)
    y = spd_solve(a, b, backend=backend)
    (y * torch.tensor(cotangent, dtype=torch.float32, device=dev)).sum().backward()
    return host(y), host(a.grad), host(b.grad)


def test_reference_problem_matches_dense_solve_and_autograd(gpu_lib):
    announce("spd_solve 7x6x6 reference problem")
    rng = np.random.default_rng(4)
    a = rng.normal(size=(7, 6, 6)).astype(np.float32)
    a = a @ np.swapaxes(a, -1, -2) + 0.5 * np.eye(6, dtype=np.float32)
    rhs = rng.normal(size=(7, 6)).astype(np.float32)
    expected = np.linalg.solve(a.astype(np.float64), rhs.astype(np.float64)[..., None])[..., 0]
    got, d_a, d_rhs = solve_on_gpu(a, rhs, np.cos(expected))
    np.testing.assert_allclose(got, expected, rtol=2e-5, atol=1e-6)
    solution, lower = oracle.spd_solve(a, rhs)
    want_a, want_rhs = oracle.spd_solve_backward(lower, solution, np.cos(expected))
    np.testing.assert_allclose(d_a, want_a, rtol=2e-4, atol=2e-5)
    np.testing.assert_allclose(d_rhs, want_rhs, rtol=2e-4, atol=2e-5)
    np.testing.assert_array_equal(d_a, np.swapaxes(d_a, -1, -2))


@pytest.mark.parametrize("count,dim", [(1000, 64), (37, 17), (5, 1), (9, 63)])
def test_solution_and_gradients_match_oracle(gpu_lib, count, dim):
    announce(f"spd_solve N={count} d={dim} (upper triangle holds garbage)")
    a, stored, rhs = spd(count, dim, seed=count + dim, garbage_upper=True)
    g = np.random.default_rng(3).normal(size=rhs.shape)
    got, d_a, d_rhs = solve_on_gpu(stored, rhs, g, backend="blocked")
    solution, lower = oracle.spd_solve(a, rhs)
    want_a, want_rhs = oracle.spd_solve_backward(lower, solution, g)
    assert normwise(got, solution) <= 1e-4
    assert normwise(d_rhs, want_rhs) <= 1e-3
    assert normwise(d_a, want_a) <= 1e-3


def test_batch_dims_and_every_backend_agree(gpu_lib):
    from mamba4_amd import SOLVERS, spd_solve

    announce("spd_solve batch [2,3] every backend")
    a, _, rhs = spd(6, 12, seed=5)
    dev = torch.device("cuda:0")
    at = torch.tensor(a.reshape(2, 3, 12, 12), dtype=torch.float32, device=dev)
    bt = torch.tensor(rhs.reshape(2, 3, 12), dtype=torch.float32, device=dev)
    first = None
    for backend in SOLVERS:
        y = host(spd_solve(at, bt, backend=backend))
        assert y.shape == (2, 3, 12)
        if first is None:
            first = y
            solution, _ = oracle.spd_solve(a, rhs)
            assert normwise(y.reshape(6, 12), solution) <= 1e-4
        np.testing.assert_array_equal(y, first)
