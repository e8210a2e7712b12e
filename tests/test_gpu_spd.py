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


@pytest.mark.parametrize("count,dim", [(3, 65), (5, 100), (4, 128), (3, 129), (2, 200), (1, 384)])
def test_wide_systems_match_oracle(gpu_lib, count, dim):
    """Widths above 64 (one block per system; LDS-resident up to 128, in the
    factor buffer above), the reference's any-width solve
    (lm/kernels/mamba4.py:164-217)."""
    announce(f"spd_solve wide N={count} d={dim} (upper triangle holds garbage)")
    a, stored, rhs = spd(count, dim, seed=count + dim, garbage_upper=True)
    g = np.random.default_rng(dim).normal(size=rhs.shape)
    got, d_a, d_rhs = solve_on_gpu(stored, rhs, g, backend="loop")
    solution, lower = oracle.spd_solve(a, rhs)
    want_a, want_rhs = oracle.spd_solve_backward(lower, solution, g)
    assert normwise(got, solution) <= 1e-4
    assert normwise(d_rhs, want_rhs) <= 1e-3
    assert normwise(d_a, want_a) <= 1e-3
    np.testing.assert_array_equal(d_a, np.swapaxes(d_a, -1, -2))


@pytest.mark.parametrize("dim", [65, 160])
def test_wide_stored_factor_reproduces_the_system(gpu_lib, dim):
    """The dense factor the C ABI stores above width 64: L below the
    diagonal, 1/L_ii on it, zero above, with L L^T = precision."""
    from mamba4_amd import _lib

    announce(f"m4mr_spd_solve dense factor d={dim}")
    lib = _lib.load()
    a, stored, rhs = spd(2, dim, seed=dim, garbage_upper=True)
    dev = torch.device("cuda:0")
    at = torch.tensor(stored, dtype=torch.float32, device=dev)
    bt = torch.tensor(rhs, dtype=torch.float32, device=dev)
    y = torch.empty_like(bt)
    floats = lib.m4mr_spd_factor_floats(dim)
    assert floats == dim * dim
    f = torch.full((2, floats), float("nan"), dtype=torch.float32, device=dev)
    rc = lib.m4mr_spd_solve(at.data_ptr(), bt.data_ptr(), 2, dim, y.data_ptr(), f.data_ptr(),
                            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.m4mr_last_error().decode()
    torch.cuda.synchronize()
    factor = host(f).reshape(2, dim, dim).astype(np.float64)
    assert np.all(np.triu(factor, 1) == 0)
    pivots = 1.0 / np.einsum("nii->ni", factor)
    lower = np.tril(factor, -1) + pivots[..., None] * np.eye(dim)
    rebuilt = lower @ np.swapaxes(lower, -1, -2)
    assert normwise(rebuilt, a) <= 1e-5


def test_wide_non_definite_system_gives_nan(gpu_lib):
    announce("spd_solve wide d=96 non-definite")
    from mamba4_amd import spd_solve

    dev = torch.device("cuda:0")
    a = -torch.eye(96, device=dev).expand(2, 96, 96).contiguous()
    y = spd_solve(a, torch.ones(2, 96, device=dev))
    assert torch.isnan(y).all()
