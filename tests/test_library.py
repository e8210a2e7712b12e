"""Host-only checks of the C ABI and the Python boundary (no GPU needed)."""

import ctypes

import numpy as np
import pytest
import torch

from mamba4_amd import _lib
from mamba4_amd import memory


def test_library_exports_every_header_function():
    lib = _lib.load()
    names = _lib.header_functions()
    assert "m4mr_forward" in names and "m4mr_backward" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of date"


def test_version_and_kernel_names():
    lib = _lib.load()
    assert lib.m4mr_version().decode().startswith("mamba4_memread")
    names = _lib.kernel_names()
    assert "fwd_factor" in names and "factored_solve" in names


def test_invalid_sizes_are_rejected_before_any_launch():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    rc = lib.m4mr_forward(*([null] * 8), 0, 16, 1, 64, 64, *([null] * 8), null)
    assert rc == _lib.EINVAL
    assert "positive" in lib.m4mr_last_error().decode()
    rc = lib.m4mr_forward(*([null] * 8), 1, 16, 1, 64, 65, *([null] * 8), null)
    assert rc == _lib.EINVAL
    assert "chunk" in lib.m4mr_last_error().decode()
    rc = lib.m4mr_forward(*([null] * 8), 1, 16, 1, 96, 16, *([null] * 8), null)
    assert rc == _lib.EINVAL
    assert "value_dim" in lib.m4mr_last_error().decode()
    rc = lib.m4mr_forward(*([null] * 8), 1, 16, 1, 128, 16, *([null] * 8), null)
    assert rc == _lib.EINVAL
    assert "NULL" in lib.m4mr_last_error().decode()
    rc = lib.m4mr_decode_step(*([null] * 8), 6, 4, 64, null, null, null)
    assert rc == _lib.EINVAL
    rc = lib.m4mr_decode_step(*([null] * 8), 8, 4, 32, null, null, null)
    assert rc == _lib.EINVAL
    assert "value_dim" in lib.m4mr_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(_lib.EINVAL)


def test_workspace_size_covers_every_intermediate():
    B, T, H, c = 2, 100, 3, 16
    count = -(-T // c)
    for width in (64, 128):
        need = _lib.load().m4mr_backward_workspace_bytes(B, T, H, width, c)
        tiles = width // 64
        floats = B * T * H * 64 + (1 + tiles) * B * H * count * 4096 + B * H * count * 64
        assert need >= 4 * floats
        assert need % 256 == 0
    assert _lib.load().m4mr_backward_workspace_bytes(B, T, H, 64, 0) == 0
    assert _lib.load().m4mr_backward_workspace_bytes(B, T, H, 80, c) == 0


def test_python_api_rejects_cpu_tensors_and_unknown_solvers():
    k = torch.zeros(1, 4, 1, 8)
    v = torch.zeros(1, 4, 1, 8)
    with pytest.raises(ValueError, match="ROCm device"):
        memory.selective_gaussian_memory(k, v, k, 0.5, -0.1, torch.ones(1, 8))
    with pytest.raises(ValueError, match="Unknown SPD solve backend"):
        memory.selective_gaussian_memory(k, v, k, 0.5, -0.1, torch.ones(1, 8), solver="qr")


def test_shape_mismatch_message_matches_reference():
    k = torch.zeros(1, 4, 1, 8)
    with pytest.raises(ValueError, match="keys, values and queries disagree"):
        memory.selective_gaussian_memory(
            k, torch.zeros(1, 5, 1, 8), k, 0.5, -0.1, torch.ones(1, 8)
        )


def test_synthetic_inputs_follow_the_documented_distributions():
    from mamba4_amd.inputs import synthetic_inputs, round_to_bf16

    d = synthetic_inputs(2, 64, 3, cotangents=True)
    assert np.all(d["keys"][:, 0] == 0)  # shifted: the first write has a zero key
    np.testing.assert_allclose(np.linalg.norm(d["keys"][:, 1:], axis=-1), 1, rtol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(d["queries"], axis=-1), 1, rtol=1e-6)
    assert np.all(d["log_decay"] < 0) and np.all((d["beta"] > 0) & (d["beta"] < 1))
    assert d["floor"].shape == (3, 64) and np.all(d["floor"] == np.float32(1e-2))
    x = np.array([1.0, 1.00390625, 1.0078125, 3.14159], np.float32)
    np.testing.assert_array_equal(
        round_to_bf16(x), torch.tensor(x).to(torch.bfloat16).float().numpy()
    )


def test_spd_solve_arguments_are_checked_before_any_launch():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    buf = ctypes.create_string_buffer(64)
    p = ctypes.c_void_p(ctypes.addressof(buf))
    assert lib.m4mr_spd_solve(p, p, 0, 6, p, null, null) == _lib.EINVAL
    assert lib.m4mr_spd_solve(p, p, 4, 4097, p, null, null) == _lib.EINVAL
    assert "dim" in lib.m4mr_last_error().decode()
    # Above width 128 the factorization runs in the factors buffer.
    assert lib.m4mr_spd_solve(p, p, 4, 129, p, null, null) == _lib.EINVAL
    assert "factors buffer is required" in lib.m4mr_last_error().decode()
    assert lib.m4mr_spd_solve(p, p, 1 << 31, 65, p, p, null) == _lib.EINVAL
    assert lib.m4mr_spd_solve(null, p, 4, 6, p, null, null) == _lib.EINVAL
    assert "NULL" in lib.m4mr_last_error().decode()
    assert lib.m4mr_spd_solve(p, p, 1 << 34, 6, p, null, null) == _lib.EINVAL
    assert lib.m4mr_spd_solve_backward(p, p, p, 4, 0, p, p, null) == _lib.EINVAL
    assert lib.m4mr_spd_solve_backward(p, p, p, 4, 4097, p, p, null) == _lib.EINVAL
    assert lib.m4mr_spd_solve_backward(p, p, null, 4, 6, p, p, null) == _lib.EINVAL
    assert lib.m4mr_factored_solve(p, p, p, 1 << 34, null) == _lib.EINVAL


def test_spd_factor_size_per_width():
    lib = _lib.load()
    assert lib.m4mr_spd_factor_floats(1) == _lib.FACTOR_FLOATS
    assert lib.m4mr_spd_factor_floats(64) == _lib.FACTOR_FLOATS
    assert lib.m4mr_spd_factor_floats(65) == 65 * 65
    assert lib.m4mr_spd_factor_floats(4096) == 4096 * 4096
    assert lib.m4mr_spd_factor_floats(0) == 0
    assert lib.m4mr_spd_factor_floats(4097) == 0


def test_spd_solve_python_checks():
    a = torch.eye(6).expand(7, 6, 6)
    with pytest.raises(ValueError, match="ROCm device"):
        memory.spd_solve(a, torch.zeros(7, 6))
    with pytest.raises(ValueError, match=r"precision \[...,d,d\]"):
        memory.spd_solve(a, torch.zeros(7, 5))
    with pytest.raises(ValueError, match="Unknown SPD solve backend"):
        memory.spd_solve(a, torch.zeros(7, 6), backend="qr")
    with pytest.raises(ValueError, match="widths <= 4096"):
        memory.spd_solve(torch.eye(4097)[None], torch.zeros(1, 4097))


def test_noalloc_backward_rejects_sizes_beyond_its_static_buffer():
    """m4mr_backward_noalloc checks its sizes before any HIP call: config 2
    fits its 128 MiB buffer, a problem four times config 2's does not."""
    lib = _lib.load()
    need = lib.m4mr_backward_workspace_bytes(16, 1024, 8, 64, 64)
    assert 0 < need <= _lib.STATIC_SCRATCH_BYTES
    assert lib.m4mr_backward_workspace_bytes(32, 1024, 16, 64, 64) > _lib.STATIC_SCRATCH_BYTES
    null = ctypes.c_void_p(0)
    rc = lib.m4mr_backward_noalloc(*([null] * 6), 32, 1024, 16, 64, 64, *([null] * 16), null)
    assert rc == _lib.EINVAL
    message = lib.m4mr_last_error().decode()
    assert "static" in message and "m4mr_backward" in message



def test_mamba3_shapes_past_the_finish_kernels_32_bit_slabs_are_rejected():
    """The Mamba-3 backward's finish kernel addresses one (head group, batch)
    slab of its row-gradient partials, ceil(T/64)*64 tokens of 128 floats,
    with 32-bit byte offsets; the shape check refuses any T whose slab would
    reach 2^31 bytes, before any HIP call (every array itself is below 2^31
    elements at B = H = P = 1)."""
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    for entry in (lib.m3s_forward, lib.m3s_forward_bf16):
        rc = entry(*([null] * 9), 1, 1 << 22, 1, 128, 1, 0, *([null] * 4), null)
        assert rc == _lib.EINVAL
        assert "T above" in lib.m4mr_last_error().decode()
        # The longest accepted T passes the shape check and fails on the NULLs.
        rc = entry(*([null] * 9), 1, (1 << 22) - 64, 1, 128, 1, 0, *([null] * 4), null)
        assert rc == _lib.EINVAL
        assert "NULL" in lib.m4mr_last_error().decode()
