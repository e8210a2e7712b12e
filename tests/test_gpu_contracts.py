"""GPU checks of the memory read's contracts beyond parity.

* A forward that takes no gradient factors without storing (the reference's
  store_factors=False mode, lm/kernels/mamba4_fused.py:183-232, reached
  through the primal chunk_solve, :323-326): every output equals the storing
  forward bit for bit, matches the float64 oracle, and no factor buffer is
  allocated.
* The backward issues only triangular solves with the stored factors and
  chunk contractions: it launches no factorization
  (lm/kernels/mamba4_fused.py:340-366 reruns none).
* The factor kernel's bounded wait between its two waves never yields a
  plausible wrong answer: when it gives up (forced from the host with
  M4MR_TURN_POLLS=-1), every later solution and factor of the block's
  sequences is NaN, every kernel exits normally, and the next call is exact.

Tolerances as in test_gpu_parity: normwise <= 1e-4 on outputs against
float64 at floor 1e-2.
"""

import numpy as np
import pytest
import torch

from oracle import memread as oracle
from tests.gpu_helpers import FACTOR_INDEX, LOWER, NAMES, announce, host, normwise

pytestmark = pytest.mark.gpu


def _inputs(batch, time, heads, value_dim=64, seed=3, bf16=False):
    from mamba4_amd.inputs import synthetic_inputs

    data = synthetic_inputs(batch, time, heads, value_dim=value_dim, seed=seed,
                            cotangents=True, bf16=bf16)
    t = {n: torch.tensor(data[n], device="cuda:0") for n in NAMES}
    if bf16:
        for n in ("keys", "values", "queries"):
            t[n] = t[n].to(torch.bfloat16)
    return data, t


@pytest.mark.parametrize("value_dim,chunk,time,bf16", [(64, 64, 150, False), (128, 16, 90, False),
                                                       (64, 64, 130, True), (64, 5, 33, False)])
def test_store_free_forward_equals_storing_forward(gpu_lib, value_dim, chunk, time, bf16):
    from mamba4_amd import memory

    announce(f"store-free forward P={value_dim} chunk={chunk} T={time} bf16={bf16}")
    data, t = _inputs(3, time, 5, value_dim=value_dim, bf16=bf16)
    args = [t[n] for n in NAMES]
    stored = memory.memread_forward(*args, None, None, chunk)
    free = memory.memread_forward(*args, None, None, chunk, store_factors=False)
    torch.cuda.synchronize()
    assert stored[5] is not None and free[5] is None
    for i, (a, b) in enumerate(zip(stored, free)):
        if i != 5:
            assert torch.equal(a, b), i
    # Against the float64 oracle (the bf16 case reads the bf16-rounded values).
    x = [np.asarray(data[n], np.float64) for n in NAMES]
    out, var, s, c = oracle.dense_reference(*x)
    assert normwise(host(free[0]), out) <= 1e-4
    assert normwise(host(free[1]), var) <= 1e-4
    assert normwise(host(free[2]), s) <= 1e-5
    assert normwise(host(free[3]), c) <= 1e-5


def test_no_grad_forward_allocates_no_factor_buffer(gpu_lib):
    """selective_gaussian_memory under no gradient: store-free, and its peak
    device allocation stays far below one factor buffer; the same call with
    gradients allocates it."""
    from mamba4_amd import _lib, selective_gaussian_memory

    batch, time, heads = 4, 1024, 8
    factor_bytes = batch * time * heads * _lib.FACTOR_FLOATS * 4
    announce(f"no-grad forward memory B{batch} T{time} H{heads}")
    data, t = _inputs(batch, time, heads, seed=5)
    args = [t[n] for n in NAMES]
    peaks = {}
    outputs = {}
    for mode in ("no_grad", "grad"):
        grad_args = [a.clone().requires_grad_(mode == "grad") for a in args]
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        with torch.set_grad_enabled(mode == "grad"):
            r = selective_gaussian_memory(*grad_args)
        torch.cuda.synchronize()
        peaks[mode] = torch.cuda.max_memory_allocated() - base
        outputs[mode] = (r.output.detach(), r.variance.detach())
        del r, grad_args
    assert peaks["no_grad"] < factor_bytes / 2, peaks
    assert peaks["grad"] >= factor_bytes, peaks
    assert torch.equal(outputs["no_grad"][0], outputs["grad"][0])
    assert torch.equal(outputs["no_grad"][1], outputs["grad"][1])


def test_mixer_read_no_grad_equals_grad_path(gpu_lib):
    """mixer_read without a gradient takes the store-free factor kernel; its
    outputs equal the differentiable call's bit for bit."""
    from mamba4_amd import mixer_read

    rng = np.random.default_rng(11)
    B, T, H = 2, 100, 3

    def g(*shape, scale=1.0):
        return torch.tensor(rng.normal(size=shape) * scale, dtype=torch.float32,
                            device="cuda:0")

    args = [g(B, T, H, 64), g(B, T, H, 64), g(B, T, H, 64), g(B, T, H), g(B, T, H),
            g(H, scale=0.1), g(H, scale=0.1), g(H, scale=0.1), g(H, 64), g(H, scale=0.1) + 1,
            g(H, scale=0.1)]
    announce("mixer_read no-grad vs grad")
    with torch.no_grad():
        free = mixer_read(*args)
    grad_args = [a.clone().requires_grad_(True) for a in args]
    stored = mixer_read(*grad_args)
    torch.cuda.synchronize()
    assert torch.equal(free.output, stored.output.detach())
    assert torch.equal(free.variance, stored.variance.detach())
    assert torch.equal(free.state.evidence, stored.state.evidence.detach())


def test_backward_launches_no_factorization(gpu_lib):
    """m4mr_backward runs the re-solve with the stored factors and the chunk
    kernels only: zero factor or SPD-solve launches."""
    from mamba4_amd import _lib, memory

    announce("backward launch census")
    data, t = _inputs(2, 200, 3, seed=9)
    args = [t[n] for n in NAMES]
    fwd = memory.memread_forward(*args, None, None, 64)
    torch.cuda.synchronize()
    d_out = torch.tensor(data["d_output"], device="cuda:0")
    d_var = torch.tensor(data["d_variance"], device="cuda:0")
    _lib.profile_reset()
    _lib.profile_select(None)
    _lib.profile_enable(True)
    try:
        memory.memread_backward(*args, *fwd[4:], 64, d_out, d_var, None, None)
        torch.cuda.synchronize()
    finally:
        _lib.profile_enable(False)
    launches = {name: _lib.profile_read(name)[1] for name in _lib.kernel_names()}
    _lib.profile_reset()
    assert launches["fwd_factor"] == 0 and launches["spd_solve"] == 0, launches
    assert launches["decode_step"] == 0, launches
    assert launches["factored_solve"] == 1, launches
    assert launches["bwd_grads"] == 1, launches


def test_factor_wait_give_up_poisons_instead_of_corrupting(gpu_lib, monkeypatch):
    """M4MR_TURN_POLLS=-1 makes every turn wait of the factor kernel give up
    (the host forces the condition; the kernel's waits all end).  Every token
    after the first of each 32-token sub-chunk must then read NaN, with NaN
    solutions and factors, while the chunk-boundary states, which the factor
    kernel does not touch, stay finite.  Clearing the variable restores the
    exact results."""
    from mamba4_amd import memory

    time, chunk = 96, 64
    data, t = _inputs(2, time, 5, seed=13)
    args = [t[n] for n in NAMES]
    announce("factor kernel turn wait forced to give up")
    monkeypatch.setenv("M4MR_TURN_POLLS", "-1")
    bad = memory.memread_forward(*args, None, None, chunk)
    torch.cuda.synchronize()
    monkeypatch.delenv("M4MR_TURN_POLLS")
    announce("factor kernel after the forced give-up")
    good = memory.memread_forward(*args, None, None, chunk)
    torch.cuda.synchronize()
    starts = np.arange(time) % 32 == 0  # first token of each sub-chunk
    out, var, solved, factors = (host(bad[i]) for i in (0, 1, 4, 5))
    assert np.isnan(out[:, ~starts]).all() and np.isnan(var[:, ~starts]).all()
    assert np.isnan(solved[:, ~starts]).all()
    # Every lower-triangle entry (above the diagonal a stored quad holds zeros).
    assert np.isnan(factors[:, ~starts][..., FACTOR_INDEX[LOWER]]).all()
    assert np.isfinite(host(bad[6])).all() and np.isfinite(host(bad[7])).all()
    x = [np.asarray(data[n], np.float64) for n in NAMES]
    ref_out, ref_var, _, _ = oracle.dense_reference(*x)
    assert normwise(host(good[0]), ref_out) <= 1e-4
    assert normwise(host(good[1]), ref_var) <= 1e-4
