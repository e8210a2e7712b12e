"""Full-size BASELINE configurations on the GPU.

The HIP path runs the whole workload; the float64 oracle checks a subset of
batch rows (rows are independent sequences), and size-independent
properties are checked on every row:

* every output, state and gradient is finite;
* 0 <= variance <= |q|^2 / min(floor) (floor bound,
  lm/tests/test_mamba4.py:46-58);
* the shifted first token has a zero key, so its variance is
  sum(q^2 / floor) and its read is zero (lm/tests/test_mamba4.py:364-375);
* a one-row slice run on its own reproduces that row of the full batch
  bit for bit (rows share no state), on the same chunk-boundary state walk
  as the full batch took.
Tolerance: normwise max|d| / max|ref| <= 1e-4 on outputs, <= 1e-3 on
gradients.
"""

import os

import numpy as np
import pytest

from mamba4_amd.inputs import workload_inputs
from oracle import memread as oracle
from tests.gpu_helpers import NAMES, announce, normwise, run_gpu

pytestmark = pytest.mark.gpu


def rows_of(data, rows):
    return {k: (v[rows] if k != "floor" else v) for k, v in data.items()}


def check_properties(data, got):
    for key, value in got.items():
        assert np.isfinite(value).all(), key
    q = data["queries"].astype(np.float64)
    bound = np.sum(q * q, axis=-1) / data["floor"].min()
    assert (got["variance"] >= -1e-6).all()
    assert (got["variance"] <= bound * (1 + 1e-5)).all()
    first = np.sum(q[:, 0] ** 2 / data["floor"][None].astype(np.float64), axis=-1)
    np.testing.assert_allclose(got["variance"][:, 0], first, rtol=1e-5)
    assert np.abs(got["output"][:, 0]).max() == 0.0


def run_config(name, oracle_row, grad_tol=1e-3):
    data = workload_inputs(name, seed=0, cotangents=True)
    cot = (data["d_output"], data["d_variance"], None, None)
    from mamba4_amd import _lib

    announce(f"{name} full size fwd+bwd")
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        full = run_gpu(data, chunk=64, cotangents=_cotangents(data))
    finally:
        _lib.profile_enable(False)
    walk = "fused" if _lib.profile_read("fwd_states")[1] else "split"
    _lib.profile_reset()
    check_properties(data, full)
    announce(f"{name} one-row slice, {walk} state walk")
    sliced = rows_of(data, slice(oracle_row, oracle_row + 1))
    saved = os.environ.get("M4MR_STATE_WALK")
    os.environ["M4MR_STATE_WALK"] = walk
    try:
        one = run_gpu(sliced, chunk=64, cotangents=_cotangents(sliced))
    finally:
        if saved is None:
            del os.environ["M4MR_STATE_WALK"]
        else:
            os.environ["M4MR_STATE_WALK"] = saved
    for key in ["output", "variance", "evidence", "cross", "d_keys", "d_values",
                "d_queries", "d_beta", "d_log_decay"]:
        np.testing.assert_array_equal(one[key][0], full[key][oracle_row], err_msg=key)
    args = [sliced[n].astype(np.float64) for n in NAMES]
    out, var, s, c = oracle.dense_reference(*args)
    for key, ref in zip(["output", "variance", "evidence", "cross"], (out, var, s, c)):
        err = normwise(one[key], ref)
        assert err <= 1e-4, (name, key, err)
    _, res = oracle.forward(*args, chunk=64)
    grads = oracle.backward(res, sliced["d_output"], sliced["d_variance"])
    for n in NAMES:
        err = normwise(one["d_" + n], grads[n])
        assert err <= grad_tol, (name, n, err)
    del cot


def _cotangents(data):
    zero_s = np.zeros(data["keys"].shape[:1] + (data["keys"].shape[2], 64, 64), np.float32)
    return (data["d_output"], data["d_variance"], zero_s, zero_s)


def test_config2_full_size(gpu_lib):
    run_config("config2", oracle_row=15)


def test_config3_full_size_bf16_inputs_slow_decay(gpu_lib):
    run_config("config3", oracle_row=31)


def test_config4_decode_full_size(gpu_lib):
    """Decode at the config-4 shape: 2048 sequences x 8 heads of resident
    states (here the end states of a 16-token prefill), two in-place steps.
    A sample of states is checked against the float64 oracle's decode_step;
    every read must be finite and satisfy the floor bound."""
    import torch

    from mamba4_amd import SelectiveState, selective_decode_, selective_gaussian_memory
    from mamba4_amd.inputs import synthetic_inputs
    from tests.gpu_helpers import host, to_device

    batch, heads = 2048, 8
    data = synthetic_inputs(batch, 17, heads, decay_mean=3.0, seed=4)
    announce("config4 decode: 16-token prefill for the resident states")
    prefix = to_device([data[n][:, :16] if n != "floor" else data[n] for n in NAMES])
    with torch.no_grad():
        state = selective_gaussian_memory(*prefix, chunk_size=16).state
    evidence, cross = state.evidence.contiguous(), state.cross.contiguous()
    sample = np.arange(0, batch, 97)
    s_ref = host(evidence)[sample]
    c_ref = host(cross)[sample]
    for step in range(2):
        announce(f"config4 decode: in-place step {step}")
        t = 16 if step == 0 else 15
        tok = to_device([data[n][:, t] for n in NAMES if n != "floor"])
        floor = to_device([data["floor"]])[0]
        out = selective_decode_(SelectiveState(evidence, cross), *tok, floor)
        got_out, got_var = host(out.output), host(out.variance)
        assert np.isfinite(got_out).all() and np.isfinite(got_var).all()
        q = data["queries"][:, t].astype(np.float64)
        assert (got_var >= -1e-6).all()
        assert (got_var <= np.sum(q * q, -1) / data["floor"].min() * (1 + 1e-5)).all()
        args = [data[n][sample, t] for n in ["keys", "values", "queries", "beta", "log_decay"]]
        ref_out, ref_var, s_ref, c_ref = oracle.decode_step(s_ref, c_ref, *args, data["floor"])
        assert normwise(got_out[sample], ref_out) <= 1e-4
        assert normwise(got_var[sample], ref_var) <= 1e-4
        assert normwise(host(evidence)[sample], s_ref) <= 1e-5
        assert normwise(host(cross)[sample], c_ref) <= 1e-5

