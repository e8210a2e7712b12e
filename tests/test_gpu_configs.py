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
from tests.gpu_helpers import NAMES, announce, host, normwise, run_gpu

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


def run_abi(data, bf16, chunk=64):
    """Forward (storing factors) and backward through the C ABI: with
    ``bf16`` the keys, values and queries are torch.bfloat16 tensors (the
    arrays hold bf16-rounded values, so the conversion is exact) and
    m4mr_forward_bf16 / m4mr_backward_bf16 read them; the gradients are
    float32 either way."""
    import torch

    from mamba4_amd import memory

    t = {n: torch.tensor(data[n], device="cuda:0") for n in NAMES}
    if bf16:
        for n in ("keys", "values", "queries"):
            t[n] = t[n].to(torch.bfloat16)
            assert torch.equal(t[n].float().cpu(), torch.tensor(data[n])), n
    args = [t[n] for n in NAMES]
    output, variance, final_s, final_c, solved, factors, start_s, start_c = \
        memory.memread_forward(*args, None, None, chunk)
    d_out = torch.tensor(data["d_output"], device="cuda:0")
    d_var = torch.tensor(data["d_variance"], device="cuda:0")
    grads = memory.memread_backward(*args, solved, factors, start_s, start_c, chunk, d_out,
                                    d_var, None, None)
    torch.cuda.synchronize()
    got = {"output": host(output), "variance": host(variance), "evidence": host(final_s),
           "cross": host(final_c)}
    for n, g in zip(NAMES, grads):
        assert g.dtype == torch.float32
        got["d_" + n] = host(g)
    return got


def run_config(name, oracle_row, grad_tol=1e-3, bf16=False):
    data = workload_inputs(name, seed=0, cotangents=True)
    from mamba4_amd import _lib

    def run(d):
        if bf16:
            return run_abi(d, bf16=True)
        return run_gpu(d, chunk=64, cotangents=_cotangents(d))

    announce(f"{name} full size fwd+bwd{' (bf16 q/k/v entry points)' if bf16 else ''}")
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        full = run(data)
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
        one = run(sliced)
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


def _cotangents(data):
    zero_s = np.zeros(data["keys"].shape[:1] + (data["keys"].shape[2], 64, 64), np.float32)
    return (data["d_output"], data["d_variance"], zero_s, zero_s)


def test_config2_full_size(gpu_lib):
    run_config("config2", oracle_row=15)


def test_config3_full_size_bf16_inputs_slow_decay(gpu_lib):
    """Config 3 with its keys, values and queries as torch.bfloat16 tensors:
    the bf16 entry points run at the full B32 L1024 H12 shape."""
    run_config("config3", oracle_row=31, bf16=True)


def test_config4_decode_full_size(gpu_lib):
    """Decode at the config-4 shape: 2048 sequences x 8 heads of resident
    states, the end states of the config's 1024-token prefill with
    lambda = sigmoid(N(3,1)) (the states the benchmark decodes from), then
    two in-place steps.  Two sampled prefill rows' end states are checked
    against a float64 recurrence of their inputs; a sample of states is
    checked through each step against the float64 oracle's decode_step; every
    read must be finite and satisfy the floor bound."""
    import torch

    from mamba4_amd import SelectiveState, selective_decode_
    from mamba4_amd.inputs import decode_states, device_tokens
    from tests.gpu_helpers import host

    batch, heads, context = 2048, 8, 1024
    announce("config4 decode: 1024-token prefill for the resident states")
    evidence, cross, floor, kept = decode_states(batch, heads, context, seed=0,
                                                 keep_rows=(5, 1500))
    for row, x in kept.items():
        lam = np.exp(x["log_decay"])
        s = np.zeros((heads, 64, 64))
        c = np.zeros((heads, 64, 64))
        for t in range(context):
            k, v, b = x["keys"][t], x["values"][t], x["beta"][t]
            s = lam[t, :, None, None] * s + b[:, None, None] * k[:, :, None] * k[:, None, :]
            c = lam[t, :, None, None] * c + b[:, None, None] * v[:, :, None] * k[:, None, :]
        assert normwise(host(evidence[row]), s) <= 1e-5, row
        assert normwise(host(cross[row]), c) <= 1e-5, row
    floor_h = host(floor)
    sample = np.arange(0, batch, 97)
    s_ref = host(evidence)[sample]
    c_ref = host(cross)[sample]
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(1)
    for step in range(2):
        announce(f"config4 decode: in-place step {step}")
        tok = device_tokens(gen, (batch, heads), shift=False)
        out = selective_decode_(SelectiveState(evidence, cross), *tok, floor)
        got_out, got_var = host(out.output), host(out.variance)
        assert np.isfinite(got_out).all() and np.isfinite(got_var).all()
        q = host(tok[2])
        assert (got_var >= -1e-6).all()
        assert (got_var <= np.sum(q * q, -1) / floor_h.min() * (1 + 1e-5)).all()
        args = [host(t)[sample] for t in tok]
        ref_out, ref_var, s_ref, c_ref = oracle.decode_step(s_ref, c_ref, *args, floor_h)
        assert normwise(got_out[sample], ref_out) <= 1e-4
        assert normwise(got_var[sample], ref_var) <= 1e-4
        assert normwise(host(evidence)[sample], s_ref) <= 1e-5
        assert normwise(host(cross)[sample], c_ref) <= 1e-5
