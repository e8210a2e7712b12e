"""GPU parity of the HIP memory read against the pinned CPU oracle.

Tolerances (fp32 HIP vs float64 oracle):
* reference test shapes (floor >= 0.25): the reference's own tolerances,
  values rtol 3e-5 / atol 3e-6 (lm/tests/test_mamba4.py:43), gradients
  rtol 2e-4 / atol 2e-5 (:103, :404);
* benchmark configs (floor 1e-2): normwise max|d| / max|ref| <= 1e-4 on
  outputs and state, <= 1e-3 on gradients.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import memread as oracle
from tests.gpu_helpers import (FACTOR_INDEX, LOWER, NAMES, announce, host, normwise,
                               pack_factors, run_gpu, to_device, unpack_factors)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "config0.npz")


def arrays(time=13, heads=3, dim=4, value_dim=5, seed=0, batch=2):
    """The reference test fixture's distributions (lm/tests/test_mamba4.py:19-29)."""
    rng = np.random.default_rng(seed)
    k = rng.normal(size=(batch, time, heads, dim)).astype(np.float32)
    q = rng.normal(size=k.shape).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    v = rng.normal(size=(batch, time, heads, value_dim)).astype(np.float32)
    beta = rng.uniform(0.05, 1.0, size=k.shape[:-1]).astype(np.float32)
    decay = rng.uniform(0.3, 0.999, size=k.shape[:-1]).astype(np.float32)
    floor = rng.uniform(0.25, 1.5, size=(heads, dim)).astype(np.float32)
    return dict(keys=k, values=v, queries=q, beta=beta, log_decay=np.log(decay), floor=floor)


@pytest.mark.parametrize("chunk", [1, 4, 5, 13, 16, 64])
def test_chunked_reads_match_dense_oracle(gpu_lib, chunk):
    # lm/tests/test_mamba4.py:32-43, every chunk size incl. padded chunks.
    data = arrays()
    announce(f"chunked reads chunk={chunk} B2 T13 H3 D4 P5")
    got = run_gpu(data, chunk=chunk)
    want = oracle.dense_reference(*(data[n] for n in NAMES))
    for key, ref in zip(["output", "variance", "evidence", "cross"], want):
        np.testing.assert_allclose(got[key], ref, rtol=3e-5, atol=3e-6, err_msg=key)


@pytest.mark.parametrize("chunk", [4, 8, 64])
def test_all_gradients_match_oracle(gpu_lib, chunk):
    # lm/tests/test_mamba4.py:84-104 and :382-404, with an initial state and
    # cotangents on every output including the final state.
    data = arrays(time=21, dim=6)
    rng = np.random.default_rng(12)
    root = rng.normal(size=(2, 3, 6, 6)) / 6
    s0 = (root @ np.swapaxes(root, -1, -2)).astype(np.float32)
    c0 = (rng.normal(size=(2, 3, 5, 6)) * 0.3).astype(np.float32)
    d_out = rng.normal(size=data["values"].shape).astype(np.float32)
    d_var = rng.normal(size=data["beta"].shape).astype(np.float32)
    d_s = rng.normal(size=s0.shape).astype(np.float32)
    d_s = 0.5 * (d_s + np.swapaxes(d_s, -1, -2))
    d_c = rng.normal(size=c0.shape).astype(np.float32)
    announce(f"gradients chunk={chunk} B2 T21 H3 D6 P5")
    got = run_gpu(data, chunk=chunk, initial=(s0, c0), cotangents=(d_out, d_var, d_s, d_c))
    args = [data[n].astype(np.float64) for n in NAMES]
    _, res = oracle.forward(*args, chunk=chunk, initial=(s0, c0))
    want = oracle.backward(res, d_out, d_var, d_s, d_c)
    for n in NAMES:
        np.testing.assert_allclose(got["d_" + n], want[n], rtol=2e-4, atol=2e-5, err_msg=n)
        assert np.linalg.norm(got["d_" + n]) > 1e-6, n
    np.testing.assert_allclose(
        got["d_initial_evidence"], want["initial_evidence"], rtol=2e-4, atol=2e-5
    )
    np.testing.assert_allclose(got["d_initial_cross"], want["initial_cross"], rtol=2e-4, atol=2e-5)


def test_config0_matches_golden_fixture(gpu_lib):
    g = np.load(GOLDEN)
    data = {n: g["in_" + n] for n in NAMES}
    cot = (g["d_output"], g["d_variance"], g["d_final_evidence"], g["d_final_cross"])
    announce("config0 golden B2 L256 H1 D64 fwd+bwd")
    got = run_gpu(data, chunk=64, cotangents=cot)
    for key in ["output", "variance", "evidence", "cross"]:
        err = normwise(got[key], g[key])
        assert err <= 1e-4, (key, err)
    for n in NAMES:
        err = normwise(got["d_" + n], g["grad_" + n])
        assert err <= 1e-3, (n, err)


def test_config0_chunk_sizes_agree_with_golden(gpu_lib):
    g = np.load(GOLDEN)
    data = {n: g["in_" + n] for n in NAMES}
    for chunk in (16, 32, 37):
        announce(f"config0 chunk={chunk}")
        got = run_gpu(data, chunk=chunk)
        assert normwise(got["output"], g["output"]) <= 1e-4, chunk
        assert normwise(got["variance"], g["variance"]) <= 1e-4, chunk


def test_continuation_and_decode_match_prefill(gpu_lib):
    # lm/tests/test_mamba4.py:107-134.
    from mamba4_amd import SelectiveState, selective_decode, selective_gaussian_memory

    data = arrays()
    announce("continuation + decode B2 T13 H3 D4 P5")
    full = run_gpu(data, chunk=4)
    first = run_gpu({n: (data[n][:, :6] if n != "floor" else data[n]) for n in NAMES}, chunk=4)
    second = run_gpu(
        {n: (data[n][:, 6:] if n != "floor" else data[n]) for n in NAMES},
        chunk=4,
        initial=(first["evidence"], first["cross"]),
    )
    np.testing.assert_allclose(second["output"], full["output"][:, 6:], rtol=3e-5, atol=3e-6)
    dev = torch.device("cuda:0")
    state = SelectiveState(torch.zeros(2, 3, 4, 4, device=dev), torch.zeros(2, 3, 5, 4, device=dev))
    t = lambda a: torch.tensor(a, device=dev)  # noqa: E731
    for i in range(13):
        step = selective_decode(
            state, t(data["keys"][:, i]), t(data["values"][:, i]), t(data["queries"][:, i]),
            t(data["beta"][:, i]), t(data["log_decay"][:, i]), t(data["floor"]),
        )
        state = step.state
        np.testing.assert_allclose(host(step.output), full["output"][:, i], rtol=3e-5, atol=3e-6)
        np.testing.assert_allclose(host(step.variance), full["variance"][:, i], rtol=3e-5, atol=3e-6)
    np.testing.assert_allclose(host(state.evidence), full["evidence"], rtol=3e-5, atol=3e-6)


def test_exact_recall_of_orthonormal_keys(gpu_lib):
    # lm/tests/test_mamba4.py:137-152: read(k_i) = v_i / (1 + floor / beta).
    dim, value_dim = 4, 3
    keys = np.eye(dim, dtype=np.float32)[None, :, None, :]
    values = np.random.default_rng(1).normal(size=(1, dim, 1, value_dim)).astype(np.float32)
    data = dict(
        keys=keys, values=values, queries=keys, beta=np.full((1, dim, 1), 2.0, np.float32),
        log_decay=np.zeros((1, dim, 1), np.float32), floor=np.full((1, dim), 1e-3, np.float32),
    )
    announce("exact recall")
    got = run_gpu(data, chunk=2)
    np.testing.assert_allclose(got["output"], values / (1 + 5e-4), rtol=1e-5)


def test_stored_factors_reproduce_each_precision(gpu_lib):
    """Calls m4mr_forward through the C ABI and unpacks the packed factors."""
    data = arrays(time=10, heads=2, dim=64, value_dim=64, seed=3)
    data["floor"] = np.full_like(data["floor"], 0.05)
    B, T, H, c = 2, 10, 2, 4
    dev = torch.device("cuda:0")
    ins = to_device([data[n] for n in NAMES])
    f32 = dict(dtype=torch.float32, device=dev)
    count, starts = -(-T // c), -(-T // c)
    outs = dict(
        output=torch.empty(B, T, H, 64, **f32), variance=torch.empty(B, T, H, **f32),
        final_s=torch.empty(B, H, 64, 64, **f32), final_c=torch.empty(B, H, 64, 64, **f32),
        solved=torch.empty(B, T, H, 64, **f32), factors=torch.empty(B, T, H, 2176, **f32),
        start_s=torch.empty(B, H, starts, 64, 64, **f32), start_c=torch.empty(B, H, count, 64, 64, **f32),
    )
    announce("C-ABI forward, factor unpack B2 T10 H2 D64")
    rc = gpu_lib.m4mr_forward(
        *(t.data_ptr() for t in ins), None, None, B, T, H, 64, c,
        *(t.data_ptr() for t in outs.values()), torch.cuda.current_stream().cuda_stream,
    )
    assert rc == 0, gpu_lib.m4mr_last_error()
    torch.cuda.synchronize()
    lower = unpack_factors(host(outs["factors"]))
    diag = np.einsum("...ii->...i", lower)
    true_lower = np.tril(lower, -1) + np.einsum("...i,ij->...ij", 1 / diag, np.eye(64))
    rebuilt = true_lower @ np.swapaxes(true_lower, -1, -2)
    for t in range(T):
        _, _, s_t, _ = oracle.dense_reference(
            *(data[n][:, : t + 1] if n != "floor" else data[n] for n in NAMES)
        )
        a_t = s_t + data["floor"][None, :, :, None] * np.eye(64)
        assert normwise(rebuilt[:, t], a_t) < 1e-5, t
    y = np.linalg.solve(
        rebuilt, data["queries"].astype(np.float64)[..., None]
    )[..., 0]
    assert normwise(host(outs["solved"]), y) < 1e-4


def test_factored_solve_entry_point(gpu_lib):
    rng = np.random.default_rng(8)
    N = 37
    a = rng.normal(size=(N, 64, 64))
    a = a @ np.swapaxes(a, -1, -2) / 64 + 0.1 * np.eye(64)
    packed = pack_factors(oracle.cholesky_reciprocal(a))
    rhs = rng.normal(size=(N, 64))
    fac, r = to_device([packed, rhs])
    z = torch.empty_like(r)
    announce("factored_solve N=37")
    rc = gpu_lib.m4mr_factored_solve(
        fac.data_ptr(), r.data_ptr(), z.data_ptr(), N, torch.cuda.current_stream().cuda_stream
    )
    assert rc == 0
    torch.cuda.synchronize()
    want = np.linalg.solve(a, rhs[..., None])[..., 0]
    assert normwise(host(z), want) < 1e-4


def test_nonpositive_floor_propagates_nan(gpu_lib):
    # Failure mode of the reference (lm/kernels/mamba4_fused.py:111): a
    # non-positive pivot gives NaN rather than an error.
    data = arrays(time=5)
    data["keys"][:, 0] = 0.0
    data["floor"][0, 0] = -1.0
    announce("negative floor NaN propagation")
    got = run_gpu(data, chunk=4)
    assert np.isnan(got["variance"][:, 0, 0]).all()
    assert np.isfinite(got["variance"][:, :, 1:]).all()


def decode_problem(batch=4, heads=8, seed=21, steps=1):
    """Resident states after a 96-token prefill (slow decay, floor 1e-2),
    then `steps` new tokens, as BASELINE config 4 at a small batch."""
    from mamba4_amd.inputs import synthetic_inputs

    pre = synthetic_inputs(batch, 96 + steps, heads, decay_mean=3.0, seed=seed)
    head = {n: (pre[n][:, :96] if n != "floor" else pre[n]) for n in NAMES}
    _, _, s, c = oracle.dense_reference(*(head[n] for n in NAMES))
    tail = {n: (pre[n][:, 96:] if n != "floor" else pre[n]) for n in NAMES}
    return s.astype(np.float32), c.astype(np.float32), tail


def test_decode_in_place_matches_oracle_over_steps(gpu_lib):
    from mamba4_amd import SelectiveState, selective_decode_

    s, c, tail = decode_problem(steps=5)
    dev = torch.device("cuda:0")
    state = SelectiveState(torch.tensor(s, device=dev), torch.tensor(c, device=dev))
    want_s, want_c = s.astype(np.float64), c.astype(np.float64)
    announce("in-place decode B4 H8 D64, 5 steps")
    for i in range(5):
        args = [tail[n][:, i] if n != "floor" else tail[n] for n in NAMES]
        step = selective_decode_(state, *(torch.tensor(a, device=dev) for a in args))
        out, var, want_s, want_c = oracle.decode_step(want_s, want_c, *args)
        assert normwise(host(step.output), out) <= 1e-4, i
        assert normwise(host(step.variance), var) <= 1e-4, i
    assert normwise(host(state.evidence), want_s) <= 1e-5
    assert normwise(host(state.cross), want_c) <= 1e-5


def test_decode_gradients_match_one_token_oracle(gpu_lib):
    from mamba4_amd import SelectiveState, selective_decode

    s, c, tail = decode_problem(batch=2, heads=3, seed=5)
    dev = torch.device("cuda:0")
    args = [tail[n][:, 0] if n != "floor" else tail[n] for n in NAMES]
    tensors = [torch.tensor(a, device=dev, requires_grad=True) for a in args]
    st = [torch.tensor(x, device=dev, requires_grad=True) for x in (s, c)]
    rng = np.random.default_rng(3)
    d_out = rng.normal(size=(2, 3, 64))
    d_var = rng.normal(size=(2, 3))
    announce("differentiable decode B2 H3 D64")
    step = selective_decode(SelectiveState(*st), *tensors)
    loss = (step.output * torch.tensor(d_out, device=dev, dtype=torch.float32)).sum()
    loss = loss + (step.variance * torch.tensor(d_var, device=dev, dtype=torch.float32)).sum()
    loss.backward()
    one = {n: (tail[n][:, :1] if n != "floor" else tail[n]) for n in NAMES}
    _, res = oracle.forward(*(one[n].astype(np.float64) for n in NAMES), chunk=1, initial=(s, c))
    want = oracle.backward(res, d_out[:, None], d_var[:, None])
    for n, t in zip(NAMES, tensors):
        got = host(t.grad)
        ref = want[n][:, 0] if n != "floor" else want[n]
        assert normwise(got, ref) <= 1e-3, n
    assert normwise(host(st[0].grad), want["initial_evidence"]) <= 1e-3
    assert normwise(host(st[1].grad), want["initial_cross"]) <= 1e-3


@pytest.mark.parametrize("time, chunk", [(90, 64), (1, 64), (33, 64), (65, 64), (7, 3)])
def test_ragged_lengths_and_empty_sub_chunks(gpu_lib, time, chunk):
    """Sequence ends inside a chunk, an empty second sub-chunk (T=90: the
    last chunk holds 26 tokens), a single token, and chunk boundaries +-1."""
    data = arrays(time=time, heads=3, dim=64, value_dim=64, seed=time)
    data["floor"] = np.full_like(data["floor"], 0.05)
    announce(f"ragged T={time} chunk={chunk}")
    got = run_gpu(data, chunk=chunk)
    want = oracle.dense_reference(*(data[n] for n in NAMES))
    for key, ref in zip(["output", "variance", "evidence", "cross"], want):
        assert normwise(got[key], ref) <= 1e-5, (key, time, chunk)


@pytest.mark.parametrize("scale", [1e-3, 1e-2, 1.0, 1e2])
def test_outputs_and_gradients_hold_at_every_input_scale(gpu_lib, scale):
    """Keys scaled by s and the floor by s^2 scale every evidence matrix by
    s^2: the same problem at another magnitude.  The factorization's trailing
    updates carry panel values as f16 pieces, so a row whose floor lies
    outside [2^-8, 2^8) is factored at a power-of-two scale (s^2 = 1e-6:
    panel values near 1e-3 would otherwise sit in f16's subnormal range, and
    s^2 = 1e4 tests the other side); the tolerances are the configs' own."""
    from mamba4_amd.inputs import synthetic_inputs

    data = synthetic_inputs(2, 160, 2, seed=31, floor_value=1e-2, cotangents=True)
    data["keys"] = (data["keys"] * scale).astype(np.float32)
    data["floor"] = (data["floor"] * scale * scale).astype(np.float32)
    d_out, d_var = data["d_output"], data["d_variance"]
    zeros_s = np.zeros((2, 2, 64, 64), np.float32)
    zeros_c = np.zeros((2, 2, 64, 64), np.float32)
    announce(f"input scale {scale:g}: B2 T160 H2 D64, floor 1e-2 x {scale * scale:g}")
    got = run_gpu(data, chunk=64, cotangents=(d_out, d_var, zeros_s, zeros_c))
    args = [data[n].astype(np.float64) for n in NAMES]
    (out, var, s_end, c_end), res = oracle.forward(*args, chunk=64)
    for key, ref in zip(["output", "variance", "evidence", "cross"], (out, var, s_end, c_end)):
        assert normwise(got[key], ref) <= 1e-4, (key, normwise(got[key], ref))
    want = oracle.backward(res, d_out.astype(np.float64), d_var.astype(np.float64))
    for n in NAMES:
        assert normwise(got["d_" + n], want[n]) <= 1e-3, (n, normwise(got["d_" + n], want[n]))


@pytest.mark.parametrize("value_dim,chunk", [(128, 64), (100, 16), (128, 5)])
def test_wide_value_heads_forward_and_gradients(gpu_lib, value_dim, chunk):
    """P = 128 value heads, the reference's trained memory_head_dim
    (lm/configs/mamba4-60m.json, mamba4-125m.json): every value-dependent
    product runs per 64-column value tile.  P = 100 is zero-padded to 128."""
    data = arrays(time=150, heads=2, dim=64, value_dim=value_dim, seed=21)
    rng = np.random.default_rng(22)
    root = rng.normal(size=(2, 2, 64, 64)) / 64
    s0 = (root @ np.swapaxes(root, -1, -2)).astype(np.float32)
    c0 = (rng.normal(size=(2, 2, value_dim, 64)) * 0.3).astype(np.float32)
    d_out = rng.normal(size=data["values"].shape).astype(np.float32)
    d_var = rng.normal(size=data["beta"].shape).astype(np.float32)
    d_s = rng.normal(size=s0.shape).astype(np.float32)
    d_s = 0.5 * (d_s + np.swapaxes(d_s, -1, -2))
    d_c = rng.normal(size=c0.shape).astype(np.float32)
    announce(f"wide values P={value_dim} chunk={chunk} B2 T150 H2 D64")
    got = run_gpu(data, chunk=chunk, initial=(s0, c0), cotangents=(d_out, d_var, d_s, d_c))
    args = [data[n].astype(np.float64) for n in NAMES]
    (out, var, s_end, c_end), res = oracle.forward(*args, chunk=chunk, initial=(s0, c0))
    for key, ref in zip(["output", "variance", "evidence", "cross"], (out, var, s_end, c_end)):
        assert normwise(got[key], ref) <= 1e-4, key
    want = oracle.backward(res, d_out, d_var, d_s, d_c)
    for n in NAMES:
        assert normwise(got["d_" + n], want[n]) <= 1e-3, n
    assert normwise(got["d_initial_evidence"], want["initial_evidence"]) <= 1e-3
    assert normwise(got["d_initial_cross"], want["initial_cross"]) <= 1e-3


def test_wide_value_heads_decode_in_place(gpu_lib):
    from mamba4_amd import SelectiveState, selective_decode, selective_decode_

    pre = arrays(time=40, heads=4, dim=64, value_dim=128, seed=32, batch=3)
    _, _, s, c = oracle.dense_reference(*(pre[n] for n in NAMES))
    s, c = s.astype(np.float32), c.astype(np.float32)
    dev = torch.device("cuda:0")
    state = SelectiveState(torch.tensor(s, device=dev), torch.tensor(c, device=dev))
    want_s, want_c = s.astype(np.float64), c.astype(np.float64)
    tok = arrays(time=3, heads=4, dim=64, value_dim=128, seed=33, batch=3)
    tok["floor"] = pre["floor"]
    announce("in-place decode P=128 B3 H4 D64, 3 steps")
    for i in range(3):
        args = [tok[n][:, i] if n != "floor" else tok[n] for n in NAMES]
        step = selective_decode_(state, *(torch.tensor(a, device=dev) for a in args))
        out, var, want_s, want_c = oracle.decode_step(want_s, want_c, *args)
        assert normwise(host(step.output), out) <= 1e-4, i
        assert normwise(host(step.variance), var) <= 1e-4, i
    assert normwise(host(state.evidence), want_s) <= 1e-5
    assert normwise(host(state.cross), want_c) <= 1e-5
    # A narrower value width (96) pads to 128 on the copying path.
    narrow = SelectiveState(torch.tensor(s, device=dev), torch.tensor(c[:, :, :96], device=dev))
    args = [tok[n][:, 0] if n != "floor" else tok[n] for n in NAMES]
    args[1] = args[1][..., :96]
    step = selective_decode(narrow, *(torch.tensor(a, device=dev) for a in args))
    out, var, _, _ = oracle.decode_step(s.astype(np.float64), c[:, :, :96].astype(np.float64),
                                        *args)
    assert normwise(host(step.output), out) <= 1e-4
    assert normwise(host(step.variance), var) <= 1e-4



@pytest.fixture(params=["split", "fused", "fused1"])
def state_walk(request, monkeypatch):
    """Both chunk-boundary state paths (M4MR_STATE_WALK), forced at any size;
    the fused walk with two LDS step buffers and with one (M4MR_STATE_BUFFERS)."""
    monkeypatch.setenv("M4MR_STATE_WALK", request.param[:5])
    monkeypatch.setenv("M4MR_STATE_BUFFERS", "1" if request.param == "fused1" else "2")
    return request.param[:5]


@pytest.mark.parametrize("value_dim,chunk,time", [(5, 4, 21), (64, 64, 90), (128, 48, 100)])
def test_state_walks_match_oracle(gpu_lib, state_walk, value_dim, chunk, time):
    """Forward and every gradient through either state path, with an initial
    state and final-state cotangents: ragged last chunks with an empty second
    sub-chunk (T = 90, 100), P = 128, and chunks without sub-chunks (4)."""
    from mamba4_amd import _lib

    dim = 6 if value_dim == 5 else 64
    data = arrays(time=time, heads=3, dim=dim, value_dim=value_dim, seed=time)
    rng = np.random.default_rng(time + 1)
    root = rng.normal(size=(2, 3, dim, dim)) / dim
    s0 = (root @ np.swapaxes(root, -1, -2)).astype(np.float32)
    c0 = (rng.normal(size=(2, 3, value_dim, dim)) * 0.3).astype(np.float32)
    d_out = rng.normal(size=data["values"].shape).astype(np.float32)
    d_var = rng.normal(size=data["beta"].shape).astype(np.float32)
    d_s = rng.normal(size=s0.shape).astype(np.float32)
    d_s = 0.5 * (d_s + np.swapaxes(d_s, -1, -2))
    d_c = rng.normal(size=c0.shape).astype(np.float32)
    announce(f"state walk {state_walk} P={value_dim} chunk={chunk} T={time} B2 H3 D{dim}")
    _lib.profile_reset()
    _lib.profile_enable(True)
    try:
        got = run_gpu(data, chunk=chunk, initial=(s0, c0), cotangents=(d_out, d_var, d_s, d_c))
    finally:
        _lib.profile_enable(False)
    ran = {k: _lib.profile_read(k)[1] for k in ("fwd_states", "bwd_states", "fwd_scan", "bwd_scan")}
    _lib.profile_reset()
    fused = state_walk == "fused"
    assert ran == {"fwd_states": int(fused), "bwd_states": int(fused),
                   "fwd_scan": int(not fused), "bwd_scan": int(not fused)}, ran
    args = [data[n].astype(np.float64) for n in NAMES]
    (out, var, s_end, c_end), res = oracle.forward(*args, chunk=chunk, initial=(s0, c0))
    for key, ref in zip(["output", "variance", "evidence", "cross"], (out, var, s_end, c_end)):
        assert normwise(got[key], ref) <= 1e-5, key
    want = oracle.backward(res, d_out, d_var, d_s, d_c)
    for n in NAMES:
        assert normwise(got["d_" + n], want[n]) <= 1e-4, n
    assert normwise(got["d_initial_evidence"], want["initial_evidence"]) <= 1e-4
    assert normwise(got["d_initial_cross"], want["initial_cross"]) <= 1e-4


def test_state_walk_choice_at_full_batch(gpu_lib, monkeypatch):
    """At B*H*(1 + P/64) >= compute units the fused walk is the default, and
    both walks agree on every output and gradient (summation order only)."""
    from mamba4_amd import _lib

    batch, heads, time = 32, 8, 70
    data = arrays(time=time, heads=heads, dim=64, value_dim=64, seed=5, batch=batch)
    data["floor"] = np.full_like(data["floor"], 0.05)
    rng = np.random.default_rng(6)
    cot = (rng.normal(size=data["values"].shape).astype(np.float32),
           rng.normal(size=data["beta"].shape).astype(np.float32),
           np.zeros((batch, heads, 64, 64), np.float32),
           np.zeros((batch, heads, 64, 64), np.float32))
    results = {}
    for mode in ["auto", "split"]:
        if mode == "auto":
            monkeypatch.delenv("M4MR_STATE_WALK", raising=False)
        else:
            monkeypatch.setenv("M4MR_STATE_WALK", mode)
        announce(f"state walk {mode} B{batch} H{heads} T{time}")
        _lib.profile_reset()
        _lib.profile_enable(True)
        try:
            results[mode] = run_gpu(data, chunk=64, cotangents=cot)
        finally:
            _lib.profile_enable(False)
        results[mode + "_fused"] = _lib.profile_read("fwd_states")[1]
        _lib.profile_reset()
    assert results["auto_fused"] == 1 and results["split_fused"] == 0
    # Rounding differences of the two summation orders, amplified by the
    # solves in the gradients (floor 0.05).
    for key, ref in results["split"].items():
        assert normwise(results["auto"][key], ref) <= (1e-4 if key.startswith("d_") else 1e-5), key
    # The final state against a float64 recurrence of the same inputs.
    k, v = data["keys"].astype(np.float64), data["values"].astype(np.float64)
    lam = np.exp(data["log_decay"].astype(np.float64))
    b = data["beta"].astype(np.float64)
    s = np.zeros((batch, heads, 64, 64))
    c = np.zeros((batch, heads, 64, 64))
    for t in range(time):
        kt = k[:, t]
        s = lam[:, t, :, None, None] * s + b[:, t, :, None, None] * kt[..., :, None] * kt[..., None, :]
        c = lam[:, t, :, None, None] * c + b[:, t, :, None, None] * v[:, t][..., :, None] * kt[..., None, :]
    assert normwise(results["auto"]["evidence"], s) <= 1e-5
    assert normwise(results["auto"]["cross"], c) <= 1e-5


@pytest.mark.parametrize("value_dim,chunk,batch,heads", [(64, 64, 2, 3), (128, 48, 2, 2),
                                                         (64, 64, 32, 8)])
def test_bf16_inputs_match_the_upcast_path_bit_for_bit(gpu_lib, value_dim, chunk, batch, heads):
    """bfloat16 keys, values and queries go to m4mr_forward_bf16 /
    m4mr_backward_bf16, which widen them in the kernels; the reference
    upcasts them first (lm/kernels/mamba4.py:263-265).  Widening is exact,
    so outputs, states and every gradient equal the float32 path on the
    upcast arrays bit for bit (both state walks: B*H = 6, 4 and 256)."""
    from mamba4_amd import SelectiveState, _lib, selective_gaussian_memory

    data = arrays(time=90, heads=heads, dim=64, value_dim=value_dim, seed=value_dim + batch,
                  batch=batch)
    data["floor"] = np.full_like(data["floor"], 0.05)
    rng = np.random.default_rng(7)
    root = rng.normal(size=(batch, heads, 64, 64)) / 64
    s0 = (root @ np.swapaxes(root, -1, -2)).astype(np.float32)
    c0 = (rng.normal(size=(batch, heads, value_dim, 64)) * 0.3).astype(np.float32)
    d_out = torch.tensor(rng.normal(size=data["values"].shape), dtype=torch.float32,
                         device="cuda:0")
    d_var = torch.tensor(rng.normal(size=data["beta"].shape), dtype=torch.float32,
                         device="cuda:0")
    announce(f"bf16 inputs P={value_dim} chunk={chunk} B{batch} H{heads} T90")
    results = []
    for dtype in (torch.bfloat16, torch.float32):
        qkv = [torch.tensor(data[n], device="cuda:0").to(torch.bfloat16).to(dtype)
               .requires_grad_(True) for n in ("keys", "values", "queries")]
        rest = [torch.tensor(data[n], device="cuda:0").requires_grad_(True)
                for n in ("beta", "log_decay", "floor")]
        init = [torch.tensor(a, device="cuda:0").requires_grad_(True) for a in (s0, c0)]
        _lib.profile_reset()
        _lib.profile_enable(True)
        try:
            r = selective_gaussian_memory(qkv[0], qkv[1], qkv[2], *rest, chunk_size=chunk,
                                          initial=SelectiveState(*init))
            ((r.output * d_out).sum() + (r.variance * d_var).sum()
             + r.state.evidence.sum() + r.state.cross.sum()).backward()
        finally:
            _lib.profile_enable(False)
        _lib.profile_reset()
        torch.cuda.synchronize()
        grads = [t.grad.float() for t in qkv + rest + init]
        results.append([r.output, r.variance, r.state.evidence, r.state.cross] + grads)
    # The bfloat16 inputs' gradients reach them rounded to bfloat16 (autograd
    # casts a gradient to its input's dtype); everything else is float32.
    for i, (got, want) in enumerate(zip(*results)):
        if 4 <= i < 7:
            want = want.to(torch.bfloat16).float()
        assert torch.equal(got, want), i
