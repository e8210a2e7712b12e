"""mixer_read: the mixer prologue, the memory read and the read gating fused
into one pass (lm/models/mamba4.py:183-273 without the projections and the
order head).

The fused op is checked against the composed float64 oracle (oracle.mixer
around oracle.memread: outputs normwise <= 1e-4, gradients <= 1e-3, the
north-star tolerances) and against the separate kernels (memory_inputs ->
selective_gaussian_memory -> gated_read) on the same state walk: the read
kernel and the state walk normalise each key and query row with the
prologue kernel's own arithmetic, the factor kernel sums a row's squares in
another order, so the two paths agree to float32 rounding (1e-5).  The fused op's
gradients (m4mr_mixer_read_backward: the gating's VJP inside the first
backward kernel, the prologue's inside the last, the state walk weighted by
the read gate) agree with the separate kernels' VJPs to 1e-4, with every
cotangent set (output, variance, final state, shifted key) and with the
optional ones left out.
"""

import numpy as np
import pytest

from test_mixer import BETA_MAX, FLOOR_MIN, GRAD_OF, PROLOGUE_ARGS, raw_inputs

MIXER_ARGS = ["key", "value", "query", "beta_raw", "dt_raw", "beta_bias", "dt_bias", "a_log",
              "floor_raw", "confidence_scale", "skip"]


def _gpu(x, names, grad=False):
    import torch

    return {n: torch.tensor(np.asarray(x[n], np.float32), device="cuda:0", requires_grad=grad)
            for n in names}


def _host(t):
    return t.detach().cpu().numpy().astype(np.float64)


def _fused(t, **kw):
    from mamba4_amd import mixer_read

    return mixer_read(*(t[n] for n in MIXER_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN, **kw)


def _separate(t, chunk_size=64, key_shift=True, previous=None, initial=None):
    from mamba4_amd import gated_read, memory_inputs, selective_gaussian_memory

    inputs = memory_inputs(*(t[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX,
                           floor_min=FLOOR_MIN, key_shift=key_shift, previous=previous)
    result = selective_gaussian_memory(inputs.keys, t["value"], inputs.queries, inputs.beta,
                                       inputs.log_decay, inputs.floor, chunk_size=chunk_size,
                                       initial=initial)
    out = gated_read(result.output, result.variance, t["value"], t["confidence_scale"],
                     t["skip"])
    return out, result.variance, result.state, inputs.shifted


def test_mixer_read_rejects_host_tensors_and_bad_shapes():
    import torch

    from mamba4_amd import mixer_read

    x = raw_inputs(batch=1, time=4, heads=2, dim=64, value_dim=64)
    t = {n: torch.tensor(np.asarray(x[n], np.float32)) for n in MIXER_ARGS}
    with pytest.raises(ValueError):
        mixer_read(*(t[n] for n in MIXER_ARGS))


@pytest.mark.gpu
@pytest.mark.parametrize("value_dim,with_previous", [(64, False), (128, True)])
def test_mixer_read_matches_oracle(gpu_lib, value_dim, with_previous):
    from gpu_helpers import announce, normwise
    from oracle import memread
    from oracle import mixer as oracle

    announce(f"mixer_read vs oracle value_dim={value_dim} previous={with_previous}")
    x = raw_inputs(batch=2, time=80, heads=2, dim=64, value_dim=value_dim, seed=21)
    t = _gpu(x, MIXER_ARGS + ["previous"], grad=True)
    prev = t["previous"] if with_previous else None
    res = _fused(t, previous=prev)
    d_out = np.random.default_rng(22).normal(size=res.output.shape)
    (res.output * _gpu({"d": d_out}, ["d"])["d"]).sum().backward()

    xp = x["previous"] if with_previous else None
    keys, queries, beta, log_decay, floor, shifted = oracle.prologue(
        *(x[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN, previous=xp)
    (read, variance, _, _), saved = memread.forward(keys, x["value"], queries, beta, log_decay,
                                                    floor, chunk=64)
    expected = oracle.epilogue(read, variance, x["value"], x["confidence_scale"], x["skip"])
    assert normwise(_host(res.output), expected) <= 1e-4
    assert normwise(_host(res.variance), variance) <= 1e-4
    np.testing.assert_array_equal(_host(res.shifted), shifted.astype(np.float32))
    ge = oracle.epilogue_backward(read, variance, x["value"], x["confidence_scale"], x["skip"],
                                  d_out)
    gm = memread.backward(saved, ge["d_read"], ge["d_variance"])
    gp = oracle.prologue_backward(*(x[n] for n in PROLOGUE_ARGS), gm["keys"], gm["queries"],
                                  gm["beta"], gm["log_decay"], gm["floor"], None,
                                  beta_max=BETA_MAX, previous=xp)
    expected_grads = {GRAD_OF[n][2:]: gp[GRAD_OF[n]] for n in PROLOGUE_ARGS}
    expected_grads["value"] = gm["values"] + ge["d_value"]
    expected_grads["confidence_scale"] = ge["d_confidence_scale"]
    expected_grads["skip"] = ge["d_skip"]
    for n in MIXER_ARGS:
        err = normwise(_host(t[n].grad), expected_grads[n])
        assert err <= 1e-3, (n, err)
    if with_previous:
        assert normwise(_host(t["previous"].grad), gp["d_previous"]) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize(
    "batch,time,heads,value_dim,chunk,key_shift,with_previous,with_initial",
    [(2, 80, 3, 64, 64, True, False, False), (2, 80, 3, 64, 16, True, True, True),
     (3, 37, 2, 128, 64, False, False, True), (1, 1, 4, 64, 64, True, True, False)],
)
def test_mixer_read_matches_separate_path(gpu_lib, monkeypatch, batch, time, heads, value_dim,
                                          chunk, key_shift, with_previous, with_initial):
    import torch

    from gpu_helpers import announce, normwise
    from mamba4_amd import SelectiveState

    # The fused op always takes the fused state walk; so does the separate path
    # here (with one LDS step buffer in the cases with an initial state).
    monkeypatch.setenv("M4MR_STATE_WALK", "fused")
    monkeypatch.setenv("M4MR_STATE_BUFFERS", "1" if with_initial else "2")
    announce(f"mixer_read vs separate B{batch} T{time} H{heads} P{value_dim} chunk={chunk} "
             f"shift={key_shift} previous={with_previous} initial={with_initial}")
    x = raw_inputs(batch=batch, time=time, heads=heads, dim=64, value_dim=value_dim, seed=23)
    rng = np.random.default_rng(24)
    g = rng.normal(size=(batch, heads, 64, 64))
    x["init_s"] = np.einsum("bhij,bhkj->bhik", g, g) / 64
    x["init_c"] = rng.normal(size=(batch, heads, value_dim, 64))
    names = MIXER_ARGS + ["previous", "init_s", "init_c"]
    fused_t, sep_t = _gpu(x, names, grad=True), _gpu(x, names, grad=True)
    kw = dict(chunk_size=chunk, key_shift=key_shift)

    def extras(t):
        return (t["previous"] if with_previous else None,
                SelectiveState(t["init_s"], t["init_c"]) if with_initial else None)

    prev, init = extras(fused_t)
    res = _fused(fused_t, previous=prev, initial=init, **kw)
    prev, init = extras(sep_t)
    out, variance, state, shifted = _separate(sep_t, previous=prev, initial=init, **kw)
    assert normwise(_host(res.output), _host(out)) <= 1e-5
    assert normwise(_host(res.variance), _host(variance)) <= 1e-5
    assert normwise(_host(res.state.evidence), _host(state.evidence)) <= 1e-5
    assert normwise(_host(res.state.cross), _host(state.cross)) <= 1e-5
    if key_shift:
        torch.testing.assert_close(res.shifted, shifted, rtol=0, atol=0)
    else:
        assert res.shifted is None and shifted is None
    d_out = torch.tensor(rng.normal(size=out.shape), dtype=torch.float32, device="cuda:0")
    d_var = torch.tensor(rng.normal(size=variance.shape), dtype=torch.float32, device="cuda:0")
    d_s = torch.tensor(rng.normal(size=state.evidence.shape), dtype=torch.float32,
                       device="cuda:0")
    d_sh = torch.tensor(rng.normal(size=(batch, heads, 64)), dtype=torch.float32,
                        device="cuda:0")
    for t, (o, v, s, sh) in ((fused_t, (res.output, res.variance, res.state.evidence,
                                         res.shifted)),
                             (sep_t, (out, variance, state.evidence, shifted))):
        loss = (o * d_out).sum() + (v * d_var).sum() + (s * d_s).sum()
        if key_shift:
            loss = loss + (sh * d_sh).sum()
        loss.backward()
    for n in names:
        a, b = fused_t[n].grad, sep_t[n].grad
        if b is None:
            assert a is None, n
            continue
        assert normwise(_host(a), _host(b)) <= 1e-4, n


@pytest.mark.gpu
def test_mixer_read_backward_with_output_cotangent_only(gpu_lib, monkeypatch):
    """Only the output enters the loss: the variance, final-state and
    shifted-key cotangents reach the fused backward as NULL (zero)."""
    import torch

    from gpu_helpers import announce, normwise

    monkeypatch.setenv("M4MR_STATE_WALK", "fused")
    announce("mixer_read backward, output cotangent only, B2 T150 H3 P128")
    x = raw_inputs(batch=2, time=150, heads=3, dim=64, value_dim=128, seed=27)
    fused_t, sep_t = _gpu(x, MIXER_ARGS + ["previous"], grad=True), _gpu(
        x, MIXER_ARGS + ["previous"], grad=True)
    res = _fused(fused_t, previous=fused_t["previous"])
    out, _, _, _ = _separate(sep_t, previous=sep_t["previous"])
    d_out = torch.tensor(np.random.default_rng(28).normal(size=out.shape), dtype=torch.float32,
                         device="cuda:0")
    (res.output * d_out).sum().backward()
    (out * d_out).sum().backward()
    for n in MIXER_ARGS + ["previous"]:
        assert normwise(_host(fused_t[n].grad), _host(sep_t[n].grad)) <= 1e-4, n


@pytest.mark.gpu
def test_mixer_read_cache_continuation(gpu_lib):
    """Two calls, the second from the first's state and shifted key, equal
    one call over the whole sequence (the cached decode path's contract)."""
    from gpu_helpers import announce, normwise

    announce("mixer_read cache continuation")
    x = raw_inputs(batch=2, time=96, heads=2, dim=64, value_dim=64, seed=25)
    t = _gpu(x, MIXER_ARGS)
    full = _fused(t)
    cut = 40
    head = {n: (v[:, :cut] if v.dim() >= 3 else v) for n, v in t.items()}
    tail = {n: (v[:, cut:] if v.dim() >= 3 else v) for n, v in t.items()}
    first = _fused({n: v.contiguous() for n, v in head.items()})
    second = _fused({n: v.contiguous() for n, v in tail.items()}, previous=first.shifted,
                    initial=first.state)
    import torch

    assert normwise(_host(torch.cat([first.output, second.output], 1)), _host(full.output)) <= 1e-5
    assert normwise(_host(second.state.evidence), _host(full.state.evidence)) <= 1e-5
    torch.testing.assert_close(second.shifted, full.shifted, rtol=0, atol=0)


@pytest.mark.gpu
def test_mixer_read_full_size(gpu_lib, monkeypatch):
    """The config-2 shape (B16 T1024 H8, D=P=64): the fused forward and
    backward against the separate kernels, and a batch row against the
    oracle."""
    import torch

    from gpu_helpers import announce, normwise
    from oracle import memread
    from oracle import mixer as oracle

    monkeypatch.setenv("M4MR_STATE_WALK", "fused")
    announce("mixer_read full size B16 T1024 H8")
    x = raw_inputs(batch=16, time=1024, heads=8, dim=64, value_dim=64, seed=26)
    t, ts = _gpu(x, MIXER_ARGS, grad=True), _gpu(x, MIXER_ARGS, grad=True)
    res = _fused(t)
    out, variance, _, _ = _separate(ts)
    assert normwise(_host(res.output), _host(out)) <= 1e-5
    assert normwise(_host(res.variance), _host(variance)) <= 1e-5
    rng = np.random.default_rng(29)
    d_out = torch.tensor(rng.normal(size=out.shape), dtype=torch.float32, device="cuda:0")
    d_var = torch.tensor(rng.normal(size=variance.shape), dtype=torch.float32, device="cuda:0")
    ((res.output * d_out).sum() + (res.variance * d_var).sum()).backward()
    ((out * d_out).sum() + (variance * d_var).sum()).backward()
    for n in MIXER_ARGS:
        assert normwise(_host(t[n].grad), _host(ts[n].grad)) <= 1e-4, n
    row = {n: (x[n][3:4] if np.ndim(x[n]) >= 3 else x[n]) for n in x}
    keys, queries, beta, log_decay, floor, _ = oracle.prologue(
        *(row[n] for n in PROLOGUE_ARGS), beta_max=BETA_MAX, floor_min=FLOOR_MIN)
    (read, var, _, _), _ = memread.forward(keys, row["value"], queries, beta, log_decay, floor,
                                           chunk=64)
    expected = oracle.epilogue(read, var, row["value"], row["confidence_scale"], row["skip"])
    assert normwise(_host(res.output[3:4]), expected) <= 1e-4
