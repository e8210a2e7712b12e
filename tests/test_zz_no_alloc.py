"""The allocation-free backward, m4mr_backward_noalloc, through the C ABI.

It runs the kernels of m4mr_backward in the same order with its workspace
in the library's static device buffer instead of the caller's, so every
gradient must equal m4mr_backward's bit for bit.  Two calls in a row, the
second with a smaller input, so the second starts from the first call's
leftover buffer contents.
"""

import numpy as np
import pytest
import torch

from tests.gpu_helpers import NAMES, announce

pytestmark = pytest.mark.gpu


def _problem(batch, time, heads, width, chunk, seed):
    from mamba4_amd import memory
    from mamba4_amd.inputs import synthetic_inputs

    data = synthetic_inputs(batch, time, heads, value_dim=width, seed=seed, cotangents=True)
    dev = torch.device("cuda:0")
    inputs = [torch.tensor(data[n], device=dev) for n in NAMES]
    residuals = memory.memread_forward(*inputs, None, None, chunk)[4:]
    rng = np.random.default_rng(seed + 1)

    def normal(*shape):
        return torch.tensor(rng.normal(size=shape), dtype=torch.float32, device=dev)

    cotangents = [torch.tensor(data["d_output"], device=dev),
                  torch.tensor(data["d_variance"], device=dev),
                  normal(batch, heads, 64, 64), normal(batch, heads, width, 64)]
    return inputs, residuals, cotangents


def _noalloc(inputs, residuals, cotangents, chunk):
    from mamba4_amd import _lib

    batch, time, heads, _ = inputs[0].shape
    width = inputs[1].shape[-1]
    f32 = dict(dtype=torch.float32, device=inputs[0].device)
    grads = [torch.empty(t.shape, **f32) for t in inputs]
    grads += [torch.empty(batch, heads, 64, 64, **f32), torch.empty(batch, heads, width, 64, **f32)]
    _lib.check(_lib.load().m4mr_backward_noalloc(
        *(t.data_ptr() for t in inputs), batch, time, heads, width, chunk,
        *(t.data_ptr() for t in residuals), *(t.data_ptr() for t in cotangents),
        *(g.data_ptr() for g in grads), torch.cuda.current_stream().cuda_stream))
    return grads


@pytest.mark.parametrize("shapes", [((2, 300, 5, 128, 64), (1, 70, 3, 64, 16))])
def test_noalloc_backward_equals_backward_twice_in_a_row(gpu_lib, shapes):
    from mamba4_amd import memory

    for call, (batch, time, heads, width, chunk) in enumerate(shapes):
        announce(f"m4mr_backward_noalloc call {call}: B{batch} T{time} H{heads} P{width} "
                 f"chunk {chunk}")
        inputs, residuals, cotangents = _problem(batch, time, heads, width, chunk, seed=call)
        torch.cuda.synchronize()
        got = _noalloc(inputs, residuals, cotangents, chunk)
        want = memory.memread_backward(*inputs, *residuals, chunk, *cotangents)
        torch.cuda.synchronize()
        assert len(got) == len(want) == 8
        for i, (g, w) in enumerate(zip(got, want)):
            assert torch.isfinite(g).all(), i
            assert torch.equal(g, w), i


def test_noalloc_backward_takes_the_spill_free_state_walk(gpu_lib, monkeypatch):
    """More backward state walks than two per compute unit (B*H*(1+P/64) =
    528 > 2 x 256) make m4mr_backward take the one-buffer walk, held to 80
    VGPRs, where the compiler may spill to runtime-provided scratch;
    m4mr_backward_noalloc takes the two-buffer walk instead, whatever
    M4MR_STATE_BUFFERS asks, and must still equal m4mr_backward bit for bit
    (both walks give the same states)."""
    from mamba4_amd import memory

    batch, time, heads, width, chunk = 8, 64, 33, 64, 64
    for buffers in (None, "1"):
        if buffers is None:
            monkeypatch.delenv("M4MR_STATE_BUFFERS", raising=False)
        else:
            monkeypatch.setenv("M4MR_STATE_BUFFERS", buffers)
        announce(f"m4mr_backward_noalloc B{batch} T{time} H{heads} P{width} chunk {chunk}, "
                 f"M4MR_STATE_BUFFERS={buffers}")
        inputs, residuals, cotangents = _problem(batch, time, heads, width, chunk, seed=7)
        torch.cuda.synchronize()
        got = _noalloc(inputs, residuals, cotangents, chunk)
        want = memory.memread_backward(*inputs, *residuals, chunk, *cotangents)
        torch.cuda.synchronize()
        for i, (g, w) in enumerate(zip(got, want)):
            assert torch.isfinite(g).all(), i
            assert torch.equal(g, w), i


def test_noalloc_backward_allocates_nothing_and_replays_in_a_graph(gpu_lib):
    """After a warm-up call (the first call on a device resolves the static
    buffer's address and belongs outside any capture), a second call leaves
    the device's free memory unchanged, and the call captured in a HIP graph
    replays to m4mr_backward's bits three times, with eager work and
    synchronisations between the replays."""
    from mamba4_amd import _lib, memory

    batch, time, heads, width, chunk = 2, 200, 3, 64, 64
    announce(f"m4mr_backward_noalloc graph capture B{batch} T{time} H{heads} P{width}")
    inputs, residuals, cotangents = _problem(batch, time, heads, width, chunk, seed=11)
    want = memory.memread_backward(*inputs, *residuals, chunk, *cotangents)
    _noalloc(inputs, residuals, cotangents, chunk)  # warm-up
    torch.cuda.synchronize()
    f32 = dict(dtype=torch.float32, device=inputs[0].device)
    grads = [torch.empty(t.shape, **f32) for t in inputs]
    grads += [torch.empty(batch, heads, 64, 64, **f32), torch.empty(batch, heads, width, 64, **f32)]
    lib = _lib.load()

    def call():
        _lib.check(lib.m4mr_backward_noalloc(
            *(t.data_ptr() for t in inputs), batch, time, heads, width, chunk,
            *(t.data_ptr() for t in residuals), *(t.data_ptr() for t in cotangents),
            *(g.data_ptr() for g in grads), torch.cuda.current_stream().cuda_stream))

    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    call()
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after == free_before
    for g, w in zip(grads, want):
        assert torch.equal(g, w)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    torch.cuda.synchronize()
    for replay in range(3):
        for g in grads:
            g.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (g, w) in enumerate(zip(grads, want)):
            assert torch.equal(g, w), (replay, i)
    del graph
