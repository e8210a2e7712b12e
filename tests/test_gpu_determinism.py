"""Determinism and reentrancy of the C ABI (the drop-in boundary's threading
contract: XLA may call a handler from several threads, on several streams).

* The same forward and backward at the config-2 shape, run twice, give the
  same bits in every output, residual and gradient: no kernel of the memory
  read uses atomics in its outputs, and the floor gradient is summed in a
  fixed order.
* Two host threads calling m4mr_forward / m4mr_backward at once, each on its
  own stream with its own inputs (one at P = 64, one at P = 128, so both
  kinds of launch configuration are looked up concurrently), give the same
  bits as the same calls made one after the other on one stream.  ctypes
  releases the GIL around each foreign call, so the calls overlap on the
  host and their kernels on the device.
"""

import threading

import pytest
import torch

from tests.gpu_helpers import NAMES, announce

pytestmark = pytest.mark.gpu


def _device_problem(batch, time, heads, width, seed):
    from mamba4_amd.inputs import synthetic_inputs

    data = synthetic_inputs(batch, time, heads, value_dim=width, seed=seed, cotangents=True)
    dev = torch.device("cuda:0")
    inputs = [torch.tensor(data[n], device=dev) for n in NAMES]
    cotangents = [torch.tensor(data["d_output"], device=dev),
                  torch.tensor(data["d_variance"], device=dev)]
    return inputs, cotangents


def _fwd_bwd(inputs, cotangents, chunk=64):
    """Forward with the factor store, then the backward, on the calling
    thread's current stream; every array the two entry points write."""
    from mamba4_amd import memory

    fwd = memory.memread_forward(*inputs, None, None, chunk)
    grads = memory.memread_backward(*inputs, *fwd[4:], chunk, *cotangents, None, None)
    return list(fwd) + list(grads)


def test_config2_forward_and_backward_are_bit_reproducible(gpu_lib):
    announce("determinism: config 2 (B16 T1024 H8 P64) fwd+bwd twice")
    inputs, cotangents = _device_problem(16, 1024, 8, 64, seed=0)
    first = _fwd_bwd(inputs, cotangents)
    torch.cuda.synchronize()
    second = _fwd_bwd(inputs, cotangents)
    torch.cuda.synchronize()
    assert len(first) == len(second) == 16
    for i, (a, b) in enumerate(zip(first, second)):
        assert torch.isfinite(a).all(), i
        assert torch.equal(a, b), i


def test_concurrent_calls_from_two_threads_on_two_streams(gpu_lib):
    cases = [(4, 512, 8, 64, 1), (2, 384, 6, 128, 2)]
    problems = [_device_problem(*case) for case in cases]
    announce("reentrancy: sequential reference runs")
    want = [_fwd_bwd(*p) for p in problems]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in cases]
    for rep in range(3):
        announce(f"reentrancy: two threads, two streams, repetition {rep}")
        got = [None, None]
        errors = []
        start = threading.Barrier(2)

        def run(i):
            try:
                with torch.cuda.stream(streams[i]):
                    start.wait()
                    got[i] = _fwd_bwd(*problems[i])
                    streams[i].synchronize()
            except BaseException as exc:  # reported on the main thread
                errors.append(exc)

        threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in threads), "a thread did not finish"
        assert not errors, errors
        torch.cuda.synchronize()
        for i in range(2):
            for j, (a, b) in enumerate(zip(got[i], want[i])):
                assert torch.equal(a, b), (rep, i, j)
