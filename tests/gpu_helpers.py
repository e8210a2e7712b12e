"""Shared helpers for the GPU parity tests (imported by tests only)."""

import sys

import numpy as np
import torch

NAMES = ["keys", "values", "queries", "beta", "log_decay", "floor"]


def announce(msg):
    """Name the case before a GPU step, so a box-level failure is traceable."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def to_device(arrays, grad=False):
    dev = torch.device("cuda:0")
    return [torch.tensor(np.asarray(a, np.float32), device=dev, requires_grad=grad) for a in arrays]


def normwise(actual, expected):
    """max |actual - expected| / max |expected| (the tolerance measure)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    scale = max(float(np.max(np.abs(expected))), 1e-30)
    return float(np.max(np.abs(actual - expected))) / scale


def host(t):
    return t.detach().cpu().numpy().astype(np.float64)


def run_gpu(data, chunk=64, initial=None, cotangents=None, names=NAMES):
    """Forward (and backward when cotangents are given) through the public API."""
    from mamba4_amd import SelectiveState, selective_gaussian_memory

    grad = cotangents is not None
    tensors = to_device([data[n] for n in names], grad=grad)
    init = None
    init_tensors = []
    if initial is not None:
        init_tensors = to_device(initial, grad=grad)
        init = SelectiveState(*init_tensors)
    result = selective_gaussian_memory(*tensors, chunk_size=chunk, initial=init)
    out = {
        "output": host(result.output),
        "variance": host(result.variance),
        "evidence": host(result.state.evidence),
        "cross": host(result.state.cross),
    }
    if grad:
        d_out, d_var, d_s, d_c = to_device(cotangents)
        loss = (result.output * d_out).sum() + (result.variance * d_var).sum()
        loss = loss + (result.state.evidence * d_s).sum() + (result.state.cross * d_c).sum()
        loss.backward()
        for n, t in zip(names, tensors):
            out["d_" + n] = host(t.grad)
        if initial is not None:
            out["d_initial_evidence"] = host(init_tensors[0].grad)
            out["d_initial_cross"] = host(init_tensors[1].grad)
    torch.cuda.synchronize()
    return out


def run_quad(m, q):
    """First quad of the run of column quad q of row slot m in a stored factor."""
    base = 32 * m * m + 8 * m
    if q <= 4 * m:
        return base + 16 * q
    return base + 16 * (4 * m + 1) + {1: -4, 2: 4, 3: 8}[q - 4 * m]


def factor_index():
    """[64, 64] float offsets of L_ij (j <= i) in a stored factor, -1 above."""
    index = np.full((64, 64), -1)
    for i in range(64):
        a, m = i % 16, i // 16
        for j in range(i + 1):
            index[i, j] = 4 * (run_quad(m, j // 4) + a) + j % 4
    return index


FACTOR_INDEX = factor_index()
LOWER = FACTOR_INDEX >= 0


def unpack_factors(packed):
    lower = np.zeros(packed.shape[:-1] + (64, 64))
    lower[..., LOWER] = packed[..., FACTOR_INDEX[LOWER]]
    return lower


def pack_factors(lower):
    packed = np.zeros(lower.shape[:-2] + (2176,))
    packed[..., FACTOR_INDEX[LOWER]] = lower[..., LOWER]
    return packed
