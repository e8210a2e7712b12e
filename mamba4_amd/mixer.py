"""The memory read's caller preprocessing and read gating on MI355X.

``SelectiveMemoryMixer.__call__`` (lm/models/mamba4.py:126-337) turns its
projections into the memory read's inputs and gates the reads.  This module
runs those two steps on the gfx950 HIP library, differentiably:

* ``memory_inputs`` -- lm/models/mamba4.py:183-237: the key shift (each
  value is written under the previous position's key; position 0 takes the
  cached key or zero), unit normalisation of keys and queries
  (``_unit``, :37-39), ``beta = beta_max * sigmoid(beta_raw + beta_bias)``,
  ``log_decay = -exp(a_log) * softplus(dt_raw + dt_bias)`` and
  ``floor = floor_min + softplus(floor_raw)``.
* ``gated_read`` -- lm/models/mamba4.py:266-273: the confidence gate
  ``read * sigmoid(1 - confidence_scale * log1p(variance))`` and the skip
  ``+ D * value``.

Their outputs feed ``selective_gaussian_memory`` / ``selective_decode`` in
the same order as the reference's mixer.  Gradients reach every input and
parameter; the per-head parameter gradients are summed in a fixed order.
"""

from typing import NamedTuple, Optional

import torch

from mamba4_amd import _lib
from mamba4_amd.memory import _ptr, _require_device, _stream


class MemoryInputs(NamedTuple):
    keys: torch.Tensor
    queries: torch.Tensor
    beta: torch.Tensor
    log_decay: torch.Tensor
    floor: torch.Tensor
    shifted: Optional[torch.Tensor]  # the last raw key, the next call's `previous`


def _f32(t):
    return t.to(torch.float32).contiguous()


def _workspace(lib, batch, time, heads, device):
    nbytes = lib.m4mr_mixer_workspace_bytes(batch, time, heads)
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


class _Prologue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                previous, beta_max, floor_min, key_shift):
        lib = _lib.load()
        batch, time, heads, dim = key.shape
        keys, queries = torch.empty_like(key), torch.empty_like(query)
        beta, log_decay = torch.empty_like(beta_raw), torch.empty_like(dt_raw)
        floor = torch.empty_like(floor_raw)
        shifted = key.new_empty((batch, heads, dim)) if key_shift else None
        _lib.check(
            lib.m4mr_prologue_forward(
                _ptr(key), _ptr(query), _ptr(beta_raw), _ptr(dt_raw), _ptr(beta_bias),
                _ptr(dt_bias), _ptr(a_log), _ptr(floor_raw), _ptr(previous), batch, time,
                heads, dim, beta_max, floor_min, int(key_shift), _ptr(keys), _ptr(queries),
                _ptr(beta), _ptr(log_decay), _ptr(floor), _ptr(shifted), _stream(),
            )
        )
        ctx.save_for_backward(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log,
                              floor_raw, previous)
        ctx.beta_max, ctx.key_shift = beta_max, key_shift
        return keys, queries, beta, log_decay, floor, shifted

    @staticmethod
    def backward(ctx, d_keys, d_queries, d_beta, d_log_decay, d_floor, d_shifted):
        lib = _lib.load()
        key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, previous = (
            ctx.saved_tensors)
        batch, time, heads, dim = key.shape

        def dense(g, like):
            return torch.zeros_like(like) if g is None else _f32(g)

        d_keys, d_queries = dense(d_keys, key), dense(d_queries, query)
        d_beta, d_log_decay = dense(d_beta, beta_raw), dense(d_log_decay, dt_raw)
        d_floor = dense(d_floor, floor_raw)
        d_shifted = None if d_shifted is None else _f32(d_shifted)
        grads = [torch.empty_like(t) for t in (key, query, beta_raw, dt_raw, beta_bias,
                                               dt_bias, a_log, floor_raw)]
        d_previous = None if previous is None else torch.empty_like(previous)
        workspace, nbytes = _workspace(lib, batch, time, heads, key.device)
        _lib.check(
            lib.m4mr_prologue_backward(
                _ptr(key), _ptr(query), _ptr(beta_raw), _ptr(dt_raw), _ptr(beta_bias),
                _ptr(dt_bias), _ptr(a_log), _ptr(floor_raw), _ptr(previous), batch, time,
                heads, dim, ctx.beta_max, int(ctx.key_shift), _ptr(d_keys), _ptr(d_queries),
                _ptr(d_beta), _ptr(d_log_decay), _ptr(d_floor), _ptr(d_shifted),
                *(_ptr(g) for g in grads), _ptr(d_previous), _ptr(workspace), nbytes,
                _stream(),
            )
        )
        return (*grads, d_previous, None, None, None)


def memory_inputs(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, *,
                  beta_max=1.0, floor_min=0.25, key_shift=True, previous=None):
    """The memory read's inputs from the mixer's projections.

    key, query [B,T,H,D] (after the mixer's convolution and activation);
    beta_raw, dt_raw [B,T,H]; beta_bias, dt_bias, a_log [H]; floor_raw [H,D];
    previous [B,H,D], the cached raw key of the preceding call (None: a zero
    key at position 0).  Returns ``MemoryInputs(keys, queries, beta,
    log_decay, floor, shifted)``; ``shifted`` is the raw key of position T-1
    with ``key_shift`` (the next call's ``previous``), else None.
    """
    if beta_max <= 0:
        raise ValueError("memory_beta_max must be positive")
    if floor_min <= 0:
        raise ValueError("Selective floor must be positive and above its minimum")
    tensors = [key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, previous]
    _require_device(*tensors)
    key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw = (
        _f32(t) for t in tensors[:8])
    batch, time, heads, dim = key.shape
    if query.shape != key.shape or dim % 4:
        raise ValueError("memory_inputs needs key and query [B,T,H,D] with D a multiple of 4")
    if beta_raw.shape != (batch, time, heads) or dt_raw.shape != (batch, time, heads):
        raise ValueError("memory_inputs needs beta_raw and dt_raw [B,T,H]")
    if any(t.shape != (heads,) for t in (beta_bias, dt_bias, a_log)):
        raise ValueError("memory_inputs needs beta_bias, dt_bias and a_log [H]")
    if floor_raw.shape != (heads, dim):
        raise ValueError("memory_inputs needs floor_raw [H,D]")
    if previous is not None:
        previous = _f32(previous)
        if previous.shape != (batch, heads, dim):
            raise ValueError("memory_inputs needs previous [B,H,D]")
    out = _Prologue.apply(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                          previous, float(beta_max), float(floor_min), bool(key_shift))
    return MemoryInputs(*out)


class _Epilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, read, variance, value, confidence_scale, skip):
        lib = _lib.load()
        batch, time, heads, width = read.shape
        out = torch.empty_like(read)
        _lib.check(
            lib.m4mr_epilogue_forward(
                _ptr(read), _ptr(variance), _ptr(value), _ptr(confidence_scale), _ptr(skip),
                batch, time, heads, width, _ptr(out), _stream(),
            )
        )
        ctx.save_for_backward(read, variance, value, confidence_scale, skip)
        return out

    @staticmethod
    def backward(ctx, d_out):
        lib = _lib.load()
        read, variance, value, confidence_scale, skip = ctx.saved_tensors
        batch, time, heads, width = read.shape
        d_out = _f32(d_out)
        grads = [torch.empty_like(t) for t in (read, variance, value, confidence_scale, skip)]
        workspace, nbytes = _workspace(lib, batch, time, heads, read.device)
        _lib.check(
            lib.m4mr_epilogue_backward(
                _ptr(read), _ptr(variance), _ptr(value), _ptr(confidence_scale), _ptr(skip),
                batch, time, heads, width, _ptr(d_out), _ptr(grads[0]), _ptr(grads[1]),
                _ptr(grads[2]), _ptr(grads[3]), _ptr(grads[4]), _ptr(workspace), nbytes,
                _stream(),
            )
        )
        return tuple(grads)


def gated_read(read, variance, value, confidence_scale, skip):
    """read * sigmoid(1 - confidence_scale * log1p(variance)) + skip * value.

    read, value [B,T,H,P] (P a multiple of 4); variance [B,T,H];
    confidence_scale, skip [H] (the mixer's ``confidence_scale`` and ``D``).
    """
    tensors = [read, variance, value, confidence_scale, skip]
    _require_device(*tensors)
    read, variance, value, confidence_scale, skip = (_f32(t) for t in tensors)
    batch, time, heads, width = read.shape
    if value.shape != read.shape or width % 4:
        raise ValueError("gated_read needs read and value [B,T,H,P] with P a multiple of 4")
    if variance.shape != (batch, time, heads):
        raise ValueError("gated_read needs variance [B,T,H]")
    if confidence_scale.shape != (heads,) or skip.shape != (heads,):
        raise ValueError("gated_read needs confidence_scale and skip [H]")
    return _Epilogue.apply(read, variance, value, confidence_scale, skip)
