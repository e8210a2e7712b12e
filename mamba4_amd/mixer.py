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
* ``mixer_read`` -- both fused with the memory read itself
  (lm/models/mamba4.py:183-273 without the projections and the order head):
  the memory-read kernels take the raw projections, transforming them as
  they load them, and the read kernel gates its output.

Their outputs feed ``selective_gaussian_memory`` / ``selective_decode`` in
the same order as the reference's mixer.  Gradients reach every input and
parameter; the per-head parameter gradients are summed in a fixed order.
"""

import ctypes
from typing import NamedTuple, Optional

import torch

from mamba4_amd import _lib
from mamba4_amd.memory import SelectiveState, _ptr, _require_device, _stream, memread_backward


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


def _prologue_forward(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                      previous, beta_max, floor_min, key_shift):
    """m4mr_prologue_forward: (keys, queries, beta, log_decay, floor, shifted)."""
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
    return keys, queries, beta, log_decay, floor, shifted


def _prologue_backward(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                       previous, beta_max, key_shift, d_keys, d_queries, d_beta, d_log_decay,
                       d_floor, d_shifted):
    """m4mr_prologue_backward: gradients of key, query, beta_raw, dt_raw,
    beta_bias, dt_bias, a_log, floor_raw and previous (None without one)."""
    lib = _lib.load()
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
            heads, dim, beta_max, int(key_shift), _ptr(d_keys), _ptr(d_queries),
            _ptr(d_beta), _ptr(d_log_decay), _ptr(d_floor), _ptr(d_shifted),
            *(_ptr(g) for g in grads), _ptr(d_previous), _ptr(workspace), nbytes,
            _stream(),
        )
    )
    return (*grads, d_previous)


class _Prologue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                previous, beta_max, floor_min, key_shift):
        out = _prologue_forward(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log,
                                floor_raw, previous, beta_max, floor_min, key_shift)
        ctx.save_for_backward(key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log,
                              floor_raw, previous)
        ctx.beta_max, ctx.key_shift = beta_max, key_shift
        return out

    @staticmethod
    def backward(ctx, d_keys, d_queries, d_beta, d_log_decay, d_floor, d_shifted):
        grads = _prologue_backward(*ctx.saved_tensors, ctx.beta_max, ctx.key_shift, d_keys,
                                   d_queries, d_beta, d_log_decay, d_floor, d_shifted)
        return (*grads, None, None, None)


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
        return _epilogue_backward(*ctx.saved_tensors, d_out)


def _epilogue_backward(read, variance, value, confidence_scale, skip, d_out):
    """m4mr_epilogue_backward: gradients of read, variance, value,
    confidence_scale and skip."""
    lib = _lib.load()
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


class MixerRead(NamedTuple):
    output: torch.Tensor             # gated read [B,T,H,P]
    variance: torch.Tensor           # [B,T,H]
    state: SelectiveState            # final evidence [B,H,D,D] and cross [B,H,P,D]
    shifted: Optional[torch.Tensor]  # raw key of position T-1 with key_shift, else None


class _MixerRead(torch.autograd.Function):
    """m4mr_mixer_forward, and its VJP in one launch sequence
    (m4mr_mixer_read_backward): the gating's VJP folded into the first
    backward kernel, the prologue's into the last."""

    @staticmethod
    def forward(ctx, key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                previous, confidence_scale, skip, init_s, init_c, beta_max, floor_min,
                key_shift, chunk, store_factors):
        lib = _lib.load()
        batch, time, heads, dim = key.shape
        width = value.shape[-1]
        count, starts = _lib.start_counts(time, chunk)
        f32 = dict(dtype=torch.float32, device=key.device)
        output = torch.empty((batch, time, heads, width), **f32)
        read = torch.empty_like(output)
        variance = torch.empty((batch, time, heads), **f32)
        beta, log_decay = torch.empty_like(variance), torch.empty_like(variance)
        floor = torch.empty((heads, dim), **f32)
        final_s = torch.empty((batch, heads, dim, dim), **f32)
        final_c = torch.empty((batch, heads, width, dim), **f32)
        solved = torch.empty((batch, time, heads, dim), **f32)
        # Without a gradient to take, the factors are not stored (the
        # reference's store_factors=False mode, lm/kernels/mamba4_fused.py:183-232).
        factors = (torch.empty((batch, time, heads, _lib.FACTOR_FLOATS), **f32)
                   if store_factors else None)
        start_s = torch.empty((batch, heads, starts, dim, dim), **f32)
        start_c = torch.empty((batch, heads, count, width, dim), **f32)
        shifted = torch.empty((batch, heads, dim), **f32) if key_shift else None
        params = _lib.MixerParams(
            _ptr(beta_bias), _ptr(dt_bias), _ptr(a_log), _ptr(floor_raw), _ptr(previous),
            _ptr(confidence_scale), _ptr(skip), beta_max, floor_min, int(key_shift),
        )
        _lib.check(
            lib.m4mr_mixer_forward(
                _ptr(key), _ptr(value), _ptr(query), _ptr(beta_raw), _ptr(dt_raw),
                ctypes.byref(params), _ptr(init_s), _ptr(init_c), batch, time, heads, width,
                chunk, _ptr(output), _ptr(read), _ptr(variance), _ptr(beta), _ptr(log_decay),
                _ptr(floor), _ptr(final_s), _ptr(final_c),
                _ptr(solved), _ptr(factors), _ptr(start_s), _ptr(start_c), _ptr(shifted),
                _stream(),
            )
        )
        ctx.save_for_backward(key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log,
                              floor_raw, previous, confidence_scale, skip, read, variance,
                              beta, log_decay, floor, solved, factors, start_s, start_c)
        ctx.beta_max, ctx.floor_min, ctx.key_shift, ctx.chunk = (beta_max, floor_min,
                                                                 key_shift, chunk)
        ctx.has_initial = init_s is not None
        return output, variance, final_s, final_c, shifted

    @staticmethod
    def backward(ctx, d_output, d_variance, d_final_s, d_final_c, d_shifted):
        (key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, previous,
         confidence_scale, skip, read, variance, beta, log_decay, floor, solved, factors,
         start_s, start_c) = ctx.saved_tensors
        lib = _lib.load()
        batch, time, heads, dim = key.shape
        width = value.shape[-1]
        if d_output is None:
            d_output = torch.zeros_like(read)
        grads = [torch.empty_like(t) for t in (key, value, query, beta_raw, dt_raw, beta_bias,
                                               dt_bias, a_log, floor_raw)]
        d_previous = None if previous is None else torch.empty_like(previous)
        d_scale, d_skip = torch.empty_like(confidence_scale), torch.empty_like(skip)
        f32 = dict(dtype=torch.float32, device=key.device)
        d_init_s = torch.empty((batch, heads, dim, dim), **f32)
        d_init_c = torch.empty((batch, heads, width, dim), **f32)
        nbytes = lib.m4mr_mixer_read_backward_workspace_bytes(batch, time, heads, width,
                                                              ctx.chunk)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=key.device)
        params = _lib.MixerParams(
            _ptr(beta_bias), _ptr(dt_bias), _ptr(a_log), _ptr(floor_raw), _ptr(previous),
            _ptr(confidence_scale), _ptr(skip), ctx.beta_max, ctx.floor_min, int(ctx.key_shift),
        )
        cot = [None if t is None else _f32(t)
               for t in (d_output, d_variance, d_final_s, d_final_c, d_shifted)]
        d_key, d_value, d_query, d_beta_raw, d_dt_raw, d_beta_bias, d_dt_bias, d_a_log, \
            d_floor_raw = grads
        _lib.check(
            lib.m4mr_mixer_read_backward(
                _ptr(key), _ptr(value), _ptr(query), _ptr(dt_raw), ctypes.byref(params), batch,
                time, heads, width, ctx.chunk, _ptr(read), _ptr(variance), _ptr(beta),
                _ptr(log_decay), _ptr(floor), _ptr(solved), _ptr(factors), _ptr(start_s),
                _ptr(start_c), *(_ptr(t) for t in cot), _ptr(d_key), _ptr(d_value),
                _ptr(d_query), _ptr(d_beta_raw), _ptr(d_dt_raw), _ptr(d_beta_bias),
                _ptr(d_dt_bias), _ptr(d_a_log), _ptr(d_floor_raw), _ptr(d_previous),
                _ptr(d_scale), _ptr(d_skip), _ptr(d_init_s), _ptr(d_init_c), _ptr(workspace),
                nbytes, _stream(),
            )
        )
        d_init = (d_init_s, d_init_c) if ctx.has_initial else (None, None)
        return (d_key, d_value, d_query, d_beta_raw, d_dt_raw, d_beta_bias, d_dt_bias, d_a_log,
                d_floor_raw, d_previous, d_scale, d_skip, *d_init,
                None, None, None, None, None)


def mixer_read_separate_backward(ctx_tensors, beta_max, key_shift, chunk, d_output, d_variance,
                                 d_final_s, d_final_c, d_shifted):
    """The same VJP as three separate steps: m4mr_epilogue_backward,
    m4mr_mixer_backward, m4mr_prologue_backward (and an add for the value's
    two paths).  ``ctx_tensors`` are _MixerRead's saved tensors.  Returns
    the gradients of key, value, query, beta_raw, dt_raw, beta_bias, dt_bias,
    a_log, floor_raw, previous, confidence_scale, skip, init_s and init_c."""
    (key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, previous,
     confidence_scale, skip, read, variance, beta, log_decay, floor, solved, factors,
     start_s, start_c) = ctx_tensors
    d_read, d_var, d_skip_value, d_scale, d_skip = _epilogue_backward(
        read, variance, value, confidence_scale, skip, d_output)
    if d_variance is not None:
        d_var = d_var + _f32(d_variance)
    (d_keys, d_values, d_queries, d_beta, d_log_decay, d_floor, d_init_s,
     d_init_c) = memread_backward(key, value, query, beta, log_decay, floor, solved,
                                  factors, start_s, start_c, chunk, d_read, d_var,
                                  d_final_s, d_final_c, mixer=(previous, key_shift))
    (d_key, d_query, d_beta_raw, d_dt_raw, d_beta_bias, d_dt_bias, d_a_log, d_floor_raw,
     d_previous) = _prologue_backward(
        key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw, previous,
        beta_max, key_shift, d_keys, d_queries, d_beta, d_log_decay, d_floor, d_shifted)
    return (d_key, d_values + d_skip_value, d_query, d_beta_raw, d_dt_raw, d_beta_bias,
            d_dt_bias, d_a_log, d_floor_raw, d_previous, d_scale, d_skip, d_init_s, d_init_c)


def mixer_read(key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
               confidence_scale, skip, *, beta_max=1.0, floor_min=0.25, key_shift=True,
               previous=None, chunk_size=64, initial=None):
    """The mixer's memory read from its raw projections, in one fused pass.

    Equal to ``memory_inputs`` (key shift, unit normalisation, gates), then
    ``selective_gaussian_memory``, then ``gated_read``
    (lm/models/mamba4.py:183-273 without the projections and the order
    head), without their separate passes over keys, queries and values.
    key, query [B,T,H,64]; value [B,T,H,P] with P = 64 or 128; beta_raw,
    dt_raw [B,T,H]; beta_bias, dt_bias, a_log, confidence_scale, skip [H];
    floor_raw [H,64]; previous [B,H,64] (None: a zero key at position 0);
    ``initial`` a SelectiveState.  Returns ``MixerRead(output, variance,
    state, shifted)``; gradients reach every tensor argument.
    """
    if beta_max <= 0:
        raise ValueError("memory_beta_max must be positive")
    if floor_min <= 0:
        raise ValueError("Selective floor must be positive and above its minimum")
    if chunk_size < 1:
        raise ValueError("chunk_size must be positive")
    tensors = [key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
               confidence_scale, skip, previous]
    _require_device(*tensors)
    (key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
     confidence_scale, skip) = (_f32(t) for t in tensors[:11])
    batch, time, heads, dim = key.shape
    width = value.shape[-1]
    if dim != _lib.KEY_DIM or query.shape != key.shape:
        raise ValueError(f"mixer_read needs key and query [B,T,H,{_lib.KEY_DIM}]")
    if value.shape[:3] != key.shape[:3] or width not in (_lib.VALUE_DIM, _lib.MAX_VALUE_DIM):
        raise ValueError("mixer_read needs value [B,T,H,P] with P = 64 or 128")
    if beta_raw.shape != (batch, time, heads) or dt_raw.shape != (batch, time, heads):
        raise ValueError("mixer_read needs beta_raw and dt_raw [B,T,H]")
    if any(t.shape != (heads,) for t in (beta_bias, dt_bias, a_log, confidence_scale, skip)):
        raise ValueError("mixer_read needs beta_bias, dt_bias, a_log, confidence_scale and "
                         "skip [H]")
    if floor_raw.shape != (heads, dim):
        raise ValueError("mixer_read needs floor_raw [H,64]")
    if previous is not None:
        previous = _f32(previous)
        if previous.shape != (batch, heads, dim):
            raise ValueError("mixer_read needs previous [B,H,64]")
    init_s = init_c = None
    if initial is not None:
        init_s, init_c = _f32(initial.evidence), _f32(initial.cross)
        _require_device(init_s, init_c)
        if init_s.shape != (batch, heads, dim, dim) or init_c.shape != (batch, heads, width, dim):
            raise ValueError("mixer_read needs an initial state [B,H,64,64], [B,H,P,64]")
    chunk = min(int(chunk_size), _lib.MAX_CHUNK)
    differentiable = [key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                      previous, confidence_scale, skip, init_s, init_c]
    store = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in differentiable)
    with torch.cuda.device(key.device):
        output, variance, final_s, final_c, shifted = _MixerRead.apply(
            key, value, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
            previous, confidence_scale, skip, init_s, init_c, float(beta_max),
            float(floor_min), bool(key_shift), chunk, store)
    return MixerRead(output, variance, SelectiveState(final_s, final_c), shifted)
