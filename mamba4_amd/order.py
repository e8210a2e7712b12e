"""The order head's gated vector scan on MI355X.

Mirrors ``order_memory_chunked(values, log_decay, chunk_size=64)`` and
``order_memory(values, decay)`` (lm/models/mamba4.py:46-95): per batch row,
head and channel, ``h_t = lam_t h_(t-1) + (1 - lam_t) v_t`` from zero, with
``lam = exp(log_decay)`` and the inflow ``-expm1(log_decay)``.  The mixer's
order head (lm/models/mamba4.py:274-289) calls it on the values and
``log_sigmoid(order_logits)``; its cached decode step
(``order_decay * cache + (1 - order_decay) * value``, :283-287) is
``order_memory_chunked`` over one token with ``initial=cache``.

Runs on the gfx950 HIP library (``m4mr_order_forward`` /
``m4mr_order_backward``); gradients reach the values, the log decays and the
initial state.
"""

import torch

from mamba4_amd import _lib
from mamba4_amd.memory import _ptr, _require_device, _stream

MAX_WIDTH = 256


def _f32(t):
    return t.to(torch.float32).contiguous()


def _workspace(lib, batch, time, heads, width, chunk, device):
    nbytes = lib.m4mr_order_workspace_bytes(batch, time, heads, width, chunk)
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


class _OrderScan(torch.autograd.Function):
    @staticmethod
    def forward(ctx, values, log_decay, initial, chunk):
        lib = _lib.load()
        batch, time, heads, width = values.shape
        output = torch.empty_like(values)
        workspace, nbytes = _workspace(lib, batch, time, heads, width, chunk, values.device)
        _lib.check(
            lib.m4mr_order_forward(
                _ptr(values), _ptr(log_decay), _ptr(initial), batch, time, heads, width, chunk,
                _ptr(output), _ptr(workspace), nbytes, _stream(),
            )
        )
        ctx.save_for_backward(values, log_decay, initial, output)
        ctx.chunk = chunk
        return output

    @staticmethod
    def backward(ctx, d_output):
        lib = _lib.load()
        values, log_decay, initial, output = ctx.saved_tensors
        batch, time, heads, width = values.shape
        d_output = _f32(d_output)
        d_values = torch.empty_like(values)
        d_log_decay = torch.empty_like(log_decay)
        d_initial = None if initial is None else torch.empty_like(initial)
        workspace, nbytes = _workspace(lib, batch, time, heads, width, ctx.chunk, values.device)
        _lib.check(
            lib.m4mr_order_backward(
                _ptr(values), _ptr(log_decay), _ptr(initial), _ptr(output), _ptr(d_output),
                batch, time, heads, width, ctx.chunk, _ptr(d_values), _ptr(d_log_decay),
                _ptr(d_initial), _ptr(workspace), nbytes, _stream(),
            )
        )
        return d_values, d_log_decay, d_initial, None


def order_memory_chunked(values, log_decay, chunk_size=64, *, initial=None):
    """The gated vector scan of lm/models/mamba4.py:59-95 on the GPU.

    values [B,T,H,W] (W <= 256), log_decay [B,T,H]; returns h [B,T,H,W] in
    float32.  ``chunk_size`` only sets the kernels' chunking (chunks above 64
    tokens run as 64: the result is the same up to rounding).  ``initial``
    [B,H,W] is the state before the first token (zero by default).
    """
    tensors = [values, log_decay] + ([] if initial is None else [initial])
    _require_device(*tensors)
    if values.dim() != 4 or log_decay.shape != values.shape[:3]:
        raise ValueError("order_memory_chunked needs values [B,T,H,W] and log_decay [B,T,H]")
    batch, time, heads, width = values.shape
    if width < 1 or width > MAX_WIDTH:
        raise ValueError(f"order_memory_chunked supports value widths 1..{MAX_WIDTH}")
    if chunk_size < 1:
        raise ValueError("chunk_size must be positive")
    if initial is not None and initial.shape != (batch, heads, width):
        raise ValueError("order_memory_chunked needs initial [B,H,W]")
    if time == 0:
        return values.new_zeros(values.shape, dtype=torch.float32)
    chunk = min(int(chunk_size), _lib.MAX_CHUNK)
    return _OrderScan.apply(
        _f32(values), _f32(log_decay), None if initial is None else _f32(initial), chunk
    )


def order_memory(values, decay, *, initial=None):
    """The same scan from the decays themselves (lm/models/mamba4.py:46-56)."""
    return order_memory_chunked(values, torch.log(decay.to(torch.float32)), initial=initial)
