"""The FlashMamba Mamba-3 SISO scan on MI355X.

Mirrors ``mamba3_fused`` (lm/kernels/flashmamba.py:1125-1162), the Mamba-3
mixer's scan in the projection layout (called from lm/models/mamba3.py:104):
shared query and key rows ``c, b`` [B,T,N], values ``x`` [B,T,H*P], per-head
``adt, dt, trap_logits`` [B,T,H], shared angle rates ``angles`` [B,T,A] and
per-head biases ``q_bias, k_bias`` [H,1,N]; returns ``y`` [B,T,H*P] and the
final state [B,H,N,P].  Gradients reach all nine inputs (the reference's
custom VJP, :1000-1110, plus the autodiff of its weight and angle glue).

Runs on the gfx950 HIP library (``m3s_forward`` / ``m3s_backward``,
include/mamba3_scan.h); there is no other implementation.  With ``c``, ``b``
and ``x`` all bfloat16 (a bfloat16 model) it takes ``m3s_forward_bf16`` /
``m3s_backward_bf16``: the products take bfloat16 operands with float32
accumulation where the reference's fused kernels round to the model dtype
(lm/kernels/flashmamba.py:575-786), ``y`` and ``d_x`` come back in bfloat16
and the other gradients in their inputs' dtypes (:1088-1099).  Otherwise the
arithmetic is float32 (other inputs are widened on entry; ``y`` returns in
``x``'s dtype).  The final state is float32 either way, as in the reference.
"""

import torch

from mamba4_amd import _lib
from mamba4_amd.memory import _ptr, _require_device, _stream

CHUNK = 64
MAX_STATE = 128
MAX_VALUE = 64
MAX_HEADS = 128
STATE_FLOATS = 8192
PHASE_FLOATS = 64


def _f32(t):
    return t.to(torch.float32).contiguous()


class _FusedScan(torch.autograd.Function):
    """c, b, x float32, or all three bfloat16 (the bfloat16 entry points);
    the other inputs float32."""

    @staticmethod
    def forward(ctx, c, b, x, adt, dt, trap, angles, q_bias, k_bias):
        lib = _lib.load()
        bf16 = x.dtype == torch.bfloat16
        batch, time, state = c.shape
        heads = dt.shape[-1]
        width = x.shape[-1] // heads
        count = angles.shape[-1]
        chunks = (time + CHUNK - 1) // CHUNK
        y = torch.empty_like(x)
        final = torch.empty(batch, heads, state, width, dtype=torch.float32, device=x.device)
        starts = torch.empty(batch, heads, chunks, STATE_FLOATS, dtype=torch.float32,
                             device=x.device)
        phases = torch.empty(batch, heads, chunks, PHASE_FLOATS, dtype=torch.float32,
                             device=x.device)
        entry = lib.m3s_forward_bf16 if bf16 else lib.m3s_forward
        _lib.check(
            entry(
                _ptr(c), _ptr(b), _ptr(x), _ptr(adt), _ptr(dt), _ptr(trap),
                _ptr(angles) if count else None, _ptr(q_bias), _ptr(k_bias), batch, time,
                heads, state, width, count, _ptr(y), _ptr(final), _ptr(starts), _ptr(phases),
                _stream(),
            )
        )
        ctx.save_for_backward(c, b, x, adt, dt, trap, angles, q_bias, k_bias, starts, phases)
        return y, final

    @staticmethod
    def backward(ctx, d_y, d_final):
        lib = _lib.load()
        c, b, x, adt, dt, trap, angles, q_bias, k_bias, starts, phases = ctx.saved_tensors
        batch, time, state = c.shape
        heads = dt.shape[-1]
        width = x.shape[-1] // heads
        count = angles.shape[-1]
        bf16 = x.dtype == torch.bfloat16
        # The cotangent in the model dtype (the reference's d_y.astype(x.dtype), :1008).
        d_y = torch.zeros_like(x) if d_y is None else d_y.to(x.dtype).contiguous()
        d_final = None if d_final is None else _f32(d_final)
        grads = [torch.empty(t.shape, dtype=x.dtype if i == 2 else torch.float32,
                             device=t.device)
                 for i, t in enumerate((c, b, x, adt, dt, trap, angles, q_bias, k_bias))]
        nbytes = lib.m3s_backward_workspace_bytes(batch, time, heads, state, width, count)
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        entry = lib.m3s_backward_bf16 if bf16 else lib.m3s_backward
        _lib.check(
            entry(
                _ptr(c), _ptr(b), _ptr(x), _ptr(adt), _ptr(dt), _ptr(trap),
                _ptr(angles) if count else None, _ptr(q_bias), _ptr(k_bias), batch, time,
                heads, state, width, count, _ptr(starts), _ptr(phases), _ptr(d_y),
                _ptr(d_final), *(_ptr(g) if (i != 6 or count) else None
                                 for i, g in enumerate(grads)),
                _ptr(workspace), nbytes, _stream(),
            )
        )
        return tuple(g.to(t.dtype) for g, t in zip(grads, (c, b, x, adt, dt, trap, angles,
                                                           q_bias, k_bias)))


def mamba3_fused(c, b, x, adt, dt, trap_logits, angles, *, q_bias, k_bias, chunk_size=CHUNK,
                 interpret=None, heads_per_step=None):
    """SISO Mamba-3 with one shared query and key per token (one group).

    Same arguments and results as lm/kernels/flashmamba.py:1125-1162.
    ``chunk_size``, ``interpret`` and ``heads_per_step`` only schedule the
    reference's TPU kernel; they are accepted and do not change the result
    (these kernels run chunks of 64 tokens).
    """
    del chunk_size, interpret, heads_per_step
    _require_device(c, b, x, adt, dt, trap_logits, angles, q_bias, k_bias)
    if c.dim() != 3 or b.shape != c.shape or x.dim() != 3 or x.shape[:2] != c.shape[:2]:
        raise ValueError("mamba3_fused needs c, b [B,T,N] and x [B,T,H*P]")
    batch, time, state = c.shape
    if dt.dim() != 3 or dt.shape[:2] != (batch, time):
        raise ValueError("mamba3_fused needs dt [B,T,H]")
    heads = dt.shape[-1]
    if adt.shape != dt.shape or trap_logits.shape != dt.shape:
        raise ValueError("mamba3_fused needs adt, dt, trap_logits [B,T,H]")
    if x.shape[-1] % heads:
        raise ValueError("x's last axis must be H*P")
    width = x.shape[-1] // heads
    if angles.dim() != 3 or angles.shape[:2] != (batch, time):
        raise ValueError("mamba3_fused needs angles [B,T,A]")
    count = angles.shape[-1]
    if q_bias.numel() != heads * state or k_bias.numel() != heads * state:
        raise ValueError("mamba3_fused needs q_bias, k_bias [H,1,N]")
    if state % 2 or state > MAX_STATE or width > MAX_VALUE or heads > MAX_HEADS:
        raise ValueError(f"mamba3_fused supports even N <= {MAX_STATE}, P <= {MAX_VALUE}, "
                         f"H <= {MAX_HEADS}")
    if 2 * count > state:
        raise ValueError("mamba3_fused needs A <= N/2 angle rates")
    if time == 0:
        return x.new_zeros(x.shape), x.new_zeros((batch, heads, state, width),
                                                 dtype=torch.float32)
    bf16 = c.dtype == b.dtype == x.dtype == torch.bfloat16
    rows = (lambda t: t.contiguous()) if bf16 else _f32
    y, final = _FusedScan.apply(
        rows(c), rows(b), rows(x), _f32(adt), _f32(dt), _f32(trap_logits), _f32(angles),
        _f32(q_bias).reshape(q_bias.shape), _f32(k_bias).reshape(k_bias.shape),
    )
    return y.to(x.dtype), final
