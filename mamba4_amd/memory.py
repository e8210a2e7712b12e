"""Mamba 4 selective memory read on MI355X: the lm/kernels/mamba4.py API.

Same names, arguments, NamedTuples and error behaviour as the reference's
``selective_gaussian_memory`` (lm/kernels/mamba4.py:228-338),
``selective_decode`` (:341-355), ``selective_initial_state`` (:221-225),
``spd_solve`` (:190-217), ``SelectiveState`` / ``SelectiveResult``
(:18-28), with torch tensors on a
ROCm device in place of JAX arrays.  Every call runs the gfx950 HIP library
through its C ABI on the current torch stream; there is no other
implementation, and CPU tensors are rejected.

A differentiable forward stores each token's Cholesky factor, and the
backward consumes the residual set the reference tags ``"memory_solve"``
(lm/kernels/mamba4_fused.py:333-336): it issues only triangular solves and
chunk contractions, never a second factorization.  A forward that takes no
gradient factors without storing (the reference's store_factors=False
mode, lm/kernels/mamba4_fused.py:183-232).
"""

from typing import NamedTuple

import torch
import torch.nn.functional as F

from mamba4_amd import _lib

# Solver strings the reference accepts (lm/config.py:50,
# lm/kernels/mamba4.py:164-182,249) plus "mi355x".  All of them select the
# HIP path: the factorization backend changes only the arithmetic schedule,
# never the solved system (lm/kernels/mamba4.py:193-194).
SOLVERS = (None, "loop", "blocked", "unrolled", "auto", "fused", "mi355x")
MEMORY_SOLVE = "memory_solve"


class SelectiveState(NamedTuple):
    """Evidence-only sufficient statistics; precision adds the fixed floor."""

    evidence: torch.Tensor
    cross: torch.Tensor


class SelectiveResult(NamedTuple):
    output: torch.Tensor
    variance: torch.Tensor
    state: SelectiveState


def _check_solver(solver):
    if solver not in SOLVERS:
        raise ValueError(f"Unknown SPD solve backend {solver}")


def _stream():
    return ctypes_stream(torch.cuda.current_stream())


def ctypes_stream(stream):
    return stream.cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _require_device(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(
                "the MI355X memory read needs ROCm device tensors; got a CPU tensor"
            )


def selective_initial_state(batch, heads, key_dim, value_dim, device="cuda"):
    return SelectiveState(
        torch.zeros((batch, heads, key_dim, key_dim), dtype=torch.float32, device=device),
        torch.zeros((batch, heads, value_dim, key_dim), dtype=torch.float32, device=device),
    )


def _value_width(value_dim):
    """The library's value width for `value_dim` columns: 64 or 128."""
    if value_dim > _lib.MAX_VALUE_DIM:
        raise ValueError(
            f"value widths must be <= {_lib.MAX_VALUE_DIM}; got {value_dim}"
        )
    return _lib.VALUE_DIM if value_dim <= _lib.VALUE_DIM else _lib.MAX_VALUE_DIM


def memread_forward(keys, values, queries, beta, log_decay, floor, init_s, init_c, chunk,
                    store_factors=True):
    """m4mr_forward (or m4mr_forward_bf16 for bfloat16 keys, values and
    queries) on contiguous padded inputs: returns (output, variance,
    final_evidence, final_cross, solved, factors, start_evidence, start_cross).
    Without ``store_factors`` no factor buffer is allocated and ``factors``
    is None: the kernels factor and solve without storing, the reference's
    store_factors=False mode (lm/kernels/mamba4_fused.py:183-232); every
    other array is bit-identical."""
    lib = _lib.load()
    batch, time, heads, _ = keys.shape
    width = values.shape[-1]
    count, starts = _lib.start_counts(time, chunk)
    dev = keys.device
    f32 = dict(dtype=torch.float32, device=dev)
    output = torch.empty((batch, time, heads, width), **f32)
    variance = torch.empty((batch, time, heads), **f32)
    final_s = torch.empty((batch, heads, 64, 64), **f32)
    final_c = torch.empty((batch, heads, width, 64), **f32)
    solved = torch.empty((batch, time, heads, 64), **f32)
    factors = (torch.empty((batch, time, heads, _lib.FACTOR_FLOATS), **f32)
               if store_factors else None)
    start_s = torch.empty((batch, heads, starts, 64, 64), **f32)
    start_c = torch.empty((batch, heads, count, width, 64), **f32)
    # bfloat16 keys, values and queries are read and widened in the kernels.
    entry = lib.m4mr_forward_bf16 if keys.dtype == torch.bfloat16 else lib.m4mr_forward
    _lib.check(
        entry(
            _ptr(keys), _ptr(values), _ptr(queries), _ptr(beta), _ptr(log_decay),
            _ptr(floor), _ptr(init_s), _ptr(init_c), batch, time, heads, width, chunk,
            _ptr(output), _ptr(variance), _ptr(final_s), _ptr(final_c),
            _ptr(solved), _ptr(factors), _ptr(start_s), _ptr(start_c), _stream(),
        )
    )
    return output, variance, final_s, final_c, solved, factors, start_s, start_c


class _MemoryRead(torch.autograd.Function):
    """Custom VJP around m4mr_forward / m4mr_backward (D = 64, P = 64 or 128;
    keys, values and queries float32, or all bfloat16 through the _bf16
    entry points)."""

    @staticmethod
    def forward(ctx, keys, values, queries, beta, log_decay, floor, init_s, init_c, chunk):
        output, variance, final_s, final_c, solved, factors, start_s, start_c = memread_forward(
            keys, values, queries, beta, log_decay, floor, init_s, init_c, chunk
        )
        # The residual set the reference checkpoints as "memory_solve".
        ctx.save_for_backward(
            keys, values, queries, beta, log_decay, floor, solved, factors, start_s, start_c
        )
        ctx.chunk = chunk
        ctx.has_initial = init_s is not None
        return output, variance, final_s, final_c

    @staticmethod
    def backward(ctx, d_output, d_variance, d_final_s, d_final_c):
        grads = memread_backward(*ctx.saved_tensors, ctx.chunk, d_output, d_variance,
                                 d_final_s, d_final_c)
        d_init = grads[6:] if ctx.has_initial else (None, None)
        return (*grads[:6], *d_init, None)


def memread_backward(keys, values, queries, beta, log_decay, floor, solved, factors, start_s,
                     start_c, chunk, d_output, d_variance, d_final_s, d_final_c, mixer=None):
    """m4mr_backward on the forward's inputs and residual set: returns
    (d_keys, d_values, d_queries, d_beta, d_log_decay, d_floor, d_init_evidence,
    d_init_cross), all float32.  None cotangents are zero.  With
    ``mixer = (previous, key_shift)``, keys and queries are the mixer's raw
    projections and m4mr_mixer_backward normalises them on load (the
    gradients are still those of the normalised keys and queries)."""
    lib = _lib.load()
    batch, time, heads, _ = keys.shape
    width = values.shape[-1]

    def dense(g, like):
        if g is None:
            return torch.zeros(like.shape, dtype=torch.float32, device=like.device)
        return g.to(torch.float32).contiguous()

    d_output = dense(d_output, values)
    d_variance = dense(d_variance, beta)
    d_final_s = None if d_final_s is None else d_final_s.to(torch.float32).contiguous()
    d_final_c = None if d_final_c is None else d_final_c.to(torch.float32).contiguous()
    f32 = dict(dtype=torch.float32, device=keys.device)
    grads = [torch.empty(t.shape, **f32) for t in (keys, values, queries, beta, log_decay,
                                                    floor)]
    d_init_s = torch.empty((batch, heads, _lib.KEY_DIM, _lib.KEY_DIM), **f32)
    d_init_c = torch.empty((batch, heads, width, _lib.KEY_DIM), **f32)
    nbytes = lib.m4mr_backward_workspace_bytes(batch, time, heads, width, chunk)
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=keys.device)
    tail = (batch, time, heads, width, chunk, _ptr(solved), _ptr(factors), _ptr(start_s),
            _ptr(start_c), _ptr(d_output), _ptr(d_variance), _ptr(d_final_s), _ptr(d_final_c),
            *(_ptr(g) for g in grads), _ptr(d_init_s), _ptr(d_init_c), _ptr(workspace), nbytes,
            _stream())
    head = (_ptr(keys), _ptr(values), _ptr(queries), _ptr(beta), _ptr(log_decay), _ptr(floor))
    if mixer is not None:
        previous, key_shift = mixer
        _lib.check(lib.m4mr_mixer_backward(*head, _ptr(previous), int(key_shift), *tail))
    else:
        entry = lib.m4mr_backward_bf16 if keys.dtype == torch.bfloat16 else lib.m4mr_backward
        _lib.check(entry(*head, *tail))
    return (*grads, d_init_s, d_init_c)


class _SpdSolve(torch.autograd.Function):
    """Custom VJP around m4mr_spd_solve / m4mr_spd_solve_backward."""

    @staticmethod
    def forward(ctx, precision, rhs):
        lib = _lib.load()
        count, dim = rhs.shape
        f32 = dict(dtype=torch.float32, device=rhs.device)
        solution = torch.empty((count, dim), **f32)
        factors = torch.empty((count, lib.m4mr_spd_factor_floats(dim)), **f32)
        _lib.check(
            lib.m4mr_spd_solve(
                _ptr(precision), _ptr(rhs), count, dim, _ptr(solution), _ptr(factors), _stream()
            )
        )
        ctx.save_for_backward(factors, solution)
        return solution

    @staticmethod
    def backward(ctx, gradient):
        lib = _lib.load()
        factors, solution = ctx.saved_tensors
        count, dim = solution.shape
        gradient = gradient.to(torch.float32).contiguous()
        d_precision = torch.empty((count, dim, dim), dtype=torch.float32, device=solution.device)
        d_rhs = torch.empty_like(solution)
        _lib.check(
            lib.m4mr_spd_solve_backward(
                _ptr(factors), _ptr(solution), _ptr(gradient), count, dim,
                _ptr(d_precision), _ptr(d_rhs), _stream(),
            )
        )
        return d_precision, d_rhs


def spd_solve(precision, rhs, backend=None):
    """Solve precision @ y = rhs for SPD [...,d,d] precision and [...,d] rhs.

    Only the lower triangle is read.  The backward pass reuses the stored
    Cholesky factor: z = A^-1 g, d rhs = z and d A = -sym(z y^T); no
    inverse is formed and nothing is refactored.  Every reference backend
    string selects the same HIP solve (the backend changes only the
    arithmetic schedule, never the solved system, lm/kernels/mamba4.py:193-194).
    Widths up to 64 solve four systems per wave; wider ones (up to 4096) one
    system per 256-thread block.
    """
    _check_solver(backend)
    precision = torch.as_tensor(precision)
    rhs = torch.as_tensor(rhs)
    dim = rhs.shape[-1]
    if precision.shape != rhs.shape + (dim,):
        raise ValueError(
            f"spd_solve needs precision [...,d,d] and rhs [...,d]; got "
            f"{tuple(precision.shape)} and {tuple(rhs.shape)}"
        )
    if dim > _lib.SPD_MAX_DIM:
        raise ValueError(f"spd_solve supports widths <= {_lib.SPD_MAX_DIM}; got {dim}")
    _require_device(precision, rhs)
    batch = rhs.shape[:-1]
    if rhs.numel() == 0:
        return torch.zeros(rhs.shape, dtype=torch.float32, device=rhs.device)
    flat_a = precision.to(torch.float32).reshape(-1, dim, dim).contiguous()
    flat_b = rhs.to(torch.float32).reshape(-1, dim).contiguous()
    with torch.cuda.device(rhs.device):
        solution = _SpdSolve.apply(flat_a, flat_b)
    return solution.reshape(batch + (dim,))


def _pad_last(x, width, value=0.0):
    extra = width - x.shape[-1]
    return x if extra == 0 else F.pad(x, (0, extra), value=value)


def selective_gaussian_memory(
    keys,
    values,
    queries,
    beta,
    log_decay,
    floor,
    *,
    chunk_size=64,
    initial=None,
    solver=None,
):
    """Exact chunked reads of the fixed-floor selective Gaussian memory.

    keys/queries [B,T,H,D], values [B,T,H,P], beta and log_decay [B,T,H]
    (log_decay <= 0), floor [H,D] positive; D <= 64, P <= 128.  With
    S_t = lam_t S_(t-1) + beta_t k k^T and C_t likewise, each token reads
    C_t y_t and q_t^T y_t where (S_t + diag(floor)) y_t = q_t.  Returns
    SelectiveResult(output [B,T,H,P], variance [B,T,H],
    SelectiveState(evidence [B,H,D,D], cross [B,H,P,D])); gradients reach
    every input and ``initial``.
    """
    _check_solver(solver)
    keys, values, queries = (torch.as_tensor(a) for a in (keys, values, queries))
    batch, time, heads, dim = keys.shape
    value_dim = values.shape[-1]
    if queries.shape != keys.shape or values.shape[:3] != keys.shape[:3]:
        raise ValueError("Selective memory keys, values and queries disagree")
    _require_device(keys, values, queries)
    # bfloat16 keys, values and queries stay bfloat16: the kernels widen them
    # on load, exactly as the reference's upcast (lm/kernels/mamba4.py:263-265).
    # Any other mix is upcast here.
    if not all(a.dtype == torch.bfloat16 for a in (keys, values, queries)):
        keys, values, queries = (a.to(torch.float32) for a in (keys, values, queries))
    if dim > _lib.KEY_DIM:
        raise ValueError(f"key widths must be <= {_lib.KEY_DIM}; got {dim}")
    width = _value_width(value_dim)
    if chunk_size < 1:
        raise ValueError("chunk_size must be positive")
    device = keys.device
    shape = (batch, time, heads)
    beta = torch.as_tensor(beta, dtype=torch.float32, device=device).expand(shape)
    log_decay = torch.as_tensor(log_decay, dtype=torch.float32, device=device).expand(shape)
    floor = torch.as_tensor(floor, dtype=torch.float32, device=device).expand(heads, dim)
    _require_device(beta, log_decay, floor)
    # Padded key coordinates form an identity block (zero keys, unit floor):
    # they solve to zero and leave the true coordinates unchanged
    # (lm/kernels/mamba4_fused.py:292-297).  Padded values read nothing.
    k = _pad_last(keys, _lib.KEY_DIM).contiguous()
    q = _pad_last(queries, _lib.KEY_DIM).contiguous()
    v = _pad_last(values, width).contiguous()
    f = _pad_last(floor, _lib.KEY_DIM, value=1.0).contiguous()
    init_s = init_c = None
    if initial is not None:
        init_s = torch.as_tensor(initial.evidence).to(torch.float32)
        init_c = torch.as_tensor(initial.cross).to(torch.float32)
        _require_device(init_s, init_c)
        init_s = F.pad(init_s, (0, _lib.KEY_DIM - dim, 0, _lib.KEY_DIM - dim)).contiguous()
        init_c = F.pad(
            init_c, (0, _lib.KEY_DIM - dim, 0, width - value_dim)
        ).contiguous()
    chunk = min(int(chunk_size), _lib.MAX_CHUNK)
    args = (k, v, q, beta.contiguous(), log_decay.contiguous(), f, init_s, init_c, chunk)
    differentiable = (keys, values, queries, beta, log_decay, floor, init_s, init_c)
    with torch.cuda.device(device):
        if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in differentiable
        ):
            output, variance, final_s, final_c = _MemoryRead.apply(*args)
        else:
            # No gradient: factor and solve without storing the factors, as
            # the reference's primal chunk_solve does
            # (lm/kernels/mamba4_fused.py:323-326).
            output, variance, final_s, final_c = memread_forward(*args, store_factors=False)[:4]
    return SelectiveResult(
        output[..., :value_dim],
        variance,
        SelectiveState(final_s[..., :dim, :dim], final_c[..., :value_dim, :dim]),
    )


def selective_decode(state, key, value, query, beta, log_decay, floor, solver=None):
    """One exact write/read from a cached state: O(D^3 + P D) refactor.

    state.evidence [B,H,D,D], state.cross [B,H,P,D]; key/query [B,H,D];
    value [B,H,P]; beta/log_decay [B,H]; floor [H,D].  Returns
    SelectiveResult(output [B,H,P], variance [B,H], new state); the input
    state is not modified (see ``selective_decode_`` for the in-place form).
    Widths below 64 are zero-padded like the prefill path.
    """
    _check_solver(solver)
    evidence = torch.as_tensor(state.evidence)
    cross = torch.as_tensor(state.cross)
    _require_device(evidence, cross)
    inputs = (evidence, cross, key, value, query, beta, log_decay, floor)
    if torch.is_grad_enabled() and any(
        isinstance(t, torch.Tensor) and t.requires_grad for t in inputs
    ):
        # A differentiable step is the one-token prefill from `state`: the
        # same HIP kernels with the custom VJP attached.
        one = selective_gaussian_memory(
            torch.as_tensor(key)[:, None],
            torch.as_tensor(value)[:, None],
            torch.as_tensor(query)[:, None],
            torch.as_tensor(beta, device=evidence.device).expand(evidence.shape[:2])[:, None],
            torch.as_tensor(log_decay, device=evidence.device).expand(evidence.shape[:2])[:, None],
            floor,
            chunk_size=1,
            initial=SelectiveState(evidence, cross),
            solver=solver,
        )
        return SelectiveResult(one.output[:, 0], one.variance[:, 0], one.state)
    dim, value_dim = evidence.shape[-1], cross.shape[-2]
    if dim > _lib.KEY_DIM:
        raise ValueError(f"key widths must be <= {_lib.KEY_DIM}; got {dim}")
    width = _value_width(value_dim)
    kd, vd = _lib.KEY_DIM - dim, width - value_dim
    padded = SelectiveState(
        F.pad(evidence.to(torch.float32), (0, kd, 0, kd)).contiguous(),
        F.pad(cross.to(torch.float32), (0, kd, 0, vd)).contiguous(),
    )
    device = evidence.device
    floor = torch.as_tensor(floor, dtype=torch.float32, device=device).expand(
        evidence.shape[1], dim
    )
    out = selective_decode_(
        padded,
        _pad_last(torch.as_tensor(key, device=device).to(torch.float32), _lib.KEY_DIM),
        _pad_last(torch.as_tensor(value, device=device).to(torch.float32), width),
        _pad_last(torch.as_tensor(query, device=device).to(torch.float32), _lib.KEY_DIM),
        beta,
        log_decay,
        _pad_last(floor, _lib.KEY_DIM, value=1.0),
        solver,
    )
    return SelectiveResult(
        out.output[..., :value_dim],
        out.variance,
        SelectiveState(
            out.state.evidence[..., :dim, :dim], out.state.cross[..., :value_dim, :dim]
        ),
    )


def selective_decode_(state, key, value, query, beta, log_decay, floor, solver=None):
    """In-place ``selective_decode``: overwrites ``state`` with the new state.

    Needs float32 contiguous state tensors with D = 64 and P = 64 or 128.
    """
    _check_solver(solver)
    lib = _lib.load()
    evidence, cross = state.evidence, state.cross
    _require_device(evidence, cross)
    batch, heads, dim, _ = evidence.shape
    value_dim = cross.shape[-2]
    if dim != _lib.KEY_DIM or value_dim not in (_lib.VALUE_DIM, _lib.MAX_VALUE_DIM):
        raise ValueError("the in-place decode needs D = 64 and P = 64 or 128 states")
    if evidence.dtype != torch.float32 or not evidence.is_contiguous() or not cross.is_contiguous():
        raise ValueError("the in-place decode needs contiguous float32 states")
    device = evidence.device
    f32 = dict(dtype=torch.float32, device=device)
    key, value, query = (torch.as_tensor(a).to(**f32).contiguous() for a in (key, value, query))
    beta = torch.as_tensor(beta, **f32).expand(batch, heads).contiguous()
    log_decay = torch.as_tensor(log_decay, **f32).expand(batch, heads).contiguous()
    floor = torch.as_tensor(floor, **f32).expand(heads, dim).contiguous()
    output = torch.empty((batch, heads, value_dim), **f32)
    variance = torch.empty((batch, heads), **f32)
    with torch.cuda.device(device):
        _lib.check(
            lib.m4mr_decode_step(
                _ptr(evidence), _ptr(cross), _ptr(key), _ptr(value), _ptr(query),
                _ptr(beta), _ptr(log_decay), _ptr(floor), batch * heads, heads, value_dim,
                _ptr(output), _ptr(variance), _stream(),
            )
        )
    return SelectiveResult(output, variance, state)


DIAGNOSTIC_KEYS = (
    "precision_min_eigenvalue",
    "precision_max_eigenvalue",
    "precision_max_condition",
    "state_all_finite",
    "cross_max_abs",
    "floor_min",
    "floor_max",
)


def selective_diagnostics(state, floor):
    """Spectral and finiteness probes of the final selective precision
    (lm/kernels/mamba4.py:358-376): the extreme eigenvalues of the
    symmetrised evidence + diag(floor) over every state, the largest
    condition number, whether the state is finite, the largest cross
    magnitude and the floor's range, as 0-dim tensors under the reference's
    keys (``state_all_finite`` a bool tensor).

    ``state.evidence`` [..., D, D] (D <= 64) and ``state.cross`` [..., P, D]
    on the GPU; ``floor`` broadcasts to [..., D].  The eigenvalues come from
    a Jacobi iteration on the device (m4mr_diagnostics).
    """
    lib = _lib.load()
    evidence, cross = state.evidence, state.cross
    _require_device(evidence, cross)
    dim = evidence.shape[-1]
    if evidence.shape[-2] != dim or cross.shape[-1] != dim:
        raise ValueError("evidence must be [..., D, D] and cross [..., P, D]")
    if dim > _lib.KEY_DIM:
        raise ValueError(f"selective_diagnostics supports widths <= {_lib.KEY_DIM}; got {dim}")
    lead = tuple(evidence.shape[:-2])
    if tuple(cross.shape[:-2]) != lead:
        raise ValueError("evidence and cross must share their leading dimensions")
    count = 1
    for n in lead:
        count *= n
    device = evidence.device
    f32 = dict(dtype=torch.float32, device=device)
    value_dim = cross.shape[-2]
    evidence = evidence.to(**f32).reshape(count, dim, dim).contiguous()
    cross = cross.to(**f32).reshape(count, value_dim, dim).contiguous()
    floor = torch.as_tensor(floor).to(**f32)
    # Every state carries its own floor row (the kernel's "head" index runs
    # over the states); the range of the broadcast floor is the floor's own.
    per_floor = torch.broadcast_to(floor, lead + (dim,)).reshape(count, dim).contiguous()
    per_state = torch.empty((count, 4), **f32)
    summary = torch.empty((7,), **f32)
    with torch.cuda.device(device):
        _lib.check(
            lib.m4mr_diagnostics(
                _ptr(evidence), _ptr(cross), _ptr(per_floor), 1, count, dim, value_dim,
                _ptr(per_state), _ptr(summary), _stream(),
            )
        )
    out = {k: summary[i] for i, k in enumerate(DIAGNOSTIC_KEYS)}
    out["state_all_finite"] = summary[3] > 0.5
    return out
