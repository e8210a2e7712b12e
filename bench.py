#!/usr/bin/env python3
"""Memory-read fwd+bwd benchmark on one MI355X (BASELINE.json metric).

A step is one forward (chunk states, per-token factor + solve + factor
store, reads) and one backward (dy, factored re-solve, reverse carry,
gradient contractions, floor reduction) of the memory read over one batch
of synthetic config-2 input (B=16, L=1024, H=8, D=P=64, fp32), called
through the C ABI with every buffer preallocated in HBM before the timed
region.  Prints one JSON line with the throughput, the roofline of the
dominant kernel (HIP events on the launch stream), the factorization's
fp32 rate (with and without the factor store), factor-streaming bandwidth
and a CPU baseline (the NumPy oracle on config 0 and on one whole batch row
of the same workload, on this host's cores).

With --workload ref125m the step is the same fwd+bwd at the one shape the
reference publishes timings for (B=16, L=1024, H=12, D=64, P=128; inputs
and projected-loss cotangents of scripts/kernel_benchmark.py:37-47,214-224),
with vs_baseline against its TPU v4 figure (67.98 ms,
lm/results/speed-125m/bench-kernels.json:291).

With --workload config4 a step is instead one in-place decode step of
2048 sequences x 8 heads of resident (S, C) states: the
states are the end states of a 1024-token gated recurrence with
lambda = sigmoid(N(3,1)), built by this library's own forward, and each step
writes one new token into every state, refactors and reads.

With --workload config3 the step is the same fwd+bwd at BASELINE config 3
(B=32, L=1024, H=12, slow decay) with bfloat16 keys, values and queries
read natively by the kernels (m4mr_forward_bf16 / m4mr_backward_bf16).

With --workload mixer a step is the memory read's neighbours on the same
config-2 shape: the mixer prologue (key shift, unit q/k, gates, floor) and
epilogue (confidence gate, D-skip), and the order head's gated scan, each
forward and backward; every kernel is HBM-bound and reported against 8 TB/s.

With --workload mixer_read a step is the mixer's memory path forward at the
config-2 shape through the fused entry point (m4mr_mixer_forward: prologue,
memory read and read gating in one pass over the raw projections); the same
forward through the three separate entry points is timed beside it.  The
training step (forward and m4mr_mixer_read_backward, the whole VJP in one
launch sequence) is timed against the separate entry points' and against
the fused forward with the three separate backward calls.

With --workload mamba3 a step is the FlashMamba Mamba-3 scan (mamba3_fused,
lm/kernels/flashmamba.py:1125-1162) forward and backward at the 125M model's
Mamba-3 mixer shape (B=16, L=1024, H=24 heads of P=64, N=128, A=32 angle
rates; lm/configs/mamba4-125m.json), fp32, through m3s_forward /
m3s_backward; the roofline is the dominant kernel's MFMA rate against the
fp32 peak.  --workload mamba3_bf16 is the same step for a bfloat16 model
(c, b, x and d_y in bfloat16, m3s_forward_bf16 / m3s_backward_bf16: the
reference's bfloat16 matrix operands), its roofline against the dense bf16
MFMA peak.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--workload config2|config3|ref125m|config4|mixer|mixer_read|mamba3
                                   |mamba3_bf16]
"""

import argparse
import json
import os
import sys
import time

CORES = len(os.sched_getaffinity(0))
for _var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
    os.environ.setdefault(_var, str(CORES))

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "memory-read fwd+bwd tokens/sec at B16 L1024 H8 d64; % fp32 peak, % HBM BW"
CONFIG3_METRIC = "memory-read fwd+bwd tokens/sec at B32 L1024 H12 d64, bf16 q/k/v"
REF125M_METRIC = ("memory-read fwd+bwd tokens/sec at B16 L1024 H12 d64 P128 "
                  "(the reference's kernel_benchmark shape)")
# The reference's published fused fwd+bwd at that shape on one TPU v4:
# 67.98 ms for 16 x 1024 tokens (lm/results/speed-125m/bench-kernels.json:291).
REF125M_TPU_TOKENS_PER_S = 16 * 1024 / 0.06798
HBM_PEAK_GBPS = 8000.0
FP32_PEAK_TFLOPS = 157.3
BF16_PEAK_TFLOPS = 2500.0  # dense bf16 MFMA (no sparsity)
FACTOR_BYTES = 8320  # packed lower factor per token-head
CHOLESKY_FLOP = 89440  # D^3/3 + D^2/2 + D/6 at D = 64
RESOLVE_BYTES = 8832  # factor + rhs + z per token-head in the backward re-solve

NAMES = ["keys", "values", "queries", "beta", "log_decay", "floor"]
CAUSAL_PAIRS = 2080  # (t, s) pairs with s <= t in a 64-token chunk

# Algorithmic work per token-head of each kernel at D = P = 64, chunk 64:
# (bound, amount, unit).  HBM kernels count the bytes their algorithm must
# move; contraction kernels count 2 flop per multiply-add of their products.
KERNEL_WORK = {
    "fwd_factor": ("hbm", FACTOR_BYTES, "B"),
    "factored_solve": ("hbm", RESOLVE_BYTES, "B"),
    # Causal products count their s <= t pairs only (64 * 65 / 2 = 2,080 of
    # 4,096 per 64-token chunk, i.e. 2 * 2,080 flop per token-head at width
    # 64); full chunk products count 2 * 4,096.
    "fwd_read": ("mfma", 2 * (2 * CAUSAL_PAIRS + 4096), "flop"),  # Y K^T, (G) V causal; Y C0^T
    "bwd_dy": ("mfma", 2 * (2 * CAUSAL_PAIRS + 4096), "flop"),  # dO V^T, (G) K causal; dO C0
    # gy, gz, gv and the three masked contractions over t causal; G^T k, G k,
    # H k, H^T v, y^T S0, dO^T C0 full
    "bwd_grads": ("mfma", 2 * (6 * CAUSAL_PAIRS + 6 * 4096), "flop"),
    "fwd_stats": ("mfma", 2 * 8192, "flop"),  # K^T diag K, V^T diag K
    "fwd_scan": ("hbm", 16384 * 3 * 2 // 64, "B"),  # r+w of 2 evidence + 1 cross state / chunk
    "bwd_local": ("mfma", 2 * 8192, "flop"),  # Z^T diag Y, dO^T diag Y
    "bwd_scan": ("hbm", 16384 * 2 * 2 // 64, "B"),  # r+w of 1 evidence + 1 cross state / chunk
    "floor_reduce": ("hbm", 4, "B"),
    # Fused state walks: read k and v (or z, y and dO) once, beta and log
    # decay, write one evidence state per 32-token sub-chunk (forward) or
    # chunk and one cross state per chunk: 16 KiB / 32 + 16 KiB / 64.
    "fwd_states": ("hbm", 256 + 256 + 8 + 512 + 256, "B"),
    "bwd_states": ("hbm", 3 * 256 + 4 + 256 + 256, "B"),
}


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "config2_hbm_traffic.md")
DECODE_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "config4_decode_hbm_traffic.md")
MAMBA3_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "mamba3_scan_hbm_traffic.md")

# Config 4 (decode): 2048 sequences x 8 heads of resident 64x64 states.
DECODE_METRIC = "decode-step tokens/sec, 2048 sequences x 8 heads d64 resident states; % HBM BW"
DECODE_BATCH, DECODE_HEADS, DECODE_CONTEXT = 2048, 8, 1024
# HBM bytes one decode step must move per (sequence, head) state with the
# API's full-matrix state layout: read + write of S and of C (4 x 16 KiB),
# the token's key, value and query (3 x 256 B), beta and log_decay, and the
# output row and variance.
DECODE_STATE_BYTES = 4 * 16384 + 3 * 256 + 8 + 256 + 4


def measured_traffic(kernel, summary=TRAFFIC_SUMMARY):
    """HBM bytes per launch of `kernel` from a committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by its copy-kernel calibration),
    or None when the summary does not list it."""
    try:
        lines = open(summary).read().splitlines()
    except OSError:
        return None
    for line in lines:
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 6 and cells[0] == kernel:
            return float(cells[5].replace(",", "")) * 1e6
    return None


def roofline(kernel, ms, token_heads, traffic=True):
    bound, amount, unit = KERNEL_WORK[kernel]
    seconds = ms / 1e3
    if bound == "hbm":
        achieved = amount * token_heads / seconds / 1e9
        peak, unit_out = HBM_PEAK_GBPS, "GB/s"
    else:
        achieved = amount * token_heads / seconds / 1e12
        peak, unit_out = FP32_PEAK_TFLOPS, "TFLOP/s"
    return {
        "kernel": kernel,
        "bound": bound,
        "achieved": achieved,
        "peak": peak,
        "unit": unit_out,
        "frac": achieved / peak,
        "traffic": measured_traffic(kernel) if traffic else None,
        "traffic_unit": "B per launch (rocprofv3, profiles/config2_hbm_traffic.md)",
        "algorithmic_bytes" if bound == "hbm" else "algorithmic_flop": amount * token_heads,
    }


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=30)
    p.add_argument("--chunk", type=int, default=64)
    p.add_argument("--workload", default="config2",
                   choices=["config2", "config3", "ref125m", "config4", "mixer", "mixer_read",
                            "mamba3", "mamba3_bf16"])
    p.add_argument("--no-cpu-baseline", action="store_true")
    return p.parse_args()


class Problem:
    """Device buffers for one fwd+bwd step through the C ABI."""

    def __init__(self, data, chunk, bf16_inputs=False):
        import torch

        from mamba4_amd import _lib

        self.lib = _lib.load()
        self.bf16 = bf16_inputs
        self.check = _lib.check
        dev = torch.device("cuda:0")
        self.B, self.T, self.H, _ = data["keys"].shape
        self.chunk = chunk
        count, starts = _lib.start_counts(self.T, chunk)
        B, T, H = self.B, self.T, self.H

        def put(a):
            return torch.tensor(np.asarray(a, np.float32), device=dev)

        self.inputs = [put(data[n]) for n in NAMES]
        if bf16_inputs:
            # Keys, values and queries in bfloat16, read by the _bf16 entry points.
            self.inputs[:3] = [t.to(torch.bfloat16) for t in self.inputs[:3]]
        self.d_output = put(data["d_output"])
        self.d_variance = put(data["d_variance"])
        self.P = P = data["values"].shape[-1]
        f32 = dict(dtype=torch.float32, device=dev)
        self.fwd_out = [
            torch.empty(B, T, H, P, **f32),  # output
            torch.empty(B, T, H, **f32),  # variance
            torch.empty(B, H, 64, 64, **f32),  # final evidence
            torch.empty(B, H, P, 64, **f32),  # final cross
            torch.empty(B, T, H, 64, **f32),  # solved
            torch.empty(B, T, H, _lib.FACTOR_FLOATS, **f32),  # factors
            torch.empty(B, H, starts, 64, 64, **f32),  # start evidence
            torch.empty(B, H, count, P, 64, **f32),  # start cross
        ]
        self.grads = [torch.empty(t.shape, **f32) for t in self.inputs]
        self.d_init = [torch.empty(B, H, 64, 64, **f32), torch.empty(B, H, P, 64, **f32)]
        self.ws_bytes = self.lib.m4mr_backward_workspace_bytes(B, T, H, P, chunk)
        self.workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=dev)
        self.stream = torch.cuda.current_stream().cuda_stream

    def forward(self, store=True):
        """The forward; with store=False no factors are stored (factors = NULL,
        the forward of a call that takes no gradient)."""
        p = [t.data_ptr() for t in self.inputs]
        o = [t.data_ptr() for t in self.fwd_out]
        if not store:
            o[5] = None
        entry = self.lib.m4mr_forward_bf16 if self.bf16 else self.lib.m4mr_forward
        self.check(entry(*p, None, None, self.B, self.T, self.H, self.P, self.chunk, *o,
                         self.stream))

    def backward(self):
        p = [t.data_ptr() for t in self.inputs]
        o = self.fwd_out
        entry = self.lib.m4mr_backward_bf16 if self.bf16 else self.lib.m4mr_backward
        self.check(
            entry(
                *p, self.B, self.T, self.H, self.P, self.chunk, o[4].data_ptr(), o[5].data_ptr(),
                o[6].data_ptr(), o[7].data_ptr(), self.d_output.data_ptr(),
                self.d_variance.data_ptr(), None, None, *(g.data_ptr() for g in self.grads),
                *(g.data_ptr() for g in self.d_init), self.workspace.data_ptr(), self.ws_bytes,
                self.stream,
            )
        )


class Decode:
    """Config-4 resident states and token sets for in-place decode steps."""

    TOKEN_SETS = 8

    def __init__(self, seed=0, slice_rows=128):
        import torch

        from mamba4_amd import _lib
        from mamba4_amd.inputs import decode_states, device_tokens

        self.lib = _lib.load()
        self.check = _lib.check
        B, H, T = DECODE_BATCH, DECODE_HEADS, DECODE_CONTEXT
        # End states of a T-token recurrence (config-0 distributions,
        # lambda = sigmoid(N(3,1))), built by this library's forward.
        self.evidence, self.cross, self.floor, _ = decode_states(B, H, T, seed=seed,
                                                                  slice_rows=slice_rows)
        gen = torch.Generator(device="cuda:0")
        gen.manual_seed(seed + 1)
        self.tokens = [device_tokens(gen, (B, H), shift=False) for _ in range(self.TOKEN_SETS)]
        f32 = dict(dtype=torch.float32, device="cuda:0")
        self.output = torch.empty(B, H, 64, **f32)
        self.variance = torch.empty(B, H, **f32)
        self.stream = torch.cuda.current_stream().cuda_stream
        self.calls = 0
        torch.cuda.synchronize()

    def step(self):
        k, v, q, beta, log_decay = self.tokens[self.calls % self.TOKEN_SETS]
        self.calls += 1
        self.check(
            self.lib.m4mr_decode_step(
                self.evidence.data_ptr(), self.cross.data_ptr(), k.data_ptr(), v.data_ptr(),
                q.data_ptr(), beta.data_ptr(), log_decay.data_ptr(), self.floor.data_ptr(),
                DECODE_BATCH * DECODE_HEADS, DECODE_HEADS, 64, self.output.data_ptr(),
                self.variance.data_ptr(), self.stream,
            )
        )


def decode_cpu_baseline(decode, sample=2048):
    """The NumPy oracle's decode_step (float32) on `sample` of the states."""
    from oracle import memread as oracle

    states = sample // DECODE_HEADS
    s = decode.evidence[:states].cpu().numpy()
    c = decode.cross[:states].cpu().numpy()
    k, v, q, beta, log_decay = (t[:states].cpu().numpy() for t in decode.tokens[0])
    floor = decode.floor.cpu().numpy()
    start = time.perf_counter()
    oracle.decode_step(s, c, k, v, q, beta, log_decay, floor, dtype=np.float32)
    seconds = time.perf_counter() - start
    step_seconds = seconds * (DECODE_BATCH * DECODE_HEADS) / (states * DECODE_HEADS)
    return {
        "value": DECODE_BATCH / step_seconds,
        "unit": "tokens/s",
        "cores": int(os.environ.get("OPENBLAS_NUM_THREADS", CORES)),
        "kind": "port",
        "sample": (
            f"oracle.memread.decode_step in float32 NumPy on {states} of the 2048 sequences "
            f"({states * DECODE_HEADS} states), {seconds:.2f} s, scaled to a full step; "
            f"BLAS threads = {os.environ.get('OPENBLAS_NUM_THREADS')}"
        ),
    }


def main_decode(args):
    import torch

    from mamba4_amd import _lib

    decode = Decode(seed=0)
    steps = args.steps
    for _ in range(args.warmup):
        decode.step()
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        decode.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.profile_enable(False)
    total, count = _lib.profile_read("decode_step")
    _lib.profile_reset()
    seconds = (t1 - t0) / steps
    kernel_s = total / count / 1e3
    states = DECODE_BATCH * DECODE_HEADS
    achieved = DECODE_STATE_BYTES * states / kernel_s / 1e9
    assert torch.isfinite(decode.variance).all(), "decode produced non-finite reads"
    line = {
        "metric": DECODE_METRIC,
        "value": DECODE_BATCH / seconds,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": seconds * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (
                "config4: in-place decode step, 2048 sequences x 8 heads, D=P=64 fp32, "
                "states = end states of a 1024-token recurrence (lambda = sigmoid(N(3,1)))"
            ),
            "sequences": DECODE_BATCH,
            "heads": DECODE_HEADS,
            "key_dim": 64,
            "value_dim": 64,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_step",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": measured_traffic("decode_step", DECODE_TRAFFIC_SUMMARY),
            "traffic_unit": "B per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "algorithmic_bytes": DECODE_STATE_BYTES * states,
        },
        "kernel_ms": {"decode_step": kernel_s * 1e3},
        "copy_kernel_GBps": copy_bandwidth_gbps(),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = decode_cpu_baseline(decode)
    print(json.dumps(line), flush=True)


# Algorithmic HBM bytes per token-head of the mixer-path kernels at D = P = 64
# (each input read once, each output written once).
MIXER_METRIC = "mixer-path fwd+bwd tokens/sec at B16 L1024 H8 d64 (prologue, epilogue, order scan)"
MIXER_WORK = {
    "prologue_forward": 2 * 256 + 8 + 2 * 256 + 8,
    "prologue_backward": 2 * 256 + 8 + 2 * 256 + 8 + 2 * 256 + 8,
    "epilogue_forward": 2 * 256 + 4 + 256,
    "epilogue_backward": 3 * 256 + 4 + 2 * 256 + 4,
    "order_forward": 256 + 4 + 256,
    "order_backward": 3 * 256 + 4 + 256 + 4,
}
# Kernels of each step of the mixer workload.
MIXER_KERNELS = {
    "prologue_forward": ["prologue_forward"],
    "prologue_backward": ["prologue_backward", "head_sums"],
    "epilogue_forward": ["epilogue_forward"],
    "epilogue_backward": ["epilogue_backward", "head_sums"],
    "order_forward": ["order_local", "order_carry", "order_apply"],
    "order_backward": ["order_bwd_local", "order_bwd_carry", "order_bwd_apply"],
}


def main_mixer(args):
    import torch

    from mamba4_amd import _lib

    lib = _lib.load()
    check = _lib.check
    B, T, H, D = 16, 1024, 8, 64
    gen = torch.Generator(device="cuda:0").manual_seed(0)
    f32 = dict(dtype=torch.float32, device="cuda:0")

    def rand(*shape):
        return torch.randn(*shape, generator=gen, **f32)

    key, query, value, read = rand(B, T, H, D), rand(B, T, H, D), rand(B, T, H, D), rand(B, T, H, D)
    beta_raw, dt_raw, order_raw = rand(B, T, H), rand(B, T, H), rand(B, T, H) + 2
    variance = rand(B, T, H).abs()
    beta_bias, dt_bias, a_log, conf, skip = rand(H), rand(H), rand(H) * 0.1, rand(H), rand(H)
    floor_raw, previous = rand(H, D), rand(B, H, D)
    log_order = torch.nn.functional.logsigmoid(order_raw)
    e = torch.empty_like
    keys, queries, beta, log_decay, floor, shifted = (e(key), e(query), e(beta_raw), e(dt_raw),
                                                      e(floor_raw), e(previous))
    g = [e(key), e(query), e(beta_raw), e(dt_raw), e(beta_bias), e(dt_bias), e(a_log),
         e(floor_raw), e(previous)]
    out, d_read, d_var, d_value, d_conf, d_skip = e(read), e(read), e(variance), e(value), e(conf), e(skip)
    ordered, d_vals, d_logs = e(value), e(value), e(log_order)
    mix_ws = torch.empty(lib.m4mr_mixer_workspace_bytes(B, T, H), dtype=torch.uint8, device="cuda:0")
    ord_bytes = lib.m4mr_order_workspace_bytes(B, T, H, D, 64)
    ord_ws = torch.empty(ord_bytes, dtype=torch.uint8, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731

    def step():
        check(lib.m4mr_prologue_forward(
            p(key), p(query), p(beta_raw), p(dt_raw), p(beta_bias), p(dt_bias), p(a_log),
            p(floor_raw), p(previous), B, T, H, D, 1.0, 0.25, 1, p(keys), p(queries), p(beta),
            p(log_decay), p(floor), p(shifted), st))
        check(lib.m4mr_prologue_backward(
            p(key), p(query), p(beta_raw), p(dt_raw), p(beta_bias), p(dt_bias), p(a_log),
            p(floor_raw), p(previous), B, T, H, D, 1.0, 1, p(keys), p(queries), p(beta),
            p(log_decay), p(floor), p(shifted), *(p(t) for t in g), p(mix_ws), mix_ws.numel(), st))
        check(lib.m4mr_epilogue_forward(p(read), p(variance), p(value), p(conf), p(skip), B, T, H,
                                        D, p(out), st))
        check(lib.m4mr_epilogue_backward(p(read), p(variance), p(value), p(conf), p(skip), B, T,
                                         H, D, p(out), p(d_read), p(d_var), p(d_value), p(d_conf),
                                         p(d_skip), p(mix_ws), mix_ws.numel(), st))
        check(lib.m4mr_order_forward(p(value), p(log_order), None, B, T, H, D, 64, p(ordered),
                                     p(ord_ws), ord_bytes, st))
        check(lib.m4mr_order_backward(p(value), p(log_order), None, p(ordered), p(out), B, T, H,
                                      D, 64, p(d_vals), p(d_logs), None, p(ord_ws), ord_bytes, st))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(min(args.steps, 10)):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernel_ms = {}
    for name in _lib.kernel_names():
        total, count = _lib.profile_read(name)
        if count:
            kernel_ms[name] = total / count
    _lib.profile_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    seconds = (time.perf_counter() - t0) / args.steps
    token_heads = B * T * H
    parts = {}
    for part, names in MIXER_KERNELS.items():
        ms = sum(kernel_ms.get(n, 0.0) for n in names)
        gbps = MIXER_WORK[part] * token_heads / (ms / 1e3) / 1e9
        parts[part] = {"ms": ms, "achieved_GBps": gbps, "frac": gbps / HBM_PEAK_GBPS}
    dominant = max(parts, key=lambda k: parts[k]["ms"])
    line = {
        "metric": MIXER_METRIC,
        "value": B * T / seconds,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": seconds * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "mixer path, B=16 L=1024 H=8 D=P=64 fp32", "batch": B,
                   "seq_len": T, "heads": H, "key_dim": D, "value_dim": D},
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": parts[dominant]["achieved_GBps"],
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": parts[dominant]["frac"],
            "traffic": None,
            "algorithmic_bytes": MIXER_WORK[dominant] * token_heads,
        },
        "parts": parts,
        "kernel_ms": kernel_ms,
    }
    print(json.dumps(line), flush=True)


MIXER_READ_METRIC = ("mixer memory-path forward tokens/sec at B16 L1024 H8 d64 (prologue, "
                     "memory read and read gating fused)")


def main_mixer_read(args):
    import ctypes

    import torch

    from mamba4_amd import _lib

    lib = _lib.load()
    check = _lib.check
    B, T, H, D = 16, 1024, 8, 64
    gen = torch.Generator(device="cuda:0").manual_seed(0)
    f32 = dict(dtype=torch.float32, device="cuda:0")

    def rand(*shape):
        return torch.randn(*shape, generator=gen, **f32)

    key, query, value = rand(B, T, H, D), rand(B, T, H, D), rand(B, T, H, D)
    beta_raw, dt_raw = rand(B, T, H), rand(B, T, H)
    beta_bias, dt_bias, a_log = rand(H), rand(H) - 2.0, rand(H).abs()
    conf, skip, floor_raw = rand(H).abs() * 0.2, rand(H), rand(H, D)
    count, starts = _lib.start_counts(T, 64)
    e = torch.empty
    output, read = e(B, T, H, D, **f32), e(B, T, H, D, **f32)
    variance, shifted = e(B, T, H, **f32), e(B, H, D, **f32)
    final_s, final_c = e(B, H, D, D, **f32), e(B, H, D, D, **f32)
    solved, factors = e(B, T, H, D, **f32), e(B, T, H, _lib.FACTOR_FLOATS, **f32)
    start_s, start_c = e(B, H, starts, D, D, **f32), e(B, H, count, D, D, **f32)
    keys, queries, beta, log_decay = e(B, T, H, D, **f32), e(B, T, H, D, **f32), e(B, T, H, **f32), e(B, T, H, **f32)
    floor = e(H, D, **f32)
    params = _lib.MixerParams(beta_bias.data_ptr(), dt_bias.data_ptr(), a_log.data_ptr(),
                              floor_raw.data_ptr(), None, conf.data_ptr(), skip.data_ptr(),
                              1.0, 0.25, 1)
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731

    def fused():
        check(lib.m4mr_mixer_forward(
            p(key), p(value), p(query), p(beta_raw), p(dt_raw), ctypes.byref(params), None, None,
            B, T, H, D, 64, p(output), p(read), p(variance), p(beta), p(log_decay), p(floor),
            p(final_s), p(final_c), p(solved),
            p(factors), p(start_s), p(start_c), p(shifted), st))

    def separate():
        check(lib.m4mr_prologue_forward(
            p(key), p(query), p(beta_raw), p(dt_raw), p(beta_bias), p(dt_bias), p(a_log),
            p(floor_raw), None, B, T, H, D, 1.0, 0.25, 1, p(keys), p(queries), p(beta),
            p(log_decay), p(floor), p(shifted), st))
        check(lib.m4mr_forward(
            p(keys), p(value), p(queries), p(beta), p(log_decay), p(floor), None, None, B, T, H,
            D, 64, p(read), p(variance), p(final_s), p(final_c), p(solved), p(factors),
            p(start_s), p(start_c), st))
        check(lib.m4mr_epilogue_forward(p(read), p(variance), p(value), p(conf), p(skip), B, T,
                                        H, D, p(output), st))

    # The backward legs: epilogue VJP, memory-read VJP, prologue VJP.
    d_out = rand(B, T, H, D)
    d_read, d_var, d_val_skip = e(B, T, H, D, **f32), e(B, T, H, **f32), e(B, T, H, D, **f32)
    d_conf, d_skip = e(H, **f32), e(H, **f32)
    g_mem = [e(B, T, H, D, **f32), e(B, T, H, D, **f32), e(B, T, H, D, **f32), e(B, T, H, **f32),
             e(B, T, H, **f32), e(H, D, **f32), e(B, H, D, D, **f32), e(B, H, D, D, **f32)]
    g_pro = [e(B, T, H, D, **f32), e(B, T, H, D, **f32), e(B, T, H, **f32), e(B, T, H, **f32),
             e(H, **f32), e(H, **f32), e(H, **f32), e(H, D, **f32)]
    bwd_bytes = lib.m4mr_backward_workspace_bytes(B, T, H, D, 64)
    bwd_ws = torch.empty(bwd_bytes, dtype=torch.uint8, device="cuda:0")
    mix_bytes = lib.m4mr_mixer_workspace_bytes(B, T, H)
    mix_ws = torch.empty(mix_bytes, dtype=torch.uint8, device="cuda:0")

    def backward(fused_memread):
        check(lib.m4mr_epilogue_backward(p(read), p(variance), p(value), p(conf), p(skip), B, T,
                                         H, D, p(d_out), p(d_read), p(d_var), p(d_val_skip),
                                         p(d_conf), p(d_skip), p(mix_ws), mix_bytes, st))
        tail = (B, T, H, D, 64, p(solved), p(factors), p(start_s), p(start_c), p(d_read),
                p(d_var), None, None, *(p(g) for g in g_mem), p(bwd_ws), bwd_bytes, st)
        if fused_memread:
            check(lib.m4mr_mixer_backward(p(key), p(value), p(query), p(beta), p(log_decay),
                                          p(floor), None, 1, *tail))
        else:
            check(lib.m4mr_backward(p(keys), p(value), p(queries), p(beta), p(log_decay),
                                    p(floor), *tail))
        check(lib.m4mr_prologue_backward(
            p(key), p(query), p(beta_raw), p(dt_raw), p(beta_bias), p(dt_bias), p(a_log),
            p(floor_raw), None, B, T, H, D, 1.0, 1, p(g_mem[0]), p(g_mem[2]), p(g_mem[3]),
            p(g_mem[4]), p(g_mem[5]), None, *(p(g) for g in g_pro), None, p(mix_ws), mix_bytes,
            st))
        g_mem[1].add_(d_val_skip)  # the value's two paths meet

    # The whole mixer VJP in one launch sequence (m4mr_mixer_read_backward).
    mr_bytes = lib.m4mr_mixer_read_backward_workspace_bytes(B, T, H, D, 64)
    mr_ws = torch.empty(mr_bytes, dtype=torch.uint8, device="cuda:0")
    g_mr = [e(B, T, H, D, **f32), e(B, T, H, D, **f32), e(B, T, H, D, **f32), e(B, T, H, **f32),
            e(B, T, H, **f32), e(H, **f32), e(H, **f32), e(H, **f32), e(H, D, **f32)]
    g_mr_tail = [e(H, **f32), e(H, **f32), e(B, H, D, D, **f32), e(B, H, D, D, **f32)]

    def fused_backward():
        check(lib.m4mr_mixer_read_backward(
            p(key), p(value), p(query), p(dt_raw), ctypes.byref(params), B, T, H, D, 64, p(read),
            p(variance), p(beta), p(log_decay), p(floor), p(solved), p(factors), p(start_s),
            p(start_c), p(d_out), None, None, None, None, *(p(g) for g in g_mr), None,
            *(p(g) for g in g_mr_tail), p(mr_ws), mr_bytes, st))

    def fused_train():
        fused()
        fused_backward()

    def partial_train():
        fused()
        backward(True)

    def separate_train():
        separate()
        backward(False)

    def timed(fn, steps):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    # The separate path's state walk is the fused walk too (the fused entry
    # point always takes it).  The two are timed in alternation, best of
    # three each, so that neither gets the colder clocks of the first run.
    os.environ["M4MR_STATE_WALK"] = "fused"
    runs = [(timed(fused, args.steps), timed(separate, args.steps)) for _ in range(3)]
    seconds = min(r[0] for r in runs)
    separate_seconds = min(r[1] for r in runs)
    train = [(timed(fused_train, args.steps), timed(separate_train, args.steps),
              timed(partial_train, args.steps)) for _ in range(3)]
    train_seconds = min(r[0] for r in train)
    separate_train_seconds = min(r[1] for r in train)
    partial_train_seconds = min(r[2] for r in train)
    # Per-kernel milliseconds per fused training step (library timers).
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    profiled = min(args.steps, 10)
    for _ in range(profiled):
        fused_train()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernel_ms = {}
    for name in _lib.kernel_names():
        total, count = _lib.profile_read(name)
        if count:
            kernel_ms[name] = total / profiled
    _lib.profile_reset()
    line = {
        "metric": MIXER_READ_METRIC,
        "value": B * T / seconds,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": seconds * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "mixer memory path forward, B=16 L=1024 H=8 D=P=64 fp32",
                   "batch": B, "seq_len": T, "heads": H, "key_dim": D, "value_dim": D},
        "separate_ms_per_step": separate_seconds * 1e3,
        "fused_speedup": separate_seconds / seconds,
        "train_ms_per_step": train_seconds * 1e3,
        "separate_train_ms_per_step": separate_train_seconds * 1e3,
        "train_speedup": separate_train_seconds / train_seconds,
        "partial_train_ms_per_step": partial_train_seconds * 1e3,
        "train_kernel_ms": kernel_ms,
    }
    print(json.dumps(line), flush=True)


MAMBA3_METRIC = ("Mamba-3 fused scan fwd+bwd tokens/sec at B16 L1024 H24 P64 N128 A32 "
                 "(125M mixer shape); % fp32 MFMA peak")
MAMBA3_BF16_METRIC = ("Mamba-3 fused scan fwd+bwd tokens/sec, bf16 model, at B16 L1024 H24 P64 "
                      "N128 A32 (125M mixer shape); % bf16 MFMA peak")
# Algorithmic flop per (chunk of 64 tokens, head) of each scan kernel at
# N = 128, P = 64: 2 flop per multiply-add of the products the algorithm
# needs, causal products counted over the 2080 (t, s <= t) pairs only.
MAMBA3_FLOP = {
    "m3_walk": 2 * 128 * 64 * 64,                                # K^T (u V)
    "m3_out": 2 * (2080 * 128 + 64 * 128 * 64 + 2080 * 64),      # Q K^T, Q S0, (S o W) V
    "m3_walk_bwd": 2 * 128 * 64 * 64,                            # Q^T (e^p dY)
    "m3_grad": 2 * (3 * 2080 * 128 + 4 * 64 * 128 * 64 + 2 * 2080 * 64),
}


def mamba3_cpu_baseline(host):
    """oracle.mamba3 (float64 NumPy) forward and backward on batch row 0."""
    from oracle import mamba3 as oracle

    row = {n: (v[:1] if n not in ("q_bias", "k_bias") else v) for n, v in host.items()
           if n != "d_y"}
    start = time.perf_counter()
    oracle.forward(*(row[n] for n in oracle.ARGS))
    oracle.backward(*(row[n] for n in oracle.ARGS), host["d_y"][:1], None)
    seconds = time.perf_counter() - start
    _, T, H = row["dt"].shape
    return {
        "value": T / seconds,
        "unit": "tokens/s",
        "cores": int(os.environ.get("OPENBLAS_NUM_THREADS", CORES)),
        "kind": "port",
        "sample": (f"oracle.mamba3 fwd+bwd in float64 NumPy on batch row 0 of the workload "
                   f"(B=1, L={T}, H={H}; 1/16 of the step), {seconds:.1f} s"),
    }


def main_mamba3(args, bf16=False):
    import torch

    from mamba4_amd import _lib
    from mamba4_amd.inputs import MAMBA3_ARGS, mamba3_inputs

    lib = _lib.load()
    check = _lib.check
    B, T, H, N, P, A = 16, 1024, 24, 128, 64, 32
    NC = (T + 63) // 64
    host = mamba3_inputs(batch=B, length=T, heads=H, dim=N, width=P, angle_count=A, seed=0)
    host["d_y"] = np.random.default_rng(1).normal(size=host["x"].shape)
    dev = {n: torch.tensor(np.asarray(v, np.float32), device="cuda:0") for n, v in host.items()}
    rows = ("c", "b", "x", "d_y")
    if bf16:
        for n in rows:
            dev[n] = dev[n].to(torch.bfloat16)
    forward = lib.m3s_forward_bf16 if bf16 else lib.m3s_forward
    backward = lib.m3s_backward_bf16 if bf16 else lib.m3s_backward
    peak = BF16_PEAK_TFLOPS if bf16 else FP32_PEAK_TFLOPS
    f32 = dict(dtype=torch.float32, device="cuda:0")
    y = torch.empty(B, T, H * P, dtype=dev["x"].dtype, device="cuda:0")
    final = torch.empty(B, H, N, P, **f32)
    starts = torch.empty(B, H, NC, 8192, **f32)
    phases = torch.empty(B, H, NC, 64, **f32)
    grads = [torch.empty(dev[n].shape, dtype=dev[n].dtype if n == "x" else torch.float32,
                         device="cuda:0") for n in MAMBA3_ARGS]
    nbytes = lib.m3s_backward_workspace_bytes(B, T, H, N, P, A)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    st = torch.cuda.current_stream().cuda_stream
    ins = [dev[n].data_ptr() for n in MAMBA3_ARGS]
    dims = (B, T, H, N, P, A)

    def step():
        check(forward(*ins, *dims, y.data_ptr(), final.data_ptr(), starts.data_ptr(),
                      phases.data_ptr(), st))
        check(backward(*ins, *dims, starts.data_ptr(), phases.data_ptr(), dev["d_y"].data_ptr(),
                       None, *(g.data_ptr() for g in grads), ws.data_ptr(), nbytes, st))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_select(None)
    _lib.profile_enable(True)
    for _ in range(min(args.steps, 10)):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernel_ms = {}
    for name in _lib.kernel_names():
        total, count = _lib.profile_read(name)
        if count:
            kernel_ms[name] = total / count
    _lib.profile_reset()
    dominant = max(MAMBA3_FLOP, key=lambda k: kernel_ms.get(k, 0.0))
    # Timed region: events only on the dominant kernel's launches.
    _lib.profile_select(dominant)
    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    seconds = (time.perf_counter() - t0) / args.steps
    _lib.profile_enable(False)
    total, count = _lib.profile_read(dominant)
    _lib.profile_reset()
    _lib.profile_select(None)
    dom_ms = total / count
    units = B * NC * H
    achieved = MAMBA3_FLOP[dominant] * units / (dom_ms / 1e3) / 1e12
    kernels = {}
    for name, flop in MAMBA3_FLOP.items():
        ms = kernel_ms.get(name)
        if ms:
            rate = flop * units / (ms / 1e3) / 1e12
            kernels[name] = {"ms": ms, "TFLOPs": rate, "frac": rate / peak}
    line = {
        "metric": MAMBA3_BF16_METRIC if bf16 else MAMBA3_METRIC,
        "value": B * T / seconds,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": seconds * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if bf16 else "f32",
        "data": "synthetic",
        "config": {"workload": "mamba3 scan fwd+bwd, B=16 L=1024 H=24 P=64 N=128 A=32 "
                               + ("bf16 model (bf16 operands, f32 accumulation)" if bf16
                                  else "fp32"),
                   "batch": B, "seq_len": T, "heads": H, "state_dim": N, "head_dim": P,
                   "angles": A},
        "roofline": {
            "kernel": dominant,
            "bound": "mfma",
            "achieved": achieved,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": achieved / peak,
            "traffic": None if bf16 else measured_traffic(dominant, MAMBA3_TRAFFIC_SUMMARY),
            "traffic_unit": "B per launch (rocprofv3, profiles/mamba3_scan_hbm_traffic.md)",
            "algorithmic_flop": MAMBA3_FLOP[dominant] * units,
        },
        "kernels": kernels,
        "kernel_ms": kernel_ms,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = mamba3_cpu_baseline(host)
    print(json.dumps(line), flush=True)


def _best_seconds(fn, reps=10):
    """Shortest of `reps` timed calls of fn (after two untimed ones)."""
    import torch

    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        stop.record()
        stop.synchronize()
        best = min(best, start.elapsed_time(stop) / 1e3)
    return best


def stream_probes_gbps(nbytes):
    """Write-only and read-only rates over an nbytes float32 buffer: torch's
    fill_ (a vectorized store-only kernel) and row sums over 4096-float rows
    (torch's fastest read-only reduction here; a whole-buffer sum reads at
    about 4 TB/s), best of ten.  What a library kernel reaches on this box
    for the factor store and load, next to the 8 TB/s read+write peak."""
    import torch

    buf = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda:0")
    rows = buf[: (nbytes // 4) // 4096 * 4096].view(-1, 4096)
    out = torch.empty(rows.shape[0], dtype=torch.float32, device="cuda:0")
    write = nbytes / _best_seconds(lambda: buf.fill_(1.0)) / 1e9
    read = rows.numel() * 4 / _best_seconds(lambda: torch.sum(rows, dim=1, out=out)) / 1e9
    del buf, rows, out
    return write, read


def copy_bandwidth_gbps():
    """Read+write bandwidth of a 2 GiB device-to-device copy (torch copy_)."""
    import torch

    n = 1 << 29
    a = torch.empty(n, dtype=torch.float32, device="cuda:0").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    start.record()
    for _ in range(reps):
        b.copy_(a)
    stop.record()
    torch.cuda.synchronize()
    seconds = start.elapsed_time(stop) / 1e3 / reps
    del a, b
    return 2 * n * 4 / seconds / 1e9


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def median_seconds(fn, runs=5):
    """One warm-up call, then the median wall time of `runs` calls."""
    fn()
    times = []
    for _ in range(runs):
        start = time.perf_counter()
        fn()
        times.append(time.perf_counter() - start)
    return float(np.median(times))


def oracle_legs(data):
    """Median seconds and token-head rates of the NumPy oracle (float32,
    chunk 64) forward and forward+backward on `data`."""
    from oracle import memread as oracle

    args = [data[n] for n in NAMES]

    def fwd():
        return oracle.forward(*args, chunk=64, dtype=np.float32)

    def fwd_bwd():
        _, res = fwd()
        oracle.backward(res, data["d_output"], data["d_variance"])

    B, T, H, _ = data["keys"].shape
    legs = {}
    for label, fn in (("fwd", fwd), ("fwd_bwd", fwd_bwd)):
        seconds = median_seconds(fn)
        legs[label] = {"median_s": seconds, "token_heads_per_s": B * T * H / seconds}
    return legs


def cpu_baseline(data, workload, config0=True):
    """The CPU baseline of the plan in BASELINE.md: this build's NumPy
    restatement of the reference algorithm (oracle.memread, float32) on this
    host, BLAS on every core, one warm-up then the median of five runs,
    forward and forward+backward.  Config 0 runs in full.  The benchmarked
    workload runs on one whole batch row (B=1, every head, the full length):
    the oracle's cost is linear in the batch, so the row's tokens/s is the
    CPU's tokens/s for the whole batch, measured rather than scaled."""
    sample = {n: (a[:1] if n != "floor" else a) for n, a in data.items()}
    legs = {}
    if config0:
        from mamba4_amd.inputs import workload_inputs

        for label, leg in oracle_legs(workload_inputs("config0", seed=0, cotangents=True)).items():
            legs["config0_" + label + "_tokens_per_s"] = leg["token_heads_per_s"]
    sampled = oracle_legs(sample)
    _, T, H, _ = sample["keys"].shape
    for label, leg in sampled.items():
        legs[workload + "_" + label + "_tokens_per_s"] = T / leg["median_s"]
    threads = os.environ.get("OPENBLAS_NUM_THREADS")
    return {
        "value": T / sampled["fwd_bwd"]["median_s"],
        "unit": "tokens/s",
        "cores": int(threads or CORES),
        "kind": "port",
        "sample": (
            f"oracle.memread fwd+bwd in float32 NumPy on batch row 0 of the {workload} "
            f"workload (B=1, L={T}, H={H}: {T} tokens), median of 5 after 1 warm-up "
            f"({sampled['fwd_bwd']['median_s']:.3f} s per row); config 0 in full; "
            f"BLAS threads = {threads}, {CORES} cores in the affinity mask"
        ),
        "cpu_model": cpu_model(),
        "legs": legs,
    }


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one MI355X: the memory read shards over (batch, head) with "
            "no communication, and this build runs on one GPU only; use --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from mamba4_amd import _lib
    from mamba4_amd.inputs import workload_inputs

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(2)
    if args.workload == "config4":
        return main_decode(args)
    if args.workload == "mixer_read":
        return main_mixer_read(args)
    if args.workload == "mixer":
        return main_mixer(args)
    if args.workload in ("mamba3", "mamba3_bf16"):
        return main_mamba3(args, bf16=args.workload == "mamba3_bf16")
    if args.workload == "ref125m":
        from mamba4_amd.inputs import reference_benchmark_inputs

        data = reference_benchmark_inputs(seed=0)
    else:
        data = workload_inputs(args.workload, seed=0, cotangents=True)
    problem = Problem(data, args.chunk, bf16_inputs=args.workload == "config3")
    B, T, H, P = problem.B, problem.T, problem.H, problem.P
    token_heads = B * T * H

    for _ in range(args.warmup):
        problem.forward()
        problem.backward()
    torch.cuda.synchronize()

    # Per-kernel breakdown from an untimed pass with every launch bracketed
    # by HIP events; it names the dominant kernel.
    _lib.profile_reset()
    _lib.profile_select(None)
    _lib.profile_enable(True)
    for _ in range(min(args.steps, 10)):
        problem.forward()
        problem.backward()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernels = {}
    for name in _lib.kernel_names():
        total, count = _lib.profile_read(name)
        if count:
            kernels[name] = total / count
    _lib.profile_reset()
    dominant = max(kernels, key=kernels.get)

    # Timed region: only the dominant kernel carries events, so the step time
    # is not stretched by markers between the other launches.
    _lib.profile_select(dominant)
    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        problem.forward()
        problem.backward()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    _lib.profile_enable(False)
    seconds = (t1 - t0) / args.steps
    total, count = _lib.profile_read(dominant)
    kernels[dominant] = total / count
    _lib.profile_reset()
    _lib.profile_select(None)
    # The factor kernel without the factor store (a forward that takes no
    # gradient), timed on its own after the timed region.
    _lib.profile_select("fwd_factor")
    _lib.profile_enable(True)
    for _ in range(min(args.steps, 10)):
        problem.forward(store=False)
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    total, count = _lib.profile_read("fwd_factor")
    factor_only_ms = total / count
    _lib.profile_reset()
    _lib.profile_select(None)
    factor_s = kernels["fwd_factor"] / 1e3
    resolve_s = kernels["factored_solve"] / 1e3
    store_gbps = FACTOR_BYTES * token_heads / factor_s / 1e9
    load_gbps = RESOLVE_BYTES * token_heads / resolve_s / 1e9
    copy_gbps = copy_bandwidth_gbps()
    write_probe, read_probe = stream_probes_gbps(FACTOR_BYTES * token_heads)

    vs_baseline = None
    if args.workload == "config3":
        metric = CONFIG3_METRIC
        workload = ("config3: memory-read fwd+bwd, B=32 L=1024 H=12 D=P=64, bf16 q/k/v read "
                    "natively (fp32 arithmetic), lambda = sigmoid(N(4,1)), floor 1e-2")
    elif args.workload == "ref125m":
        metric = REF125M_METRIC
        workload = ("ref125m: memory-read fwd+bwd at the reference's published shape, B=16 "
                    "L=1024 H=12 D=64 P=128 fp32, the inputs and projected-loss cotangents of "
                    "scripts/kernel_benchmark.py:37-47,214-224")
        vs_baseline = B * T / seconds / REF125M_TPU_TOKENS_PER_S
    else:
        metric = METRIC
        workload = "config2: memory-read fwd+bwd, B=16 L=1024 H=8 D=P=64 fp32, floor 1e-2"
    # Contraction kernels' flop counts are per token-head at P = 64; the
    # factor kernels' work does not depend on P.
    p_free = P == 64 or dominant in ("fwd_factor", "factored_solve")
    line = {
        "metric": metric,
        "value": B * T / seconds,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": seconds * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": vs_baseline,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "batch": B,
            "seq_len": T,
            "heads": H,
            "key_dim": 64,
            "value_dim": P,
            "chunk": args.chunk,
        },
        # The committed rocprof traffic summary is for config 2.
        "roofline": (roofline(dominant, kernels[dominant], token_heads,
                              traffic=args.workload == "config2") if p_free else None),
        "factorization_fp32": {
            "kernel": "fwd_factor",
            "achieved_tflops": CHOLESKY_FLOP * token_heads / factor_s / 1e12,
            "peak_tflops": FP32_PEAK_TFLOPS,
            "frac": CHOLESKY_FLOP * token_heads / factor_s / 1e12 / FP32_PEAK_TFLOPS,
        },
        # The same kernel without the factor store: the factorization alone.
        "factor_only_ms": factor_only_ms,
        "factorization_fp32_store_free": {
            "kernel": "fwd_factor (factors = NULL)",
            "achieved_tflops": CHOLESKY_FLOP * token_heads / factor_only_ms / 1e9,
            "peak_tflops": FP32_PEAK_TFLOPS,
            "frac": CHOLESKY_FLOP * token_heads / factor_only_ms / 1e9 / FP32_PEAK_TFLOPS,
        },
        "factor_streaming_hbm": {
            "store_GBps": store_gbps,
            "store_frac": store_gbps / HBM_PEAK_GBPS,
            "load_GBps": load_gbps,
            "load_frac": load_gbps / HBM_PEAK_GBPS,
            "copy_kernel_GBps": copy_gbps,
            "write_probe_GBps": write_probe,
            "store_frac_of_write_probe": store_gbps / write_probe,
            "read_probe_GBps": read_probe,
            "load_frac_of_read_probe": load_gbps / read_probe,
        },
        "kernel_ms": kernels,
        "kernel_roofline": ({k: roofline(k, v, token_heads, traffic=False)["frac"]
                             for k, v in kernels.items()} if P == 64 else None),
    }
    if args.workload == "ref125m":
        line["baseline"] = {
            "value": REF125M_TPU_TOKENS_PER_S,
            "unit": "tokens/s",
            "hardware": "1x TPU v4",
            "source": "lm/results/speed-125m/bench-kernels.json:291 (67.98 ms fused fwd+bwd)",
        }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(data, args.workload,
                                            config0=args.workload == "config2")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
