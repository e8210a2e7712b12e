"""selective_diagnostics on the GPU (m4mr_diagnostics) against the oracle.

The eigenvalue extremes come from a float64 Jacobi iteration on the float32
state, rounded to float32: they are checked to 2e-7 of themselves (fp32
rounding is 6e-8) plus 1e-10 of the state's largest eigenvalue, and the
condition number to 5e-7 relative; the finiteness flag, the cross maximum
and the floor range are exact.
"""

import numpy as np
import pytest
import torch

from oracle import memread as oracle
from tests.gpu_helpers import announce, run_gpu

pytestmark = pytest.mark.gpu


def _diagnose(evidence, cross, floor):
    from mamba4_amd import SelectiveState, selective_diagnostics

    dev = torch.device("cuda:0")
    state = SelectiveState(torch.tensor(evidence, dtype=torch.float32, device=dev),
                           torch.tensor(cross, dtype=torch.float32, device=dev))
    got = selective_diagnostics(state, torch.tensor(floor, dtype=torch.float32, device=dev))
    torch.cuda.synchronize()
    return {k: v.item() for k, v in got.items()}


def _check(got, want, scale):
    assert set(got) == set(oracle.DIAGNOSTIC_KEYS)
    for key in ("precision_min_eigenvalue", "precision_max_eigenvalue"):
        assert abs(got[key] - want[key]) <= 2e-7 * abs(want[key]) + 1e-10 * scale, (
            key, got[key], want[key])
    assert got["precision_max_condition"] == pytest.approx(want["precision_max_condition"], rel=5e-7)
    assert got["state_all_finite"] == want["state_all_finite"]
    for key in ("cross_max_abs", "floor_min", "floor_max"):
        assert got[key] == np.float32(want[key]), key


def _known_state(seed, batch, heads, dim, value_dim, low=1e-3, high=50.0):
    rng = np.random.default_rng(seed)
    mu = np.exp(rng.uniform(np.log(low), np.log(high), size=(batch, heads, dim)))
    q, _ = np.linalg.qr(rng.normal(size=(batch, heads, dim, dim)))
    precision = np.einsum("bhij,bhj,bhkj->bhik", q, mu, q)
    floor = rng.uniform(0.01, 0.5, size=(heads, dim)).astype(np.float32)
    evidence = (precision - floor[None, :, :, None] * np.eye(dim)).astype(np.float32)
    cross = rng.normal(size=(batch, heads, value_dim, dim)).astype(np.float32)
    return evidence, cross, floor


@pytest.mark.parametrize("dim", [1, 2, 17, 63, 64])
def test_diagnostics_match_oracle_on_known_spectra(gpu_lib, dim):
    announce(f"selective_diagnostics known spectra D={dim}")
    evidence, cross, floor = _known_state(dim, 3, 4, dim, 5)
    want = oracle.diagnostics(evidence, cross, floor)
    _check(_diagnose(evidence, cross, floor), want, want["precision_max_eigenvalue"])


def test_diagnostics_of_a_forward_end_state(gpu_lib):
    """The end state of a config-2-like forward (unit keys, sigmoid gates,
    floor 1e-2), as the mixer probes it (lm/models/mamba4.py:290-310)."""
    from mamba4_amd.inputs import synthetic_inputs

    data = synthetic_inputs(2, 256, 4, seed=42)
    announce("selective_diagnostics of a forward end state B2 T256 H4 D64")
    got = run_gpu(data, chunk=64)
    want = oracle.diagnostics(got["evidence"], got["cross"], data["floor"])
    _check(_diagnose(got["evidence"], got["cross"], data["floor"]), want,
           want["precision_max_eigenvalue"])


def test_diagnostics_symmetrise_broadcast_and_flag_non_finite(gpu_lib):
    announce("selective_diagnostics: skew part, shared floor, planted NaN and inf")
    evidence, cross, floor = _known_state(7, 2, 3, 12, 4)
    rng = np.random.default_rng(8)
    skew = rng.normal(size=evidence.shape).astype(np.float32)
    skew = skew - np.swapaxes(skew, -1, -2)
    want = oracle.diagnostics(evidence + skew, cross, floor)
    _check(_diagnose(evidence + skew, cross, floor), want, want["precision_max_eigenvalue"])
    # A floor shared by every head ([D]).
    shared = floor[0]
    want = oracle.diagnostics(evidence, cross, shared)
    _check(_diagnose(evidence, cross, shared), want, want["precision_max_eigenvalue"])
    # NaN in cross: not finite, NaN maximum, eigenvalues unaffected.
    bad = cross.copy()
    bad[1, 2, 0, 5] = np.nan
    got = _diagnose(evidence, bad, floor)
    assert got["state_all_finite"] is False and np.isnan(got["cross_max_abs"])
    assert np.isfinite(got["precision_min_eigenvalue"])
    # inf in evidence: not finite, NaN eigenvalue extremes and condition.
    bad = evidence.copy()
    bad[0, 1, 3, 4] = np.inf
    got = _diagnose(bad, cross, floor)
    assert got["state_all_finite"] is False
    assert np.isnan(got["precision_min_eigenvalue"]) and np.isnan(got["precision_max_condition"])
    assert np.isfinite(got["cross_max_abs"])


def test_diagnostics_rejects_wide_states(gpu_lib):
    from mamba4_amd import SelectiveState, selective_diagnostics

    dev = torch.device("cuda:0")
    state = SelectiveState(torch.zeros(1, 1, 65, 65, device=dev), torch.zeros(1, 1, 4, 65, device=dev))
    with pytest.raises(ValueError):
        selective_diagnostics(state, torch.ones(65, device=dev))
