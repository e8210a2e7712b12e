// Spectral and finiteness probes of the final selective precision: restates
// selective_diagnostics (lm/kernels/mamba4.py:358-376).
//
// diag_eigen_kernel: one 64-lane wave per (batch, head) state.  The
// symmetrised precision (E + E^T) / 2 + diag(floor) goes to LDS in float64
// (exact for float32 inputs) and a cyclic Jacobi iteration diagonalises it:
// each round rotates n/2 disjoint index pairs (the round-robin "circle"
// ordering, so a sweep of n - 1 rounds meets every pair once), lane k
// computing pair k's rotation, then every lane applying all of the round's
// rotations to its column (rows p, q) and then to its row (columns p, q),
// and lane k finally setting a_pp - t a_pq, a_qq + t a_pq and a zero a_pq
// (Rutishauser's form, which keeps the diagonal from collecting the
// rotations' rounding).  Sweeps stop once the off-diagonal mass is below
// 2^-100 of the diagonal's (or after kMaxSweeps, so every state ends); the
// extreme diagonal entries are the extreme eigenvalues, rounded to float32.
// In float32 the same iteration lands 1e-7 to 2e-6 of the largest
// eigenvalue off float64 eigvalsh on 64-wide states; in float64 the
// result is float64 eigvalsh's to within the final rounding.  This is a
// monitoring probe, off every hot path.
// The same pass takes the state's finiteness and the cross statistics'
// largest magnitude.
//
// diag_summary_kernel: one block reduces the per-state values and the floor.
#include "common.hpp"

namespace m4 {

constexpr int kMaxSweeps = 40;

__device__ __forceinline__ float wave_min(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fminf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

// Pair k of round r of the circle ordering of m (even) indices: index 0
// stays, 1..m-1 turn one place per round.
__device__ __forceinline__ void circle_pair(int k, int r, int m, int& p, int& q) {
  const int ring = m - 1;
  if (k == 0) {
    p = 0;
    q = r % ring + 1;
  } else {
    p = (r + k) % ring + 1;
    q = (r - k + ring) % ring + 1;
  }
}

// per_state[4 bh + 0..3] = min eigenvalue, max eigenvalue (both NaN when the
// precision has a non-finite entry, as eigvalsh gives), 1 if every entry of
// the state (evidence and cross) is finite else 0, max |cross| (NaN if a
// cross entry is NaN, as jnp.max gives).
__global__ __launch_bounds__(64) void diag_eigen_kernel(const float* __restrict__ evidence,
                                                        const float* __restrict__ cross,
                                                        const float* __restrict__ floor, int H,
                                                        int D, int P, float* __restrict__ per_state) {
  __shared__ double a[64][65];
  __shared__ double rc[32], rs[32], rt[32];
  const int bh = blockIdx.x, h = bh % H, lane = threadIdx.x;
  const float* E = evidence + (long)bh * D * D;
  bool finite = true, prec_finite = true, cross_nan = false;
  if (lane < D) {
    const float fl = floor[h * D + lane];
    prec_finite = isfinite(fl);
    for (int j = 0; j < D; ++j) {
      const float x = E[lane * D + j], y = E[j * D + lane];
      finite = finite && isfinite(x);
      a[lane][j] = 0.5 * ((double)x + (double)y) + (j == lane ? (double)fl : 0.0);
    }
  }
  prec_finite = prec_finite && finite;
  float cmax = 0.f;
  const float* C = cross + (long)bh * P * D;
  for (long i = lane; i < (long)P * D; i += 64) {
    const float v = C[i];
    finite = finite && isfinite(v);
    cross_nan = cross_nan || isnan(v);
    cmax = fmaxf(cmax, fabsf(v));
  }
  // Uniform over the wave from here on.
  prec_finite = wave_min(prec_finite ? 1.f : 0.f) > 0.f;
  __syncthreads();
  const int m = D + (D & 1);  // an odd width pairs its last index with a dummy
  for (int sweep = 0; sweep < kMaxSweeps && D > 1 && prec_finite; ++sweep) {
    double off = 0.0, dia = 0.0;
    if (lane < D)
      for (int j = 0; j < D; ++j) {
        const double v = a[lane][j];
        if (j == lane)
          dia += v * v;
        else
          off += v * v;
      }
    off = wave_sum(off);
    dia = wave_sum(dia);
    // Uniform over the wave (kMaxSweeps bounds the loop regardless).
    if (!(off > 0x1p-100 * dia)) break;
    for (int r = 0; r < m - 1; ++r) {
      double app = 0.0, aqq = 0.0, apq0 = 0.0;
      if (lane < m / 2) {
        int p, q;
        circle_pair(lane, r, m, p, q);
        double c = 1.0, s = 0.0, t = 0.0;
        if (p < D && q < D) {
          app = a[p][p];
          aqq = a[q][q];
          apq0 = a[p][q];
          if (apq0 != 0.0) {
            const double tau = (aqq - app) / (2.0 * apq0);
            // t = tan of the angle that zeroes a_pq (the smaller root);
            // 1 / (2 tau) once tau^2 would overflow.
            t = fabs(tau) < 1e150 ? copysign(1.0, tau) / (fabs(tau) + sqrt(1.0 + tau * tau))
                                  : 0.5 / tau;
            c = 1.0 / sqrt(1.0 + t * t);
            s = t * c;
          }
        }
        rc[lane] = c;
        rs[lane] = s;
        rt[lane] = t;
      }
      __syncthreads();
      // Rows p, q of this lane's column (A <- J^T A), then columns p, q of
      // its row (A <- A J): the round's pairs are disjoint, so their
      // rotations commute.
      if (lane < D)
        for (int k = 0; k < m / 2; ++k) {
          int p, q;
          circle_pair(k, r, m, p, q);
          if (p < D && q < D) {
            const double c = rc[k], s = rs[k], x = a[p][lane], y = a[q][lane];
            a[p][lane] = c * x - s * y;
            a[q][lane] = s * x + c * y;
          }
        }
      __syncthreads();
      if (lane < D)
        for (int k = 0; k < m / 2; ++k) {
          int p, q;
          circle_pair(k, r, m, p, q);
          if (p < D && q < D) {
            const double c = rc[k], s = rs[k], x = a[lane][p], y = a[lane][q];
            a[lane][p] = c * x - s * y;
            a[lane][q] = s * x + c * y;
          }
        }
      __syncthreads();
      // The pair's own entries, from the values the round started with
      // (only this pair's rotation touches a_pp, a_qq and a_pq).
      if (lane < m / 2) {
        int p, q;
        circle_pair(lane, r, m, p, q);
        if (p < D && q < D && rt[lane] != 0.0) {
          a[p][p] = app - rt[lane] * apq0;
          a[q][q] = aqq + rt[lane] * apq0;
          a[p][q] = 0.0;
          a[q][p] = 0.0;
        }
      }
      __syncthreads();
    }
  }
  const float ev = lane < D ? (float)a[lane][lane] : 0.f;
  const float lo = wave_min(lane < D ? ev : INFINITY), hi = wave_max(lane < D ? ev : -INFINITY);
  // A NaN eigenvalue reads as NaN in both extremes (fminf / fmaxf drop it).
  const bool nan_ev = !prec_finite || wave_max(isnan(ev) ? 1.f : 0.f) > 0.f;
  const bool all_finite = wave_min(finite ? 1.f : 0.f) > 0.f;
  const bool any_cross_nan = wave_max(cross_nan ? 1.f : 0.f) > 0.f;
  cmax = wave_max(cmax);
  if (lane == 0) {
    per_state[4 * bh + 0] = nan_ev ? NAN : lo;
    per_state[4 * bh + 1] = nan_ev ? NAN : hi;
    per_state[4 * bh + 2] = all_finite ? 1.f : 0.f;
    per_state[4 * bh + 3] = any_cross_nan ? NAN : cmax;
  }
}

// summary[0..6] = min eigenvalue, max eigenvalue, max condition (per state,
// max / max(min, 1e-30)), all finite (1 / 0), max |cross|, min floor, max
// floor (lm/kernels/mamba4.py:368-376).  One 256-thread block.
__global__ __launch_bounds__(256) void diag_summary_kernel(const float* __restrict__ per_state,
                                                           int states, const float* __restrict__ floor,
                                                           int floors, float* __restrict__ summary) {
  __shared__ float part[7][8];
  float lo = INFINITY, hi = -INFINITY, cond = -INFINITY, fin = 1.f, cm = 0.f;
  float flo = INFINITY, fhi = -INFINITY;
  bool nan_ev = false, nan_cross = false, nan_floor = false;
  for (int i = threadIdx.x; i < states; i += 256) {
    const float a = per_state[4 * i], b = per_state[4 * i + 1];
    nan_ev = nan_ev || isnan(a) || isnan(b);
    nan_cross = nan_cross || isnan(per_state[4 * i + 3]);
    lo = fminf(lo, a);
    hi = fmaxf(hi, b);
    cond = fmaxf(cond, b / fmaxf(a, 1e-30f));
    fin = fminf(fin, per_state[4 * i + 2]);
    cm = fmaxf(cm, per_state[4 * i + 3]);
  }
  for (int i = threadIdx.x; i < floors; i += 256) {
    const float f = floor[i];
    nan_floor = nan_floor || isnan(f);
    flo = fminf(flo, f);
    fhi = fmaxf(fhi, f);
  }
  const float vals[7] = {lo, hi, cond, fin, cm, flo, fhi};
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < 7; ++k) {
    const bool is_min = k == 0 || k == 3 || k == 5;
    const float v = is_min ? wave_min(vals[k]) : wave_max(vals[k]);
    if (l == 0) part[k][w] = v;
  }
  const bool any_ev = __syncthreads_or(nan_ev), any_cross = __syncthreads_or(nan_cross);
  const bool any_floor = __syncthreads_or(nan_floor);
  if (threadIdx.x < 7) {
    const int k = threadIdx.x;
    const bool is_min = k == 0 || k == 3 || k == 5;
    float v = part[k][0];
    for (int j = 1; j < 4; ++j) v = is_min ? fminf(v, part[k][j]) : fmaxf(v, part[k][j]);
    // The reference's jnp.min / jnp.max propagate NaN; fminf / fmaxf drop
    // it, so it is put back where the reference would have it.
    if ((k <= 2 && any_ev) || (k == 4 && any_cross) || (k >= 5 && any_floor)) v = NAN;
    summary[k] = v;
  }
}

}  // namespace m4
