// Per-token factorization, solves and factor streaming.
//
// fwd_factor_kernel restates the token loop of _solve_kernel
// (lm/kernels/mamba4_fused.py:116-152): starting from the chunk's start
// evidence it applies each token's gated rank-one update
// E = lam E + beta k k^T (:90-92), factors E + diag(floor) by Cholesky with
// reciprocal pivots (:93-113), solves L L^T y = q (:45-75) and stores the
// packed factor.  One 64-lane wave owns one (batch, head, chunk) sequence;
// lane i holds row i of the evidence and of the working matrix in VGPRs.
// Column j is finished at step j (pivot by readlane, column scaled in
// registers), broadcast through LDS, and its trailing update is a rank-one
// FMA sweep over the row.  The finished factor, kept column-major in LDS
// for the backward substitution, is then streamed to HBM one column (64 - j
// contiguous floats) per coalesced store.
//
// factored_solve_kernel restates _factored_kernel (:155-174): the two
// substitutions with a stored factor, which it stages in LDS with coalesced
// 16-byte loads.
//
// decode_step_kernel restates selective_decode (lm/kernels/mamba4.py:341-355)
// for resident states updated in place.
#include "common.hpp"

namespace m4 {

__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Cholesky of A = a + diag(floor) held as rows on lanes (lane i owns a[0..63]
// of row i), then y = A^-1 q.  On return a[j] (j < i) holds L_ij, a[i] holds
// 1/L_ii and a[j] (j > i) is zero.  colbuf is 64 floats and lcol 64*LDT
// floats of LDS private to the wave; on return lcol[j*LDT + i] holds column
// j of the factor (zero above the diagonal, 1/L_jj on it).
__device__ __forceinline__ float cholesky_solve_rows(float (&a)[64], float fi, float qi,
                                                     float* colbuf, float* lcol) {
  const int i = lane_id();
  float dinv = 0.f;
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    const float piv = readlane_f(a[j] + fi, j);
    const float r = 1.0f / __fsqrt_rn(piv);
    const float col = a[j] * r;
    const float lj = i > j ? col : (i == j ? r : 0.f);
    a[j] = lj;
    dinv = i == j ? r : dinv;
    colbuf[i] = col;
    lcol[j * LDT + i] = lj;
    __syncthreads();
#pragma unroll
    for (int k = j + 1; k < 64; ++k) a[k] -= col * colbuf[k];
    __syncthreads();
  }
  // L w = q, then L^T y = w; lane j keeps w_j, y_j.
  float rres = qi, wk = 0.f;
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    const float wj = readlane_f(rres * dinv, j);
    wk = i == j ? wj : wk;
    rres -= a[j] * wj;
  }
  float u = wk, yk = 0.f;
#pragma unroll
  for (int j = 63; j >= 0; --j) {
    const float yj = readlane_f(u * dinv, j);
    yk = i == j ? yj : yk;
    u -= lcol[i * LDT + j] * yj;
  }
  return yk;
}

__global__ __launch_bounds__(64) void fwd_factor_kernel(
    Dims d, const float* __restrict__ keys, const float* __restrict__ queries,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ floor, const float* __restrict__ start_s,
    float* __restrict__ solved, float* __restrict__ factors) {
  const int seq = blockIdx.x;
  const int n = seq % d.NC, bh = seq / d.NC, b = bh / d.H, h = bh % d.H;
  const int i = threadIdx.x;
  __shared__ float kbuf[64];
  __shared__ float colbuf[64];
  __shared__ float lcol[64 * LDT];

  float s[64], a[64];
  const float* s0 = start_s + ((long)seq * 64 + i) * 64;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const f4 v = *reinterpret_cast<const f4*>(s0 + 4 * q);
    s[4 * q] = v[0];
    s[4 * q + 1] = v[1];
    s[4 * q + 2] = v[2];
    s[4 * q + 3] = v[3];
  }
  const float fi = floor[h * 64 + i];
  const int len = chunk_len(d, n);
  for (int tt = 0; tt < len; ++tt) {
    const long th = token_head(d, b, n * d.chunk + tt, h);
    const float ki = keys[th * 64 + i];
    const float qi = queries[th * 64 + i];
    const float bt = beta[th];
    const float lam = expf(log_decay[th]);
    kbuf[i] = ki;
    __syncthreads();
    const float bk = bt * ki;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      s[j] = lam * s[j] + bk * kbuf[j];
      a[j] = s[j];
    }
    __syncthreads();
    const float y = cholesky_solve_rows(a, fi, qi, colbuf, lcol);
    solved[th * 64 + i] = y;
    // Stream the packed factor: column j is 64 - j contiguous floats.  A
    // rolled loop keeps the 64 store addresses out of registers.
    float* fac = factors + th * FACTOR;
#pragma unroll 1
    for (int j = 0; j < 64; ++j)
      if (i >= j) fac[factor_col(j) + i - j] = lcol[j * LDT + i];
    __syncthreads();
  }
}

// z = A^-1 rhs from stored factors; one wave per token-head, four per block.
__global__ __launch_bounds__(256) void factored_solve_kernel(const float* __restrict__ factors,
                                                             const float* rhs, float* z, long N) {
  const int w = threadIdx.x >> 6, i = lane_id();
  const long th_raw = (long)blockIdx.x * 4 + w;
  const long th = th_raw < N ? th_raw : N - 1;
  __shared__ float lds[4][FACTOR];
  float* L = lds[w];
  const f4* src = reinterpret_cast<const f4*>(factors + th * FACTOR);
  for (int e = i; e < FACTOR / 4; e += 64) {
    const f4 v = src[e];
    L[4 * e] = v[0];
    L[4 * e + 1] = v[1];
    L[4 * e + 2] = v[2];
    L[4 * e + 3] = v[3];
  }
  const float rhs_i = rhs[th * 64 + i];
  __syncthreads();
  float r = rhs_i, wk = 0.f;
#pragma unroll
  for (int j = 0; j < 64; ++j) {
    const float wj = readlane_f(r, j) * L[factor_col(j)];
    wk = i == j ? wj : wk;
    const float lij = L[factor_col(j) + i - j];  // in range for every lane
    r -= (i > j ? lij : 0.f) * wj;
  }
  float u = wk, zk = 0.f;
#pragma unroll
  for (int j = 63; j >= 0; --j) {
    const float zj = readlane_f(u, j) * L[factor_col(j)];
    zk = i == j ? zj : zk;
    const float lji = L[factor_col(i) + j - i];  // in range for every lane
    u -= (i < j ? lji : 0.f) * zj;
  }
  if (th_raw < N) z[th * 64 + i] = zk;
}

// One decode step per (batch*head) state, in place.
__global__ __launch_bounds__(64) void decode_step_kernel(
    float* __restrict__ evidence, float* __restrict__ cross, const float* __restrict__ key,
    const float* __restrict__ value, const float* __restrict__ query,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ floor, int H, float* __restrict__ output,
    float* __restrict__ variance) {
  const long nidx = blockIdx.x;
  const int i = threadIdx.x;
  __shared__ float kbuf[64];
  __shared__ float colbuf[64];
  __shared__ float lcol[64 * LDT];
  float sr[64], cr[64], a[64];
  float* srow = evidence + (nidx * 64 + i) * 64;
  float* crow = cross + (nidx * 64 + i) * 64;
  const float ki = key[nidx * 64 + i], vi = value[nidx * 64 + i], qi = query[nidx * 64 + i];
  const float bt = beta[nidx], lam = expf(log_decay[nidx]);
  const float fi = floor[(nidx % H) * 64 + i];
  kbuf[i] = ki;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    f4 sv = *reinterpret_cast<const f4*>(srow + 4 * q);
    f4 cv = *reinterpret_cast<const f4*>(crow + 4 * q);
    const f4 kv = *reinterpret_cast<const f4*>(kbuf + 4 * q);
    sv = lam * sv + (bt * ki) * kv;
    cv = lam * cv + (bt * vi) * kv;
    *reinterpret_cast<f4*>(srow + 4 * q) = sv;
    *reinterpret_cast<f4*>(crow + 4 * q) = cv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sr[4 * q + e] = sv[e];
      cr[4 * q + e] = cv[e];
    }
  }
#pragma unroll
  for (int j = 0; j < 64; ++j) a[j] = sr[j];
  __syncthreads();
  const float y = cholesky_solve_rows(a, fi, qi, colbuf, lcol);
  kbuf[i] = y;
  __syncthreads();
  float out = 0.f;
#pragma unroll
  for (int j = 0; j < 64; ++j) out += cr[j] * kbuf[j];
  output[nidx * 64 + i] = out;
  float v = qi * y;
  v = row16_sum(v);
  v = group4_sum(v);
  if (i == 0) variance[nidx] = v;
}

}  // namespace m4
