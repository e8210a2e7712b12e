// Batched SPD solves wider than 64 (spd_solve, lm/kernels/mamba4.py:188-217,
// whose _factor_and_solve :164-187 takes any width).  Widths up to 64 take
// the four-systems-per-wave kernels of factor.hip; these take one 256-thread
// block per system:
//
//   - the system's lower triangle is copied into M (row stride ld, upper
//     triangle zeroed): LDS for dim <= 128 (stride dim + 1, so a column
//     read across lanes is conflict-free), else the caller's factor buffer
//     in global memory;
//   - right-looking Cholesky, one column per step: the reciprocal pivot
//     1/L_jj = rsq(M_jj) (v_rsq_f32, as the 64-wide path and the
//     reference's lax.rsqrt pivot), the column scaled below the diagonal and
//     copied into an LDS vector, then the rank-one update of the trailing
//     lower triangle, rows split over eight groups of 32 lanes, columns over
//     the group's lanes, so a row's update is one contiguous run; M_jj ends
//     holding 1/L_jj;
//   - forward substitution L w = b by columns (every step scales the final
//     w_j and updates the entries below it in parallel) and backward
//     substitution L^T y = w by rows of L (contiguous), one barrier per
//     step.
//
// A non-positive pivot gives NaN, which propagates to the solution, as the
// reference's does.  Stored factor (dense, [dim][dim] row-major): L below the
// diagonal, 1/L_ii on it, zero above.
#include "common.hpp"

namespace m4 {

// M: the system's lower triangle (row stride ld); col: dim floats of LDS.
__device__ void wide_factor(float* M, int ld, int dim, float* col) {
  const int tid = threadIdx.x, grp = tid >> 5, c = tid & 31;
  for (int j = 0; j < dim; ++j) {
    const float rs = __builtin_amdgcn_rsqf(M[j * ld + j]);
    for (int i = j + 1 + tid; i < dim; i += kWideThreads) {
      const float l = M[i * ld + j] * rs;
      M[i * ld + j] = l;
      col[i] = l;
    }
    __syncthreads();  // column j is final and in col
    for (int i = j + 1 + grp; i < dim; i += kWideThreads / 32) {
      const float lij = col[i];
      for (int k = j + 1 + c; k <= i; k += 32) M[i * ld + k] -= lij * col[k];
    }
    // Every thread read M_jj before the barrier above; no step after this
    // one reads or writes it.
    if (tid == 0) M[j * ld + j] = rs;
    __syncthreads();  // the trailing update is done before the next pivot
  }
}

// L w = b then L^T y = w with M holding the factor as wide_factor leaves it.
// w: dim floats of LDS holding b on entry (overwritten); t: dim floats of
// LDS, y on return.
__device__ void wide_solve(const float* M, int ld, int dim, float* w, float* t) {
  const int tid = threadIdx.x;
  for (int j = 0; j < dim; ++j) {
    // w_j is final: every column before j has updated it (barrier below).
    const float wj = w[j] * M[j * ld + j];
    for (int i = j + 1 + tid; i < dim; i += kWideThreads) w[i] -= M[i * ld + j] * wj;
    if (tid == 0) t[j] = wj;
    __syncthreads();
  }
  for (int i = tid; i < dim; i += kWideThreads) w[i] = t[i];
  __syncthreads();
  for (int j = dim - 1; j >= 0; --j) {
    const float yj = w[j] * M[j * ld + j];
    for (int i = tid; i < j; i += kWideThreads) w[i] -= M[j * ld + i] * yj;
    if (tid == 0) t[j] = yj;
    __syncthreads();
  }
}

// precision [N,dim,dim] (only k <= i read), rhs [N,dim] -> solution [N,dim]
// and, when factors is non-null, the dense factor [N,dim,dim].  LDS = false
// (dim > 128) factors in `factors`, which must then be non-null.
template <bool LDS>
__global__ __launch_bounds__(kWideThreads) void spd_wide_kernel(
    const float* __restrict__ precision, const float* __restrict__ rhs, int dim,
    float* __restrict__ solution, float* __restrict__ factors) {
  extern __shared__ float sm[];
  const long n = blockIdx.x, dd = (long)dim * dim;
  const int tid = threadIdx.x;
  float* const col = sm;
  float* const w = col + dim;
  float* const t = w + dim;
  const int ld = LDS ? dim + 1 : dim;
  float* const M = LDS ? t + dim : factors + n * dd;
  const float* const A = precision + n * dd;
  for (long e = tid; e < dd; e += kWideThreads) {
    const int i = (int)(e / dim), k = (int)(e - (long)i * dim);
    M[i * ld + k] = k <= i ? A[e] : 0.f;
  }
  for (int i = tid; i < dim; i += kWideThreads) w[i] = rhs[n * dim + i];
  __syncthreads();
  wide_factor(M, ld, dim, col);
  wide_solve(M, ld, dim, w, t);
  for (int i = tid; i < dim; i += kWideThreads) solution[n * dim + i] = t[i];
  if (LDS && factors)
    for (long e = tid; e < dd; e += kWideThreads) {
      const int i = (int)(e / dim), k = (int)(e - (long)i * dim);
      factors[n * dd + e] = M[i * ld + k];
    }
}

// VJP (lm/kernels/mamba4.py:204-215): z = A^-1 g from the stored dense
// factor, d_rhs = z, d_precision = -(z y^T + y z^T) / 2 (exactly symmetric).
template <bool LDS>
__global__ __launch_bounds__(kWideThreads) void spd_wide_backward_kernel(
    const float* __restrict__ factors, const float* __restrict__ solution,
    const float* __restrict__ d_solution, int dim, float* __restrict__ d_precision,
    float* __restrict__ d_rhs) {
  extern __shared__ float sm[];
  const long n = blockIdx.x, dd = (long)dim * dim;
  const int tid = threadIdx.x;
  float* const y = sm;
  float* const w = y + dim;
  float* const t = w + dim;
  const int ld = LDS ? dim + 1 : dim;
  const float* M = factors + n * dd;
  if (LDS) {
    float* const Ml = t + dim;
    for (long e = tid; e < dd; e += kWideThreads) {
      const int i = (int)(e / dim), k = (int)(e - (long)i * dim);
      Ml[i * ld + k] = factors[n * dd + e];
    }
    M = Ml;
  }
  for (int i = tid; i < dim; i += kWideThreads) {
    w[i] = d_solution[n * dim + i];
    y[i] = solution[n * dim + i];
  }
  __syncthreads();
  wide_solve(M, ld, dim, w, t);
  for (int i = tid; i < dim; i += kWideThreads) d_rhs[n * dim + i] = t[i];
  for (long e = tid; e < dd; e += kWideThreads) {
    // Both products rounded on their own, so d_precision is exactly
    // symmetric.
#pragma clang fp contract(off)
    const int i = (int)(e / dim), k = (int)(e - (long)i * dim);
    d_precision[n * dd + e] = -0.5f * (t[i] * y[k] + y[i] * t[k]);
  }
}

template __global__ void spd_wide_kernel<true>(const float*, const float*, int, float*, float*);
template __global__ void spd_wide_kernel<false>(const float*, const float*, int, float*, float*);
template __global__ void spd_wide_backward_kernel<true>(const float*, const float*, const float*,
                                                        int, float*, float*);
template __global__ void spd_wide_backward_kernel<false>(const float*, const float*, const float*,
                                                         int, float*, float*);

}  // namespace m4
