// Chunk-boundary states: the forward decayed carry of chunk statistics and
// the backward reverse carry of start-state cotangents.
//
// Forward (lm/kernels/mamba4_fused.py:411-425 with chunk_carry,
// lm/kernels/prefix.py:27-44): per (b, h) the chunks are walked in order,
//   start[n] = running,  running = exp(P_last,n) running + X_n^T diag(tail_n) K_n
// with X = K for the evidence and X = V for the cross statistics.
// Backward: the transpose of that carry, walked in reverse,
//   end[n] = running,  running = U_n + exp(P_last,n) running,
// U_n = sum_t exp(P_t) (-(z_t y_t^T + y_t z_t^T)/2) for the evidence and
// sum_t exp(P_t) dout_t y_t^T for the cross statistics.
//
// Grid (B*H, 8): blockIdx.y 0..3 owns evidence rows [16y, 16y+16), 4..7 the
// cross rows [16(y-4), ...).  Each of the 256 threads keeps 4 consecutive
// columns of one row in registers for the whole walk, so the running state
// never leaves the chip; every chunk costs one read of its token rows.
#include "common.hpp"

namespace m4 {

__global__ __launch_bounds__(256) void fwd_states_kernel(
    Dims d, const float* __restrict__ keys, const float* __restrict__ values,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ init_s, const float* __restrict__ init_c,
    float* __restrict__ start_s, float* __restrict__ start_c,
    float* __restrict__ final_s, float* __restrict__ final_c) {
  const int bh = blockIdx.x, b = bh / d.H, h = bh % d.H;
  const bool cross = blockIdx.y >= 4;
  const int r0 = 16 * (blockIdx.y & 3);
  const int tid = threadIdx.x, row = tid >> 4, col = (tid & 15) * 4;

  __shared__ float kbuf[MAXC * 64];
  __shared__ float xbuf[MAXC * 16];
  __shared__ ChunkScalars cs;

  const float* init = cross ? init_c : init_s;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  if (init) acc = *reinterpret_cast<const f4*>(init + ((long)bh * 64 + r0 + row) * 64 + col);
  const float* xsrc = cross ? values : keys;
  float* starts = cross ? start_c : start_s;

  for (int n = 0; n < d.NC; ++n) {
    const int len = chunk_len(d, n);
    for (int e = tid; e < len * 16; e += 256) {
      const int s = e >> 4, q = (e & 15) * 4;
      const long th = token_head(d, b, n * d.chunk + s, h);
      *reinterpret_cast<f4*>(kbuf + s * 64 + q) = *reinterpret_cast<const f4*>(keys + th * 64 + q);
    }
    for (int e = tid; e < len * 4; e += 256) {
      const int s = e >> 2, q = (e & 3) * 4;
      const long th = token_head(d, b, n * d.chunk + s, h);
      *reinterpret_cast<f4*>(xbuf + s * 16 + q) =
          *reinterpret_cast<const f4*>(xsrc + th * 64 + r0 + q);
    }
    load_chunk_scalars(cs, d, beta, log_decay, b, h, n);
    __syncthreads();
    *reinterpret_cast<f4*>(starts + (((long)bh * d.NC + n) * 64 + r0 + row) * 64 + col) = acc;
    const float decay = expf(cs.prefix[MAXC - 1]);
    acc *= decay;
    for (int s = 0; s < len; ++s) {
      const float x = xbuf[s * 16 + row] * cs.tail[s];
      const f4 kv = *reinterpret_cast<const f4*>(kbuf + s * 64 + col);
      acc += x * kv;
    }
    __syncthreads();
  }
  float* fin = cross ? final_c : final_s;
  *reinterpret_cast<f4*>(fin + ((long)bh * 64 + r0 + row) * 64 + col) = acc;
}

__global__ __launch_bounds__(256) void bwd_states_kernel(
    Dims d, const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ solved, const float* __restrict__ z,
    const float* __restrict__ d_output, const float* __restrict__ d_final_s,
    const float* __restrict__ d_final_c, float* __restrict__ end_s, float* __restrict__ end_c,
    float* __restrict__ d_init_s, float* __restrict__ d_init_c) {
  const int bh = blockIdx.x, b = bh / d.H, h = bh % d.H;
  const bool cross = blockIdx.y >= 4;
  const int r0 = 16 * (blockIdx.y & 3);
  const int tid = threadIdx.x, row = tid >> 4, col = (tid & 15) * 4;

  __shared__ float ybuf[MAXC * 64];
  __shared__ float zbuf[MAXC * 64];  // z (evidence) or dout (cross)
  __shared__ ChunkScalars cs;

  const float* fin = cross ? d_final_c : d_final_s;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  if (fin) acc = *reinterpret_cast<const f4*>(fin + ((long)bh * 64 + r0 + row) * 64 + col);
  const float* other = cross ? d_output : z;
  float* ends = cross ? end_c : end_s;

  for (int n = d.NC - 1; n >= 0; --n) {
    const int len = chunk_len(d, n);
    for (int e = tid; e < len * 16; e += 256) {
      const int s = e >> 4, q = (e & 15) * 4;
      const long th = token_head(d, b, n * d.chunk + s, h);
      *reinterpret_cast<f4*>(ybuf + s * 64 + q) = *reinterpret_cast<const f4*>(solved + th * 64 + q);
      *reinterpret_cast<f4*>(zbuf + s * 64 + q) = *reinterpret_cast<const f4*>(other + th * 64 + q);
    }
    load_chunk_scalars(cs, d, beta, log_decay, b, h, n);
    __syncthreads();
    *reinterpret_cast<f4*>(ends + (((long)bh * d.NC + n) * 64 + r0 + row) * 64 + col) = acc;
    acc *= expf(cs.prefix[MAXC - 1]);
    const int i = r0 + row;
    for (int t = 0; t < len; ++t) {
      const float w = expf(cs.prefix[t]);
      const f4 yv = *reinterpret_cast<const f4*>(ybuf + t * 64 + col);
      if (cross) {
        acc += (w * zbuf[t * 64 + i]) * yv;
      } else {
        const f4 zv = *reinterpret_cast<const f4*>(zbuf + t * 64 + col);
        acc -= (0.5f * w) * (zbuf[t * 64 + i] * yv + ybuf[t * 64 + i] * zv);
      }
    }
    __syncthreads();
  }
  float* dinit = cross ? d_init_c : d_init_s;
  *reinterpret_cast<f4*>(dinit + ((long)bh * 64 + r0 + row) * 64 + col) = acc;
}

}  // namespace m4
