// Chunk-level contractions on fp32 MFMA (v_mfma_f32_16x16x4_f32).
//
// One 256-thread block (4 waves) per (batch, head, chunk) sequence; every
// operand is a <=64x64 tile staged in LDS and each wave produces a 16-row
// strip of each 64x64 product (tile_mma in common.hpp).  Masks and decay
// weights W_ts = beta_s exp(P_t - P_s) (s <= t) are applied elementwise on
// the accumulators.
//
//   fwd_read_kernel   reads (lm/kernels/mamba4_fused.py:439-447):
//                     out = ((Y K^T) * W) V + exp(P) Y C0^T, variance = q.y
//   bwd_dy_kernel     cotangent of y:  ybar = ((dOut V^T) * W) K
//                     + exp(P) dOut C0 + dvar q
//   bwd_grads_kernel  every token gradient of _chunk_solve_backward
//                     (lm/kernels/mamba4_fused.py:343-366) plus the read,
//                     chunk-statistic and prefix adjoints
//   floor_reduce_kernel  d floor = sum over (batch, chunk) in a fixed order.
#include "common.hpp"

namespace m4 {

struct SeqIndex {
  int b, h, n, len;
  long seq;
};

__device__ __forceinline__ SeqIndex seq_index(const Dims& d) {
  SeqIndex s;
  s.seq = blockIdx.x;
  s.n = (int)(s.seq % d.NC);
  const int bh = (int)(s.seq / d.NC);
  s.b = bh / d.H;
  s.h = bh % d.H;
  s.len = chunk_len(d, s.n);
  return s;
}

struct TokenRows {
  const float* base;
  Dims d;
  int b, h, t0;
  __device__ const float* operator()(int s) const {
    return base + token_head(d, b, t0 + s, h) * 64;
  }
};

__device__ __forceinline__ TokenRows rows_of(const float* base, const Dims& d, const SeqIndex& si) {
  return TokenRows{base, d, si.b, si.h, si.n * d.chunk};
}

__global__ __launch_bounds__(256) void fwd_read_kernel(
    Dims d, const float* __restrict__ keys, const float* __restrict__ values,
    const float* __restrict__ queries, const float* __restrict__ beta,
    const float* __restrict__ log_decay, const float* __restrict__ solved,
    const float* __restrict__ start_c, float* __restrict__ output,
    float* __restrict__ variance) {
  extern __shared__ float smem[];
  float* Y = smem;
  float* K = Y + TILE;  // keys, then values
  float* G = K + TILE;
  float* C0 = G + TILE;
  __shared__ ChunkScalars cs;
  const SeqIndex si = seq_index(d);
  const int w = threadIdx.x >> 6;

  load_rows(Y, si.len, rows_of(solved, d, si));
  load_rows(K, si.len, rows_of(keys, d, si));
  load_chunk_scalars(cs, d, beta, log_decay, si.b, si.h, si.n);
  __syncthreads();

  f4 acc[4];
  zero4(acc);
  tile_mma<false, true>(acc, Y, LDT, K, LDT, 64, w);  // scores y_t . k_s
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = acc_row(w, r), s = acc_col(jb);
      float v = 0.f;
      if (s <= t && t < si.len) v = acc[jb][r] * cs.beta[s] * expf(cs.prefix[t] - cs.prefix[s]);
      G[t * LDT + s] = v;
    }
  __syncthreads();
  load_rows(K, si.len, rows_of(values, d, si));
  load_matrix(C0, start_c + si.seq * 4096);
  __syncthreads();

  f4 out[4], inh[4];
  zero4(out);
  zero4(inh);
  const int kpad = (si.len + 3) & ~3;
  tile_mma<false, false>(out, G, LDT, K, LDT, kpad, w);  // within-chunk reads
  tile_mma<false, true>(inh, Y, LDT, C0, LDT, 64, w);    // inherited reads y_t . C0[p]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = acc_row(w, r);
    if (t < si.len) {
      const float carried = expf(cs.prefix[t]);
      float* dst = output + token_head(d, si.b, si.n * d.chunk + t, si.h) * 64;
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) dst[acc_col(jb)] = out[jb][r] + carried * inh[jb][r];
    }
  }
  if (threadIdx.x < si.len) {
    const int t = threadIdx.x;
    const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
    const float* q = queries + th * 64;
    float v = 0.f;
    for (int e = 0; e < 64; ++e) v += q[e] * Y[t * LDT + e];
    variance[th] = v;
  }
}

__global__ __launch_bounds__(256) void bwd_dy_kernel(
    Dims d, const float* __restrict__ keys, const float* __restrict__ values,
    const float* __restrict__ queries, const float* __restrict__ beta,
    const float* __restrict__ log_decay, const float* __restrict__ start_c,
    const float* __restrict__ d_output, const float* __restrict__ d_variance,
    float* __restrict__ ybar) {
  extern __shared__ float smem[];
  float* DO = smem;
  float* V = DO + TILE;  // values, then keys
  float* G = V + TILE;
  float* C0 = G + TILE;
  __shared__ ChunkScalars cs;
  const SeqIndex si = seq_index(d);
  const int w = threadIdx.x >> 6;

  load_rows(DO, si.len, rows_of(d_output, d, si));
  load_rows(V, si.len, rows_of(values, d, si));
  load_chunk_scalars(cs, d, beta, log_decay, si.b, si.h, si.n);
  __syncthreads();

  f4 acc[4];
  zero4(acc);
  tile_mma<false, true>(acc, DO, LDT, V, LDT, 64, w);  // dout_t . v_s
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = acc_row(w, r), s = acc_col(jb);
      float v = 0.f;
      if (s <= t && t < si.len) v = acc[jb][r] * cs.beta[s] * expf(cs.prefix[t] - cs.prefix[s]);
      G[t * LDT + s] = v;
    }
  __syncthreads();
  load_rows(V, si.len, rows_of(keys, d, si));
  load_matrix(C0, start_c + si.seq * 4096);
  __syncthreads();

  f4 within[4], inh[4];
  zero4(within);
  zero4(inh);
  const int kpad = (si.len + 3) & ~3;
  tile_mma<false, false>(within, G, LDT, V, LDT, kpad, w);  // sum_s G[t][s] k_s
  tile_mma<false, false>(inh, DO, LDT, C0, LDT, 64, w);     // C0^T dout_t
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = acc_row(w, r);
    if (t < si.len) {
      const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
      const float carried = expf(cs.prefix[t]);
      const float dv = d_variance[th];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int e = acc_col(jb);
        ybar[th * 64 + e] = within[jb][r] + carried * inh[jb][r] + dv * queries[th * 64 + e];
      }
    }
  }
}

__global__ __launch_bounds__(256) void bwd_grads_kernel(
    Dims d, const float* __restrict__ keys, const float* __restrict__ values,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ solved, const float* __restrict__ z,
    const float* __restrict__ d_output, const float* __restrict__ d_variance,
    const float* __restrict__ start_s, const float* __restrict__ start_c,
    const float* __restrict__ end_s, const float* __restrict__ end_c,
    float* __restrict__ d_keys, float* __restrict__ d_values, float* __restrict__ d_queries,
    float* __restrict__ d_beta, float* __restrict__ d_log_decay,
    float* __restrict__ floor_part) {
  extern __shared__ float smem[];
  float* Kt = smem;       // keys, then S0
  float* Vt = Kt + TILE;  // values, then C0
  float* Yt = Vt + TILE;
  float* Zt = Yt + TILE;
  float* Dt = Zt + TILE;  // dout
  float* M1 = Dt + TILE;  // W * gy, then G_end
  float* M2 = M1 + TILE;  // W * (gv - gz), then H_end
  __shared__ ChunkScalars cs;
  __shared__ float colpart[4][64];
  __shared__ float rowE[64], colD2[64], quad[64], startdot[64];
  __shared__ float red[256];
  const SeqIndex si = seq_index(d);
  const int w = threadIdx.x >> 6, l = lane_id();
  const int kpad = (si.len + 3) & ~3;

  load_rows(Kt, si.len, rows_of(keys, d, si));
  load_rows(Vt, si.len, rows_of(values, d, si));
  load_rows(Yt, si.len, rows_of(solved, d, si));
  load_rows(Zt, si.len, rows_of(z, d, si));
  load_rows(Dt, si.len, rows_of(d_output, d, si));
  load_chunk_scalars(cs, d, beta, log_decay, si.b, si.h, si.n);
  __syncthreads();

  // Phase 1: gy = Y K^T, gz = Z K^T, gv = dOut V^T and their weighted mixes.
  {
    f4 gy[4], gz[4], gv[4];
    zero4(gy);
    zero4(gz);
    zero4(gv);
    tile_mma<false, true>(gy, Yt, LDT, Kt, LDT, 64, w);
    tile_mma<false, true>(gz, Zt, LDT, Kt, LDT, 64, w);
    tile_mma<false, true>(gv, Dt, LDT, Vt, LDT, 64, w);
    float rsum[4] = {0.f, 0.f, 0.f, 0.f};
    float csum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = acc_row(w, r), s = acc_col(jb);
        float my = 0.f, mz = 0.f, d2 = 0.f;
        if (s <= t && t < si.len) {
          const float dec = expf(cs.prefix[t] - cs.prefix[s]);
          const float mix = gv[jb][r] - gz[jb][r];
          d2 = dec * gy[jb][r] * mix;
          my = dec * cs.beta[s] * gy[jb][r];
          mz = dec * cs.beta[s] * mix;
        }
        M1[t * LDT + s] = my;
        M2[t * LDT + s] = mz;
        rsum[r] += cs.beta[s] * d2;
        csum[jb] += d2;
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = row16_sum(rsum[r]);
      if ((l & 15) == 0) rowE[acc_row(w, r)] = v;
    }
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const float v = group4_sum(csum[jb]);
      if (l < 16) colpart[w][acc_col(jb)] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int s = threadIdx.x;
    colD2[s] = colpart[0][s] + colpart[1][s] + colpart[2][s] + colpart[3][s];
  }

  // Phase 2: within-chunk key and value gradients.
  f4 dk[4], dv[4];
  zero4(dk);
  zero4(dv);
  {
    f4 tmp[4];
    zero4(tmp);
    tile_mma<true, false>(dk, M2, LDT, Yt, LDT, kpad, w);   // sum_t W(gv-gz)[t][s] y_t
    tile_mma<true, false>(tmp, M1, LDT, Zt, LDT, kpad, w);  // sum_t W gy[t][s] z_t
    tile_mma<true, false>(dv, M1, LDT, Dt, LDT, kpad, w);   // sum_t W gy[t][s] dout_t
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) dk[jb] -= tmp[jb];
  }
  __syncthreads();

  // Phase 3: chunk-end terms through the end-state cotangents G, H.
  load_matrix(M1, end_s + si.seq * 4096);
  load_matrix(M2, end_c + si.seq * 4096);
  __syncthreads();
  {
    f4 gk[4], hk[4], hv[4];
    zero4(gk);
    zero4(hk);
    zero4(hv);
    tile_mma<false, true>(gk, Kt, LDT, M1, LDT, 64, w);   // G k_s
    tile_mma<false, false>(gk, Kt, LDT, M1, LDT, 64, w);  // + G^T k_s
    tile_mma<false, true>(hk, Kt, LDT, M2, LDT, 64, w);   // H k_s
    tile_mma<false, false>(hv, Vt, LDT, M2, LDT, 64, w);  // H^T v_s
    float qpart[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = acc_row(w, r), e = acc_col(jb);
        qpart[r] += 0.5f * Kt[s * LDT + e] * gk[jb][r] + Vt[s * LDT + e] * hk[jb][r];
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int s = acc_row(w, r);
      const float qv = row16_sum(qpart[r]);
      if ((l & 15) == 0) quad[s] = qv;
      if (s < si.len) {
        const float tl = cs.tail[s];
        const long th = token_head(d, si.b, si.n * d.chunk + s, si.h);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int e = acc_col(jb);
          d_keys[th * 64 + e] = dk[jb][r] + tl * (gk[jb][r] + hv[jb][r]);
          d_values[th * 64 + e] = dv[jb][r] + tl * hk[jb][r];
        }
      }
    }
  }
  __syncthreads();

  // Phase 4: start-state terms <A_bar_t, S0>, <C_bar_t, C0> and <G,S0>+<H,C0>.
  // The chunk's start evidence is the start of its first sub-chunk.
  const long bh = si.seq / d.NC;
  load_matrix(Kt, start_s + (bh * d.NS + (long)si.n * d.rsub) * 4096);
  load_matrix(Vt, start_c + si.seq * 4096);
  __syncthreads();
  {
    float part = 0.f;
    for (int e = threadIdx.x; e < 4096; e += 256) {
      const int row = e >> 6, col = e & 63;
      part += M1[row * LDT + col] * Kt[row * LDT + col] + M2[row * LDT + col] * Vt[row * LDT + col];
    }
    red[threadIdx.x] = part;
    f4 ys[4], dc[4];
    zero4(ys);
    zero4(dc);
    tile_mma<false, false>(ys, Yt, LDT, Kt, LDT, 64, w);  // y_t^T S0
    tile_mma<false, false>(dc, Dt, LDT, Vt, LDT, 64, w);  // dout_t^T C0
    float sp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = acc_row(w, r), e = acc_col(jb);
        sp[r] += dc[jb][r] * Yt[t * LDT + e] - ys[jb][r] * Zt[t * LDT + e];
      }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = acc_row(w, r);
      const float v = row16_sum(sp[r]);
      if ((l & 15) == 0) startdot[t] = expf(cs.prefix[t]) * v;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    float v = red[threadIdx.x] + red[threadIdx.x + 64] + red[threadIdx.x + 128] + red[threadIdx.x + 192];
    v = group4_sum(row16_sum(v));
    red[threadIdx.x] = v;  // every lane of wave 0 holds the total
  }
  __syncthreads();

  // Phase 5: beta and log-decay gradients (wave 0), queries and floor.
  if (threadIdx.x < 64) {
    const int t = threadIdx.x;
    const float p_last = cs.prefix[MAXC - 1];
    float eend = 0.f, dp = 0.f, db = 0.f;
    if (t < si.len) {
      eend = cs.tail[t] * quad[t];
      dp = rowE[t] - cs.beta[t] * colD2[t] + startdot[t] - eend;
      db = colD2[t] + expf(p_last - cs.prefix[t]) * quad[t];
    }
    const float eend_total = group4_sum(row16_sum(eend));
    if (t == si.len - 1) dp += expf(p_last) * red[0] + eend_total;
    // d log_decay_r = sum_{t >= r} d prefix_t (reverse inclusive sum).
    float suffix = dp;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_down(suffix, o, 64);
      if (t + o < 64) suffix += y;
    }
    if (t < si.len) {
      const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
      d_beta[th] = db;
      d_log_decay[th] = suffix;
    }
  }
  for (int e = threadIdx.x; e < si.len * 64; e += 256) {
    const int t = e >> 6, c = e & 63;
    const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
    d_queries[th * 64 + c] = Zt[t * LDT + c] + d_variance[th] * Yt[t * LDT + c];
  }
  if (threadIdx.x < 64) {
    const int c = threadIdx.x;
    float v = 0.f;
    for (int t = 0; t < si.len; ++t) v -= Zt[t * LDT + c] * Yt[t * LDT + c];
    floor_part[si.seq * 64 + c] = v;
  }
}

// d floor[h][c] = sum_{b, n} floor_part[(b*H + h)*NC + n][c] in a fixed
// order: thread (q, c4) sums entries e = q, q+16, ... of the flattened
// (b, n) index as float4 columns 4c4..4c4+3, then the 16 partials are added
// in q order.  Deterministic run to run.
__global__ __launch_bounds__(256) void floor_reduce_kernel(Dims d, const float* __restrict__ part,
                                                          float* __restrict__ d_floor) {
  const int h = blockIdx.x, q = threadIdx.x >> 4, c4 = threadIdx.x & 15;
  const int entries = d.B * d.NC;
  __shared__ f4 partial[16][16];
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  for (int e = q; e < entries; e += 16) {
    const int b = e / d.NC, n = e % d.NC;
    acc += *reinterpret_cast<const f4*>(part + (((long)b * d.H + h) * d.NC + n) * 64 + 4 * c4);
  }
  partial[q][c4] = acc;
  __syncthreads();
  if (threadIdx.x < 16) {
    f4 total = partial[0][threadIdx.x];
    for (int k = 1; k < 16; ++k) total += partial[k][threadIdx.x];
    *reinterpret_cast<f4*>(d_floor + h * 64 + 4 * threadIdx.x) = total;
  }
}

}  // namespace m4
