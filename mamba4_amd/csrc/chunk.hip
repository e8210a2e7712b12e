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

__device__ __forceinline__ SeqIndex seq_at(const Dims& d, long seq) {
  SeqIndex s;
  s.seq = seq;
  s.n = (int)(s.seq % d.NC);
  const int bh = (int)(s.seq / d.NC);
  s.b = bh / d.H;
  s.h = bh % d.H;
  s.len = chunk_len(d, s.n);
  return s;
}

__device__ __forceinline__ SeqIndex seq_index(const Dims& d) { return seq_at(d, blockIdx.x); }

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

// Persistent: block i handles chunks i, i + gridDim.x, ...  The next chunk's
// tiles load into registers while this chunk is computed: Y, K and C0 right
// after this chunk's are in LDS, its queries once this chunk's variance is
// done, its values once this chunk's values are in LDS (at most five tiles
// in flight per thread, keeping two blocks per CU).
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
  float* C0 = G + TILE;  // C0 transposed: C0[e][p]
  __shared__ ChunkScalars cs;
  const long nseq = (long)d.B * d.H * d.NC;
  const int w = threadIdx.x >> 6, c4 = 4 * (lane_id() & 15);
  long seq = blockIdx.x;
  SeqIndex si = seq_at(d, seq);
  TileRegs ry, rk, rv, rq;
  TileRegsT rc;
  ry.fetch_rows(si.len, rows_of(solved, d, si));
  rk.fetch_rows(si.len, rows_of(keys, d, si));
  rc.fetch_matrix(start_c + si.seq * 4096);
  rq.fetch_rows(si.len, rows_of(queries, d, si));
  rv.fetch_rows(si.len, rows_of(values, d, si));

  for (;;) {
    ry.store(Y);
    rk.store(K);
    rc.store(C0);
    load_chunk_scalars(cs, d, beta, log_decay, si.b, si.h, si.n);
    __syncthreads();
    const long next = seq + gridDim.x;
    const bool more = next < nseq;  // uniform over the block
    const SeqIndex sn = seq_at(d, more ? next : seq);
    if (more) {
      ry.fetch_rows(sn.len, rows_of(solved, d, sn));
      rk.fetch_rows(sn.len, rows_of(keys, d, sn));
      rc.fetch_matrix(start_c + sn.seq * 4096);
    }

    // variance_t = q_t . y_t: this thread's four tile-fetch rows, summed over
    // the 16 lanes that hold the rest of each row.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = (threadIdx.x >> 4) + 16 * j;
      const f4 prod = rq.v[j] * *reinterpret_cast<const f4*>(Y + t * LDT + c4);
      const float v = row16_sum(prod[0] + prod[1] + prod[2] + prod[3]);
      if ((threadIdx.x & 15) == 0 && t < si.len)
        variance[token_head(d, si.b, si.n * d.chunk + t, si.h)] = v;
    }
    if (more) rq.fetch_rows(sn.len, rows_of(queries, d, sn));

    f4 acc[4];
    zero4(acc);
    tile_mma<false, true>(acc, Y, K, 64, w);  // scores y_t . k_s
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = acc_row(w, q), s = acc_col<false>(jb);
        float v = 0.f;
        if (s <= t && t < si.len)
          v = acc[jb][q] * cs.beta[s] * expf(cs.prefix[t] - cs.prefix[s]);
        G[t * LDT + s] = v;
      }
    __syncthreads();
    rv.store(K);
    __syncthreads();
    if (more) rv.fetch_rows(sn.len, rows_of(values, d, sn));

    f4 out[4], inh[4];
    zero4(out);
    zero4(inh);
    tile_mma<false, false>(out, G, K, k_terms(si.len), w);  // within-chunk reads
    tile_mma<false, false>(inh, Y, C0, 64, w);              // inherited reads y_t . C0[p]
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = acc_row(w, q);
      if (t < si.len) {
        const float carried = expf(cs.prefix[t]);
        float* dst = output + token_head(d, si.b, si.n * d.chunk + t, si.h) * 64;
        *reinterpret_cast<f4*>(dst + c4) = quad_row(out, q) + carried * quad_row(inh, q);
      }
    }
    if (!more) break;
    __syncthreads();  // the tiles and scalars are read; the next chunk may overwrite them
    si = sn;
    seq = next;
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
  const int w = threadIdx.x >> 6, c4 = 4 * (lane_id() & 15);

  TileRegs rd, rv, rk, rc;
  rd.fetch_rows(si.len, rows_of(d_output, d, si));
  rv.fetch_rows(si.len, rows_of(values, d, si));
  rk.fetch_rows(si.len, rows_of(keys, d, si));
  rc.fetch_matrix(start_c + si.seq * 4096);
  // Queries and d_variance of this lane's accumulator rows (read in the epilogue).
  f4 qv[4];
  float dvar[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = acc_row(w, q);
    qv[q] = f4{0.f, 0.f, 0.f, 0.f};
    dvar[q] = 0.f;
    if (t < si.len) {
      const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
      qv[q] = *reinterpret_cast<const f4*>(queries + th * 64 + c4);
      dvar[q] = d_variance[th];
    }
  }
  rd.store(DO);
  rv.store(V);
  rc.store(C0);
  load_chunk_scalars(cs, d, beta, log_decay, si.b, si.h, si.n);
  __syncthreads();

  f4 acc[4];
  zero4(acc);
  tile_mma<false, true>(acc, DO, V, 64, w);  // dout_t . v_s
#pragma unroll
  for (int jb = 0; jb < 4; ++jb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = acc_row(w, q), s = acc_col<false>(jb);
      float v = 0.f;
      if (s <= t && t < si.len) v = acc[jb][q] * cs.beta[s] * expf(cs.prefix[t] - cs.prefix[s]);
      G[t * LDT + s] = v;
    }
  __syncthreads();
  rk.store(V);
  __syncthreads();

  f4 within[4], inh[4];
  zero4(within);
  zero4(inh);
  tile_mma<false, false>(within, G, V, k_terms(si.len), w);  // sum_s G[t][s] k_s
  tile_mma<false, false>(inh, DO, C0, 64, w);                // C0^T dout_t
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = acc_row(w, q);
    if (t < si.len) {
      const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
      const float carried = expf(cs.prefix[t]);
      *reinterpret_cast<f4*>(ybar + th * 64 + c4) =
          quad_row(within, q) + carried * quad_row(inh, q) + dvar[q] * qv[q];
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
  __shared__ f4 fpart[4][16];
  const SeqIndex si = seq_index(d);
  const int w = threadIdx.x >> 6, l = lane_id(), c4 = 4 * (l & 15);
  const int kt = k_terms(si.len);
  // d_variance of this thread's tile-fetch rows (threadIdx/16 + 16j).
  float dvar[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = (threadIdx.x >> 4) + 16 * j;
    dvar[j] = t < si.len ? d_variance[token_head(d, si.b, si.n * d.chunk + t, si.h)] : 0.f;
  }

  {
    TileRegs r[5];
    r[0].fetch_rows(si.len, rows_of(keys, d, si));
    r[1].fetch_rows(si.len, rows_of(values, d, si));
    r[2].fetch_rows(si.len, rows_of(solved, d, si));
    r[3].fetch_rows(si.len, rows_of(z, d, si));
    r[4].fetch_rows(si.len, rows_of(d_output, d, si));
    r[0].store(Kt);
    r[1].store(Vt);
    r[2].store(Yt);
    r[3].store(Zt);
    r[4].store(Dt);
  }
  load_chunk_scalars(cs, d, beta, log_decay, si.b, si.h, si.n);
  // The end-state cotangents of phase 3 load while phases 1 and 2 run.
  TileRegs rg, rh;
  rg.fetch_matrix(end_s + si.seq * 4096);
  rh.fetch_matrix(end_c + si.seq * 4096);
  __syncthreads();

  // Phase 1: gy = Y K^T, gz = Z K^T, gv = dOut V^T and their weighted mixes.
  {
    f4 gy[4], gz[4], gv[4];
    zero4(gy);
    zero4(gz);
    zero4(gv);
    tile_mma<false, true>(gy, Yt, Kt, 64, w);
    tile_mma<false, true>(gz, Zt, Kt, 64, w);
    tile_mma<false, true>(gv, Dt, Vt, 64, w);
    float rsum[4] = {0.f, 0.f, 0.f, 0.f};
    float csum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = acc_row(w, q), s = acc_col<false>(jb);
        float my = 0.f, mz = 0.f, d2 = 0.f;
        if (s <= t && t < si.len) {
          const float dec = expf(cs.prefix[t] - cs.prefix[s]);
          const float mix = gv[jb][q] - gz[jb][q];
          d2 = dec * gy[jb][q] * mix;
          my = dec * cs.beta[s] * gy[jb][q];
          mz = dec * cs.beta[s] * mix;
        }
        M1[t * LDT + s] = my;
        M2[t * LDT + s] = mz;
        rsum[q] += cs.beta[s] * d2;
        csum[jb] += d2;
      }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float v = row16_sum(rsum[q]);
      if ((l & 15) == 0) rowE[acc_row(w, q)] = v;
    }
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const float v = group4_sum(csum[jb]);
      if (l < 16) colpart[w][acc_col<false>(jb)] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int s = threadIdx.x;
    colD2[s] = colpart[0][s] + colpart[1][s] + colpart[2][s] + colpart[3][s];
  }

  // Phase 2: within-chunk key and value gradients (rows s, columns 4r..4r+3).
  f4 dk[4], dv[4];
  zero4(dk);
  zero4(dv);
  {
    f4 tmp[4];
    zero4(tmp);
    tile_mma<true, false>(dk, M2, Yt, kt, w);   // sum_t W(gv-gz)[t][s] y_t
    tile_mma<true, false>(tmp, M1, Zt, kt, w);  // sum_t W gy[t][s] z_t
    tile_mma<true, false>(dv, M1, Dt, kt, w);   // sum_t W gy[t][s] dout_t
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) dk[jb] -= tmp[jb];
  }
  __syncthreads();

  // Phase 3: chunk-end terms through the end-state cotangents G, H.  G is
  // replaced by G + G^T in LDS (each off-diagonal pair by one thread), so
  // (G + G^T) k_s is a single product.
  rg.store(M1);
  rh.store(M2);
  // The start states of phase 4 load while phase 3 runs.
  const long bh = si.seq / d.NC;
  TileRegs rs, rc;
  rs.fetch_matrix(start_s + (bh * d.NS + (long)si.n * d.rsub) * 4096);
  rc.fetch_matrix(start_c + si.seq * 4096);
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int i = e >> 6, j = e & 63;
    if (i < j) {
      const float v = M1[i * LDT + j] + M1[j * LDT + i];
      M1[i * LDT + j] = v;
      M1[j * LDT + i] = v;
    } else if (i == j) {
      M1[i * LDT + i] *= 2.f;
    }
  }
  __syncthreads();
  {
    f4 gk[4], hk[4], hv[4];
    zero4(gk);
    zero4(hk);
    zero4(hv);
    tile_mma<false, false>(gk, Kt, M1, 64, w);       // (G + G^T) k_s
    tile_mma<false, true, true>(hk, Kt, M2, 64, w);  // H k_s
    tile_mma<false, false>(hv, Vt, M2, 64, w);       // H^T v_s
    float qpart[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int s = acc_row(w, q);
      const f4 kr = *reinterpret_cast<const f4*>(Kt + s * LDT + c4);
      const f4 vr = *reinterpret_cast<const f4*>(Vt + s * LDT + c4);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) qpart[q] += 0.5f * kr[jb] * gk[jb][q] + vr[jb] * hk[jb][q];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int s = acc_row(w, q);
      const float qv = row16_sum(qpart[q]);
      if ((l & 15) == 0) quad[s] = qv;
      if (s < si.len) {
        const float tl = cs.tail[s];
        const long th = token_head(d, si.b, si.n * d.chunk + s, si.h);
        *reinterpret_cast<f4*>(d_keys + th * 64 + c4) =
            quad_row(dk, q) + tl * (quad_row(gk, q) + quad_row(hv, q));
        *reinterpret_cast<f4*>(d_values + th * 64 + c4) = quad_row(dv, q) + tl * quad_row(hk, q);
      }
    }
  }
  __syncthreads();

  // Phase 4: start-state terms <A_bar_t, S0>, <C_bar_t, C0> and <G,S0>+<H,C0>
  // (<G, S0> = <G + G^T, S0> / 2 since S0 is symmetric).  The chunk's start
  // evidence is the start of its first sub-chunk.
  rs.store(Kt);
  rc.store(Vt);
  __syncthreads();
  {
    float part = 0.f;
    for (int e = threadIdx.x; e < 4096; e += 256) {
      const int row = e >> 6, col = e & 63;
      part += 0.5f * M1[row * LDT + col] * Kt[row * LDT + col] +
              M2[row * LDT + col] * Vt[row * LDT + col];
    }
    red[threadIdx.x] = part;
    f4 ys[4], dc[4];
    zero4(ys);
    zero4(dc);
    tile_mma<false, false>(ys, Yt, Kt, 64, w);  // y_t^T S0
    tile_mma<false, false>(dc, Dt, Vt, 64, w);  // dout_t^T C0
    float sp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = acc_row(w, q);
      const f4 yr = *reinterpret_cast<const f4*>(Yt + t * LDT + c4);
      const f4 zr = *reinterpret_cast<const f4*>(Zt + t * LDT + c4);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) sp[q] += dc[jb][q] * yr[jb] - ys[jb][q] * zr[jb];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = acc_row(w, q);
      const float v = row16_sum(sp[q]);
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
  // Queries, d q_t = z_t + dvar_t y_t, in the tile-fetch layout (rows
  // r0 + 16j, columns q4..q4+3), and the floor partial -sum_t z_t * y_t:
  // per thread over its four rows, then over the lanes and waves holding the
  // same columns, in a fixed order.
  {
    f4 fsum = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = (threadIdx.x >> 4) + 16 * j;
      const f4 zr = *reinterpret_cast<const f4*>(Zt + t * LDT + c4);
      const f4 yr = *reinterpret_cast<const f4*>(Yt + t * LDT + c4);
      if (t < si.len) {
        const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
        *reinterpret_cast<f4*>(d_queries + th * 64 + c4) = zr + dvar[j] * yr;
      }
      fsum -= zr * yr;  // zero past the chunk's tokens
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) fsum[i] = group4_sum(fsum[i]);
    if (l < 16) fpart[w][l] = fsum;
    __syncthreads();
    if (threadIdx.x < 16) {
      const f4 total = fpart[0][threadIdx.x] + fpart[1][threadIdx.x] + fpart[2][threadIdx.x] +
                       fpart[3][threadIdx.x];
      *reinterpret_cast<f4*>(floor_part + si.seq * 64 + 4 * threadIdx.x) = total;
    }
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
