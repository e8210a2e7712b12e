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

// Row s of a chunk's token-major slab: `width` elements (float32 or
// bfloat16) per token-head, the 64 columns from `offset` (a value tile of a
// P-wide row).
template <typename T>
struct TokenRows {
  const T* base;
  Dims d;
  int b, h, t0, width, offset;
  __device__ const T* operator()(int s) const {
    return base + token_head(d, b, t0 + s, h) * width + offset;
  }
};

// A chunk's `rows` token rows into a RowTile (consecutive tokens are H rows
// of `width` apart).
template <typename T, int NTH>
__device__ __forceinline__ void fetch_tokens(RowTile<T, NTH>& R, int rows, const TokenRows<T>& tr) {
  R.fetch_tokens(rows, tr(0), (unsigned)(tr.d.H * tr.width));
}

template <typename T>
__device__ __forceinline__ TokenRows<T> rows_of(const T* base, const Dims& d, const SeqIndex& si) {
  return TokenRows<T>{base, d, si.b, si.h, si.n * d.chunk, 64, 0};
}

// Value tile v of a P-wide row slab (values, reads and their cotangents).
template <typename T>
__device__ __forceinline__ TokenRows<T> value_rows(const T* base, const Dims& d,
                                                   const SeqIndex& si, int v) {
  return TokenRows<T>{base, d, si.b, si.h, si.n * d.chunk, d.P, 64 * v};
}

// Tile v of chunk `seq`'s cross state [P, 64] (NV stacked 64x64 tiles).
__device__ __forceinline__ const float* cross_tile(const float* base, const Dims& d, long seq,
                                                   int v) {
  return base + (seq * d.NV + v) * 4096;
}

// G[t][s] = scores(t, s) x_t beta_s exp(P_t - P_s) for s <= t < len, zero
// elsewhere, for strip W (acc: its scores in the tile_mma layout; x: row
// factors, the read gates of the gated backward, when ROWS).  Blocks jb < W
// lie below the diagonal, jb = W straddles it and blocks jb > W are zero:
// one straight-line body per strip, with no exponentials for the zero
// blocks and the mask a select rather than a branch per element.
template <int W, bool ROWS>
__device__ __forceinline__ void causal_weights_strip(const f4 acc[4], float* G,
                                                     const ChunkScalars& cs, int len,
                                                     const float* x) {
  const int r = lane_id() & 15;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int t = acc_row(W, q);
    const float pt = cs.prefix[t];
    const bool in = t < len;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int s = 16 * jb + r;  // acc_col<false>(jb)
      float v = 0.f;
      if (jb <= W) {
        float a = acc[jb][q];
        if constexpr (ROWS) a *= x[q];
        const float e = a * cs.beta[s] * expf(pt - cs.prefix[s]);
        v = in && (jb < W || s <= t) ? e : 0.f;
      }
      G[t * LDT + s] = v;
    }
  }
}
template <bool ROWS>
__device__ __forceinline__ void causal_weights(const f4 acc[4], float* G, const ChunkScalars& cs,
                                               int len, int w, const float* x = nullptr) {
  switch (w) {
    case 0: causal_weights_strip<0, ROWS>(acc, G, cs, len, x); break;
    case 1: causal_weights_strip<1, ROWS>(acc, G, cs, len, x); break;
    case 2: causal_weights_strip<2, ROWS>(acc, G, cs, len, x); break;
    default: causal_weights_strip<3, ROWS>(acc, G, cs, len, x); break;
  }
}

// Persistent: block i handles chunks i, i + gridDim.x, ...  The next chunk's
// tiles load into registers while this chunk is computed: Y right after
// this chunk's tiles are in LDS, its queries once this chunk's variance is
// done, K and C0 once the scores are in LDS, its values once this chunk's
// values are in LDS (at most five tiles in flight per thread, keeping two
// blocks per CU).  Every wave of the CU reaches each of these points at
// about the same time, so the loads go out in four smaller bursts rather
// than one: a wave issuing into a full memory pipeline stalls until it
// drains, and the later bursts drain under the products.
//
// MIX: keys and queries come from the mixer's raw projections (`mix`,
// transformed on load: the key rows shifted and normalised at staging, the
// queries normalised where used), and the output is gated (`gate`), the
// ungated read kept in gate.read.
template <typename In, bool MIX, int NV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_read_kernel(
    Dims d, const In* __restrict__ keys, const In* __restrict__ values,
    const In* __restrict__ queries, const float* __restrict__ beta,
    const float* __restrict__ log_decay, const float* __restrict__ solved,
    const float* __restrict__ start_c, float* __restrict__ output,
    float* __restrict__ variance, MixerIn mix, ReadGate gate) {
  extern __shared__ float smem[];
  // Value tiles per row: compile-time for one (every branch on it folds,
  // so the compiler can count the loads in flight at each wait), else read.
  const int nv = NV == 1 ? 1 : d.NV;
  float* Y = smem;
  float* K = Y + TILE;  // keys, then values
  float* G = K + TILE;
  float* C0 = G + TILE;  // C0 transposed: C0[e][p]
  __shared__ ChunkScalars cs;
  __shared__ float gate_s[MIX ? MAXC : 1];  // MIX: the chunk's read gates
  const long nseq = (long)d.B * d.H * d.NC;
  // The wave's 16-row strip (its causal products cost strip + 1 blocks).
  // Blocks in the grid's second half take the strips in reverse order: a
  // CU's two blocks are normally one from each half, so each SIMD then holds
  // strips k and 3 - k (k + 1 and 4 - k blocks of causal products) instead
  // of two heavy or two light waves.
  const int w = (threadIdx.x >> 6) ^ (blockIdx.x >= gridDim.x / 2 ? 3 : 0);
  const int c4 = 4 * (lane_id() & 15);
  long seq = blockIdx.x;
  SeqIndex si = seq_at(d, seq);
  RowTile<float> ry;
  RowTile<In> rk, rv, rq;
  TileRegsT rc;
  // MIX key rows: the raw source row of each position (the zero row of
  // position 0 reads its query row and is zeroed at staging).
  auto fetch_keys = [&](const SeqIndex& s) {
    if constexpr (MIX) {
      rk.fetch_mix_keys(s.len, mix, d, s.b, s.h, s.n * d.chunk);
    } else {
      fetch_tokens(rk, s.len, rows_of(keys, d, s));
    }
  };
  auto fetch_queries = [&](const SeqIndex& s) {
    if constexpr (MIX)
      fetch_tokens(rq, s.len, rows_of(mix.query, d, s));
    else
      fetch_tokens(rq, s.len, rows_of(queries, d, s));
  };
  // The chunk's log decays and betas, lane s of wave 0 holding token s's
  // (the other lanes read out of range), fetched with its first tiles.
  // MIX: the head's gate parameters too.
  float sg, sb, hscale = 0.f, hskip = 0.f;
  auto fetch_scalars = [&](const SeqIndex& s) {
    const unsigned st = (unsigned)d.H * 4, bytes = s.len > 0 ? (unsigned)(s.len - 1) * st + 4 : 0;
    const long th = token_head(d, s.b, s.n * d.chunk, s.h);
    const unsigned off = threadIdx.x < 64 ? threadIdx.x * st : kNoRow;
    sg = buf_load1(buf_rsrc(log_decay + th, bytes), off);
    sb = buf_load1(buf_rsrc(beta + th, bytes), off);
    if constexpr (MIX) {
      hscale = gate.confidence_scale[s.h];
      hskip = gate.skip[s.h];
    }
  };
  fetch_tokens(ry, si.len, rows_of(solved, d, si));
  fetch_scalars(si);
  fetch_keys(si);
  rc.fetch_matrix(cross_tile(start_c, d, si.seq, 0));
  fetch_queries(si);
  fetch_tokens(rv, si.len, value_rows(values, d, si, 0));

  for (;;) {
    ry.store(Y);
    if constexpr (MIX)
      rk.store_unit(K, mix.key_shift && !mix.previous && si.n == 0);
    else
      rk.store(K);
    rc.store(C0);
    if (threadIdx.x < 64) finish_chunk_scalars(cs, sg, sb);
    const float scale = hscale, skip = hskip;  // this chunk's head
    __syncthreads();
    const long next = seq + gridDim.x;
    const bool more = next < nseq;  // uniform over the block
    // After a block's last chunk the same loads are issued with no rows in
    // range (zeros, no memory access): every chunk issues the same loads, so
    // each wait counts exactly.
    SeqIndex sn = seq_at(d, more ? next : seq);
    if (!more) sn.len = 0;
    fetch_tokens(ry, sn.len, rows_of(solved, d, sn));
    fetch_scalars(sn);

    // variance_t = q_t . y_t: this thread's four tile-fetch rows, summed over
    // the 16 lanes that hold the rest of each row.
    float vrow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = (threadIdx.x >> 4) + 16 * j;
      const f4 qt = MIX ? mix_unit(rq.get(j)) : rq.get(j);
      const f4 prod = qt * *reinterpret_cast<const f4*>(Y + t * LDT + c4);
      const float v = row16_sum(prod[0] + prod[1] + prod[2] + prod[3]);
      vrow[j] = v;
      if ((threadIdx.x & 15) == 0 && t < si.len)
        variance[token_head(d, si.b, si.n * d.chunk + t, si.h)] = v;
    }
    if constexpr (MIX) {
      // The epilogue's gate of each row, evaluated once per row.
      float g[4];
      per_row<4>(vrow, g, [&](float v) { return read_gate(scale, v); });
      if ((threadIdx.x & 15) == 0)
#pragma unroll
        for (int j = 0; j < 4; ++j) gate_s[(threadIdx.x >> 4) + 16 * j] = g[j];
    }
    fetch_queries(sn);

    f4 acc[4];
    zero4(acc);
    tile_mma_causal<false>(acc, Y, K, w);  // scores y_t . k_s, s <= t
    causal_weights<false>(acc, G, cs, si.len, w);
    fetch_keys(sn);
    // With more than one value tile, rc carries this chunk's later tiles and
    // prefetches after the last of them.
    if (nv == 1) rc.fetch_matrix(cross_tile(start_c, d, sn.seq, 0), more);
#pragma unroll 1
    for (int v = 0; v < nv; ++v) {
      if (v > 0) {
        // Value tile v and cross tile v replace tile v - 1 once every wave
        // has read it.
        fetch_tokens(rv, si.len, value_rows(values, d, si, v));
        rc.fetch_matrix(cross_tile(start_c, d, si.seq, v));
        __syncthreads();
        rc.store(C0);
      } else {
        __syncthreads();
      }
      rv.store(K);
      __syncthreads();
      if (v == nv - 1) {
        fetch_tokens(rv, sn.len, value_rows(values, d, sn, 0));
        if (nv > 1) rc.fetch_matrix(cross_tile(start_c, d, sn.seq, 0), more);
      }

      f4 out[4], inh[4];
      zero4(out);
      zero4(inh);
      // within-chunk reads: G[t][s] is zero past s = t
      tile_mma_causal_terms<false, false>(out, G, K, si.len, w);
      tile_mma<false, false>(inh, Y, C0, 64, w);              // inherited reads y_t . C0[p]
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = acc_row(w, q);
        if (t < si.len) {
          const float carried = expf(cs.prefix[t]);
          const long row = token_head(d, si.b, si.n * d.chunk + t, si.h) * d.P + 64 * v;
          const f4 x = quad_row(out, q) + carried * quad_row(inh, q);
          if constexpr (MIX) {
            // The epilogue's arithmetic: g x + D value (value tile v is in K).
            const float g = gate_s[t];
            const f4 val = *reinterpret_cast<const f4*>(K + t * LDT + c4);
            *reinterpret_cast<f4*>(gate.read + row + c4) = x;
            *reinterpret_cast<f4*>(output + row + c4) = g * x + skip * val;
          } else {
            *reinterpret_cast<f4*>(output + row + c4) = x;
          }
        }
      }
    }
    if (!more) break;
    __syncthreads();  // the tiles and scalars are read; the next chunk may overwrite them
    si = sn;
    seq = next;
  }
}

// Persistent like fwd_read_kernel: block i handles chunks i, i + gridDim.x,
// ...; the next chunk's dout, value and C0 tiles load into registers once
// this chunk's last value tile is in LDS, its keys once this chunk's keys are
// staged, and its queries and d_variance after this chunk's epilogue.
//
// MIX: keys and queries from the mixer's raw projections, as in
// fwd_read_kernel (keys shifted and normalised at staging, queries
// normalised where used).  GATE (with MIX): d_output is the cotangent of
// the mixer's gated output and d_variance unused; the read's cotangent is
// g_t d_out_t, applied to the rows of the products (all linear in them),
// and its variance cotangent d_var_t = (d_out_t . read_t) g (1 - g)
// (-scale / (1 + var_t)) plus mg.d_var_in, written to mg.d_var; the
// per-chunk sums of -(d_out . read) g (1 - g) log1p(var) and d_out . value
// go to mg.dy_part (epilogue_backward_kernel's arithmetic).
template <typename In, bool MIX, bool GATE, int NV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_dy_kernel(
    Dims d, const In* __restrict__ keys, const In* __restrict__ values,
    const In* __restrict__ queries, const float* __restrict__ beta,
    const float* __restrict__ log_decay, const float* __restrict__ start_c,
    const float* __restrict__ d_output, const float* __restrict__ d_variance,
    float* __restrict__ ybar, MixerIn mix, MixerGrad mg) {
  static_assert(!GATE || MIX, "the gated backward reads the mixer's raw rows");
  extern __shared__ float smem[];
  // Value tiles per row: compile-time for one (every branch on it folds,
  // so the compiler can count the loads in flight at each wait), else read.
  // (GATE: read, which keeps its registers within bounds.)
  const int nv = NV == 1 && !GATE ? 1 : d.NV;
  float* DO = smem;
  float* V = DO + TILE;  // values, then keys
  float* G = V + TILE;
  float* C0 = G + TILE;
  __shared__ ChunkScalars cs;
  __shared__ float epart[GATE ? 4 : 1][2];  // GATE: per-wave gate-parameter partials
  const long nseq = (long)d.B * d.H * d.NC;
  // The wave's 16-row strip (its causal products cost strip + 1 blocks),
  // reversed in the grid's second half as in fwd_read_kernel.
  const int w = (threadIdx.x >> 6) ^ (blockIdx.x >= gridDim.x / 2 ? 3 : 0);
  const int c4 = 4 * (lane_id() & 15);
  long seq = blockIdx.x;
  SeqIndex si = seq_at(d, seq);

  RowTile<float> rd;
  RowTile<In> rv, rk;
  TileRegs rc;
  // Queries and d_variance of this lane's accumulator rows (read in the
  // epilogue; zero past the chunk).  GATE: the variance cotangent from
  // mg.d_var_in (zero without it) and the variance itself, in gvar.
  RowQuad<In> qv[4];
  float dvar[4], gvar[4];
  auto fetch_rows_q = [&](const SeqIndex& s) {
    const long th = token_head(d, s.b, s.n * d.chunk, s.h);
    const unsigned st = (unsigned)d.H * 64;
    const In* qsrc;
    if constexpr (MIX)
      qsrc = mix.query;
    else
      qsrc = queries;
    const BufRsrc rq = buf_rsrc(qsrc + th * 64, ((unsigned)(s.len - 1) * st + 64) * sizeof(In));
    const unsigned sbytes = ((unsigned)(s.len - 1) * d.H + 1) * 4;
    const float* dv_src = GATE ? mg.d_var_in : d_variance;
    const BufRsrc rv2 = buf_rsrc(dv_src ? dv_src + th : d_output, dv_src ? sbytes : 0);
    const BufRsrc rvar = buf_rsrc(GATE ? mg.variance + th : d_output, GATE ? sbytes : 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const unsigned t = acc_row(w, q);
      qv[q].load(rq, (t * st + c4) * sizeof(In));
      dvar[q] = buf_load1(rv2, t * d.H * 4);
      if constexpr (GATE) gvar[q] = buf_load1(rvar, t * d.H * 4);
    }
  };
  // The chunk's log decays and betas (lane s of wave 0: token s; the other
  // lanes read out of range), fetched with its first tiles.  GATE: the
  // head's confidence scale too.
  float sg, sb, hscale = 0.f;
  auto fetch_scalars = [&](const SeqIndex& s) {
    const unsigned st = (unsigned)d.H * 4, bytes = s.len > 0 ? (unsigned)(s.len - 1) * st + 4 : 0;
    const long th = token_head(d, s.b, s.n * d.chunk, s.h);
    const unsigned off = threadIdx.x < 64 ? threadIdx.x * st : kNoRow;
    sg = buf_load1(buf_rsrc(log_decay + th, bytes), off);
    sb = buf_load1(buf_rsrc(beta + th, bytes), off);
    if constexpr (GATE) hscale = mg.scale[s.h];
  };
  auto fetch_keys = [&](const SeqIndex& s) {
    if constexpr (MIX) {
      rk.fetch_mix_keys(s.len, mix, d, s.b, s.h, s.n * d.chunk);
    } else {
      fetch_tokens(rk, s.len, rows_of(keys, d, s));
    }
  };
  // GATE: the read rows of value tile v of chunk s (zero past the chunk),
  // this lane's accumulator rows, for the variance cotangent.  Tile 0's
  // load with the chunk's first tiles, the others' before their products.
  f4 rq[4];
  auto fetch_read = [&](const SeqIndex& s, int v) {
    if constexpr (GATE) {
      const long th = token_head(d, s.b, s.n * d.chunk, s.h);
      const unsigned st = (unsigned)d.H * d.P;
      const BufRsrc rr = buf_rsrc(mg.read + th * d.P + 64 * v,
                                  s.len > 0 ? ((unsigned)(s.len - 1) * st + 64) * 4 : 0);
#pragma unroll
      for (int q = 0; q < 4; ++q) rq[q] = buf_load4(rr, ((unsigned)acc_row(w, q) * st + c4) * 4);
    }
  };
  fetch_tokens(rd, si.len, value_rows(d_output, d, si, 0));
  fetch_tokens(rv, si.len, value_rows(values, d, si, 0));
  fetch_scalars(si);
  fetch_keys(si);
  rc.fetch_matrix(cross_tile(start_c, d, si.seq, 0));
  fetch_rows_q(si);
  fetch_read(si, 0);

  for (;;) {
    rd.store(DO);
    rv.store(V);
    rc.store(C0);
    if (threadIdx.x < 64) finish_chunk_scalars(cs, sg, sb);
    const float scale = hscale;  // this chunk's head (GATE)
    __syncthreads();
    const long next = seq + gridDim.x;
    const bool more = next < nseq;  // uniform over the block
    // After a block's last chunk the same loads are issued with no rows in
    // range (zeros, no memory access), so each wait counts exactly.
    SeqIndex sn = seq_at(d, more ? next : seq);
    if (!more) sn.len = 0;

    // Both products sum over the value tiles: dout_t . v_s and C0^T dout_t.
    f4 acc[4], inh[4];
    zero4(acc);
    zero4(inh);
    // GATE: d_out_t . read_t and d_out_t . value_t of this lane's rows.
    float dotr[4] = {0.f, 0.f, 0.f, 0.f}, dotv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int v = 0; v < nv; ++v) {
      if (v > 0) {
        // Tile v replaces tile v - 1 once every wave has read it.
        fetch_tokens(rd, si.len, value_rows(d_output, d, si, v));
        fetch_tokens(rv, si.len, value_rows(values, d, si, v));
        rc.fetch_matrix(cross_tile(start_c, d, si.seq, v));
        __syncthreads();
        rd.store(DO);
        rv.store(V);
        rc.store(C0);
        __syncthreads();
      }
      // The last chunk of a block fetches its own inputs again (unused):
      // every chunk issues the same loads, so each wait counts exactly.
      if (v == nv - 1) {
        fetch_tokens(rd, sn.len, value_rows(d_output, d, sn, 0));
        fetch_tokens(rv, sn.len, value_rows(values, d, sn, 0));
        rc.fetch_matrix(cross_tile(start_c, d, sn.seq, 0), more);
        fetch_scalars(sn);
      }
      if (v > 0) fetch_read(si, v);  // in flight during the products
      tile_mma_causal<false>(acc, DO, V, w);      // dout_t . v_s, s <= t
      tile_mma<false, false>(inh, DO, C0, 64, w);  // C0^T dout_t
      if constexpr (GATE) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int t = acc_row(w, q);
          const f4 dq = *reinterpret_cast<const f4*>(DO + t * LDT + c4);
          const f4 vq = *reinterpret_cast<const f4*>(V + t * LDT + c4);
          dotr[q] += dq[0] * rq[q][0] + dq[1] * rq[q][1] + dq[2] * rq[q][2] + dq[3] * rq[q][3];
          dotv[q] += dq[0] * vq[0] + dq[1] * vq[1] + dq[2] * vq[2] + dq[3] * vq[3];
        }
      }
    }
    fetch_read(sn, 0);  // the next chunk's first read rows
    // GATE: each row's gate, its variance cotangent and the chunk's
    // contributions to the gate parameters' gradients.
    float gate[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (GATE) {
      float pscale = 0.f, pskip = 0.f;
      // Per row (once per row): log1p(var), the gate and d log1p / d var.
      float lvs[4], slopes[4];
      per_row<4>(gvar, lvs, [](float v) { return log1pf(v); });
      per_row<4>(gvar, slopes, [&](float v) { return -scale / (1.f + v); });
      per_row<4>(gvar, gate, [&](float v) { return read_gate(scale, v); });
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = acc_row(w, q);
        const float dr = row16_sum(dotr[q]), dsk = row16_sum(dotv[q]);
        const float lv = lvs[q];
        const float slope = dr * gate[q] * (1.f - gate[q]);
        dvar[q] += slope * slopes[q];
        if ((lane_id() & 15) == 0 && t < si.len)
          mg.d_var[token_head(d, si.b, si.n * d.chunk + t, si.h)] = dvar[q];
        // Rows past the chunk read zeros: their terms vanish.
        pscale += -slope * lv;
        pskip += dsk;
      }
      pscale = group4_sum(pscale);
      pskip = group4_sum(pskip);
      if (lane_id() == 0) {
        epart[threadIdx.x >> 6][0] = pscale;
        epart[threadIdx.x >> 6][1] = pskip;
      }
    }
    causal_weights<GATE>(acc, G, cs, si.len, w, gate);
    __syncthreads();
    if constexpr (GATE)
      // The chunk's gate-parameter partials, the four waves' in order.
      if (threadIdx.x < 2) {
        const long at = ((long)si.h * 2 + threadIdx.x) * ((long)d.B * d.NC) +
                        (long)si.b * d.NC + si.n;
        mg.dy_part[at] = ((epart[0][threadIdx.x] + epart[1][threadIdx.x]) +
                          epart[2][threadIdx.x]) + epart[3][threadIdx.x];
      }
    if constexpr (MIX)
      rk.store_unit(V, mix.key_shift && !mix.previous && si.n == 0);
    else
      rk.store(V);
    __syncthreads();
    fetch_keys(sn);

    f4 within[4];
    zero4(within);
    // sum_s G[t][s] k_s: G[t][s] is zero past s = t
    tile_mma_causal_terms<false, false>(within, G, V, si.len, w);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int t = acc_row(w, q);
      if (t < si.len) {
        const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
        const float carried = expf(cs.prefix[t]);
        const f4 qn = MIX ? mix_unit(qv[q].get()) : qv[q].get();
        *reinterpret_cast<f4*>(ybar + th * 64 + c4) =
            quad_row(within, q) + (carried * gate[q]) * quad_row(inh, q) + dvar[q] * qn;
      }
    }
    if (!more) break;
    fetch_rows_q(sn);
    __syncthreads();  // the tiles and scalars are read; the next chunk may overwrite them
    si = sn;
    seq = next;
  }
}

// Eight waves per chunk: wave w8 computes the 16-row strip ws of every
// product, columns of half hf = w8 / 4 (two of the four 16-column blocks;
// tile_mma_half), so each SIMD runs two waves of one chunk and one wave's
// epilogue, LDS staging and barriers overlap the other's MFMAs.  Row sums
// that span both halves meet in LDS and are added in half order.
//
// The causal products skip what the mask zeroes: the within-chunk scores
// (phase 1) only their blocks with s <= t, the masked contractions over t
// (phase 2) only their terms t >= s.  Strip ws then costs ws + 1 blocks in
// phase 1 and 4 - ws term blocks in phase 2, so the strips are paired
// {k, 3 - k} on the waves k and k + 4 that share a SIMD (ws = w8 for
// w8 < 4, 7 - w8 above).
//
// Persistent, one block per compute unit (the seven tiles take 122 KB of
// LDS): block i handles chunks i, i + gridDim.x, ...  The next chunk's five
// row tiles and its scalars load into registers while this chunk is
// computed, one tile at a time between the products of phases 3-5: every
// block runs the same phases at about the same time, so issuing all of
// them at once would only move the burst (its issue stalls the waves while
// the whole chip's requests drain), not hide it.
//
// Value-dependent terms run once per 64-column value tile (NV <= 2): gv and
// H^T v sum over the tiles, d values and H k are per tile; the tiles are
// restaged in an order that starts from the tile already in LDS.
constexpr int GRADS_THREADS = 512;
constexpr int MAX_NV = 2;

//
// MIX: keys from the mixer's raw projections, shifted and normalised at
// staging (as in fwd_read_kernel).  GATE (with MIX): d_output is the
// cotangent of the mixer's gated output, gated on load (d_variance is then
// bwd_dy's mg.d_var), the values take the skip term skip d_out, and the
// gradients go through the prologue's VJP (prologue_backward_kernel's
// arithmetic): the keys' and queries' unit normalisation to the raw rows
// (key t's source row is raw key t - 1 with the shift, or the cached key),
// the gates to beta_raw and dt_raw, and per-chunk partials of the per-head
// gate-bias and a_log gradients to mg.grads_part.
template <typename In, bool MIX, bool GATE, int NV>
__global__ __launch_bounds__(GRADS_THREADS) void bwd_grads_kernel(
    Dims d, const In* __restrict__ keys, const In* __restrict__ values,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ solved, const float* __restrict__ z,
    const float* __restrict__ d_output, const float* __restrict__ d_variance,
    const float* __restrict__ start_s, const float* __restrict__ start_c,
    const float* __restrict__ end_s, const float* __restrict__ end_c,
    float* __restrict__ d_keys, float* __restrict__ d_values, float* __restrict__ d_queries,
    float* __restrict__ d_beta, float* __restrict__ d_log_decay,
    float* __restrict__ floor_part, MixerIn mix, MixerGrad mg) {
  static_assert(!GATE || MIX, "the gated backward reads the mixer's raw rows");
  extern __shared__ float smem[];
  // Value tiles per row: compile-time for one (every branch on it folds,
  // so the compiler can count the loads in flight at each wait), else read.
  const int nv = NV == 1 ? 1 : d.NV;
  float* Kt = smem;       // keys, then S0 (but for GATE)
  float* Vt = Kt + TILE;  // a value tile, then a C0 tile
  float* Yt = Vt + TILE;
  float* Zt = Yt + TILE;
  float* Dt = Zt + TILE;  // a dout tile
  float* M1 = Dt + TILE;  // W * gy transposed (M1[s][t]), then G_end
  float* M2 = M1 + TILE;  // W * (gv - gz) transposed, then an H_end tile
  // GATE: S0 in an eighth tile, so the unit keys stay in Kt for phase 5.
  float* S0t = GATE ? M2 + TILE : Kt;
  __shared__ float kinv[GATE ? 64 : 1];  // GATE: each key row's 1 / norm
  __shared__ ChunkScalars cs;
  __shared__ float colpart[4][64];
  __shared__ float rowpart[2][64], quadpart[2][64], startpart[2][64];
  __shared__ float rowE[64], colD2[64], quad[64], startdot[64];
  __shared__ float red[GRADS_THREADS];
  __shared__ f4 fpart[8][16];
  const long nseq = (long)d.B * d.H * d.NC;
  long seq = blockIdx.x;
  SeqIndex si = seq_at(d, seq);

  // The row tiles of a chunk (keys, value tile 0, y, z, dout tile 0) in the
  // tile-fetch layout, and its log decays, betas and d_variance.
  RowTile<In, GRADS_THREADS> tk, tv;
  RowTile<float, GRADS_THREADS> ty, tz, td;
  auto fetch_keys = [&](const SeqIndex& sx) {
    if constexpr (MIX) {
      tk.fetch_mix_keys(sx.len, mix, d, sx.b, sx.h, sx.n * d.chunk);
    } else {
      fetch_tokens(tk, sx.len, rows_of(keys, d, sx));
    }
  };
  // Token tt's log decay and beta in thread tt < 64, d_variance of this
  // thread's tile-fetch rows; zero past the chunk (out-of-range offsets).
  // GATE: the variance of the same rows (for their read gates).
  // GATE: the head's gate parameters too.
  float pg = 0.f, pbt = 0.f, pdv[2], pgv[2], hpar[4] = {0.f, 0.f, 0.f, 0.f};
  auto fetch_scalars = [&](const SeqIndex& sx) {
    const unsigned tt = threadIdx.x, st = (unsigned)d.H * 4;
    const unsigned bytes = sx.len > 0 ? (unsigned)(sx.len - 1) * st + 4 : 0;
    const long th = token_head(d, sx.b, sx.n * d.chunk, sx.h);
    const unsigned off = tt < 64 ? tt * st : kNoRow;
    pg = buf_load1(buf_rsrc(log_decay + th, bytes), off);
    pbt = buf_load1(buf_rsrc(beta + th, bytes), off);
    const BufRsrc rv = buf_rsrc(d_variance + th, bytes);
#pragma unroll
    for (int j = 0; j < 2; ++j) pdv[j] = buf_load1(rv, ((tt >> 4) + 32 * j) * st);
    if constexpr (GATE) {
      const BufRsrc rg = buf_rsrc(mg.variance + th, bytes);
#pragma unroll
      for (int j = 0; j < 2; ++j) pgv[j] = buf_load1(rg, ((tt >> 4) + 32 * j) * st);
      hpar[0] = mg.scale[sx.h];
      hpar[1] = mg.skip[sx.h];
      hpar[2] = mg.a_log[sx.h];
      hpar[3] = mg.dt_bias[sx.h];
    }
  };
  fetch_keys(si);
  fetch_tokens(tv, si.len, value_rows(values, d, si, 0));
  fetch_tokens(ty, si.len, rows_of(solved, d, si));
  fetch_tokens(tz, si.len, rows_of(z, d, si));
  fetch_tokens(td, si.len, value_rows(d_output, d, si, 0));
  fetch_scalars(si);

  for (;;) {
    // The thread index passes through an empty asm once per chunk, so the
    // compiler rebuilds the loop-invariant LDS and row addresses in each
    // chunk instead of keeping about ninety of them live across the loop.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int w8 = tid >> 6, ws = w8 < 4 ? w8 : 7 - w8, hf = w8 >> 2, l = tid & 63;
    const int r = l & 15, c4 = 4 * r;
    const int kt = k_terms(si.len), last = nv - 1;
    // Column blocks of this wave's half that hold some s <= t of its strip,
    // and the first t of its strip (the masked products vanish outside).
    const int causal_nj = min(2, max(0, ws - 2 * hf + 1)), t_begin = 16 * ws;
    // d_variance of this thread's tile-fetch rows (tid/16 + 32j).
    const float dvar[2] = {pdv[0], pdv[1]};
    // GATE: the read gates of those rows; the dout tiles are gated as staged.
    // This chunk's head parameters: confidence scale, skip, a_log, dt_bias.
    const float scale = hpar[0], skip = hpar[1], a_log = hpar[2], dt_bias = hpar[3];
    float gr[2] = {1.f, 1.f};
    if constexpr (GATE) per_row<2>(pgv, gr, [&](float v) { return read_gate(scale, v); });
    auto store_dout = [&](const RowTile<float, GRADS_THREADS>& t) {
      if constexpr (GATE)
        t.store_scaled(Dt, gr);
      else
        t.store(Dt);
    };

    if constexpr (MIX)
      tk.store_unit(Kt, mix.key_shift && !mix.previous && si.n == 0, GATE ? kinv : nullptr);
    else
      tk.store(Kt);
    tv.store(Vt);
    ty.store(Yt);
    tz.store(Zt);
    store_dout(td);
    if (tid < 64) finish_chunk_scalars(cs, pg, pbt);
    // The end-state cotangents of phase 3 load while phases 1 and 2 run (of H,
    // the last value tile, the one phase 3 starts from).
    TileRegs2 rg, rh;
    rg.fetch_matrix(end_s + si.seq * 4096);
    rh.fetch_matrix(cross_tile(end_c, d, si.seq, last));
    __syncthreads();

    // Phase 1: gy = Y K^T, gz = Z K^T, gv = sum over value tiles of dOut V^T,
    // and their weighted mixes.  Leaves the last value and dout tiles in LDS.
    {
      f4 gy[2], gz[2], gv[2];
      zero2(gy);
      zero2(gz);
      zero2(gv);
      tile_mma_half<false, true>(gy, Yt, Kt, 64, ws, hf, 0, causal_nj);
      tile_mma_half<false, true>(gz, Zt, Kt, 64, ws, hf, 0, causal_nj);
      tile_mma_half<false, true>(gv, Dt, Vt, 64, ws, hf, 0, causal_nj);
#pragma unroll 1
      for (int v = 1; v < nv; ++v) {
        RowTile<In, GRADS_THREADS> rv;
        RowTile<float, GRADS_THREADS> rd;
        fetch_tokens(rv, si.len, value_rows(values, d, si, v));
        fetch_tokens(rd, si.len, value_rows(d_output, d, si, v));
        __syncthreads();
        rv.store(Vt);
        store_dout(rd);
        __syncthreads();
        tile_mma_half<false, true>(gv, Dt, Vt, 64, ws, hf, 0, causal_nj);
      }
      // The mixes go to LDS transposed, M[s][t] (a lane's four accumulator
      // rows t are adjacent there: one 16-byte store per column block), so
      // phase 2 reads them as row-major A operands.
      float rsum[4] = {0.f, 0.f, 0.f, 0.f};
      float csum[2] = {0.f, 0.f};
      // Column block jb lies below the strip's diagonal (jb < ws), on it
      // (jb = ws) or above it (jb > ws: all zero, no exponentials); the mask
      // is a select, not a branch per element.
      const int wsu = __builtin_amdgcn_readfirstlane(ws), hfu = __builtin_amdgcn_readfirstlane(hf);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int jb = 2 * hfu + j, s = 16 * jb + r;
        f4 m1v = {0.f, 0.f, 0.f, 0.f}, m2v = {0.f, 0.f, 0.f, 0.f};
        if (jb <= wsu) {
          const float ps = cs.prefix[s], bs = cs.beta[s];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int t = acc_row(ws, q);
            const bool keep = t < si.len && (jb < wsu || s <= t);
            const float dec = expf(cs.prefix[t] - ps);
            const float mix = gv[j][q] - gz[j][q];
            const float d2 = keep ? dec * gy[j][q] * mix : 0.f;
            m1v[q] = keep ? dec * bs * gy[j][q] : 0.f;
            m2v[q] = keep ? dec * bs * mix : 0.f;
            rsum[q] += bs * d2;
            csum[j] += d2;
          }
        }
        *reinterpret_cast<f4*>(M1 + s * LDT + acc_row(ws, 0)) = m1v;
        *reinterpret_cast<f4*>(M2 + s * LDT + acc_row(ws, 0)) = m2v;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v = row16_sum(rsum[q]);
        if (r == 0) rowpart[hf][acc_row(ws, q)] = v;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float v = group4_sum(csum[j]);
        if (l < 16) colpart[ws][16 * (2 * hf + j) + r] = v;
      }
    }
    __syncthreads();
    if (tid < 64) {
      const int s = tid;
      colD2[s] = colpart[0][s] + colpart[1][s] + colpart[2][s] + colpart[3][s];
      rowE[s] = rowpart[0][s] + rowpart[1][s];
    }

    // Phase 2: within-chunk key gradient and the value gradient of each tile
    // (rows s, QUAD columns 4r + 2hf + j).  Tiles from the last down, so the
    // first dout tile is in LDS afterwards.
    f4 dk[2], dv[MAX_NV][2];
    zero2(dk);
    {
      f4 tmp[2];
      zero2(tmp);
      tile_mma_half<false, false>(dk, M2, Yt, kt, ws, hf, t_begin);   // sum_t W(gv-gz)[t][s] y_t
      tile_mma_half<false, false>(tmp, M1, Zt, kt, ws, hf, t_begin);  // sum_t W gy[t][s] z_t
#pragma unroll
      for (int j = 0; j < 2; ++j) dk[j] -= tmp[j];
    }
#pragma unroll
    for (int v = MAX_NV - 1; v >= 0; --v) {
      zero2(dv[v]);
      if (v < nv) {
        if (v < last) {
          RowTile<float, GRADS_THREADS> rd;
          fetch_tokens(rd, si.len, value_rows(d_output, d, si, v));
          __syncthreads();
          store_dout(rd);
          __syncthreads();
        }
        tile_mma_half<false, false>(dv[v], M1, Dt, kt, ws, hf, t_begin);  // sum_t W gy[t][s] dout_t
      }
    }
    __syncthreads();

    float2 dkq[4];  // GATE: this thread's d keys until M1 is free
    // Phase 3: chunk-end terms through the end-state cotangents G, H:
    // (G + G^T) k_s as one product (the evidence walk stores G + G^T, which
    // is symmetric).  H and the values go tile by tile from the last, leaving
    // the first tile of each in LDS.
    rg.store(M1);
    rh.store(M2);
    // The start states of phase 4 load while phase 3 runs, then the first of
    // the next chunk's tiles.
    const long bh = si.seq / d.NC;
    TileRegs2 rs, rc;
    const long next = seq + gridDim.x;
    const bool more = next < nseq;  // uniform over the block
    // The last chunk of a block fetches its own tiles again (unused): every
    // load stays unconditional.  (Issuing them with no rows in range instead,
    // as fwd_read and bwd_dy do, ran 2 us slower here.)
    const SeqIndex sx = seq_at(d, more ? next : seq);
    // The two waves on a SIMD (ws, hf = 0 and 1) issue these loads before
    // and after their first product, so one computes while the other waits
    // to issue.
    auto fetch_phase4 = [&]() {
      rs.fetch_matrix(start_s + (bh * d.NS + (long)si.n * d.rsub) * 4096);
      rc.fetch_matrix(cross_tile(start_c, d, si.seq, 0));
      fetch_tokens(ty, sx.len, rows_of(solved, d, sx));
    };
    if (hf == 0) fetch_phase4();
    __syncthreads();
    {
      f4 gk[2], hv[2];
      zero2(gk);
      zero2(hv);
      if (hf == 0) fetch_tokens(tz, sx.len, rows_of(z, d, sx));
      tile_mma_half<false, false>(gk, Kt, M1, 64, ws, hf);  // (G + G^T) k_s
      if (hf == 1) {
        fetch_phase4();
        fetch_tokens(tz, sx.len, rows_of(z, d, sx));
      }
      float qpart[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float2 kr = *reinterpret_cast<const float2*>(Kt + acc_row(ws, q) * LDT + c4 + 2 * hf);
        qpart[q] += 0.5f * kr.x * gk[0][q] + 0.5f * kr.y * gk[1][q];
      }
#pragma unroll
      for (int v = MAX_NV - 1; v >= 0; --v) {
        if (v < nv) {
          if (v < last) {
            RowTile<In, GRADS_THREADS> rv;
            TileRegs2 rhv;
            fetch_tokens(rv, si.len, value_rows(values, d, si, v));
            rhv.fetch_matrix(cross_tile(end_c, d, si.seq, v));
            __syncthreads();
            rv.store(Vt);
            rhv.store(M2);
            __syncthreads();
          }
          // GATE: the skip term's d_out rows, in flight during the products.
          float2 sk_dout[4];
          if constexpr (GATE) {
            const unsigned st = (unsigned)d.H * d.P;
            const long th0 = token_head(d, si.b, si.n * d.chunk, si.h);
            const BufRsrc ro = buf_rsrc(mg.d_out + th0 * d.P + 64 * v,
                                        ((unsigned)(si.len - 1) * st + 64) * 4);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              sk_dout[q] = buf_load2(ro, ((unsigned)acc_row(ws, q) * st + c4 + 2 * hf) * 4);
          }
          f4 hk[2];
          zero2(hk);
          tile_mma_half<false, true, true>(hk, Kt, M2, 64, ws, hf);  // H k_s
          tile_mma_half<false, false>(hv, Vt, M2, 64, ws, hf);       // H^T v_s, summed
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int s = acc_row(ws, q);
            const float2 vr = *reinterpret_cast<const float2*>(Vt + s * LDT + c4 + 2 * hf);
            qpart[q] += vr.x * hk[0][q] + vr.y * hk[1][q];
            if (s < si.len) {
              const float tl = cs.tail[s];
              const long th = token_head(d, si.b, si.n * d.chunk + s, si.h);
              const long at = th * d.P + 64 * v + c4 + 2 * hf;
              float2 gv2 = float2{dv[v][0][q] + tl * hk[0][q], dv[v][1][q] + tl * hk[1][q]};
              if constexpr (GATE) {
                // The skip's term of the value gradient: skip d_out.
                gv2.x += skip * sk_dout[q].x;
                gv2.y += skip * sk_dout[q].y;
              }
              *reinterpret_cast<float2*>(d_values + at) = gv2;
            }
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int s = acc_row(ws, q);
        const float qv = row16_sum(qpart[q]);
        if (r == 0) quadpart[hf][s] = qv;
        const float tl = cs.tail[s];
        const float2 dkv =
            float2{dk[0][q] + tl * (gk[0][q] + hv[0][q]), dk[1][q] + tl * (gk[1][q] + hv[1][q])};
        if constexpr (GATE) {
          dkq[q] = dkv;  // staged in M1 once G is read (phase 5 takes it to the raw rows)
        } else if (s < si.len) {
          const long th = token_head(d, si.b, si.n * d.chunk + s, si.h);
          *reinterpret_cast<float2*>(d_keys + th * 64 + c4 + 2 * hf) = dkv;
        }
      }
    }
    __syncthreads();
    if constexpr (GATE)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float2*>(M1 + acc_row(ws, q) * LDT + c4 + 2 * hf) = dkq[q];
    if (tid < 64) quad[tid] = quadpart[0][tid] + quadpart[1][tid];
    fetch_keys(sx);
    // GATE: the raw query rows of this thread's tile-fetch rows (zero past
    // the chunk), for phase 5; in flight during phase 4.
    f4 xq[2];
    if constexpr (GATE) {
      const unsigned st = (unsigned)d.H * 64;
      const BufRsrc rq = buf_rsrc(mix.query + token_head(d, si.b, si.n * d.chunk, si.h) * 64,
                                  ((unsigned)(si.len - 1) * st + 64) * 4);
#pragma unroll
      for (int j = 0; j < 2; ++j) xq[j] = buf_load4(rq, (((tid >> 4) + 32 * j) * st + c4) * 4);
    }

    // Phase 4: start-state terms <A_bar_t, S0>, <C_bar_t, C0> and <G,S0>+<H,C0>,
    // the C0 terms summed over the value tiles from the first (whose H and
    // dout tiles are in LDS).  <G, S0> and, with one value tile, <H, C0> come
    // from the fetch registers (both operands in the same layout).  The
    // chunk's start evidence is the start of its first sub-chunk.
    rs.store(S0t);
    rc.store(Vt);
    __syncthreads();
    {
      // <G, S0> = <G + G^T, S0> / 2 (S0 symmetric).
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) part += rg.v[j][i] * rs.v[j][i];
      part *= 0.5f;
      f4 ys[2], dc[2];
      zero2(ys);
      zero2(dc);
      tile_mma_half<false, false>(ys, Yt, S0t, 64, ws, hf);  // y_t^T S0
      fetch_tokens(tv, sx.len, value_rows(values, d, sx, 0));
#pragma unroll 1
      for (int v = 0; v < nv; ++v) {
        if (v > 0) {
          TileRegs2 rhv, rcv;
          RowTile<float, GRADS_THREADS> rd;
          rhv.fetch_matrix(cross_tile(end_c, d, si.seq, v));
          rcv.fetch_matrix(cross_tile(start_c, d, si.seq, v));
          fetch_tokens(rd, si.len, value_rows(d_output, d, si, v));
          __syncthreads();
          rhv.store(M2);
          rcv.store(Vt);
          store_dout(rd);
          __syncthreads();
        }
        if (nv == 1) {
#pragma unroll
          for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) part += rh.v[j][i] * rc.v[j][i];
        } else {
          for (int e = tid; e < 4096; e += GRADS_THREADS) {
            const int row = e >> 6, col = e & 63;
            part += M2[row * LDT + col] * Vt[row * LDT + col];
          }
        }
        tile_mma_half<false, false>(dc, Dt, Vt, 64, ws, hf);  // dout_t^T C0, summed
      }
      red[tid] = part;
      fetch_tokens(td, sx.len, value_rows(d_output, d, sx, 0));
      fetch_scalars(sx);
      float sp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int t = acc_row(ws, q);
        const float2 yr = *reinterpret_cast<const float2*>(Yt + t * LDT + c4 + 2 * hf);
        const float2 zr = *reinterpret_cast<const float2*>(Zt + t * LDT + c4 + 2 * hf);
        sp[q] += dc[0][q] * yr.x - ys[0][q] * zr.x;
        sp[q] += dc[1][q] * yr.y - ys[1][q] * zr.y;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v = row16_sum(sp[q]);
        if (r == 0) startpart[hf][acc_row(ws, q)] = v;
      }
    }
    __syncthreads();
    if (tid < 64) {
      const int t = tid;
      startdot[t] = expf(cs.prefix[t]) * (startpart[0][t] + startpart[1][t]);
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < GRADS_THREADS / 64; ++k) v += red[t + 64 * k];
      v = group4_sum(row16_sum(v));
      red[t] = v;  // every lane of wave 0 holds the total
    }
    __syncthreads();

    // Phase 5: beta and log-decay gradients (wave 0), queries and floor.
    if (tid < 64) {
      const int t = tid;
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
      const float suffix = wave_suffix_sum(dp);
      const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
      if constexpr (GATE) {
        // The gates' VJP: beta = beta_max sigmoid(beta_raw + bias), so
        // d beta_raw = d beta beta (1 - beta / beta_max); log decay =
        // -exp(a_log) softplus(dt_raw + bias), so d dt_raw = d log_decay
        // (-exp(a_log) sigmoid(dt_raw + bias)) and d a_log = d log_decay
        // log_decay.  Past the chunk every term is zero (zero loads).
        const unsigned st = (unsigned)d.H * 4;
        const long th0 = token_head(d, si.b, si.n * d.chunk, si.h);
        const unsigned bytes = (unsigned)(si.len - 1) * st + 4;
        const float draw = buf_load1(buf_rsrc(mg.dt_raw + th0, bytes), t * st);
        const float ld = buf_load1(buf_rsrc(log_decay + th0, bytes), t * st);
        const float bt = cs.beta[t];
        const float dbr = mg.beta_max != 0.f ? db * bt * (1.f - bt / mg.beta_max) : 0.f;
        const float ddt = -suffix * expf(a_log) * mix_sigmoid(draw + dt_bias);
        if (t < si.len) {
          mg.d_beta_raw[th] = dbr;
          mg.d_dt_raw[th] = ddt;
        }
        const float sums[3] = {group4_sum(row16_sum(t < si.len ? dbr : 0.f)),
                               group4_sum(row16_sum(t < si.len ? ddt : 0.f)),
                               group4_sum(row16_sum(t < si.len ? suffix * ld : 0.f))};
        if (t < 3) {
          const long at = ((long)si.h * 3 + t) * ((long)d.B * d.NC) + (long)si.b * d.NC + si.n;
          mg.grads_part[at] = t == 0 ? sums[0] : t == 1 ? sums[1] : sums[2];
        }
      } else if (t < si.len) {
        d_beta[th] = db;
        d_log_decay[th] = suffix;
      }
    }
    // Queries, d q_t = z_t + dvar_t y_t, in the tile-fetch layout (rows
    // r0 + 32j, columns c4..c4+3), and the floor partial -sum_t z_t * y_t:
    // per thread over its two rows, then over the lanes and waves holding the
    // same columns, in a fixed order.
    {
      f4 fsum = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = (tid >> 4) + 32 * j;
        const f4 zr = *reinterpret_cast<const f4*>(Zt + t * LDT + c4);
        const f4 yr = *reinterpret_cast<const f4*>(Yt + t * LDT + c4);
        const long th = token_head(d, si.b, si.n * d.chunk + t, si.h);
        if constexpr (GATE) {
          // Through the unit normalisations to the raw rows (mix_unit_vjp):
          // the queries from their raw rows, the keys from their unit rows
          // (still in Kt) and 1 / norms.
          const int tp = si.n * d.chunk + t;  // position in the sequence
          const bool in = t < si.len;
          const float rq = mix_inv_norm(xq[j]);
          const f4 dq = mix_unit_vjp(xq[j] * rq, rq, zr + dvar[j] * yr);
          if (in) *reinterpret_cast<f4*>(mg.d_query + th * 64 + c4) = dq;
          // Key t's source row: raw key t - 1 with the shift (position 0:
          // the cached key, or none: a zero row, whose cotangent is zero).
          const f4 dk = mix_unit_vjp(*reinterpret_cast<const f4*>(Kt + t * LDT + c4), kinv[t],
                                     *reinterpret_cast<const f4*>(M1 + t * LDT + c4));
          const bool zero_src = mix.key_shift && tp == 0 && !mix.previous;
          float* dst = nullptr;
          if (in) {
            if (!mix.key_shift)
              dst = mg.d_key + th * 64;
            else if (tp > 0)
              dst = mg.d_key + token_head(d, si.b, tp - 1, si.h) * 64;
            else if (mg.d_previous)
              dst = mg.d_previous + ((long)si.b * d.H + si.h) * 64;
          }
          if (dst) *reinterpret_cast<f4*>(dst + c4) = zero_src ? f4{0.f, 0.f, 0.f, 0.f} : dk;
          // The last raw key feeds only the cache entry (its cotangent,
          // or zero); without the shift the cached key feeds nothing.
          if (in && mix.key_shift && tp == d.T - 1)
            *reinterpret_cast<f4*>(mg.d_key + th * 64 + c4) =
                mg.d_shifted ? *reinterpret_cast<const f4*>(
                                   mg.d_shifted + ((long)si.b * d.H + si.h) * 64 + c4)
                             : f4{0.f, 0.f, 0.f, 0.f};
          if (in && tp == 0 && mg.d_previous && !mix.key_shift)
            *reinterpret_cast<f4*>(mg.d_previous + ((long)si.b * d.H + si.h) * 64 + c4) =
                f4{0.f, 0.f, 0.f, 0.f};
        } else if (t < si.len) {
          *reinterpret_cast<f4*>(d_queries + th * 64 + c4) = zr + dvar[j] * yr;
        }
        fsum -= zr * yr;  // zero past the chunk's tokens
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) fsum[i] = group4_sum(fsum[i]);
      if (l < 16) fpart[w8][l] = fsum;
      __syncthreads();
      if (tid < 16) {
        f4 total = fpart[0][tid];
#pragma unroll
        for (int k = 1; k < 8; ++k) total += fpart[k][tid];
        *reinterpret_cast<f4*>(floor_part + si.seq * 64 + 4 * tid) = total;
      }
    }
    if (!more) break;
    seq = next;
    si = sx;
    __syncthreads();  // phase 5 has read the tiles and partial sums
  }
}

#define M4_CHUNK_KERNELS(In, MIX, GATE, NV)                                                   \
  template __global__ void bwd_dy_kernel<In, MIX, GATE, NV>(                                   \
      Dims, const In*, const In*, const In*, const float*, const float*, const float*,         \
      const float*, const float*, float*, MixerIn, MixerGrad);                                 \
  template __global__ void bwd_grads_kernel<In, MIX, GATE, NV>(                                \
      Dims, const In*, const In*, const float*, const float*, const float*, const float*,      \
      const float*, const float*, const float*, const float*, const float*, const float*,      \
      float*, float*, float*, float*, float*, float*, MixerIn, MixerGrad);
#define M4_READ_KERNEL(In, MIX, NV)                                                           \
  template __global__ void fwd_read_kernel<In, MIX, NV>(                                       \
      Dims, const In*, const In*, const In*, const float*, const float*, const float*,         \
      const float*, float*, float*, MixerIn, ReadGate);
M4_READ_KERNEL(float, false, 1)
M4_READ_KERNEL(float, false, 2)
M4_READ_KERNEL(bf16_t, false, 1)
M4_READ_KERNEL(bf16_t, false, 2)
M4_READ_KERNEL(float, true, 1)
M4_READ_KERNEL(float, true, 2)
M4_CHUNK_KERNELS(float, false, false, 1)
M4_CHUNK_KERNELS(float, false, false, 2)
M4_CHUNK_KERNELS(bf16_t, false, false, 1)
M4_CHUNK_KERNELS(bf16_t, false, false, 2)
M4_CHUNK_KERNELS(float, true, false, 1)
M4_CHUNK_KERNELS(float, true, false, 2)
M4_CHUNK_KERNELS(float, true, true, 1)
M4_CHUNK_KERNELS(float, true, true, 2)
#undef M4_READ_KERNEL
#undef M4_CHUNK_KERNELS

// d floor[h][4c4 .. 4c4+3] = sum over (b, n) of floor_part[(b*H + h)*NC + n]
// in a fixed order: block (h, c4) of 256 threads, thread i sums entries
// e = i, i + 256, ... of the flattened (b, n) index, then a fixed tree adds
// the 256 partials.  Deterministic run to run.
// floor_raw (the mixer's fused backward; may be null): the result is carried
// through floor = floor_min + softplus(floor_raw), d floor_raw = d floor
// sigmoid(floor_raw).
__device__ __forceinline__ void floor_block(const Dims& d, const float* __restrict__ part,
                                            float* __restrict__ d_floor,
                                            const float* __restrict__ floor_raw, int h, int c4,
                                            f4* partial) {
  const int entries = d.B * d.NC;
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  for (int e = threadIdx.x; e < entries; e += 256) {
    const int b = e / d.NC, n = e % d.NC;
    acc += *reinterpret_cast<const f4*>(part + (((long)b * d.H + h) * d.NC + n) * 64 + 4 * c4);
  }
  partial[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) partial[threadIdx.x] += partial[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    f4 out = partial[0];
    if (floor_raw) {
      const f4 fr = *reinterpret_cast<const f4*>(floor_raw + h * 64 + 4 * c4);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e] *= mix_sigmoid(fr[e]);
    }
    *reinterpret_cast<f4*>(d_floor + h * 64 + 4 * c4) = out;
  }
}

__global__ __launch_bounds__(256) void floor_reduce_kernel(Dims d, const float* __restrict__ part,
                                                          float* __restrict__ d_floor,
                                                          const float* __restrict__ floor_raw) {
  __shared__ f4 partial[256];
  floor_block(d, part, d_floor, floor_raw, blockIdx.x >> 4, blockIdx.x & 15, partial);
}

// The fused mixer backward's last launch: blocks 0 .. 16H - 1 reduce the
// floor_raw gradient (floor_block), the next 5H the per-head parameter
// gradients from the per-chunk partials (B NC of them per head and
// parameter): block 16H + 5h + j sums dy_part[(2h + j) B NC ..] for j < 2
// (d confidence_scale, d skip) or grads_part[(3h + j - 2) B NC ..] (d
// beta_bias, d dt_bias, d a_log), thread i over entries i, i + 256, ... in
// order, then a fixed tree.  Deterministic run to run.
__global__ __launch_bounds__(256) void mixer_finish_kernel(
    Dims d, const float* __restrict__ floor_part, float* __restrict__ d_floor_raw,
    const float* __restrict__ floor_raw, const float* __restrict__ dy_part,
    const float* __restrict__ grads_part, float* __restrict__ d_scale,
    float* __restrict__ d_skip, float* __restrict__ d_beta_bias, float* __restrict__ d_dt_bias,
    float* __restrict__ d_a_log) {
  __shared__ f4 partial[256];
  const int floor_blocks = d.H * 16;
  if ((int)blockIdx.x < floor_blocks) {
    floor_block(d, floor_part, d_floor_raw, floor_raw, blockIdx.x >> 4, blockIdx.x & 15,
                partial);
    return;
  }
  const int k = blockIdx.x - floor_blocks, h = k / 5, j = k % 5;
  const long chunks = (long)d.B * d.NC;
  const float* src = j < 2 ? dy_part + (2L * h + j) * chunks : grads_part + (3L * h + j - 2) * chunks;
  float acc = 0.f;
  for (long e = threadIdx.x; e < chunks; e += 256) acc += src[e];
  float* red = reinterpret_cast<float*>(partial);
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float* out = j == 0 ? d_scale : j == 1 ? d_skip : j == 2 ? d_beta_bias : j == 3 ? d_dt_bias
                                                                                      : d_a_log;
    out[h] = red[0];
  }
}

}  // namespace m4
