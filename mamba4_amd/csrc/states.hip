// Chunk-boundary states: chunk statistics on MFMA plus an elementwise scan.
//
// Forward (lm/kernels/mamba4_fused.py:411-425 with chunk_carry,
// lm/kernels/prefix.py:27-44).  fwd_stats_kernel computes, for every chunk
// in parallel, the statistics K^T diag(tail) K of each sub-chunk and
// V^T diag(tail) K of the chunk, tail_s = beta_s exp(P_last - P_s), and
// writes them into the start-state buffers.  fwd_scan_kernel then turns them
// into start states in place, walking chunks in order per matrix element:
//   start[u] = running;  running = exp(sum of log decays in u) running + stat[u]
// and writes the final state.
//
// Value-dependent states (cross statistics and their cotangents) are NV
// stacked 64x64 tiles per state; each tile is one more product, and the scans
// treat the NV * 4096 elements of a cross state alike.
//
// Backward: the transpose of that carry.  bwd_local_kernel computes each
// chunk's start-state cotangents U = -(M + M^T)/2, M = Z^T diag(e^P) Y, and
// V = dOut^T diag(e^P) Y; bwd_scan_kernel walks chunks in reverse,
//   end[n] = running;  running = U_n + exp(sum of log decays in n) running,
// leaving each chunk's end-state cotangent and the initial-state gradient.
// The evidence end-state cotangents G are stored as G + G^T: every use the
// chunk gradients make of G is through its symmetric part ((G + G^T) k,
// k^T G k, <G, S> with S symmetric), and a symmetric G + G^T takes one
// product where G itself takes two.
#include "common.hpp"

namespace m4 {

__device__ __forceinline__ float* mat(float* base, long index) { return base + index * 4096; }

template <typename In>
__global__ __launch_bounds__(256) void fwd_stats_kernel(
    Dims d, const In* __restrict__ keys, const In* __restrict__ values,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    float* __restrict__ start_s, float* __restrict__ start_c) {
  extern __shared__ float smem[];
  float* K = smem;
  float* V = K + TILE;
  float* W = V + TILE;
  __shared__ ChunkScalars cs;
  const long seq = blockIdx.x;
  const int n = (int)(seq % d.NC), bh = (int)(seq / d.NC), b = bh / d.H, h = bh % d.H;
  const int len = chunk_len(d, n), w = threadIdx.x >> 6, c4 = 4 * (lane_id() & 15);
  const int kt = k_terms(len);
  auto rows = [&](const In* base, int width, int offset) {
    return [=](int s) { return base + token_head(d, b, n * d.chunk + s, h) * width + offset; };
  };
  TileRegs rk, rv;
  rk.fetch_rows(len, rows(keys, 64, 0));
  rv.fetch_rows(len, rows(values, d.P, 0));
  rk.store(K);
  rv.store(V);
  load_chunk_scalars(cs, d, beta, log_decay, b, h, n);
  __syncthreads();

  for (int u = 0; u < d.rsub; ++u) {
    const int first = sub_first(d, u), cnt = sub_len(d, n, u);
    const float p_end = cnt > 0 ? cs.prefix[first + cnt - 1] : 0.f;
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
      const int s = e >> 6, c = e & 63;
      const bool in = s >= first && s < first + cnt;
      W[s * LDT + c] = in ? cs.beta[s] * expf(p_end - cs.prefix[s]) * K[s * LDT + c] : 0.f;
    }
    __syncthreads();
    f4 acc[4];
    zero4(acc);
    tile_mma<true, false>(acc, W, K, kt, w);  // sum_s tail_s k_s k_s^T
    float* out = mat(start_s, (long)bh * d.NS + (long)n * d.rsub + u);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f4*>(out + acc_row(w, q) * 64 + c4) = quad_row(acc, q);
    __syncthreads();
  }
  for (int v = 0; v < d.NV; ++v) {
    if (v > 0) {
      // Value tile v replaces tile v - 1 once every wave has read it.
      rv.fetch_rows(len, rows(values, d.P, 64 * v));
      __syncthreads();
      rv.store(V);
      __syncthreads();
    }
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
      const int s = e >> 6, c = e & 63;
      W[s * LDT + c] = s < len ? cs.tail[s] * V[s * LDT + c] : 0.f;
    }
    __syncthreads();
    f4 acc[4];
    zero4(acc);
    tile_mma<true, false>(acc, W, K, kt, w);  // sum_s tail_s v_s k_s^T
    float* out = mat(start_c, ((long)bh * d.NC + n) * d.NV + v);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f4*>(out + acc_row(w, q) * 64 + c4) = quad_row(acc, q);
  }
}

// exp(sum of log decays) over the tokens of step `i` of the scan: a
// sub-chunk (evidence) or a chunk (cross statistics).
__device__ __forceinline__ float step_decay(const Dims& d, const float* log_decay, int b, int h,
                                            int i, bool sub) {
  int first, cnt;
  if (sub) {
    const int n = i / d.rsub, u = i % d.rsub;
    first = n * d.chunk + sub_first(d, u);
    cnt = sub_len(d, n, u);
  } else {
    first = i * d.chunk;
    cnt = chunk_len(d, i);
  }
  float g = 0.f;
#pragma unroll 8
  for (int t = 0; t < cnt; ++t) g += log_decay[token_head(d, b, first + t, h)];
  return expf(g);
}

// Steps of a scan whose loads are issued together.
constexpr int SCAN_BATCH = 8;

// Grid (B*H, 4 + 4 NV): y in 0..3 scans evidence elements [1024y, 1024y+1024)
// over the NS sub-chunks, y >= 4 the cross-statistic elements
// [1024(y-4), 1024(y-3)) of the NV * 4096 per state over NC chunks.
__global__ __launch_bounds__(256) void fwd_scan_kernel(
    Dims d, const float* __restrict__ log_decay, const float* __restrict__ init_s,
    const float* __restrict__ init_c, float* __restrict__ start_s, float* __restrict__ start_c,
    float* __restrict__ final_s, float* __restrict__ final_c) {
  const int bh = blockIdx.x, b = bh / d.H, h = bh % d.H;
  const bool cross = blockIdx.y >= 4;
  const int elem = 1024 * (cross ? blockIdx.y - 4 : blockIdx.y) + 4 * threadIdx.x;
  const int steps = cross ? d.NC : d.NS;
  const long size = cross ? 4096L * d.NV : 4096L;  // floats per state
  float* buf = (cross ? start_c : start_s) + (long)bh * steps * size;
  const float* init = cross ? init_c : init_s;
  __shared__ float decay[256];
  f4 running = f4{0.f, 0.f, 0.f, 0.f};
  if (init) running = *reinterpret_cast<const f4*>(init + (long)bh * size + elem);
  for (int base = 0; base < steps; base += 256) {
    const int count = min(256, steps - base);
    __syncthreads();
    if (threadIdx.x < count)
      decay[threadIdx.x] = step_decay(d, log_decay, b, h, base + threadIdx.x, !cross);
    __syncthreads();
    for (int i0 = 0; i0 < count; i0 += SCAN_BATCH) {
      const int m = min(SCAN_BATCH, count - i0);
      f4 stat[SCAN_BATCH];
#pragma unroll
      for (int j = 0; j < SCAN_BATCH; ++j)
        if (j < m) stat[j] = *reinterpret_cast<const f4*>(buf + (long)(base + i0 + j) * size + elem);
#pragma unroll
      for (int j = 0; j < SCAN_BATCH; ++j)
        if (j < m) {
          *reinterpret_cast<f4*>(buf + (long)(base + i0 + j) * size + elem) = running;
          running = decay[i0 + j] * running + stat[j];
        }
    }
  }
  float* fin = cross ? final_c : final_s;
  *reinterpret_cast<f4*>(fin + (long)bh * size + elem) = running;
}

__global__ __launch_bounds__(256) void bwd_local_kernel(
    Dims d, const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ solved, const float* __restrict__ z,
    const float* __restrict__ d_output, float* __restrict__ end_s, float* __restrict__ end_c) {
  extern __shared__ float smem[];
  float* Y = smem;
  float* Zw = Y + TILE;
  float* Dw = Zw + TILE;
  float* M = Dw + TILE;
  __shared__ ChunkScalars cs;
  const long seq = blockIdx.x;
  const int n = (int)(seq % d.NC), bh = (int)(seq / d.NC), b = bh / d.H, h = bh % d.H;
  const int len = chunk_len(d, n), w = threadIdx.x >> 6, c4 = 4 * (lane_id() & 15);
  const int kt = k_terms(len);
  auto rows = [&](const float* base, int width, int offset) {
    return [=](int s) { return base + token_head(d, b, n * d.chunk + s, h) * width + offset; };
  };
  TileRegs ry, rz, rd;
  ry.fetch_rows(len, rows(solved, 64, 0));
  rz.fetch_rows(len, rows(z, 64, 0));
  rd.fetch_rows(len, rows(d_output, d.P, 0));
  ry.store(Y);
  rz.store(Zw);
  rd.store(Dw);
  load_chunk_scalars(cs, d, beta, log_decay, b, h, n);
  __syncthreads();
  for (int e = threadIdx.x; e < len * 64; e += 256) {
    const int t = e >> 6, c = e & 63;
    const float carried = expf(cs.prefix[t]);
    Zw[t * LDT + c] *= carried;
    Dw[t * LDT + c] *= carried;
  }
  __syncthreads();
  f4 acc[4];
  zero4(acc);
  tile_mma<true, false>(acc, Zw, Y, kt, w);  // M = sum_t e^P z_t y_t^T
#pragma unroll
  for (int q = 0; q < 4; ++q)
    *reinterpret_cast<f4*>(M + acc_row(w, q) * LDT + c4) = quad_row(acc, q);
  __syncthreads();
  float* us = mat(end_s, (long)bh * d.NC + n);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = acc_row(w, q);
    f4 v;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) v[jb] = -(acc[jb][q] + M[(c4 + jb) * LDT + i]);
    *reinterpret_cast<f4*>(us + i * 64 + c4) = v;
  }
  for (int v = 0; v < d.NV; ++v) {
    if (v > 0) {
      // Value tile v of the read cotangent replaces tile v - 1.
      rd.fetch_rows(len, rows(d_output, d.P, 64 * v));
      __syncthreads();
      rd.store(Dw);
      __syncthreads();
      for (int e = threadIdx.x; e < len * 64; e += 256) {
        const int t = e >> 6, c = e & 63;
        Dw[t * LDT + c] *= expf(cs.prefix[t]);
      }
      __syncthreads();
    }
    zero4(acc);
    tile_mma<true, false>(acc, Dw, Y, kt, w);  // V = sum_t e^P dout_t y_t^T
    float* uc = mat(end_c, ((long)bh * d.NC + n) * d.NV + v);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f4*>(uc + acc_row(w, q) * 64 + c4) = quad_row(acc, q);
  }
}

// Grid (B*H, 4 + 4 NV) as fwd_scan_kernel, walking chunks in reverse.
__global__ __launch_bounds__(256) void bwd_scan_kernel(
    Dims d, const float* __restrict__ log_decay, const float* __restrict__ d_final_s,
    const float* __restrict__ d_final_c, float* __restrict__ end_s, float* __restrict__ end_c,
    float* __restrict__ d_init_s, float* __restrict__ d_init_c) {
  const int bh = blockIdx.x, b = bh / d.H, h = bh % d.H;
  const bool cross = blockIdx.y >= 4;
  const int elem = 1024 * (cross ? blockIdx.y - 4 : blockIdx.y) + 4 * threadIdx.x;
  const long size = cross ? 4096L * d.NV : 4096L;  // floats per state
  float* buf = (cross ? end_c : end_s) + (long)bh * d.NC * size;
  const float* fin = cross ? d_final_c : d_final_s;
  __shared__ float decay[256];
  // Evidence: the scan carries G + G^T (it starts from D + D^T and adds the
  // local terms 2U = -(M + M^T), as bwd_local_kernel stores them), so every
  // stored end-state cotangent is symmetric; the initial-state gradient is
  // the full one, half the carried sum plus the decayed antisymmetric part
  // of D.  Cross states carry their cotangent as is.
  f4 running = f4{0.f, 0.f, 0.f, 0.f}, anti = f4{0.f, 0.f, 0.f, 0.f};
  float total = 1.f;  // the product of every chunk's decay
  if (fin) {
    running = *reinterpret_cast<const f4*>(fin + (long)bh * size + elem);
    if (!cross) {
      const int i = elem >> 6, j = elem & 63;
      f4 tr;
#pragma unroll
      for (int e = 0; e < 4; ++e) tr[e] = fin[(long)bh * size + (j + e) * 64 + i];
      anti = 0.5f * (running - tr);
      running += tr;
    }
  }
  for (int top = d.NC; top > 0; top -= 256) {
    const int count = min(256, top);
    __syncthreads();
    if (threadIdx.x < count)
      decay[threadIdx.x] = step_decay(d, log_decay, b, h, top - count + threadIdx.x, false);
    __syncthreads();
    for (int i0 = count - 1; i0 >= 0; i0 -= SCAN_BATCH) {
      const int m = min(SCAN_BATCH, i0 + 1);
      f4 local[SCAN_BATCH];
#pragma unroll
      for (int j = 0; j < SCAN_BATCH; ++j)
        if (j < m) local[j] = *reinterpret_cast<const f4*>(buf + (long)(top - count + i0 - j) * size + elem);
#pragma unroll
      for (int j = 0; j < SCAN_BATCH; ++j)
        if (j < m) {
          *reinterpret_cast<f4*>(buf + (long)(top - count + i0 - j) * size + elem) = running;
          running = local[j] + decay[i0 - j] * running;
          total *= decay[i0 - j];
        }
    }
  }
  float* dinit = cross ? d_init_c : d_init_s;
  if (!cross) running = 0.5f * running + total * anti;
  *reinterpret_cast<f4*>(dinit + (long)bh * size + elem) = running;
}

// ---------------------------------------------------------------------------
// Fused statistics and carry, for batches with enough (b, h) sequences to
// fill the chip.  One 512-thread block walks one state sequence of one (b, h)
// chunk by chunk, keeping the carried state in its MFMA accumulators:
// blockIdx.y 0 is the evidence, y = 1 + v cross tile v.  Each chunk (each
// sub-chunk, for the forward evidence) stores the state it starts from, then
// takes state = decay * state + sum_t wt_t a_t b_t^T over its tokens; the
// statistics never go through HBM.
//   forward:  a = key (evidence) or value tile, b = key,
//             wt = beta_t exp(P_last - P_t);  states ascend from init.
//   backward: evidence a, b = (z, y) and (y, z) with wt = -exp(P_t) / 2,
//             cross a = d_output tile, b = y with wt = exp(P_t) (MIX: the
//             read gate g_t exp(P_t), d_output being the cotangent of the
//             mixer's gated output g_t read_t + skip value_t);  states
//             descend from the final-state cotangent (the transpose of the
//             forward carry, as bwd_local_kernel + bwd_scan_kernel).
// A step's rows load into registers two steps before it multiplies.  NBUF =
// 2: LDS holds two step buffers and each step takes one barrier (the next
// step staged while this one multiplies).  NBUF = 1: one buffer, staged
// between two barriers, half the LDS, so three blocks fit a CU instead of
// two; the launch takes it when the walks would not fit the chip at two per
// CU (the extra resident blocks beat the exposed staging there).
// Wave w computes rows 16 (w % 4) .. +15 and column quads' halves w / 4 of
// the 64x64 state tile.

constexpr int STATES_THREADS = 512;

// One chunk step in LDS: per part (the forward evidence's sub-chunks, else
// the whole chunk) the token weights, zero outside the part, the decay over
// the part and its token range [lo, hi).
struct alignas(16) StepBuffer {  // wt is read as float4
  float wt[2][MAXC];
  float decay[2];
  int lo[2], hi[2];
};

// acc += (A diag(wt))^T-by-B over k in [k0, k0 + 16) for rows 16 s.. of the
// result and its columns 4r + 2hf + j (j = 0, 1): A(i, k) = A[k][16s + i]
// wt[k], B(k, c) = B[k][c] (the tile_mma_half QUAD convention).
__device__ __forceinline__ void weighted_block(f4 acc[2], const float* A, const float* B,
                                               const float* wt, int k0, int s, int hf) {
  const int l = lane_id(), r = l & 15, kk = k0 + 4 * (l >> 4);
  const f4 t = *reinterpret_cast<const f4*>(wt + kk);
  f4 a;
#pragma unroll
  for (int e = 0; e < 4; ++e) a[e] = A[(kk + e) * LDT + 16 * s + r] * t[e];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float2 b = *reinterpret_cast<const float2*>(B + (kk + e) * LDT + 4 * r + 2 * hf);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b.x, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b.y, acc[1], 0, 0, 0);
  }
}

// In: element type of the forward's key and value rows (the backward's rows
// are float32).
// The one-buffer backward walk is held to six waves per SIMD (three blocks
// per CU, as its LDS allows), a budget of 80 VGPRs at which the compiler
// may spill to per-lane scratch (it fits today); the two-buffer walks have
// room to spare.
template <bool BWD, typename In, bool MIX, int NBUF>
__global__ __launch_bounds__(STATES_THREADS)
__attribute__((amdgpu_waves_per_eu(NBUF == 1 && BWD ? 6 : 1))) void states_kernel(Dims d,
                                                                                  StateArgs g) {
  // MIX: the forward's keys come from the mixer's raw projections; the
  // backward's cross weights take the mixer's read gate.
  constexpr bool MIX_KEYS = MIX && !BWD, GATED = MIX && BWD;
  const In* rows_a = static_cast<const In*>(g.rows_a);
  const In* rows_ac = static_cast<const In*>(g.rows_ac);
  const In* rows_b = static_cast<const In*>(g.rows_b);
  extern __shared__ float smem[];  // buffer u: b tile at 2u TILE, a tile at (2u + 1) TILE
  __shared__ StepBuffer sb[2];
  const int bh = blockIdx.x, b = bh / d.H, h = bh % d.H;
  const bool cross = blockIdx.y > 0;
  const int v = cross ? (int)blockIdx.y - 1 : 0;
  // The forward evidence stores a state per sub-chunk: its chunk steps have
  // rsub parts.
  const int parts = !BWD && !cross ? d.rsub : 1;
  const int steps = d.NC;
  // Evidence a rows: the keys themselves (forward) or z (backward).
  const bool own_a = cross || BWD;
  const int w = threadIdx.x >> 6, s = w & 3, hf = w >> 2, l = lane_id();
  const int elem = (16 * s + 4 * (l >> 4)) * 64 + 4 * (l & 15) + 2 * hf;  // + 64 q + j

  // The state stored before part `part` of chunk n.
  auto state_index = [&](int n, int part) {
    return cross ? ((long)bh * d.NC + n) * d.NV + v : ((long)bh * d.NC + n) * parts + part;
  };
  const long edge = cross ? (long)bh * d.NV + v : bh;

  // MIX forward: the head's gate parameters, loaded once (the gates are
  // computed per step on the walk's critical path).
  // The backward's gated cross walk: the head's confidence scale.
  float rate = 0.f, dt_bias = 0.f, beta_bias = 0.f, cscale = 0.f;
  if constexpr (GATED) cscale = g.confidence_scale[h];
  if constexpr (MIX_KEYS) {
    rate = expf(g.gates.a_log[h]);
    dt_bias = g.gates.dt_bias[h];
    beta_bias = g.gates.beta_bias[h];
    // The evidence walks of batch row 0 write their head's floor; each
    // evidence walk its (b, h)'s shifted key.
    if (!cross && b == 0 && threadIdx.x < 64)
      g.gates.floor[h * 64 + threadIdx.x] =
          g.gates.floor_min + mix_softplus(g.gates.floor_raw[h * 64 + threadIdx.x]);
    if (!cross && g.gates.shifted && threadIdx.x < 16)
      *reinterpret_cast<f4*>(g.gates.shifted + ((long)b * d.H + h) * 64 + 4 * threadIdx.x) =
          *reinterpret_cast<const f4*>(g.mix.key + token_head(d, b, d.T - 1, h) * 64 +
                                       4 * threadIdx.x);
  }
  f4 acc[2];
  zero2(acc);
  if (const float* first = cross ? g.first_c : g.first_s) {
    const float* src = first + edge * 4096 + elem;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float2 x = *reinterpret_cast<const float2*>(src + 64 * q);
      acc[0][q] = x.x;
      acc[1][q] = x.y;
    }
  }
  // The backward evidence walk adds M + M^T per step (M = Z^T W Y), so its
  // state is S = D + A + A^T with A the decayed sum of the M alone (one
  // product per step instead of two) and D the decayed final-state cotangent
  // (which need not be symmetric): acc holds A, dscale the decay of D, and
  // A^T comes back through an LDS tile when a state is stored.  The chunk
  // end states are stored as S + S^T = dscale (D + D^T) + 2 (A + A^T), which
  // is all the chunk gradients use of them (exactly symmetric: each element
  // and its mirror add the same two terms), so dfin holds D + D^T; the
  // initial-state gradient is the full S, with D read again at the end.
  // Both step buffer counts do this, so a batch's rows give the same bits
  // whichever variant the batch size selects.  The symmetric store needs
  // about 100 VGPRs in the two-buffer walk; the one-buffer walk is held to
  // 80 for three blocks per CU.
  const bool sym = BWD && !cross;
  const int r0 = 16 * s + 4 * (l >> 4), c0 = 4 * (l & 15) + 2 * hf;  // elem's row and column
  f4 dfin[2];
  float dscale = 1.f;
  dfin[0] = acc[0];
  dfin[1] = acc[1];
  const float* const d_final = sym && g.first_s ? g.first_s + edge * 4096 : nullptr;
  if (sym) {
    zero2(acc);
    if (d_final)
#pragma unroll
      for (int j = 0; j < 2; ++j) dfin[j] += *reinterpret_cast<const f4*>(d_final + (c0 + j) * 64 + r0);
  }
  float* const tr = smem + 2 * NBUF * TILE;  // the transpose tile (backward only)
  // The state this lane holds (rows r0 + q, columns c0 + j), for dst
  // (+ 64 q + j); the backward evidence's chunk end states as S + S^T, its
  // last (the initial-state gradient, `last`) as S.
  auto state_now = [&](float2 (&out)[4], bool last) {
    if (sym) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float2*>(tr + (r0 + q) * LDT + c0) = float2{acc[0][q], acc[1][q]};
      __syncthreads();
      f4 t[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) t[j] = *reinterpret_cast<const f4*>(tr + (c0 + j) * LDT + r0);
      if (last) {
        f4 dd[2];
        zero2(dd);
        if (d_final)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float2 x = *reinterpret_cast<const float2*>(d_final + elem + 64 * q);
            dd[0][q] = x.x;
            dd[1][q] = x.y;
          }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          out[q] = float2{dscale * dd[0][q] + acc[0][q] + t[0][q],
                          dscale * dd[1][q] + acc[1][q] + t[1][q]};
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          out[q] = float2{dscale * dfin[0][q] + 2.f * (acc[0][q] + t[0][q]),
                          dscale * dfin[1][q] + 2.f * (acc[1][q] + t[1][q])};
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) out[q] = float2{acc[0][q], acc[1][q]};
    }
  };
  auto store_state = [&](const float2 (&v)[4], float* dst) {
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<float2*>(dst + 64 * q) = v[q];
  };
  auto put_state = [&](float* dst) {
    float2 v[4];
    state_now(v, true);
    store_state(v, dst);
  };
  // A step's start states (one per part), taken before its products and
  // stored after its staging: the staging's waits for the loads issued a step
  // earlier then come before these stores in issue order, so they never
  // wait for a store (the wait counter retires loads and stores in order).
  // (parts <= 2: the forward evidence's two sub-chunks, else one; the two
  // sets are named, not indexed, so they stay in registers.)
  float2 held0[4], held1[4];
  int held_i = 0;  // the step the held states start
  auto store_held = [&]() {
    float* base = cross ? g.steps_c : g.steps_s;
    store_state(held0, base + state_index(held_i, 0) * 4096 + elem);
    if (parts == 2) store_state(held1, base + state_index(held_i, 1) * 4096 + elem);
  };

  // Rows and scalars of one step on their way from HBM to LDS.  Two sets
  // rotate, so a step's loads are issued two steps before it multiplies.
  struct StepRegs {
    RowTile<In, STATES_THREADS> ra, rb;
    float pg, pb;
  };
  // MIX (forward): the b rows are the keys from the mixer's raw projections
  // (shifted; position 0's zero row reads its query row and is zeroed at
  // staging), normalised at staging.
  const MixerIn& mix = g.mix;
  // Every step issues the same loads: a step past the walk's end (i outside
  // 0 .. steps - 1) loads with no rows in range (zeros, no memory access), so
  // the compiler can count the memory operations in flight and each wait
  // retires only what it needs.
  auto fetch = [&](StepRegs& R, int i) {
    const bool valid = i >= 0 && i < steps;
    const int ic = valid ? i : 0;
    const int first = ic * d.chunk, cnt = valid ? chunk_len(d, ic) : 0;
    if constexpr (MIX_KEYS) {
      R.rb.fetch_mix_keys(cnt, mix, d, b, h, first);
    } else {
      R.rb.fetch_tokens(cnt, rows_b + token_head(d, b, first, h) * 64, (unsigned)d.H * 64);
    }
    {
      // (The forward evidence walk has no a rows: no rows in range.)
      const int width = cross ? d.P : 64, offset = cross ? 64 * v : 0;
      R.ra.fetch_tokens(own_a ? cnt : 0,
                        (cross ? rows_ac : rows_a) + token_head(d, b, first, h) * width + offset,
                        (unsigned)(d.H * width));
    }
    // Wave 0's lane l: token l's log decay and beta (zero past the chunk; the
    // other waves read out of range).  MIX forward: their raw projections
    // dt_raw and beta_raw; the backward's gated cross walk: the variance in
    // place of beta.
    const long th = token_head(d, b, first, h);
    const unsigned bytes = cnt > 0 ? (unsigned)(cnt - 1) * d.H * 4 + 4 : 0;
    const unsigned off = w == 0 ? (unsigned)l * d.H * 4 : kNoRow;
    R.pg = buf_load1(buf_rsrc((MIX_KEYS ? g.gates.dt_raw : g.log_decay) + th, bytes), off);
    const float* pb_src = BWD ? g.variance : MIX_KEYS ? g.gates.beta_raw : g.beta;
    R.pb = BWD && !(GATED && cross) ? 0.f : buf_load1(buf_rsrc(pb_src + th, bytes), off);
  };
  auto stage = [&](const StepRegs& R, int u, int i) {
    if constexpr (MIX_KEYS)
      R.rb.store_unit(smem + 2 * u * TILE, mix.key_shift && !mix.previous && i == 0);
    else
      R.rb.store(smem + 2 * u * TILE);
    if (own_a) R.ra.store(smem + (2 * u + 1) * TILE);
    if (w == 0) {
      const int cnt = chunk_len(d, i), cut = parts == 2 ? min(d.sub, cnt) : cnt;
      float pg = R.pg, pb = R.pb;
      if constexpr (MIX_KEYS) {
        // The gates from their raw projections (zero past the chunk); the
        // evidence walk writes them out for the factor and read kernels.
        const bool in = l < cnt;
        // mix_log_decay and mix_beta with the head's parameters preloaded.
        pg = in ? -rate * mix_softplus(R.pg + dt_bias) : 0.f;
        pb = in ? g.gates.beta_max * mix_sigmoid(R.pb + beta_bias) : 0.f;
        if (!cross && in) {
          const long th = token_head(d, b, i * d.chunk + l, h);
          g.gates.log_decay[th] = pg;
          g.gates.beta[th] = pb;
        }
      }
      // Inclusive log-decay prefix over the chunk; part 0 ends at token
      // `cut` - 1 (the sub-chunk boundary, or the chunk end).
      const float p = wave_inclusive_sum(pg), last = read_lane(p, 63);
      const float mid = cut > 0 ? read_lane(p, cut - 1) : 0.f;  // cut is uniform
      if (BWD) {
        float c = cross ? 1.f : -0.5f;
        if (GATED && cross) c = read_gate(cscale, pb);
        sb[u].wt[0][l] = c * expf(p);
      } else {
        sb[u].wt[0][l] = l < cut ? pb * expf(mid - p) : 0.f;
        sb[u].wt[1][l] = l >= cut ? pb * expf(last - p) : 0.f;
      }
      if (l == 0) {
        sb[u].decay[0] = expf(parts == 2 ? mid : last);
        sb[u].decay[1] = expf(last - mid);
        sb[u].lo[0] = 0;
        sb[u].hi[0] = cut;
        sb[u].lo[1] = cut;
        sb[u].hi[1] = cnt;
      }
    }
  };

  const int i0 = BWD ? steps - 1 : 0, stride = BWD ? -1 : 1;
  // Step k's products on LDS buffer u.
  auto multiply = [&](int k, int u) {
    const int i = i0 + k * stride;
    const float* tb = smem + 2 * u * TILE;
    const float* ta = own_a ? smem + (2 * u + 1) * TILE : tb;
    held_i = i;
    auto one_part = [&](int part, float2 (&held)[4]) {
      state_now(held, false);
      const float dk = sb[u].decay[part];
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[j] *= dk;
      dscale *= dk;
      // 16-token blocks that hold the part's tokens; the weights are zero
      // outside the part.
      const int lo = sb[u].lo[part], hi = lo < sb[u].hi[part] ? sb[u].hi[part] : 0;
      for (int k0 = lo & ~15; k0 < hi; k0 += 16) weighted_block(acc, ta, tb, sb[u].wt[part], k0, s, hf);
    };
    one_part(0, held0);
    if (parts == 2) one_part(1, held1);
  };
  if constexpr (NBUF == 1 && BWD) {
    // One register set, loaded one step ahead (the backward walk's 16 fewer
    // VGPRs keep three blocks per CU; the other blocks cover the shorter
    // lead).
    StepRegs R;
    fetch(R, i0);
    stage(R, 0, i0);
    __syncthreads();
    fetch(R, i0 + stride);
    for (int k = 0; k < steps; ++k) {
      multiply(k, 0);
      __syncthreads();  // every wave is done with the buffer
      if (k + 1 < steps) stage(R, 0, i0 + (k + 1) * stride);
      store_held();
      fetch(R, i0 + (k + 2) * stride);
      __syncthreads();
    }
  } else {
    StepRegs R0, R1;
    fetch(R0, i0);
    fetch(R1, i0 + stride);
    stage(R0, 0, i0);
    __syncthreads();
    // Step k multiplies LDS buffer k & 1 (NBUF = 2); `next` holds step k + 1
    // (staged at the end), `spare` (step k, already staged) receives step
    // k + 2.
    auto step = [&](int k, const StepRegs& next, StepRegs& spare) {
      const int i = i0 + k * stride, u = NBUF == 2 ? k & 1 : 0;
      fetch(spare, i + 2 * stride);
      multiply(k, u);
      if constexpr (NBUF == 2) {
        if (k + 1 < steps) stage(next, u ^ 1, i + stride);
      } else {
        __syncthreads();  // every wave is done with the buffer
        if (k + 1 < steps) stage(next, 0, i + stride);
      }
      store_held();
      __syncthreads();
    };
    // Two steps per iteration (the register sets alternate).  The first
    // iteration is peeled and an odd last step follows the loop, so the loop
    // is entered with the loads and stores in flight that each iteration
    // leaves and its body has no conditional loads: the compiler's count of
    // what is in flight at each wait stays exact.
    if (steps >= 2) {
      step(0, R1, R0);
      step(1, R0, R1);
      int k = 2;
      for (; k + 1 < steps; k += 2) {
        step(k, R1, R0);
        step(k + 1, R0, R1);
      }
      if (k < steps) step(k, R1, R0);
    } else {
      step(0, R1, R0);
    }
  }
  put_state((cross ? g.last_c : g.last_s) + edge * 4096 + elem);
}

#define M4_STATES(BWD, IN, MIX)                                          \
  template __global__ void states_kernel<BWD, IN, MIX, 1>(Dims, StateArgs); \
  template __global__ void states_kernel<BWD, IN, MIX, 2>(Dims, StateArgs);
M4_STATES(false, float, false)
M4_STATES(false, bf16_t, false)
M4_STATES(true, float, false)
M4_STATES(false, float, true)
M4_STATES(true, float, true)
#undef M4_STATES
template __global__ void fwd_stats_kernel<float>(Dims, const float*, const float*, const float*,
                                                 const float*, float*, float*);
template __global__ void fwd_stats_kernel<bf16_t>(Dims, const bf16_t*, const bf16_t*,
                                                  const float*, const float*, float*, float*);

}  // namespace m4
