// Shared device helpers for the gfx950 memory-read kernels.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>

namespace m4 {

constexpr int KD = 64;      // key width D
constexpr int VD = 64;      // value width P
constexpr int MAXC = 64;    // largest chunk
constexpr int LDT = 68;     // row stride of a 64x64 LDS tile: 16-byte rows, and rows
                            // r = 0..7 start in distinct 4-bank groups
constexpr int TILE = 64 * LDT;

typedef float f4 __attribute__((ext_vector_type(4)));

// Inputs may be float32 or bfloat16 (raw 16-bit storage): loads widen to
// float32, exactly (a bfloat16 is the high half of a float32).
typedef unsigned short bf16_t;

__device__ __forceinline__ f4 load4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f4 load4(const bf16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return f4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
            __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u)};
}
__device__ __forceinline__ float load1(const float* p) { return *p; }

// Raw buffer loads: an offset at or past the resource's byte size reads zero
// without a memory access, so rows past a chunk's end need no branch (and a
// wait for one load counts exactly the loads issued after it).
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr unsigned kNoRow = 0x80000000u;  // an offset past any resource
__device__ __forceinline__ BufRsrc buf_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ float buf_load1(BufRsrc r, unsigned off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float2 buf_load2(BufRsrc r, unsigned off) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ f4 buf_load4(BufRsrc r, unsigned off) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float load1(const bf16_t* p) {
  return __uint_as_float((unsigned)*p << 16);
}

// Problem shape.  Chunks of `chunk` tokens carry the decayed statistics;
// each chunk splits into `rsub` sub-chunks of up to `sub` tokens, and the
// factor kernel starts one token sequence per sub-chunk from its stored
// evidence (NS = NC * rsub start states).  Value rows (values, reads and
// their cotangents) are P = 64 NV floats wide; a cross state [P, 64] is NV
// stacked 64x64 tiles, and every value-dependent product runs per tile.
struct Dims {
  int B, T, H, chunk, NC;
  int sub, rsub, NS;
  int P, NV;
};

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Flat index of token-head (b, t, h) in [B,T,H] order.
__device__ __forceinline__ long token_head(const Dims& d, int b, int t, int h) {
  return ((long)b * d.T + t) * d.H + h;
}

// Tokens present in chunk n (the last chunk may be short).
__device__ __forceinline__ int chunk_len(const Dims& d, int n) {
  int left = d.T - n * d.chunk;
  return left < d.chunk ? left : d.chunk;
}

// First token (within chunk n) and length of sub-chunk u of chunk n.
__device__ __forceinline__ int sub_first(const Dims& d, int u) { return u * d.sub; }
__device__ __forceinline__ int sub_len(const Dims& d, int n, int u) {
  const int first = u * d.sub, end = min(chunk_len(d, n), first + d.sub);
  return end > first ? end - first : 0;
}

// Cross-lane reads on DPP and permlane (no LDS round trip).  dpp_read<CTRL,
// ROW_MASK>(x) is x at the lane CTRL selects; rows masked off and sources
// out of range read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_read(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, true));
}

__device__ __forceinline__ float read_lane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Inclusive prefix sum across the 64 lanes of a wave: within each 16-lane
// row by row_shr 1, 2, 4, 8, then row r + 1 takes the end of row r
// (row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3).
__device__ __forceinline__ float wave_inclusive_sum(float x) {
  x += dpp_read<0x111>(x);
  x += dpp_read<0x112>(x);
  x += dpp_read<0x114>(x);
  x += dpp_read<0x118>(x);
  x += dpp_read<0x142, 0xa>(x);
  x += dpp_read<0x143, 0xc>(x);
  return x;
}

// Reverse inclusive sum (lane t: sum over lanes u >= t): within each row by
// row_shl 1, 2, 4, 8, then the totals of the later rows (read from lanes
// 16, 32, 48) are added.
__device__ __forceinline__ float wave_suffix_sum(float x) {
  x += dpp_read<0x101>(x);
  x += dpp_read<0x102>(x);
  x += dpp_read<0x104>(x);
  x += dpp_read<0x108>(x);
  const float s1 = read_lane(x, 16), s2 = read_lane(x, 32), s3 = read_lane(x, 48);
  const int row = lane_id() >> 4;
  return x + (row == 0 ? s1 + (s2 + s3) : row == 1 ? s2 + s3 : row == 2 ? s3 : 0.f);
}

// Sum over the 16 lanes of a row (lanes differing in bits 0..3): the pairs,
// quads, halves and rows meet in the order of xor 1, 2, 4, 8 butterflies,
// and every lane receives the same total.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_read<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_read<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_read<0x141>(x);  // row_half_mirror
  x += dpp_read<0x140>(x);  // row_mirror
  return x;
}

// Sum over the 4 lane groups of 16 (lanes differing in bits 4..5), in the
// order of xor 16 then xor 32 butterflies.  permlane16_swap(x, x) yields the
// rows (x0, x0, x2, x2) and (x1, x1, x3, x3); permlane32_swap(x, x) yields
// (x0, x1, x0, x1) and (x2, x3, x2, x3).
__device__ __forceinline__ float group4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The mixer's raw keys and queries as the memory read's inputs, transformed
// on load (SelectiveMemoryMixer.__call__, lm/models/mamba4.py:183-195,
// 37-39): key t is the unit-normalised raw key t - 1 with the shift
// (position 0: the cached `previous` key, or a zero row), queries are
// unit-normalised, x rsqrt(sum x^2 + 1e-6).  (beta, the log decay and the
// floor, one value per token-head or per head, come precomputed.)
struct MixerIn {
  const float* key;       // raw keys [B,T,H,64]
  const float* query;     // raw queries [B,T,H,64]
  const float* previous;  // [B,H,64], or null: a zero key at position 0
  int key_shift;
};

__device__ __forceinline__ float mix_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// log(1 + e^x) without overflow.
__device__ __forceinline__ float mix_softplus(float x) {
  return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
}

// The prologue's gates from the raw gate projections (SelectiveMemoryMixer,
// lm/models/mamba4.py:196-237), computed where the fused mixer forward's
// state walk first needs them and written out there for the later kernels
// and the backward: beta = beta_max sigmoid(beta_raw + beta_bias), log
// decay = -exp(a_log) softplus(dt_raw + dt_bias), floor = floor_min +
// softplus(floor_raw), and with the key shift the raw key of position T - 1
// (`shifted`, may be null).
struct MixerGates {
  const float *beta_raw, *dt_raw;                     // [B,T,H]
  const float *beta_bias, *dt_bias, *a_log;           // [H]
  const float* floor_raw;                             // [H,64]
  float beta_max, floor_min;
  float *beta, *log_decay;                            // [B,T,H]
  float* floor;                                       // [H,64]
  float* shifted;                                     // [B,H,64]
};

__device__ __forceinline__ float mix_beta(const MixerGates& g, float raw, int h) {
  return g.beta_max * mix_sigmoid(raw + g.beta_bias[h]);
}
__device__ __forceinline__ float mix_log_decay(const MixerGates& g, float raw, int h) {
  return -expf(g.a_log[h]) * mix_softplus(raw + g.dt_bias[h]);
}

// Raw source row of position t's key (null: the zero row).
__device__ __forceinline__ const float* mix_key_row(const MixerIn& m, const Dims& d, int b, int t,
                                                    int h) {
  if (!m.key_shift) return m.key + token_head(d, b, t, h) * 64;
  if (t > 0) return m.key + token_head(d, b, t - 1, h) * 64;
  return m.previous ? m.previous + ((long)b * d.H + h) * 64 : nullptr;
}

// Sum over the 16 lanes of a DPP row by row-local swizzles (every lane
// receives the total; no LDS round trip).
__device__ __forceinline__ float row16_sum_dpp(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, true));
  return x;
}

// Unit normalisation of a row held as one 4-float quad per lane of a
// 16-lane DPP row.
__device__ __forceinline__ float mix_inv_norm(const f4& v) {
  float s = 0.f;
  s += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  return __builtin_amdgcn_rsqf(row16_sum_dpp(s) + 1e-6f);
}
__device__ __forceinline__ f4 mix_unit(const f4& v) { return v * mix_inv_norm(v); }

// VJP of the unit normalisation u = x r, r = rsqrt(sum x^2 + 1e-6), from u
// and r: dx = r (g - u (u . g)) (prologue_backward_kernel's arithmetic,
// rearranged).  Rows as in mix_unit.
__device__ __forceinline__ f4 mix_unit_vjp(const f4& u, float r, const f4& g) {
  const float ug = row16_sum_dpp(u[0] * g[0] + u[1] * g[1] + u[2] * g[2] + u[3] * g[3]);
  return r * (g - ug * u);
}

// The mixer's read gating fused into the read (lm/models/mamba4.py:266-273):
// out = read sigmoid(1 - confidence_scale log1p(variance)) + skip value,
// per head; the ungated read is written to `read` as well (the backward's
// residual).
struct ReadGate {
  const float* confidence_scale;  // [H]
  const float* skip;              // [H] (the mixer's D)
  float* read;                    // [B,T,H,P]
};

// The rest of the mixer's VJP folded into the memory read's backward (GATE
// kernels; lm/models/mamba4.py:183-237, 266-273 differentiated): the read
// gating out = g read + skip value with g = sigmoid(1 - scale log1p(var)),
// and the prologue's unit normalisation and gates.  The memory read's own
// cotangents are then g d_out and the variance cotangent d_var, which
// bwd_dy forms and writes for bwd_grads.  Per-chunk partial sums of the
// per-head parameter gradients go to dy_part ([H][2][B NC]: d scale,
// d skip) and grads_part ([H][3][B NC]: d beta_bias, d dt_bias, d a_log),
// entry (h, j, b NC + n), which mixer_finish_kernel sums into d_scale ..
// d_a_log.
struct MixerGrad {
  const float* d_out;     // [B,T,H,P] cotangent of the gated output
  const float* read;      // [B,T,H,P] the forward's ungated read
  const float* variance;  // [B,T,H]
  const float* d_var_in;  // [B,T,H] cotangent of the variance output, or null
  const float* scale;     // [H] confidence scale
  const float* skip;      // [H]
  float* d_var;           // [B,T,H] the read's variance cotangent (workspace)
  float* dy_part;
  const float* dt_raw;    // [B,T,H]
  const float* dt_bias;   // [H]
  const float* a_log;     // [H]
  float beta_max;
  const float* d_shifted;  // [B,H,64] cotangent of the cached key, or null
  float* d_key;            // [B,T,H,64] raw key gradient
  float* d_query;          // [B,T,H,64] raw query gradient
  float* d_beta_raw;       // [B,T,H]
  float* d_dt_raw;         // [B,T,H]
  float* d_previous;       // [B,H,64], or null
  float* grads_part;
  float *d_scale, *d_skip, *d_beta_bias, *d_dt_bias, *d_a_log;  // [H] each
};

// The read gate of a token: sigmoid(1 - scale log1p(var)).
__device__ __forceinline__ float read_gate(float scale, float var) {
  return mix_sigmoid(1.f - scale * log1pf(var));
}

// x at lane SRC of this lane's 16-lane DPP row (row_newbcast).
template <int SRC>
__device__ __forceinline__ float row_lane(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + SRC, 0xf, 0xf, true));
}

// One value per row of the N rows a 16-lane row holds (every lane has all N
// inputs in[0..N-1]): lane k < N evaluates f(in[k]) once, and every lane
// receives the N results, so a costly per-row function runs once per row
// instead of once per lane and row.
template <int N, typename F>
__device__ __forceinline__ void per_row(const float (&in)[N], float (&out)[N], F f) {
  const int k = threadIdx.x & 15;
  // The inputs pass through an empty asm as registers, so the selection
  // below stays a chain of selects (not a load from a stack copy of in[]).
  float v[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    v[i] = in[i];
    asm volatile("" : "+v"(v[i]));
  }
  float x = v[0];
#pragma unroll
  for (int i = 1; i < N; ++i) x = k == i ? v[i] : x;
  const float y = f(x);
  if constexpr (N > 0) out[0] = row_lane<0>(y);
  if constexpr (N > 1) out[1] = row_lane<1>(y);
  if constexpr (N > 2) out[2] = row_lane<2>(y);
  if constexpr (N > 3) out[3] = row_lane<3>(y);
}

// Per-chunk log-decay prefix, tail weights and chunk length, staged in LDS
// by wave 0: prefix[s] = sum_{r<=s} g_r, tail[s] = beta_s exp(P_last - P_s),
// beta[s]; entries past the chunk's tokens are beta = 0, g = 0 padding.
struct ChunkScalars {
  float prefix[MAXC];
  float tail[MAXC];
  float beta[MAXC];
};

// Wave 0 (lane s holds token s's log decay g and beta bt, zero past the
// chunk): the prefix, betas and tails of the chunk.
__device__ __forceinline__ void finish_chunk_scalars(ChunkScalars& cs, float g, float bt) {
  const int s = lane_id();
  const float p = wave_inclusive_sum(g);
  const float last = read_lane(p, 63);
  cs.prefix[s] = p;
  cs.beta[s] = bt;
  cs.tail[s] = bt * expf(last - p);
}

__device__ inline void load_chunk_scalars(ChunkScalars& cs, const Dims& d, const float* beta,
                                          const float* log_decay, int b, int h, int n) {
  if (threadIdx.x < 64) {
    const int s = threadIdx.x;
    const int len = chunk_len(d, n);
    float g = 0.f, bt = 0.f;
    if (s < len) {
      long th = token_head(d, b, n * d.chunk + s, h);
      g = log_decay[th];
      bt = beta[th];
    }
    finish_chunk_scalars(cs, g, bt);
  }
}

// 64x64 tile product on MFMA 16x16x4 f32, one 16-row strip per wave:
//   acc += A B,  rows i in [16w, 16w+16),  K (a multiple of 16) terms,
//   A(i,k) = TA ? A[k*LDT + i] : A[i*LDT + k],
//   B(k,j) = TB ? B[j*LDT + k] : B[k*LDT + j].
// MFMA operand layout (16x16x4): lane (g = lane>>4, r = lane&15) supplies
// A(row r, k-slot g) and B(k-slot g, column r); accumulator element q of the
// lane is C(row 4g+q, column r).  Within each 16-wide block of k, MFMA step
// e feeds lane group g the term k = k0 + 4g + e, so every lane's four k are
// adjacent and a k-contiguous operand arrives in one 16-byte LDS read.
// Column order of the result (see acc_col):
//   QUAD = false: accumulator jb holds columns 16jb + r;
//   QUAD = true:  accumulator jb holds columns 4r + jb, so a lane's four
//                 accumulators are four adjacent columns of one row and a
//                 k-major B (TB = false) arrives in one 16-byte read per e.
// TB = false with QUAD = false falls back to scalar B reads.
// nb < 4 (TB = true, QUAD = false only; uniform over the wave): only the
// first nb column blocks are computed, the others left as they are.
template <bool TA, bool TB, bool QUAD>
__device__ __forceinline__ void mma_block(f4 acc[4], const float* A, const float* B, int k0,
                                          int w, int nb = 4) {
  const int l = lane_id(), r = l & 15, kk = k0 + 4 * (l >> 4);
  f4 a;
  if (TA) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = A[(kk + e) * LDT + 16 * w + r];
  } else {
    a = *reinterpret_cast<const f4*>(A + (16 * w + r) * LDT + kk);
  }
  if (TB) {
    f4 b[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int col = QUAD ? 4 * r + jb : 16 * jb + r;
      if (jb < nb) b[jb] = *reinterpret_cast<const f4*>(B + col * LDT + kk);
    }
    // Consecutive MFMAs go to different accumulators (no dependent chain).
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
        if (jb < nb) acc[jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[jb][e], acc[jb], 0, 0, 0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f4 b;
      if (QUAD) {
        b = *reinterpret_cast<const f4*>(B + (kk + e) * LDT + 4 * r);
      } else {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) b[jb] = B[(kk + e) * LDT + 16 * jb + r];
      }
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
        acc[jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[jb], acc[jb], 0, 0, 0);
    }
  }
}

template <bool TA, bool TB, bool QUAD = !TB>
__device__ __forceinline__ void tile_mma(f4 acc[4], const float* A, const float* B, int K, int w) {
  if (K == 64) {
#pragma unroll
    for (int k0 = 0; k0 < 64; k0 += 16) mma_block<TA, TB, QUAD>(acc, A, B, k0, w);
  } else {
    for (int k0 = 0; k0 < K; k0 += 16) mma_block<TA, TB, QUAD>(acc, A, B, k0, w);
  }
}

// The causal scores of strip w: A B^T (B k-contiguous) for the column
// blocks jb <= w only, the blocks a mask s <= t keeps; the others are left
// as they are (the caller masks them to zero).  One straight-line body per
// strip (w is uniform over the wave).
template <bool TA, int NB>
__device__ __forceinline__ void tile_mma_cols(f4 acc[4], const float* A, const float* B, int w) {
#pragma unroll
  for (int k0 = 0; k0 < 64; k0 += 16) mma_block<TA, true, false>(acc, A, B, k0, w, NB);
}
template <bool TA>
__device__ __forceinline__ void tile_mma_causal(f4 acc[4], const float* A, const float* B, int w) {
  switch (w) {
    case 0: tile_mma_cols<TA, 1>(acc, A, B, w); break;
    case 1: tile_mma_cols<TA, 2>(acc, A, B, w); break;
    case 2: tile_mma_cols<TA, 3>(acc, A, B, w); break;
    default: tile_mma_cols<TA, 4>(acc, A, B, w); break;
  }
}

// A B over the token terms s <= t of strip w (A a causally masked score
// tile, zero past the chunk's len tokens): 16 (w + 1) terms, fewer for a
// short chunk; one unrolled body per strip when the chunk is full.
template <bool TA, bool TB, bool QUAD = !TB>
__device__ __forceinline__ void tile_mma_causal_terms(f4 acc[4], const float* A, const float* B,
                                                      int len, int w) {
  if (len >= 16 * (w + 1)) {
    switch (w) {
      case 0: mma_block<TA, TB, QUAD>(acc, A, B, 0, w); break;
      case 1:
#pragma unroll
        for (int k0 = 0; k0 < 32; k0 += 16) mma_block<TA, TB, QUAD>(acc, A, B, k0, w);
        break;
      case 2:
#pragma unroll
        for (int k0 = 0; k0 < 48; k0 += 16) mma_block<TA, TB, QUAD>(acc, A, B, k0, w);
        break;
      default:
#pragma unroll
        for (int k0 = 0; k0 < 64; k0 += 16) mma_block<TA, TB, QUAD>(acc, A, B, k0, w);
        break;
    }
  } else {
    for (int k0 = 0; k0 < len; k0 += 16) mma_block<TA, TB, QUAD>(acc, A, B, k0, w);
  }
}

// Terms a product over `len` tokens needs: len rounded up to 16 (the tiles
// are zero past len).
__device__ __forceinline__ int k_terms(int len) { return (len + 15) & ~15; }

__device__ __forceinline__ void zero4(f4 acc[4]) {
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) acc[jb] = f4{0.f, 0.f, 0.f, 0.f};
}

// Row / column of accumulator element (jb, q) for wave w and this lane.
__device__ __forceinline__ int acc_row(int w, int q) { return 16 * w + 4 * (lane_id() >> 4) + q; }
template <bool QUAD>
__device__ __forceinline__ int acc_col(int jb) {
  return QUAD ? 4 * (lane_id() & 15) + jb : 16 * jb + (lane_id() & 15);
}

// Row q of a QUAD accumulator set: columns 4r..4r+3 of row acc_row(w, q).
__device__ __forceinline__ f4 quad_row(const f4 acc[4], int q) {
  return f4{acc[0][q], acc[1][q], acc[2][q], acc[3][q]};
}

// Half of a 64x64 tile product for one of two waves sharing a 16-row strip:
// acc[j] is the 16-column block jb = 2 hf + j of tile_mma's result (same
// operand conventions, same accumulator layout per block).  A QUAD block jb
// holds columns 4r + jb, so a wave's two blocks are columns 4r + 2hf, +1.
// Only the first nj blocks (1 or 2, uniform over the wave) are computed.
template <bool TA, bool TB, bool QUAD>
__device__ __forceinline__ void mma_block_half(f4 acc[2], const float* A, const float* B, int k0,
                                               int w, int hf, int nj) {
  const int l = lane_id(), r = l & 15, kk = k0 + 4 * (l >> 4);
  f4 a;
  if (TA) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = A[(kk + e) * LDT + 16 * w + r];
  } else {
    a = *reinterpret_cast<const f4*>(A + (16 * w + r) * LDT + kk);
  }
  if (TB) {
    f4 b[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int jb = 2 * hf + j, col = QUAD ? 4 * r + jb : 16 * jb + r;
      if (j < nj) b[j] = *reinterpret_cast<const f4*>(B + col * LDT + kk);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (j < nj) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[j][e], acc[j], 0, 0, 0);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float b[2];
      if (QUAD) {
        const float2 v = *reinterpret_cast<const float2*>(B + (kk + e) * LDT + 4 * r + 2 * hf);
        b[0] = v.x;
        b[1] = v.y;
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          if (j < nj) b[j] = B[(kk + e) * LDT + 16 * (2 * hf + j) + r];
      }
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (j < nj) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[j], acc[j], 0, 0, 0);
    }
  }
}

// acc += the wave's half of A B over contraction terms [k_begin, K) (both
// multiples of 16), computing its first nj column blocks.  Terms and blocks
// left out must be known zero in the product (causal masks).
template <bool TA, bool TB, bool QUAD = !TB>
__device__ __forceinline__ void tile_mma_half(f4 acc[2], const float* A, const float* B, int K,
                                              int w, int hf, int k_begin = 0, int nj = 2) {
  if (nj <= 0) return;
  if (K == 64 && k_begin == 0) {
#pragma unroll
    for (int k0 = 0; k0 < 64; k0 += 16) mma_block_half<TA, TB, QUAD>(acc, A, B, k0, w, hf, nj);
  } else {
    for (int k0 = k_begin; k0 < K; k0 += 16) mma_block_half<TA, TB, QUAD>(acc, A, B, k0, w, hf, nj);
  }
}

__device__ __forceinline__ void zero2(f4 acc[2]) {
  acc[0] = f4{0.f, 0.f, 0.f, 0.f};
  acc[1] = f4{0.f, 0.f, 0.f, 0.f};
}

// Kernels built on these tiles run 256 threads (4 waves).
constexpr int BLOCK = 256;

// SPD solves wider than 64 (spd_wide.hip): one 256-thread block per
// system, factored in LDS up to kWideLdsDim, in the factor buffer above.
constexpr int kWideThreads = 256;
constexpr int kWideLdsDim = 128;
constexpr int kWideMaxDim = 4096;
// LDS floats a block takes: the column, two vectors and, for LDS systems,
// the matrix (row stride dim + 1).
__host__ __device__ constexpr long wide_lds_floats(int dim) {
  return 3L * dim + (dim <= kWideLdsDim ? (long)dim * (dim + 1) : 0L);
}

// One 64x64 tile staged through registers: thread i fetches the float4 at
// column quad i%16 of rows i/16 + 16j (j = 0..3), and stores it later.  A
// kernel fetches every tile of a phase before storing any, so all of the
// phase's global loads are in flight together.
struct TileRegs {
  f4 v[4];

  // Rows [0, rows) of a token-major slab, row(s) = global pointer of row s;
  // rows past `rows` are zero.
  template <typename RowPtr>
  __device__ __forceinline__ void fetch_rows(int rows, RowPtr row) {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + 16 * j;
      v[j] = r < rows ? load4(row(r) + q) : f4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // A dense row-major 64x64 matrix.
  __device__ __forceinline__ void fetch_matrix(const float* src) {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = *reinterpret_cast<const f4*>(src + (r0 + 16 * j) * 64 + q);
  }
  // The same through a buffer resource that is empty unless `any`: zeros and
  // no memory access otherwise, with the same instructions either way.
  __device__ __forceinline__ void fetch_matrix(const float* src, bool any) {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
    const BufRsrc rs = buf_rsrc(src, any ? 4096 * 4 : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = __builtin_bit_cast(
          f4, __builtin_amdgcn_raw_buffer_load_b128(rs, ((r0 + 16 * j) * 64 + q) * 4, 0, 0));
  }

  __device__ __forceinline__ void store(float* tile) const {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<f4*>(tile + (r0 + 16 * j) * LDT + q) = v[j];
  }
};

// A chunk's 64 token rows held by an NTH-thread block (thread i: column quad
// i % 16 of rows i / 16 + (NTH / 16) j), in the input's own dtype: float32
// as f4, bfloat16 as its raw 8 bytes, widened where the rows are stored or
// read (a widening right after the load would make every load wait for the
// one before it).  fetch_tokens reads rows [0, rows) at base + r * stride
// elements through buffer loads (zero past `rows`, no branch);
// fetch_mix_keys (float32) reads the mixer's shifted key rows.
template <typename In, int NTH = 256>
struct RowTile {
  static constexpr bool F32 = std::is_same<In, float>::value;
  static constexpr int J = 1024 / NTH, RS = NTH / 16;
  typedef typename std::conditional<F32, f4, uint2>::type Raw;
  Raw v[J];

  __device__ __forceinline__ void fetch_tokens(int rows, const In* base, unsigned stride) {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
    const BufRsrc rs =
        buf_rsrc(base, rows > 0 ? ((unsigned)(rows - 1) * stride + 64) * sizeof(In) : 0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const unsigned off = ((r0 + RS * j) * stride + q) * sizeof(In);
      if constexpr (F32)
        v[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      else
        v[j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
    }
  }
  // The mixer's key rows of the chunk at position t0 (with the key shift,
  // row r holds position t0 + r - 1's raw key and position 0's row is the
  // decode cache's key, or zero without one): every path issues the same
  // loads, out-of-range ones reading zero.
  __device__ __forceinline__ void fetch_mix_keys(int rows, const MixerIn& m, const Dims& d, int b,
                                                 int h, int t0) {
    static_assert(F32, "the mixer's rows are float32");
    const int adj = m.key_shift && t0 == 0 ? 1 : 0;  // row 0 holds no key row
    const int first = m.key_shift && t0 > 0 ? t0 - 1 : t0;
    const int n = rows - adj;
    const unsigned stride = (unsigned)d.H * 64;
    const BufRsrc rs = buf_rsrc(m.key + token_head(d, b, first, h) * 64,
                                n > 0 ? ((unsigned)(n - 1) * stride + 64) * 4 : 0);
    const float* prev = m.previous ? m.previous + ((long)b * d.H + h) * 64 : m.key;
    const BufRsrc rp = buf_rsrc(prev, rows > 0 && adj && m.previous ? 256 : 0);
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int r = r0 + RS * j;
      const unsigned off = r >= adj ? ((unsigned)(r - adj) * stride + q) * 4 : kNoRow;
      f4 x = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
      if (j == 0) {
        const f4 pv = __builtin_bit_cast(
            f4, __builtin_amdgcn_raw_buffer_load_b128(rp, r == 0 ? q * 4 : kNoRow, 0, 0));
        if (r == 0 && adj) x = pv;
      }
      v[j] = x;
    }
  }
  __device__ __forceinline__ f4 get(int j) const {
    if constexpr (F32)
      return v[j];
    else
      return f4{__uint_as_float(v[j].x << 16), __uint_as_float(v[j].x & 0xffff0000u),
                __uint_as_float(v[j].y << 16), __uint_as_float(v[j].y & 0xffff0000u)};
  }
  __device__ __forceinline__ void store(float* tile) const {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < J; ++j) *reinterpret_cast<f4*>(tile + (r0 + RS * j) * LDT + q) = get(j);
  }
  // Row j of this thread scaled by sc[j] (the mixer's read gate of its token).
  __device__ __forceinline__ void store_scaled(float* tile, const float (&sc)[J]) const {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < J; ++j)
      *reinterpret_cast<f4*>(tile + (r0 + RS * j) * LDT + q) = sc[j] * get(j);
  }
  // The rows unit-normalised (mix_unit), row 0 as a zero row if zero_row0.
  // inv (may be null): each row's 1 / norm, rsqrt(sum x^2 + 1e-6), as well.
  __device__ __forceinline__ void store_unit(float* tile, bool zero_row0,
                                             float* inv = nullptr) const {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int r = r0 + RS * j;
      const f4 x = zero_row0 && r == 0 ? f4{0.f, 0.f, 0.f, 0.f} : get(j);
      if (inv) {
        const float rn = mix_inv_norm(x);
        *reinterpret_cast<f4*>(tile + r * LDT + q) = x * rn;
        if ((threadIdx.x & 15) == 0) inv[r] = rn;
      } else {
        *reinterpret_cast<f4*>(tile + r * LDT + q) = mix_unit(x);
      }
    }
  }
};

// Four consecutive elements of one row, held raw as RowTile holds them.
template <typename In>
struct RowQuad;

template <>
struct RowQuad<float> {
  f4 v;
  __device__ __forceinline__ void load(BufRsrc r, unsigned off) {
    v = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  }
  __device__ __forceinline__ f4 get() const { return v; }
};

template <>
struct RowQuad<bf16_t> {
  uint2 v;
  __device__ __forceinline__ void load(BufRsrc r, unsigned off) {
    v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  }
  __device__ __forceinline__ f4 get() const {
    return f4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
              __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u)};
  }
};

// A dense 64x64 matrix in a 512-thread block: thread i holds column quad
// i%16 of rows i/16 + 32j (j = 0, 1).
struct TileRegs2 {
  f4 v[2];

  __device__ __forceinline__ void fetch_matrix(const float* src) {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < 2; ++j) v[j] = *reinterpret_cast<const f4*>(src + (r0 + 32 * j) * 64 + q);
  }

  __device__ __forceinline__ void store(float* tile) const {
    const int r0 = threadIdx.x >> 4, q = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int j = 0; j < 2; ++j) *reinterpret_cast<f4*>(tile + (r0 + 32 * j) * LDT + q) = v[j];
  }
};

// The transpose of a dense row-major 64x64 matrix: tile[c][r] = src[r][c].
// Fetch j of wave w covers the 16x16 block b = 4 j + w: lane L holds row
// 16 (b / 4) + L / 4, columns 16 (b % 4) + 4 (L % 4) .. +3.  Each load
// instruction reads 16 row pieces of 64 contiguous bytes (not one cache
// line per lane), and the scalar LDS stores of a wave fall in 64 distinct
// banks (LDT = 4 mod 64).
struct TileRegsT {
  f4 v[4];

  __device__ __forceinline__ static void slot(int j, int& r, int& c) {
    const int L = threadIdx.x & 63, b = 4 * j + (threadIdx.x >> 6);
    r = 16 * (b >> 2) + (L >> 2);
    c = 16 * (b & 3) + 4 * (L & 3);
  }

  __device__ __forceinline__ void fetch_matrix(const float* src) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int r, c;
      slot(j, r, c);
      v[j] = *reinterpret_cast<const f4*>(src + r * 64 + c);
    }
  }
  // Through a buffer resource that is empty unless `any` (as TileRegs).
  __device__ __forceinline__ void fetch_matrix(const float* src, bool any) {
    const BufRsrc rs = buf_rsrc(src, any ? 4096 * 4 : 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int r, c;
      slot(j, r, c);
      v[j] = __builtin_bit_cast(f4,
                                __builtin_amdgcn_raw_buffer_load_b128(rs, (r * 64 + c) * 4, 0, 0));
    }
  }

  __device__ __forceinline__ void store(float* tile) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int r, c;
      slot(j, r, c);
#pragma unroll
      for (int i = 0; i < 4; ++i) tile[(c + i) * LDT + r] = v[j][i];
    }
  }
};

// Arguments of the fused chunk-boundary state walk (states_kernel).
struct StateArgs {
  // Row slabs: float32, or in the forward the caller's input type.
  const void* rows_a;    // evidence a rows: forward keys (unused), backward z
  const void* rows_ac;   // cross a rows: forward values, backward d_output
  const void* rows_b;    // b rows: forward keys, backward solved
  const float* beta;
  const float* log_decay;
  const float* first_s;  // state before the first step (NULL: zero)
  const float* first_c;
  float* steps_s;        // the state each step starts from
  float* steps_c;
  float* last_s;         // the state after the last step
  float* last_c;
  MixerIn mix;           // forward with the mixer's projections (MIX): keys and gates
  MixerGates gates;      // forward (MIX): the gates from their raw projections
  // Backward of the mixer's gated output (MIX): the cross a rows are the
  // gated output's cotangent d_out, so the read's cotangent is g_t d_out_t
  // with the read gate g_t = read_gate(confidence_scale, variance_t).
  const float* variance;
  const float* confidence_scale;
};

// Shape of the order head's scan: values [B,T,H,W] in chunks of `chunk`
// tokens, NC of them.
struct OrderDims {
  int B, T, H, W, chunk, NC;
};

}  // namespace m4
