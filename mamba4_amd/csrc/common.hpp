// Shared device helpers for the gfx950 memory-read kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace m4 {

constexpr int KD = 64;      // key width D
constexpr int VD = 64;      // value width P
constexpr int MAXC = 64;    // largest chunk
constexpr int LDT = 65;     // row stride of a 64x64 LDS tile (odd: conflict-free columns)
constexpr int TILE = 64 * LDT;

typedef float f4 __attribute__((ext_vector_type(4)));

// Problem shape.  Chunks of `chunk` tokens carry the decayed statistics;
// each chunk splits into `rsub` sub-chunks of up to `sub` tokens, and the
// factor kernel starts one token sequence per sub-chunk from its stored
// evidence (NS = NC * rsub start states).
struct Dims {
  int B, T, H, chunk, NC;
  int sub, rsub, NS;
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

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ float wave_inclusive_sum(float x) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    float y = __shfl_up(x, o, 64);
    if (l >= o) x += y;
  }
  return x;
}

// Sum over the 16 lanes of a row (lanes differing in bits 0..3).
__device__ __forceinline__ float row16_sum(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  x += __shfl_xor(x, 4, 64);
  x += __shfl_xor(x, 8, 64);
  return x;
}

// Sum over the 4 lane groups of 16 (lanes differing in bits 4..5).
__device__ __forceinline__ float group4_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

// Per-chunk log-decay prefix, tail weights and chunk length, staged in LDS
// by wave 0: prefix[s] = sum_{r<=s} g_r, tail[s] = beta_s exp(P_last - P_s),
// beta[s]; entries past the chunk's tokens are beta = 0, g = 0 padding.
struct ChunkScalars {
  float prefix[MAXC];
  float tail[MAXC];
  float beta[MAXC];
};

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
    float p = wave_inclusive_sum(g);
    float last = __shfl(p, 63, 64);
    cs.prefix[s] = p;
    cs.beta[s] = bt;
    cs.tail[s] = bt * expf(last - p);
  }
}

// 64x64 tile GEMM on MFMA 16x16x4 f32, one 16-row strip per wave:
//   acc[jb] += sum_k A(i, k) B(k, j),  i in [16w, 16w+16), j in [16jb, 16jb+16)
// A(i,k) = TA ? A[k*lda + i] : A[i*lda + k];  B(k,j) = TB ? B[j*ldb + k] : B[k*ldb + j].
// Operand lane layout (verified on gfx950): A lane = i + 16k, B lane = j + 16k;
// result acc[jb][r] = C[16w + 4*(lane>>4) + r][16jb + (lane&15)].
// K must be a multiple of 4 with zero padding past the real extent.
template <bool TA, bool TB>
__device__ __forceinline__ void tile_mma(f4 acc[4], const float* A, int lda, const float* B,
                                         int ldb, int K, int w) {
  const int l = lane_id();
  const int r = l & 15, kq = l >> 4;
  for (int k0 = 0; k0 < K; k0 += 4) {
    const int k = k0 + kq;
    const float a = TA ? A[k * lda + 16 * w + r] : A[(16 * w + r) * lda + k];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const float bv = TB ? B[(16 * jb + r) * ldb + k] : B[k * ldb + 16 * jb + r];
      acc[jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bv, acc[jb], 0, 0, 0);
    }
  }
}

__device__ __forceinline__ void zero4(f4 acc[4]) {
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) acc[jb] = f4{0.f, 0.f, 0.f, 0.f};
}

// Row / column of accumulator element (jb, r) for wave w and this lane.
__device__ __forceinline__ int acc_row(int w, int r) { return 16 * w + 4 * (lane_id() >> 4) + r; }
__device__ __forceinline__ int acc_col(int jb) { return 16 * jb + (lane_id() & 15); }

// Copy rows [0, rows) of a [*, width=64] token-major global slab into a
// 64xLDT LDS tile, zero-filling rows [rows, 64).  src(row) gives the row's
// global pointer.  Uses all threads of the block.
template <typename RowPtr>
__device__ inline void load_rows(float* tile, int rows, RowPtr src) {
  for (int e = threadIdx.x; e < 64 * 16; e += blockDim.x) {
    const int row = e >> 4, q = (e & 15) * 4;
    f4 v = f4{0.f, 0.f, 0.f, 0.f};
    if (row < rows) v = *reinterpret_cast<const f4*>(src(row) + q);
    float* dst = tile + row * LDT + q;
    dst[0] = v[0];
    dst[1] = v[1];
    dst[2] = v[2];
    dst[3] = v[3];
  }
}

// Copy a dense row-major 64x64 global matrix into a 64xLDT LDS tile.
__device__ inline void load_matrix(float* tile, const float* src) {
  for (int e = threadIdx.x; e < 64 * 16; e += blockDim.x) {
    const int row = e >> 4, q = (e & 15) * 4;
    f4 v = *reinterpret_cast<const f4*>(src + row * 64 + q);
    float* dst = tile + row * LDT + q;
    dst[0] = v[0];
    dst[1] = v[1];
    dst[2] = v[2];
    dst[3] = v[3];
  }
}

}  // namespace m4
