// Mamba-3 SISO scan in FlashMamba's fused projection layout, for gfx950.
//
// Operator: mamba3_fused (lm/kernels/flashmamba.py:1125-1162) over fused_scan
// (:901-1111).  One shared query row c_t and key row b_t per token [B,T,N],
// values x [B,T,H*P], per-head log decays adt, steps dt, trapezoid logits
// [B,T,H], shared angle rates [B,T,A], per-head biases [H,N].  Per head:
//   theta_t = sum_{s<=t} angles_s dt_s;  q_t = rot(c_t + qb, theta_t),
//   k_t = rot(b_t + kb, theta_t);  gamma = dt sigmoid(trap),
//   scale_s = gamma_s + dt_{s+1} (1 - sigmoid(trap_{s+1})),
//   within a chunk with p_t = sum of adt over the chunk up to t:
//   y_t = sum_{s<t} e^{p_t - p_s} scale_s (q_t.k_s) v_s + gamma_t (q_t.k_t) v_t
//         + e^{p_t} q_t^T S,    S <- e^{p_L} S + sum_s e^{p_L - p_s} scale_s k_s v_s^T.
//
// Kernels (chunks of C = 64 tokens, one token per lane of a wave; the state
// S is a 128 x 64 float32 tile, N <= 128 and P <= 64 are zero-padded):
//   walk_kernel<false>  one block per (b, h): walks the chunks in order,
//                       stores each chunk's start state and start phase, and
//                       the final state (the sequential part: one MFMA
//                       product K^T (u v) per chunk).
//   out_kernel          one block per (b, chunk, h): y from the stored start
//                       state (scores, masked decay weights, two products).
//   walk_kernel<true>   one block per (b, h), chunks in reverse: the state
//                       cotangent at each chunk end.
//   grad_kernel         one block per (b, chunk, head group): every gradient
//                       of the chunk for the group's heads; the shared rows'
//                       gradients accumulate over the group's heads in
//                       registers.
//   finish_kernel       four blocks per (b, chunk): sums the groups, adds the
//                       phase gradient carried from later chunks, and turns
//                       gamma / scale gradients into dt and trap gradients.
//   bias_kernel         one block per head: the bias gradients.
// All arithmetic is float32 (MFMA v_mfma_f32_16x16x4f32).
#include <hip/hip_runtime.h>

#include "scan3.hpp"

namespace m3 {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Inputs in the model dtype: float32, or bfloat16 as raw bits.  With
// bfloat16 rows and values the kernels also take the reference's bfloat16
// matrix operands (is_bf16<In>).
template <typename In>
struct is_bf16 {
  static constexpr bool value = false;
};
template <>
struct is_bf16<bf16_t> {
  static constexpr bool value = true;
};

__device__ __forceinline__ float lo_bf(unsigned u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_bf(unsigned u) { return __uint_as_float(u & 0xffff0000u); }

// Inputs are fetched as the raw register image of their dtype (Raw<In>::Pair
// for two consecutive elements, ::Quad for four) and decoded to float32 by
// dec() where they are used, so a load is waited for at its use, not at its
// issue (a bfloat16 load decoded on arrival would stall every load after it).
typedef unsigned u2 __attribute__((ext_vector_type(2)));
template <typename In>
struct Raw {
  typedef float2 Pair;
  typedef f4 Quad;
};
template <>
struct Raw<bf16_t> {
  typedef unsigned Pair;
  typedef u2 Quad;
};
// Inputs load through buffer resources, each spanning one chunk's valid
// tokens (or one head's row): the hardware's range check returns zeros for
// an offset at or past the resource's size, so padding tokens and
// coordinates need no branch around their loads.  Every load of a prefetch
// then issues unconditionally, and the waits at the uses count exactly the
// loads issued after the awaited one instead of draining them all.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr unsigned kNoLoad = 0x80000000u;  // an offset past every resource here
// bytes < 2^31: the host rejects shapes whose largest resource (one
// (group, batch) slab of the finish kernel's row-gradient partials,
// ceil(T / C) * C * NT floats) would reach 2^31 bytes; every other resource
// spans one chunk or one row.
__device__ __forceinline__ Rsrc rsrc(const void* base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ float ldb(Rsrc r, unsigned off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float2 raw2(Rsrc r, unsigned off, const float*) {
  return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ unsigned raw2(Rsrc r, unsigned off, const bf16_t*) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ f4 raw4(Rsrc r, unsigned off, const float*) {
  return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ u2 raw4(Rsrc r, unsigned off, const bf16_t*) {
  return __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
// The first min(n, 4) of four consecutive elements at any alignment (zeros
// after), one element per load: rows whose width is not a multiple of 4.
__device__ __forceinline__ f4 raw4_n(Rsrc r, unsigned off, int n, const float*) {
  f4 v;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = ldb(r, k < n ? off + 4 * k : kNoLoad);
  return v;
}
__device__ __forceinline__ u2 raw4_n(Rsrc r, unsigned off, int n, const bf16_t*) {
  unsigned e[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    e[k] = __builtin_amdgcn_raw_buffer_load_b16(r, k < n ? off + 2 * k : kNoLoad, 0, 0);
  return u2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
}
__device__ __forceinline__ float2 dec(float2 r) { return r; }
__device__ __forceinline__ float2 dec(unsigned r) { return float2{lo_bf(r), hi_bf(r)}; }
__device__ __forceinline__ f4 dec(f4 r) { return r; }
__device__ __forceinline__ f4 dec(u2 r) {
  return f4{lo_bf(r.x), hi_bf(r.x), lo_bf(r.y), hi_bf(r.y)};
}
__device__ __forceinline__ void st1(float* p, float v) { *p = v; }
__device__ __forceinline__ void st1(bf16_t* p, float v) {
  *p = __builtin_bit_cast(bf16_t, static_cast<__bf16>(v));
}

// x rounded to bfloat16 (to nearest, ties to even: v_cvt_pk_bf16_f32), as
// float: the reference's .astype(model dtype) of a float32 value.
__device__ __forceinline__ float round_bf(float x) {
  return static_cast<float>(static_cast<__bf16>(x));
}
template <bool BF>
__device__ __forceinline__ float2 round_bf2(float2 v) {
  if constexpr (BF) return float2{round_bf(v.x), round_bf(v.y)};
  return v;
}

__device__ __forceinline__ bf16x2 cvt2(float a, float b) {
  return __builtin_convertvector(f2{a, b}, bf16x2);
}
__device__ __forceinline__ bf16x4 pack4(f4 a) {
  const bf16x2 p0 = cvt2(a[0], a[1]), p1 = cvt2(a[2], a[3]);
  return bf16x4{p0[0], p0[1], p1[0], p1[1]};
}
__device__ __forceinline__ bf16x8 pack8(f4 a, f4 b) {
  const bf16x2 p0 = cvt2(a[0], a[1]), p1 = cvt2(a[2], a[3]), p2 = cvt2(b[0], b[1]),
               p3 = cvt2(b[2], b[3]);
  return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// The thread index through an empty asm: values derived from it cannot be
// hoisted out of the kernels' chunk and head loops, so index arithmetic is
// recomputed per iteration instead of occupying registers across the loop.
__device__ __forceinline__ int tix() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int lane_id() { return tix() & 63; }

// DPP move of x (as bits) with zeros where the source lane is out of range.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp0(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, true));
}

// Inclusive sum over the lanes of a wave: Hillis-Steele within each 16-lane
// row (row_shr 1, 2, 4, 8), then row 0's total into rows 1 and 3
// (row_bcast:15) and row 1's running total into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ float wave_scan(float x) {
  x += dpp0<0x111, 0xf>(x);
  x += dpp0<0x112, 0xf>(x);
  x += dpp0<0x114, 0xf>(x);
  x += dpp0<0x118, 0xf>(x);
  x += dpp0<0x142, 0xa>(x);
  x += dpp0<0x143, 0xc>(x);
  return x;
}

__device__ __forceinline__ float lane63(float x) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

__device__ __forceinline__ float wave_sum(float x) { return lane63(wave_scan(x)); }

// Sum over the 16 lanes sharing bits 4..5 of the lane index (row_ror 8, 4,
// 2, 1 within each row of 16: every lane ends with the row's total).
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp0<0x128, 0xf>(x);
  x += dpp0<0x124, 0xf>(x);
  x += dpp0<0x122, 0xf>(x);
  x += dpp0<0x121, 0xf>(x);
  return x;
}

// Sum over the 4 lanes sharing bits 0..3 of the lane index (one per row), in
// the order of xor 16 then xor 32 butterflies: permlane16_swap(x, x) yields
// the rows (x0, x0, x2, x2) and (x1, x1, x3, x3), permlane32_swap(x, x)
// yields (x0, x1, x0, x1) and (x2, x3, x2, x3).
__device__ __forceinline__ float group4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// sin and cos of x (|x| < 2^16): x = k pi/2 + r with k = rint(2x/pi) and r by
// Cody-Waite reduction (pi/2 as three float32 parts; k * part is exact for
// |k| < 2^16 in the first, rounded once by the fused multiply-add in the
// others), then Taylor polynomials of sin r and cos r on |r| <= pi/4 through
// r^9 and r^10 (truncation below 2e-9), and the quadrant k mod 4.
__device__ __forceinline__ void sin_cos(float x, float* sn, float* cs) {
  const float k = rintf(x * 0.636619772f);
  float r = fmaf(-k, 1.5703125f, x);
  r = fmaf(-k, 4.838267923332751e-4f, r);
  r = fmaf(-k, 2.5632829e-12f, r);
  const float r2 = r * r;
  float ps = fmaf(r2, 2.7557319e-6f, -1.9841270e-4f);
  ps = fmaf(r2, ps, 8.3333333e-3f);
  ps = fmaf(r2, ps, -1.6666667e-1f);
  const float sr = fmaf(r * r2, ps, r);
  float pc = fmaf(r2, -2.7557319e-7f, 2.4801587e-5f);
  pc = fmaf(r2, pc, -1.3888889e-3f);
  pc = fmaf(r2, pc, 4.1666668e-2f);
  pc = fmaf(r2, pc, -0.5f);
  const float cr = fmaf(r2, pc, 1.f);
  const int quad = static_cast<int>(k) & 3;
  const float s0 = (quad & 1) ? cr : sr, c0 = (quad & 1) ? sr : cr;
  *sn = (quad & 2) ? -s0 : s0;
  *cs = ((quad + 1) & 2) ? -c0 : c0;
}

// x - 2 pi k with k = rint(x / 2 pi), in [-pi, pi]: 2 pi as two float32 parts,
// the first (6.28125) with 8 significant bits, so k times it is exact for
// |k| < 2^16.  Keeps each chunk's stored start phase small, so the phases
// inside a chunk stay far below sin_cos's 2^16 limit however long the
// sequence.
__device__ __forceinline__ float reduce_turns(float x) {
  const float k = rintf(x * 0.159154943f);
  return fmaf(-k, 1.9353071795864769e-3f, fmaf(-k, 6.28125f, x));
}

// Four consecutive-in-k operand values: one 16-byte LDS read when the
// operand is contiguous along k (stride 1), four reads otherwise.
template <int STRIDE>
__device__ __forceinline__ f4 load_k4(const float* p) {
  if constexpr (STRIDE == 1) {
    return *reinterpret_cast<const f4*>(p);
  } else {
    return f4{p[0], p[STRIDE], p[2 * STRIDE], p[3 * STRIDE]};
  }
}

// acc[j] += A[r0 .. r0+16, kb .. ke) * B[kb .. ke, c0 + 16 j .. +16) for j < J,
// with A(r, k) = A[r * AR + k * AK] and B(k, c) = B[k * BK + c * BC] in LDS;
// kb and ke are multiples of 16.  Result element acc[j][i] is (row
// r0 + 4 (lane / 16) + i, column c0 + 16 j + lane % 16).  Within each block
// of 16 k the lanes of group q = lane / 16 take k = 4 q + e at MFMA step e
// (the same assignment for A and B, so the sum is unchanged), which makes a
// lane's four A (or B) values of the block contiguous when AK (BK) is 1.
// All of a block's operands are read before its 4 J MFMAs issue.
//
// BF: both operands rounded to bfloat16 (the reference's model-dtype
// operands, float32 accumulation), on v_mfma_f32_16x16x32_bf16 over blocks
// of 32 k (lane group q takes k = 8 q .. 8 q + 7 of each, as eight
// consecutive operand values) and v_mfma_f32_16x16x16_bf16 for a last block
// of 16 (k = 4 q .. 4 q + 3).
template <int J, int AR, int AK, int BK, int BC, bool BF = false>
__device__ __forceinline__ void mma(f4 (&acc)[J], const float* A, int r0, const float* B, int c0,
                                    int kb, int ke) {
  const int l = lane_id(), r = l & 15, q = l >> 4;
  if constexpr (BF) {
    const float* pa = A + (r0 + r) * AR + 8 * q * AK;
    const float* pb = B + 8 * q * BK + (c0 + r) * BC;
    int k = kb;
#pragma unroll 2
    for (; k + 32 <= ke; k += 32) {
      const bf16x8 a = pack8(load_k4<AK>(pa + k * AK), load_k4<AK>(pa + (k + 4) * AK));
      bf16x8 b[J];
#pragma unroll
      for (int j = 0; j < J; ++j)
        b[j] = pack8(load_k4<BK>(pb + k * BK + 16 * j * BC),
                     load_k4<BK>(pb + (k + 4) * BK + 16 * j * BC));
#pragma unroll
      for (int j = 0; j < J; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[j], acc[j], 0, 0, 0);
    }
    if (k < ke) {
      const bf16x4 a = pack4(load_k4<AK>(A + (r0 + r) * AR + (k + 4 * q) * AK));
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const bf16x4 b = pack4(load_k4<BK>(B + (k + 4 * q) * BK + (c0 + 16 * j + r) * BC));
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                           __builtin_bit_cast(s16x4, b),
                                                           acc[j], 0, 0, 0);
      }
    }
  } else {
    const float* pa = A + (r0 + r) * AR + 4 * q * AK;
    const float* pb = B + 4 * q * BK + (c0 + r) * BC;
#pragma unroll 2
    for (int k = kb; k < ke; k += 16) {
      const f4 a = load_k4<AK>(pa + k * AK);
      f4 b[J];
#pragma unroll
      for (int j = 0; j < J; ++j) b[j] = load_k4<BK>(pb + k * BK + 16 * j * BC);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < J; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[j][e], acc[j], 0, 0, 0);
    }
  }
}

// acc[jb] += A[r0 .. r0+16, kb .. ke) * B[kb .. ke, c0 + J r + jb] for jb < J
// (J = 2 or 4), B(k, c) = B[k * BK + c]: lane r's J accumulators are J
// adjacent columns of one row, so each k's B values for all J tiles arrive
// in one 8- or 16-byte LDS read, where a B strided along k (BK > 1) costs
// mma one read per element.  Result element acc[jb][i] is (row
// r0 + 4 (lane / 16) + i, column c0 + J (lane % 16) + jb).  A, the k
// assignment and BF as in mma.
template <int J, int AR, int AK, int BK, bool BF = false>
__device__ __forceinline__ void mma_quad(f4 (&acc)[J], const float* A, int r0, const float* B,
                                         int c0, int kb, int ke) {
  typedef float fJ __attribute__((ext_vector_type(J)));
  const int l = lane_id(), r = l & 15, q = l >> 4;
  const float* pb = B + c0 + J * r;
  auto ldb_row = [&](int k) { return *reinterpret_cast<const fJ*>(pb + k * BK); };
  if constexpr (BF) {
    const float* pa = A + (r0 + r) * AR + 8 * q * AK;
    int k = kb;
#pragma unroll 1
    for (; k + 32 <= ke; k += 32) {
      const bf16x8 a = pack8(load_k4<AK>(pa + k * AK), load_k4<AK>(pa + (k + 4) * AK));
      // Each pair of k rows is rounded as it arrives: pk[jb][e] holds
      // k = 8 q + 2 e, +1 of column jb.
      bf16x2 pk[J][4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const fJ x0 = ldb_row(k + 8 * q + 2 * e), x1 = ldb_row(k + 8 * q + 2 * e + 1);
#pragma unroll
        for (int jb = 0; jb < J; ++jb) pk[jb][e] = cvt2(x0[jb], x1[jb]);
      }
#pragma unroll
      for (int jb = 0; jb < J; ++jb) {
        const bf16x8 b = bf16x8{pk[jb][0][0], pk[jb][0][1], pk[jb][1][0], pk[jb][1][1],
                                pk[jb][2][0], pk[jb][2][1], pk[jb][3][0], pk[jb][3][1]};
        acc[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[jb], 0, 0, 0);
      }
    }
    if (k < ke) {
      const bf16x4 a = pack4(load_k4<AK>(A + (r0 + r) * AR + (k + 4 * q) * AK));
      fJ bv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = ldb_row(k + 4 * q + e);
#pragma unroll
      for (int jb = 0; jb < J; ++jb) {
        const bf16x4 b = pack4(f4{bv[0][jb], bv[1][jb], bv[2][jb], bv[3][jb]});
        acc[jb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                            __builtin_bit_cast(s16x4, b),
                                                            acc[jb], 0, 0, 0);
      }
    }
  } else {
    const float* pa = A + (r0 + r) * AR + 4 * q * AK;
#pragma unroll 2
    for (int k = kb; k < ke; k += 16) {
      const f4 a = load_k4<AK>(pa + k * AK);
      fJ bv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = ldb_row(k + 4 * q + e);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int jb = 0; jb < J; ++jb)
          acc[jb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], bv[e][jb], acc[jb], 0, 0, 0);
    }
  }
}

// mma over the first jn (1..4, the same for the whole wave) of four column
// tiles: each count is its own straight-line instantiation, so no MFMA sits
// under a per-tile branch.
template <int AR, int AK, int BK, int BC>
__device__ __forceinline__ void mma_first(f4 (&acc)[4], const float* A, int r0, const float* B,
                                          int c0, int kb, int ke, int jn) {
  switch (jn) {
    case 1:
      mma<1, AR, AK, BK, BC>(*reinterpret_cast<f4(*)[1]>(acc), A, r0, B, c0, kb, ke);
      break;
    case 2:
      mma<2, AR, AK, BK, BC>(*reinterpret_cast<f4(*)[2]>(acc), A, r0, B, c0, kb, ke);
      break;
    case 3:
      mma<3, AR, AK, BK, BC>(*reinterpret_cast<f4(*)[3]>(acc), A, r0, B, c0, kb, ke);
      break;
    default:
      mma<4, AR, AK, BK, BC>(acc, A, r0, B, c0, kb, ke);
      break;
  }
}

template <int J>
__device__ __forceinline__ void zero(f4 (&acc)[J]) {
#pragma unroll
  for (int j = 0; j < J; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
}

// ---------------------------------------------------------------------------
// bfloat16 LDS tiles.  With bfloat16 operands the products' LDS operands are
// stored already rounded (to nearest even, as mma<..., BF> rounds a float32
// tile at its read), so every product is unchanged, with half the LDS bytes
// and no conversion per read.  Row strides of 68 words (= 4 mod 64) for
// [.][NT] tiles and 36 words for [.][PT] tiles spread a product's 16-byte
// operand reads over the banks.
constexpr int LQB = NT + 8;
constexpr int LVB = PT + 8;

template <bool BF>
struct Tile {
  typedef float T;
  static constexpr int LQt = LQ, LVt = LV;
};
template <>
struct Tile<true> {
  typedef bf16_t T;
  static constexpr int LQt = LQB, LVt = LVB;
};

typedef unsigned u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16_t to_bf(float x) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(x));
}
__device__ __forceinline__ unsigned to_bf2(float a, float b) {
  return __builtin_bit_cast(unsigned, cvt2(a, b));
}

// A tile's element, two adjacent elements, four adjacent elements.
__device__ __forceinline__ void put(float* p, float x) { *p = x; }
__device__ __forceinline__ void put(bf16_t* p, float x) { *p = to_bf(x); }
__device__ __forceinline__ void put2(float* p, float a, float b) {
  *reinterpret_cast<float2*>(p) = float2{a, b};
}
__device__ __forceinline__ void put2(bf16_t* p, float a, float b) {
  *reinterpret_cast<unsigned*>(p) = to_bf2(a, b);
}
__device__ __forceinline__ void put4(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }
__device__ __forceinline__ void put4(bf16_t* p, f4 v) {
  *reinterpret_cast<u2*>(p) = u2{to_bf2(v[0], v[1]), to_bf2(v[2], v[3])};
}
__device__ __forceinline__ float get(const float* p) { return *p; }
__device__ __forceinline__ float get(const bf16_t* p) { return lo_bf(*p); }
__device__ __forceinline__ f4 get4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f4 get4(const bf16_t* p) { return dec(*reinterpret_cast<const u2*>(p)); }

// Eight (four) consecutive-in-k bfloat16 operand values, k stride S: one
// 16-byte (8-byte) read when S is 1.
template <int S>
__device__ __forceinline__ bf16x8 load_k8(const bf16_t* p) {
  if constexpr (S == 1) {
    return *reinterpret_cast<const bf16x8*>(p);
  } else {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __builtin_bit_cast(__bf16, p[e * S]);
    return v;
  }
}
template <int S>
__device__ __forceinline__ bf16x4 load_k4b(const bf16_t* p) {
  if constexpr (S == 1) {
    return *reinterpret_cast<const bf16x4*>(p);
  } else {
    bf16x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __builtin_bit_cast(__bf16, p[e * S]);
    return v;
  }
}

// mma on bfloat16 tiles (the same k assignment and result layout).
template <int J, int AR, int AK, int BK, int BC, bool BF>
__device__ __forceinline__ void mma(f4 (&acc)[J], const bf16_t* A, int r0, const bf16_t* B,
                                    int c0, int kb, int ke) {
  static_assert(BF, "bfloat16 tiles hold bfloat16 operands");
  const int l = lane_id(), r = l & 15, q = l >> 4;
  const bf16_t* pa = A + (r0 + r) * AR + 8 * q * AK;
  const bf16_t* pb = B + 8 * q * BK + (c0 + r) * BC;
  int k = kb;
#pragma unroll 1
  for (; k + 32 <= ke; k += 32) {
    const bf16x8 a = load_k8<AK>(pa + k * AK);
    bf16x8 b[J];
#pragma unroll
    for (int j = 0; j < J; ++j) b[j] = load_k8<BK>(pb + k * BK + 16 * j * BC);
#pragma unroll
    for (int j = 0; j < J; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[j], acc[j], 0, 0, 0);
  }
  if (k < ke) {
    const bf16x4 a = load_k4b<AK>(A + (r0 + r) * AR + (k + 4 * q) * AK);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const bf16x4 b = load_k4b<BK>(B + (k + 4 * q) * BK + (c0 + 16 * j + r) * BC);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                         __builtin_bit_cast(s16x4, b),
                                                         acc[j], 0, 0, 0);
    }
  }
}

// mma_quad on bfloat16 tiles (J = 4): each k's four B values are one 8-byte
// read (two words, columns jb = 0, 1 and 2, 3), and a tile's operand pairs
// are assembled with one byte permute per pair of k.
template <int J, int AR, int AK, int BK, bool BF>
__device__ __forceinline__ void mma_quad(f4 (&acc)[J], const bf16_t* A, int r0, const bf16_t* B,
                                         int c0, int kb, int ke) {
  static_assert(BF && J == 4, "bfloat16 tiles: four columns per lane");
  const int l = lane_id(), r = l & 15, q = l >> 4;
  const bf16_t* pb = B + c0 + 4 * r;
  auto row = [&](int k) { return *reinterpret_cast<const u2*>(pb + k * BK); };
  // Column jb of rows x0 (low half) and x1 (high half).
  auto pair = [&](u2 x0, u2 x1, int jb) {
    return __builtin_amdgcn_perm(x1[jb >> 1], x0[jb >> 1], (jb & 1) ? 0x07060302u : 0x05040100u);
  };
  const bf16_t* pa = A + (r0 + r) * AR + 8 * q * AK;
  int k = kb;
#pragma unroll 1
  for (; k + 32 <= ke; k += 32) {
    const bf16x8 a = load_k8<AK>(pa + k * AK);
    u2 x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = row(k + 8 * q + e);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const u4 w = u4{pair(x[0], x[1], jb), pair(x[2], x[3], jb), pair(x[4], x[5], jb),
                      pair(x[6], x[7], jb)};
      acc[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, w),
                                                        acc[jb], 0, 0, 0);
    }
  }
  if (k < ke) {
    const bf16x4 a = load_k4b<AK>(A + (r0 + r) * AR + (k + 4 * q) * AK);
    u2 x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = row(k + 4 * q + e);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const u2 w = u2{pair(x[0], x[1], jb), pair(x[2], x[3], jb)};
      acc[jb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                          __builtin_bit_cast(s16x4, w),
                                                          acc[jb], 0, 0, 0);
    }
  }
}

// mma over the first jn (0..2, the same for the whole wave) of two column
// tiles, each count its own straight-line instantiation (float32 or
// bfloat16 tiles).
template <int AR, int AK, int BK, int BC, bool BF = false, typename TT>
__device__ __forceinline__ void mma_first2(f4 (&acc)[2], const TT* A, int r0, const TT* B, int c0,
                                           int kb, int ke, int jn) {
  if (jn >= 2) {
    mma<2, AR, AK, BK, BC, BF>(acc, A, r0, B, c0, kb, ke);
  } else if (jn == 1) {
    mma<1, AR, AK, BK, BC, BF>(*reinterpret_cast<f4(*)[1]>(acc), A, r0, B, c0, kb, ke);
  }
}

__device__ __forceinline__ long tok_index(const Shape& s, int b, int t) {
  return (long)b * s.T + t;
}
__device__ __forceinline__ long state_offset(const Shape& s, int b, int h, int c) {
  return (((long)b * s.H + h) * s.NC + c) * (long)(NT * PT);
}
__device__ __forceinline__ long phase_offset(const Shape& s, int b, int h, int c) {
  return (((long)b * s.H + h) * s.NC + c) * (long)AM;
}

// Per-token scalars of chunk c for head h, one token per lane (lane < 64):
// p (chunk-local running log decay), e^p, gamma, scale, u = scale e^{p_L - p}
// and dt, written to LDS arrays of 64.  Padding tokens get zeros (and p
// equal to the last real token's), so they contribute nothing.
struct Scalars {
  float *p, *ep, *gam, *scale, *u, *dt;
};

// The raw per-token inputs of one lane's token (zeros past T).
struct TokenIn {
  float a, d, tr, dn, trn;
};

// The buffer resource of chunk c's tokens (those below T, and up to `extra`
// tokens past the chunk) in a [B, T, width] array.
template <typename E>
__device__ __forceinline__ Rsrc chunk_rsrc(const Shape& s, const E* base, int b, int c,
                                           long width, int extra = 0) {
  return rsrc(base + tok_index(s, b, c * C) * width,
              (long)min(C + extra, s.T - c * C) * width * (long)sizeof(E));
}

// Lane l's token c C + l and the next token's dt and trapezoid weight, for
// the block's first wave (token_scalars' wave; the other waves' offsets are
// out of range, zeros without a memory access: each of these loads gathers
// one float per token).  The resources span one token past the chunk, and
// lane l < 64 < C + 1 is in range exactly when its token is below T (its
// next token likewise).
__device__ __forceinline__ TokenIn fetch_token(const Shape& s, const float* adt, const float* dt,
                                               const float* trap, int b, int h, int c) {
  const int tid = tix();
  const unsigned o = tid < 64 ? (tid * s.H + h) * 4 : kNoLoad;
  const unsigned on = tid < 64 ? o + s.H * 4 : kNoLoad;
  const Rsrc ra = chunk_rsrc(s, adt, b, c, s.H, 1), rd = chunk_rsrc(s, dt, b, c, s.H, 1),
             rt = chunk_rsrc(s, trap, b, c, s.H, 1);
  return TokenIn{ldb(ra, o), ldb(rd, o), ldb(rt, o), ldb(rd, on), ldb(rt, on)};
}

// The A start phases of an item (zeros past A).
__device__ __forceinline__ float fetch_phase(const Shape& s, const float* theta0, int b, int h,
                                             int c) {
  return ldb(rsrc(theta0 + phase_offset(s, b, h, c), 4L * s.A), tix() * 4);
}

__device__ void token_scalars(const TokenIn& in, const Scalars& o) {
  const int l = lane_id();
  const float a = in.a, d = in.d, tr = in.tr, dn = in.dn, trn = in.trn;
  const float sig = 1.f / (1.f + expf(-tr)), sign = 1.f / (1.f + expf(-trn));
  const float gam = d * sig, scale = gam + dn * (1.f - sign);
  const float p = wave_scan(a), pl = lane63(p);
  o.p[l] = p;
  o.ep[l] = expf(p);
  o.gam[l] = gam;
  o.scale[l] = scale;
  o.u[l] = scale * expf(pl - p);
  o.dt[l] = d;
}

// Phase table of chunk c: tab[t * LA + j] = th0[j] + sum_{s <= t} angles_s,j dt_s
// (j < A), one token per lane, angles j = w + NW m split over the NW waves
// of the block, dt from the chunk's scalars in LDS (zero past T).  With
// `advance`, th0[j] moves to the chunk's end phase reduced modulo 2 pi (th0
// lives in LDS and each j belongs to one wave, whose lanes read it before
// lane 63 writes it).
//
// This lane's token's angle rates j = w + NW m (zeros past T and A), kept in
// registers by a kernel that reuses them (one float per token and angle:
// each load gathers 64 tokens).
template <int NW = 4>
__device__ __forceinline__ void fetch_angles(const Shape& s, const float* ang, int b, int c,
                                             float (&xs)[64 / NW]) {
  const int w = tix() >> 6;
  const Rsrc r = chunk_rsrc(s, ang, b, c, s.A);
  const unsigned o = lane_id() * s.A * 4;
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) {
    const int j = w + NW * m;
    xs[m] = ldb(r, j < s.A ? o + 4 * j : kNoLoad);
  }
}

// The phase table from register-held angle rates.
template <int NW = 4>
__device__ void phase_table(const Shape& s, const float (&rates)[64 / NW], const float* dts,
                            float* th0, float* tab, bool advance) {
  const int l = lane_id(), w = tix() >> 6;
  const float d = dts[l];
  float xs[64 / NW];
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) xs[m] = rates[m] * d;
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) {
    const int j = w + NW * m;
    if (j >= s.A) break;
    const float incl = wave_scan(xs[m]);
    const float base = th0[j];
    tab[l * LA + j] = base + incl;
    if (advance) {
      __builtin_amdgcn_wave_barrier();
      if (l == 63) th0[j] = reduce_turns(base + incl);
    }
  }
}

// The chunk's angle rates as one block: [tokens][A] is contiguous in memory,
// so a 512-thread block reads it in eight coalesced loads per thread (A <=
// 64; zeros past the chunk's tokens), stage_angles writes them into the phase
// table's [C][LA] layout and phase_table_staged turns them into phases in
// place.
template <int NTH = 512>
__device__ __forceinline__ void fetch_angle_block(const Shape& s, const float* ang, int b, int c,
                                                  float (&a)[4096 / NTH]) {
  const Rsrc r = chunk_rsrc(s, ang, b, c, s.A);
  const int tid = tix();
#pragma unroll
  for (int k = 0; k < 4096 / NTH; ++k) a[k] = ldb(r, (tid + NTH * k) * 4);
}

template <int NTH = 512>
__device__ __forceinline__ void stage_angles(const Shape& s, const float (&a)[4096 / NTH],
                                             float* tab) {
  const int tid = tix();
#pragma unroll
  for (int k = 0; k < 4096 / NTH; ++k) {
    const int e = tid + NTH * k;
    if (e < C * s.A) tab[(e / s.A) * LA + e % s.A] = a[k];
  }
}

template <int NW = 4>
__device__ void phase_table_staged(const Shape& s, const float* dts, float* th0, float* tab,
                                   bool advance) {
  const int l = lane_id(), w = tix() >> 6;
  const float d = dts[l];
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) {
    const int j = w + NW * m;
    if (j >= s.A) break;
    const float incl = wave_scan(tab[l * LA + j] * d);
    const float base = th0[j];
    tab[l * LA + j] = base + incl;
    if (advance) {
      __builtin_amdgcn_wave_barrier();
      if (l == 63) th0[j] = reduce_turns(base + incl);
    }
  }
}

// Rotated rows of chunk c into LDS [C][LQ]: dst[t][n] = rot(src_t + bias, theta_t)[n]
// for t < C, n < NT, zero for padding tokens and coordinates.  One pair
// (2j, 2j+1) per lane, tokens w, w + 4, ... per wave; every global read is
// issued before the first rotation.  With two sources both are rotated by
// the same angles.  bfloat16 sources: the bias-added rows are rounded to
// bfloat16 before the rotation (_rotated, lm/kernels/flashmamba.py:582-585).
// This lane's pair (2 l, 2 l + 1) of a head's N biases (zeros past N).
__device__ __forceinline__ float2 fetch_bias_pair(const Shape& s, const float* bias) {
  return raw2(rsrc(bias, 4L * s.N), 8 * lane_id(), bias);
}

template <int NSRC, int NW = 4, typename In = float>
__device__ __forceinline__ void fetch_rows(const Shape& s, const In* const (&src)[2],
                                           const float* const (&bias)[2], int b, int c,
                                           typename Raw<In>::Pair (&u)[NSRC][64 / NW],
                                           float2 (&bs)[NSRC]) {
  const int n = 2 * lane_id(), w = tix() >> 6;
#pragma unroll
  for (int k = 0; k < NSRC; ++k) {
    const Rsrc r = chunk_rsrc(s, src[k], b, c, s.N);
#pragma unroll
    for (int m = 0; m < 64 / NW; ++m)
      u[k][m] = raw2(r, n < s.N ? ((w + NW * m) * s.N + n) * sizeof(In) : kNoLoad, src[k]);
    bs[k] = fetch_bias_pair(s, bias[k]);
  }
}

template <int NSRC, int NW = 4, int LD = LQ, typename Pair = float2, typename TT = float>
__device__ __forceinline__ void rotate_fetched(const Shape& s, const Pair (&u)[NSRC][64 / NW],
                                               const float2 (&bs)[NSRC], TT* const (&dst)[2],
                                               const float* tab, int c) {
  constexpr bool BF = !__is_same(Pair, float2);
  const int j = lane_id(), n = 2 * j, w = tix() >> 6;
  const bool col = n < s.N;
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) {
    const int t = w + NW * m, tt = c * C + t;
    const bool valid = col && tt < s.T;
    float sn = 0.f, cs = 1.f;
    if (valid && j < s.A) sin_cos(tab[t * LA + j], &sn, &cs);
#pragma unroll
    for (int k = 0; k < NSRC; ++k) {
      const float2 x = dec(u[k][m]);
      const float2 v =
          round_bf2<BF>(valid ? float2{x.x + bs[k].x, x.y + bs[k].y} : float2{0.f, 0.f});
      put2(dst[k] + t * LD + n, v.x * cs - v.y * sn, v.x * sn + v.y * cs);
    }
  }
}

// Value rows of head h for chunk c into LDS [C][LV], each row t scaled by
// row_scale[t] (nullptr: 1); zeros past T and P.  Four 16-byte rows pieces
// per thread, all read before any is stored (fetch_values, store_values).
// V4: P is a multiple of 4 (one vector load per piece; otherwise one load
// per element), chosen per launch so no kernel holds both paths.
template <int NTH, bool V4, typename In>
__device__ __forceinline__ void fetch_values(const Shape& s, const In* src, int b, int c, int h,
                                             typename Raw<In>::Quad (&v)[1024 / NTH]) {
  const Rsrc r = chunk_rsrc(s, src, b, c, (long)s.H * s.P);
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    const int e = tix() + NTH * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
    const unsigned off = ((t * s.H + h) * s.P + p) * sizeof(In);
    v[i] = V4 ? raw4(r, p < s.P ? off : kNoLoad, src) : raw4_n(r, off, s.P - p, src);
  }
}

// Into a [C][LD] tile of float32 or bfloat16 (bfloat16 inputs unscaled go
// in as their bits).
template <int NTH, int LD = LV, typename Quad, typename TT>
__device__ __forceinline__ void store_values(const Quad (&v)[1024 / NTH], const float* row_scale,
                                             TT* dst) {
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    const int e = tix() + NTH * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
    if constexpr (__is_same(TT, bf16_t) && __is_same(Quad, u2)) {
      if (!row_scale) {
        *reinterpret_cast<u2*>(dst + t * LD + p) = v[i];
        continue;
      }
    }
    put4(dst + t * LD + p, row_scale ? dec(v[i]) * row_scale[t] : dec(v[i]));
  }
}

// Value rows of head h for chunk c into LDS transposed, [PT][LV]: for
// i < 1024 / NTH, thread (wave w, lane L) takes the pieces (t, p .. p + 3)
// of block bi = i NTH / 64 + w, t = 16 (bi / 4) + L / 4, p = 16 (bi % 4) +
// 4 (L % 4) (zeros past T and P): each load instruction reads 16 tokens'
// 16-column pieces (not 64 tokens' rows, one cache line per lane), and each
// transposed LDS store ((p + k) LV + t, LV = 4 mod 64) hits 64 distinct
// banks.  fetch_values_t reads this thread's pieces into registers,
// store_values_t writes them.
template <int NTH>
__device__ __forceinline__ void value_slot(int i, int& t, int& p) {
  const int tid = tix(), L = tid & 63, bi = i * (NTH / 64) + (tid >> 6);
  t = 16 * (bi >> 2) + (L >> 2);
  p = 16 * (bi & 3) + 4 * (L & 3);
}

template <int NTH, bool V4, typename In>
__device__ __forceinline__ void fetch_values_t(const Shape& s, const In* src, int b, int c,
                                               int h, typename Raw<In>::Quad (&v)[1024 / NTH]) {
  const Rsrc r = chunk_rsrc(s, src, b, c, (long)s.H * s.P);
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    int t, p;
    value_slot<NTH>(i, t, p);
    const unsigned off = ((t * s.H + h) * s.P + p) * sizeof(In);
    v[i] = V4 ? raw4(r, p < s.P ? off : kNoLoad, src) : raw4_n(r, off, s.P - p, src);
  }
}

template <int NTH, int LD = LV, typename Quad, typename TT>
__device__ __forceinline__ void store_values_t(const Quad (&v)[1024 / NTH], TT* dst) {
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    int t, p;
    value_slot<NTH>(i, t, p);
    const f4 x = dec(v[i]);
#pragma unroll
    for (int k = 0; k < 4; ++k) put(dst + (p + k) * LD + t, x[k]);
  }
}

// A stored [NT][PT] state tile in registers: for i < 2048 / NTH, thread
// (wave w, lane L) holds the four elements (n, p .. p + 3) of block
// bi = i NTH / 64 + w, with n = 16 (bi / 4) + L / 4 and p = 16 (bi % 4) +
// 4 (L % 4).  Each load instruction reads one 16 x 16 block (16 row pieces
// of 64 contiguous bytes, not 64 lanes each in its own cache line), and
// each transposed LDS store instruction ((p + k) LQ + n, LQ = 4 mod 64)
// hits 64 distinct banks.
template <int NTH>
__device__ __forceinline__ void state_slot(int i, int& n, int& p) {
  const int tid = tix(), L = tid & 63, bi = i * (NTH / 64) + (tid >> 6);
  n = 16 * (bi >> 2) + (L >> 2);
  p = 16 * (bi & 3) + 4 * (L & 3);
}

template <int NTH = 256>
__device__ __forceinline__ void fetch_state_t(const float* src, f4 (&v)[2048 / NTH]) {
#pragma unroll
  for (int i = 0; i < 2048 / NTH; ++i) {
    int n, p;
    state_slot<NTH>(i, n, p);
    v[i] = *reinterpret_cast<const f4*>(src + n * PT + p);
  }
}

// Into LDS transposed, [PT][LD] (float32 or bfloat16).
template <int NTH = 256, int LD = LQ, typename TT>
__device__ __forceinline__ void store_state_t(const f4 (&v)[2048 / NTH], TT* dst) {
#pragma unroll
  for (int i = 0; i < 2048 / NTH; ++i) {
    int n, p;
    state_slot<NTH>(i, n, p);
#pragma unroll
    for (int k = 0; k < 4; ++k) put(dst + (p + k) * LD + n, v[i][k]);
  }
}



// ---------------------------------------------------------------------------
// State walks.  Forward (BWD = false): rows = keys b with k_bias, vals = x
// scaled by u; S starts at zero; each chunk stores its start state to
// `saved`, its start phase to theta0, then S <- e^{p_L} S + K^T (u v).
// Backward (BWD = true): rows = queries c with q_bias, vals = d_y scaled by
// e^p; S starts at d_final and the chunks run in reverse; each stores S (the
// cotangent of the state at the chunk's end) to `saved`, then
// S <- e^{p_L} S + Q^T (e^p dy).
//
// Rows of S are independent, so each (b, h) runs as two blocks of four
// waves, block `half` holding state rows 64 half .. +63 (coordinate pairs,
// and angles, 32 half .. +31): three of them share a compute unit where
// two eight-wave blocks fit, and every compute unit carries the same work
// (with one block per sequence a third of the units held two and set the
// pace).  Both halves read all of a chunk's values and compute its
// per-token scalars.
// LDS: the half's rotated rows [C][LQH], vals [C][LV], its phase table
// [C][LA] (columns = the half's angles), th0 [AM], scalars.
constexpr int LQH = 64 + 4;

template <bool BWD, typename In, bool V4>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void walk_kernel(
    Shape s, const In* rows, const float* bias, const In* vals, const float* adt, const float* dt,
    const float* trap, const float* ang, float* theta0, float* saved, const float* init,
    float* final_state) {
  constexpr bool BF = is_bf16<In>::value;
  extern __shared__ float sm[];
  float* rt = sm;
  float* vt = rt + C * LQH;
  float* tab = vt + C * LV;
  float* th0 = tab + C * LA;
  float* sc = th0 + AM;
  const Scalars S{sc, sc + 64, sc + 128, sc + 192, sc + 256, sc + 320};
  // Both halves of a sequence on one XCD (blocks go round-robin over the
  // eight), so the second half's value reads hit that XCD's L2.
  const int G = 2 * s.B * s.H, x = blockIdx.x;
  int half, bh;
  if (x < (G & ~15)) {
    const int slot = x >> 3;
    half = slot & 1;
    bh = (slot >> 1) * 8 + (x & 7);
  } else {
    half = x & 1;
    bh = x >> 1;
  }
  const int b = bh / s.H, h = bh % s.H;
  const int n0 = 64 * half, j0 = 32 * half;   // first state row and angle of the half
  const int na = max(0, min(32, s.A - j0));  // the half's angles
  const int tid = tix(), w = tid >> 6, l = lane_id(), r = l & 15, q = l >> 4;

  // Four waves: wave w holds state rows n0 + 16 w .. +15 as four 16-column
  // tiles.
  f4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = n0 + 16 * w + 4 * q + i, p = 16 * j + r;
      float v = 0.f;
      if (BWD && init && n < s.N && p < s.P) v = init[(((long)b * s.H + h) * s.N + n) * s.P + p];
      acc[j][i] = v;
    }
  }
  if (!BWD && tid < AM) th0[tid] = 0.f;
  // This lane's coordinate pair (32 per half, two tokens per wave step).
  const int pr = l & 31, n = n0 + 2 * pr;
  const bool col = n < s.N;
  const float2 bs = raw2(rsrc(bias + (long)h * s.N, 4L * s.N), col ? n * 4 : kNoLoad, bias);

  // Every global input of a chunk is fetched into registers one chunk ahead,
  // while the previous chunk's product runs.
  TokenIn tin;
  float rates[8], th_in = 0.f;
  typename Raw<In>::Pair u[8];
  typename Raw<In>::Quad v[4];
  auto fetch = [&](int c) {
    tin = fetch_token(s, adt, dt, trap, b, h, c);
    {
      // The half's angle rates of the chunk's tokens: [t][j0 + j'], j' < na.
      const Rsrc ra = chunk_rsrc(s, ang, b, c, s.A);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int e = tid + 256 * k, t = e >> 5, jj = e & 31;
        rates[k] = ldb(ra, jj < na ? (t * s.A + j0 + jj) * 4 : kNoLoad);
      }
    }
    if (BWD)
      th_in = ldb(rsrc(theta0 + phase_offset(s, b, h, c) + j0, 4L * na), tid < 64 ? tid * 4 : kNoLoad);
    const Rsrc rr = chunk_rsrc(s, rows, b, c, s.N);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int t = 2 * (w + 4 * m) + (l >> 5);
      u[m] = raw2(rr, col ? (t * s.N + n) * sizeof(In) : kNoLoad, rows);
    }
    fetch_values<256, V4>(s, vals, b, c, h, v);
  };
  fetch(BWD ? s.NC - 1 : 0);

  for (int step = 0; step < s.NC; ++step) {
    const int c = BWD ? s.NC - 1 - step : step;
    __syncthreads();  // the previous chunk's reads of the LDS tiles are done
    // This chunk's state (a lane's four rows of one column), stored by waves
    // 1-3 while wave 0 turns the token inputs into the chunk's scalars.
    float* out = saved + state_offset(s, b, h, c);
    if (w != 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[(n0 + 16 * w + 4 * q + i) * PT + 16 * j + r] = acc[j][i];
    }
    if (w == 0) token_scalars(tin, S);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = tid + 256 * k;
      tab[(e >> 5) * LA + (e & 31)] = rates[k];
    }
    if (BWD) {
      if (tid < na) th0[tid] = th_in;
    } else {
      // Lanes at or past the half's angles store out of range (dropped).
      __builtin_amdgcn_raw_buffer_store_b32(
          __float_as_uint(th0[tid & (AM - 1)]),
          rsrc(theta0 + phase_offset(s, b, h, c) + j0, 4L * na), tid * 4, 0, 0);
    }
    __syncthreads();
    // The half's phase table: angles j' = w + 4 m, one token per lane; the
    // eight scans of a wave are independent and run interleaved (every read
    // of th0 comes before lane 63's writes).
    {
      const float d = S.dt[l];
      float x[8], base[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        x[m] = tab[l * LA + w + 4 * m] * d;
        base[m] = th0[w + 4 * m];
      }
#pragma unroll
      for (int m = 0; m < 8; ++m) x[m] = base[m] + wave_scan(x[m]);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int jj = w + 4 * m;
        if (jj < na) {
          tab[l * LA + jj] = x[m];
          if (!BWD && l == 63) th0[jj] = reduce_turns(x[m]);
        }
      }
    }
    __syncthreads();
    // Rotated rows (one pair per lane, two tokens per step) and scaled
    // values into LDS.
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int t = 2 * (w + 4 * m) + (l >> 5), tt = c * C + t;
      const bool valid = col && tt < s.T;
      float sn = 0.f, cs = 1.f;
      if (valid && pr < na) sin_cos(tab[t * LA + pr], &sn, &cs);
      // The bias-added row in the model dtype, then rotated in float32 (:582-585).
      const float2 um = dec(u[m]);
      const float2 x2 = round_bf2<BF>(valid ? float2{um.x + bs.x, um.y + bs.y}
                                            : float2{0.f, 0.f});
      *reinterpret_cast<float2*>(rt + t * LQH + 2 * pr) =
          float2{x2.x * cs - x2.y * sn, x2.x * sn + x2.y * cs};
    }
    store_values<256>(v, BWD ? S.ep : S.u, vt);
    // The next chunk's inputs (this chunk's again after the last: every
    // iteration issues the same loads), then wave 0's rows of the state.
    fetch(step + 1 < s.NC ? (BWD ? c - 1 : c + 1) : c);
    if (w == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[(n0 + 16 * w + 4 * q + i) * PT + 16 * j + r] = acc[j][i];
    }
    __syncthreads();
    const float decay = expf(S.p[63]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] *= decay;
    // rows^T vals: A(n, t) = rt[t * LQH + n], B(t, p) = vt[t * LV + p].
    mma<4, 1, LQH, LV, 1, BF>(acc, rt, 16 * w, vt, 0, 0, C);
  }
  if (!BWD && final_state) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int nn = n0 + 16 * w + 4 * q + i, p = 16 * j + r;
        if (nn < s.N && p < s.P)
          final_state[(((long)b * s.H + h) * s.N + nn) * s.P + p] = acc[j][i];
      }
  }
}

// Block index -> (b, chunk, h), heads fastest.  Consecutive blocks land on
// different XCDs (round robin over 8); the remap gives each XCD a contiguous
// run of (b, chunk) pairs, so the heads of one chunk share its rows in one L2.
__device__ __forceinline__ int xcd_block(int total) {
  const int id = blockIdx.x;
  if (total % 8) return id;
  return (id % 8) * (total / 8) + id / 8;
}

// The same remap of a persistent kernel's item index (its grid a multiple
// of 8, so item it runs on the XCD of block it % 8 as in xcd_block).
__device__ __forceinline__ int xcd_item(int it, int total) {
  if (total % 8) return it;
  return (it % 8) * (total / 8) + it / 8;
}

// ---------------------------------------------------------------------------
// Output of each (b, chunk, h) item: y = (S o W) V + diag(e^p) Q S0 with scores
// S = Q K^T and W_ts = e^{p_t - p_s} scale_s (s < t), gamma_t (s = t).
// LDS: Q [C][LQt], K [C][LQt] (later S o W as [C][LVt]), H0 transposed
// [PT][LQt] (first the phase table), V transposed [PT][LVt], scalars.  With
// bfloat16 tiles that is 62 KB, and two blocks of eight waves share a compute
// unit (float32: 122 KB, one block of sixteen waves).
template <typename In, bool V4>
__global__ __launch_bounds__(is_bf16<In>::value ? 512 : 1024) void out_kernel(Shape s, const In* cq, const In* bk,
                                                  const In* x, const float* adt,
                                                  const float* dt, const float* trap,
                                                  const float* ang, const float* qb,
                                                  const float* kb, const float* theta0,
                                                  const float* starts, In* y) {
  constexpr bool BF = is_bf16<In>::value;
  // Waves per block: float32 (one 122 KB block per CU) sixteen, four per
  // SIMD; bfloat16 (two 62 KB blocks per CU) eight.
  constexpr int NW = BF ? 8 : 16, NTH = 64 * NW;
  // The products' LDS operands: float32, or bfloat16 rounded where written.
  typedef typename Tile<BF>::T TT;
  constexpr int LQt = Tile<BF>::LQt, LVt = Tile<BF>::LVt;
  extern __shared__ float sm[];
  TT* const qt = reinterpret_cast<TT*>(sm);
  TT* const kt = qt + C * LQt;
  TT* const h0 = kt + C * LQt;
  // H0's region also holds the float32 phase table, [C][LA].
  TT* const vt = h0 + (BF ? PT * LQt : NT * LV);
  float* tab = reinterpret_cast<float*>(h0);
  float* th0 = reinterpret_cast<float*>(vt + PT * LVt);
  float* sc = th0 + AM;
  const Scalars S{sc, sc + 64, sc + 128, sc + 192, sc + 256, sc + 320};
  const int total = s.B * s.NC * s.H;
  const In* const src[2] = {cq, bk};

  // Every global input of an item, fetched into registers while the
  // previous item's products run.
  struct Fetched {
    TokenIn tin;
    float th, rates[4096 / NTH];
    typename Raw<In>::Pair u[2][64 / NW];
    float2 bs[2];
    f4 hv[2048 / NTH];
    typename Raw<In>::Quad vv[1024 / NTH];
  };
  auto item_of = [&](int it, int& b, int& c, int& h) {
    const int id = xcd_item(it, total);
    h = id % s.H;
    c = (id / s.H) % s.NC;
    b = id / (s.H * s.NC);
  };
  auto fetch = [&](Fetched& F, int it) {
    int b, c, h;
    item_of(it, b, c, h);
    F.tin = fetch_token(s, adt, dt, trap, b, h, c);
    F.th = fetch_phase(s, theta0, b, h, c);
    fetch_angle_block<NTH>(s, ang, b, c, F.rates);
    const float* const bsrc[2] = {qb + (long)h * s.N, kb + (long)h * s.N};
    fetch_rows<2, NW>(s, src, bsrc, b, c, F.u, F.bs);
    fetch_state_t<NTH>(starts + state_offset(s, b, h, c), F.hv);
    fetch_values_t<NTH, V4>(s, x, b, c, h, F.vv);
  };

  // Persistent: block i handles items i, i + gridDim.x, ... (b, chunk, h),
  // heads fastest, each XCD a contiguous run of (b, chunk) pairs.
  Fetched F;
  int it = blockIdx.x;
  if (it < total) fetch(F, it);
  for (; it < total; it += gridDim.x) {
    int b, c, h;
    item_of(it, b, c, h);
    const int tid = tix(), l = lane_id(), r = l & 15, q = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

    if (w == 0) token_scalars(F.tin, S);
    if (tid < s.A) th0[tid] = F.th;
    stage_angles<NTH>(s, F.rates, tab);
    // The values transposed, [PT][LV] (their region holds no staging
    // table), while wave 0 derives the token scalars.
    store_values_t<NTH, LVt>(F.vv, vt);
    __syncthreads();
    phase_table_staged<NW>(s, S.dt, th0, tab, false);
    __syncthreads();
    {
      TT* const dst[2] = {qt, kt};
      rotate_fetched<2, NW, LQt>(s, F.u, F.bs, dst, tab, c);
    }
    __syncthreads();  // the phase table (in h0's space) is read
    // The start state transposed, [PT][LQ] (as the values), so that every
    // product reads both operands contiguously along k.
    store_state_t<NTH, LQt>(F.hv, h0);
    __syncthreads();
    if constexpr (NW == 16) {
      // Sixteen waves: wave w = m + 4 wr (SIMD m) owns row block wr and
      // column tile wq = (m - wr) mod 4, so every SIMD holds each row block
      // once and two or three of the ten causal score tiles (eight waves:
      // 239 us against 266 us at B16 L1024 H24).  The first eight waves
      // issue the next item's loads before the scores, the others after.
      const int wq = ((w & 3) - (w >> 2)) & 3, wr2 = w >> 2;
      const int next = it + gridDim.x;
      if (w < 8) fetch(F, next < total ? next : it);
      f4 sco[1], qh[1];
      zero(sco);
      zero(qh);
      if (wq <= wr2) mma<1, LQt, 1, 1, LQt, BF>(sco, qt, 16 * wr2, kt, 16 * wq, 0, NT);
      if (w >= 8) fetch(F, next < total ? next : it);
      mma<1, LQt, 1, 1, LQt, BF>(qh, qt, 16 * wr2, h0, 16 * wq, 0, NT);
      __syncthreads();  // every wave is done with K
      TT* const gs = kt;
      if (wq <= wr2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * wr2 + 4 * q + i, u = 16 * wq + r;
          float wt = 0.f;
          if (t > u) wt = expf(fminf(S.p[t] - S.p[u], 0.f)) * S.scale[u];
          else if (t == u) wt = S.gam[t];
          put(gs + t * LVt + u, sco[0][i] * wt);
        }
      }
      __syncthreads();  // a row block's S o W comes from four waves
      f4 acc[1];
      zero(acc);
      mma<1, LVt, 1, 1, LVt, BF>(acc, gs, 16 * wr2, vt, 16 * wq, 0, 16 * (wr2 + 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * wr2 + 4 * q + i, p = 16 * wq + r, tt = c * C + t;
        if (tt < s.T && p < s.P)
          st1(y + (tok_index(s, b, tt) * s.H + h) * s.P + p, acc[0][i] + S.ep[t] * qh[0][i]);
      }
      __syncthreads();  // the tiles and scalars are read before the next item's staging
      continue;
    }
    // Eight waves: wave w owns column half wc = w >> 2 and row block wr =
    // w & 3, mirrored (3 - (w & 3)) in the second half, so the two waves on
    // each SIMD (w, w + 4) hold row blocks whose causal work sums to the same.
    const int wc = w >> 2, wr = wc ? 3 - (w & 3) : w & 3;
    // The next item's inputs load while this one's products run (no global
    // load is waited for before the next item's staging).  The two waves on
    // a SIMD issue them at different points (before and after the scores),
    // so one wave's products run while the other waits to issue its loads.
    const int next = it + gridDim.x;
    if (wc == 0) fetch(F, next < total ? next : it);

    const int ns = min(2, max(0, wr + 1 - 2 * wc));
    f4 sco[2], qh[2];
    zero(sco);
    zero(qh);
    mma_first2<LQt, 1, 1, LQt, BF>(sco, qt, 16 * wr, kt, 32 * wc, 0, NT, ns);
    if (wc == 1) fetch(F, next < total ? next : it);
    mma<2, LQt, 1, 1, LQt, BF>(qh, qt, 16 * wr, h0, 32 * wc, 0, NT);
    __syncthreads();  // every wave is done with K
    TT* const gs = kt;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int jt = 2 * wc + j;
      if (jt > wr) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * wr + 4 * q + i, u = 16 * jt + r;
        float wt = 0.f;
        if (t > u) wt = expf(fminf(S.p[t] - S.p[u], 0.f)) * S.scale[u];
        else if (t == u) wt = S.gam[t];
        put(gs + t * LVt + u, sco[j][i] * wt);
      }
    }
    __syncthreads();  // a row block's S o W comes from both of its waves
    f4 acc[2];
    zero(acc);
    // B(s, p) = Vt[p * LV + s].
    mma<2, LVt, 1, 1, LVt, BF>(acc, gs, 16 * wr, vt, 32 * wc, 0, 16 * (wr + 1));
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * wr + 4 * q + i, p = 32 * wc + 16 * j + r, tt = c * C + t;
        if (tt < s.T && p < s.P)
          st1(y + (tok_index(s, b, tt) * s.H + h) * s.P + p, acc[j][i] + S.ep[t] * qh[j][i]);
      }
    __syncthreads();  // the tiles and scalars are read before the next item's staging
  }
}

// ---------------------------------------------------------------------------
// Gradients of one (b, chunk) for the heads of group g.  Per head, with
// G = dS o W (dS = dY V^T), the chunk's start state H0 and end cotangent dH1:
//   dQ = G K + diag(e^p) dY H0^T          dK = G^T Q + diag(u) V dH1^T
//   dV = (S o W)^T dY + diag(u) K dH1
//   dgamma_t = S_tt dS_tt;  with F_ts = S_ts dS_ts e^{p_t - p_s} (s < t):
//   dscale_s = sum_t F_ts + e^{p_L - p_s} g_s,  g_s = v_s . (K dH1)_s
//   dp_t = sum_s F_ts scale_s - sum_t' F_t't scale_t + e^{p_t} dy_t . (Q H0)_t
//          - u_t g_t + [t = last] (sum_s u_s g_s + e^{p_L} <dH1, H0>)
//   d adt_s = sum_{t >= s} dp_t (within the chunk)
// then the rotation's transpose (dq -> d(c + qb)) and the phase gradient
// dtheta_t,j = dq_{2j+1} q_{2j} - dq_{2j} q_{2j+1} (+ the same for k), summed
// from the end of the chunk: R_t = sum_{t' >= t} dtheta_t'.
// LDS: R1 = 2 NT LV floats (Q, K; later H0, dH1 transposed; later dQ, dK),
// R2 = 2 NT LV floats (H0, dH1 transposed; later V, dY, S o W, G), phase
// table [C][LA], scalars.
template <typename In, bool V4>
__global__ __launch_bounds__(512) void grad_kernel(Shape s, int groups, const In* cq,
                                                   const In* bk, const In* x,
                                                   const float* adt, const float* dt,
                                                   const float* trap, const float* ang,
                                                   const float* qb, const float* kb,
                                                   const float* theta0, const float* starts,
                                                   const float* dh1, const In* dy, GradOut o) {
  constexpr bool BF = is_bf16<In>::value;
  // The products' LDS operands: float32, or bfloat16 rounded where they are
  // written (the dQ / dK epilogue tiles stay float32).
  typedef typename Tile<BF>::T TT;
  constexpr int LQt = Tile<BF>::LQt, LVt = Tile<BF>::LVt;
  In* const dx = static_cast<In*>(o.dx);
  extern __shared__ float sm[];
  float* R1 = sm;
  float* R2 = R1 + 2 * NT * LV;
  float* tab = R2 + 2 * NT * LV;
  float* th0 = tab + C * LA;
  float* sc = th0 + AM;
  const Scalars S{sc, sc + 64, sc + 128, sc + 192, sc + 256, sc + 320};
  // Every reduction over waves goes through one LDS slot per contributing
  // wave, summed in a fixed order afterwards (no atomics), so the gradients
  // are identical run to run.  Row sums: one slot per column half; column
  // sums: one per row block; the H0 . dH1 product: one per wave.
  float* s_rowE = sc + 384;   // [2][64]
  float* s_qd = sc + 512;     // [2][64]
  float* s_g = sc + 640;      // [2][64]
  float* s_colF = sc + 768;   // [4][64]
  float* s_colE = sc + 1024;  // [4][64]
  float* s_dgd = sc + 1280;   // [64]
  float* hsum = sc + 1344;    // [8]
  // The bias and dt partials of the rotation and phase passes, one row per
  // wave, in R2 (unused from the last dY / V product to the next head).
  float* qbp = R2;            // [8][NT]
  float* kbp = R2 + 8 * NT;   // [8][NT]
  float* ddtp = R2 + 16 * NT; // [8][64]

  const int total = s.B * s.NC * groups, id = xcd_block(total);
  const int g = id % groups, c = (id / groups) % s.NC, b = id / (groups * s.NC);
  const int hpg = (s.H + groups - 1) / groups, h_begin = g * hpg;
  const int h_end = min(s.H, h_begin + hpg);
  // Eight waves: wave w owns column half wc = w >> 2 of every 64-row tile's
  // columns and its row block wr = w & 3, mirrored (3 - (w & 3)) in the
  // second half, so the two waves on each SIMD (w, w + 4) hold row blocks
  // whose causal work sums to the same.  This group's sums over its
  // heads: the rotated-back row gradients of this thread's 8 (token
  // w + 8 m, pair) slots and the angle gradients of its 8 (token = lane,
  // angle w + 8 m) slots stay in registers until the last head.
  float2 dcacc[8], dbacc[8];
  float dang[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    dcacc[m] = float2{0.f, 0.f};
    dbacc[m] = float2{0.f, 0.f};
    dang[m] = 0.f;
  }
  // The chunk's raw query and key rows and its angle rates are the same for
  // every head: this thread's 8 (token, pair) slots and 8 (token = lane,
  // angle w + 8 m) rates are read once and kept in registers.
  typename Raw<In>::Pair rc[8], rb[8];
  float rates[8];
  fetch_angles<8>(s, ang, b, c, rates);
  {
    const int tid = tix(), l = tid & 63, w = tid >> 6;
    const Rsrc r0 = chunk_rsrc(s, cq, b, c, s.N), r1 = chunk_rsrc(s, bk, b, c, s.N);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const unsigned off = 2 * l < s.N ? ((w + 8 * m) * s.N + 2 * l) * sizeof(In) : kNoLoad;
      rc[m] = raw2(r0, off, cq);
      rb[m] = raw2(r1, off, bk);
    }
  }

  // A head's own inputs, fetched into registers while the previous head's
  // last phases run: its per-token scalars, start phase, start state and
  // end cotangent (read once: staged transposed for the products with Q
  // and K, and with float32 tiles staged again from the same registers for
  // the products with dY and V) and biases.  Its values and d_y load at the head's start, for its fourth
  // phase.
  struct HeadIn {
    TokenIn tin;
    float th;
    f4 hs[4], hg[4];
    float2 bq, bk;
  };
  auto fetch_head = [&](HeadIn& F, int h) {
    F.tin = fetch_token(s, adt, dt, trap, b, h, c);
    F.th = fetch_phase(s, theta0, b, h, c);
    fetch_state_t<512>(starts + state_offset(s, b, h, c), F.hs);
    fetch_state_t<512>(dh1 + state_offset(s, b, h, c), F.hg);
    F.bq = fetch_bias_pair(s, qb + (long)h * s.N);
    F.bk = fetch_bias_pair(s, kb + (long)h * s.N);
  };
  HeadIn F;
  if (h_begin < h_end) fetch_head(F, h_begin);

  for (int h = h_begin; h < h_end; ++h) {
    const int tid = tix(), l = tid & 63, r = l & 15, q = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wc = w >> 2;
    const int wr = wc ? 3 - (w & 3) : w & 3;
    const int n2 = 2 * l;  // this lane's coordinate pair in the rotation passes
    __syncthreads();  // the previous head is done with every LDS array
    typename Raw<In>::Quad vx[2], vd[2];
    fetch_values<512, V4>(s, x, b, c, h, vx);
    fetch_values<512, V4>(s, dy, b, c, h, vd);
    if (w == 0) token_scalars(F.tin, S);
    if (tid < s.A) th0[tid] = F.th;
    // Column sums: the row blocks above a column block contribute nothing.
    if (tid < 256) {
      s_colF[tid] = 0.f;
      s_colE[tid] = 0.f;
    }
    __syncthreads();
    phase_table<8>(s, rates, S.dt, th0, tab, false);
    __syncthreads();
    TT* const qt = reinterpret_cast<TT*>(R1);
    TT* const kt = qt + C * LQt;
    // The start state and end cotangent transposed, [PT][LQt], for Q H0 and
    // K dH1 with both operands contiguous along n.  bfloat16 tiles: in R1
    // after Q and K, where they stay for the dY and V products of the
    // second half; float32: in R2, staged again into R1 for those.
    TT* const h0 = BF ? kt + C * LQt : reinterpret_cast<TT*>(R2);
    TT* const g1 = h0 + PT * LQt;
    store_state_t<512, LQt>(F.hs, h0);
    store_state_t<512, LQt>(F.hg, g1);
    {
      // <H0, dH1> from the registers (both tiles in the same layout).
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) part += F.hs[i][k] * F.hg[i][k];
      part = wave_sum(part);
      if (l == 0) hsum[w] = part;
    }
    const float2 bq = F.bq, bkv = F.bk;
    {
      const bool col = n2 < s.N;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int t = w + 8 * m, tt = c * C + t;
        const bool valid = col && tt < s.T;
        float sn = 0.f, cs = 1.f;
        if (valid && l < s.A) sin_cos(tab[t * LA + l], &sn, &cs);
        const float2 cm = dec(rc[m]), bm = dec(rb[m]);
        const float2 u = round_bf2<BF>(valid ? float2{cm.x + bq.x, cm.y + bq.y}
                                             : float2{0.f, 0.f});
        const float2 v = round_bf2<BF>(valid ? float2{bm.x + bkv.x, bm.y + bkv.y}
                                             : float2{0.f, 0.f});
        put2(qt + t * LQt + n2, u.x * cs - u.y * sn, u.x * sn + u.y * cs);
        put2(kt + t * LQt + n2, v.x * cs - v.y * sn, v.x * sn + v.y * cs);
      }
    }
    __syncthreads();

    // Q H0, K dH1 and the scores (rows 16 wr .. +15, columns 32 wc .. +31;
    // the scores' causal tiles jt = 2 wc + j <= wr only).
    const int ns = min(2, max(0, wr + 1 - 2 * wc));
    f4 sco[2], qh[2], kg[2];
    zero(sco);
    zero(qh);
    zero(kg);
    mma_first2<LQt, 1, 1, LQt, BF>(sco, qt, 16 * wr, kt, 32 * wc, 0, NT, ns);
    // B(n, p) = H0t[p * LQt + n].
    mma<2, LQt, 1, 1, LQt, BF>(qh, qt, 16 * wr, h0, 32 * wc, 0, NT);
    mma<2, LQt, 1, 1, LQt, BF>(kg, kt, 16 * wr, g1, 32 * wc, 0, NT);
    __syncthreads();
    // V, dY, S o W and G as [C][LVt] tiles.  With bfloat16 tiles R2 has
    // room for transposed copies of G and dY, and S o W is kept transposed
    // only, so every operand of G^T Q and (S o W)^T dY is contiguous along k.
    TT* const vt = reinterpret_cast<TT*>(R2);
    TT* const dyt = vt + C * LVt;
    TT* const gs = vt + 2 * C * LVt;  // float32: [t][s]; bfloat16: [s][t]
    TT* const gm = vt + 3 * C * LVt;
    TT* const gmt = vt + 4 * C * LVt;  // bfloat16: G transposed
    TT* const dyT = vt + 5 * C * LVt;  // bfloat16: dY transposed, [p][t]
    store_values<512, LVt>(vx, nullptr, vt);
    store_values<512, LVt>(vd, nullptr, dyt);
    if constexpr (BF) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + 512 * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
        const u2 x = vd[i];
        dyT[p * LVt + t] = (bf16_t)x.x;
        dyT[(p + 1) * LVt + t] = (bf16_t)(x.x >> 16);
        dyT[(p + 2) * LVt + t] = (bf16_t)x.y;
        dyT[(p + 3) * LVt + t] = (bf16_t)(x.y >> 16);
      }
    }
    __syncthreads();

    f4 dsc[2];
    zero(dsc);
    // dY V^T: A(t, p) = dY[t * LVt + p], B(p, s) = V[s * LVt + p].
    mma_first2<LVt, 1, 1, LVt, BF>(dsc, dyt, 16 * wr, vt, 32 * wc, 0, PT, ns);
    {
      float qd[4] = {0.f, 0.f, 0.f, 0.f}, gg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * wr + 4 * q + i, p = 32 * wc + 16 * j + r;
          qd[i] += qh[j][i] * get(dyt + t * LVt + p);
          gg[i] += kg[j][i] * get(vt + t * LVt + p);
        }
      float rowE[4] = {0.f, 0.f, 0.f, 0.f};
      float colF[2] = {0.f, 0.f}, colE[2] = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int jt = 2 * wc + j;
        if (jt > wr) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 16 * wr + 4 * q + i, u = 16 * jt + r;
            put(gs + (BF ? u * LVt + t : t * LVt + u), 0.f);
            put(gm + t * LVt + u, 0.f);
            if constexpr (BF) put(gmt + u * LVt + t, 0.f);
          }
          continue;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * wr + 4 * q + i, u = 16 * jt + r;
          const float st = sco[j][i], ds = dsc[j][i];
          float wt = 0.f;
          if (t > u) {
            const float dec = expf(fminf(S.p[t] - S.p[u], 0.f));
            const float f = st * ds * dec;
            wt = dec * S.scale[u];
            rowE[i] += f * S.scale[u];
            colF[j] += f;
            colE[j] += f * S.scale[u];
          } else if (t == u) {
            wt = S.gam[t];
            s_dgd[t] = st * ds;
          }
          put(gs + (BF ? u * LVt + t : t * LVt + u), st * wt);
          put(gm + t * LVt + u, ds * wt);
          if constexpr (BF) put(gmt + u * LVt + t, ds * wt);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = row16_sum(qd[i]), bb = row16_sum(gg[i]), e = row16_sum(rowE[i]);
        if (r == 0) {
          // The two column halves of a row block sum into the same rows.
          const int t = 64 * wc + 16 * wr + 4 * q + i;
          s_qd[t] = a;
          s_g[t] = bb;
          s_rowE[t] = e;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int jt = 2 * wc + j;
        if (jt > wr) break;
        float f = colF[j], e = colE[j];
        f = group4_sum(f);
        e = group4_sum(e);
        if (q == 0) {
          s_colF[64 * wr + 16 * jt + r] = f;
          s_colE[64 * wr + 16 * jt + r] = e;
        }
      }
    }
    __syncthreads();

    // Rows 16 wr .. +15; dQ and dK columns 64 wc .. +63, dV columns 32 wc .. +31.
    f4 dq[4], dk[4], dv[2];
    zero(dq);
    zero(dk);
    zero(dv);
    // G K: A(t, s) = G[t * LVt + s], B(s, n) = K[s * LQt + n].
    mma_quad<4, LVt, 1, LQt, BF>(dq, gm, 16 * wr, kt, 64 * wc, 0, 16 * (wr + 1));
    if constexpr (BF) {
      // G^T Q: A(s, t) = Gt[s * LVt + t], B(t, n) = Q[t * LQt + n].
      mma_quad<4, LVt, 1, LQt, BF>(dk, gmt, 16 * wr, qt, 64 * wc, 16 * wr, C);
      // (S o W)^T dY: A(s, t) = (S o W)t[s * LVt + t], B(t, p) = dYt[p * LVt + t].
      mma<2, LVt, 1, 1, LVt, BF>(dv, gs, 16 * wr, dyT, 32 * wc, 16 * wr, C);
    } else {
      // G^T Q: A(s, t) = G[t * LV + s], B(t, n) = Q[t * LQ + n].
      mma_quad<4, 1, LV, LQ, BF>(dk, gm, 16 * wr, qt, 64 * wc, 16 * wr, C);
      // (S o W)^T dY.
      mma<2, 1, LV, LV, 1, BF>(dv, gs, 16 * wr, dyt, 32 * wc, 16 * wr, C);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * wr + 4 * q + i, p = 32 * wc + 16 * j + r, tt = c * C + t;
        if (tt < s.T && p < s.P)
          st1(dx + (tok_index(s, b, tt) * s.H + h) * s.P + p, dv[j][i] + S.u[t] * kg[j][i]);
      }
    __syncthreads();  // Q, K, S o W and G are no longer read
    // dY is scaled by e^p before its product (the reference rounds the scaled
    // cotangent, :740); V's factor u is applied to the product's rows after
    // it with bfloat16 operands (the reference scales v dH1^T, :749-750),
    // before it in float32, where the two agree.
#pragma unroll
    for (int i = 0; i < C * PT / 2048; ++i) {
      const int e = tid + 512 * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
      put4(dyt + t * LVt + p, get4(dyt + t * LVt + p) * S.ep[t]);
      if constexpr (!BF) put4(vt + t * LVt + p, get4(vt + t * LVt + p) * S.u[t]);
    }
    TT* const h0b = BF ? h0 : reinterpret_cast<TT*>(R1);
    if constexpr (!BF) {
      store_state_t<512, LQt>(F.hs, h0b);
      store_state_t<512, LQt>(F.hg, h0b + PT * LQt);
    }
    __syncthreads();
    // Every register of F is staged: the next head's inputs load during this
    // head's remaining phases (which wait for no global load).  The two waves
    // on a SIMD issue them before and after their first product, so one
    // wave's products run while the other waits to issue its loads.
    if (wc == 0 && h + 1 < h_end) fetch_head(F, h + 1);
    // diag(e^p) dY H0^T: A(t, p) = dYe[t * LVt + p], B(p, n) = H0t[p * LQt + n].
    mma_quad<4, LVt, 1, LQt, BF>(dq, dyt, 16 * wr, h0b, 64 * wc, 0, PT);
    if (wc == 1 && h + 1 < h_end) fetch_head(F, h + 1);
    if constexpr (BF) {
      f4 vd[4];
      zero(vd);
      mma_quad<4, LVt, 1, LQt, BF>(vd, vt, 16 * wr, h0b + PT * LQt, 64 * wc, 0, PT);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) dk[j][i] += S.u[16 * wr + 4 * q + i] * vd[j][i];
    } else {
      mma_quad<4, LVt, 1, LQt>(dk, vt, 16 * wr, h0b + PT * LQt, 64 * wc, 0, PT);
    }
    __syncthreads();
    float* dqt = R1;
    float* dkt = R1 + C * LQ;
    // mma_quad's layout: a lane's four accumulators are columns
    // 64 wc + 4 r .. +3 of its rows, one 16-byte store per row.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wr + 4 * q + i, n = 64 * wc + 4 * r;
      *reinterpret_cast<f4*>(dqt + t * LQ + n) = f4{dq[0][i], dq[1][i], dq[2][i], dq[3][i]};
      *reinterpret_cast<f4*>(dkt + t * LQ + n) = f4{dk[0][i], dk[1][i], dk[2][i], dk[3][i]};
    }
    __syncthreads();

    // Through the rotations: one pair per lane, tokens w, w + 8, ...
    {
      const bool col = n2 < s.N;
      float2 sq = float2{0.f, 0.f}, sk = float2{0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int t = w + 8 * m, tt = c * C + t;
        if (!col || tt >= s.T) continue;
        const float2 gq = *reinterpret_cast<const float2*>(dqt + t * LQ + n2);
        const float2 gk = *reinterpret_cast<const float2*>(dkt + t * LQ + n2);
        float2 duq = gq, duk = gk;
        if (l < s.A) {
          float sn, cs;
          sin_cos(tab[t * LA + l], &sn, &cs);
          const float2 cm = dec(rc[m]), bm = dec(rb[m]);
          const float2 uq = round_bf2<BF>(float2{cm.x + bq.x, cm.y + bq.y});
          const float2 uk = round_bf2<BF>(float2{bm.x + bkv.x, bm.y + bkv.y});
          const float q0 = uq.x * cs - uq.y * sn, q1 = uq.x * sn + uq.y * cs;
          const float k0 = uk.x * cs - uk.y * sn, k1 = uk.x * sn + uk.y * cs;
          tab[t * LA + l] = gq.y * q0 - gq.x * q1 + gk.y * k0 - gk.x * k1;
          duq = float2{gq.x * cs + gq.y * sn, -gq.x * sn + gq.y * cs};
          duk = float2{gk.x * cs + gk.y * sn, -gk.x * sn + gk.y * cs};
        }
        dcacc[m].x += duq.x;
        dcacc[m].y += duq.y;
        dbacc[m].x += duk.x;
        dbacc[m].y += duk.y;
        sq.x += duq.x;
        sq.y += duq.y;
        sk.x += duk.x;
        sk.y += duk.y;
      }
      *reinterpret_cast<float2*>(qbp + w * NT + n2) = sq;
      *reinterpret_cast<float2*>(kbp + w * NT + n2) = sk;
    }
    __syncthreads();
    // Phase gradients summed from the chunk's end (one token per lane).
    {
      const int tt = c * C + l;
      const bool valid = tt < s.T;
      float ddt = 0.f;
      const float(&av)[8] = rates;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int j = w + 8 * m;
        if (j >= s.A) break;
        const float xv = valid ? tab[l * LA + j] : 0.f;
        const float incl = wave_scan(xv), tot = lane63(incl);
        const float R = tot - incl + xv;
        dang[m] += R * S.dt[l];
        ddt += R * av[m];
        if (l == 0) o.D[phase_offset(s, b, h, c) + j] = R;
      }
      ddtp[w * 64 + l] = ddt;
    }
    if (tid < NT) {
      const long at = (((long)b * s.NC + c) * s.H + h) * NT + tid;
      float aq = 0.f, ak = 0.f;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        aq += qbp[v * NT + tid];
        ak += kbp[v * NT + tid];
      }
      o.qb_part[at] = aq;
      o.kb_part[at] = ak;
    }
    __syncthreads();
    if (w == 0) {
      const int tt = c * C + l;
      const float pl = S.p[63];
      const float qd = s_qd[l] + s_qd[64 + l], gl = s_g[l] + s_g[64 + l];
      const float rowE = s_rowE[l] + s_rowE[64 + l];
      float colF = 0.f, colE = 0.f, hs = 0.f, ddt = 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        colF += s_colF[64 * v + l];
        colE += s_colE[64 * v + l];
      }
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        hs += hsum[v];
        ddt += ddtp[v * 64 + l];
      }
      const float ug = wave_sum(S.u[l] * gl);
      float dp = rowE - colE + S.ep[l] * qd - S.u[l] * gl;
      if (l == 63) dp += ug + expf(pl) * hs;
      const float dscale = colF + expf(pl - S.p[l]) * gl;
      const float incl = wave_scan(dp), tot = lane63(incl);
      const float dadt = tot - incl + dp;
      if (tt < s.T) {
        const long i = tok_index(s, b, tt) * s.H + h;
        o.d_adt[i] = dadt;
        o.dgam[i] = s_dgd[l] + dscale;
        o.dscale[i] = dscale;
        o.ddt_loc[i] = ddt;
      }
    }
  }

  // The group's sums, written once.
  {
    const int tid = tix(), w = tid >> 6, l = tid & 63;
    const long tp = (long)s.NC * C;
    float* dcp = o.dc_part + ((long)g * s.B + b) * tp * NT;
    float* dbp = o.db_part + ((long)g * s.B + b) * tp * NT;
    float* dap = o.dang_part + ((long)g * s.B + b) * tp * AM;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const long at = (long)(c * C + w + 8 * m) * NT + 2 * l;
      *reinterpret_cast<float2*>(dcp + at) = dcacc[m];
      *reinterpret_cast<float2*>(dbp + at) = dbacc[m];
      dap[(long)(c * C + l) * AM + w + 8 * m] = dang[m];
    }
  }
}

// ---------------------------------------------------------------------------
// Per (b, chunk, quarter of its tokens): phase gradients carried from later
// chunks, the group sums, and the dt / trap gradients (gamma = dt sigma,
// prev = dt (1 - sigma); scale_t = gamma_t + prev_{t+1}, so
// d prev_t = d scale_{t-1}).
__global__ __launch_bounds__(256) void finish_kernel(Shape s, int groups, const float* dt,
                                                     const float* trap, const float* ang,
                                                     GradOut o, float* d_c, float* d_b,
                                                     float* d_dt, float* d_trap,
                                                     float* d_angles) {
  extern __shared__ float sm[];
  float* suf = sm;                    // [H][LA] phase gradient from later chunks
  float* angs = suf + s.H * LA;       // [C][A + 1] the chunk's angle rates
  float* dts = angs + C * (s.A + 1);  // [C][H + 1] the chunk's dt
  // kFinishParts blocks per (b, chunk), each taking C / kFinishParts of its
  // tokens.
  constexpr int TPB = C / kFinishParts;
  const int part = blockIdx.x % kFinishParts, bc = blockIdx.x / kFinishParts;
  const int b = bc / s.NC, c = bc % s.NC, tid = tix();
  const int t0 = TPB * part, rows = max(0, min(TPB, s.T - c * C - t0));
  const long tp = (long)s.NC * C;
  // The row gradients first: their group sums read no LDS, so their loads
  // are in flight with the staging loads below.  A thread's K elements load
  // together for each group (buffer loads, out of range past the rows), so a
  // group costs one round trip rather than one per element.
  {
    constexpr int K = TPB * NT / 256;
    float ac[K], ab[K];
    unsigned off[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = tid + 256 * k, t = t0 + e / s.N, n = e % s.N;
      off[k] = e < rows * s.N ? (unsigned)((c * C + t) * NT + n) * 4 : kNoLoad;
      ac[k] = ab[k] = 0.f;
    }
    for (int g = 0; g < groups; ++g) {
      const long slab = ((long)g * s.B + b) * tp * NT;
      const Rsrc rc = rsrc(o.dc_part + slab, tp * NT * 4), rb = rsrc(o.db_part + slab, tp * NT * 4);
      float xc[K], xb[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        xc[k] = ldb(rc, off[k]);
        xb[k] = ldb(rb, off[k]);
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        ac[k] += xc[k];
        ab[k] += xb[k];
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = tid + 256 * k, t = t0 + e / s.N, n = e % s.N, tt = c * C + t;
      if (e < rows * s.N) {
        d_c[tok_index(s, b, tt) * s.N + n] = ac[k];
        d_b[tok_index(s, b, tt) * s.N + n] = ab[k];
      }
    }
  }
  // The block's angle rates and dt rows (contiguous: rows x A, rows x H
  // from token t0), and the later chunks' phase gradients of every head:
  // each set's loads issued together before its LDS stores.
  {
    const long tok = tok_index(s, b, c * C + t0);
    const Rsrc ra = rsrc(ang + tok * s.A, (long)rows * s.A * 4);
    const Rsrc rd = rsrc(dt + tok * s.H, (long)rows * s.H * 4);
    constexpr int KA = TPB * AM / 256, KH = TPB * kMaxHeads / 256;
    float xa[KA], xd[KH];
#pragma unroll
    for (int k = 0; k < KA; ++k) xa[k] = ldb(ra, (tid + 256 * k) * 4);
#pragma unroll
    for (int k = 0; k < KH; ++k) xd[k] = ldb(rd, (tid + 256 * k) * 4);
#pragma unroll
    for (int k = 0; k < KA; ++k) {
      const int e = tid + 256 * k;
      if (e < rows * s.A) angs[(t0 + e / s.A) * (s.A + 1) + e % s.A] = xa[k];
    }
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const int e = tid + 256 * k;
      if (e < rows * s.H) dts[(t0 + e / s.H) * (s.H + 1) + e % s.H] = xd[k];
    }
    for (int e0 = 0; e0 < s.H * s.A; e0 += 1024) {
      float xs[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int e = e0 + tid + 256 * k;
        xs[k] = e < s.H * s.A ? o.D[phase_offset(s, b, e / s.A, c) + e % s.A] : 0.f;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int e = e0 + tid + 256 * k;
        if (e < s.H * s.A) suf[(e / s.A) * LA + e % s.A] = xs[k];
      }
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int e = tid; e < rows * s.H; e += 256) {
    const int t = t0 + e / s.H, h = e % s.H, tt = c * C + t;
    const long i = tok_index(s, b, tt) * s.H + h;
    const float d = dts[t * (s.H + 1) + h], sig = 1.f / (1.f + expf(-trap[i]));
    const float dg = o.dgam[i], dprev = tt > 0 ? o.dscale[i - s.H] : 0.f;
    float carried = 0.f;
    for (int j = 0; j < s.A; ++j) carried += suf[h * LA + j] * angs[t * (s.A + 1) + j];
    d_dt[i] = dg * sig + dprev * (1.f - sig) + o.ddt_loc[i] + carried;
    d_trap[i] = (dg - dprev) * d * sig * (1.f - sig);
  }
  {
    // The angle gradients: the group sums' loads of a thread's elements
    // issued together per group (out of range past the rows).
    constexpr int KA = TPB * AM / 256;
    float acc[KA];
    unsigned off[KA];
#pragma unroll
    for (int k = 0; k < KA; ++k) {
      const int e = tid + 256 * k, t = t0 + e / max(s.A, 1), j = e % max(s.A, 1);
      off[k] = e < rows * s.A ? (unsigned)((c * C + t) * AM + j) * 4 : kNoLoad;
      acc[k] = 0.f;
    }
    for (int g = 0; g < groups; ++g) {
      const Rsrc rg = rsrc(o.dang_part + ((long)g * s.B + b) * tp * AM, tp * AM * 4);
      float x[KA];
#pragma unroll
      for (int k = 0; k < KA; ++k) x[k] = ldb(rg, off[k]);
#pragma unroll
      for (int k = 0; k < KA; ++k) acc[k] += x[k];
    }
#pragma unroll
    for (int k = 0; k < KA; ++k) {
      const int e = tid + 256 * k;
      if (e < rows * s.A) {
        const int t = t0 + e / s.A, j = e % s.A, tt = c * C + t;
        float a = acc[k];
        for (int h = 0; h < s.H; ++h) a += suf[h * LA + j] * dts[t * (s.H + 1) + h];
        d_angles[tok_index(s, b, tt) * s.A + j] = a;
      }
    }
  }
}

// Phase-gradient totals of the chunks after each chunk: o.D[b,h,c,j] becomes
// sum_{c' > c} D[b,h,c',j], a reverse exclusive scan over the chunks with one
// thread per (b, h, j), so finish_kernel reads one row per chunk.
__global__ __launch_bounds__(256) void suffix_kernel(Shape s, GradOut o) {
  const long id = (long)blockIdx.x * 256 + tix();
  if (id >= (long)s.B * s.H * s.A) return;
  const int j = (int)(id % s.A);
  const long bh = id / s.A;
  float* d = o.D + bh * s.NC * AM + j;
  float acc = 0.f;
  // Eight chunks' totals are read before any is overwritten, so their loads
  // are in flight together.
  for (int c1 = s.NC; c1 > 0; c1 -= 8) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = c1 - 1 - i >= 0 ? d[(long)(c1 - 1 - i) * AM] : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (c1 - 1 - i >= 0) d[(long)(c1 - 1 - i) * AM] = acc;
      acc += v[i];
    }
  }
}

// Bias gradients: sums over (b, chunk) of the per-head partials; eight
// threads per coordinate take every eighth (b, chunk) and combine in LDS.
__global__ __launch_bounds__(1024) void bias_kernel(Shape s, GradOut o, float* d_qb, float* d_kb) {
  // Block (h, 32 of the NT columns): 32 slices of the (b, chunk) partials
  // per column, each slice's loads issued eight at a time, then the slices
  // added in a fixed order.
  __shared__ float part[2][32][33];
  const int h = blockIdx.x / (NT / 32), n0 = 32 * (blockIdx.x % (NT / 32));
  const int col = tix() & 31, slice = tix() >> 5, n = n0 + col;
  const int total = s.B * s.NC;
  float aq = 0.f, ak = 0.f;
  for (int bc0 = slice; bc0 < total; bc0 += 32 * 8) {
    float q8[8], k8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int bc = bc0 + 32 * i;
      const long at = ((long)min(bc, total - 1) * s.H + h) * NT + n;
      q8[i] = bc < total ? o.qb_part[at] : 0.f;
      k8[i] = bc < total ? o.kb_part[at] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      aq += q8[i];
      ak += k8[i];
    }
  }
  part[0][slice][col] = aq;
  part[1][slice][col] = ak;
  __syncthreads();
  if (slice == 0 && n < s.N) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      sq += part[0][i][col];
      sk += part[1][i][col];
    }
    d_qb[(long)h * s.N + n] = sq;
    d_kb[(long)h * s.N + n] = sk;
  }
}

#define M3_SCAN_KERNELS(In, V4)                                                                \
  template __global__ void walk_kernel<false, In, V4>(Shape, const In*, const float*, const In*, \
                                                      const float*, const float*, const float*,  \
                                                      const float*, float*, float*,              \
                                                      const float*, float*);                     \
  template __global__ void walk_kernel<true, In, V4>(Shape, const In*, const float*, const In*,  \
                                                     const float*, const float*, const float*,   \
                                                     const float*, float*, float*, const float*, \
                                                     float*);                                    \
  template __global__ void out_kernel<In, V4>(Shape, const In*, const In*, const In*,            \
                                              const float*, const float*, const float*,          \
                                              const float*, const float*, const float*,          \
                                              const float*, const float*, In*);                  \
  template __global__ void grad_kernel<In, V4>(Shape, int, const In*, const In*, const In*,      \
                                               const float*, const float*, const float*,         \
                                               const float*, const float*, const float*,         \
                                               const float*, const float*, const float*,         \
                                               const In*, GradOut);
M3_SCAN_KERNELS(float, true)
M3_SCAN_KERNELS(float, false)
M3_SCAN_KERNELS(bf16_t, true)
M3_SCAN_KERNELS(bf16_t, false)
#undef M3_SCAN_KERNELS

}  // namespace m3
