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
__device__ __forceinline__ float2 ld2(const float* p) {
  return *reinterpret_cast<const float2*>(p);
}
__device__ __forceinline__ float2 ld2(const bf16_t* p) {
  const unsigned u = *reinterpret_cast<const unsigned*>(p);
  return float2{lo_bf(u), hi_bf(u)};
}
__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f4 ld4(const bf16_t* p) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  return f4{lo_bf(u.x), hi_bf(u.x), lo_bf(u.y), hi_bf(u.y)};
}
__device__ __forceinline__ float ld1(const float* p) { return *p; }
__device__ __forceinline__ float ld1(const bf16_t* p) { return lo_bf(*p); }
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

// mma over the first jn (0..2, the same for the whole wave) of two column
// tiles, each count its own straight-line instantiation.
template <int AR, int AK, int BK, int BC, bool BF = false>
__device__ __forceinline__ void mma_first2(f4 (&acc)[2], const float* A, int r0, const float* B,
                                           int c0, int kb, int ke, int jn) {
  if (jn >= 2) {
    mma<2, AR, AK, BK, BC, BF>(acc, A, r0, B, c0, kb, ke);
  } else if (jn == 1) {
    mma<1, AR, AK, BK, BC, BF>(*reinterpret_cast<f4(*)[1]>(acc), A, r0, B, c0, kb, ke);
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

__device__ __forceinline__ long tok_index(const Shape& s, int b, int t) {
  return (long)b * s.T + t;
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

__device__ __forceinline__ TokenIn fetch_token(const Shape& s, const float* adt, const float* dt,
                                               const float* trap, int b, int h, int c) {
  const int t = c * C + lane_id();
  const bool valid = t < s.T, next = t + 1 < s.T;
  const long i = tok_index(s, b, t) * s.H + h;
  return TokenIn{valid ? adt[i] : 0.f, valid ? dt[i] : 0.f, valid ? trap[i] : 0.f,
                 next ? dt[i + s.H] : 0.f, next ? trap[i + s.H] : 0.f};
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

__device__ void token_scalars(const Shape& s, const float* adt, const float* dt,
                              const float* trap, int b, int h, int c, const Scalars& o) {
  token_scalars(fetch_token(s, adt, dt, trap, b, h, c), o);
}

// Phase table of chunk c: tab[t * LA + j] = th0[j] + sum_{s <= t} angles_s,j dt_s
// (j < A), one token per lane, angles split over the four waves.  With
// `advance`, th0[j] moves to the chunk's end phase reduced modulo 2 pi (th0
// lives in LDS and each j belongs to one wave, whose lanes read it before
// lane 63 writes it).
// This lane's token's angle rates j = w + NW m (zeros past T and A), for a
// block of NW waves.
template <int NW = 4>
__device__ __forceinline__ void fetch_angles(const Shape& s, const float* ang, int b, int c,
                                             float (&xs)[64 / NW]) {
  const int w = tix() >> 6, t = c * C + lane_id();
  const bool valid = t < s.T;
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) {
    const int j = w + NW * m;
    xs[m] = valid && j < s.A ? ang[tok_index(s, b, t) * s.A + j] : 0.f;
  }
}

// The phase table from fetched angle rates and this lane's dt.
template <int NW = 4>
__device__ void phase_table(const Shape& s, const float (&rates)[64 / NW], float d, float* th0,
                            float* tab, bool advance) {
  const int l = lane_id(), w = tix() >> 6;
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

template <int NW = 4>
__device__ void phase_table(const Shape& s, const float* ang, const float* dt, int b, int h,
                            int c, float* th0, float* tab, bool advance) {
  const int t = c * C + lane_id();
  const float d = t < s.T ? dt[tok_index(s, b, t) * s.H + h] : 0.f;
  float rates[64 / NW];
  fetch_angles<NW>(s, ang, b, c, rates);
  phase_table<NW>(s, rates, d, th0, tab, advance);
}

// Rotated rows of chunk c into LDS [C][LQ]: dst[t][n] = rot(src_t + bias, theta_t)[n]
// for t < C, n < NT, zero for padding tokens and coordinates.  One pair
// (2j, 2j+1) per lane, tokens w, w + 4, ... per wave; every global read is
// issued before the first rotation.  With two sources both are rotated by
// the same angles.  bfloat16 sources: the bias-added rows are rounded to
// bfloat16 before the rotation (_rotated, lm/kernels/flashmamba.py:582-585).
template <int NSRC, int NW = 4, typename In = float>
__device__ __forceinline__ void fetch_rows(const Shape& s, const In* const (&src)[2],
                                           const float* const (&bias)[2], int b, int c,
                                           float2 (&u)[NSRC][64 / NW], float2 (&bs)[NSRC]) {
  const int j = lane_id(), n = 2 * j, w = tix() >> 6;
  const bool col = n < s.N;
#pragma unroll
  for (int m = 0; m < 64 / NW; ++m) {
    const int tt = c * C + w + NW * m;
    const bool valid = col && tt < s.T;
#pragma unroll
    for (int k = 0; k < NSRC; ++k)
      u[k][m] = valid ? ld2(src[k] + tok_index(s, b, tt) * s.N + n) : float2{0.f, 0.f};
  }
#pragma unroll
  for (int k = 0; k < NSRC; ++k)
    bs[k] = col ? *reinterpret_cast<const float2*>(bias[k] + n) : float2{0.f, 0.f};
}

template <int NSRC, int NW = 4, bool BF = false>
__device__ __forceinline__ void rotate_fetched(const Shape& s, const float2 (&u)[NSRC][64 / NW],
                                               const float2 (&bs)[NSRC], float* const (&dst)[2],
                                               const float* tab, int c) {
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
      const float2 v = round_bf2<BF>(
          valid ? float2{u[k][m].x + bs[k].x, u[k][m].y + bs[k].y} : float2{0.f, 0.f});
      *reinterpret_cast<float2*>(dst[k] + t * LQ + n) =
          float2{v.x * cs - v.y * sn, v.x * sn + v.y * cs};
    }
  }
}

template <int NSRC, int NW = 4, typename In = float>
__device__ void rotate_rows(const Shape& s, const In* const (&src)[2],
                            const float* const (&bias)[2], float* const (&dst)[2], const float* tab,
                            int b, int c) {
  float2 u[NSRC][64 / NW], bs[NSRC];
  fetch_rows<NSRC, NW>(s, src, bias, b, c, u, bs);
  rotate_fetched<NSRC, NW, is_bf16<In>::value>(s, u, bs, dst, tab, c);
}

// Value rows of head h for chunk c into LDS [C][LV], each row t scaled by
// row_scale[t] (nullptr: 1); zeros past T and P.  Four 16-byte rows pieces
// per thread, all read before any is stored (fetch_values, store_values).
template <int NTH = 256, typename In = float>
__device__ __forceinline__ void fetch_values(const Shape& s, const In* src, int b, int c, int h,
                                             f4 (&v)[1024 / NTH]) {
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    const int e = tix() + NTH * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
    const int tt = c * C + t;
    v[i] = f4{0.f, 0.f, 0.f, 0.f};
    if (tt < s.T) {
      const In* row = src + (tok_index(s, b, tt) * s.H + h) * s.P;
      if (s.P % 4 == 0) {
        if (p < s.P) v[i] = ld4(row + p);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (p + k < s.P) v[i][k] = ld1(row + p + k);
      }
    }
  }
}

template <int NTH = 256>
__device__ __forceinline__ void store_values(const f4 (&v)[1024 / NTH], const float* row_scale,
                                             float* dst) {
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    const int e = tix() + NTH * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
    *reinterpret_cast<f4*>(dst + t * LV + p) = row_scale ? v[i] * row_scale[t] : v[i];
  }
}

template <int NTH = 256, typename In = float>
__device__ void load_values(const Shape& s, const In* src, int b, int c, int h,
                            const float* row_scale, float* dst) {
  f4 v[1024 / NTH];
  fetch_values<NTH>(s, src, b, c, h, v);
  store_values<NTH>(v, row_scale, dst);
}

// Value rows of head h for chunk c into LDS transposed, [PT][LV]: thread e
// takes token t = e % C (consecutive lanes, conflict-free LDS stores) and
// columns 4 (e / C) .. +3; zeros past T and P.  fetch_values_t reads this
// thread's pieces into registers, store_values_t writes them.
template <int NTH = 256, typename In = float>
__device__ __forceinline__ void fetch_values_t(const Shape& s, const In* src, int b, int c,
                                               int h, f4 (&v)[1024 / NTH]) {
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    const int e = tix() + NTH * i, t = e % C, p = 4 * (e / C), tt = c * C + t;
    v[i] = f4{0.f, 0.f, 0.f, 0.f};
    if (tt < s.T) {
      const In* row = src + (tok_index(s, b, tt) * s.H + h) * s.P;
      if (s.P % 4 == 0) {
        if (p < s.P) v[i] = ld4(row + p);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (p + k < s.P) v[i][k] = ld1(row + p + k);
      }
    }
  }
}

template <int NTH = 256>
__device__ __forceinline__ void store_values_t(const f4 (&v)[1024 / NTH], float* dst) {
#pragma unroll
  for (int i = 0; i < 1024 / NTH; ++i) {
    const int e = tix() + NTH * i, t = e % C, p = 4 * (e / C);
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[(p + k) * LV + t] = v[i][k];
  }
}

template <int NTH = 256, typename In = float>
__device__ void load_values_t(const Shape& s, const In* src, int b, int c, int h,
                              float* dst) {
  f4 v[1024 / NTH];
  fetch_values_t<NTH>(s, src, b, c, h, v);
  store_values_t<NTH>(v, dst);
}

// A stored [NT][PT] state tile into LDS transposed, [PT][LQ]: thread e takes
// row n = e % NT (consecutive lanes, conflict-free LDS stores) and columns
// 4 (e / NT) .. +3, all read before any is stored.
template <int NTH = 256>
__device__ __forceinline__ void fetch_state_t(const float* src, f4 (&v)[2048 / NTH]) {
#pragma unroll
  for (int i = 0; i < 2048 / NTH; ++i) {
    const int e = tix() + NTH * i;
    v[i] = *reinterpret_cast<const f4*>(src + (e % NT) * PT + 4 * (e / NT));
  }
}

template <int NTH = 256>
__device__ __forceinline__ void store_state_t(const f4 (&v)[2048 / NTH], float* dst) {
#pragma unroll
  for (int i = 0; i < 2048 / NTH; ++i) {
    const int e = tix() + NTH * i, n = e % NT, p = 4 * (e / NT);
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[(p + k) * LQ + n] = v[i][k];
  }
}

// The same registers (row n = e % NT, columns 4 (e / NT) .. +3) into the
// untransposed [NT][LV] layout: one 16-byte store each.
template <int NTH = 256>
__device__ __forceinline__ void store_state_rows(const f4 (&v)[2048 / NTH], float* dst) {
#pragma unroll
  for (int i = 0; i < 2048 / NTH; ++i) {
    const int e = tix() + NTH * i, n = e % NT, p = 4 * (e / NT);
    *reinterpret_cast<f4*>(dst + n * LV + p) = v[i];
  }
}

template <int NTH = 256>
__device__ void load_state_t(const float* src, float* dst) {
  f4 v[2048 / NTH];
  fetch_state_t<NTH>(src, v);
  store_state_t<NTH>(v, dst);
}

__device__ __forceinline__ long state_offset(const Shape& s, int b, int h, int c) {
  return (((long)b * s.H + h) * s.NC + c) * (long)(NT * PT);
}
__device__ __forceinline__ long phase_offset(const Shape& s, int b, int h, int c) {
  return (((long)b * s.H + h) * s.NC + c) * (long)AM;
}

// ---------------------------------------------------------------------------
// State walks.  Forward (BWD = false): rows = keys b with k_bias, vals = x
// scaled by u; S starts at zero; each chunk stores its start state to
// `saved`, its start phase to theta0, then S <- e^{p_L} S + K^T (u v).
// Backward (BWD = true): rows = queries c with q_bias, vals = d_y scaled by
// e^p; S starts at d_final and the chunks run in reverse; each stores S (the
// cotangent of the state at the chunk's end) to `saved`, then
// S <- e^{p_L} S + Q^T (e^p dy).
// LDS: rows [C][LQ], vals [C][LV], phase table [C][LA], th0 [AM], scalars.
template <bool BWD, typename In>
__global__ __launch_bounds__(512) void walk_kernel(Shape s, const In* rows, const float* bias,
                                                   const In* vals, const float* adt,
                                                   const float* dt, const float* trap,
                                                   const float* ang, float* theta0, float* saved,
                                                   const float* init, float* final_state) {
  constexpr bool BF = is_bf16<In>::value;
  extern __shared__ float sm[];
  float* rt = sm;
  float* vt = rt + C * LQ;
  float* tab = vt + C * LV;
  float* th0 = tab + C * LA;
  float* sc = th0 + AM;
  const Scalars S{sc, sc + 64, sc + 128, sc + 192, sc + 256, sc + 320};
  const int bh = blockIdx.x, b = bh / s.H, h = bh % s.H;
  const int tid = tix(), w = tid >> 6, l = lane_id(), r = l & 15, q = l >> 4;

  // Eight waves: wave w holds state rows 16 w .. 16 w + 15 as four 16-column
  // tiles.
  f4 acc[1][4];
#pragma unroll
  for (int rt2 = 0; rt2 < 1; ++rt2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * w + 4 * q + i, p = 16 * j + r;
        float v = 0.f;
        if (BWD && init && n < s.N && p < s.P) v = init[(((long)b * s.H + h) * s.N + n) * s.P + p];
        acc[rt2][j][i] = v;
      }
    }
  }
  if (!BWD && tid < AM) th0[tid] = 0.f;
  const bool col = 2 * l < s.N;
  const float2 bs = col ? *reinterpret_cast<const float2*>(bias + (long)h * s.N + 2 * l)
                        : float2{0.f, 0.f};

  // Every global input of a chunk is fetched into registers one chunk ahead,
  // while the previous chunk's product runs.
  TokenIn tin;
  float rates[8], th_in = 0.f;
  float2 u[8];
  f4 v[2];
  auto fetch = [&](int c) {
    tin = fetch_token(s, adt, dt, trap, b, h, c);
    fetch_angles<8>(s, ang, b, c, rates);
    if (BWD && tid < s.A) th_in = theta0[phase_offset(s, b, h, c) + tid];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int tt = c * C + w + 8 * m;
      u[m] = col && tt < s.T ? ld2(rows + tok_index(s, b, tt) * s.N + 2 * l) : float2{0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 512 * i, t = e / (PT / 4), p = 4 * (e % (PT / 4)), tt = c * C + t;
      v[i] = f4{0.f, 0.f, 0.f, 0.f};
      if (tt < s.T) {
        const In* row = vals + (tok_index(s, b, tt) * s.H + h) * s.P;
        if (s.P % 4 == 0) {
          if (p < s.P) v[i] = ld4(row + p);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k)
            if (p + k < s.P) v[i][k] = ld1(row + p + k);
        }
      }
    }
  };
  fetch(BWD ? s.NC - 1 : 0);

  for (int step = 0; step < s.NC; ++step) {
    const int c = BWD ? s.NC - 1 - step : step;
    __syncthreads();  // the previous chunk's reads of the LDS tiles are done
    if (w == 0) token_scalars(tin, S);
    if (BWD) {
      if (tid < s.A) th0[tid] = th_in;
    } else {
      if (tid < s.A) theta0[phase_offset(s, b, h, c) + tid] = th0[tid];
    }
    __syncthreads();
    phase_table<8>(s, rates, tin.d, th0, tab, !BWD);
    __syncthreads();
    // Rotated rows (one pair per lane) and scaled values into LDS.
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int t = w + 8 * m, tt = c * C + t;
      const bool valid = col && tt < s.T;
      float sn = 0.f, cs = 1.f;
      if (valid && l < s.A) sin_cos(tab[t * LA + l], &sn, &cs);
      // The bias-added row in the model dtype, then rotated in float32 (:582-585).
      const float2 x2 = round_bf2<BF>(valid ? float2{u[m].x + bs.x, u[m].y + bs.y}
                                            : float2{0.f, 0.f});
      *reinterpret_cast<float2*>(rt + t * LQ + 2 * l) =
          float2{x2.x * cs - x2.y * sn, x2.x * sn + x2.y * cs};
    }
    const float* row_scale = BWD ? S.ep : S.u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 512 * i, t = e / (PT / 4), p = 4 * (e % (PT / 4));
      *reinterpret_cast<f4*>(vt + t * LV + p) = v[i] * row_scale[t];
    }
    // Store this chunk's state (a lane's four rows of one column).
    float* out = saved + state_offset(s, b, h, c);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) out[(16 * w + 4 * q + i) * PT + 16 * j + r] = acc[0][j][i];
    if (step + 1 < s.NC) fetch(BWD ? c - 1 : c + 1);
    __syncthreads();
    const float decay = expf(S.p[63]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[0][j] *= decay;
    // rows^T vals: A(n, t) = rt[t * LQ + n], B(t, p) = vt[t * LV + p].
    mma<4, 1, LQ, LV, 1, BF>(acc[0], rt, 16 * w, vt, 0, 0, C);
  }
  if (!BWD && final_state) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int n = 16 * w + 4 * q + i, p = 16 * j + r;
        if (n < s.N && p < s.P)
          final_state[(((long)b * s.H + h) * s.N + n) * s.P + p] = acc[0][j][i];
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
// LDS: Q [C][LQ], K [C][LQ] (later S o W as [C][LV]), H0 transposed
// [PT][LQ] (first the phase table), V transposed [PT][LV], scalars.
template <typename In>
__global__ __launch_bounds__(512) void out_kernel(Shape s, const In* cq, const In* bk,
                                                  const In* x, const float* adt,
                                                  const float* dt, const float* trap,
                                                  const float* ang, const float* qb,
                                                  const float* kb, const float* theta0,
                                                  const float* starts, In* y) {
  constexpr bool BF = is_bf16<In>::value;
  extern __shared__ float sm[];
  float* qt = sm;
  float* kt = qt + C * LQ;
  float* h0 = kt + C * LQ;
  float* tab = h0;
  float* vt = h0 + NT * LV;
  float* th0 = vt + C * LV;
  float* sc = th0 + AM;
  const Scalars S{sc, sc + 64, sc + 128, sc + 192, sc + 256, sc + 320};
  const int total = s.B * s.NC * s.H;
  const In* const src[2] = {cq, bk};

  // Every global input of an item, fetched into registers while the
  // previous item's products run.
  struct Fetched {
    TokenIn tin;
    float th, rates[8];
    float2 u[2][8], bs[2];
    f4 hv[4], vv[2];
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
    const int tid = tix();
    F.th = tid < s.A ? theta0[phase_offset(s, b, h, c) + tid] : 0.f;
    fetch_angles<8>(s, ang, b, c, F.rates);
    const float* const bsrc[2] = {qb + (long)h * s.N, kb + (long)h * s.N};
    fetch_rows<2, 8>(s, src, bsrc, b, c, F.u, F.bs);
    fetch_state_t<512>(starts + state_offset(s, b, h, c), F.hv);
    fetch_values_t<512>(s, x, b, c, h, F.vv);
  };

  // Persistent: block i handles items i, i + gridDim.x, ... (b, chunk, h),
  // heads fastest, each XCD a contiguous run of (b, chunk) pairs.
  Fetched F;
  int it = blockIdx.x;
  if (it < total) fetch(F, it);
  for (; it < total; it += gridDim.x) {
    int b, c, h;
    item_of(it, b, c, h);
    // Eight waves: wave w owns row block wr = w & 3 and column half wc = w >> 2.
    const int tid = tix(), l = lane_id(), r = l & 15, q = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wr = w & 3, wc = w >> 2;

    if (w == 0) token_scalars(F.tin, S);
    if (tid < s.A) th0[tid] = F.th;
    __syncthreads();
    phase_table<8>(s, F.rates, F.tin.d, th0, tab, false);
    __syncthreads();
    {
      float* const dst[2] = {qt, kt};
      rotate_fetched<2, 8, BF>(s, F.u, F.bs, dst, tab, c);
    }
    __syncthreads();  // the phase table (in h0's space) is read
    // The start state and the values transposed ([PT][LQ], [PT][LV]), so that
    // every product reads both operands contiguously along k.
    store_state_t<512>(F.hv, h0);
    store_values_t<512>(F.vv, vt);
    __syncthreads();
    // The next item's inputs load while this one's products run (no global
    // load is waited for before the next item's staging).
    const int next = it + gridDim.x;
    fetch(F, next < total ? next : it);

    const int ns = min(2, max(0, wr + 1 - 2 * wc));
    f4 sco[2], qh[2];
    zero(sco);
    zero(qh);
    mma_first2<LQ, 1, 1, LQ, BF>(sco, qt, 16 * wr, kt, 32 * wc, 0, NT, ns);
    mma<2, LQ, 1, 1, LQ, BF>(qh, qt, 16 * wr, h0, 32 * wc, 0, NT);
    __syncthreads();  // every wave is done with K
    float* gs = kt;
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
        gs[t * LV + u] = sco[j][i] * wt;
      }
    }
    __syncthreads();  // a row block's S o W comes from both of its waves
    f4 acc[2];
    zero(acc);
    // B(s, p) = Vt[p * LV + s].
    mma<2, LV, 1, 1, LV, BF>(acc, gs, 16 * wr, vt, 32 * wc, 0, 16 * (wr + 1));
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
// LDS: R1 = 2 NT LV floats (Q, K; later H0, dH1; later dQ, dK), R2 = 2 NT LV
// floats (H0, dH1; later V, dY, S o W, G), phase table [C][LA], scalars.
template <typename In>
__global__ __launch_bounds__(512) void grad_kernel(Shape s, int groups, const In* cq,
                                                   const In* bk, const In* x,
                                                   const float* adt, const float* dt,
                                                   const float* trap, const float* ang,
                                                   const float* qb, const float* kb,
                                                   const float* theta0, const float* starts,
                                                   const float* dh1, const In* dy, GradOut o) {
  constexpr bool BF = is_bf16<In>::value;
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
  // Eight waves: wave w owns row block wr = w & 3 of every 64-row tile and
  // column half wc = w >> 2 of its columns.  This group's sums over its
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
  float2 rc[8], rb[8];
  float rates[8];
  fetch_angles<8>(s, ang, b, c, rates);
  {
    const int tid = tix(), l = tid & 63, w = tid >> 6;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int tt = c * C + w + 8 * m;
      const bool ok = 2 * l < s.N && tt < s.T;
      rc[m] = ok ? ld2(cq + tok_index(s, b, tt) * s.N + 2 * l) : float2{0.f, 0.f};
      rb[m] = ok ? ld2(bk + tok_index(s, b, tt) * s.N + 2 * l) : float2{0.f, 0.f};
    }
  }

  // A head's own inputs, fetched into registers while the previous head's
  // last phases run: its per-token scalars, start phase, start state and
  // end cotangent (in the transposed-staging layout; the same registers
  // later fill the untransposed copies, so the pair is read once) and
  // biases.  Its values and d_y load at the head's start, for its fourth
  // phase.
  struct HeadIn {
    TokenIn tin;
    float th;
    f4 hs[4], hg[4];
    float2 bq, bk;
  };
  auto fetch_head = [&](HeadIn& F, int h) {
    F.tin = fetch_token(s, adt, dt, trap, b, h, c);
    const int tid = tix(), n2 = 2 * (tid & 63);
    F.th = tid < s.A ? theta0[phase_offset(s, b, h, c) + tid] : 0.f;
    fetch_state_t<512>(starts + state_offset(s, b, h, c), F.hs);
    fetch_state_t<512>(dh1 + state_offset(s, b, h, c), F.hg);
    F.bq = F.bk = float2{0.f, 0.f};
    if (n2 < s.N) {
      F.bq = *reinterpret_cast<const float2*>(qb + (long)h * s.N + n2);
      F.bk = *reinterpret_cast<const float2*>(kb + (long)h * s.N + n2);
    }
  };
  HeadIn F;
  if (h_begin < h_end) fetch_head(F, h_begin);

  for (int h = h_begin; h < h_end; ++h) {
    const int tid = tix(), l = tid & 63, r = l & 15, q = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), wr = w & 3, wc = w >> 2;
    const int n2 = 2 * l;  // this lane's coordinate pair in the rotation passes
    __syncthreads();  // the previous head is done with every LDS array
    f4 vx[2], vd[2];
    fetch_values<512>(s, x, b, c, h, vx);
    fetch_values<512>(s, dy, b, c, h, vd);
    if (w == 0) token_scalars(F.tin, S);
    if (tid < s.A) th0[tid] = F.th;
    // Column sums: the row blocks above a column block contribute nothing.
    if (tid < 256) {
      s_colF[tid] = 0.f;
      s_colE[tid] = 0.f;
    }
    __syncthreads();
    phase_table<8>(s, rates, F.tin.d, th0, tab, false);
    __syncthreads();
    float* qt = R1;
    float* kt = R1 + C * LQ;
    // The start state and end cotangent transposed, [PT][LQ], for Q H0 and
    // K dH1 with both operands contiguous along n.
    float* h0 = R2;
    float* g1 = R2 + NT * LV;
    store_state_t<512>(F.hs, h0);
    store_state_t<512>(F.hg, g1);
    const float2 bq = F.bq, bkv = F.bk;
    {
      const bool col = n2 < s.N;
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int t = w + 8 * m, tt = c * C + t;
        const bool valid = col && tt < s.T;
        float sn = 0.f, cs = 1.f;
        if (valid && l < s.A) sin_cos(tab[t * LA + l], &sn, &cs);
        const float2 u = round_bf2<BF>(valid ? float2{rc[m].x + bq.x, rc[m].y + bq.y}
                                             : float2{0.f, 0.f});
        const float2 v = round_bf2<BF>(valid ? float2{rb[m].x + bkv.x, rb[m].y + bkv.y}
                                             : float2{0.f, 0.f});
        *reinterpret_cast<float2*>(qt + t * LQ + n2) =
            float2{u.x * cs - u.y * sn, u.x * sn + u.y * cs};
        *reinterpret_cast<float2*>(kt + t * LQ + n2) =
            float2{v.x * cs - v.y * sn, v.x * sn + v.y * cs};
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
    mma_first2<LQ, 1, 1, LQ, BF>(sco, qt, 16 * wr, kt, 32 * wc, 0, NT, ns);
    // B(n, p) = H0t[p * LQ + n].
    mma<2, LQ, 1, 1, LQ, BF>(qh, qt, 16 * wr, h0, 32 * wc, 0, NT);
    mma<2, LQ, 1, 1, LQ, BF>(kg, kt, 16 * wr, g1, 32 * wc, 0, NT);
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
    __syncthreads();
    float* vt = R2;
    float* dyt = R2 + C * LV;
    float* gs = R2 + 2 * C * LV;
    float* gm = R2 + 3 * C * LV;
    store_values<512>(vx, nullptr, vt);
    store_values<512>(vd, nullptr, dyt);
    __syncthreads();

    f4 dsc[2];
    zero(dsc);
    // dY V^T: A(t, p) = dY[t * LV + p], B(p, s) = V[s * LV + p].
    mma_first2<LV, 1, 1, LV, BF>(dsc, dyt, 16 * wr, vt, 32 * wc, 0, PT, ns);
    {
      float qd[4] = {0.f, 0.f, 0.f, 0.f}, gg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * wr + 4 * q + i, p = 32 * wc + 16 * j + r;
          qd[i] += qh[j][i] * dyt[t * LV + p];
          gg[i] += kg[j][i] * vt[t * LV + p];
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
            gs[t * LV + u] = 0.f;
            gm[t * LV + u] = 0.f;
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
          gs[t * LV + u] = st * wt;
          gm[t * LV + u] = ds * wt;
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
    // G K: A(t, s) = G[t * LV + s], B(s, n) = K[s * LQ + n].
    mma<4, LV, 1, LQ, 1, BF>(dq, gm, 16 * wr, kt, 64 * wc, 0, 16 * (wr + 1));
    // G^T Q: A(s, t) = G[t * LV + s], B(t, n) = Q[t * LQ + n].
    mma<4, 1, LV, LQ, 1, BF>(dk, gm, 16 * wr, qt, 64 * wc, 16 * wr, C);
    // (S o W)^T dY.
    mma<2, 1, LV, LV, 1, BF>(dv, gs, 16 * wr, dyt, 32 * wc, 16 * wr, C);
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
    for (int e = tid; e < C * PT; e += 512) {
      const int t = e / PT, p = e % PT;
      dyt[t * LV + p] *= S.ep[t];
      if (!BF) vt[t * LV + p] *= S.u[t];
    }
    store_state_rows<512>(F.hs, R1);
    store_state_rows<512>(F.hg, R1 + NT * LV);
    __syncthreads();
    // Every register of F is staged: the next head's inputs load during this
    // head's remaining phases (which wait for no global load).
    if (h + 1 < h_end) fetch_head(F, h + 1);
    // diag(e^p) dY H0^T: A(t, p) = dYe[t * LV + p], B(p, n) = H0[n * LV + p].
    mma<4, LV, 1, 1, LV, BF>(dq, dyt, 16 * wr, R1, 64 * wc, 0, PT);
    if constexpr (BF) {
      f4 vd[4];
      zero(vd);
      mma<4, LV, 1, 1, LV, BF>(vd, vt, 16 * wr, R1 + NT * LV, 64 * wc, 0, PT);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) dk[j][i] += S.u[16 * wr + 4 * q + i] * vd[j][i];
    } else {
      mma<4, LV, 1, 1, LV>(dk, vt, 16 * wr, R1 + NT * LV, 64 * wc, 0, PT);
    }
    __syncthreads();
    float* dqt = R1;
    float* dkt = R1 + C * LQ;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * wr + 4 * q + i, n = 64 * wc + 16 * j + r;
        dqt[t * LQ + n] = dq[j][i];
        dkt[t * LQ + n] = dk[j][i];
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
          const float2 uq = round_bf2<BF>(float2{rc[m].x + bq.x, rc[m].y + bq.y});
          const float2 uk = round_bf2<BF>(float2{rb[m].x + bkv.x, rb[m].y + bkv.y});
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
  float* suf = sm;                    // [H][AM] phase gradient from later chunks
  float* angs = suf + s.H * AM;       // [C][A + 1] the chunk's angle rates
  float* dts = angs + C * (s.A + 1);  // [C][H + 1] the chunk's dt
  // Four blocks per (b, chunk), each taking 16 of its tokens.
  const int part = blockIdx.x % 4, bc = blockIdx.x / 4;
  const int b = bc / s.NC, c = bc % s.NC, tid = tix();
  const int t0 = 16 * part, rows = max(0, min(16, s.T - c * C - t0));
  for (int e = tid; e < rows * s.A; e += 256) {
    const int t = t0 + e / s.A, j = e % s.A;
    angs[t * (s.A + 1) + j] = ang[tok_index(s, b, c * C + t) * s.A + j];
  }
  for (int e = tid; e < rows * s.H; e += 256) {
    const int t = t0 + e / s.H, h = e % s.H;
    dts[t * (s.H + 1) + h] = dt[tok_index(s, b, c * C + t) * s.H + h];
  }
  for (int e = tid; e < s.H * s.A; e += 256) {
    const int h = e / s.A, j = e % s.A;
    suf[h * AM + j] = o.D[phase_offset(s, b, h, c) + j];
  }
  __syncthreads();
  const long tp = (long)s.NC * C;
#pragma unroll 4
  for (int e = tid; e < rows * s.H; e += 256) {
    const int t = t0 + e / s.H, h = e % s.H, tt = c * C + t;
    const long i = tok_index(s, b, tt) * s.H + h;
    const float d = dts[t * (s.H + 1) + h], sig = 1.f / (1.f + expf(-trap[i]));
    const float dg = o.dgam[i], dprev = tt > 0 ? o.dscale[i - s.H] : 0.f;
    float carried = 0.f;
    for (int j = 0; j < s.A; ++j) carried += suf[h * AM + j] * angs[t * (s.A + 1) + j];
    d_dt[i] = dg * sig + dprev * (1.f - sig) + o.ddt_loc[i] + carried;
    d_trap[i] = (dg - dprev) * d * sig * (1.f - sig);
  }
#pragma unroll 4
  for (int e = tid; e < rows * s.A; e += 256) {
    const int t = t0 + e / s.A, j = e % s.A, tt = c * C + t;
    float acc = 0.f;
    for (int g = 0; g < groups; ++g) acc += o.dang_part[(((long)g * s.B + b) * tp + tt) * AM + j];
    for (int h = 0; h < s.H; ++h) acc += suf[h * AM + j] * dts[t * (s.H + 1) + h];
    d_angles[tok_index(s, b, tt) * s.A + j] = acc;
  }
#pragma unroll 8
  for (int e = tid; e < rows * s.N; e += 256) {
    const int t = t0 + e / s.N, n = e % s.N, tt = c * C + t;
    float ac = 0.f, ab = 0.f;
    for (int g = 0; g < groups; ++g) {
      const long at = (((long)g * s.B + b) * tp + tt) * NT + n;
      ac += o.dc_part[at];
      ab += o.db_part[at];
    }
    d_c[tok_index(s, b, tt) * s.N + n] = ac;
    d_b[tok_index(s, b, tt) * s.N + n] = ab;
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
  for (int c = s.NC - 1; c >= 0; --c) {
    const float v = d[(long)c * AM];
    d[(long)c * AM] = acc;
    acc += v;
  }
}

// Bias gradients: sums over (b, chunk) of the per-head partials; eight
// threads per coordinate take every eighth (b, chunk) and combine in LDS.
__global__ __launch_bounds__(1024) void bias_kernel(Shape s, GradOut o, float* d_qb, float* d_kb) {
  __shared__ float part[2][8][NT];
  const int h = blockIdx.x, n = tix() % NT, slice = tix() / NT;
  float aq = 0.f, ak = 0.f;
  for (int bc = slice; bc < s.B * s.NC; bc += 8) {
    const long at = ((long)bc * s.H + h) * NT + n;
    aq += o.qb_part[at];
    ak += o.kb_part[at];
  }
  part[0][slice][n] = aq;
  part[1][slice][n] = ak;
  __syncthreads();
  if (slice == 0 && n < s.N) {
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sq += part[0][i][n];
      sk += part[1][i][n];
    }
    d_qb[(long)h * s.N + n] = sq;
    d_kb[(long)h * s.N + n] = sk;
  }
}

#define M3_SCAN_KERNELS(In)                                                                    \
  template __global__ void walk_kernel<false, In>(Shape, const In*, const float*, const In*,     \
                                                  const float*, const float*, const float*,      \
                                                  const float*, float*, float*, const float*,    \
                                                  float*);                                       \
  template __global__ void walk_kernel<true, In>(Shape, const In*, const float*, const In*,      \
                                                 const float*, const float*, const float*,       \
                                                 const float*, float*, float*, const float*,     \
                                                 float*);                                        \
  template __global__ void out_kernel<In>(Shape, const In*, const In*, const In*, const float*,  \
                                          const float*, const float*, const float*,              \
                                          const float*, const float*, const float*,              \
                                          const float*, In*);                                    \
  template __global__ void grad_kernel<In>(Shape, int, const In*, const In*, const In*,          \
                                           const float*, const float*, const float*,             \
                                           const float*, const float*, const float*,             \
                                           const float*, const float*, const float*, const In*,  \
                                           GradOut);
M3_SCAN_KERNELS(float)
M3_SCAN_KERNELS(bf16_t)
#undef M3_SCAN_KERNELS

}  // namespace m3
