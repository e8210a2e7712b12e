// Four 64x64 SPD matrices per wave, one per 16-lane DPP row.
//
// Lane a of row-group mu (lane = 16*mu + a) owns rows a, a+16, a+32, a+48 of
// matrix mu: slot m holds row a+16m, columns 0..15+16m, in A[m][k].  Slots
// are sized for the longest row of the slot (a = 15), so columns past a row's
// diagonal are scratch that is zeroed after the factorization.  Every
// cross-lane value the factorization and the two substitutions need lives in
// the same 16-lane row, so it moves by DPP row_newbcast (broadcast of one
// lane of the row), folded into the consuming FMA where the compiler can.
// No LDS is touched and 74% of the issued FMA lanes do useful work.
//
// Factor storage ("quad runs"): row i = a + 16m holds the column quads
// 0..i/4.  For each row slot m and column quad q, the quads of the lanes that
// hold it (a >= 4 max(0, q - 4m)) are stored contiguously in lane order, so
// one 16-byte store or load instruction of a 16-lane row covers a 64..256-byte
// run and whole 128-byte lines over a slot.  Slots follow each other and runs
// go in increasing q: 544 quads, 2176 floats per matrix; the diagonal holds
// the reciprocal pivot 1/L_ii.
#pragma once

#include <utility>

#include "common.hpp"

namespace m4 {

constexpr int ROWS_FACTOR = 2176;  // floats per stored factor

// Quads before row slot m: slot m holds 16 (4m + 1) + 12 + 8 + 4 quads.
__host__ __device__ constexpr int slot_base(int m) { return 32 * m * m + 8 * m; }

// Lane a's quad q of row slot m is quad run_quad(m, q) + a of the factor.
// Runs q <= 4m hold all 16 lanes; runs q = 4m + r (r = 1, 2, 3) start at
// lane 4r.
__host__ __device__ constexpr int run_quad(int m, int q) {
  return slot_base(m) + (q <= 4 * m ? 16 * q
                                    : 16 * (4 * m + 1) + (q == 4 * m + 1   ? -4
                                                          : q == 4 * m + 2 ? 4
                                                                           : 8));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

// Value of x at lane `src` of this lane's 16-lane row (src known after unrolling).
__device__ __forceinline__ float bcast16(float x, int src) {
  switch (src) {
    case 0: return dpp<0x150>(x);
    case 1: return dpp<0x151>(x);
    case 2: return dpp<0x152>(x);
    case 3: return dpp<0x153>(x);
    case 4: return dpp<0x154>(x);
    case 5: return dpp<0x155>(x);
    case 6: return dpp<0x156>(x);
    case 7: return dpp<0x157>(x);
    case 8: return dpp<0x158>(x);
    case 9: return dpp<0x159>(x);
    case 10: return dpp<0x15A>(x);
    case 11: return dpp<0x15B>(x);
    case 12: return dpp<0x15C>(x);
    case 13: return dpp<0x15D>(x);
    case 14: return dpp<0x15E>(x);
    default: return dpp<0x15F>(x);
  }
}

// Sum over the 16 lanes of the row; every lane receives the total.
__device__ __forceinline__ float sum16(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  return x;
}

// Maximum over the 16 lanes of the row; every lane receives it.
__device__ __forceinline__ float max16(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return x;
}

// acc += src[lane L of the row] * mul as one v_fmac_f32_dpp (row_newbcast:L).
// The caller guarantees src was not written by the previous two VALU
// instructions (see factor_step).
template <int L>
__device__ __forceinline__ void fmac_bcast(float& acc, float src, float mul) {
  asm volatile("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
               : "+v"(acc)
               : "v"(src), "v"(mul), "n"(L));
}

// Column K of every row slot that holds it (slots m >= K/16 and >= J/16)
// takes l_iJ l_KJ, l_KJ broadcast from lane K%16 of slot K/16 and l_iJ
// = L[m][J] of this lane.
template <int J, int K>
__device__ __forceinline__ void update_column(float (&A)[4][64], const float (&L)[4][64]) {
  constexpr int r = K >> 4, mj = J >> 4, m0 = r > mj ? r : mj;
#pragma unroll
  for (int m = m0; m < 4; ++m) fmac_bcast<(K & 15)>(A[m][K], A[r][J], L[m][J]);
}

template <int J, int... I>
__device__ __forceinline__ void update_columns(float (&A)[4][64], const float (&L)[4][64],
                                               std::integer_sequence<int, I...>) {
  (update_column<J, J + 1 + I>(A, L), ...);
}

constexpr int slot_cols(int m) { return 16 * (m + 1); }

template <int Off, int... I>
constexpr std::integer_sequence<int, (Off + I)...> offset_sequence(std::integer_sequence<int, I...>) {
  return {};
}

// Factorization convention.  The working matrix is held negated: before
// column J is eliminated, A[m][k] holds -(E + diag(floor) - sum_{j<J} l_ij
// l_kj) without the floor, i.e. -E minus the updates so far.  Every update
// then adds l_ij l_kj (an FMA with no negation), the pivot is floor - A_JJ,
// and the trailing blocks accumulate their MFMA updates in place (D = C + A B).
//
// Block layouts.  "Rows": lane (mu, a) holds row 16I + a of matrix mu in
// A[I][16K + c], c = 0..15 (the slot layout above).  "Exchanged": lane
// (g, j) holds in A[I][16K + 4mu + e] element (16I + j, 16K + 4g + e) of
// matrix mu.  exchange_block converts one 16x16 block of all four matrices
// between the two (it is its own inverse).  Exchanged is the accumulator
// layout of the four-block 16x16 MFMA shapes for four blocks whose rows are
// block columns, and rows is their operand layout (panel_update), so the
// trailing updates read the panel in rows and accumulate in exchanged; only
// a trailing block column that becomes the next panel is exchanged.

// One elimination step of column J inside its 16-column panel P = J/16,
// with the forward substitution of the right-hand side r folded in: the
// pivot floor - A_JJ is broadcast from lane J%16, column J becomes l_iJ =
// -A_iJ / sqrt(pivot), every later column of the panel takes l_iJ l_KJ by one
// DPP-fed FMA per slot, and r_i takes -l_iJ w_J with w_J = r_J / l_JJ.  The
// step records -w_J in nw (lane J%16 of slot J/16) and 1/l_JJ on the
// diagonal.
// Columns right of the panel are updated by panel_update.
template <int J>
__device__ __forceinline__ void factor_step(float (&A)[4][64], const float (&fl)[4],
                                            float (&r)[4], float (&nw)[4], int a) {
  constexpr int mj = J >> 4, lj = J & 15, panel_end = 16 * mj + 15;
  const float piv = bcast16(fl[mj] - A[mj][J], lj);
  // v_rsq_f32 (1 ulp), as the reference's lax.rsqrt pivot
  // (lm/kernels/mamba4_fused.py:111); a non-positive pivot gives NaN.
  const float rs = __builtin_amdgcn_rsqf(piv);
#pragma unroll
  for (int m = mj; m < 4; ++m) A[m][J] = -A[m][J] * rs;
  // The sub-diagonal values are materialised here: the compiler would
  // otherwise fold the reciprocal pivot into their f16 split (panel_update)
  // and keep the panel's sixteen pivots live up to it.
#pragma unroll
  for (int m = mj + 1; m < 4; ++m) asm volatile("" : "+v"(A[m][J]));
  float nwj = -r[mj] * rs;  // -w_J in lane J%16: r_J is final once column J is reached
  // GFX9 needs two wait states between a VALU write of a VGPR and a DPP read
  // of it, and the compiler's hazard tracking does not see inside inline asm.
  // The DPP sources of this step are column J of slot mj and -w_J; passing
  // them through this s_nop as in/out operands orders their writes before
  // the nop and every DPP read after it.  (The build re-checks this hazard on
  // the compiled code, see mamba4_amd/check_dpp_hazards.py.)
  asm volatile("s_nop 1" : "+v"(A[mj][J]), "+v"(nwj));
  // A[m][k] += l_ij * l_kj as one v_fmac_f32_dpp per element, the l_kj
  // operand broadcast straight from lane k%16 (the compiler keeps the
  // broadcast in a separate v_mov_b32_dpp otherwise).
  update_columns<J>(A, A, std::make_integer_sequence<int, panel_end - J>{});
#pragma unroll
  for (int m = mj; m < 4; ++m) fmac_bcast<lj>(r[m], nwj, A[m][J]);
  nw[mj] = a == lj ? nwj : nw[mj];
  A[mj][J] = a == lj ? rs : A[mj][J];
}

template <int... J>
__device__ __forceinline__ void factor_steps(float (&A)[4][64], const float (&fl)[4],
                                             float (&r)[4], float (&nw)[4], int a,
                                             std::integer_sequence<int, J...>) {
  (factor_step<J>(A, fl, r, nw, a), ...);
}

// Exchange of lane groups and register quads: q[g][e] is element e of
// register quad g.  Afterwards lane (g, a) holds in quad mu what lane
// (mu, a) held in quad g (a 4x4 transpose of 16-lane rows against quads;
// its own inverse).  Two v_permlane32_swap then two v_permlane16_swap per
// element: permlane32_swap(x, y) yields rows (x0, x1, y0, y1) and
// (x2, x3, y2, y3), permlane16_swap(x, y) yields (x0, y0, x2, y2) and
// (x1, y1, x3, y3) (checked on gfx950 with an in-bounds probe).
__device__ __forceinline__ void exchange_quads(float& q0, float& q1, float& q2, float& q3) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(q0), __float_as_uint(q2),
                                                  false, false);
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(q1), __float_as_uint(q3),
                                                  false, false);
  const auto t = __builtin_amdgcn_permlane16_swap(r[0], s[0], false, false);
  const auto u = __builtin_amdgcn_permlane16_swap(r[1], s[1], false, false);
  q0 = __uint_as_float(t[0]);
  q1 = __uint_as_float(t[1]);
  q2 = __uint_as_float(u[0]);
  q3 = __uint_as_float(u[1]);
}

// The 16x16 block of columns C0..C0+15 of one row slot, exchanged in place.
template <int C0>
__device__ __forceinline__ void exchange_block(float (&row)[64]) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    exchange_quads(row[C0 + e], row[C0 + 4 + e], row[C0 + 8 + e], row[C0 + 12 + e]);
}

typedef float f16 __attribute__((ext_vector_type(16)));

// Slots I > P of block column C, exchanged in place.
template <int P, int C>
__device__ __forceinline__ void exchange_below(float (&A)[4][64]) {
  if constexpr (P < 1) exchange_block<16 * C>(A[1]);
  if constexpr (P < 2) exchange_block<16 * C>(A[2]);
  if constexpr (P < 3) exchange_block<16 * C>(A[3]);
}

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// x = hi + lo + O(2^-22 |x|): hi = f16(x) (round to nearest), lo = f16(x -
// hi) with x - hi formed exactly by v_fma_mix (x * 1 - hi, the f16 source
// selected by op_sel).  Products of f16 values are exact in the MFMA's fp32
// sums.  Three instructions per pair of values; the closing s_nop gives the
// MFMA that reads the pieces the two wait states a VALU write needs before
// an MFMA operand read (the compiler does not see inside the asm).
__device__ __forceinline__ void split_f16(const float* x, h4& hi, h4& lo) {
  unsigned h01, h23, l01, l23;
  asm volatile(
      "v_cvt_pk_f16_f32 %0, %4, %5\n\t"
      "v_cvt_pk_f16_f32 %1, %6, %7\n\t"
      "v_fma_mixlo_f16 %2, %4, 1.0, -%0 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %2, %5, 1.0, -%0 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixlo_f16 %3, %6, 1.0, -%1 op_sel_hi:[0,0,1]\n\t"
      "v_fma_mixhi_f16 %3, %7, 1.0, -%1 op_sel:[0,0,1] op_sel_hi:[0,0,1]\n\t"
      "s_nop 1"
      : "=&v"(h01), "=&v"(h23), "=&v"(l01), "=&v"(l23)
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));
  hi = __builtin_bit_cast(h4, (uint2{h01, h23}));
  lo = __builtin_bit_cast(h4, (uint2{l01, l23}));
}

// One MFMA of trailing block (I, K): A_IK += a b^T for all four matrices (the
// working matrix is negated), a from slot K and b from slot I (rows layout),
// the block in the exchanged layout.  v_mfma_f32_16x16x4_4b_f16 takes
// A_b[i][0..3] from lane 16b + i and B_b[j][0..3] from lane 16b + j and leaves
// D_b[i][j] += sum_k A_b[i][k] B_b[j][k] in lane j + 16(i/4), register
// 4b + i%4 (checked on gfx950 with an in-bounds probe), so D_mu[i][j] is
// element (16I + j, 16K + i) of matrix mu: register A[I][16K + 4mu + e] of
// lane (g, j) with i = 4g + e, the exchanged layout.
template <int P, int I, int K>
__device__ __forceinline__ void block_term(float (&A)[4][64], const h4& a, const h4& b) {
  f16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = A[I][16 * K + r];
  acc = __builtin_amdgcn_mfma_f32_16x16x4f16(a, b, acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; ++r) A[I][16 * K + r] = acc[r];
}

// Trailing block (I, K) after panel P in fp32: A_IK += L_IP L_KP^T as sixteen
// chained rank-one v_mfma_f32_16x16x1_4b_f32, one per panel column, with the
// operand and accumulator layouts of block_term (lane 16b + i holds A_b[i],
// D_b[i][j] += A_b[i] B_b[j] in lane j + 16(i/4), register 4b + i%4).
template <int P, int I, int K>
__device__ __forceinline__ void block_f32(float (&A)[4][64]) {
  f16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = A[I][16 * K + r];
#pragma unroll
  for (int c = 0; c < 16; ++c)
    acc = __builtin_amdgcn_mfma_f32_16x16x1f32(A[K][16 * P + c], A[I][16 * P + c], acc, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < 16; ++r) A[I][16 * K + r] = acc[r];
}

// Calls f(I, K) (as integral constants) for every trailing block of panel P.
template <int P, typename F>
__device__ __forceinline__ void for_trailing_blocks(F&& f) {
  using std::integral_constant;
  if constexpr (P == 0) {
    f(integral_constant<int, 1>{}, integral_constant<int, 1>{});
    f(integral_constant<int, 2>{}, integral_constant<int, 1>{});
    f(integral_constant<int, 3>{}, integral_constant<int, 1>{});
    f(integral_constant<int, 2>{}, integral_constant<int, 2>{});
    f(integral_constant<int, 3>{}, integral_constant<int, 2>{});
    f(integral_constant<int, 3>{}, integral_constant<int, 3>{});
  } else if constexpr (P == 1) {
    f(integral_constant<int, 2>{}, integral_constant<int, 2>{});
    f(integral_constant<int, 3>{}, integral_constant<int, 2>{});
    f(integral_constant<int, 3>{}, integral_constant<int, 3>{});
  } else if constexpr (P == 2) {
    f(integral_constant<int, 3>{}, integral_constant<int, 3>{});
  }
}

// Rank-16 update of the trailing blocks after panel P, then the next panel's
// block column back to the rows layout.
//
// F16 (the memory read's factorization): four panel columns per MFMA: each
// fp32 panel value is split into f16 hi + lo and the product L_K L_I^T is
// formed as hi hi^T + hi lo^T + lo hi^T (the dropped lo lo^T is below 2^-22
// of it), three instructions per four columns, 12 per block instead of the 16
// rank-one v_mfma_f32_16x16x1_4b_f32 of an fp32 update.  Both shapes issue in
// 32 cycles, but the f16 one runs beside the other wave's VALU work while the
// fp32 one holds the SIMD (measured on gfx950: an FMA wave sharing a SIMD with
// an MFMA wave ran 1.14x its time alone beside the f16 shape, 2.9x beside the
// fp32 one).  The pieces bound the panel values to |l| < 65504 (evidence
// diagonals below 4.29e9), and below 2^-3 the lo piece is subnormal, so a
// value carries an absolute error up to 2^-25 rather than 2^-22 of itself.
//
// !F16 (generic SPD solves and the decode step): the fp32 rank-one updates,
// exact to fp32 for every finite matrix.
template <int P, bool F16>
__device__ __forceinline__ void panel_update(float (&A)[4][64]) {
  if constexpr (P < 3) {
    if constexpr (F16) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        // One column group's pieces live at a time (12 registers at P = 0).
        __builtin_amdgcn_sched_barrier(0);
        h4 hi[4], lo[4];
#pragma unroll
        for (int m = P + 1; m < 4; ++m) split_f16(&A[m][16 * P + 4 * g], hi[m], lo[m]);
#pragma unroll
        for (int t = 0; t < 3; ++t)
          for_trailing_blocks<P>([&](auto Ic, auto Kc) {
            constexpr int I = decltype(Ic)::value, K = decltype(Kc)::value;
            block_term<P, I, K>(A, t == 2 ? lo[K] : hi[K], t == 1 ? lo[I] : hi[I]);
          });
      }
    } else {
      for_trailing_blocks<P>([&](auto Ic, auto Kc) {
        block_f32<P, decltype(Ic)::value, decltype(Kc)::value>(A);
      });
    }
    exchange_below<P, P + 1>(A);
  }
}

// Wave priorities.  The two waves of a SIMD run the same passes offset by a
// turn, and the factorization is bound by dependent chains (each column's
// pivot, scale and next-column update; the backward substitution's 16-lane
// sums) more than by issue.  A panel's elimination therefore runs at
// priority 1 and its MFMA trailing update at 0: when both waves are ready,
// the instruction of a chain issues first and the other wave's independent
// MFMA and split work fills the chain's stalls.  (fwd_factor_kernel raises
// the backward substitution to 2 the same way.)  Measured at config 2: the
// factor kernel 0.304 -> 0.293 ms; priorities 3 and 3, a separate level
// for each column's pivot chain, or one for the turn gained nothing more.
template <int P, bool F16>
__device__ __forceinline__ void factor_panel(float (&A)[4][64], const float (&fl)[4],
                                             float (&r)[4], float (&nw)[4], int a) {
  __builtin_amdgcn_s_setprio(1);
  factor_steps(A, fl, r, nw, a, offset_sequence<16 * P>(std::make_integer_sequence<int, 16>{}));
  __builtin_amdgcn_s_setprio(0);
  panel_update<P, F16>(A);
}

// Blocked right-looking Cholesky of E + diag(floor) with the forward
// substitution of r folded in.  On entry A holds -E: block column 0 in the
// rows layout, blocks (I, K >= 1) exchanged (factor_rows16 converts a full
// rows-layout input).  Four 16-column panels: each is eliminated column by
// column with DPP-fed FMAs (factor_step), then the trailing blocks take the
// panel's rank-16 update on MFMA (panel_update).  On return A holds L below
// the diagonal, 1/L_ii on it and zeros above (rows layout), r is consumed
// and nw = -L^-1 r.  All steps are expanded at compile time so every
// register index is static.  F16 selects the trailing-update form
// (panel_update).
//
// Scaled form (sexp = s != 0): the caller passes -c E, c = 2^2s, and
// c diag(floor) in fl; the factorization runs on c E, whose factor is 2^s L,
// and on return A and nw are brought back to L and -L^-1 r (every value
// times 2^-s, the diagonal's reciprocal pivots times 2^s).  Power-of-two
// scalings (v_ldexp_f32) are exact.
template <bool F16>
__device__ __forceinline__ void factor_exchanged(float (&A)[4][64], const float (&fl)[4],
                                                 float (&r)[4], float (&nw)[4], int sexp = 0) {
  const int a = threadIdx.x & 15;
#pragma unroll
  for (int m = 0; m < 4; ++m) nw[m] = 0.f;
  factor_panel<0, F16>(A, fl, r, nw, a);
  factor_panel<1, F16>(A, fl, r, nw, a);
  factor_panel<2, F16>(A, fl, r, nw, a);
  factor_panel<3, F16>(A, fl, r, nw, a);
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int c = 1; c < 16; ++c) A[m][16 * m + c] = c > a ? 0.f : A[m][16 * m + c];
  // Skipped when no row of the wave is scaled (a wave-uniform branch; folded
  // away when sexp is the literal 0).
  if (__builtin_amdgcn_ballot_w64(sexp != 0)) {
    // Opaque here, so the diagonal's exponents are not hoisted out of the
    // caller's loop into sixteen live registers.
    int se = sexp;
    asm volatile("" : "+v"(se));
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      nw[m] = __builtin_ldexpf(nw[m], se);  // -L^-1 r = 2^s (-(2^s L)^-1 r)
#pragma unroll
      for (int k = 0; k < slot_cols(m); ++k)
        A[m][k] = __builtin_ldexpf(A[m][k], k == 16 * m + a ? se : -se);
    }
  }
}

// The same from a rows-layout -E: the six trailing blocks are exchanged first.
template <bool F16>
__device__ __forceinline__ void factor_rows16(float (&A)[4][64], const float (&fl)[4],
                                              float (&r)[4], float (&nw)[4]) {
  exchange_block<16>(A[1]);
  exchange_block<16>(A[2]);
  exchange_block<32>(A[2]);
  exchange_block<16>(A[3]);
  exchange_block<32>(A[3]);
  exchange_block<48>(A[3]);
  factor_exchanged<F16>(A, fl, r, nw);
}

// y = L^-T w from nw = -w (factor_rows16 / factor_exchanged).
template <int J>
__device__ __forceinline__ void backward_step_nw(const float (&A)[4][64], const float (&nw)[4],
                                                 float (&y)[4], int a) {
  constexpr int mj = J >> 4, lj = J & 15;
  float p = 0.f;
#pragma unroll
  for (int m = mj; m < 4; ++m) p += A[m][J] * y[m];
  const float yj = -(nw[mj] + sum16(p)) * A[mj][J];
  y[mj] = a == lj ? yj : y[mj];
}

template <int... J>
__device__ __forceinline__ void backward_steps_nw(const float (&A)[4][64], const float (&nw)[4],
                                                  float (&y)[4], int a,
                                                  std::integer_sequence<int, J...>) {
  (backward_step_nw<63 - J>(A, nw, y, a), ...);
}

__device__ __forceinline__ void backward_rows16(const float (&A)[4][64], const float (&nw)[4],
                                                float (&y)[4]) {
  const int a = threadIdx.x & 15;
#pragma unroll
  for (int m = 0; m < 4; ++m) y[m] = 0.f;
  backward_steps_nw(A, nw, y, a, std::make_integer_sequence<int, 64>{});
}

// y = (L L^T)^-1 r for a factor from factor_rows16; r is consumed.
template <int J>
__device__ __forceinline__ void forward_step(const float (&A)[4][64], float (&r)[4],
                                             float (&w)[4], int a) {
  constexpr int mj = J >> 4, lj = J & 15;
  const float wj = bcast16(r[mj] * A[mj][J], lj);
  w[mj] = a == lj ? wj : w[mj];
#pragma unroll
  for (int m = mj; m < 4; ++m) r[m] -= A[m][J] * wj;
}

template <int J>
__device__ __forceinline__ void backward_step(const float (&A)[4][64], const float (&w)[4],
                                              float (&y)[4], int a) {
  constexpr int mj = J >> 4, lj = J & 15;
  float p = 0.f;
#pragma unroll
  for (int m = mj; m < 4; ++m) p += A[m][J] * y[m];
  const float yj = (w[mj] - sum16(p)) * A[mj][J];
  y[mj] = a == lj ? yj : y[mj];
}

template <int... J>
__device__ __forceinline__ void solve_steps(const float (&A)[4][64], float (&r)[4], float (&w)[4],
                                            float (&y)[4], int a,
                                            std::integer_sequence<int, J...>) {
  (forward_step<J>(A, r, w, a), ...);
  (backward_step<63 - J>(A, w, y, a), ...);
}

__device__ __forceinline__ void solve_rows16(const float (&A)[4][64], float (&r)[4], float (&y)[4]) {
  const int a = threadIdx.x & 15;
  float w[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 4; ++m) y[m] = 0.f;
  solve_steps(A, r, w, y, a, std::make_integer_sequence<int, 64>{});
}

// Quad-run factor store / load for this lane's four rows.
__device__ __forceinline__ void store_rows16(const float (&A)[4][64], float* __restrict__ fac) {
  const int a = threadIdx.x & 15;
  f4* lane = reinterpret_cast<f4*>(fac) + a;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int p = (a + 16 * m) >> 2;
#pragma unroll
    for (int q = 0; q < 4 * m + 4; ++q)
      if (q <= p)
        // Non-temporal: the factors are read back only by the backward pass.
        __builtin_nontemporal_store(
            f4{A[m][4 * q], A[m][4 * q + 1], A[m][4 * q + 2], A[m][4 * q + 3]},
            &lane[run_quad(m, q)]);
  }
}

// Every load is unconditional (a load under a per-lane branch would make
// the compiler wait for it inside the branch, serialising the stream).  In a
// run q = 4m + r (r = 1..3, lanes 4r..15) the lanes below 4r read the run's
// first quad, so each instruction touches only its own run's lines, and zero
// what they read.  The loads go column quad by column quad (q outer), in the
// order the forward substitution consumes them: vmcnt retires loads in issue
// order, so the first steps wait for the first few quads, not for all 40.
__device__ __forceinline__ void load_rows16(float (&A)[4][64], const float* __restrict__ fac) {
  const int a = threadIdx.x & 15;
  const f4* base = reinterpret_cast<const f4*>(fac);
#pragma unroll
  for (int q = 0; q < 16; ++q) {
#pragma unroll
    for (int m = q / 4; m < 4; ++m) {  // slot m holds quads q <= 4m + 3
      const int r = q - 4 * m;  // > 0: a partial run starting at lane 4r
      const int lane = r > 0 ? max(a, 4 * r) : a;
      // Non-temporal: each factor is read once, by this solve.
      const f4 v = __builtin_nontemporal_load(base + run_quad(m, q) + lane);
      const bool in = r <= 0 || a >= 4 * r;
      A[m][4 * q] = in ? v[0] : 0.f;
      A[m][4 * q + 1] = in ? v[1] : 0.f;
      A[m][4 * q + 2] = in ? v[2] : 0.f;
      A[m][4 * q + 3] = in ? v[3] : 0.f;
    }
  }
}

}  // namespace m4
