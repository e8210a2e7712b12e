// Per-token factorization, solves and factor streaming (four matrices per
// wave, one per 16-lane row; see rows16.hpp for the layout).
//
// fwd_factor_kernel restates the token loop of _solve_kernel
// (lm/kernels/mamba4_fused.py:116-152): starting from the chunk's start
// evidence it applies each token's gated rank-one update
// E = lam E + beta k k^T (:90-92), factors E + diag(floor) by Cholesky with
// reciprocal pivots (:93-113), solves L L^T y = q (:45-75) and stores the
// factor.  A wave pair runs four (batch, head, sub-chunk) sequences that
// share the sub-chunk index, one per 16-lane row, its two waves taking
// alternate tokens; the running evidence of each sequence lives in LDS
// between tokens (40 KB per pair, quad-interleaved so every 16-byte access
// is conflict-free), the working matrix in VGPRs.  A block holds four pairs
// (eight waves, 160 KB of LDS: one block per CU).
//
// factored_solve_kernel restates _factored_kernel (:155-174): stream four
// stored factors per wave into registers and run the two substitutions.
//
// decode_step_kernel restates selective_decode (lm/kernels/mamba4.py:341-355)
// for four resident states per wave, updated in place.
#include "rows16.hpp"

namespace m4 {

// Quad index of slot (m, 4q) within a lane's 160 evidence slots.
__device__ __forceinline__ constexpr int slot_quad(int m, int q) {
  return (m == 0 ? 0 : m == 1 ? 4 : m == 2 ? 12 : 24) + q;
}

__device__ __forceinline__ int wave_max4(int x) {
  const int a0 = __builtin_amdgcn_readlane(x, 0), a1 = __builtin_amdgcn_readlane(x, 16);
  const int a2 = __builtin_amdgcn_readlane(x, 32), a3 = __builtin_amdgcn_readlane(x, 48);
  return max(max(a0, a1), max(a2, a3));
}

// One token's inputs for this lane's four rows: key and query rows a+16m,
// beta and the log decay.  The decay's exponential is taken where it is used,
// so nothing waits on these loads until the next token's turn; the factor
// stores issued in between then stay in flight (vmcnt counts loads and stores
// in issue order).
struct TokenInputs {
  float k[4], q[4], beta, log_lam;
  long th;
};

template <typename In>
__device__ __forceinline__ void load_token(TokenInputs& in, const Dims& d, const In* keys,
                                           const In* queries, const float* beta,
                                           const float* log_decay, int b, int h, int t, int a) {
  in.th = token_head(d, b, t, h);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    in.k[m] = load1(keys + in.th * 64 + a + 16 * m);
    in.q[m] = load1(queries + in.th * 64 + a + 16 * m);
  }
  in.beta = beta[in.th];
  in.log_lam = log_decay[in.th];
}

// MIX: the token's raw key and query (the shifted raw key row, whose zero
// row at position 0 reads the query row and is zeroed by mix_token).
__device__ __forceinline__ void load_token_mix(TokenInputs& in, bool& kzero, const Dims& d,
                                               const MixerIn& mix, const float* beta,
                                               const float* log_decay, int b, int h, int t,
                                               int a) {
  in.th = token_head(d, b, t, h);
  const float* kp = mix_key_row(mix, d, b, t, h);
  kzero = kp == nullptr;
  if (kzero) kp = mix.query + in.th * 64;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    in.k[m] = kp[a + 16 * m];
    in.q[m] = mix.query[in.th * 64 + a + 16 * m];
  }
  in.beta = beta[in.th];
  in.log_lam = log_decay[in.th];
}

// MIX: unit-normalise the key and query rows (the 16 lanes of the row hold
// its 64 elements, 4 each).
__device__ __forceinline__ void mix_token(TokenInputs& in, bool kzero) {
  float sk = 0.f, sq = 0.f;
  sk += in.k[0] * in.k[0] + in.k[1] * in.k[1] + in.k[2] * in.k[2] + in.k[3] * in.k[3];
  sq += in.q[0] * in.q[0] + in.q[1] * in.q[1] + in.q[2] * in.q[2] + in.q[3] * in.q[3];
  const float rk = kzero ? 0.f : __builtin_amdgcn_rsqf(sum16(sk) + 1e-6f);
  const float rq = __builtin_amdgcn_rsqf(sum16(sq) + 1e-6f);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    in.k[m] *= rk;
    in.q[m] *= rq;
  }
}

// Where rows past their sequence send their factor and solution: the
// stores stay unconditional, so the wait for the next token's loads can
// count them (a store skipped on some path would make the compiler wait for
// every outstanding store).  Written concurrently with garbage; never read.
__device__ __align__(256) float g_discard[ROWS_FACTOR + 64];

// Wait until the evidence buffer holds the updates of tokens 0..tt-1.  The
// other wave of the pair publishes each of its turns by raising the count
// (an LDS max); a wait lasts at most one factorization of that wave plus its
// turn.  Bounded all the same, at `polls` polls (2^16 by default, about
// 2 ms).  Returns the count last seen: below tt when the wait gave up.
typedef __attribute__((address_space(3))) volatile int lds_int;

// The count of a poisoned pair: above every token count, so every later wait
// passes at once and sees it.
constexpr int kPoisoned = 1 << 24;

__device__ __forceinline__ int wait_turn(lds_int* count, int tt, int polls) {
  int seen = __builtin_amdgcn_readfirstlane(*count);
  for (int i = 0; seen < tt && i < polls; ++i) {
    __builtin_amdgcn_s_sleep(1);
    seen = __builtin_amdgcn_readfirstlane(*count);
  }
  asm volatile("" ::: "memory");  // no evidence read moves above the wait
  return seen;
}

// count = max(count, v) in LDS (a published count never goes down, so a
// poisoned pair stays poisoned).
__device__ __forceinline__ void raise_count(lds_int* count, int v) {
  __hip_atomic_fetch_max((__attribute__((address_space(3))) int*)count, v, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Two waves share the four sequences of a pair and take alternate tokens:
// wave w factors tokens base+w for base = 0, 2, 4, ...  The running evidence
// lives in LDS; each wave in its turn reads it, applies its token's rank-one
// update, writes it back and keeps the updated copy in registers.  A turn
// starts as soon as the other wave's previous turn is published (a token
// count in LDS, no block barrier), so each wave runs turn, factorization,
// turn, ... without waiting out the other wave's turn, the two waves offset
// by one turn.  A pair holds one 40 KB evidence buffer.
//
// PAIRS pairs per block (waves 2p, 2p + 1 form pair p).  Four: a CU holds
// one eight-wave block rather than four two-wave ones, the same waves per
// SIMD, about 5% faster on the same work (measured; two-wave blocks spent
// more of each pass waiting for the other wave's turn).  Two: the launch
// takes these when the four-pair blocks would not fill the chip in whole
// rounds; the last round's blocks then spread over every CU at one wave per
// SIMD (each wave issues faster alone) instead of filling part of the chip
// at two.  Only the grid changes: every sequence runs the same code.
//
// A wave whose wait gives up (wait_turn) may read the evidence before the
// other wave's update: it poisons the pair's count at once, and every turn of
// either wave from then on takes a NaN decay, so every later factor and
// solution of the pair's sequences is NaN rather than plausible and wrong.
// A negative `polls` makes every wait but the first token's give up (a test
// of this path; the host never sets it otherwise).
//
// MIX: keys and queries come from the mixer's raw projections (`mix`),
// shifted and normalised as each token is loaded.  STORE = false: the factors
// are not stored (`factors` is unused), the reference's store_factors=False
// mode (lm/kernels/mamba4_fused.py:183-232), for forwards that take no
// gradient.
template <typename In, bool MIX, bool STORE, int PAIRS>
__global__ __launch_bounds__(128 * PAIRS) void fwd_factor_kernel(
    Dims d, const In* __restrict__ keys, const In* __restrict__ queries,
    const float* __restrict__ beta, const float* __restrict__ log_decay,
    const float* __restrict__ floor, const float* __restrict__ start_s,
    float* __restrict__ solved, float* __restrict__ factors, MixerIn mix, int polls) {
  const int lane = threadIdx.x & 63, a = lane & 15, mu = lane >> 4;
  const int wave8 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int pair = wave8 >> 1, wave = wave8 & 1;
  const int BH = d.B * d.H;
  const long nseq = (long)BH * d.NS;
  long seq = ((long)blockIdx.x * PAIRS + pair) * 4 + mu;
  const bool active = seq < nseq;
  if (!active) seq = nseq - 1;
  // Sequences are ordered sub-chunk-major, so a wave's four rows share the
  // sub-chunk index and read neighbouring heads.
  const int ns = (int)(seq / BH), bh = (int)(seq % BH), b = bh / d.H, h = bh % d.H;
  const int n = ns / d.rsub, u = ns % d.rsub;
  const int len = active ? sub_len(d, n, u) : 0;
  const int t0 = n * d.chunk + sub_first(d, u);
  const int steps = wave_max4(len);

  // The running evidence, negated (the factorization's working convention).
  __shared__ f4 evidence_all[PAIRS][40 * 64];  // per pair: [quad][lane]
  f4* const evidence = evidence_all[pair];
  // The turn count lives in the pair's buffer (the four fill the CU's LDS):
  // word 0 of lane 0's quad (0, 3), row 0,
  // columns 12..15 of sequence 0, above the diagonal.  No turn writes that
  // quad; the factorization reads it as scratch and zeroes it.
  lds_int* const turn_count = (lds_int*)(&evidence[slot_quad(0, 3) * 64]);
  // A row whose head's largest floor lies outside [2^-8, 2^8) factors c E,
  // c = 2^2s with c max(floor) in [0.5, 2), and brings the factor back to L
  // (exact power-of-two scalings; factor_exchanged).  The trailing updates
  // carry the panel values as f16 pieces, whose lo piece turns subnormal
  // below 2^-3 and whose hi piece overflows above 65504: scaled so, every
  // row's largest pivot is at least about 0.7 and the pieces' absolute error
  // stays under fp32's own rounding of c E, whatever the inputs' scale, and
  // a piece overflows only for evidence above 4.29e9 / c.  Other rows (the
  // models' floors) factor E as it is.
  float fl[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) fl[m] = floor[h * 64 + a + 16 * m];
  const int fexp = __builtin_amdgcn_frexp_expf(max16(fmaxf(fmaxf(fl[0], fl[1]), fmaxf(fl[2], fl[3]))));
  const int sexp = fexp >= -7 && fexp <= 8 ? 0 : min(max((1 - fexp) >> 1, -60), 60);
  const float c = __builtin_ldexpf(1.f, 2 * sexp);
#pragma unroll
  for (int m = 0; m < 4; ++m) fl[m] *= c;
  {
    // Both waves of the pair stage the start evidence: wave 0 slots 0..2 (24 quads),
    // wave 1 slot 3 (16 quads).
    const float* s0 = start_s + ((long)bh * d.NS + ns) * 4096;
    if (wave == 0) {
#pragma unroll
      for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int q = 0; q < 4 * m + 4; ++q)
          evidence[slot_quad(m, q) * 64 + lane] =
              -c * *reinterpret_cast<const f4*>(s0 + (a + 16 * m) * 64 + 4 * q);
      if (lane == 0) *turn_count = 0;  // after this lane's quad (0, 3): LDS writes stay in order
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q)
        evidence[slot_quad(3, q) * 64 + lane] =
            -c * *reinterpret_cast<const f4*>(s0 + (a + 48) * 64 + 4 * q);
    }
  }
  // Rows past their sequence read token 0 (in bounds; never stored).
  auto token = [&](int tt) { return tt < len ? t0 + tt : 0; };
  TokenInputs cur;
  bool kzero = false;
  if constexpr (MIX) {
    load_token_mix(cur, kzero, d, mix, beta, log_decay, b, h, token(wave), a);
    mix_token(cur, kzero);
  } else {
    load_token(cur, d, keys, queries, beta, log_decay, b, h, token(wave), a);
    // As at the end of each pass below: no load of `cur` is left pending at
    // the loop's head.
    asm volatile("" ::"v"(cur.k[0]), "v"(cur.k[1]), "v"(cur.k[2]), "v"(cur.k[3]), "v"(cur.q[0]),
                 "v"(cur.q[1]), "v"(cur.q[2]), "v"(cur.q[3]), "v"(cur.beta), "v"(cur.log_lam));
  }
  // Nor of the floor (its loads would otherwise sink into the loop's
  // preheader and every pass would wait for them behind the last stores).
  asm volatile("" ::"v"(fl[0]), "v"(fl[1]), "v"(fl[2]), "v"(fl[3]));
  __syncthreads();

  for (int base = 0; base < steps; base += 2) {
    const int tt = base + wave;
    if (tt >= steps) break;       // uniform over the wave (wave 1, odd step counts)
    const bool valid = tt < len;  // per 16-lane row
    float A[4][64];
    const int seen = wait_turn(turn_count, tt, polls);
    const bool gave_up = seen < tt || (polls < 0 && tt > 0);
    if (gave_up && lane == 0) raise_count(turn_count, kPoisoned);
    const float lam = gave_up || seen >= kPoisoned ? __builtin_nanf("") : expf(cur.log_lam);
    const float cbeta = __builtin_ldexpf(cur.beta, 2 * sexp);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const float nbk = -cbeta * cur.k[m];
#pragma unroll
      for (int q = 0; q < 4 * m + 4; ++q) {
        f4 sv = evidence[slot_quad(m, q) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int k = 4 * q + e;
          sv[e] = lam * sv[e] + nbk * bcast16(cur.k[k >> 4], k & 15);
          A[m][k] = sv[e];
        }
        if (m != 0 || q != 3 || lane != 0) evidence[slot_quad(m, q) * 64 + lane] = sv;
        // Every fourth quad: keeps the compiler from hoisting all 40 LDS
        // reads ahead of the arithmetic (which would need 160 more
        // registers) while four reads stay in flight together.
        if ((q & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
    }
    // The trailing blocks (I, K >= 1) read back exchanged from the buffer
    // this wave just wrote (LDS accesses of a wave complete in order): lane
    // (g, j) takes quad 4K + g of row 16I + j of every sequence mu into
    // A[I][16K + 4mu .. +3].  Replaces six register block exchanges (96
    // lane swaps) by 24 reads.
    const int g = lane >> 4;
#pragma unroll
    for (int I = 1; I < 4; ++I)
#pragma unroll
      for (int K = 1; K <= I; ++K)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const f4 v = evidence[slot_quad(I, 4 * K + g) * 64 + 16 * s + a];
#pragma unroll
          for (int e = 0; e < 4; ++e) A[I][16 * K + 4 * s + e] = v[e];
        }
    // Publish the turn once every LDS access of it has completed.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) raise_count(turn_count, tt + 1);

    // Prefetch this wave's next token; the factorization covers the latency.
    TokenInputs next;
    if constexpr (MIX)
      load_token_mix(next, kzero, d, mix, beta, log_decay, b, h, token(tt + 2), a);
    else
      load_token(next, d, keys, queries, beta, log_decay, b, h, token(tt + 2), a);
    float nw[4], y[4];
    factor_exchanged<true>(A, fl, cur.q, nw, sexp);
    // MIX: the next token's key and query are normalised here (their loads
    // landed during the factorization), so the chain of the 16-lane norms
    // runs beside the backward substitution's rather than in front of the
    // next turn (the mixer's factor kernel 0.301 -> 0.296 ms at config 2).
    if constexpr (MIX) mix_token(next, kzero);
    // The substitution's chain of dependent 16-lane sums at priority 2 (see
    // factor_panel in rows16.hpp); the stores and the next turn at 0.
    __builtin_amdgcn_s_setprio(2);
    backward_rows16(A, nw, y);
    __builtin_amdgcn_s_setprio(0);
    float* const sol = valid ? solved + cur.th * 64 : g_discard + ROWS_FACTOR;
#pragma unroll
    for (int m = 0; m < 4; ++m) sol[a + 16 * m] = y[m];
    if constexpr (STORE) store_rows16(A, valid ? factors + cur.th * ROWS_FACTOR : g_discard);
    // Wait for the next token's loads here, where the wait can count the
    // stores just issued (vmcnt retires in order; the loads came first): the
    // polling loop in front of the next turn makes the compiler wait for
    // every outstanding store instead.  (MIX waited above.)
    if constexpr (!MIX)
      asm volatile("" ::"v"(next.k[0]), "v"(next.k[1]), "v"(next.k[2]), "v"(next.k[3]),
                   "v"(next.q[0]), "v"(next.q[1]), "v"(next.q[2]), "v"(next.q[3]),
                   "v"(next.beta), "v"(next.log_lam));
    cur = next;
  }
}

#define M4_FWD_FACTOR(IN, MIX, STORE)                                                      \
  template __global__ void fwd_factor_kernel<IN, MIX, STORE, 4>(                           \
      Dims, const IN*, const IN*, const float*, const float*, const float*, const float*, \
      float*, float*, MixerIn, int);                                                       \
  template __global__ void fwd_factor_kernel<IN, MIX, STORE, 2>(                           \
      Dims, const IN*, const IN*, const float*, const float*, const float*, const float*, \
      float*, float*, MixerIn, int);
M4_FWD_FACTOR(float, false, true)
M4_FWD_FACTOR(bf16_t, false, true)
M4_FWD_FACTOR(float, true, true)
M4_FWD_FACTOR(float, false, false)
M4_FWD_FACTOR(bf16_t, false, false)
M4_FWD_FACTOR(float, true, false)
#undef M4_FWD_FACTOR

// z = A^-1 rhs from stored factors; four token-heads per wave.
__global__ __launch_bounds__(64) void factored_solve_kernel(const float* __restrict__ factors,
                                                            const float* rhs, float* z, long N) {
  const int lane = threadIdx.x, a = lane & 15, mu = lane >> 4;
  long th = (long)blockIdx.x * 4 + mu;
  const bool active = th < N;
  if (!active) th = N - 1;
  // The right-hand side first: the forward substitution needs it at its
  // first step, and loads retire in issue order.
  float r[4], y[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) r[m] = rhs[th * 64 + a + 16 * m];
  float A[4][64];
  load_rows16(A, factors + th * ROWS_FACTOR);
  solve_rows16(A, r, y);
  if (active)
#pragma unroll
    for (int m = 0; m < 4; ++m) z[th * 64 + a + 16 * m] = y[m];
}

// Batched SPD solve, four systems per wave: precision [N,dim,dim] (only
// k <= i is read), rhs [N,dim] -> solution [N,dim] and, when `factors` is
// non-null, each system's factor in the quad-run layout.  Systems are
// padded to 64 with an identity block, so the padded coordinates solve to
// zero, as the reference pads its lanes with identity systems
// (lm/kernels/mamba4_fused.py:292-299).  Restates _factor_and_solve
// (lm/kernels/mamba4.py:164-187).
__global__ __launch_bounds__(64) void spd_solve_kernel(const float* __restrict__ precision,
                                                       const float* __restrict__ rhs, long N,
                                                       int dim, float* __restrict__ solution,
                                                       float* __restrict__ factors) {
  const int lane = threadIdx.x, a = lane & 15, mu = lane >> 4;
  long n = (long)blockIdx.x * 4 + mu;
  const bool active = n < N;
  if (!active) n = N - 1;
  const float* P = precision + n * dim * dim;
  float A[4][64];
  if (dim == 64) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int i = a + 16 * m, p = i >> 2;
#pragma unroll
      for (int q = 0; q < 4 * m + 4; ++q) {
        f4 v = f4{0.f, 0.f, 0.f, 0.f};
        if (q <= p) v = *reinterpret_cast<const f4*>(P + i * 64 + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) A[m][4 * q + e] = 4 * q + e <= i ? -v[e] : 0.f;
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int i = a + 16 * m;
#pragma unroll
      for (int k = 0; k < slot_cols(m); ++k) {
        float v = k == i ? 1.f : 0.f;
        if (i < dim && k <= i) v = P[i * dim + k];
        A[m][k] = -v;
      }
    }
  }
  const float zero[4] = {0.f, 0.f, 0.f, 0.f};
  float r[4], nw[4], y[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int i = a + 16 * m;
    r[m] = i < dim ? rhs[n * dim + i] : 0.f;
  }
  factor_rows16<false>(A, zero, r, nw);
  backward_rows16(A, nw, y);
  if (active) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
      if (a + 16 * m < dim) solution[n * dim + a + 16 * m] = y[m];
    if (factors) store_rows16(A, factors + n * ROWS_FACTOR);
  }
}

// VJP of the batched SPD solve (lm/kernels/mamba4.py:204-215): z = A^-1 g
// from the stored factor, d_rhs = z and d_precision = -(z y^T + y z^T) / 2.
__global__ __launch_bounds__(64) void spd_backward_kernel(
    const float* __restrict__ factors, const float* __restrict__ solution,
    const float* __restrict__ d_solution, long N, int dim, float* __restrict__ d_precision,
    float* __restrict__ d_rhs) {
  const int lane = threadIdx.x, a = lane & 15, mu = lane >> 4;
  long n = (long)blockIdx.x * 4 + mu;
  const bool active = n < N;
  if (!active) n = N - 1;
  float g[4], y[4], z[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int i = a + 16 * m;
    g[m] = i < dim ? d_solution[n * dim + i] : 0.f;
    y[m] = i < dim ? solution[n * dim + i] : 0.f;
  }
  float A[4][64];
  load_rows16(A, factors + n * ROWS_FACTOR);
  solve_rows16(A, g, z);
  if (!active) return;
#pragma unroll
  for (int m = 0; m < 4; ++m)
    if (a + 16 * m < dim) d_rhs[n * dim + a + 16 * m] = z[m];
  float* dP = d_precision + n * dim * dim;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    float yk[4], zk[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = 4 * q + e;
      yk[e] = bcast16(y[k >> 4], k & 15);
      zk[e] = bcast16(z[k >> 4], k & 15);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int i = a + 16 * m;
      if (i >= dim) continue;
      f4 v;
      {
        // Both products rounded on their own (no contraction into an FMA),
        // so the sum, and d_precision, is exactly symmetric.
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = -0.5f * (z[m] * yk[e] + y[m] * zk[e]);
      }
      if (dim == 64) {
        *reinterpret_cast<f4*>(dP + i * 64 + 4 * q) = v;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * q + e < dim) dP[i * dim + 4 * q + e] = v[e];
      }
    }
  }
}

// One decode step for four (batch*head) states per wave, in place.
//
// The states stream through coalesced passes: in each, the 16 lanes of DPP
// row mu sweep whole 256-byte rows of state mu (lane c holds column quad c),
// so one 16-byte access instruction covers four full rows.  The update
// lam S + beta k k^T (and lam C + beta v k^T) is applied in that layout, the
// row's key (or value) arriving by DPP broadcast from the lane that holds it.
// The factorization needs rows a+16m in lane a: each 16-row slot of the
// updated S passes through a 17 KB LDS buffer (rows padded to 17 quads, so
// both the quad-wise writes and the row-wise reads are conflict-free).
// Two waves per SIMD: the value, query and key quad are read again after the
// factorization rather than held in registers across it.
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void
decode_step_kernel(float* __restrict__ evidence, float* __restrict__ cross,
                   const float* __restrict__ key, const float* __restrict__ value,
                   const float* __restrict__ query, const float* __restrict__ beta,
                   const float* __restrict__ log_decay, const float* __restrict__ floor, long N,
                   int H, int NV, float* __restrict__ output, float* __restrict__ variance) {
  const int lane = threadIdx.x, a = lane & 15, mu = lane >> 4;
  long nidx = (long)blockIdx.x * 4 + mu;
  const bool active = nidx < N;
  if (!active) nidx = N - 1;
  float* S = evidence + nidx * 4096;
  const int P = 64 * NV;  // value width; the cross state is NV stacked 64x64 tiles
  float kr[4], qr[4], fl[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    kr[m] = key[nidx * 64 + a + 16 * m];
    qr[m] = query[nidx * 64 + a + 16 * m];
    fl[m] = floor[(nidx % H) * 64 + a + 16 * m];
  }
  // Column quad a of the key: k[4a .. 4a+3].
  f4 kq = *reinterpret_cast<const f4*>(key + nidx * 64 + 4 * a);
  const float bt = beta[nidx], lam = expf(log_decay[nidx]);
  __shared__ f4 stage[4 * 16 * 17];  // [state][row][quad], 17 quads per row
  f4* mine = stage + mu * 16 * 17;

  float A[4][64];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // Coalesced update of rows 16m .. 16m+15; the row's key comes from the
    // lane that holds it in this row's slot (bcast16 of kr[m]).  All 16
    // loads are issued before the first store (a store between them would
    // leave one load in flight at a time).
    f4* rows = reinterpret_cast<f4*>(S + 16 * m * 64) + a;
    f4 sv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) sv[r] = __builtin_nontemporal_load(rows + 16 * r);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float bk = bt * bcast16(kr[m], r);
      sv[r] = lam * sv[r] + bk * kq;
      mine[r * 17 + a] = sv[r];
    }
    if (active)
#pragma unroll
      for (int r = 0; r < 16; ++r) __builtin_nontemporal_store(sv[r], rows + 16 * r);
    __syncthreads();
    // Into the factorization layout, negated: block column 0 as row a of this
    // slot, blocks (m, K >= 1) exchanged (lane (g, j) takes quad 4K + g of
    // row j of every state).
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f4 v = mine[a * 17 + q];
#pragma unroll
      for (int e = 0; e < 4; ++e) A[m][4 * q + e] = -v[e];
    }
#pragma unroll
    for (int K = 1; K <= m; ++K)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f4 v = stage[s * 16 * 17 + a * 17 + 4 * K + mu];
#pragma unroll
        for (int e = 0; e < 4; ++e) A[m][16 * K + 4 * s + e] = -v[e];
      }
    __syncthreads();
  }
  float nw[4], y[4];
  factor_exchanged<false>(A, fl, qr, nw);
  backward_rows16(A, nw, y);
#pragma unroll
  for (int m = 0; m < 4; ++m) qr[m] = query[nidx * 64 + a + 16 * m];
  kq = *reinterpret_cast<const f4*>(key + nidx * 64 + 4 * a);
  // y[4a .. 4a+3] for the coalesced read: y_j lives in lane j%16, slot j/16.
  __shared__ float ys[4][64];
#pragma unroll
  for (int m = 0; m < 4; ++m) ys[mu][a + 16 * m] = y[m];
  __syncthreads();
  const f4 yq = *reinterpret_cast<const f4*>(&ys[mu][4 * a]);
  for (int v = 0; v < NV; ++v) {
    float* C = cross + (nidx * NV + v) * 4096;
    float vr[4], out[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) vr[m] = value[nidx * P + 64 * v + a + 16 * m];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      // As for S: the slot's 16 row loads go out together.
      f4* rows = reinterpret_cast<f4*>(C + 16 * m * 64) + a;
      f4 cv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) cv[r] = __builtin_nontemporal_load(rows + 16 * r);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float bv = bt * bcast16(vr[m], r);
        cv[r] = lam * cv[r] + bv * kq;
        // Row 16m + r of the read, summed over the 16 column quads.
        const float part =
            sum16(cv[r][0] * yq[0] + cv[r][1] * yq[1] + cv[r][2] * yq[2] + cv[r][3] * yq[3]);
        out[m] = a == r ? part : out[m];
      }
      if (active)
#pragma unroll
        for (int r = 0; r < 16; ++r) __builtin_nontemporal_store(cv[r], rows + 16 * r);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m)
      if (active) output[nidx * P + 64 * v + a + 16 * m] = out[m];
  }
  float var = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) var += qr[m] * y[m];
  var = sum16(var);
  if (active && a == 0) variance[nidx] = var;
}

}  // namespace m4
