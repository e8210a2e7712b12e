// The order head's gated vector scan (lm/models/mamba4.py:46-95, called at
// :274-289): per batch row, head and channel,
//   h_t = lam_t h_(t-1) + (1 - lam_t) v_t,   lam_t = exp(log_decay_t),
// with the inflow 1 - lam_t taken as -expm1(log_decay_t) as the reference's
// chunked form does, from h_(-1) = initial (zero when absent).
//
// Layout: values and output [B,T,H,W], log_decay [B,T,H], initial and the
// initial-state gradient [B,H,W].  One thread per channel; a block covers
// every channel of one (b, h) and one chunk of tokens, so a wave's access to
// a token is one contiguous row of up to 64 floats.  Three passes each way:
//   forward:  order_local  - each chunk's scan from zero: its end state and
//                            total log decay;
//             order_carry  - the state every chunk starts from, chunk by
//                            chunk per (b, h, channel), in place;
//             order_apply  - each chunk's scan from its start state.
//   backward: the same three over the reverse recurrence of the cotangent
//             g_t = dout_t + lam_(t+1) g_(t+1): d v_t = (1 - lam_t) g_t,
//             d log_decay_t = lam_t sum_c g_t,c (h_(t-1),c - v_t,c) (summed
//             over channels in a fixed order), d initial = lam_0 g_0.
#include "common.hpp"

namespace m4 {

__device__ __forceinline__ long order_row(const OrderDims& d, int b, int t, int h) {
  return ((long)b * d.T + t) * d.H + h;
}

// Block (b, h, n) of a grid over B*H*NC chunks.
struct OrderBlock {
  int b, h, n, bh, t0, len;
};

__device__ __forceinline__ OrderBlock order_block(const OrderDims& d) {
  OrderBlock o;
  o.n = blockIdx.x % d.NC;
  o.bh = blockIdx.x / d.NC;
  o.b = o.bh / d.H;
  o.h = o.bh % d.H;
  o.t0 = o.n * d.chunk;
  o.len = min(d.chunk, d.T - o.t0);
  return o;
}

// The per-chunk kernels walk their chunk in groups of ORDER_GROUP tokens, a
// group's loads issued before the previous group is used, every load
// unconditional (tokens past the chunk's length re-read its last row and are
// then masked to value 0).  A token's decay and inflow are the same for every
// channel: lane l computes them for the chunk's token l once (zero log decay
// past the chunk's end, which leaves the scan as it is), and each step reads
// them from that lane.
// The grids hold about one wave per chunk, a few per SIMD: the kernels are
// built for two waves per SIMD, so the scheduler keeps the group loads
// ahead of their use instead of minimising registers.
constexpr int ORDER_GROUP = 16;
constexpr int ORDER_GROUPS = MAXC / ORDER_GROUP;

struct RowGroup {
  float x[ORDER_GROUP];
};

// Loads group `g` of channel c from `rows` (W-float rows): the chunk's row t
// is at first[t * stride] with first = &rows[chunk's first row][c] and
// stride = H W; tokens past the chunk re-read its last row.
__device__ __forceinline__ void load_group(RowGroup& r, const OrderBlock& o, int g,
                                           const float* first, long stride) {
#pragma unroll
  for (int i = 0; i < ORDER_GROUP; ++i)
    r.x[i] = first[min(g * ORDER_GROUP + i, o.len - 1) * stride];
  // Keep the group's loads here, ahead of the previous group's use (the
  // scheduler would otherwise sink each load next to its use).
  __builtin_amdgcn_sched_barrier(0);
}

// Per-token gate of the chunk held by lane l = token l: the log decay (0
// past the chunk), lam = exp and the inflow 1 - lam = -expm1.
struct TokenGates {
  float lg, lam, inflow;

  __device__ __forceinline__ TokenGates(const OrderDims& d, const OrderBlock& o,
                                        const float* log_decay) {
    const int l = lane_id();
    lg = l < o.len ? log_decay[order_row(d, o.b, o.t0 + min(l, o.len - 1), o.h)] : 0.f;
    lam = expf(lg);
    inflow = -expm1f(lg);
  }
  // Summed log decay of the chunk (every lane receives it).
  __device__ __forceinline__ float total() const {
    return group4_sum(row16_sum(lg));
  }
};

__device__ __forceinline__ float lane_value(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Forward pass 1: ends[bh][n][c] = the chunk's scan from zero at its last
// token; totals[bh][n] = its summed log decay.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void order_local_kernel(OrderDims d, const float* values,
                                                          const float* log_decay, float* ends,
                                                          float* totals) {
  const OrderBlock o = order_block(d);
  const int c = threadIdx.x, cc = min(c, d.W - 1);
  const TokenGates gate(d, o, log_decay);
  const float g = gate.total();
  const long stride = (long)d.H * d.W;
  const float* first = values + order_row(d, o.b, o.t0, o.h) * d.W + cc;
  RowGroup r[2];
  load_group(r[0], o, 0, first, stride);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < ORDER_GROUPS; ++k) {
    if (k + 1 < ORDER_GROUPS) load_group(r[(k + 1) & 1], o, k + 1, first, stride);
#pragma unroll
    for (int i = 0; i < ORDER_GROUP; ++i) {
      const int t = k * ORDER_GROUP + i;
      s = lane_value(gate.lam, t) * s + lane_value(gate.inflow, t) * r[k & 1].x[i];
    }
  }
  const long slot = (long)o.bh * d.NC + o.n;
  if (c < d.W) ends[slot * d.W + c] = s;
  if (c == 0) totals[slot] = g;
}

// Chunks of a carry whose loads are issued together.
constexpr int ORDER_CARRY_BATCH = 8;

// Forward pass 2, grid B*H: turns ends into the state each chunk starts from
// (in place), starting from `initial`.
__global__ __launch_bounds__(256) void order_carry_kernel(OrderDims d, const float* initial,
                                                          float* ends, const float* totals) {
  const int bh = blockIdx.x, c = threadIdx.x;
  if (c >= d.W) return;
  float s = initial ? initial[(long)bh * d.W + c] : 0.f;
  for (int n0 = 0; n0 < d.NC; n0 += ORDER_CARRY_BATCH) {
    float local[ORDER_CARRY_BATCH], decay[ORDER_CARRY_BATCH];
#pragma unroll
    for (int j = 0; j < ORDER_CARRY_BATCH; ++j) {
      const long slot = (long)bh * d.NC + min(n0 + j, d.NC - 1);
      local[j] = ends[slot * d.W + c];
      decay[j] = totals[slot];
    }
#pragma unroll
    for (int j = 0; j < ORDER_CARRY_BATCH; ++j)
      if (n0 + j < d.NC) {
        ends[((long)bh * d.NC + n0 + j) * d.W + c] = s;
        s = expf(decay[j]) * s + local[j];
      }
  }
}

// Forward pass 3: each chunk's scan from its start state.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void order_apply_kernel(OrderDims d, const float* values,
                                                          const float* log_decay,
                                                          const float* starts, float* output) {
  const OrderBlock o = order_block(d);
  const int c = threadIdx.x, cc = min(c, d.W - 1);
  const TokenGates gate(d, o, log_decay);
  const long stride = (long)d.H * d.W;
  const float* first = values + order_row(d, o.b, o.t0, o.h) * d.W + cc;
  RowGroup r[2];
  load_group(r[0], o, 0, first, stride);
  float s = starts[((long)o.bh * d.NC + o.n) * d.W + cc];
  float* out = output + order_row(d, o.b, o.t0, o.h) * d.W + c;
#pragma unroll
  for (int k = 0; k < ORDER_GROUPS; ++k) {
    if (k + 1 < ORDER_GROUPS) load_group(r[(k + 1) & 1], o, k + 1, first, stride);
#pragma unroll
    for (int i = 0; i < ORDER_GROUP; ++i) {
      const int t = k * ORDER_GROUP + i;
      s = lane_value(gate.lam, t) * s + lane_value(gate.inflow, t) * r[k & 1].x[i];
      if (t < o.len && c < d.W) out[t * stride] = s;
    }
  }
}

// Backward pass 1: the chunk's reverse scan of the cotangent from zero;
// heads[bh][n][c] = lam_first g_first (what reaches the previous chunk),
// totals[bh][n] = the chunk's summed log decay.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void order_bwd_local_kernel(OrderDims d, const float* d_output,
                                                              const float* log_decay,
                                                              float* heads, float* totals) {
  const OrderBlock o = order_block(d);
  const int c = threadIdx.x, cc = min(c, d.W - 1);
  const TokenGates gate(d, o, log_decay);
  const float g = gate.total();
  const long stride = (long)d.H * d.W;
  const float* first = d_output + order_row(d, o.b, o.t0, o.h) * d.W + cc;
  RowGroup r[2];
  load_group(r[1], o, ORDER_GROUPS - 1, first, stride);
  float acc = 0.f;
#pragma unroll
  for (int k = ORDER_GROUPS - 1; k >= 0; --k) {
    if (k > 0) load_group(r[(k - 1) & 1], o, k - 1, first, stride);
#pragma unroll
    for (int i = ORDER_GROUP - 1; i >= 0; --i) {
      const int t = k * ORDER_GROUP + i;
      acc = lane_value(gate.lam, t) * ((t < o.len ? r[k & 1].x[i] : 0.f) + acc);
    }
  }
  const long slot = (long)o.bh * d.NC + o.n;
  if (c < d.W) heads[slot * d.W + c] = acc;
  if (c == 0) totals[slot] = g;
}

// Backward pass 2, grid B*H: heads become the cotangent reaching each
// chunk's last token from later chunks (in place); what reaches the initial
// state is its gradient.
__global__ __launch_bounds__(256) void order_bwd_carry_kernel(OrderDims d, float* heads,
                                                              const float* totals,
                                                              float* d_initial) {
  const int bh = blockIdx.x, c = threadIdx.x;
  if (c >= d.W) return;
  float s = 0.f;
  for (int top = d.NC; top > 0; top -= ORDER_CARRY_BATCH) {
    float local[ORDER_CARRY_BATCH], decay[ORDER_CARRY_BATCH];
#pragma unroll
    for (int j = 0; j < ORDER_CARRY_BATCH; ++j) {
      const long slot = (long)bh * d.NC + max(top - 1 - j, 0);
      local[j] = heads[slot * d.W + c];
      decay[j] = totals[slot];
    }
#pragma unroll
    for (int j = 0; j < ORDER_CARRY_BATCH; ++j)
      if (top - 1 - j >= 0) {
        heads[((long)bh * d.NC + top - 1 - j) * d.W + c] = s;
        s = local[j] + expf(decay[j]) * s;
      }
  }
  if (d_initial) d_initial[(long)bh * d.W + c] = s;
}

constexpr int ORDER_MAX_WAVES = 4;  // W <= 256
constexpr int ORDER_HALF = MAXC / 2;

template <int CTRL>
__device__ __forceinline__ float order_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

// x[i] + x[i + half] exchanged with the lane whose bit `bit` differs, via a
// DPP pattern pairing exactly those lanes within a row: the lane with the
// bit set keeps (and sums) the upper element.
template <int CTRL, int BIT, int HALF>
__device__ __forceinline__ void dpp_stage(float (&x)[ORDER_HALF], int l) {
  const bool hi = (l >> BIT) & 1;
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    const float send = hi ? x[i] : x[i + HALF];
    const float keep = hi ? x[i + HALF] : x[i];
    x[i] = keep + order_dpp<CTRL>(send);
  }
}

// Sum over a wave's 64 lanes of x[0..31]: afterwards every lane holds the
// total of element l >> 1 (lane l).  A butterfly: each exchange halves the
// elements a lane keeps, selected by one lane bit.  Bits 5 and 4 exchange by
// v_permlane32_swap / v_permlane16_swap (the two results are the own and the
// partner's element of the kept half), bits 3..0 by DPP row_mirror (lane
// 15 - i), row_half_mirror (7 - i) and quad permutations, each pairing lanes
// that differ in that bit and agree in the bits above it.
__device__ __forceinline__ float wave_sums32(float (&x)[ORDER_HALF]) {
  const int l = lane_id();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[i]),
                                                    __float_as_uint(x[i + 16]), false, false);
    x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[i]),
                                                    __float_as_uint(x[i + 8]), false, false);
    x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  dpp_stage<0x140, 3, 4>(x, l);  // row_mirror
  dpp_stage<0x141, 2, 2>(x, l);  // row_half_mirror
  dpp_stage<0x4E, 1, 1>(x, l);   // quad_perm [2,3,0,1]
  return x[0] + order_dpp<0xB1>(x[0]);  // quad_perm [1,0,3,2]
}

// Backward pass 3: the chunk's reverse scan from the carried cotangent,
// d values, and d log_decay summed over channels (within each wave by the
// butterfly above, then over the waves in order).  Groups of the chunk from
// the last down, each loaded while the one after it is used.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void order_bwd_apply_kernel(
    OrderDims d, const float* values, const float* log_decay, const float* initial,
    const float* output, const float* d_output, const float* carried, float* d_values,
    float* d_log_decay) {
  __shared__ float part[ORDER_MAX_WAVES][MAXC];
  const OrderBlock o = order_block(d);
  const int c = threadIdx.x, wave = c >> 6, l = lane_id();
  const bool on = c < d.W;
  const int cc = min(c, d.W - 1);
  const TokenGates gate(d, o, log_decay);
  float acc = on ? carried[((long)o.bh * d.NC + o.n) * d.W + c] : 0.f;
  // The state before the chunk: the previous token's output, or the initial
  // state (zero when absent) before the first token.
  const float h_before = o.t0 > 0   ? output[order_row(d, o.b, o.t0 - 1, o.h) * d.W + cc]
                         : initial ? initial[(long)o.bh * d.W + cc]
                                   : 0.f;
  struct Group {
    float dy[ORDER_GROUP], v[ORDER_GROUP], prev[ORDER_GROUP];
  };
  auto load = [&](Group& r, int g) {
#pragma unroll
    for (int i = 0; i < ORDER_GROUP; ++i) {
      const int t = min(g * ORDER_GROUP + i, o.len - 1);
      const long row = order_row(d, o.b, o.t0 + t, o.h);
      r.dy[i] = d_output[row * d.W + cc];
      r.v[i] = values[row * d.W + cc];
      r.prev[i] = t > 0 ? output[(row - d.H) * d.W + cc] : h_before;
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  Group r[2];
  float term[ORDER_HALF];
  load(r[1], ORDER_GROUPS - 1);
#pragma unroll
  for (int k = ORDER_GROUPS - 1; k >= 0; --k) {
    if (k > 0) load(r[(k - 1) & 1], k - 1);
    const Group& cur = r[k & 1];
#pragma unroll
    for (int i = ORDER_GROUP - 1; i >= 0; --i) {
      const int t = k * ORDER_GROUP + i;
      const bool in = t < o.len && on;
      const float gt = (in ? cur.dy[i] : 0.f) + acc;
      if (in) d_values[order_row(d, o.b, o.t0 + t, o.h) * d.W + c] = lane_value(gate.inflow, t) * gt;
      term[t % ORDER_HALF] = in ? gt * (cur.prev[i] - cur.v[i]) : 0.f;
      acc = lane_value(gate.lam, t) * gt;
    }
    if (k % 2 == 0) {  // a half of the chunk is done
      const float sum = wave_sums32(term);
      if ((l & 1) == 0) part[wave][k / 2 * ORDER_HALF + (l >> 1)] = sum;
    }
  }
  __syncthreads();
  const int waves = (int)(blockDim.x >> 6);
  if (c < o.len) {  // wave 0: lane c holds token c's gate
    float sum = 0.f;
    for (int w = 0; w < waves; ++w) sum += part[w][c];
    d_log_decay[order_row(d, o.b, o.t0 + c, o.h)] = gate.lam * sum;
  }
}

}  // namespace m4
