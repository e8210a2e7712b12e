// The memory read's caller preprocessing and read gating
// (SelectiveMemoryMixer.__call__, lm/models/mamba4.py:183-237, 266-273).
//
// prologue_forward_kernel   key shift (each value written under the previous
//                           position's key, :183-195), unit normalisation of
//                           keys and queries (_unit, :37-39), the evidence
//                           gate beta = beta_max sigmoid(beta_raw + bias)
//                           (:196-210), log decay = -exp(a_log) softplus(dt_raw
//                           + dt_bias) (:211-221) and the floor floor_min +
//                           softplus(floor_raw) (:231-237).
// prologue_backward_kernel  its VJP per token-head, plus per-block partial sums
//                           of the per-head parameter gradients.
// epilogue_forward_kernel   read sigmoid(1 - scale log1p(variance)) + D value
//                           (:266-273).
// epilogue_backward_kernel  its VJP and per-block partials.
// head_sums_kernel          the per-head parameter gradients: the per-block
//                           partials summed in block order (deterministic).
//
// Every kernel takes 16 lanes per token-head (one 16-lane DPP row), so a
// 64-float row is one 16-byte access per lane; rows of other widths (a
// multiple of 4) loop over quads.  Rows are [B,T,H,width] and gates [B,T,H].
#include "common.hpp"

namespace m4 {

constexpr int MIX_ROWS = 16;  // token-heads per 256-thread block

__device__ __forceinline__ float sigmoidf(float x) { return mix_sigmoid(x); }
__device__ __forceinline__ float softplusf(float x) { return mix_softplus(x); }

// Sum over the 16 lanes of this thread's row; every lane receives the total.
__device__ __forceinline__ float row_sum(float x) { return row16_sum(x); }

// x * rsqrt(sum x^2 + 1e-6) for the row of `width` floats at `src` (null:
// a zero row); writes `dst`.  Lane l of the row holds quads l, l + 16, ...
__device__ void unit_row(const float* src, float* dst, int width, int l) {
  float s = 0.f;
  for (int c = 4 * l; c < width; c += 64) {
    const f4 v = src ? *reinterpret_cast<const f4*>(src + c) : f4{0.f, 0.f, 0.f, 0.f};
    s += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  }
  const float r = __builtin_amdgcn_rsqf(row_sum(s) + 1e-6f);
  for (int c = 4 * l; c < width; c += 64) {
    const f4 v = src ? *reinterpret_cast<const f4*>(src + c) : f4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<f4*>(dst + c) = v * r;
  }
}

// VJP of unit_row: r (dy - y (y . dy)) with y = x r.
__device__ void unit_row_vjp(const float* src, const float* dy, float* dx, int width, int l) {
  float s = 0.f;
  for (int c = 4 * l; c < width; c += 64) {
    const f4 v = src ? *reinterpret_cast<const f4*>(src + c) : f4{0.f, 0.f, 0.f, 0.f};
    s += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  }
  const float r = __builtin_amdgcn_rsqf(row_sum(s) + 1e-6f);
  float yd = 0.f;
  for (int c = 4 * l; c < width; c += 64) {
    const f4 v = src ? *reinterpret_cast<const f4*>(src + c) : f4{0.f, 0.f, 0.f, 0.f};
    const f4 g = *reinterpret_cast<const f4*>(dy + c);
    yd += r * (v[0] * g[0] + v[1] * g[1] + v[2] * g[2] + v[3] * g[3]);
  }
  yd = row_sum(yd);
  for (int c = 4 * l; c < width; c += 64) {
    const f4 v = src ? *reinterpret_cast<const f4*>(src + c) : f4{0.f, 0.f, 0.f, 0.f};
    const f4 g = *reinterpret_cast<const f4*>(dy + c);
    *reinterpret_cast<f4*>(dx + c) = r * (g - (r * yd) * v);
  }
}

// Token-head th = (b T + t) H + h of this thread's row, or -1 past the end.
struct MixRow {
  long th;
  int b, t, h, l;
};

__device__ __forceinline__ MixRow mix_row(int B, int T, int H) {
  MixRow r;
  r.th = (long)blockIdx.x * MIX_ROWS + (threadIdx.x >> 4);
  r.l = threadIdx.x & 15;
  const long n = (long)B * T * H;
  if (r.th >= n) {
    r.th = -1;
    r.b = r.t = r.h = 0;
    return r;
  }
  r.h = (int)(r.th % H);
  const long bt = r.th / H;
  r.t = (int)(bt % T);
  r.b = (int)(bt / T);
  return r;
}

// The source row of position t's key: key t - 1 with the shift (position 0:
// the cached `previous` key of this (b, h), or a zero row), else key t.
__device__ __forceinline__ const float* key_source(const float* key, const float* previous,
                                                   int key_shift, const MixRow& r, int T, int H,
                                                   int D) {
  if (!key_shift) return key + r.th * D;
  if (r.t > 0) return key + (r.th - H) * D;
  return previous ? previous + ((long)r.b * H + r.h) * D : nullptr;
}

__global__ __launch_bounds__(256) void prologue_forward_kernel(
    const float* __restrict__ key, const float* __restrict__ query,
    const float* __restrict__ beta_raw, const float* __restrict__ dt_raw,
    const float* __restrict__ beta_bias, const float* __restrict__ dt_bias,
    const float* __restrict__ a_log, const float* __restrict__ floor_raw,
    const float* __restrict__ previous, int B, int T, int H, int D, float beta_max,
    float floor_min, int key_shift, float* __restrict__ keys, float* __restrict__ queries,
    float* __restrict__ beta, float* __restrict__ log_decay, float* __restrict__ floor,
    float* __restrict__ shifted) {
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < H * D; i += blockDim.x)
      floor[i] = floor_min + softplusf(floor_raw[i]);
  const MixRow r = mix_row(B, T, H);
  if (r.th < 0) return;
  if (D == 64) {
    // One quad per lane, and every load issued before any arithmetic or
    // store (the general path below reads each row twice, one at a time).
    const float* ks = key_source(key, previous, key_shift, r, T, H, D);
    const int c = 4 * r.l;
    const f4 kraw = *reinterpret_cast<const f4*>((ks ? ks : query + r.th * D) + c);
    const f4 qv = *reinterpret_cast<const f4*>(query + r.th * D + c);
    const f4 kown = *reinterpret_cast<const f4*>(key + r.th * D + c);
    const float braw = beta_raw[r.th], draw = dt_raw[r.th];
    const float bb = beta_bias[r.h], db = dt_bias[r.h], al = a_log[r.h];
    const f4 kv = ks ? kraw : f4{0.f, 0.f, 0.f, 0.f};
    float sk = 0.f, sq = 0.f;
    sk += kv[0] * kv[0] + kv[1] * kv[1] + kv[2] * kv[2] + kv[3] * kv[3];
    sq += qv[0] * qv[0] + qv[1] * qv[1] + qv[2] * qv[2] + qv[3] * qv[3];
    const float rk = __builtin_amdgcn_rsqf(row_sum(sk) + 1e-6f);
    const float rq = __builtin_amdgcn_rsqf(row_sum(sq) + 1e-6f);
    *reinterpret_cast<f4*>(keys + r.th * D + c) = kv * rk;
    *reinterpret_cast<f4*>(queries + r.th * D + c) = qv * rq;
    if (key_shift && shifted && r.t == T - 1)
      *reinterpret_cast<f4*>(shifted + ((long)r.b * H + r.h) * D + c) = kown;
    if (r.l == 0) {
      beta[r.th] = beta_max * sigmoidf(braw + bb);
      log_decay[r.th] = -expf(al) * softplusf(draw + db);
    }
    return;
  }
  unit_row(key_source(key, previous, key_shift, r, T, H, D), keys + r.th * D, D, r.l);
  unit_row(query + r.th * D, queries + r.th * D, D, r.l);
  if (key_shift && shifted && r.t == T - 1)
    for (int c = 4 * r.l; c < D; c += 64)
      *reinterpret_cast<f4*>(shifted + ((long)r.b * H + r.h) * D + c) =
          *reinterpret_cast<const f4*>(key + r.th * D + c);
  if (r.l == 0) {
    beta[r.th] = beta_max * sigmoidf(beta_raw[r.th] + beta_bias[r.h]);
    log_decay[r.th] = -expf(a_log[r.h]) * softplusf(dt_raw[r.th] + dt_bias[r.h]);
  }
}

// The gates of the fused mixer read (m4mr_mixer_forward), one thread per
// token-head of [B,T,H]: the prologue's beta and log decay, and (block 0)
// its floor, with the same arithmetic; with a non-null `shifted`, the
// threads of position T-1 copy their raw key row there (the next call's
// cached key).
// Per-block partials of per-head sums: slot j of head h is the sum, in row
// order, of the values `v` of this block's rows of head h.  Lanes 0 of each
// row hold their row's values in vals[row][j].
template <int J>
__device__ void block_head_partials(float (*vals)[J], const long* ths, int H, float* part) {
  __syncthreads();
  for (int i = threadIdx.x; i < H * J; i += blockDim.x) {
    const int h = i / J, j = i % J;
    float s = 0.f;
    for (int row = 0; row < MIX_ROWS; ++row)
      if (ths[row] >= 0 && ths[row] % H == h) s += vals[row][j];
    part[(long)(h * J + j) * gridDim.x + blockIdx.x] = s;
  }
}

__global__ __launch_bounds__(256) void prologue_backward_kernel(
    const float* __restrict__ key, const float* __restrict__ query,
    const float* __restrict__ beta_raw, const float* __restrict__ dt_raw,
    const float* __restrict__ beta_bias, const float* __restrict__ dt_bias,
    const float* __restrict__ a_log, const float* __restrict__ floor_raw,
    const float* __restrict__ previous, int B, int T, int H, int D, float beta_max,
    int key_shift, const float* __restrict__ d_keys, const float* __restrict__ d_queries,
    const float* __restrict__ d_beta, const float* __restrict__ d_log_decay,
    const float* __restrict__ d_floor, const float* __restrict__ d_shifted,
    float* __restrict__ d_key, float* __restrict__ d_query, float* __restrict__ d_beta_raw,
    float* __restrict__ d_dt_raw, float* __restrict__ d_floor_raw,
    float* __restrict__ d_previous, float* __restrict__ part) {
  __shared__ float vals[MIX_ROWS][3];
  __shared__ long ths[MIX_ROWS];
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < H * D; i += blockDim.x)
      d_floor_raw[i] = d_floor[i] * sigmoidf(floor_raw[i]);
  const MixRow r = mix_row(B, T, H);
  const int row = threadIdx.x >> 4;
  if (r.l == 0) ths[row] = r.th;
  if (r.th >= 0 && D == 64) {
    // One quad per lane, every load issued before any arithmetic or store;
    // the same arithmetic, in the same order, as the general path below.
    const int c = 4 * r.l;
    const float* ks = key_source(key, previous, key_shift, r, T, H, D);
    const float* gs = d_shifted ? d_shifted + ((long)r.b * H + r.h) * D : d_queries + r.th * D;
    const f4 kraw = *reinterpret_cast<const f4*>((ks ? ks : query + r.th * D) + c);
    const f4 gk = *reinterpret_cast<const f4*>(d_keys + r.th * D + c);
    const f4 qv = *reinterpret_cast<const f4*>(query + r.th * D + c);
    const f4 gq = *reinterpret_cast<const f4*>(d_queries + r.th * D + c);
    const f4 graw = *reinterpret_cast<const f4*>(gs + c);
    const float braw = beta_raw[r.th], bb = beta_bias[r.h], dbeta = d_beta[r.th];
    const float draw = dt_raw[r.th], dtb = dt_bias[r.h], al = a_log[r.h];
    const float dl = d_log_decay[r.th];
    const f4 kv = ks ? kraw : f4{0.f, 0.f, 0.f, 0.f};
    auto vjp = [&](const f4& v, const f4& g) {
      float sum = 0.f, yd = 0.f;
      sum += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
      const float rn = __builtin_amdgcn_rsqf(row_sum(sum) + 1e-6f);
      yd += rn * (v[0] * g[0] + v[1] * g[1] + v[2] * g[2] + v[3] * g[3]);
      yd = row_sum(yd);
      return rn * (g - (rn * yd) * v);
    };
    const f4 dk = vjp(kv, gk), dq = vjp(qv, gq);
    float* dst = nullptr;
    if (!key_shift)
      dst = d_key + r.th * D;
    else if (r.t > 0)
      dst = d_key + (r.th - H) * D;
    else if (d_previous)
      dst = d_previous + ((long)r.b * H + r.h) * D;
    if (dst) *reinterpret_cast<f4*>(dst + c) = ks ? dk : f4{0.f, 0.f, 0.f, 0.f};
    if (key_shift && r.t == T - 1)
      *reinterpret_cast<f4*>(d_key + r.th * D + c) = d_shifted ? graw : f4{0.f, 0.f, 0.f, 0.f};
    *reinterpret_cast<f4*>(d_query + r.th * D + c) = dq;
    if (r.l == 0) {
      const float sg = sigmoidf(braw + bb);
      const float db = dbeta * beta_max * sg * (1.f - sg);
      const float u = draw + dtb;
      const float rate = expf(al);
      const float ddt = -dl * rate * sigmoidf(u);
      d_beta_raw[r.th] = db;
      d_dt_raw[r.th] = ddt;
      vals[row][0] = db;
      vals[row][1] = ddt;
      vals[row][2] = -dl * rate * softplusf(u);
    }
  } else if (r.th >= 0) {
    // The key row that fed position t's key gets its cotangent: key t - 1
    // (or the cached previous key at t = 0) with the shift, else key t.
    float* dst = nullptr;
    if (!key_shift)
      dst = d_key + r.th * D;
    else if (r.t > 0)
      dst = d_key + (r.th - H) * D;
    else if (d_previous)
      dst = d_previous + ((long)r.b * H + r.h) * D;
    if (dst && (!key_shift || r.t > 0 || previous)) {
      unit_row_vjp(key_source(key, previous, key_shift, r, T, H, D), d_keys + r.th * D, dst, D,
                   r.l);
    } else if (dst) {
      // No cached key fed position 0 (a zero row): its cotangent is zero.
      for (int c = 4 * r.l; c < D; c += 64)
        *reinterpret_cast<f4*>(dst + c) = f4{0.f, 0.f, 0.f, 0.f};
    }
    // With the shift, the last raw key feeds only the cache entry.
    if (key_shift && r.t == T - 1)
      for (int c = 4 * r.l; c < D; c += 64)
        *reinterpret_cast<f4*>(d_key + r.th * D + c) =
            d_shifted ? *reinterpret_cast<const f4*>(d_shifted + ((long)r.b * H + r.h) * D + c)
                      : f4{0.f, 0.f, 0.f, 0.f};
    unit_row_vjp(query + r.th * D, d_queries + r.th * D, d_query + r.th * D, D, r.l);
    if (r.l == 0) {
      const float s = sigmoidf(beta_raw[r.th] + beta_bias[r.h]);
      const float db = d_beta[r.th] * beta_max * s * (1.f - s);
      const float u = dt_raw[r.th] + dt_bias[r.h];
      const float rate = expf(a_log[r.h]);
      const float dl = d_log_decay[r.th];
      const float ddt = -dl * rate * sigmoidf(u);
      d_beta_raw[r.th] = db;
      d_dt_raw[r.th] = ddt;
      vals[row][0] = db;
      vals[row][1] = ddt;
      vals[row][2] = -dl * rate * softplusf(u);
    }
  }
  block_head_partials<3>(vals, ths, H, part);
}

__global__ __launch_bounds__(256) void epilogue_forward_kernel(
    const float* __restrict__ read, const float* __restrict__ variance,
    const float* __restrict__ value, const float* __restrict__ confidence_scale,
    const float* __restrict__ skip, int B, int T, int H, int P, float* __restrict__ out) {
  const MixRow r = mix_row(B, T, H);
  if (r.th < 0) return;
  const float g = sigmoidf(1.f - confidence_scale[r.h] * log1pf(variance[r.th]));
  const float dv = skip[r.h];
  for (int c = 4 * r.l; c < P; c += 64) {
    const f4 x = *reinterpret_cast<const f4*>(read + r.th * P + c);
    const f4 v = *reinterpret_cast<const f4*>(value + r.th * P + c);
    *reinterpret_cast<f4*>(out + r.th * P + c) = g * x + dv * v;
  }
}

__global__ __launch_bounds__(256) void epilogue_backward_kernel(
    const float* __restrict__ read, const float* __restrict__ variance,
    const float* __restrict__ value, const float* __restrict__ confidence_scale,
    const float* __restrict__ skip, int B, int T, int H, int P, const float* __restrict__ d_out,
    float* __restrict__ d_read, float* __restrict__ d_variance, float* __restrict__ d_value,
    float* __restrict__ part) {
  __shared__ float vals[MIX_ROWS][2];
  __shared__ long ths[MIX_ROWS];
  const MixRow r = mix_row(B, T, H);
  const int row = threadIdx.x >> 4;
  if (r.l == 0) ths[row] = r.th;
  if (r.th >= 0) {
    const float scale = confidence_scale[r.h], var = variance[r.th];
    const float lv = log1pf(var);
    const float g = sigmoidf(1.f - scale * lv);
    const float dv = skip[r.h];
    float dot = 0.f, dskip = 0.f;
    for (int c = 4 * r.l; c < P; c += 64) {
      const f4 x = *reinterpret_cast<const f4*>(read + r.th * P + c);
      const f4 v = *reinterpret_cast<const f4*>(value + r.th * P + c);
      const f4 d = *reinterpret_cast<const f4*>(d_out + r.th * P + c);
      *reinterpret_cast<f4*>(d_read + r.th * P + c) = g * d;
      *reinterpret_cast<f4*>(d_value + r.th * P + c) = dv * d;
      dot += d[0] * x[0] + d[1] * x[1] + d[2] * x[2] + d[3] * x[3];
      dskip += d[0] * v[0] + d[1] * v[1] + d[2] * v[2] + d[3] * v[3];
    }
    dot = row_sum(dot);
    dskip = row_sum(dskip);
    const float slope = dot * g * (1.f - g);
    if (r.l == 0) {
      d_variance[r.th] = slope * (-scale / (1.f + var));
      vals[row][0] = -slope * lv;
      vals[row][1] = dskip;
    }
  }
  block_head_partials<2>(vals, ths, H, part);
}

// o_j[h] = sum over blocks of part[(h * J + j) * blocks + block], in a fixed
// order: one 1024-thread block per (h, j); thread i sums blocks i, i + 1024,
// ... in order (eight loads in flight), then the 1024 partials are added in
// a fixed tree.  Results are identical run to run.
constexpr int HEAD_SUM_THREADS = 1024;

__global__ __launch_bounds__(HEAD_SUM_THREADS) void head_sums_kernel(
    const float* __restrict__ part, long blocks, int H, int J, float* __restrict__ o0,
    float* __restrict__ o1, float* __restrict__ o2) {
  const int h = blockIdx.x / J, j = blockIdx.x % J;
  __shared__ float red[HEAD_SUM_THREADS];
  const float* src = part + (long)(h * J + j) * blocks;
  float s = 0.f;
  for (long i0 = threadIdx.x; i0 < blocks; i0 += 8L * HEAD_SUM_THREADS) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const long i = i0 + (long)k * HEAD_SUM_THREADS;
      v[k] = i < blocks ? src[i] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) s += v[k];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = HEAD_SUM_THREADS / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float* o = j == 0 ? o0 : j == 1 ? o1 : o2;
    if (o) o[h] = red[0];
  }
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ x, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) x[i] = 0.f;
}

}  // namespace m4
