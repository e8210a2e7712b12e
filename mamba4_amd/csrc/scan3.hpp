// Shapes and kernel declarations of the gfx950 Mamba-3 scan (scan3.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace m3 {

typedef unsigned short bf16_t;  // bfloat16 bits

constexpr int C = 64;       // tokens per chunk (one per lane of a wave)
constexpr int NT = 128;     // state rows held (N <= NT; padding is zero)
constexpr int PT = 64;      // value columns held (P <= PT; padding is zero)
constexpr int AM = 64;      // angle slots (A <= N / 2 <= AM)
constexpr int LQ = NT + 4;  // LDS row stride of [C][NT] tiles
constexpr int LV = PT + 4;  // LDS row stride of [C][PT], [C][C] and [NT][PT] tiles
constexpr int LA = AM + 1;  // LDS row stride of [C][AM] phase tables

// B batch, T tokens, H heads, N state width, P value width, A angle rates,
// NC = ceil(T / C) chunks.
struct Shape {
  int B, T, H, N, P, A, NC;
};

// Outputs and per-chunk partials of grad_kernel (workspace except dx, d_adt).
struct GradOut {
  void* dx;         // [B,T,H*P] in the model dtype of x
  float* d_adt;     // [B,T,H]
  float* dgam;      // [B,T,H]  gradient of gamma (diagonal weight and scale)
  float* dscale;    // [B,T,H]  gradient of scale alone
  float* ddt_loc;   // [B,T,H]  phase gradient through dt within the chunk
  float* D;         // [B,H,NC,AM] phase-gradient total of each chunk
  float* qb_part;   // [B,NC,H,NT] query-bias gradient of each chunk
  float* kb_part;   // [B,NC,H,NT]
  float* dc_part;   // [G,B,NC*C,NT] query-row gradient of each head group
  float* db_part;   // [G,B,NC*C,NT]
  float* dang_part; // [G,B,NC*C,AM] angle gradient (chunk-local part)
};

// LDS bytes of each kernel.
constexpr size_t kWalkLds = (size_t)(C * (64 + 4) + C * LV + C * LA + AM + 384) * sizeof(float);
constexpr size_t kOutLds = (size_t)(2 * C * LQ + NT * LV + C * LV + AM + 384) * sizeof(float);
// out_kernel with bfloat16 tiles: Q, K, H0 [.][NT + 8] and V [PT][PT + 8] in
// bfloat16 (the phase table, C * (AM + 1) floats, fits in H0's tile).
constexpr size_t kOutLdsBf16 =
    (size_t)(3 * C * (NT + 8) + PT * (PT + 8)) * 2 + (size_t)(AM + 384) * sizeof(float);
static_assert((size_t)C * (NT + 8) * 2 >= (size_t)C * (AM + 1) * sizeof(float),
              "the phase table fits in H0's bfloat16 tile");
constexpr size_t kGradLds = (size_t)(4 * NT * LV + C * LA + AM + 1352) * sizeof(float);
// finish_kernel: blocks per (b, chunk); [H][LA] + [C][A + 1] + [C][H + 1]
// floats of LDS, at most this.
constexpr int kFinishParts = 8;
constexpr int kMaxHeads = 128;
constexpr size_t kFinishLdsMax =
    (size_t)(kMaxHeads * LA + C * (AM + 1) + C * (kMaxHeads + 1)) * sizeof(float);
inline size_t finish_lds(int H, int A) {
  return (size_t)(H * LA + C * (A + 1) + C * (H + 1)) * sizeof(float);
}

// In: the model dtype of the rows, values and their cotangents (float, or
// bf16_t with the reference's bfloat16 matrix operands).  V4: the value width
// P is a multiple of 4 (vector loads of value rows; otherwise per element).
template <bool BWD, typename In, bool V4>
__global__ void walk_kernel(Shape, const In*, const float*, const In*, const float*,
                            const float*, const float*, const float*, float*, float*,
                            const float*, float*);
template <typename In, bool V4>
__global__ void out_kernel(Shape, const In*, const In*, const In*, const float*, const float*,
                           const float*, const float*, const float*, const float*, const float*,
                           const float*, In*);
template <typename In, bool V4>
__global__ void grad_kernel(Shape, int, const In*, const In*, const In*, const float*,
                            const float*, const float*, const float*, const float*, const float*,
                            const float*, const float*, const float*, const In*, GradOut);
__global__ void finish_kernel(Shape, int, const float*, const float*, const float*, GradOut,
                              float*, float*, float*, float*, float*);
__global__ void suffix_kernel(Shape, GradOut);
__global__ void bias_kernel(Shape, GradOut, float*, float*);

}  // namespace m3
