/*
 * mamba3_scan.h -- C ABI of the MI355X (gfx950) Mamba-3 SISO scan in the
 * FlashMamba fused layout (the library that also holds mamba4_memread.h).
 *
 * Plain pointers and sizes only: every array is a contiguous float32 device
 * buffer in the layout named next to it, owned by the caller.  `stream` is
 * a hipStream_t passed as void* (NULL = the null stream).  No function
 * allocates, frees or synchronises.  Return values are those of
 * mamba4_memread.h (M4MR_OK, M4MR_EINVAL with nothing launched, M4MR_EHIP);
 * m4mr_last_error() gives the message.
 *
 * Shapes: B batch, T tokens, H heads (<= M3S_MAX_HEADS), N state width (even,
 * <= M3S_MAX_STATE), P value width per head (<= M3S_MAX_VALUE), A angle rates
 * (A <= N/2); chunks of M3S_CHUNK tokens, NC = ceil(T / M3S_CHUNK).
 * Limits: B*T*H*P and B*T*N below 2^31 elements, and NC * M3S_CHUNK below
 * 2^22 tokens (T <= 2^22 - 64; the backward addresses per-batch-row
 * partials with 32-bit byte offsets).
 * Alignment: c, b and the biases 8 bytes; x, d_y, starts 16 bytes.
 */
#ifndef MAMBA3_SCAN_H
#define MAMBA3_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3S_CHUNK 64
#define M3S_MAX_STATE 128
#define M3S_MAX_VALUE 64
#define M3S_MAX_HEADS 128
/* Floats of one stored chunk-start state (the state padded to 128 x 64). */
#define M3S_STATE_FLOATS 8192
/* Floats of one stored chunk-start phase (A padded to 64). */
#define M3S_PHASE_FLOATS 64

/*
 * Forward scan with residuals.
 *
 * Replaces mamba3_fused (lm/kernels/flashmamba.py:1125-1162) and the forward
 * of fused_scan's custom VJP, _fused_forward_pass / _fused_forward
 * (lm/kernels/flashmamba.py:938-997): the trapezoid weights gamma and scale
 * (:1146-1150) and the duplicated angle rates (:1113-1122) are formed inside.
 *
 * inputs   c, b [B,T,N] (queries and keys shared by the heads); x [B,T,H*P];
 *          adt, dt, trap_logits [B,T,H]; angles [B,T,A] (NULL if A = 0);
 *          q_bias, k_bias [H,N].
 * outputs  y [B,T,H*P]; final_state [B,H,N,P] (NULL: not written).
 * residuals starts [B,H,NC,M3S_STATE_FLOATS], each chunk's start state
 *          (the reference's `starts`, :976); phases [B,H,NC,M3S_PHASE_FLOATS],
 *          each chunk's start phase (the reference's `phase0`, :977).
 */
int m3s_forward(const float* c, const float* b, const float* x, const float* adt,
                const float* dt, const float* trap_logits, const float* angles,
                const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                int A, float* y, float* final_state, float* starts, float* phases, void* stream);

/*
 * m3s_forward for a bfloat16 model: c, b, x and y are bfloat16 (raw bits),
 * and every matrix product takes bfloat16 operands with float32
 * accumulation at the points where the reference's fused kernel rounds to
 * the model dtype (lm/kernels/flashmamba.py:575-586, 634-659): the
 * bias-added rows before their rotation, the rotated queries and keys, the
 * masked score mix, the carried state and the source-weighted values; y is
 * rounded once at the end.  The residuals and the final state stay float32
 * (:971-976).  Alignment: c, b 4 bytes, x 8 bytes.
 */
int m3s_forward_bf16(const uint16_t* c, const uint16_t* b, const uint16_t* x, const float* adt,
                     const float* dt, const float* trap_logits, const float* angles,
                     const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                     int A, uint16_t* y, float* final_state, float* starts, float* phases,
                     void* stream);

/* Bytes of the workspace m3s_backward needs for this shape. */
size_t m3s_backward_workspace_bytes(int B, int T, int H, int N, int P, int A);

/*
 * Backward: gradients of <y, d_y> + <final_state, d_final> for all nine
 * inputs.  Replaces _fused_backward (lm/kernels/flashmamba.py:1000-1108)
 * together with the autodiff of mamba3_fused's weight and angle-rate glue
 * (:1146-1162).
 *
 * inputs   the forward's inputs and residuals; d_y [B,T,H*P]; d_final
 *          [B,H,N,P] (NULL for zero).
 * outputs  d_c, d_b [B,T,N]; d_x [B,T,H*P]; d_adt, d_dt, d_trap [B,T,H];
 *          d_angles [B,T,A] (unused if A = 0); d_q_bias, d_k_bias [H,N].
 * workspace at least m3s_backward_workspace_bytes(...) bytes, 256-byte aligned.
 */
int m3s_backward(const float* c, const float* b, const float* x, const float* adt,
                 const float* dt, const float* trap_logits, const float* angles,
                 const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                 int A, const float* starts, const float* phases, const float* d_y,
                 const float* d_final, float* d_c, float* d_b, float* d_x, float* d_adt,
                 float* d_dt, float* d_trap, float* d_angles, float* d_q_bias, float* d_k_bias,
                 void* workspace, size_t workspace_bytes, void* stream);

/*
 * m3s_backward for a bfloat16 model (the residuals of m3s_forward_bf16):
 * c, b, x, d_y and d_x are bfloat16; the other gradients float32.  The
 * products round their operands as the reference's fused backward kernel
 * does (lm/kernels/flashmamba.py:721-751: the score mixes and their
 * cotangent, the e^p-scaled cotangent, the carried states), d_y having been
 * rounded to the model dtype (:1008).  Alignment: c, b 4 bytes, x, d_y 8.
 */
int m3s_backward_bf16(const uint16_t* c, const uint16_t* b, const uint16_t* x, const float* adt,
                      const float* dt, const float* trap_logits, const float* angles,
                      const float* q_bias, const float* k_bias, int B, int T, int H, int N,
                      int P, int A, const float* starts, const float* phases,
                      const uint16_t* d_y, const float* d_final, float* d_c, float* d_b,
                      uint16_t* d_x, float* d_adt, float* d_dt, float* d_trap, float* d_angles,
                      float* d_q_bias, float* d_k_bias, void* workspace, size_t workspace_bytes,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA3_SCAN_H */
