/*
 * mamba4_memread.h -- C ABI of the MI355X (gfx950) Mamba 4 memory read.
 *
 * Plain pointers and sizes only: every array is a contiguous float32 device
 * buffer in the layout named next to it, owned by the caller.  `stream` is
 * a hipStream_t passed as void* (NULL = the null stream).  No function
 * allocates or frees caller memory, synchronises the device, or keeps
 * state between calls other than an optional profiling log.  Functions are
 * reentrant; calls on one stream run in order.
 *
 * Shapes: B batch, T tokens, H heads, key width D = 64 (M4MR_KEY_DIM),
 * value width P = value_dim, 64 (M4MR_VALUE_DIM) or 128 (M4MR_MAX_VALUE_DIM,
 * the reference's trained memory_head_dim, lm/configs/mamba4-60m.json), chunk
 * c in [1, 64], NC = ceil(T / c) chunks.  Callers with narrower keys or
 * values pad them with zeros (and the floor with ones); the padded
 * coordinates then solve to zero and read nothing, as in
 * lm/kernels/mamba4_fused.py:292-297.
 *
 * Return value: 0 on success, M4MR_EINVAL for a bad argument (nothing is
 * launched), M4MR_EHIP for a HIP launch error.  m4mr_last_error() returns
 * the calling thread's last message.  A non-positive pivot (for example a
 * non-positive floor) is not an error: like the reference
 * (lm/kernels/mamba4_fused.py:111) it propagates NaN.
 */
#ifndef MAMBA4_MEMREAD_H
#define MAMBA4_MEMREAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M4MR_KEY_DIM 64
#define M4MR_VALUE_DIM 64
#define M4MR_MAX_VALUE_DIM 128
#define M4MR_MAX_CHUNK 64
/* Stored lower factor per token-head, 2176 floats: the lower triangle in
 * 16-byte column quads.  Row i = a + 16m (a < 16) holds quads 0..i/4; for
 * each row slot m and quad q the quads of rows a + 16m that hold it are
 * stored contiguously in increasing a, runs in increasing q, slots in
 * increasing m: row i's quad q is quad R(m,q) + a of the factor with
 * R(m,q) = 32m^2 + 8m + (q <= 4m ? 16q : 16(4m+1) + {-4, 4, 8}[q-4m-1]).
 * Entries above the diagonal inside a stored quad are zero.  The diagonal
 * holds the reciprocal pivot 1/L_ii (the reference keeps the same reciprocal
 * convention, lm/kernels/mamba4_fused.py:113).  The layout is private to the
 * residuals, as the reference's packing is (lm/kernels/mamba4_fused.py:36-42). */
#define M4MR_FACTOR_FLOATS 2176
/* Widest system m4mr_spd_solve takes (one block per system above 64). */
#define M4MR_SPD_MAX_DIM 4096

#define M4MR_OK 0
#define M4MR_EINVAL 1
#define M4MR_EHIP 2

/* Library version string, e.g. "mamba4_memread 0.1 gfx950". */
const char* m4mr_version(void);

/* Last error message of the calling thread ("" if none). */
const char* m4mr_last_error(void);

/*
 * Forward memory read, storing each token's factor (or not, see `factors`).
 *
 * Replaces selective_memory_fused (lm/kernels/mamba4_fused.py:372-454) and
 * the forward of its custom VJP, _chunk_solve_forward
 * (lm/kernels/mamba4_fused.py:329-337), behind selective_gaussian_memory
 * (lm/kernels/mamba4.py:228-262).
 *
 * inputs   keys, queries [B,T,H,D]; values [B,T,H,P]; beta, log_decay
 *          [B,T,H]; floor [H,D]; init_evidence [B,H,D,D] and init_cross
 *          [B,H,P,D] (both NULL for a zero initial state).
 * outputs  output [B,T,H,P]; variance [B,T,H]; final_evidence [B,H,D,D];
 *          final_cross [B,H,P,D].
 * residuals (what the backward consumes; the reference tags the
 *          equivalent arrays "memory_solve"):
 *          solved [B,T,H,D] (y_t = A_t^-1 q_t);
 *          factors [B,T,H,M4MR_FACTOR_FLOATS], or NULL: the forward then
 *          factors and solves without storing the factors, the reference's
 *          store_factors=False mode (lm/kernels/mamba4_fused.py:183-232,
 *          reached through the primal chunk_solve, :323-326) for forwards
 *          that take no gradient; every other output is bit-identical;
 *          start_evidence [B,H,NS,D,D], the evidence at the start of each
 *          sub-chunk (chunks above 32 tokens split in two halves of
 *          ceil(chunk/2) tokens, so NS = 2*NC, else NS = NC);
 *          start_cross [B,H,NC,P,D], the cross statistics at each chunk start.
 *          m4mr_start_counts() returns NC and NS.
 * The chunk-boundary states (here and in m4mr_backward) come from one fused
 * walk per (b, h) state sequence when B*H*(1 + P/64) reaches the device's
 * compute-unit count, else from chunk-parallel statistics plus a carry; the
 * environment variable M4MR_STATE_WALK=fused|split overrides the choice.
 * The fused walks run with one LDS step buffer (three per compute unit)
 * when they outnumber two per compute unit, else with two;
 * M4MR_STATE_BUFFERS=1|2 overrides that (the same results either way).
 * The factor kernel's two waves per pair hand the running evidence over
 * through a bounded wait (M4MR_TURN_POLLS polls, default 65536, about 2 ms);
 * a wait that gives up never yields a plausible wrong answer: every later
 * solution and factor of that block's sequences is NaN.
 * Numerics: the per-token Cholesky runs in fp32 except its trailing block
 * updates, whose fp32 panel values enter f16 MFMA products as hi + lo
 * pieces (three products per pair, exact in the fp32 sums, the dropped
 * lo*lo term below 2^-22 of each product).  A head whose largest floor lies
 * outside [2^-8, 2^8) is factored at a power-of-two scale that puts that
 * floor near 1 (exact), so the accuracy does not depend on the inputs'
 * magnitude; the f16 pieces overflow (NaN results) only for evidence above
 * 4.29e9 times the head's largest floor (rounded to a power of four).
 */
int m4mr_forward(const float* keys, const float* values, const float* queries,
                 const float* beta, const float* log_decay, const float* floor,
                 const float* init_evidence, const float* init_cross,
                 int B, int T, int H, int value_dim, int chunk,
                 float* output, float* variance,
                 float* final_evidence, float* final_cross,
                 float* solved, float* factors,
                 float* start_evidence, float* start_cross,
                 void* stream);

/*
 * m4mr_forward with bfloat16 keys, values and queries (raw 16-bit storage,
 * the caller's bf16 arrays), read and widened to float32 inside the
 * kernels; every other argument, the arithmetic and the outputs as in
 * m4mr_forward.  The reference upcasts bf16 inputs to float32 before the
 * memory read (lm/kernels/mamba4.py:263-265): results are identical to
 * m4mr_forward on the upcast arrays.
 */
int m4mr_forward_bf16(const uint16_t* keys, const uint16_t* values, const uint16_t* queries,
                      const float* beta, const float* log_decay, const float* floor,
                      const float* init_evidence, const float* init_cross,
                      int B, int T, int H, int value_dim, int chunk,
                      float* output, float* variance,
                      float* final_evidence, float* final_cross,
                      float* solved, float* factors,
                      float* start_evidence, float* start_cross,
                      void* stream);

/*
 * The mixer's per-head parameters and gates for m4mr_mixer_forward
 * (SelectiveMemoryMixer.__call__, lm/models/mamba4.py:183-237, 266-273).
 */
typedef struct {
  const float* beta_bias;        /* [H] */
  const float* dt_bias;          /* [H] */
  const float* a_log;            /* [H] */
  const float* floor_raw;        /* [H,D] */
  const float* previous;         /* [B,H,D] cached raw key of position 0, or NULL (zero key) */
  const float* confidence_scale; /* [H] */
  const float* skip;             /* [H], the mixer's D */
  float beta_max;                /* > 0 */
  float floor_min;               /* > 0 */
  int key_shift;                 /* nonzero: key t is the raw key of t - 1 */
} m4mr_mixer_params;

/*
 * The memory read fused with the mixer's prologue and read gating.  Equal
 * to m4mr_prologue_forward, then m4mr_forward, then m4mr_epilogue_forward
 * (to float32 rounding: the row norms are summed in another order), without
 * their separate passes over keys, queries and values: the memory-read
 * kernels shift and unit-normalise each raw key and query row as they load
 * it, the state walk computes the gates (beta, log_decay [B,T,H] and floor
 * [H,D], with the prologue's arithmetic) from the raw gate projections as
 * it first needs them and writes them out for the later kernels, and the
 * read kernel writes
 *   output = read * sigmoid(1 - confidence_scale[h] log1p(variance))
 *            + skip[h] * value
 * (lm/models/mamba4.py:266-273) as well as the ungated `read` (the
 * backward's residual).  Replaces, in the mixer's forward, the prologue at
 * lm/models/mamba4.py:183-237, the selective_gaussian_memory call at
 * :239-249 and the gating at :266-273.
 *
 * key, query [B,T,H,D] (D = 64) raw projections; value [B,T,H,P];
 * beta_raw, dt_raw [B,T,H]; outputs as m4mr_forward (output gated), plus
 * read [B,T,H,P].  With params->key_shift and a non-NULL `shifted`
 * [B,H,D], the raw key of position T-1 (the next call's `previous`) is
 * written there.  Always takes the fused state walk.
 */
int m4mr_mixer_forward(const float* key, const float* value, const float* query,
                       const float* beta_raw, const float* dt_raw,
                       const m4mr_mixer_params* params,
                       const float* init_evidence, const float* init_cross,
                       int B, int T, int H, int value_dim, int chunk,
                       float* output, float* read, float* variance,
                       float* beta, float* log_decay, float* floor,
                       float* final_evidence, float* final_cross,
                       float* solved, float* factors,
                       float* start_evidence, float* start_cross,
                       float* shifted, void* stream);

/*
 * Backward of the memory read inside m4mr_mixer_forward: m4mr_backward
 * with the raw keys and queries (and the key shift's `previous`, key_shift)
 * in place of the normalised ones, which bwd_dy and bwd_grads normalise as
 * they load them, and the forward's beta, log_decay and floor.  The
 * cotangents are those of the ungated read (d_read) and of the variance; the
 * gradients are those of m4mr_backward (with respect to the normalised keys
 * and queries and to the gates), for m4mr_prologue_backward to carry to the
 * raw projections.  No counterpart in the reference, whose autodiff takes
 * the same path through its prologue (lm/models/mamba4.py:183-237); it
 * saves the prologue's recomputation in the fused mixer's backward.
 * workspace as m4mr_backward.
 */
int m4mr_mixer_backward(const float* key, const float* value, const float* query,
                        const float* beta, const float* log_decay, const float* floor,
                        const float* previous, int key_shift,
                        int B, int T, int H, int value_dim, int chunk,
                        const float* solved, const float* factors,
                        const float* start_evidence, const float* start_cross,
                        const float* d_read, const float* d_variance,
                        const float* d_final_evidence, const float* d_final_cross,
                        float* d_keys, float* d_values, float* d_queries,
                        float* d_beta, float* d_log_decay, float* d_floor,
                        float* d_init_evidence, float* d_init_cross,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device workspace m4mr_mixer_read_backward needs for these sizes. */
size_t m4mr_mixer_read_backward_workspace_bytes(int B, int T, int H, int value_dim, int chunk);

/*
 * Backward of m4mr_mixer_forward as a whole: the VJP of the read gating
 * (m4mr_epilogue_backward), of the memory read from the raw keys and
 * queries (m4mr_mixer_backward) and of the prologue (m4mr_prologue_backward)
 * in one launch sequence.  The gating's VJP runs inside the first backward
 * kernel (it forms g d_output and the variance cotangent as it loads each
 * chunk), the prologue's inside the last (the unit normalisations' VJP to
 * the raw key and query rows, the gates' to beta_raw and dt_raw, per-chunk
 * partials of the per-head gradients); the state walk weighs the read's
 * cotangent by the gate.  Equal to the three calls in a row to float32
 * rounding (sums in another order).  Replaces, in the mixer's backward, the
 * VJP of lm/models/mamba4.py:183-273 that the reference's autodiff takes
 * through the prologue, selective_gaussian_memory and the gating.
 *
 * key, query [B,T,H,D] raw projections, value [B,T,H,P], dt_raw [B,T,H]
 * and params as given to m4mr_mixer_forward; read, variance, beta,
 * log_decay, floor, solved, factors, start_evidence, start_cross as it
 * returned them (factors stored).  Cotangents: d_output [B,T,H,P] of the
 * gated output (required), d_variance [B,T,H] (NULL: zero), the final
 * states' (NULL: zero) and d_shifted [B,H,D] of `shifted` (NULL: zero).
 * Gradients: d_key, d_query [B,T,H,D]; d_value [B,T,H,P]; d_beta_raw,
 * d_dt_raw [B,T,H]; d_beta_bias, d_dt_bias, d_a_log, d_confidence_scale,
 * d_skip [H]; d_floor_raw [H,D]; d_previous [B,H,D] (may be NULL; zero
 * without the key shift); d_init_evidence, d_init_cross as m4mr_backward.
 * workspace: m4mr_mixer_read_backward_workspace_bytes, 256-byte aligned.
 * Always takes the fused state walk.
 */
int m4mr_mixer_read_backward(const float* key, const float* value, const float* query,
                             const float* dt_raw, const m4mr_mixer_params* params,
                             int B, int T, int H, int value_dim, int chunk,
                             const float* read, const float* variance,
                             const float* beta, const float* log_decay, const float* floor,
                             const float* solved, const float* factors,
                             const float* start_evidence, const float* start_cross,
                             const float* d_output, const float* d_variance,
                             const float* d_final_evidence, const float* d_final_cross,
                             const float* d_shifted,
                             float* d_key, float* d_value, float* d_query,
                             float* d_beta_raw, float* d_dt_raw,
                             float* d_beta_bias, float* d_dt_bias, float* d_a_log,
                             float* d_floor_raw, float* d_previous,
                             float* d_confidence_scale, float* d_skip,
                             float* d_init_evidence, float* d_init_cross,
                             void* workspace, size_t workspace_bytes, void* stream);

/* Number of chunks NC and of evidence start states NS for T tokens. */
int m4mr_start_counts(int T, int chunk, int* chunks, int* evidence_starts);

/* Bytes of device workspace m4mr_backward needs for these sizes. */
size_t m4mr_backward_workspace_bytes(int B, int T, int H, int value_dim, int chunk);

/*
 * Backward of m4mr_forward: the VJP for every input and the initial state.
 *
 * Replaces _chunk_solve_backward (lm/kernels/mamba4_fused.py:340-366,
 * including _factored_kernel :155-174 for z = A^-1 g) together with the
 * JAX autodiff of the chunk glue around it (chunk statistics :411-415,
 * carry lm/kernels/prefix.py:27-44, prefix sums prefix.py:17-24 and reads
 * lm/kernels/mamba4_fused.py:439-447).  Only triangular solves with the
 * stored factors are used; nothing is refactored.
 *
 * cotangents d_output [B,T,H,P]; d_variance [B,T,H]; d_final_evidence
 *          [B,H,D,D] and d_final_cross [B,H,P,D] (NULL = zero).
 * gradients d_keys, d_queries [B,T,H,D]; d_values [B,T,H,P]; d_beta,
 *          d_log_decay [B,T,H]; d_floor [H,D]; d_init_evidence [B,H,D,D];
 *          d_init_cross [B,H,P,D].  The evidence cotangents are the
 *          symmetric form -(z y^T + y z^T)/2 of spd_solve's VJP
 *          (lm/kernels/mamba4.py:208-215).
 * workspace at least m4mr_backward_workspace_bytes(B, T, H, value_dim, chunk) bytes,
 *          256-byte aligned.
 */
int m4mr_backward(const float* keys, const float* values, const float* queries,
                  const float* beta, const float* log_decay, const float* floor,
                  int B, int T, int H, int value_dim, int chunk,
                  const float* solved, const float* factors,
                  const float* start_evidence, const float* start_cross,
                  const float* d_output, const float* d_variance,
                  const float* d_final_evidence, const float* d_final_cross,
                  float* d_keys, float* d_values, float* d_queries,
                  float* d_beta, float* d_log_decay, float* d_floor,
                  float* d_init_evidence, float* d_init_cross,
                  void* workspace, size_t workspace_bytes,
                  void* stream);

/*
 * m4mr_backward with bfloat16 keys, values and queries (as
 * m4mr_forward_bf16); the gradients are float32.
 */
int m4mr_backward_bf16(const uint16_t* keys, const uint16_t* values, const uint16_t* queries,
                       const float* beta, const float* log_decay, const float* floor,
                       int B, int T, int H, int value_dim, int chunk,
                       const float* solved, const float* factors,
                       const float* start_evidence, const float* start_cross,
                       const float* d_output, const float* d_variance,
                       const float* d_final_evidence, const float* d_final_cross,
                       float* d_keys, float* d_values, float* d_queries,
                       float* d_beta, float* d_log_decay, float* d_floor,
                       float* d_init_evidence, float* d_init_cross,
                       void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * m4mr_backward that allocates nothing and takes no workspace.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving and training loops
 * that allocate nothing per step, harnesses that forbid hipMalloc).  The
 * backward's intermediates (z, the end-state cotangents, the per-chunk floor
 * partials) live in a static device buffer of M4MR_STATIC_SCRATCH_BYTES
 * (128 MiB) that each GPU the library runs on holds until the process ends;
 * its address on a device is resolved at the first call on that device, so
 * make that first call outside any graph capture.  Its kernels use no
 * runtime-provided scratch either: it takes the backward state walk that
 * spills no registers, whatever the batch size or M4MR_STATE_BUFFERS.
 * Sizes whose m4mr_backward_workspace_bytes exceeds it return M4MR_EINVAL
 * before any launch (128 MiB holds B*T*H = 131072 token-heads at P = 64,
 * BASELINE config 2, with room to spare).  Every call on one GPU shares that
 * GPU's buffer: calls that overlap on one GPU (on different streams, or from
 * different threads without ordering) race and must not be issued.  Every
 * other argument and every result as in m4mr_backward (float32 keys, values
 * and queries).
 */
#define M4MR_STATIC_SCRATCH_BYTES (128u << 20)
int m4mr_backward_noalloc(const float* keys, const float* values, const float* queries,
                          const float* beta, const float* log_decay, const float* floor,
                          int B, int T, int H, int value_dim, int chunk,
                          const float* solved, const float* factors,
                          const float* start_evidence, const float* start_cross,
                          const float* d_output, const float* d_variance,
                          const float* d_final_evidence, const float* d_final_cross,
                          float* d_keys, float* d_values, float* d_queries,
                          float* d_beta, float* d_log_decay, float* d_floor,
                          float* d_init_evidence, float* d_init_cross,
                          void* stream);

/*
 * Triangular re-solve with stored factors: z_i = A_i^-1 rhs_i for N
 * token-heads, factors [N, M4MR_FACTOR_FLOATS], rhs and z [N, D] (z may
 * alias rhs).  Replaces factored_solve / _factored_kernel
 * (lm/kernels/mamba4_fused.py:316-320,155-174).
 */
int m4mr_factored_solve(const float* factors, const float* rhs, float* z,
                        long N, void* stream);

/*
 * One cached decode step, updating the state in place.
 *
 * Replaces selective_decode (lm/kernels/mamba4.py:341-355) for N = B*H
 * independent states: evidence [N,D,D] and cross [N,P,D] are read and
 * overwritten with lam*S + beta k k^T and lam*C + beta v k^T; key, query
 * [N,D]; value [N,P]; beta, log_decay [N]; floor [H,D] with head = n % H.
 * Writes output [N,P] = C y and variance [N] = q.y with
 * (S + diag(floor)) y = q.
 */
int m4mr_decode_step(float* evidence, float* cross,
                     const float* key, const float* value, const float* query,
                     const float* beta, const float* log_decay, const float* floor,
                     long N, int H, int value_dim,
                     float* output, float* variance, void* stream);

/*
 * Batched SPD solve: precision_n y_n = rhs_n for N systems of width dim
 * (1 <= dim <= M4MR_SPD_MAX_DIM).  precision [N,dim,dim] row-major, of
 * which only the lower triangle (column <= row) is read; rhs and solution
 * [N,dim].  When `factors` is non-NULL it receives each system's factor
 * [N, m4mr_spd_factor_floats(dim)], the residual m4mr_spd_solve_backward
 * consumes: for dim <= 64 the quad-run layout of M4MR_FACTOR_FLOATS (the
 * system padded to 64 with an identity block), above 64 the dense
 * [dim][dim] row-major factor (L below the diagonal, 1/L_ii on it, zero
 * above).  Above width 128 the factorization runs in `factors`, which is
 * then required; N < 2^31 above width 64.
 * Replaces spd_solve and its forward rule (lm/kernels/mamba4.py:190-201,
 * _factor_and_solve :164-187, which take any width); every reference
 * backend ("loop", "blocked", "unrolled", "auto", "fused") solves the same
 * system.
 */
int m4mr_spd_solve(const float* precision, const float* rhs, long N, int dim,
                   float* solution, float* factors, void* stream);

/*
 * Floats of one system's stored factor for m4mr_spd_solve at width dim:
 * M4MR_FACTOR_FLOATS up to 64, dim * dim above; 0 outside
 * 1..M4MR_SPD_MAX_DIM.  No counterpart in the reference, whose residual is
 * the JAX array itself (lm/kernels/mamba4.py:201).
 */
long m4mr_spd_factor_floats(int dim);

/*
 * VJP of m4mr_spd_solve (lm/kernels/mamba4.py:204-215): with
 * z = precision^-1 d_solution from the stored factors, writes
 * d_rhs = z [N,dim] and the full symmetric d_precision = -(z y^T + y z^T)/2
 * [N,dim,dim], y = solution.  No refactorization.
 */
int m4mr_spd_solve_backward(const float* factors, const float* solution,
                            const float* d_solution, long N, int dim,
                            float* d_precision, float* d_rhs, void* stream);

/*
 * Spectral and finiteness probes of a memory state: replaces
 * selective_diagnostics (lm/kernels/mamba4.py:358-376), which the mixer
 * calls on its final state when the "diagnostics" collection is mutable
 * (lm/models/mamba4.py:290-310).
 *
 * inputs   evidence [B,H,D,D], cross [B,H,P,D], floor [H,D] (1 <= D <= 64).
 * outputs  per_state [B,H,4]: for each (b, h) the smallest and largest
 *          eigenvalue of the symmetrised precision (E + E^T)/2 + diag(floor)
 *          (NaN when it has a non-finite entry), 1 if every entry of the
 *          state is finite else 0, and max |cross| (NaN if a cross entry is
 *          NaN);
 *          summary [7]: precision_min_eigenvalue, precision_max_eigenvalue,
 *          precision_max_condition (max over states of max / max(min,
 *          1e-30)), state_all_finite (1 / 0), cross_max_abs, floor_min,
 *          floor_max, in the reference's order.
 * The eigenvalues come from a cyclic Jacobi iteration in fp32, one wave per
 * state (absolute error about 1e-7 of the largest eigenvalue); the
 * reference's eigvalsh (LAPACK on the host, or its TPU lowering) has no
 * counterpart to call on the device.
 */
int m4mr_diagnostics(const float* evidence, const float* cross, const float* floor, int B, int H,
                     int D, int P, float* per_state, float* summary, void* stream);

/*
 * Mixer prologue: the memory read's inputs from the caller's projections.
 * Replaces the preprocessing inside SelectiveMemoryMixer.__call__
 * (lm/models/mamba4.py:183-237): with key_shift, position t of `keys` is
 * the raw key of t - 1 (position 0: `previous` [B,H,D], or zero when
 * previous is NULL), :183-195; keys and queries are unit-normalised,
 * x * rsqrt(sum x^2 + 1e-6) (_unit, :37-39); beta = beta_max *
 * sigmoid(beta_raw + beta_bias[h]) (:196-210); log_decay = -exp(a_log[h]) *
 * softplus(dt_raw + dt_bias[h]) (:211-221); floor = floor_min +
 * softplus(floor_raw) (:231-237).  key, query, keys, queries [B,T,H,D]
 * (D a multiple of 4); beta_raw, dt_raw, beta, log_decay [B,T,H];
 * beta_bias, dt_bias, a_log [H]; floor_raw, floor [H,D].  With key_shift and
 * a non-NULL `shifted` [B,H,D], the raw key of position T-1 (the cache entry
 * of the next call, :191-195) is written there.  beta_max and floor_min
 * must be positive (the reference raises ValueError otherwise).
 */
int m4mr_prologue_forward(const float* key, const float* query, const float* beta_raw,
                          const float* dt_raw, const float* beta_bias, const float* dt_bias,
                          const float* a_log, const float* floor_raw, const float* previous,
                          int B, int T, int H, int D, float beta_max, float floor_min,
                          int key_shift, float* keys, float* queries, float* beta,
                          float* log_decay, float* floor, float* shifted, void* stream);

/* Bytes of the workspace m4mr_prologue_backward and m4mr_epilogue_backward
 * need for their per-head partial sums. */
size_t m4mr_mixer_workspace_bytes(int B, int T, int H);

/*
 * VJP of m4mr_prologue_forward (the gradients JAX autodiff takes through
 * lm/models/mamba4.py:183-237).  Cotangents d_keys, d_queries, d_beta,
 * d_log_decay, d_floor and (with key_shift, may be NULL) d_shifted; writes
 * d_key, d_query [B,T,H,D], d_beta_raw, d_dt_raw [B,T,H], d_beta_bias,
 * d_dt_bias, d_a_log [H], d_floor_raw [H,D] and, if non-NULL, d_previous
 * [B,H,D] (zero when previous is NULL or without key_shift).  The per-head
 * sums run in a fixed order: results are identical run to run.
 */
int m4mr_prologue_backward(const float* key, const float* query, const float* beta_raw,
                           const float* dt_raw, const float* beta_bias, const float* dt_bias,
                           const float* a_log, const float* floor_raw, const float* previous,
                           int B, int T, int H, int D, float beta_max, int key_shift,
                           const float* d_keys, const float* d_queries, const float* d_beta,
                           const float* d_log_decay, const float* d_floor,
                           const float* d_shifted, float* d_key, float* d_query,
                           float* d_beta_raw, float* d_dt_raw, float* d_beta_bias,
                           float* d_dt_bias, float* d_a_log, float* d_floor_raw,
                           float* d_previous, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * Mixer epilogue: out = read * sigmoid(1 - confidence_scale[h] *
 * log1p(variance)) + skip[h] * value, the confidence gate and D-skip of
 * SelectiveMemoryMixer.__call__ (lm/models/mamba4.py:266-273).  read, value,
 * out [B,T,H,P] (P a multiple of 4); variance [B,T,H]; confidence_scale,
 * skip [H].
 */
int m4mr_epilogue_forward(const float* read, const float* variance, const float* value,
                          const float* confidence_scale, const float* skip, int B, int T, int H,
                          int P, float* out, void* stream);

/*
 * VJP of m4mr_epilogue_forward: d_read, d_value [B,T,H,P], d_variance
 * [B,T,H], d_confidence_scale, d_skip [H] (fixed-order per-head sums).
 */
int m4mr_epilogue_backward(const float* read, const float* variance, const float* value,
                           const float* confidence_scale, const float* skip, int B, int T, int H,
                           int P, const float* d_out, float* d_read, float* d_variance,
                           float* d_value, float* d_confidence_scale, float* d_skip,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * Order head scan: output[b,t,h,c] = h_t with h_t = lam_t h_(t-1) +
 * (1 - lam_t) values[b,t,h,c], lam_t = exp(log_decay[b,t,h]), the inflow
 * taken as -expm1(log_decay), from h_(-1) = initial[b,h,c] (zero when
 * initial is NULL).  Replaces order_memory_chunked
 * (lm/models/mamba4.py:59-95; order_memory :46-56 is the same scan from the
 * decays) and, over one token from the cached state, the order head's cached
 * step (:283-287).  values, output [B,T,H,W] with 1 <= W <= 256; log_decay
 * [B,T,H]; chunk 1..64 (the result does not depend on it beyond rounding).
 * workspace: m4mr_order_workspace_bytes(B, T, H, W, chunk) bytes, 256-byte
 * aligned (per-chunk carries).
 */
size_t m4mr_order_workspace_bytes(int B, int T, int H, int W, int chunk);
int m4mr_order_forward(const float* values, const float* log_decay, const float* initial,
                       int B, int T, int H, int W, int chunk, float* output, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * VJP of m4mr_order_forward (the gradients JAX autodiff takes through
 * order_memory_chunked): from `output` (the forward's) and d_output, writes
 * d_values [B,T,H,W], d_log_decay [B,T,H] (summed over channels in a fixed
 * order) and, if non-NULL, d_initial [B,H,W].
 */
int m4mr_order_backward(const float* values, const float* log_decay, const float* initial,
                        const float* output, const float* d_output, int B, int T, int H, int W,
                        int chunk, float* d_values, float* d_log_decay, float* d_initial,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Kernel timing with HIP events recorded on the launch stream.  While
 * enabled, every kernel launch is bracketed by a pair of events.
 * m4mr_profile_read() waits for the recorded events and returns the total
 * milliseconds and launch count of the kernels whose name equals `kernel`
 * (see m4mr_profile_kernel_name), then m4mr_profile_reset() clears them.
 */
void m4mr_profile_enable(int on);
/* Time only launches of `kernel` (NULL or "": every kernel). */
void m4mr_profile_select(const char* kernel);
void m4mr_profile_reset(void);
int m4mr_profile_read(const char* kernel, double* total_ms, long* launches);
/* Name of the i-th kernel the library launches, NULL past the end. */
const char* m4mr_profile_kernel_name(int i);

#ifdef __cplusplus
}
#endif

#endif /* MAMBA4_MEMREAD_H */
