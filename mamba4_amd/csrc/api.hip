// C ABI of the gfx950 memory read (declared in include/mamba4_memread.h).
//
// Each entry point validates its arguments on the host, then launches a
// fixed sequence of kernels on the caller's stream.  Nothing here allocates
// device memory or synchronises; the only global state is the optional
// profiling log (mutex-protected) and a per-thread error message.
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/mamba3_scan.h"
#include "../../include/mamba4_memread.h"
#include "common.hpp"
#include "scan3.hpp"

namespace m4 {
template <typename In>
__global__ void fwd_stats_kernel(Dims, const In*, const In*, const float*, const float*, float*,
                                 float*);
__global__ void fwd_scan_kernel(Dims, const float*, const float*, const float*, float*, float*,
                                float*, float*);
__global__ void bwd_local_kernel(Dims, const float*, const float*, const float*, const float*,
                                 const float*, float*, float*);
__global__ void bwd_scan_kernel(Dims, const float*, const float*, const float*, float*, float*,
                                float*, float*);
template <bool BWD, typename In, bool MIX, int NBUF>
__global__ void states_kernel(Dims, StateArgs);
template <typename In, bool MIX, bool STORE, int PAIRS>
__global__ void fwd_factor_kernel(Dims, const In*, const In*, const float*, const float*,
                                  const float*, const float*, float*, float*, MixerIn, int);
__global__ void factored_solve_kernel(const float*, const float*, float*, long);
__global__ void decode_step_kernel(float*, float*, const float*, const float*, const float*,
                                   const float*, const float*, const float*, long, int, int, float*,
                                   float*);
template <typename In, bool MIX, int NV>
__global__ void fwd_read_kernel(Dims, const In*, const In*, const In*, const float*,
                                const float*, const float*, const float*, float*, float*, MixerIn,
                                ReadGate);
template <typename In, bool MIX, bool GATE, int NV>
__global__ void bwd_dy_kernel(Dims, const In*, const In*, const In*, const float*,
                              const float*, const float*, const float*, const float*, float*,
                              MixerIn, MixerGrad);
template <typename In, bool MIX, bool GATE, int NV>
__global__ void bwd_grads_kernel(Dims, const In*, const In*, const float*, const float*,
                                 const float*, const float*, const float*, const float*,
                                 const float*, const float*, const float*, const float*, float*,
                                 float*, float*, float*, float*, float*, MixerIn, MixerGrad);
__global__ void floor_reduce_kernel(Dims, const float*, float*, const float*);
__global__ void mixer_finish_kernel(Dims, const float*, float*, const float*, const float*,
                                    const float*, float*, float*, float*, float*, float*);
__global__ void prologue_forward_kernel(const float*, const float*, const float*, const float*,
                                        const float*, const float*, const float*, const float*,
                                        const float*, int, int, int, int, float, float, int,
                                        float*, float*, float*, float*, float*, float*);
__global__ void prologue_backward_kernel(const float*, const float*, const float*, const float*,
                                         const float*, const float*, const float*, const float*,
                                         const float*, int, int, int, int, float, int,
                                         const float*, const float*, const float*, const float*,
                                         const float*, const float*, float*, float*, float*,
                                         float*, float*, float*, float*);
__global__ void epilogue_forward_kernel(const float*, const float*, const float*, const float*,
                                        const float*, int, int, int, int, float*);
__global__ void epilogue_backward_kernel(const float*, const float*, const float*, const float*,
                                         const float*, int, int, int, int, const float*, float*,
                                         float*, float*, float*);
__global__ void head_sums_kernel(const float*, long, int, int, float*, float*, float*);
__global__ void zero_kernel(float*, long);
__global__ void order_local_kernel(OrderDims, const float*, const float*, float*, float*);
__global__ void order_carry_kernel(OrderDims, const float*, float*, const float*);
__global__ void order_apply_kernel(OrderDims, const float*, const float*, const float*, float*);
__global__ void order_bwd_local_kernel(OrderDims, const float*, const float*, float*, float*);
__global__ void order_bwd_carry_kernel(OrderDims, float*, const float*, float*);
__global__ void order_bwd_apply_kernel(OrderDims, const float*, const float*, const float*,
                                       const float*, const float*, const float*, float*, float*);
__global__ void spd_solve_kernel(const float*, const float*, long, int, float*, float*);
__global__ void spd_backward_kernel(const float*, const float*, const float*, long, int, float*,
                                    float*);
template <bool LDS>
__global__ void spd_wide_kernel(const float*, const float*, int, float*, float*);
template <bool LDS>
__global__ void spd_wide_backward_kernel(const float*, const float*, const float*, int, float*,
                                         float*);
__global__ void diag_eigen_kernel(const float*, const float*, const float*, int, int, int, float*);
__global__ void diag_summary_kernel(const float*, int, const float*, int, float*);
}  // namespace m4

namespace {

using m4::Dims;

thread_local std::string g_error;

const char* const kKernelNames[] = {"fwd_stats",      "fwd_scan",  "fwd_states", "fwd_factor",
                                    "fwd_read",       "bwd_dy",    "factored_solve",
                                    "bwd_local",      "bwd_scan",  "bwd_states",
                                    "bwd_grads",      "floor_reduce", "decode_step",
                                    "spd_solve",      "spd_backward", "prologue_forward",
                                    "prologue_backward", "epilogue_forward",
                                    "epilogue_backward", "head_sums", "order_local",
                                    "order_carry",    "order_apply", "order_bwd_local",
                                    "order_bwd_carry", "order_bwd_apply",
                                    "m3_walk",        "m3_out",    "m3_walk_bwd", "m3_grad",
                                    "m3_finish",      "m3_bias",   "m3_suffix",
                                    "mixer_finish",   "diag_eigen", "diag_summary",
                                    "spd_wide",       "spd_wide_backward"};

struct ProfRecord {
  const char* name;
  hipEvent_t start, stop;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::string g_prof_only;         // empty: every kernel is timed
std::vector<ProfRecord> g_prof;
std::vector<hipEvent_t> g_event_pool;  // events of cleared records, reused

// An event from the pool, or a new one (called with g_prof_mu held).
hipError_t take_event(hipEvent_t* e) {
  if (!g_event_pool.empty()) {
    *e = g_event_pool.back();
    g_event_pool.pop_back();
    return hipSuccess;
  }
  return hipEventCreate(e);
}

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

constexpr size_t kStatsLdsBytes = 3 * m4::TILE * sizeof(float);
constexpr size_t kChunkLdsBytes = 4 * m4::TILE * sizeof(float);
constexpr size_t kGradsLdsBytes = 7 * m4::TILE * sizeof(float);
constexpr size_t kGradsGateLdsBytes = 8 * m4::TILE * sizeof(float);  // + the S0 tile
constexpr size_t kStatesLdsBytes = 4 * m4::TILE * sizeof(float);
// The backward walks add one tile (the evidence state's transpose).
constexpr size_t kStatesBwdExtra = m4::TILE * sizeof(float);
// The widest LDS request of the wide SPD solves (an LDS-resident 128-wide
// system, or the vectors of a 4096-wide one).
constexpr size_t kWideLdsMax =
    sizeof(float) * (m4::wide_lds_floats(m4::kWideLdsDim) > m4::wide_lds_floats(m4::kWideMaxDim)
                         ? m4::wide_lds_floats(m4::kWideLdsDim)
                         : m4::wide_lds_floats(m4::kWideMaxDim));

bool configured = false;
int g_cus = 256;  // compute units of the device (set by configure())
std::mutex g_cfg_mu;

// Grid of a persistent chunk kernel: `per_cu` resident blocks per compute
// unit, never more blocks than chunks.
unsigned persistent_grid(unsigned chunks, int per_cu) {
  const unsigned cap = (unsigned)(g_cus * per_cu);
  return chunks < cap ? chunks : cap;
}

int configure() {
  std::lock_guard<std::mutex> lock(g_cfg_mu);
  if (configured) return M4MR_OK;
  struct {
    const void* fn;
    size_t bytes;
  } big[] = {{(const void*)m4::fwd_stats_kernel<float>, kStatsLdsBytes},
             {(const void*)m4::fwd_stats_kernel<m4::bf16_t>, kStatsLdsBytes},
             {(const void*)m4::bwd_local_kernel, kChunkLdsBytes},
#define M4_CHUNK_ATTRS(NV)                                                                    \
  {(const void*)m4::fwd_read_kernel<float, false, NV>, kChunkLdsBytes},                       \
      {(const void*)m4::fwd_read_kernel<m4::bf16_t, false, NV>, kChunkLdsBytes},              \
      {(const void*)m4::fwd_read_kernel<float, true, NV>, kChunkLdsBytes},                    \
      {(const void*)m4::bwd_dy_kernel<float, false, false, NV>, kChunkLdsBytes},              \
      {(const void*)m4::bwd_dy_kernel<m4::bf16_t, false, false, NV>, kChunkLdsBytes},         \
      {(const void*)m4::bwd_dy_kernel<float, true, false, NV>, kChunkLdsBytes},               \
      {(const void*)m4::bwd_dy_kernel<float, true, true, NV>, kChunkLdsBytes},                \
      {(const void*)m4::bwd_grads_kernel<float, false, false, NV>, kGradsLdsBytes},           \
      {(const void*)m4::bwd_grads_kernel<m4::bf16_t, false, false, NV>, kGradsLdsBytes},      \
      {(const void*)m4::bwd_grads_kernel<float, true, false, NV>, kGradsLdsBytes},            \
      {(const void*)m4::bwd_grads_kernel<float, true, true, NV>, kGradsGateLdsBytes}
             M4_CHUNK_ATTRS(1),
             M4_CHUNK_ATTRS(2),
#undef M4_CHUNK_ATTRS
             {(const void*)m4::states_kernel<false, float, false, 2>, kStatesLdsBytes},
             {(const void*)m4::states_kernel<false, m4::bf16_t, false, 2>, kStatesLdsBytes},
             {(const void*)m4::states_kernel<true, float, false, 2>,
              kStatesLdsBytes + kStatesBwdExtra},
             {(const void*)m4::states_kernel<false, float, true, 2>, kStatesLdsBytes},
             {(const void*)m4::states_kernel<true, float, true, 2>,
              kStatesLdsBytes + kStatesBwdExtra},
             {(const void*)m3::walk_kernel<false, float, true>, m3::kWalkLds},
             {(const void*)m3::walk_kernel<true, float, true>, m3::kWalkLds},
             {(const void*)m3::out_kernel<float, true>, m3::kOutLds},
             {(const void*)m3::grad_kernel<float, true>, m3::kGradLds},
             {(const void*)m3::walk_kernel<false, m3::bf16_t, true>, m3::kWalkLds},
             {(const void*)m3::walk_kernel<true, m3::bf16_t, true>, m3::kWalkLds},
             {(const void*)m3::out_kernel<m3::bf16_t, true>, m3::kOutLdsBf16},
             {(const void*)m3::grad_kernel<m3::bf16_t, true>, m3::kGradLds},
             {(const void*)m3::walk_kernel<false, float, false>, m3::kWalkLds},
             {(const void*)m3::walk_kernel<true, float, false>, m3::kWalkLds},
             {(const void*)m3::out_kernel<float, false>, m3::kOutLds},
             {(const void*)m3::grad_kernel<float, false>, m3::kGradLds},
             {(const void*)m3::walk_kernel<false, m3::bf16_t, false>, m3::kWalkLds},
             {(const void*)m3::walk_kernel<true, m3::bf16_t, false>, m3::kWalkLds},
             {(const void*)m3::out_kernel<m3::bf16_t, false>, m3::kOutLdsBf16},
             {(const void*)m3::grad_kernel<m3::bf16_t, false>, m3::kGradLds},
             {(const void*)m3::finish_kernel, m3::kFinishLdsMax},
             {(const void*)m4::spd_wide_kernel<true>, kWideLdsMax},
             {(const void*)m4::spd_wide_kernel<false>, kWideLdsMax},
             {(const void*)m4::spd_wide_backward_kernel<true>, kWideLdsMax},
             {(const void*)m4::spd_wide_backward_kernel<false>, kWideLdsMax}};
  for (auto& k : big) {
    hipError_t e = hipFuncSetAttribute(k.fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)k.bytes);
    if (e != hipSuccess)
      return fail(M4MR_EHIP, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
  }
  int device = 0, cus = 0;
  if (hipGetDevice(&device) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
      cus > 0)
    g_cus = cus;
  configured = true;
  return M4MR_OK;
}

// Launch `body` on `stream`, bracketed by profiling events when enabled.
template <typename F>
int launch(const char* name, hipStream_t stream, F&& body) {
  hipEvent_t a = nullptr, b = nullptr;
  bool prof;
  {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    prof = g_prof_on && (g_prof_only.empty() || g_prof_only == name);
    if (prof && (take_event(&a) != hipSuccess || take_event(&b) != hipSuccess))
      return fail(M4MR_EHIP, std::string(name) + ": profiling event setup failed");
  }
  if (prof && hipEventRecord(a, stream) != hipSuccess)
    return fail(M4MR_EHIP, std::string(name) + ": profiling event record failed");
  body();
  hipError_t e = hipGetLastError();
  if (prof) {
    if (hipEventRecord(b, stream) != hipSuccess)
      return fail(M4MR_EHIP, std::string(name) + ": profiling event record failed");
    std::lock_guard<std::mutex> lock(g_prof_mu);
    g_prof.push_back({name, a, b});
  }
  if (e != hipSuccess) return fail(M4MR_EHIP, std::string(name) + ": " + hipGetErrorString(e));
  return M4MR_OK;
}

// The chunk-boundary states run as one fused walk per (b, h) state sequence
// when there are enough sequences to give every compute unit one; fewer
// sequences take the chunk-parallel statistics plus a separate carry.  The
// environment variable M4MR_STATE_WALK = "fused" or "split" overrides the
// choice (both give the same states up to summation order).
bool fused_states(int B, int H, const Dims& d) {
  if (const char* mode = std::getenv("M4MR_STATE_WALK")) {
    if (std::strcmp(mode, "fused") == 0) return true;
    if (std::strcmp(mode, "split") == 0) return false;
  }
  return (long)B * H * (1 + d.NV) >= g_cus;
}

// The fused walks with one LDS step buffer (three blocks per CU) when their
// blocks would not all be resident at two per CU.  M4MR_STATE_BUFFERS = "1"
// or "2" overrides the choice (the same results either way).
bool states_single_buffer(int B, int H, const Dims& d) {
  if (const char* n = std::getenv("M4MR_STATE_BUFFERS")) {
    if (std::strcmp(n, "1") == 0) return true;
    if (std::strcmp(n, "2") == 0) return false;
  }
  return (long)B * H * (1 + d.NV) > 2L * g_cus;
}

// Poll bound of the factor kernel's turn waits: 2^16, or M4MR_TURN_POLLS
// (a negative value makes every wait give up, a test of the kernel's
// give-up path: the results are then NaN).
int turn_polls() {
  if (const char* v = std::getenv("M4MR_TURN_POLLS")) return std::atoi(v);
  return 1 << 16;
}

bool bad_dims(int B, int T, int H, int P, int chunk, std::string* why) {
  if (B <= 0 || T <= 0 || H <= 0) {
    *why = "B, T and H must be positive";
    return true;
  }
  if (P != M4MR_VALUE_DIM && P != M4MR_MAX_VALUE_DIM) {
    *why = "value_dim must be 64 or 128 (pad narrower values with zeros)";
    return true;
  }
  if (chunk < 1 || chunk > M4MR_MAX_CHUNK) {
    *why = "chunk must lie in [1, 64]";
    return true;
  }
  const double tokens = (double)B * T * H;
  if (tokens * M4MR_FACTOR_FLOATS > 9.0e18 || (double)B * H * (4 + 4 * (P / 64)) > 2.0e9) {
    *why = "problem too large";
    return true;
  }
  return false;
}

Dims make_dims(int B, int T, int H, int P, int chunk) {
  Dims d;
  d.B = B;
  d.T = T;
  d.H = H;
  d.P = P;
  d.NV = P / 64;
  d.chunk = chunk;
  d.NC = (T + chunk - 1) / chunk;
  // Chunks above 32 tokens split in two sub-chunks for the factor kernel, so
  // it sees twice as many independent token sequences.
  d.rsub = chunk > 32 ? 2 : 1;
  d.sub = (chunk + d.rsub - 1) / d.rsub;
  d.NS = d.NC * d.rsub;
  return d;
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct BackwardWorkspace {
  float *z, *end_s, *end_c, *floor_part;
  size_t bytes;
};

BackwardWorkspace carve(void* base, int B, int T, int H, int P, int chunk) {
  const Dims d = make_dims(B, T, H, P, chunk);
  const size_t tok = (size_t)B * T * H;
  const size_t seqs = (size_t)B * H * d.NC;
  size_t off = 0;
  BackwardWorkspace w;
  char* p = static_cast<char*>(base);
  w.z = reinterpret_cast<float*>(p + off);
  off = align256(off + tok * 64 * sizeof(float));
  w.end_s = reinterpret_cast<float*>(p + off);
  off = align256(off + seqs * 4096 * sizeof(float));
  w.end_c = reinterpret_cast<float*>(p + off);
  off = align256(off + seqs * d.NV * 4096 * sizeof(float));
  w.floor_part = reinterpret_cast<float*>(p + off);
  off = align256(off + seqs * 64 * sizeof(float));
  w.bytes = off;
  return w;
}

// Four systems per 64-thread block on a one-dimensional grid of at most
// 2^31 - 1 blocks.
constexpr long kMaxSystems = ((1L << 31) - 1) * 4;

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

// The memory read forward and backward for float32 or bfloat16 keys,
// values and queries (the C entry points below).
// The forward launch sequence.  MIX: keys and queries come from the mixer's
// raw projections (`mix`; the plain key and query pointers are unused), the
// state walk is always the fused one, and the output is gated (`gate`).
template <typename In, bool MIX>
int forward_impl(const char* entry, const In* keys, const In* values, const In* queries,
                 const float* beta, const float* log_decay, const float* floor,
                 const float* init_evidence, const float* init_cross, int B, int T, int H,
                 int value_dim, int chunk, float* output, float* variance, float* final_evidence,
                 float* final_cross, float* solved, float* factors, float* start_evidence,
                 float* start_cross, void* stream, const m4::MixerIn& mix = {},
                 const m4::ReadGate& gate = {}, const m4::MixerGates& gates = {}) {
  g_error.clear();
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why)) return fail(M4MR_EINVAL, std::string(entry) + ": " + why);
  // factors may be NULL: the forward then factors without storing.
  const void* need[] = {MIX ? (const void*)mix.key : keys,
                        values,
                        MIX ? (const void*)mix.query : queries,
                        beta,          log_decay,   floor,
                        output,        variance,    final_evidence,
                        final_cross, solved,     start_evidence, start_cross};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, std::string(entry) + ": a required pointer is NULL");
  if (MIX && (!gate.confidence_scale || !gate.skip || !gate.read))
    return fail(M4MR_EINVAL, std::string(entry) + ": a required pointer is NULL");
  if ((init_evidence == nullptr) != (init_cross == nullptr))
    return fail(M4MR_EINVAL, std::string(entry) + ": init_evidence and init_cross must both be set or both NULL");
  const void* vec[] = {MIX ? (const void*)mix.key : keys, values,
                       MIX ? (const void*)mix.query : queries, solved, factors, output,
                       start_evidence, start_cross, final_evidence, final_cross, init_evidence,
                       init_cross, MIX ? (const void*)mix.previous : nullptr,
                       MIX ? (const void*)gate.read : nullptr};
  for (const void* p : vec)
    if (p && misaligned(p)) return fail(M4MR_EINVAL, std::string(entry) + ": arrays must be 16-byte aligned");
  if (int rc = configure()) return rc;
  const Dims d = make_dims(B, T, H, value_dim, chunk);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned seqs = (unsigned)B * H * d.NC;
  const unsigned subseqs = (unsigned)B * H * d.NS;
  int rc;
  if (MIX || fused_states(B, H, d)) {
    m4::StateArgs args{keys,            values,      keys,           beta,   log_decay,
                       init_evidence,   init_cross,  start_evidence, start_cross,
                       final_evidence,  final_cross, mix};
    args.gates = gates;
    rc = launch("fwd_states", st, [&] {
      const bool one = states_single_buffer(B, H, d);
      const auto walk = one ? m4::states_kernel<false, In, MIX, 1> : m4::states_kernel<false, In, MIX, 2>;
      hipLaunchKernelGGL(walk, dim3(B * H, 1 + d.NV), dim3(512),
                         one ? kStatesLdsBytes / 2 : kStatesLdsBytes, st, d, args);
    });
  } else {
    rc = launch("fwd_stats", st, [&] {
      hipLaunchKernelGGL(m4::fwd_stats_kernel<In>, dim3(seqs), dim3(256), kStatsLdsBytes, st, d,
                         keys, values, beta, log_decay, start_evidence, start_cross);
    });
    if (rc) return rc;
    rc = launch("fwd_scan", st, [&] {
      hipLaunchKernelGGL(m4::fwd_scan_kernel, dim3(B * H, 4 + 4 * d.NV), dim3(256), 0, st, d,
                         log_decay, init_evidence, init_cross, start_evidence, start_cross,
                         final_evidence, final_cross);
    });
  }
  if (rc) return rc;
  const int polls = turn_polls();
  rc = launch("fwd_factor", st, [&] {
    // Four sub-chunk sequences per wave pair; four pairs per block when those
    // blocks fill the chip in whole rounds (one resident per CU), else two.
    const unsigned blocks4 = (subseqs + 15) / 16;
    const int pairs = blocks4 % (unsigned)g_cus == 0 ? 4 : 2;
    const dim3 grid((subseqs + 4 * pairs - 1) / (4 * pairs)), block(128 * pairs);
    const auto kernel = factors ? (pairs == 4 ? m4::fwd_factor_kernel<In, MIX, true, 4>
                                              : m4::fwd_factor_kernel<In, MIX, true, 2>)
                                : (pairs == 4 ? m4::fwd_factor_kernel<In, MIX, false, 4>
                                              : m4::fwd_factor_kernel<In, MIX, false, 2>);
    hipLaunchKernelGGL(kernel, grid, block, 0, st, d, keys, queries, beta, log_decay, floor,
                       start_evidence, solved, factors, mix, polls);
  });
  if (rc) return rc;
  return launch("fwd_read", st, [&] {
    const auto read = d.NV == 1 ? m4::fwd_read_kernel<In, MIX, 1> : m4::fwd_read_kernel<In, MIX, 2>;
    hipLaunchKernelGGL(read, dim3(persistent_grid(seqs, 2)), dim3(256),
                       kChunkLdsBytes, st, d, keys, values, queries, beta, log_decay, solved,
                       start_cross, output, variance, mix, gate);
  });
}

// The backward launch sequence.  MIX: keys and queries come from the
// mixer's raw projections (`mix`; the plain key and query pointers are
// unused), normalised on load by bwd_dy and bwd_grads; the gradients are
// those of the normalised keys and queries, as in the plain case.  GATE
// (with MIX): d_output is the cotangent of the mixer's gated output and the
// gradients are carried on through the read gating and the prologue (`mg`;
// d_keys, d_queries, d_beta, d_log_decay and d_variance are unused, d_floor
// is the floor_raw gradient); the per-head parameter partials are left in
// mg.dy_part and mg.grads_part for the caller's head sums.
template <typename In, bool MIX, bool GATE = false>
int backward_impl(const char* entry, const In* keys, const In* values, const In* queries,
                  const float* beta, const float* log_decay, const float* floor, int B, int T,
                  int H, int value_dim, int chunk, const float* solved, const float* factors,
                  const float* start_evidence, const float* start_cross, const float* d_output,
                  const float* d_variance, const float* d_final_evidence,
                  const float* d_final_cross, float* d_keys, float* d_values, float* d_queries,
                  float* d_beta, float* d_log_decay, float* d_floor, float* d_init_evidence,
                  float* d_init_cross, void* workspace, size_t workspace_bytes, void* stream,
                  const m4::MixerIn& mix = {}, bool spill_free = false,
                  const m4::MixerGrad& mg = {}, const float* floor_raw = nullptr) {
  static_assert(!GATE || MIX, "the gated backward takes the mixer's raw rows");
  g_error.clear();
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why)) return fail(M4MR_EINVAL, std::string(entry) + ": " + why);
  if (MIX) {
    keys = reinterpret_cast<const In*>(mix.key);
    queries = reinterpret_cast<const In*>(mix.query);
    if (mix.previous && misaligned(mix.previous))
      return fail(M4MR_EINVAL, std::string(entry) + ": arrays must be 16-byte aligned");
  }
  if (GATE) {
    // The gated backward's own outputs and inputs stand in for the plain ones.
    d_output = mg.d_out;
    d_variance = mg.d_var;
    d_keys = mg.d_key;
    d_queries = mg.d_query;
    d_beta = mg.d_beta_raw;
    d_log_decay = mg.d_dt_raw;
    const void* gate_need[] = {mg.read,   mg.variance, mg.scale,      mg.skip,
                               mg.dt_raw, mg.dt_bias,  mg.a_log,      mg.dy_part,
                               mg.grads_part, floor_raw, mg.d_scale, mg.d_skip,
                               mg.d_beta_bias, mg.d_dt_bias, mg.d_a_log};
    for (const void* p : gate_need)
      if (!p) return fail(M4MR_EINVAL, std::string(entry) + ": a required pointer is NULL");
    const void* gate_vec[] = {mg.read, mg.d_shifted, mg.d_previous};
    for (const void* p : gate_vec)
      if (p && misaligned(p))
        return fail(M4MR_EINVAL, std::string(entry) + ": arrays must be 16-byte aligned");
  }
  const void* need[] = {keys,    values,     queries,         beta,         log_decay,
                        floor,   solved,     factors,         start_evidence, start_cross,
                        d_output, d_variance, d_keys,         d_values,     d_queries,
                        d_beta,  d_log_decay, d_floor,        d_init_evidence, d_init_cross,
                        workspace};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, std::string(entry) + ": a required pointer is NULL");
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(M4MR_EINVAL, std::string(entry) + ": workspace must be 256-byte aligned");
  const BackwardWorkspace ws = carve(workspace, B, T, H, value_dim, chunk);
  if (workspace_bytes < ws.bytes)
    return fail(M4MR_EINVAL, std::string(entry) + ": workspace too small (need " +
                                 std::to_string(ws.bytes) + " bytes)");
  const void* vec[] = {keys, values, queries, solved, factors, start_evidence, start_cross,
                       d_output, d_final_evidence, d_final_cross, d_init_evidence, d_init_cross};
  for (const void* p : vec)
    if (p && misaligned(p)) return fail(M4MR_EINVAL, std::string(entry) + ": arrays must be 16-byte aligned");
  if (int rc = configure()) return rc;
  const Dims d = make_dims(B, T, H, value_dim, chunk);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned seqs = (unsigned)B * H * d.NC;
  const long tokens = (long)B * T * H;
  int rc = launch("bwd_dy", st, [&] {
    const auto dy = d.NV == 1 ? m4::bwd_dy_kernel<In, MIX, GATE, 1> : m4::bwd_dy_kernel<In, MIX, GATE, 2>;
    hipLaunchKernelGGL(dy, dim3(persistent_grid(seqs, 2)),
                       dim3(256), kChunkLdsBytes, st, d, keys, values, queries, beta, log_decay,
                       start_cross, d_output, d_variance, ws.z, mix, mg);
  });
  if (rc) return rc;
  rc = launch("factored_solve", st, [&] {
    hipLaunchKernelGGL(m4::factored_solve_kernel, dim3((unsigned)((tokens + 3) / 4)), dim3(64), 0,
                       st, factors, ws.z, ws.z, tokens);
  });
  if (rc) return rc;
  // The gated backward always takes the fused walk, whose cross weights
  // take the read gate.
  if (GATE || fused_states(B, H, d)) {
    m4::StateArgs args{ws.z,             d_output,       solved,   beta,   log_decay,
                       d_final_evidence, d_final_cross,  ws.end_s, ws.end_c,
                       d_init_evidence,  d_init_cross};
    args.variance = mg.variance;
    args.confidence_scale = mg.scale;
    rc = launch("bwd_states", st, [&] {
      // The one-buffer walk is held to 80 VGPRs, where the compiler may spill
      // to per-lane scratch (device memory the HIP runtime provides with the
      // dispatch); a caller that allocates nothing (spill_free) takes the
      // two-buffer walk, which has room to spare and gives the same states.
      const bool one = !spill_free && states_single_buffer(B, H, d);
      const auto walk = one ? m4::states_kernel<true, float, GATE, 1> : m4::states_kernel<true, float, GATE, 2>;
      hipLaunchKernelGGL(walk, dim3(B * H, 1 + d.NV), dim3(512),
                         (one ? kStatesLdsBytes / 2 : kStatesLdsBytes) + kStatesBwdExtra, st, d,
                         args);
    });
  } else {
    rc = launch("bwd_local", st, [&] {
      hipLaunchKernelGGL(m4::bwd_local_kernel, dim3(seqs), dim3(256), kChunkLdsBytes, st, d,
                         beta, log_decay, solved, ws.z, d_output, ws.end_s, ws.end_c);
    });
    if (rc) return rc;
    rc = launch("bwd_scan", st, [&] {
      hipLaunchKernelGGL(m4::bwd_scan_kernel, dim3(B * H, 4 + 4 * d.NV), dim3(256), 0, st, d,
                         log_decay, d_final_evidence, d_final_cross, ws.end_s, ws.end_c,
                         d_init_evidence, d_init_cross);
    });
  }
  if (rc) return rc;
  rc = launch("bwd_grads", st, [&] {
    const auto grads = d.NV == 1 ? m4::bwd_grads_kernel<In, MIX, GATE, 1>
                                 : m4::bwd_grads_kernel<In, MIX, GATE, 2>;
    hipLaunchKernelGGL(grads, dim3(persistent_grid(seqs, 1)),
                       dim3(512), GATE ? kGradsGateLdsBytes : kGradsLdsBytes, st, d, keys,
                       values, beta, log_decay, solved,
                       ws.z, d_output, d_variance, start_evidence, start_cross, ws.end_s,
                       ws.end_c, d_keys, d_values, d_queries, d_beta, d_log_decay, ws.floor_part,
                       mix, mg);
  });
  if (rc) return rc;
  if (GATE)
    // The floor_raw gradient and the per-head parameter gradients.
    return launch("mixer_finish", st, [&] {
      hipLaunchKernelGGL(m4::mixer_finish_kernel, dim3(H * 16 + H * 5), dim3(256), 0, st, d,
                         ws.floor_part, d_floor, floor_raw, mg.dy_part, mg.grads_part,
                         mg.d_scale, mg.d_skip, mg.d_beta_bias, mg.d_dt_bias, mg.d_a_log);
    });
  return launch("floor_reduce", st, [&] {
    hipLaunchKernelGGL(m4::floor_reduce_kernel, dim3(H * 16), dim3(256), 0, st, d, ws.floor_part,
                       d_floor, nullptr);
  });
}

// The allocation-free backward's workspace: one static device array per GPU
// the library runs on, held until the process ends.  Its name in host code
// is only a stand-in for the symbol: the device address of each GPU's copy
// comes from hipGetSymbolAddress, resolved once per device (with that device
// current) and kept in g_scratch_ptr; only that address is handed to kernels.
static __device__ __align__(256) unsigned char scratch[M4MR_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` in *out (M4MR_OK), or an error.
int scratch_on_current_device(const char* entry, void** out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess)
    return fail(M4MR_EHIP, std::string(entry) + ": hipGetDevice: " + hipGetErrorString(e));
  if (device < 0 || device >= kMaxDevices)
    return fail(M4MR_EINVAL, std::string(entry) + ": device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(M4MR_EHIP, std::string(entry) + ": hipGetSymbolAddress(scratch): " +
                                 hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return M4MR_OK;
}

}  // namespace

extern "C" {

const char* m4mr_version(void) { return "mamba4_memread 0.1 gfx950"; }

const char* m4mr_last_error(void) { return g_error.c_str(); }

int m4mr_forward(const float* keys, const float* values, const float* queries,
                 const float* beta, const float* log_decay, const float* floor,
                 const float* init_evidence, const float* init_cross, int B, int T, int H,
                 int value_dim, int chunk, float* output, float* variance, float* final_evidence,
                 float* final_cross, float* solved, float* factors, float* start_evidence,
                 float* start_cross, void* stream) {
  return forward_impl<float, false>("m4mr_forward", keys, values, queries, beta, log_decay, floor,
                      init_evidence, init_cross, B, T, H, value_dim, chunk, output, variance,
                      final_evidence, final_cross, solved, factors, start_evidence, start_cross,
                      stream);
}

int m4mr_forward_bf16(const uint16_t* keys, const uint16_t* values, const uint16_t* queries,
                      const float* beta, const float* log_decay, const float* floor,
                      const float* init_evidence, const float* init_cross, int B, int T, int H,
                      int value_dim, int chunk, float* output, float* variance,
                      float* final_evidence, float* final_cross, float* solved, float* factors,
                      float* start_evidence, float* start_cross, void* stream) {
  return forward_impl<m4::bf16_t, false>("m4mr_forward_bf16", reinterpret_cast<const m4::bf16_t*>(keys),
                      reinterpret_cast<const m4::bf16_t*>(values),
                      reinterpret_cast<const m4::bf16_t*>(queries), beta, log_decay, floor,
                      init_evidence, init_cross, B, T, H, value_dim, chunk, output, variance,
                      final_evidence, final_cross, solved, factors, start_evidence, start_cross,
                      stream);
}

int m4mr_mixer_forward(const float* key, const float* value, const float* query,
                       const float* beta_raw, const float* dt_raw,
                       const m4mr_mixer_params* params, const float* init_evidence,
                       const float* init_cross, int B, int T, int H, int value_dim, int chunk,
                       float* output, float* read, float* variance, float* beta,
                       float* log_decay, float* floor, float* final_evidence,
                       float* final_cross, float* solved, float* factors,
                       float* start_evidence, float* start_cross, float* shifted, void* stream) {
  g_error.clear();
  if (!params) return fail(M4MR_EINVAL, "m4mr_mixer_forward: params is NULL");
  if (!(params->beta_max > 0.f))
    return fail(M4MR_EINVAL, "m4mr_mixer_forward: beta_max must be positive");
  if (!(params->floor_min > 0.f))
    return fail(M4MR_EINVAL, "m4mr_mixer_forward: floor_min must be positive");
  const void* need[] = {key,           query,          value,         beta_raw,
                        dt_raw,        params->beta_bias, params->dt_bias, params->a_log,
                        params->floor_raw, beta,        log_decay,     floor};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, "m4mr_mixer_forward: a required pointer is NULL");
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why))
    return fail(M4MR_EINVAL, "m4mr_mixer_forward: " + why);
  if (key && misaligned(key)) return fail(M4MR_EINVAL, "m4mr_mixer_forward: arrays must be 16-byte aligned");
  if (shifted && misaligned(shifted))
    return fail(M4MR_EINVAL, "m4mr_mixer_forward: arrays must be 16-byte aligned");
  const m4::MixerIn mix{key, query, params->previous, params->key_shift ? 1 : 0};
  const m4::ReadGate gate{params->confidence_scale, params->skip, read};
  // The fused state walk computes the gates and writes them out (with the
  // floor and the shifted key) before the factor and read kernels use them.
  m4::MixerGates gates{};
  gates.beta_raw = beta_raw;
  gates.dt_raw = dt_raw;
  gates.beta_bias = params->beta_bias;
  gates.dt_bias = params->dt_bias;
  gates.a_log = params->a_log;
  gates.floor_raw = params->floor_raw;
  gates.beta_max = params->beta_max;
  gates.floor_min = params->floor_min;
  gates.beta = beta;
  gates.log_decay = log_decay;
  gates.floor = floor;
  gates.shifted = params->key_shift ? shifted : nullptr;
  return forward_impl<float, true>("m4mr_mixer_forward", nullptr, value, nullptr, beta, log_decay,
                                   floor, init_evidence, init_cross, B, T, H, value_dim, chunk,
                                   output, variance, final_evidence, final_cross, solved, factors,
                                   start_evidence, start_cross, stream, mix, gate, gates);
}

int m4mr_mixer_backward(const float* key, const float* value, const float* query,
                        const float* beta, const float* log_decay, const float* floor,
                        const float* previous, int key_shift, int B, int T, int H,
                        int value_dim, int chunk, const float* solved, const float* factors,
                        const float* start_evidence, const float* start_cross,
                        const float* d_read, const float* d_variance,
                        const float* d_final_evidence, const float* d_final_cross,
                        float* d_keys, float* d_values, float* d_queries, float* d_beta,
                        float* d_log_decay, float* d_floor, float* d_init_evidence,
                        float* d_init_cross, void* workspace, size_t workspace_bytes,
                        void* stream) {
  g_error.clear();
  if (!key || !query) return fail(M4MR_EINVAL, "m4mr_mixer_backward: a required pointer is NULL");
  const m4::MixerIn mix{key, query, previous, key_shift ? 1 : 0};
  return backward_impl<float, true>(
      "m4mr_mixer_backward", nullptr, value, nullptr, beta, log_decay, floor, B, T, H, value_dim,
      chunk, solved, factors, start_evidence, start_cross, d_read, d_variance, d_final_evidence,
      d_final_cross, d_keys, d_values, d_queries, d_beta, d_log_decay, d_floor, d_init_evidence,
      d_init_cross, workspace, workspace_bytes, stream, mix);
}

}  // extern "C"

namespace {

// The fused mixer backward's workspace: m4mr_backward's, then the read's
// variance cotangent [B,T,H] and the per-chunk partials of the gating's
// (H x 2) and the prologue's (H x 3) per-head parameter gradients.
struct MixerReadWorkspace {
  float *d_var, *dy_part, *grads_part;
  long chunks;  // B NC, the partials per (head, parameter)
  size_t bytes;
};

MixerReadWorkspace carve_mixer(void* base, int B, int T, int H, int P, int chunk) {
  const Dims d = make_dims(B, T, H, P, chunk);
  MixerReadWorkspace w;
  size_t off = carve(nullptr, B, T, H, P, chunk).bytes;
  char* p = static_cast<char*>(base);
  w.chunks = (long)B * d.NC;
  w.d_var = reinterpret_cast<float*>(p + off);
  off = align256(off + (size_t)B * T * H * sizeof(float));
  w.dy_part = reinterpret_cast<float*>(p + off);
  off = align256(off + (size_t)H * 2 * w.chunks * sizeof(float));
  w.grads_part = reinterpret_cast<float*>(p + off);
  off = align256(off + (size_t)H * 3 * w.chunks * sizeof(float));
  w.bytes = off;
  return w;
}

}  // namespace

extern "C" {

size_t m4mr_mixer_read_backward_workspace_bytes(int B, int T, int H, int value_dim, int chunk) {
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why)) return 0;
  return carve_mixer(nullptr, B, T, H, value_dim, chunk).bytes;
}

int m4mr_mixer_read_backward(const float* key, const float* value, const float* query,
                             const float* dt_raw, const m4mr_mixer_params* params, int B, int T,
                             int H, int value_dim, int chunk, const float* read,
                             const float* variance, const float* beta, const float* log_decay,
                             const float* floor, const float* solved, const float* factors,
                             const float* start_evidence, const float* start_cross,
                             const float* d_output, const float* d_variance,
                             const float* d_final_evidence, const float* d_final_cross,
                             const float* d_shifted, float* d_key, float* d_value,
                             float* d_query, float* d_beta_raw, float* d_dt_raw,
                             float* d_beta_bias, float* d_dt_bias, float* d_a_log,
                             float* d_floor_raw, float* d_previous, float* d_confidence_scale,
                             float* d_skip, float* d_init_evidence, float* d_init_cross,
                             void* workspace, size_t workspace_bytes, void* stream) {
  const char* entry = "m4mr_mixer_read_backward";
  g_error.clear();
  if (!params) return fail(M4MR_EINVAL, std::string(entry) + ": params is NULL");
  if (!(params->beta_max > 0.f))
    return fail(M4MR_EINVAL, std::string(entry) + ": beta_max must be positive");
  const void* need[] = {key,           query,          params->dt_bias, params->a_log,
                        params->floor_raw, params->confidence_scale, params->skip,
                        d_key,         d_query,        d_beta_raw,      d_dt_raw,
                        d_beta_bias,   d_dt_bias,      d_a_log,         d_floor_raw,
                        d_confidence_scale, d_skip,    workspace};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, std::string(entry) + ": a required pointer is NULL");
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why)) return fail(M4MR_EINVAL, std::string(entry) + ": " + why);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(M4MR_EINVAL, std::string(entry) + ": workspace must be 256-byte aligned");
  const MixerReadWorkspace mw = carve_mixer(workspace, B, T, H, value_dim, chunk);
  if (workspace_bytes < mw.bytes)
    return fail(M4MR_EINVAL, std::string(entry) + ": workspace too small (need " +
                                 std::to_string(mw.bytes) + " bytes)");
  const bool shift = params->key_shift != 0;
  const m4::MixerIn mix{key, query, shift ? params->previous : nullptr, shift ? 1 : 0};
  m4::MixerGrad mg{};
  mg.d_out = d_output;
  mg.read = read;
  mg.variance = variance;
  mg.d_var_in = d_variance;
  mg.scale = params->confidence_scale;
  mg.skip = params->skip;
  mg.d_var = mw.d_var;
  mg.dy_part = mw.dy_part;
  mg.dt_raw = dt_raw;
  mg.dt_bias = params->dt_bias;
  mg.a_log = params->a_log;
  mg.beta_max = params->beta_max;
  mg.d_shifted = shift ? d_shifted : nullptr;
  mg.d_key = d_key;
  mg.d_query = d_query;
  mg.d_beta_raw = d_beta_raw;
  mg.d_dt_raw = d_dt_raw;
  mg.d_previous = d_previous;
  mg.grads_part = mw.grads_part;
  mg.d_scale = d_confidence_scale;
  mg.d_skip = d_skip;
  mg.d_beta_bias = d_beta_bias;
  mg.d_dt_bias = d_dt_bias;
  mg.d_a_log = d_a_log;
  return backward_impl<float, true, true>(
      entry, nullptr, value, nullptr, beta, log_decay, floor, B, T, H, value_dim, chunk, solved,
      factors, start_evidence, start_cross, nullptr, nullptr, d_final_evidence, d_final_cross,
      nullptr, d_value, nullptr, nullptr, nullptr, d_floor_raw, d_init_evidence, d_init_cross,
      workspace, workspace_bytes, stream, mix, /*spill_free=*/false, mg, params->floor_raw);
}

int m4mr_start_counts(int T, int chunk, int* chunks, int* evidence_starts) {
  g_error.clear();
  std::string why;
  if (bad_dims(1, T, 1, M4MR_VALUE_DIM, chunk, &why))
    return fail(M4MR_EINVAL, "m4mr_start_counts: " + why);
  const Dims d = make_dims(1, T, 1, M4MR_VALUE_DIM, chunk);
  if (chunks) *chunks = d.NC;
  if (evidence_starts) *evidence_starts = d.NS;
  return M4MR_OK;
}

size_t m4mr_backward_workspace_bytes(int B, int T, int H, int value_dim, int chunk) {
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why)) return 0;
  return carve(nullptr, B, T, H, value_dim, chunk).bytes;
}

int m4mr_backward(const float* keys, const float* values, const float* queries,
                  const float* beta, const float* log_decay, const float* floor, int B, int T,
                  int H, int value_dim, int chunk, const float* solved, const float* factors,
                  const float* start_evidence, const float* start_cross, const float* d_output,
                  const float* d_variance, const float* d_final_evidence,
                  const float* d_final_cross, float* d_keys, float* d_values, float* d_queries,
                  float* d_beta, float* d_log_decay, float* d_floor, float* d_init_evidence,
                  float* d_init_cross, void* workspace, size_t workspace_bytes, void* stream) {
  return backward_impl<float, false>("m4mr_backward", keys, values, queries, beta, log_decay, floor, B, T, H,
                       value_dim, chunk, solved, factors, start_evidence, start_cross, d_output,
                       d_variance, d_final_evidence, d_final_cross, d_keys, d_values, d_queries,
                       d_beta, d_log_decay, d_floor, d_init_evidence, d_init_cross, workspace,
                       workspace_bytes, stream);
}

int m4mr_backward_bf16(const uint16_t* keys, const uint16_t* values, const uint16_t* queries,
                       const float* beta, const float* log_decay, const float* floor, int B,
                       int T, int H, int value_dim, int chunk, const float* solved,
                       const float* factors, const float* start_evidence,
                       const float* start_cross, const float* d_output,
                       const float* d_variance, const float* d_final_evidence,
                       const float* d_final_cross, float* d_keys, float* d_values,
                       float* d_queries, float* d_beta, float* d_log_decay, float* d_floor,
                       float* d_init_evidence, float* d_init_cross, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return backward_impl<m4::bf16_t, false>("m4mr_backward_bf16", reinterpret_cast<const m4::bf16_t*>(keys),
                       reinterpret_cast<const m4::bf16_t*>(values),
                       reinterpret_cast<const m4::bf16_t*>(queries), beta, log_decay, floor, B,
                       T, H, value_dim, chunk, solved, factors, start_evidence, start_cross,
                       d_output, d_variance, d_final_evidence, d_final_cross, d_keys, d_values,
                       d_queries, d_beta, d_log_decay, d_floor, d_init_evidence, d_init_cross,
                       workspace, workspace_bytes, stream);
}

int m4mr_backward_noalloc(const float* keys, const float* values, const float* queries,
                          const float* beta, const float* log_decay, const float* floor, int B,
                          int T, int H, int value_dim, int chunk, const float* solved,
                          const float* factors, const float* start_evidence,
                          const float* start_cross, const float* d_output,
                          const float* d_variance, const float* d_final_evidence,
                          const float* d_final_cross, float* d_keys, float* d_values,
                          float* d_queries, float* d_beta, float* d_log_decay, float* d_floor,
                          float* d_init_evidence, float* d_init_cross, void* stream) {
  g_error.clear();
  std::string why;
  if (bad_dims(B, T, H, value_dim, chunk, &why))
    return fail(M4MR_EINVAL, "m4mr_backward_noalloc: " + why);
  // Sizes are checked before any HIP call.
  const size_t need = carve(nullptr, B, T, H, value_dim, chunk).bytes;
  if (need > (size_t)M4MR_STATIC_SCRATCH_BYTES)
    return fail(M4MR_EINVAL, "m4mr_backward_noalloc: these sizes need " + std::to_string(need) +
                                 " bytes of workspace, more than its static " +
                                 std::to_string((size_t)M4MR_STATIC_SCRATCH_BYTES) +
                                 "-byte buffer; use m4mr_backward with a workspace");
  void* ws = nullptr;
  if (int rc = scratch_on_current_device("m4mr_backward_noalloc", &ws)) return rc;
  return backward_impl<float, false>(
      "m4mr_backward_noalloc", keys, values, queries, beta, log_decay, floor, B, T, H, value_dim,
      chunk, solved, factors, start_evidence, start_cross, d_output, d_variance,
      d_final_evidence, d_final_cross, d_keys, d_values, d_queries, d_beta, d_log_decay, d_floor,
      d_init_evidence, d_init_cross, ws, (size_t)M4MR_STATIC_SCRATCH_BYTES, stream, {},
      /*spill_free=*/true);
}

int m4mr_factored_solve(const float* factors, const float* rhs, float* z, long N,
                        void* stream) {
  g_error.clear();
  if (N <= 0 || N > kMaxSystems)
    return fail(M4MR_EINVAL, "m4mr_factored_solve: need 0 < N < 2^33");
  if (!factors || !rhs || !z) return fail(M4MR_EINVAL, "m4mr_factored_solve: NULL pointer");
  if (misaligned(factors)) return fail(M4MR_EINVAL, "m4mr_factored_solve: factors must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return launch("factored_solve", st, [&] {
    hipLaunchKernelGGL(m4::factored_solve_kernel, dim3((unsigned)((N + 3) / 4)), dim3(64), 0, st,
                       factors, rhs, z, N);
  });
}

int m4mr_decode_step(float* evidence, float* cross, const float* key, const float* value,
                     const float* query, const float* beta, const float* log_decay,
                     const float* floor, long N, int H, int value_dim, float* output,
                     float* variance, void* stream) {
  g_error.clear();
  if (N <= 0 || N > kMaxSystems || H <= 0 || N % H != 0)
    return fail(M4MR_EINVAL, "m4mr_decode_step: N must be a positive multiple of H");
  if (value_dim != M4MR_VALUE_DIM && value_dim != M4MR_MAX_VALUE_DIM)
    return fail(M4MR_EINVAL, "m4mr_decode_step: value_dim must be 64 or 128");
  const void* need[] = {evidence, cross, key, value, query, beta, log_decay, floor, output, variance};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, "m4mr_decode_step: a required pointer is NULL");
  if (misaligned(evidence) || misaligned(cross))
    return fail(M4MR_EINVAL, "m4mr_decode_step: states must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return launch("decode_step", st, [&] {
    hipLaunchKernelGGL(m4::decode_step_kernel, dim3((unsigned)((N + 3) / 4)), dim3(64), 0, st,
                       evidence, cross, key, value, query, beta, log_decay, floor, N, H,
                       value_dim / 64, output, variance);
  });
}

long m4mr_spd_factor_floats(int dim) {
  if (dim < 1 || dim > m4::kWideMaxDim) return 0;
  return dim <= M4MR_KEY_DIM ? (long)M4MR_FACTOR_FLOATS : (long)dim * dim;
}

int m4mr_spd_solve(const float* precision, const float* rhs, long N, int dim, float* solution,
                   float* factors, void* stream) {
  g_error.clear();
  if (N <= 0 || N > kMaxSystems || dim < 1 || dim > m4::kWideMaxDim ||
      (dim > M4MR_KEY_DIM && N > INT_MAX))
    return fail(M4MR_EINVAL,
                "m4mr_spd_solve: need 0 < N < 2^33 (< 2^31 above width 64) and 1 <= dim <= 4096");
  if (!precision || !rhs || !solution)
    return fail(M4MR_EINVAL, "m4mr_spd_solve: a required pointer is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dim > M4MR_KEY_DIM) {
    const bool lds = dim <= m4::kWideLdsDim;
    if (!lds && !factors)
      return fail(M4MR_EINVAL,
                  "m4mr_spd_solve: above width 128 the factors buffer is required (the "
                  "factorization runs in it)");
    if (int rc = configure()) return rc;
    const size_t bytes = sizeof(float) * m4::wide_lds_floats(dim);
    return launch("spd_wide", st, [&] {
      hipLaunchKernelGGL(lds ? m4::spd_wide_kernel<true> : m4::spd_wide_kernel<false>,
                         dim3((unsigned)N), dim3(m4::kWideThreads), bytes, st, precision, rhs,
                         dim, solution, factors);
    });
  }
  if ((factors && misaligned(factors)) || (dim == M4MR_KEY_DIM && misaligned(precision)))
    return fail(M4MR_EINVAL, "m4mr_spd_solve: factors (and a 64-wide precision) must be 16-byte aligned");
  return launch("spd_solve", st, [&] {
    hipLaunchKernelGGL(m4::spd_solve_kernel, dim3((unsigned)((N + 3) / 4)), dim3(64), 0, st,
                       precision, rhs, N, dim, solution, factors);
  });
}

int m4mr_spd_solve_backward(const float* factors, const float* solution,
                            const float* d_solution, long N, int dim, float* d_precision,
                            float* d_rhs, void* stream) {
  g_error.clear();
  if (N <= 0 || N > kMaxSystems || dim < 1 || dim > m4::kWideMaxDim ||
      (dim > M4MR_KEY_DIM && N > INT_MAX))
    return fail(M4MR_EINVAL,
                "m4mr_spd_solve_backward: need 0 < N < 2^33 (< 2^31 above width 64) and 1 <= "
                "dim <= 4096");
  if (!factors || !solution || !d_solution || !d_precision || !d_rhs)
    return fail(M4MR_EINVAL, "m4mr_spd_solve_backward: a required pointer is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dim > M4MR_KEY_DIM) {
    const bool lds = dim <= m4::kWideLdsDim;
    if (int rc = configure()) return rc;
    const size_t bytes = sizeof(float) * m4::wide_lds_floats(dim);
    return launch("spd_wide_backward", st, [&] {
      hipLaunchKernelGGL(lds ? m4::spd_wide_backward_kernel<true>
                             : m4::spd_wide_backward_kernel<false>,
                         dim3((unsigned)N), dim3(m4::kWideThreads), bytes, st, factors, solution,
                         d_solution, dim, d_precision, d_rhs);
    });
  }
  if (misaligned(factors) || (dim == M4MR_KEY_DIM && misaligned(d_precision)))
    return fail(M4MR_EINVAL,
                "m4mr_spd_solve_backward: factors (and a 64-wide d_precision) must be 16-byte aligned");
  return launch("spd_backward", st, [&] {
    hipLaunchKernelGGL(m4::spd_backward_kernel, dim3((unsigned)((N + 3) / 4)), dim3(64), 0, st,
                       factors, solution, d_solution, N, dim, d_precision, d_rhs);
  });
}

int m4mr_diagnostics(const float* evidence, const float* cross, const float* floor, int B, int H,
                     int D, int P, float* per_state, float* summary, void* stream) {
  g_error.clear();
  if (B < 1 || H < 1 || D < 1 || D > M4MR_KEY_DIM || P < 1 || (long)B * H > INT_MAX / 4 ||
      (long)H * D > INT_MAX)
    return fail(M4MR_EINVAL, "m4mr_diagnostics: need B, H, P >= 1 and 1 <= D <= 64");
  if (!evidence || !cross || !floor || !per_state || !summary)
    return fail(M4MR_EINVAL, "m4mr_diagnostics: a required pointer is NULL");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = launch("diag_eigen", st, [&] {
    hipLaunchKernelGGL(m4::diag_eigen_kernel, dim3((unsigned)(B * H)), dim3(64), 0, st, evidence,
                       cross, floor, H, D, P, per_state);
  });
  if (rc) return rc;
  return launch("diag_summary", st, [&] {
    hipLaunchKernelGGL(m4::diag_summary_kernel, dim3(1), dim3(256), 0, st, per_state, B * H,
                       floor, H * D, summary);
  });
}

// ---------------------------------------------------------------- mixer --

namespace {

constexpr int kMixRows = 16;  // token-heads per prologue/epilogue block

bool bad_mixer_dims(int B, int T, int H, int width, std::string* why) {
  if (B <= 0 || T <= 0 || H <= 0) {
    *why = "B, T and H must be positive";
    return true;
  }
  if (width <= 0 || width % 4 != 0 || width > 4096) {
    *why = "row width must be a positive multiple of 4 (at most 4096)";
    return true;
  }
  if ((double)B * T * H * width > 9.0e18 || (double)B * T * H > 2.0e12) {
    *why = "problem too large";
    return true;
  }
  return false;
}

long mixer_blocks(int B, int T, int H) {
  return ((long)B * T * H + kMixRows - 1) / kMixRows;
}

}  // namespace

size_t m4mr_mixer_workspace_bytes(int B, int T, int H) {
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return (size_t)mixer_blocks(B, T, H) * H * 3 * sizeof(float);
}

int m4mr_prologue_forward(const float* key, const float* query, const float* beta_raw,
                          const float* dt_raw, const float* beta_bias, const float* dt_bias,
                          const float* a_log, const float* floor_raw, const float* previous,
                          int B, int T, int H, int D, float beta_max, float floor_min,
                          int key_shift, float* keys, float* queries, float* beta,
                          float* log_decay, float* floor, float* shifted, void* stream) {
  g_error.clear();
  std::string why;
  if (bad_mixer_dims(B, T, H, D, &why)) return fail(M4MR_EINVAL, "m4mr_prologue_forward: " + why);
  if (!(beta_max > 0.f)) return fail(M4MR_EINVAL, "memory_beta_max must be positive");
  if (!(floor_min > 0.f))
    return fail(M4MR_EINVAL, "Selective floor must be positive and above its minimum");
  const void* need[] = {key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                        keys, queries, beta, log_decay, floor};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, "m4mr_prologue_forward: a required pointer is NULL");
  const void* vec[] = {key, query, previous, keys, queries, shifted};
  for (const void* p : vec)
    if (p && misaligned(p))
      return fail(M4MR_EINVAL, "m4mr_prologue_forward: rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return launch("prologue_forward", st, [&] {
    hipLaunchKernelGGL(m4::prologue_forward_kernel, dim3((unsigned)mixer_blocks(B, T, H)),
                       dim3(256), 0, st, key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log,
                       floor_raw, key_shift ? previous : nullptr, B, T, H, D, beta_max,
                       floor_min, key_shift ? 1 : 0, keys, queries, beta, log_decay, floor,
                       key_shift ? shifted : nullptr);
  });
}

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
                           void* stream) {
  g_error.clear();
  std::string why;
  if (bad_mixer_dims(B, T, H, D, &why))
    return fail(M4MR_EINVAL, "m4mr_prologue_backward: " + why);
  const void* need[] = {key,         query,     beta_raw,   dt_raw,     beta_bias, dt_bias,
                        a_log,       floor_raw, d_keys,     d_queries,  d_beta,    d_log_decay,
                        d_floor,     d_key,     d_query,    d_beta_raw, d_dt_raw,  d_beta_bias,
                        d_dt_bias,   d_a_log,   d_floor_raw, workspace};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, "m4mr_prologue_backward: a required pointer is NULL");
  if (workspace_bytes < m4mr_mixer_workspace_bytes(B, T, H))
    return fail(M4MR_EINVAL, "m4mr_prologue_backward: workspace too small (need " +
                                 std::to_string(m4mr_mixer_workspace_bytes(B, T, H)) + " bytes)");
  const void* vec[] = {key, query, previous, d_keys, d_queries, d_shifted, d_key, d_query,
                       d_previous};
  for (const void* p : vec)
    if (p && misaligned(p))
      return fail(M4MR_EINVAL, "m4mr_prologue_backward: rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const long blocks = mixer_blocks(B, T, H);
  const bool shift = key_shift != 0;
  int rc = launch("prologue_backward", st, [&] {
    hipLaunchKernelGGL(m4::prologue_backward_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                       key, query, beta_raw, dt_raw, beta_bias, dt_bias, a_log, floor_raw,
                       shift ? previous : nullptr, B, T, H, D, beta_max, shift ? 1 : 0, d_keys,
                       d_queries, d_beta, d_log_decay, d_floor, shift ? d_shifted : nullptr,
                       d_key, d_query, d_beta_raw, d_dt_raw, d_floor_raw,
                       shift ? d_previous : nullptr, part);
  });
  if (rc) return rc;
  if (d_previous && !shift) {
    // Without the shift nothing reads `previous`: its cotangent is zero (a
    // fill kernel rather than a memset, so the call can be graph-captured).
    rc = launch("prologue_backward", st, [&] {
      hipLaunchKernelGGL(m4::zero_kernel, dim3((unsigned)(((long)B * H * D + 255) / 256)),
                         dim3(256), 0, st, d_previous, (long)B * H * D);
    });
    if (rc) return rc;
  }
  return launch("head_sums", st, [&] {
    hipLaunchKernelGGL(m4::head_sums_kernel, dim3(H * 3), dim3(1024), 0, st, part, blocks, H, 3,
                       d_beta_bias, d_dt_bias, d_a_log);
  });
}

int m4mr_epilogue_forward(const float* read, const float* variance, const float* value,
                          const float* confidence_scale, const float* skip, int B, int T, int H,
                          int P, float* out, void* stream) {
  g_error.clear();
  std::string why;
  if (bad_mixer_dims(B, T, H, P, &why)) return fail(M4MR_EINVAL, "m4mr_epilogue_forward: " + why);
  const void* need[] = {read, variance, value, confidence_scale, skip, out};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, "m4mr_epilogue_forward: a required pointer is NULL");
  if (misaligned(read) || misaligned(value) || misaligned(out))
    return fail(M4MR_EINVAL, "m4mr_epilogue_forward: rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return launch("epilogue_forward", st, [&] {
    hipLaunchKernelGGL(m4::epilogue_forward_kernel, dim3((unsigned)mixer_blocks(B, T, H)),
                       dim3(256), 0, st, read, variance, value, confidence_scale, skip, B, T, H,
                       P, out);
  });
}

int m4mr_epilogue_backward(const float* read, const float* variance, const float* value,
                           const float* confidence_scale, const float* skip, int B, int T, int H,
                           int P, const float* d_out, float* d_read, float* d_variance,
                           float* d_value, float* d_confidence_scale, float* d_skip,
                           void* workspace, size_t workspace_bytes, void* stream) {
  g_error.clear();
  std::string why;
  if (bad_mixer_dims(B, T, H, P, &why))
    return fail(M4MR_EINVAL, "m4mr_epilogue_backward: " + why);
  const void* need[] = {read,     variance, value,   confidence_scale,   skip,   d_out, d_read,
                        d_variance, d_value, d_confidence_scale, d_skip, workspace};
  for (const void* p : need)
    if (!p) return fail(M4MR_EINVAL, "m4mr_epilogue_backward: a required pointer is NULL");
  if (workspace_bytes < m4mr_mixer_workspace_bytes(B, T, H))
    return fail(M4MR_EINVAL, "m4mr_epilogue_backward: workspace too small (need " +
                                 std::to_string(m4mr_mixer_workspace_bytes(B, T, H)) + " bytes)");
  const void* vec[] = {read, value, d_out, d_read, d_value};
  for (const void* p : vec)
    if (misaligned(p))
      return fail(M4MR_EINVAL, "m4mr_epilogue_backward: rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  const long blocks = mixer_blocks(B, T, H);
  int rc = launch("epilogue_backward", st, [&] {
    hipLaunchKernelGGL(m4::epilogue_backward_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                       read, variance, value, confidence_scale, skip, B, T, H, P, d_out, d_read,
                       d_variance, d_value, part);
  });
  if (rc) return rc;
  return launch("head_sums", st, [&] {
    hipLaunchKernelGGL(m4::head_sums_kernel, dim3(H * 2), dim3(1024), 0, st, part, blocks, H, 2,
                       d_confidence_scale, d_skip, nullptr);
  });
}

// ---------------------------------------------------------------------------
// Order head scan.

namespace {

constexpr int kOrderMaxWidth = 256;

bool bad_order_dims(int B, int T, int H, int W, int chunk, std::string* why) {
  if (B <= 0 || T <= 0 || H <= 0) {
    *why = "B, T and H must be positive";
    return true;
  }
  if (W <= 0 || W > kOrderMaxWidth) {
    *why = "the value width must be in 1.." + std::to_string(kOrderMaxWidth);
    return true;
  }
  if (chunk <= 0 || chunk > m4::MAXC) {
    *why = "chunk must be in 1.." + std::to_string(m4::MAXC);
    return true;
  }
  if ((long)B * H * ((T + chunk - 1) / chunk) > INT32_MAX || (long)B * T * H * W > (1L << 40)) {
    *why = "problem too large";
    return true;
  }
  return false;
}

m4::OrderDims order_dims(int B, int T, int H, int W, int chunk) {
  return m4::OrderDims{B, T, H, W, chunk, (T + chunk - 1) / chunk};
}

// Chunk states [B,H,NC,W] then chunk totals [B,H,NC].
size_t order_workspace(const m4::OrderDims& d, float** states, float** totals, void* base) {
  const size_t slots = (size_t)d.B * d.H * d.NC;
  const size_t first = align256(slots * d.W * sizeof(float));
  if (base) {
    *states = static_cast<float*>(base);
    *totals = reinterpret_cast<float*>(static_cast<char*>(base) + first);
  }
  return first + align256(slots * sizeof(float));
}

unsigned order_threads(int W) { return (unsigned)(64 * ((W + 63) / 64)); }

}  // namespace

size_t m4mr_order_workspace_bytes(int B, int T, int H, int W, int chunk) {
  std::string why;
  if (bad_order_dims(B, T, H, W, chunk, &why)) return 0;
  return order_workspace(order_dims(B, T, H, W, chunk), nullptr, nullptr, nullptr);
}

int m4mr_order_forward(const float* values, const float* log_decay, const float* initial, int B,
                       int T, int H, int W, int chunk, float* output, void* workspace,
                       size_t workspace_bytes, void* stream) {
  g_error.clear();
  std::string why;
  if (bad_order_dims(B, T, H, W, chunk, &why)) return fail(M4MR_EINVAL, "m4mr_order_forward: " + why);
  if (!values || !log_decay || !output || !workspace)
    return fail(M4MR_EINVAL, "m4mr_order_forward: a required pointer is NULL");
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(M4MR_EINVAL, "m4mr_order_forward: workspace must be 256-byte aligned");
  const m4::OrderDims d = order_dims(B, T, H, W, chunk);
  float *states = nullptr, *totals = nullptr;
  if (workspace_bytes < order_workspace(d, &states, &totals, workspace))
    return fail(M4MR_EINVAL, "m4mr_order_forward: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned chunks = (unsigned)((long)B * H * d.NC), threads = order_threads(W);
  int rc = launch("order_local", st, [&] {
    hipLaunchKernelGGL(m4::order_local_kernel, dim3(chunks), dim3(threads), 0, st, d, values,
                       log_decay, states, totals);
  });
  if (rc) return rc;
  rc = launch("order_carry", st, [&] {
    hipLaunchKernelGGL(m4::order_carry_kernel, dim3(B * H), dim3(threads), 0, st, d, initial,
                       states, totals);
  });
  if (rc) return rc;
  return launch("order_apply", st, [&] {
    hipLaunchKernelGGL(m4::order_apply_kernel, dim3(chunks), dim3(threads), 0, st, d, values,
                       log_decay, states, output);
  });
}

int m4mr_order_backward(const float* values, const float* log_decay, const float* initial,
                        const float* output, const float* d_output, int B, int T, int H, int W,
                        int chunk, float* d_values, float* d_log_decay, float* d_initial,
                        void* workspace, size_t workspace_bytes, void* stream) {
  g_error.clear();
  std::string why;
  if (bad_order_dims(B, T, H, W, chunk, &why))
    return fail(M4MR_EINVAL, "m4mr_order_backward: " + why);
  if (!values || !log_decay || !output || !d_output || !d_values || !d_log_decay || !workspace)
    return fail(M4MR_EINVAL, "m4mr_order_backward: a required pointer is NULL");
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return fail(M4MR_EINVAL, "m4mr_order_backward: workspace must be 256-byte aligned");
  const m4::OrderDims d = order_dims(B, T, H, W, chunk);
  float *heads = nullptr, *totals = nullptr;
  if (workspace_bytes < order_workspace(d, &heads, &totals, workspace))
    return fail(M4MR_EINVAL, "m4mr_order_backward: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned chunks = (unsigned)((long)B * H * d.NC), threads = order_threads(W);
  int rc = launch("order_bwd_local", st, [&] {
    hipLaunchKernelGGL(m4::order_bwd_local_kernel, dim3(chunks), dim3(threads), 0, st, d,
                       d_output, log_decay, heads, totals);
  });
  if (rc) return rc;
  rc = launch("order_bwd_carry", st, [&] {
    hipLaunchKernelGGL(m4::order_bwd_carry_kernel, dim3(B * H), dim3(threads), 0, st, d, heads,
                       totals, d_initial);
  });
  if (rc) return rc;
  return launch("order_bwd_apply", st, [&] {
    hipLaunchKernelGGL(m4::order_bwd_apply_kernel, dim3(chunks), dim3(threads), 0, st, d, values,
                       log_decay, initial, output, d_output, heads, d_values, d_log_decay);
  });
}

// ------------------------------------------------------------ mamba-3 --

}  // extern "C"

namespace {

// Head groups of the gradient kernel: enough (b, chunk, group) blocks to give
// every compute unit about two, each group's heads summed in registers.
int m3_groups(int B, int T, int H) {
  const long chunks = (long)B * ((T + m3::C - 1) / m3::C);
  long g = (512 + chunks - 1) / chunks;
  if (g < 1) g = 1;
  if (g > H) g = H;
  // Equal groups of hpg heads, none empty.
  const long hpg = (H + g - 1) / g;
  return (int)((H + hpg - 1) / hpg);
}

struct M3Workspace {
  float *dh1, *dgam, *dscale, *ddt_loc, *D, *qb_part, *kb_part, *dc_part, *db_part, *dang_part;
};

// Carves the workspace (each array 256-byte aligned); returns the bytes used.
size_t m3_workspace(int B, int T, int H, M3Workspace* ws, void* base) {
  const long NC = (T + m3::C - 1) / m3::C, tp = NC * m3::C, G = m3_groups(B, T, H);
  const long counts[10] = {(long)B * H * NC * m3::NT * m3::PT, (long)B * T * H, (long)B * T * H,
                           (long)B * T * H, (long)B * H * NC * m3::AM, (long)B * NC * H * m3::NT,
                           (long)B * NC * H * m3::NT, G * B * tp * m3::NT, G * B * tp * m3::NT,
                           G * B * tp * m3::AM};
  float** slots[10] = {&ws->dh1, &ws->dgam, &ws->dscale, &ws->ddt_loc, &ws->D,
                       &ws->qb_part, &ws->kb_part, &ws->dc_part, &ws->db_part, &ws->dang_part};
  size_t off = 0;
  for (int i = 0; i < 10; ++i) {
    if (base) *slots[i] = reinterpret_cast<float*>(static_cast<char*>(base) + off);
    off += ((size_t)counts[i] * sizeof(float) + 255) & ~(size_t)255;
  }
  return off;
}

bool m3_bad_shape(const char* entry, int B, int T, int H, int N, int P, int A) {
  std::string why;
  if (B < 1 || T < 1 || H < 1) why = "need B, T, H >= 1";
  else if (H > M3S_MAX_HEADS) why = "need H <= 128";
  else if (N < 2 || N > M3S_MAX_STATE || N % 2) why = "need an even N in [2, 128]";
  else if (P < 1 || P > M3S_MAX_VALUE) why = "need P in [1, 64]";
  else if (A < 0 || 2 * A > N) why = "need 0 <= A <= N/2";
  else if ((long)B * T * H * P >= (1L << 31) || (long)B * T * N >= (1L << 31))
    why = "arrays above 2^31 elements";
  // The backward's finish kernel reads each (head group, batch row) slab of
  // its row-gradient partials, ceil(T / C) * C tokens of NT floats, through
  // one buffer resource, whose size and offsets are 32-bit byte counts.
  else if ((long)(T + m3::C - 1) / m3::C * m3::C * m3::NT * 4 >= (1L << 31))
    why = "T above 2^22 - 64 tokens";
  if (why.empty()) return false;
  fail(M4MR_EINVAL, std::string(entry) + ": " + why);
  return true;
}

bool misaligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) != 0; }

bool misaligned_to(const void* p, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) != 0;
}

// In: float, or m3::bf16_t for the bfloat16 entry points (rows, values and
// y in bfloat16; c, b need 4-byte and x 8-byte alignment there).
template <typename In>
int m3_forward_impl(const char* entry, const In* c, const In* b, const In* x, const float* adt,
                    const float* dt, const float* trap_logits, const float* angles,
                    const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                    int A, In* y, float* final_state, float* starts, float* phases,
                    void* stream) {
  g_error.clear();
  const std::string name(entry);
  if (m3_bad_shape(entry, B, T, H, N, P, A)) return M4MR_EINVAL;
  if (!c || !b || !x || !adt || !dt || !trap_logits || (A > 0 && !angles) || !q_bias ||
      !k_bias || !y || !starts || !phases)
    return fail(M4MR_EINVAL, name + ": a required pointer is NULL");
  if (misaligned_to(c, 2 * sizeof(In)) || misaligned_to(b, 2 * sizeof(In)) ||
      misaligned8(q_bias) || misaligned8(k_bias) || misaligned_to(x, 4 * sizeof(In)) ||
      misaligned(starts))
    return fail(M4MR_EINVAL, name + ": c, b need 2-element, x 4-element, the biases 8-byte "
                                    "and starts 16-byte alignment");
  if (int rc = configure()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const m3::Shape s{B, T, H, N, P, A, (T + m3::C - 1) / m3::C};
  // Value rows load as 4-element vectors when P allows (a kernel per case).
  const bool v4 = P % 4 == 0;
  const auto walk = v4 ? m3::walk_kernel<false, In, true> : m3::walk_kernel<false, In, false>;
  const auto out = v4 ? m3::out_kernel<In, true> : m3::out_kernel<In, false>;
  int rc = launch("m3_walk", st, [&] {
    hipLaunchKernelGGL(walk, dim3(2 * B * H), dim3(256), m3::kWalkLds, st, s, b, k_bias, x, adt, dt,
                       trap_logits, angles, phases, starts, nullptr, final_state);
  });
  if (rc) return rc;
  // bfloat16 tiles: two blocks per compute unit.
  const bool bf = std::is_same<In, m3::bf16_t>::value;
  return launch("m3_out", st, [&] {
    hipLaunchKernelGGL(out, dim3(persistent_grid(B * s.NC * H, bf ? 2 : 1)), dim3(bf ? 512 : 1024),
                       bf ? m3::kOutLdsBf16 : m3::kOutLds, st, s, c, b, x, adt, dt, trap_logits,
                       angles, q_bias, k_bias, phases, starts, y);
  });
}

template <typename In>
int m3_backward_impl(const char* entry, const In* c, const In* b, const In* x, const float* adt,
                     const float* dt, const float* trap_logits, const float* angles,
                     const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                     int A, const float* starts, const float* phases, const In* d_y,
                     const float* d_final, float* d_c, float* d_b, In* d_x, float* d_adt,
                     float* d_dt, float* d_trap, float* d_angles, float* d_q_bias,
                     float* d_k_bias, void* workspace, size_t workspace_bytes, void* stream) {
  g_error.clear();
  const std::string name(entry);
  if (m3_bad_shape(entry, B, T, H, N, P, A)) return M4MR_EINVAL;
  if (!c || !b || !x || !adt || !dt || !trap_logits || (A > 0 && (!angles || !d_angles)) ||
      !q_bias || !k_bias || !starts || !phases || !d_y || !d_c || !d_b || !d_x || !d_adt ||
      !d_dt || !d_trap || !d_q_bias || !d_k_bias || !workspace)
    return fail(M4MR_EINVAL, name + ": a required pointer is NULL");
  if (misaligned_to(c, 2 * sizeof(In)) || misaligned_to(b, 2 * sizeof(In)) ||
      misaligned8(q_bias) || misaligned8(k_bias) || misaligned_to(x, 4 * sizeof(In)) ||
      misaligned_to(d_y, 4 * sizeof(In)) || misaligned(starts) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255))
    return fail(M4MR_EINVAL, name + ": c, b need 2-element, x, d_y 4-element, the biases "
                                    "8-byte, starts 16-byte and the workspace 256-byte "
                                    "alignment");
  M3Workspace ws{};
  if (workspace_bytes < m3_workspace(B, T, H, &ws, workspace))
    return fail(M4MR_EINVAL, name + ": workspace too small");
  if (int rc = configure()) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const m3::Shape s{B, T, H, N, P, A, (T + m3::C - 1) / m3::C};
  const int groups = m3_groups(B, T, H);
  const m3::GradOut o{d_x,         d_adt,        ws.dgam,       ws.dscale,
                      ws.ddt_loc,  ws.D,         ws.qb_part,    ws.kb_part,
                      ws.dc_part,  ws.db_part,   ws.dang_part};
  const bool v4 = P % 4 == 0;
  const auto walk = v4 ? m3::walk_kernel<true, In, true> : m3::walk_kernel<true, In, false>;
  const auto grad = v4 ? m3::grad_kernel<In, true> : m3::grad_kernel<In, false>;
  int rc = launch("m3_walk_bwd", st, [&] {
    hipLaunchKernelGGL(walk, dim3(2 * B * H), dim3(256), m3::kWalkLds, st, s, c, q_bias, d_y, adt, dt,
                       trap_logits, angles, const_cast<float*>(phases), ws.dh1, d_final,
                       nullptr);
  });
  if (rc) return rc;
  rc = launch("m3_grad", st, [&] {
    hipLaunchKernelGGL(grad, dim3(B * s.NC * groups), dim3(512), m3::kGradLds, st, s, groups, c,
                       b, x, adt, dt, trap_logits, angles, q_bias, k_bias, phases, starts, ws.dh1,
                       d_y, o);
  });
  if (rc) return rc;
  if (A > 0) {
    rc = launch("m3_suffix", st, [&] {
      const long n = (long)B * H * A;
      hipLaunchKernelGGL(m3::suffix_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                         s, o);
    });
    if (rc) return rc;
  }
  rc = launch("m3_finish", st, [&] {
    hipLaunchKernelGGL(m3::finish_kernel, dim3(B * s.NC * m3::kFinishParts), dim3(256),
                       m3::finish_lds(H, A), st,
                       s, groups, dt, trap_logits, angles, o, d_c, d_b, d_dt, d_trap, d_angles);
  });
  if (rc) return rc;
  return launch("m3_bias", st, [&] {
    hipLaunchKernelGGL(m3::bias_kernel, dim3(H * (m3::NT / 32)), dim3(1024), 0, st, s, o, d_q_bias,
                       d_k_bias);
  });
}

const m3::bf16_t* bf(const uint16_t* p) { return reinterpret_cast<const m3::bf16_t*>(p); }

}  // namespace

extern "C" {

int m3s_forward(const float* c, const float* b, const float* x, const float* adt,
                const float* dt, const float* trap_logits, const float* angles,
                const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                int A, float* y, float* final_state, float* starts, float* phases, void* stream) {
  return m3_forward_impl("m3s_forward", c, b, x, adt, dt, trap_logits, angles, q_bias, k_bias,
                         B, T, H, N, P, A, y, final_state, starts, phases, stream);
}

int m3s_forward_bf16(const uint16_t* c, const uint16_t* b, const uint16_t* x, const float* adt,
                     const float* dt, const float* trap_logits, const float* angles,
                     const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                     int A, uint16_t* y, float* final_state, float* starts, float* phases,
                     void* stream) {
  return m3_forward_impl("m3s_forward_bf16", bf(c), bf(b), bf(x), adt, dt, trap_logits, angles,
                         q_bias, k_bias, B, T, H, N, P, A, reinterpret_cast<m3::bf16_t*>(y),
                         final_state, starts, phases, stream);
}

size_t m3s_backward_workspace_bytes(int B, int T, int H, int N, int P, int A) {
  (void)N;
  (void)P;
  (void)A;
  if (B < 1 || T < 1 || H < 1) return 0;
  return m3_workspace(B, T, H, nullptr, nullptr);
}

int m3s_backward(const float* c, const float* b, const float* x, const float* adt,
                 const float* dt, const float* trap_logits, const float* angles,
                 const float* q_bias, const float* k_bias, int B, int T, int H, int N, int P,
                 int A, const float* starts, const float* phases, const float* d_y,
                 const float* d_final, float* d_c, float* d_b, float* d_x, float* d_adt,
                 float* d_dt, float* d_trap, float* d_angles, float* d_q_bias, float* d_k_bias,
                 void* workspace, size_t workspace_bytes, void* stream) {
  return m3_backward_impl("m3s_backward", c, b, x, adt, dt, trap_logits, angles, q_bias, k_bias,
                          B, T, H, N, P, A, starts, phases, d_y, d_final, d_c, d_b, d_x, d_adt,
                          d_dt, d_trap, d_angles, d_q_bias, d_k_bias, workspace,
                          workspace_bytes, stream);
}

int m3s_backward_bf16(const uint16_t* c, const uint16_t* b, const uint16_t* x, const float* adt,
                      const float* dt, const float* trap_logits, const float* angles,
                      const float* q_bias, const float* k_bias, int B, int T, int H, int N,
                      int P, int A, const float* starts, const float* phases,
                      const uint16_t* d_y, const float* d_final, float* d_c, float* d_b,
                      uint16_t* d_x, float* d_adt, float* d_dt, float* d_trap, float* d_angles,
                      float* d_q_bias, float* d_k_bias, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return m3_backward_impl("m3s_backward_bf16", bf(c), bf(b), bf(x), adt, dt, trap_logits, angles,
                          q_bias, k_bias, B, T, H, N, P, A, starts, phases, bf(d_y), d_final,
                          d_c, d_b, reinterpret_cast<m3::bf16_t*>(d_x), d_adt, d_dt, d_trap,
                          d_angles, d_q_bias, d_k_bias, workspace, workspace_bytes, stream);
}

void m4mr_profile_enable(int on) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_prof_on = on != 0;
}

void m4mr_profile_select(const char* kernel) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_prof_only = kernel ? kernel : "";
}

void m4mr_profile_reset(void) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  for (auto& r : g_prof) {
    (void)hipEventSynchronize(r.stop);
    g_event_pool.push_back(r.start);
    g_event_pool.push_back(r.stop);
  }
  g_prof.clear();
}

int m4mr_profile_read(const char* kernel, double* total_ms, long* launches) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  double sum = 0.0;
  long count = 0;
  for (auto& r : g_prof) {
    if (std::strcmp(r.name, kernel) != 0) continue;
    if (hipEventSynchronize(r.stop) != hipSuccess) return fail(M4MR_EHIP, "profile: event sync failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
      return fail(M4MR_EHIP, "profile: elapsed time failed");
    sum += ms;
    ++count;
  }
  if (total_ms) *total_ms = sum;
  if (launches) *launches = count;
  return M4MR_OK;
}

const char* m4mr_profile_kernel_name(int i) {
  const int n = (int)(sizeof(kKernelNames) / sizeof(kKernelNames[0]));
  return (i >= 0 && i < n) ? kKernelNames[i] : nullptr;
}

}  // extern "C"
