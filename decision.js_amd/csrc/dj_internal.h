// Internal declarations shared by the HIP sources of libdj.so (runtime, kernels, launchers).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <unordered_map>
#include <vector>
#include "../../include/dj.h"

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
// native vector types for registers that must stay in registers (HIP's uint4 is a struct that can keep
// arrays of it out of SROA and in scratch memory)
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- errors
int dj_fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
#define DJ_HIP(call)                                                                                   \
  do {                                                                                                 \
    hipError_t e_ = (call);                                                                            \
    if (e_ != hipSuccess) return dj_fail(DJ_EHIP, "decision.js: %s: %s", #call, hipGetErrorString(e_)); \
  } while (0)
#define DJ_REQUIRE(cond, ...)                       \
  do {                                              \
    if (!(cond)) return dj_fail(DJ_EINVAL, __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------- objects
struct dj_weight {
  int N = 0, K = 0, bits = 0, layout = 0;
  uint8_t *codes = nullptr;   // device: plain [N, K*bits/8] or the MFMA block layout
  void *scales = nullptr;     // device: plain f16 [N, K/32] or packed u32 pairs (MFMA)
  size_t code_bytes = 0, scale_bytes = 0;
};

struct dj_snapshot {
  void *staging;  // device copy taken in stream order
  size_t bytes;
  void *host;
};

struct dj_graph_entry {
  hipGraphExec_t exec = nullptr;
  uint64_t last_use = 0;        // the context's graph clock at the last capture or replay (LRU eviction)
  std::vector<void *> staging;  // snapshot buffers written by the graph, reused on replay
  std::vector<size_t> staging_bytes;
};

struct dj_prof_slot {
  std::string name;
  hipEvent_t a, b;
};

struct dj_ctx {
  int device = 0;
  int cus = 0;
  hipStream_t stream = nullptr;
  std::unordered_map<void *, size_t> buffers;
  std::vector<dj_weight *> weights;
  // pinned staging for dj_upload (bump allocated, reset when the stream is drained)
  uint8_t *pinned = nullptr;
  size_t pinned_cap = 0, pinned_used = 0;
  // graph cache: at most graph_cap() entries, the least recently used evicted first
  std::unordered_map<uint64_t, dj_graph_entry> graphs;
  uint64_t graph_clock = 0;
  dj_rec *active = nullptr;
  // timers
  hipEvent_t t0 = nullptr, t1 = nullptr;
  // profiling
  bool profiling = false;
  std::vector<dj_prof_slot> prof_pending;
  std::vector<hipEvent_t> event_pool;
  std::unordered_map<std::string, std::pair<double, int64_t>> prof;
  std::vector<std::string> prof_order;
  std::string fault_op;  // DJ_FAULT_INJECT: the op name (or "*") that fails ...
  long fault_left = -1;  // ... this many more times (-1: every time)
  // split-K GEMM / split-KV attention workspace: f32 partials, written and read by consecutive kernels of
  // the stream (free between ops)
  float *gemm_ws = nullptr;
  size_t gemm_ws_floats = 0;
  // the device address of the library's static attention scratch on this context's GPU (dj_attention_noalloc)
  float *attn_scratch = nullptr;
};

struct dj_rec {
  dj_ctx *ctx = nullptr;
  uint64_t key = 0;
  bool capturing = false;
  bool replay = false;
  size_t snap_index = 0;
  std::vector<dj_snapshot> snaps;
  int error = 0;
  // A skinny-M product held back by one op (dj_matmul): when the next op is the residual + RMSNorm of its
  // output, the product runs split along K and the norm sums its f32 partials (no summing kernel between);
  // anything else that touches the stream first launches it as an ordinary product (dj_release_held).
  bool holding = false;
  struct {
    const uint16_t *X = nullptr;
    const dj_weight *w = nullptr;
    uint16_t *Y = nullptr;
    int M = 0;
  } held;
};

// Launches a held product as an ordinary dj_matmul (DJ_OK if nothing is held).
int dj_release_held(dj_rec *rec);
// The same for the context's active recorder, if any: called by every entry point that touches the stream
// outside an op, so work runs in the order the caller issued it.
int dj_settle(dj_ctx *c);

// ---------------------------------------------------------------- launch plumbing
// Opens an op: validates the recorder, honours replay (ops ignored) and fault injection, and starts a
// profiling slot. Returns 1 if the op must be skipped (replay), 0 to launch, or a negative status.
int dj_op_begin(dj_rec *rec, const char *name);
// Closes an op after its kernel launches: checks the launch and ends the profiling slot. `detail`
// (optional) is appended to the profile key, e.g. the GEMM shape.
int dj_op_end(dj_rec *rec, const char *name, const char *detail = nullptr);

#define DJ_OP_BEGIN(rec, name)                   \
  do {                                           \
    int s_ = dj_op_begin((rec), (name));         \
    if (s_ == 1) return DJ_OK;                   \
    if (s_ < 0) return -s_;                      \
  } while (0)

// ---------------------------------------------------------------- launchers (one per kernel family)
int dj_launch_gemm(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int glu_act,
                   const char **name, int *splits);
int dj_gemm_workspace(dj_ctx *c, size_t need_floats, float **ws);
// If `rec` holds the product whose output is Y ([T, H]), launches it split along K into the context workspace
// and returns its partials (*S slices of [T, H] f32, in split order) for the residual + RMSNorm to sum; the
// norm kernel also writes the product's f16 rounding to Y. *parts = nullptr (nothing launched) otherwise.
int dj_take_held_split(dj_rec *rec, const uint16_t *Y, int T, int H, const float **parts, int *S);
// QK_NORM_ROPE kernel launch (checked arguments)
int dj_launch_qk_norm_rope(hipStream_t s, int T, int heads, int kv, int D, int stride, uint16_t *Z, const uint16_t *qn,
                           const uint16_t *kn, int vnorm, const int32_t *pos, int pos_stride, float eps, float theta, int rot,
                           int mode);
// The optional output gate of d3's attention: O = f16(attention / (1 + exp(-G[q, h D + d]))), G rows of `stride`.
struct dj_attn_gate {
  const uint16_t *g;
  int stride;
};
// q/k RMSNorm + RoPE folded into attention (D = rot = 128): the query rows and source B's key rows are read raw
// and normalized as QK_NORM_ROPE does (qn / kn: the norm weights, either null for no norm; tab: (cos, sin) of
// the rot / 2 angles per row of B, which are also the query rows). Source A's keys are already rotated.
struct dj_attn_qkn {
  const uint16_t *qn, *kn;
  const float2 *tab;
  float eps;
};
int dj_launch_attention(dj_ctx *c, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride, dj_kv_src A,
                        dj_kv_src B, const int32_t *rng, float scale, uint16_t *O, float *ws, size_t ws_floats,
                        dj_attn_gate gate = dj_attn_gate{nullptr, 0}, const dj_attn_qkn *qkn = nullptr);
// Mean of each sequence's rows of X [T, H] into out [S, H] f32 (seqs: (start, end) pairs).
void dj_launch_mean_pool(hipStream_t s, int T, int S, int H, const uint16_t *X, const uint32_t *seqs, float *out);
// Takes the device address of the static attention scratch on the current device into c->attn_scratch.
int dj_attn_scratch_init(dj_ctx *c);
int dj_launch_copy(hipStream_t s, void *dst, const void *src, size_t bytes);

static inline int dj_cdiv(long a, long b) { return (int)((a + b - 1) / b); }

// ---------------------------------------------------------------- LDS fill by DMA (device side)
// global_load_lds (16 or 4 bytes per lane, written to LDS at M0 + 16 * lane or 4 * lane) and the "stage
// landed" wait are inline assembly on purpose: the compiler models an LDS read after a global_load_lds it
// issued as depending on every such load still in flight and waits vmcnt(0) before it, which would drain a
// whole prefetch ring each step. Hidden from it, the ring's ordering is the explicit vmcnt
// below; the compiler's own vmcnt waits for other loads only get stricter from ops it cannot see (in-order
// completion). "memory" keeps LDS reads from moving across the fill or the barrier. s_nop: one wait state
// between an SALU write of M0 and the LDS DMA that reads it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 is named as clobbered on purpose: the asm writes it
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void *src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop
// this wave's vector-memory ops older than the newest n are complete and its LDS reads have returned, then
// the workgroup barrier
template <int n>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(n >= 0 && n < 64, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(n) : "memory");
}
template <int n>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// ---------------------------------------------------------------- QK_NORM_ROPE pieces shared by its kernels
// (the standalone k_qk_norm_rope, the once-per-forward table and the qkv GEMM epilogue), so every path does
// the same arithmetic.
// (cos, sin) of rotation pair j of a token at position pos: frequency theta^(-2j/rot) (POW_NEG) or
// 1 / theta^(2j/rot) (INV_POW) as exp2(e log2 theta) — WGSL pow's definition (kernels.ts:106,
// eg2-kernels.ts:86) — and angle = f32(pos * f).
__device__ __forceinline__ float2 rope_cs(float ps, int j, int rot, float theta, int mode) {
  const float e = (float)(2 * j) / (float)rot;
  const float l2t = log2f(theta);
  const float f = mode == DJ_ROPE_POW_NEG ? exp2f(-e * l2t) : 1.0f / exp2f(e * l2t);
  float sn, cs;
  sincosf(ps * f, &sn, &cs);
  return make_float2(cs, sn);
}
// One lane's share of a head row: LPH consecutive lanes hold the row. A pair lane (pl) holds dims d0..d0+7 in
// x and their partners d0 + rot/2.. in y; a tail lane (tl) holds 8 unrotated dims in x (y zero); others hold
// zeros. Every lane of the group must call this (the row's sum of squares is a reduction over LPH lanes).
// x / rms(row) (when norm), times the norm weight w (when given), then the rotation by cs(i) = (cos, sin) of
// pair d0 + i (when rope); results rounded to f16.
struct h8x2 {
  h8 x, y;
};

// Sums over aligned groups of L lanes (L = 4 ... 64) without LDS permutes: the row-swapping permlanes add lanes
// l ^ 32 (L = 64) and l ^ 16 (L >= 32); then DPP within each 16-lane row adds l ^ 8 (row_ror 8, L >= 16), the
// mirror lane of each half-row (row_half_mirror, L >= 8), l ^ 2 and l ^ 1 (quad_perm). Each step adds a lane to its partner, so
// every lane of a group ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(L == 4 || L == 8 || L == 16 || L == 32 || L == 64, "lane groups of 4 to 64");
  if constexpr (L == 64) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  if constexpr (L >= 32) {
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  }
  if constexpr (L >= 16) v += dpp_f<0x128>(v);
  if constexpr (L >= 8) v += dpp_f<0x141>(v);
  v += dpp_f<0x4E>(v);
  return v + dpp_f<0xB1>(v);
}
// QK_NORM_ROPE's arithmetic in three pieces, so that every kernel applying it (the standalone kernel, the qkv
// product's epilogue, attention with the norm folded in) computes the same bits from the same inputs: the sum
// of squares of one lane's 8 rotation pairs (x[i], y[i]), the row's 1 / rms from the row's sum, and the
// normalized, weighted, rotated pairs. Every fused multiply-add is written out, and each f32 result is rounded
// to f32 before its conversion to f16 (f32_rounded): left to itself the compiler contracts either product of
// a rotation, or folds the conversion into a mixed-precision fma that rounds once, differently per kernel.
__device__ __forceinline__ float f32_rounded(float v) {
  asm("" : "+v"(v));
  return v;
}
__device__ __forceinline__ float pair_sumsq(h8 x, h8 y) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += __builtin_fmaf((float)x[i], (float)x[i], (float)y[i] * (float)y[i]);
  return ss;
}
__device__ __forceinline__ float norm_inv(float ss, bool norm, int D, float eps) {
  return norm ? 1.0f / sqrtf(ss / (float)D + eps) : 1.f;
}
template <typename CS>
__device__ __forceinline__ h8x2 norm_rope_pairs(h8 x, h8 y, h8 wx, h8 wy, bool has_w, bool rope, float inv, CS cs) {
  h8 xo, yo;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float a = (float)x[i] * inv, b = (float)y[i] * inv;
    if (has_w) {
      a *= (float)wx[i];
      b *= (float)wy[i];
    }
    if (rope) {
      const float2 r = cs(i);
      const float a2 = __builtin_fmaf(a, r.x, -(b * r.y)), b2 = __builtin_fmaf(b, r.x, a * r.y);
      a = a2;
      b = b2;
    }
    xo[i] = (_Float16)f32_rounded(a);
    yo[i] = (_Float16)f32_rounded(b);
  }
  return {xo, yo};
}
template <int LPH, typename CS>
__device__ __forceinline__ h8x2 norm_rope_lane(h8 x, h8 y, h8 wx, h8 wy, bool has_w, bool norm, bool rope, bool pl, int D,
                                               float eps, CS cs) {
  const float inv = norm_inv(group_sum<LPH>(pair_sumsq(x, y)), norm, D, eps);
  if (pl) return norm_rope_pairs(x, y, wx, wy, has_w, rope, inv, cs);
  h8 xo;
#pragma unroll
  for (int i = 0; i < 8; ++i) xo[i] = (_Float16)f32_rounded(has_w ? (float)x[i] * inv * (float)wx[i] : (float)x[i] * inv);
  return {xo, (h8){}};
}
