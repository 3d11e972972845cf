// q8/q4 block-dequant GEMM on gfx950 f16 MFMA (v_mfma_f32_16x16x32_f16), f32 accumulation:
//   Y[M, N] = X[M, K] . W^T, X f16 row-major, W quantized in blocks of 32 along K with an f16 scale each.
// The weight is repacked at load (dj_runtime.hip) so that one wave reads the B operand of two MFMA k-steps
// as one 16-byte (q8) or 8-byte (q4) load per lane, already in lane order. Codes become f16 in registers by
// the exponent trick (0x6400 | code is 1024 + code exactly), minus the zero point, times the scale: the
// same single RNE rounding as the reference's f16 dequantization (kernels.ts:20, 296, 541), so the GEMM
// multiplies by bit-identical f16 weights. X tiles go through LDS (double buffered, XOR-swizzled 16-byte
// chunks); each wave dequantizes only its own columns.
//
// Epilogues: plain f16 store, or the gated MLP (SiLU / tanh-GELU) on a [w1; w3] weight whose 16-column
// blocks were interleaved at load, so a lane holds a gate value and its up value side by side
// (MATMUL_SWIGLU, kernels.ts:591-599; GELU_MUL, eg2-kernels.ts:165-177).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "dj_internal.h"

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

template <int BITS> struct RawB;
template <> struct RawB<8> { u32x4 v; };
template <> struct RawB<4> { u32x2 v; };

__device__ __forceinline__ h2 pair_q(uint32_t p, h2 bias, h2 sc) {
  h2 v = __builtin_bit_cast(h2, p | 0x64006400u);
  return (v - bias) * sc;
}

// 8 f16 weights of k-step s from the lane's raw codes.
template <int BITS>
__device__ __forceinline__ h8 dequant(const RawB<BITS> &r, int s, uint32_t sp) {
  const _Float16 sv = __builtin_bit_cast(_Float16, (uint16_t)(s ? (sp >> 16) : (sp & 0xffffu)));
  const h2 sc = {sv, sv};
  h8 out;
  if constexpr (BITS == 8) {
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + zero point 128
    const uint32_t lo = s ? r.v.z : r.v.x, hi = s ? r.v.w : r.v.y;
    const h2 p0 = pair_q((lo & 0xffu) | ((lo & 0xff00u) << 8), bias, sc);
    const h2 p1 = pair_q(((lo >> 16) & 0xffu) | ((lo >> 8) & 0xff0000u), bias, sc);
    const h2 p2 = pair_q((hi & 0xffu) | ((hi & 0xff00u) << 8), bias, sc);
    const h2 p3 = pair_q(((hi >> 16) & 0xffu) | ((hi >> 8) & 0xff0000u), bias, sc);
    out = (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  } else {
    const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};  // 1024 + zero point 8
    const uint32_t w = s ? r.v.y : r.v.x;
    const h2 p0 = pair_q(w & 0x000f000fu, bias, sc);
    const h2 p1 = pair_q((w >> 4) & 0x000f000fu, bias, sc);
    const h2 p2 = pair_q((w >> 8) & 0x000f000fu, bias, sc);
    const h2 p3 = pair_q((w >> 12) & 0x000f000fu, bias, sc);
    out = (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  }
  return out;
}

// Block id -> output tile. Workgroups are dealt round-robin to the 8 XCDs (each with its own L2), so give
// each XCD a contiguous run of a grouped order (GROUP m-tiles wide): neighbours in that order share X rows
// or W columns, which then stay in one L2.
__device__ __forceinline__ void map_tile(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
  const int total = tiles_m * tiles_n;
  int lin = bid;
  if ((total & 7) == 0) lin = (bid & 7) * (total >> 3) + (bid >> 3);
  constexpr int GROUP = 8;
  const int width = GROUP * tiles_n;
  const int group = lin / width, first = group * GROUP;
  const int gsz = min(tiles_m - first, GROUP);
  const int in = lin % width;
  tm = first + in % gsz;
  tn = in / gsz;
}

__device__ __forceinline__ float act_silu(float a) { return a / (1.0f + expf(-a)); }
__device__ __forceinline__ float act_gelu_tanh(float x) {
  const float u = fminf(fmaxf(0.7978845608f * (x + 0.044715f * x * x * x), -15.0f), 15.0f);
  const float e = expf(2.0f * u);
  return 0.5f * x * (1.0f + (e - 1.0f) / (e + 1.0f));
}

template <int BITS, int WM, int WN, int FM, int FN, bool GLU>
__global__ __launch_bounds__(WM *WN * 64) void k_gemm(const uint16_t *__restrict__ X, const uint8_t *__restrict__ Wc,
                                                      const uint32_t *__restrict__ Ws, uint16_t *__restrict__ Y, int M,
                                                      int N, int K, int act, int tiles_m, int tiles_n) {
  constexpr int NT = WM * WN * 64;
  constexpr int BM = WM * FM * 16, BN = WN * FN * 16;
  constexpr int ACH = BM * 8 / NT;
  static_assert((BM * 8) % NT == 0, "A stage must split evenly over the threads");
  constexpr int CB = BITS == 8 ? 1024 : 512;
  __shared__ u32x4 As[2][BM * 8];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  map_tile(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int KT = K >> 6;

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

  // Software pipeline, unrolled by two so that both register sets are named (no dynamic indexing, which
  // would put them in scratch): A(k) is loaded two k-steps ahead into registers and stored to LDS one step
  // ahead (double-buffered LDS); B(k) (codes + scales) is loaded into registers two steps ahead.
  const int nb0 = (n0 >> 4) + wn * FN;
  const uint16_t *xrow[ACH];
  int aoff[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + i * NT, r = c >> 3, ch = c & 7;
    xrow[i] = X + (size_t)min(m0 + r, M - 1) * K + ch * 8;
    aoff[i] = r * 8 + (ch ^ (r & 7));
  }
  u32x4 a0[ACH], a1[ACH];
  RawB<BITS> b0[FN], b1[FN];
  uint32_t s0[FN], s1[FN];

#define DJ_LOAD_A(dst, kt)                                                     \
  _Pragma("unroll") for (int i = 0; i < ACH; ++i) dst[i] = *(const u32x4 *)(xrow[i] + (kt) * 64);
#define DJ_STORE_A(src, buf) _Pragma("unroll") for (int i = 0; i < ACH; ++i) As[buf][aoff[i]] = src[i];
#define DJ_LOAD_B(dst, sdst, kt)                                               \
  _Pragma("unroll") for (int j = 0; j < FN; ++j) {                             \
    const size_t blk = (size_t)(nb0 + j) * KT + (kt);                          \
    if constexpr (BITS == 8)                                                   \
      dst[j].v = *(const u32x4 *)(Wc + blk * CB + lane * 16);                  \
    else                                                                       \
      dst[j].v = *(const u32x2 *)(Wc + blk * CB + lane * 8);                   \
    sdst[j] = Ws[blk * 16 + (lane & 15)];                                      \
  }
#define DJ_COMPUTE(buf, bb, ss)                                                        \
  _Pragma("unroll") for (int s = 0; s < 2; ++s) {                                      \
    h8 bf[FN];                                                                         \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) bf[j] = dequant<BITS>(bb[j], s, ss[j]); \
    _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                   \
      const int r = wm * FM * 16 + i * 16 + (lane & 15);                               \
      const int ch = s * 4 + (lane >> 4);                                              \
      const h8 af = __builtin_bit_cast(h8, As[buf][r * 8 + (ch ^ (r & 7))]);           \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = MFMA16(af, bf[j], acc[i][j]); \
    }                                                                                  \
  }

  DJ_LOAD_A(a0, 0);
  DJ_LOAD_B(b0, s0, 0);
  if (KT > 1) {
    DJ_LOAD_A(a1, 1);
    DJ_LOAD_B(b1, s1, 1);
  }
  DJ_STORE_A(a0, 0);
  __syncthreads();

  for (int kt = 0; kt < KT; kt += 2) {
    // step kt: LDS 0 = A(kt), b0 = B(kt); a1 = A(kt+1) in flight
    if (kt + 2 < KT) DJ_LOAD_A(a0, kt + 2);
    DJ_COMPUTE(0, b0, s0);
    if (kt + 1 < KT) DJ_STORE_A(a1, 1);
    if (kt + 2 < KT) DJ_LOAD_B(b0, s0, kt + 2);
    __syncthreads();
    if (kt + 1 >= KT) break;
    // step kt+1: LDS 1 = A(kt+1), b1 = B(kt+1); a0 = A(kt+2) in flight
    if (kt + 3 < KT) DJ_LOAD_A(a1, kt + 3);
    DJ_COMPUTE(1, b1, s1);
    if (kt + 2 < KT) DJ_STORE_A(a0, 0);
    if (kt + 3 < KT) DJ_LOAD_B(b1, s1, kt + 3);
    __syncthreads();
  }
#undef DJ_LOAD_A
#undef DJ_STORE_A
#undef DJ_LOAD_B
#undef DJ_COMPUTE

  // accumulator of 16x16 MFMA: lane l holds rows 4(l/16)..+3 of column l%16
  const int rbase = m0 + wm * FM * 16 + (lane >> 4) * 4;
  if constexpr (!GLU) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * FN * 16 + j * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = rbase + i * 16 + r;
          if (m < M) Y[(size_t)m * N + n] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]);
        }
      }
  } else {
    const int I = N >> 1;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; j += 2) {
        const int col = ((nb0 + j) >> 1) * 16 + (lane & 15);  // physical block p even -> w1 block p / 2
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = rbase + i * 16 + r;
          const float a = (float)(_Float16)acc[i][j][r], b = (float)(_Float16)acc[i][j + 1][r];
          const float h = (act == DJ_ACT_SILU ? act_silu(a) : act_gelu_tanh(a)) * b;
          if (m < M) Y[(size_t)m * I + col] = __builtin_bit_cast(uint16_t, (_Float16)h);
        }
      }
  }
}

template <int BITS, int WM, int WN, int FM, int FN, bool GLU>
static void launch_cfg(hipStream_t s, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int act) {
  constexpr int BM = WM * FM * 16, BN = WN * FN * 16;
  const int tiles_m = dj_cdiv(M, BM), tiles_n = w->N / BN;
  k_gemm<BITS, WM, WN, FM, FN, GLU><<<tiles_m * tiles_n, WM * WN * 64, 0, s>>>(
      X, w->codes, (const uint32_t *)w->scales, Y, M, w->N, w->K, act, tiles_m, tiles_n);
}

// Tile configurations: (waves along M, waves along N, 16-row fragments per wave, 16-column fragments per wave).
struct GemmCfg {
  const char *tag;
  int wm, wn, fm, fn;
  int bm() const { return wm * fm * 16; }
  int bn() const { return wn * fn * 16; }
};
static const GemmCfg kCfgs[] = {
    {"128x128", 2, 2, 4, 4}, {"128x64", 2, 2, 4, 2}, {"64x128", 2, 2, 2, 4}, {"64x64", 2, 2, 2, 2},
    {"32x128", 1, 4, 2, 2},  {"128x32", 4, 1, 2, 2}, {"128x16", 4, 1, 2, 1},
};
static const int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int BITS, bool GLU>
static void launch_index(int i, hipStream_t s, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int act) {
  switch (i) {
    case 0: launch_cfg<BITS, 2, 2, 4, 4, GLU>(s, X, w, Y, M, act); break;
    case 1: launch_cfg<BITS, 2, 2, 4, 2, GLU>(s, X, w, Y, M, act); break;
    case 2: launch_cfg<BITS, 2, 2, 2, 4, GLU>(s, X, w, Y, M, act); break;
    case 3: launch_cfg<BITS, 2, 2, 2, 2, GLU>(s, X, w, Y, M, act); break;
    case 4: launch_cfg<BITS, 1, 4, 2, 2, GLU>(s, X, w, Y, M, act); break;
    case 5: launch_cfg<BITS, 4, 1, 2, 2, GLU>(s, X, w, Y, M, act); break;
    default: launch_cfg<BITS, 4, 1, 2, 1, false>(s, X, w, Y, M, act); break;
  }
}

static bool cfg_fits(const GemmCfg &c, int N, bool glu) {
  return N % c.bn() == 0 && (!glu || c.fn % 2 == 0);
}

// The tile: DJ_GEMM_TILE=<tag> forces one (tuning sweeps). Otherwise the order below, measured on MI355X
// over the configurations' shapes (M 32 to 86016, N 1024 to 9216, K 1024 to 3072): 32x128 was the fastest
// or within 5% everywhere (4 waves side by side on one A tile; more workgroups per CU hide load latency).
static int pick_cfg(int M, int N, bool glu) {
  const char *force = getenv("DJ_GEMM_TILE");
  if (force)
    for (int i = 0; i < kNumCfgs; ++i)
      if (!strcmp(force, kCfgs[i].tag) && cfg_fits(kCfgs[i], N, glu)) return i;
  static const int order[] = {4, 3, 5, 6};  // 32x128, 64x64, 128x32, 128x16
  for (int i : order)
    if (cfg_fits(kCfgs[i], N, glu)) return i;
  (void)M;
  return -1;
}

template <int BITS, bool GLU>
static int launch_bits(hipStream_t s, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int act, const char **name) {
  static const char *const names[2][2][kNumCfgs] = {
      {{"matmul_q4_128x128", "matmul_q4_128x64", "matmul_q4_64x128", "matmul_q4_64x64", "matmul_q4_32x128", "matmul_q4_128x32", "matmul_q4_128x16"},
       {"matmul_glu_q4_128x128", "matmul_glu_q4_128x64", "matmul_glu_q4_64x128", "matmul_glu_q4_64x64", "matmul_glu_q4_32x128", "matmul_glu_q4_128x32", "-"}},
      {{"matmul_q8_128x128", "matmul_q8_128x64", "matmul_q8_64x128", "matmul_q8_64x64", "matmul_q8_32x128", "matmul_q8_128x32", "matmul_q8_128x16"},
       {"matmul_glu_q8_128x128", "matmul_glu_q8_128x64", "matmul_glu_q8_64x128", "matmul_glu_q8_64x64", "matmul_glu_q8_32x128", "matmul_glu_q8_128x32", "-"}}};
  const int i = pick_cfg(M, w->N, GLU);
  if (i < 0) return dj_fail(DJ_EINVAL, "decision.js: no matmul tile fits N = %d%s", w->N, GLU ? " (gated: N % 32 == 0)" : "");
  launch_index<BITS, GLU>(i, s, X, w, Y, M, act);
  *name = names[BITS == 8][GLU][i];
  return DJ_OK;
}

int dj_launch_gemm(hipStream_t s, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int glu_act, const char **name) {
  const bool glu = glu_act >= 0;
  if (w->bits == 8) return glu ? launch_bits<8, true>(s, X, w, Y, M, glu_act, name) : launch_bits<8, false>(s, X, w, Y, M, 0, name);
  return glu ? launch_bits<4, true>(s, X, w, Y, M, glu_act, name) : launch_bits<4, false>(s, X, w, Y, M, 0, name);
}

extern "C" int dj_matmul(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M) {
  DJ_REQUIRE(w && w->layout == DJ_W_MFMA, "decision.js: matmul needs an MFMA-tiled weight (DJ_W_MFMA)");
  DJ_REQUIRE(X && Y && M >= 0, "decision.js: matmul: bad arguments");
  DJ_OP_BEGIN(rec, "matmul");
  const char *name = "matmul";
  if (M > 0) {
    int st = dj_launch_gemm(rec->ctx->stream, X, w, Y, M, -1, &name);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]", M, w->N, w->K);
  return dj_op_end(rec, name, shape);
}

extern "C" int dj_matmul_glu(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *H, int M, int act) {
  DJ_REQUIRE(w && w->layout == DJ_W_MFMA_GLU, "decision.js: matmul_glu needs a fused w1|w3 weight (DJ_W_MFMA_GLU)");
  DJ_REQUIRE(X && H && M >= 0 && (act == DJ_ACT_SILU || act == DJ_ACT_GELU_TANH), "decision.js: matmul_glu: bad arguments");
  DJ_OP_BEGIN(rec, "matmul_glu");
  const char *name = "matmul_glu";
  if (M > 0) {
    int st = dj_launch_gemm(rec->ctx->stream, X, w, H, M, act, &name);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]", M, w->N, w->K);
  return dj_op_end(rec, name, shape);
}
