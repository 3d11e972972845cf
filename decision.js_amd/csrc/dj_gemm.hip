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
#include "dj_internal.h"

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

template <int BITS> struct RawB;
template <> struct RawB<8> { uint4 v; };
template <> struct RawB<4> { uint2 v; };

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
  __shared__ uint4 As[2][BM * 8];

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

  uint4 areg[ACH];
  auto gload_a = [&](int kt) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * NT, r = c >> 3, ch = c & 7;
      const int gm = min(m0 + r, M - 1);
      areg[i] = *(const uint4 *)(X + (size_t)gm * K + kt * 64 + ch * 8);
    }
  };
  auto sstore_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + i * NT, r = c >> 3, ch = c & 7;
      As[buf][r * 8 + (ch ^ (r & 7))] = areg[i];
    }
  };
  const int nb0 = (n0 >> 4) + wn * FN;
  RawB<BITS> braw[FN], bnext[FN];
  uint32_t sraw[FN], snext[FN];
  auto gload_b = [&](int kt, RawB<BITS> *br, uint32_t *sr) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const size_t blk = (size_t)(nb0 + j) * KT + kt;
      if constexpr (BITS == 8)
        br[j].v = *(const uint4 *)(Wc + blk * CB + lane * 16);
      else
        br[j].v = *(const uint2 *)(Wc + blk * CB + lane * 8);
      sr[j] = Ws[blk * 16 + (lane & 15)];
    }
  };

  gload_a(0);
  sstore_a(0);
  gload_b(0, braw, sraw);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      gload_a(kt + 1);
      gload_b(kt + 1, bnext, snext);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      h8 bf[FN];
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = dequant<BITS>(braw[j], s, sraw[j]);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * FM * 16 + i * 16 + (lane & 15);
        const int ch = s * 4 + (lane >> 4);
        const h8 af = __builtin_bit_cast(h8, As[cur][r * 8 + (ch ^ (r & 7))]);
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = MFMA16(af, bf[j], acc[i][j]);
      }
    }
    if (more) {
      sstore_a(cur ^ 1);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        braw[j] = bnext[j];
        sraw[j] = snext[j];
      }
    }
    __syncthreads();
  }

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

template <int BITS, bool GLU>
static int launch_bits(hipStream_t s, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int act, const char **name) {
  const int N = w->N;
  if (N % 128 == 0 && M >= 2048) {
    launch_cfg<BITS, 2, 2, 8, 4, GLU>(s, X, w, Y, M, act);
    *name = BITS == 8 ? (GLU ? "matmul_glu_q8_256x128" : "matmul_q8_256x128") : (GLU ? "matmul_glu_q4_256x128" : "matmul_q4_256x128");
  } else if (N % 128 == 0) {
    launch_cfg<BITS, 2, 2, 4, 4, GLU>(s, X, w, Y, M, act);
    *name = BITS == 8 ? (GLU ? "matmul_glu_q8_128x128" : "matmul_q8_128x128") : (GLU ? "matmul_glu_q4_128x128" : "matmul_q4_128x128");
  } else if (N % 32 == 0) {
    launch_cfg<BITS, 4, 1, 2, 2, GLU>(s, X, w, Y, M, act);
    *name = BITS == 8 ? (GLU ? "matmul_glu_q8_128x32" : "matmul_q8_128x32") : (GLU ? "matmul_glu_q4_128x32" : "matmul_q4_128x32");
  } else {
    if (GLU) return dj_fail(DJ_EINVAL, "decision.js: gated matmul needs N %% 32 == 0 (N = %d)", N);
    launch_cfg<BITS, 4, 1, 2, 1, false>(s, X, w, Y, M, act);
    *name = BITS == 8 ? "matmul_q8_128x16" : "matmul_q4_128x16";
  }
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
  return dj_op_end(rec, name);
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
  return dj_op_end(rec, name);
}
