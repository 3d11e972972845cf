// GEMM on gfx950 f16 MFMA (v_mfma_f32_16x16x32_f16), f32 accumulation:
//   Y[M, N] = X[M, K] . W^T, X f16 row-major, W one of
//     q8 / q4  quantized in blocks of 32 along K with an f16 scale each (kept quantized in HBM), or
//     f16      the same weights dequantized once at load ("direct weights", the reference's directWeights
//              option, gpu.ts:16-20, 114-133) — bit-identical f16 values, twice the bytes of q8.
// Weights are repacked at load (dj_runtime.hip) so one wave reads the B operand of two MFMA k-steps with one
// 16-byte (q8), 8-byte (q4) or two 16-byte (f16) loads per lane, already in lane order. Quantized codes become
// f16 in registers by the exponent trick: 0x6400 | code is exactly 1024 + code; minus (1024 + zero point),
// times the group scale — one RNE rounding, the reference's f16 dequantization (kernels.ts:20, 296, 541).
//
// Per workgroup: WM x WN waves, each computing FM x FN 16x16 fragments. X tiles (64 K per step) go through
// double-buffered, XOR-swizzled LDS, loaded one step ahead; B goes straight to registers two steps ahead.
// The K loop is unrolled by two so both register sets have names (no dynamic indexing -> no scratch).
//
// Split-K (grid y = S): each split stores its f32 partial tile in its own workspace slice; the last split to
// arrive at a tile (per-tile counter) adds the slices in split order (deterministic), resets the counter (so
// the counters need clearing only once, at context creation, and a captured graph holds no memset), then
// runs the epilogue.
//
// Epilogues: plain f16 store, or the gated MLP (SiLU / tanh-GELU) on a [w1; w3] weight whose 16-column
// blocks were interleaved at load so a lane holds a gate value and its up value side by side
// (MATMUL_SWIGLU, kernels.ts:591-599; GELU_MUL, eg2-kernels.ts:165-177).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "dj_internal.h"

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

// Per-lane raw B of one 64-K step for one 16-column fragment.
template <int BITS> struct RawB;
template <> struct RawB<8> { u32x4 v; };         // 16 codes: [k-step 0: 8][k-step 1: 8]
template <> struct RawB<4> { u32x2 v; };         // 16 nibbles
template <> struct RawB<16> { u32x4 v0, v1; };   // 16 f16 weights

__device__ __forceinline__ h2 fma_free_dequant(uint32_t p, h2 bias, h2 sc) {
  const h2 v = __builtin_bit_cast(h2, p);
  return (v - bias) * sc;  // exact subtraction, then the one rounding of the f16 multiply
}

// The 8 f16 weights of k-step s.
template <int BITS>
__device__ __forceinline__ h8 dequant(const RawB<BITS> &r, int s, uint32_t sp) {
  if constexpr (BITS == 16) {
    return __builtin_bit_cast(h8, s ? r.v1 : r.v0);
  } else {
    const _Float16 sv = __builtin_bit_cast(_Float16, (uint16_t)(s ? (sp >> 16) : (sp & 0xffffu)));
    const h2 sc = {sv, sv};
    if constexpr (BITS == 8) {
      const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + zero point 128
      const uint32_t lo = s ? r.v.z : r.v.x, hi = s ? r.v.w : r.v.y;
      // v_perm_b32: bytes (code_a, 0x64, code_b, 0x64) = the f16 pair (1024 + code_a, 1024 + code_b)
      const h2 p0 = fma_free_dequant(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u), bias, sc);
      const h2 p1 = fma_free_dequant(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u), bias, sc);
      const h2 p2 = fma_free_dequant(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u), bias, sc);
      const h2 p3 = fma_free_dequant(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u), bias, sc);
      return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    } else {
      const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};  // 1024 + zero point 8
      const uint32_t w = s ? r.v.y : r.v.x;
      const h2 p0 = fma_free_dequant((w & 0x000f000fu) | 0x64006400u, bias, sc);
      const h2 p1 = fma_free_dequant(((w >> 4) & 0x000f000fu) | 0x64006400u, bias, sc);
      const h2 p2 = fma_free_dequant(((w >> 8) & 0x000f000fu) | 0x64006400u, bias, sc);
      const h2 p3 = fma_free_dequant(((w >> 12) & 0x000f000fu) | 0x64006400u, bias, sc);
      return (h8){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  }
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

struct GemmArgs {
  const uint16_t *X;
  const uint8_t *Wc;
  const uint32_t *Ws;
  uint16_t *Y;
  float *ws;          // split-K workspace [S, M, N] f32
  uint32_t *counter;  // split-K arrivals per tile, zero between launches
  int M, N, K, act, tiles_m, tiles_n, splits, ksteps;  // ksteps: 64-K steps per split
};

template <int BITS, int WM, int WN, int FM, int FN, bool GLU>
__global__ __launch_bounds__(WM *WN * 64) void k_gemm(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int BM = WM * FM * 16, BN = WN * FN * 16;
  constexpr int ACH = BM * 8 / NT;
  static_assert((BM * 8) % NT == 0, "an A stage must split evenly over the threads");
  constexpr int CB = BITS == 8 ? 1024 : BITS == 4 ? 512 : 2048;  // bytes per 16x64 weight block
  __shared__ u32x4 As[2][BM * 8];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  map_tile(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = g.M, K = g.K, KT = g.K >> 6;
  const int kbeg = blockIdx.y * g.ksteps;       // this split's first 64-K step
  const int KS = g.ksteps;                       // steps in this split

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

  const int nb0 = (n0 >> 4) + wn * FN;
  const uint16_t *xrow[ACH];
  int aoff[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = tid + i * NT, r = c >> 3, ch = c & 7;
    xrow[i] = g.X + (size_t)min(m0 + r, M - 1) * K + (size_t)kbeg * 64 + ch * 8;
    aoff[i] = r * 8 + (ch ^ (r & 7));
  }
  u32x4 a[ACH];
  RawB<BITS> b0[FN], b1[FN];
  uint32_t s0[FN], s1[FN];

#define DJ_LOAD_A(kt) _Pragma("unroll") for (int i = 0; i < ACH; ++i) a[i] = *(const u32x4 *)(xrow[i] + (kt) * 64);
#define DJ_STORE_A(buf) _Pragma("unroll") for (int i = 0; i < ACH; ++i) As[buf][aoff[i]] = a[i];
#define DJ_LOAD_B(dst, sdst, kt)                                              \
  _Pragma("unroll") for (int j = 0; j < FN; ++j) {                            \
    const size_t blk = (size_t)(nb0 + j) * KT + kbeg + (kt);                  \
    if constexpr (BITS == 8) {                                                \
      dst[j].v = *(const u32x4 *)(g.Wc + blk * CB + lane * 16);               \
      sdst[j] = g.Ws[blk * 16 + (lane & 15)];                                 \
    } else if constexpr (BITS == 4) {                                         \
      dst[j].v = *(const u32x2 *)(g.Wc + blk * CB + lane * 8);                \
      sdst[j] = g.Ws[blk * 16 + (lane & 15)];                                 \
    } else {                                                                  \
      dst[j].v0 = *(const u32x4 *)(g.Wc + blk * CB + lane * 32);              \
      dst[j].v1 = *(const u32x4 *)(g.Wc + blk * CB + lane * 32 + 16);         \
      sdst[j] = 0;                                                            \
    }                                                                         \
  }
#define DJ_COMPUTE(buf, bb, ss)                                                                  \
  _Pragma("unroll") for (int s = 0; s < 2; ++s) {                                                \
    h8 bf[FN];                                                                                   \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) bf[j] = dequant<BITS>(bb[j], s, ss[j]);       \
    _Pragma("unroll") for (int i = 0; i < FM; ++i) {                                             \
      const int r = wm * FM * 16 + i * 16 + (lane & 15);                                         \
      const int ch = s * 4 + (lane >> 4);                                                        \
      const h8 af = __builtin_bit_cast(h8, As[buf][r * 8 + (ch ^ (r & 7))]);                     \
      _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = MFMA16(af, bf[j], acc[i][j]);   \
    }                                                                                            \
  }

  DJ_LOAD_A(0);
  DJ_LOAD_B(b0, s0, 0);
  if (KS > 1) DJ_LOAD_B(b1, s1, 1);
  DJ_STORE_A(0);
  __syncthreads();
  // Steady state without conditionals (branches inside the loop split the accumulators' live ranges and
  // made the compiler copy them between AGPRs and VGPRs every iteration); the last 1-3 steps are peeled.
  // At the top of each iteration: LDS 0 = A(kt), b0 = B(kt), b1 = B(kt+1).
  int kt = 0;
  for (; kt + 3 < KS; kt += 2) {
    DJ_LOAD_A(kt + 1);
    DJ_COMPUTE(0, b0, s0);
    DJ_LOAD_B(b0, s0, kt + 2);
    DJ_STORE_A(1);
    __syncthreads();
    DJ_LOAD_A(kt + 2);
    DJ_COMPUTE(1, b1, s1);
    DJ_LOAD_B(b1, s1, kt + 3);
    DJ_STORE_A(0);
    __syncthreads();
  }
  const int rem = KS - kt;
  if (rem == 3) {
    DJ_LOAD_A(kt + 1);
    DJ_COMPUTE(0, b0, s0);
    DJ_LOAD_B(b0, s0, kt + 2);
    DJ_STORE_A(1);
    __syncthreads();
    DJ_LOAD_A(kt + 2);
    DJ_COMPUTE(1, b1, s1);
    DJ_STORE_A(0);
    __syncthreads();
    DJ_COMPUTE(0, b0, s0);
  } else if (rem == 2) {
    DJ_LOAD_A(kt + 1);
    DJ_COMPUTE(0, b0, s0);
    DJ_STORE_A(1);
    __syncthreads();
    DJ_COMPUTE(1, b1, s1);
  } else {
    DJ_COMPUTE(0, b0, s0);
  }
#undef DJ_LOAD_A
#undef DJ_STORE_A
#undef DJ_LOAD_B
#undef DJ_COMPUTE

  // accumulator of 16x16 MFMA: lane l holds rows 4(l/16)..+3 of column l%16
  const int rbase = m0 + wm * FM * 16 + (lane >> 4) * 4;
  const int N = g.N;
  if (g.splits > 1) {
    // each split stores its partial tile in its own f32 slice; the last to arrive adds the slices in split
    // order (deterministic: the same bits whichever split arrives last) and resets the tile's counter
    const size_t slice = (size_t)M * N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * FN * 16 + j * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = rbase + i * 16 + r;
          if (m < M) g.ws[blockIdx.y * slice + (size_t)m * N + n] = acc[i][j][r];
        }
      }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const uint32_t prev = atomicAdd(g.counter + blockIdx.x, 1u);
      last_flag = prev == (uint32_t)(g.splits - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * FN * 16 + j * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = rbase + i * 16 + r;
          if (m < M) {
            float sum = 0.0f;
            for (int k = 0; k < g.splits; ++k)
              sum += k == (int)blockIdx.y ? acc[i][j][r]
                                          : __hip_atomic_load(g.ws + k * slice + (size_t)m * N + n, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT);
            acc[i][j][r] = sum;
          }
        }
      }
    if (tid == 0) __hip_atomic_store(g.counter + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if constexpr (!GLU) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * FN * 16 + j * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = rbase + i * 16 + r;
          if (m < M) g.Y[(size_t)m * N + n] = __builtin_bit_cast(uint16_t, (_Float16)acc[i][j][r]);
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
          const float h = (g.act == DJ_ACT_SILU ? act_silu(a) : act_gelu_tanh(a)) * b;
          if (m < M) g.Y[(size_t)m * I + col] = __builtin_bit_cast(uint16_t, (_Float16)h);
        }
      }
  }
}

// ---------------------------------------------------------------- dispatch

// Tile configurations: waves along M and N, 16x16 fragments per wave along M and N.
struct GemmCfg {
  const char *tag;
  int wm, wn, fm, fn;
  int bm() const { return wm * fm * 16; }
  int bn() const { return wn * fn * 16; }
};
static const GemmCfg kCfgs[] = {
    {"256x128", 2, 2, 8, 4}, {"128x128", 2, 2, 4, 4}, {"128x64", 2, 2, 4, 2}, {"64x128", 2, 2, 2, 4},
    {"64x64", 2, 2, 2, 2},   {"32x128", 1, 4, 2, 2},  {"128x32", 4, 1, 2, 2}, {"128x16", 4, 1, 2, 1},
};
static const int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int BITS, int WM, int WN, int FM, int FN, bool GLU>
static void launch_cfg(hipStream_t s, GemmArgs a) {
  dim3 grid(a.tiles_m * a.tiles_n, a.splits);
  k_gemm<BITS, WM, WN, FM, FN, GLU><<<grid, WM * WN * 64, 0, s>>>(a);
}

template <int BITS, bool GLU>
static void launch_index(int i, hipStream_t s, GemmArgs a) {
  switch (i) {
    case 0: launch_cfg<BITS, 2, 2, 8, 4, GLU>(s, a); break;
    case 1: launch_cfg<BITS, 2, 2, 4, 4, GLU>(s, a); break;
    case 2: launch_cfg<BITS, 2, 2, 4, 2, GLU>(s, a); break;
    case 3: launch_cfg<BITS, 2, 2, 2, 4, GLU>(s, a); break;
    case 4: launch_cfg<BITS, 2, 2, 2, 2, GLU>(s, a); break;
    case 5: launch_cfg<BITS, 1, 4, 2, 2, GLU>(s, a); break;
    case 6: launch_cfg<BITS, 4, 1, 2, 2, GLU>(s, a); break;
    default: launch_cfg<BITS, 4, 1, 2, 1, false>(s, a); break;
  }
}

static bool cfg_fits(const GemmCfg &c, int N, bool glu) { return N % c.bn() == 0 && (!glu || c.fn % 2 == 0); }

// Picks (tile, splits). DJ_GEMM_TILE=<tag> and DJ_GEMM_SPLITK=<n> force them (tuning sweeps). Otherwise, from
// sweeps on MI355X over the configurations' shapes: the largest of 128x128, 128x64, 64x64, 32x128 whose grid
// still gives every CU a workgroup (within 15% of the best everywhere measured). Split-K only when even the
// smallest tile leaves most CUs idle (skinny M): its device-scope fence writes back the XCD's L2, which costs
// more than it saves once the grid covers the chip.
static void pick(int M, int N, int K, bool glu, int cus, int ws_ok, int &cfg, int &splits) {
  const char *force = getenv("DJ_GEMM_TILE");
  const char *fs = getenv("DJ_GEMM_SPLITK");
  cfg = -1;
  splits = 1;
  if (force)
    for (int i = 0; i < kNumCfgs; ++i)
      if (!strcmp(force, kCfgs[i].tag) && cfg_fits(kCfgs[i], N, glu)) cfg = i;
  auto tiles = [&](int i) { return (long)dj_cdiv(M, kCfgs[i].bm()) * (N / kCfgs[i].bn()); };
  if (cfg < 0) {
    static const int order[] = {1, 2, 4, 5, 6, 7};  // 128x128, 128x64, 64x64, 32x128, 128x32, 128x16
    for (int i : order)
      if (cfg_fits(kCfgs[i], N, glu) && tiles(i) >= cus) { cfg = i; break; }
    if (cfg < 0) {  // nothing fills the chip: the tile with the most workgroups
      long best = -1;
      for (int i : order)
        if (cfg_fits(kCfgs[i], N, glu) && tiles(i) > best) { cfg = i; best = tiles(i); }
    }
  }
  if (cfg < 0) return;
  const int KT = K / 64;
  if (fs) {
    splits = atoi(fs);
  } else {
    const long t = tiles(cfg);
    while (t * splits * 4 < cus && KT % (splits * 2) == 0 && KT / (splits * 2) >= 4) splits *= 2;
  }
  if (splits < 1 || KT % splits || !ws_ok) splits = 1;
}

// launcher state: the split-K workspace lives in the context
int dj_gemm_workspace(dj_ctx *c, size_t need_floats, size_t need_counters, float **ws, uint32_t **cnt);

template <int BITS, bool GLU>
static int launch_bits(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int act, const char **name,
                       int *splits_out) {
  static const char *const names[3][2][kNumCfgs] = {
      {{"matmul_q4_256x128", "matmul_q4_128x128", "matmul_q4_128x64", "matmul_q4_64x128", "matmul_q4_64x64", "matmul_q4_32x128", "matmul_q4_128x32", "matmul_q4_128x16"},
       {"matmul_glu_q4_256x128", "matmul_glu_q4_128x128", "matmul_glu_q4_128x64", "matmul_glu_q4_64x128", "matmul_glu_q4_64x64", "matmul_glu_q4_32x128", "matmul_glu_q4_128x32", "-"}},
      {{"matmul_q8_256x128", "matmul_q8_128x128", "matmul_q8_128x64", "matmul_q8_64x128", "matmul_q8_64x64", "matmul_q8_32x128", "matmul_q8_128x32", "matmul_q8_128x16"},
       {"matmul_glu_q8_256x128", "matmul_glu_q8_128x128", "matmul_glu_q8_128x64", "matmul_glu_q8_64x128", "matmul_glu_q8_64x64", "matmul_glu_q8_32x128", "matmul_glu_q8_128x32", "-"}},
      {{"matmul_f16_256x128", "matmul_f16_128x128", "matmul_f16_128x64", "matmul_f16_64x128", "matmul_f16_64x64", "matmul_f16_32x128", "matmul_f16_128x32", "matmul_f16_128x16"},
       {"matmul_glu_f16_256x128", "matmul_glu_f16_128x128", "matmul_glu_f16_128x64", "matmul_glu_f16_64x128", "matmul_glu_f16_64x64", "matmul_glu_f16_32x128", "matmul_glu_f16_128x32", "-"}}};
  const int N = w->N, K = w->K;
  float *ws = nullptr;
  uint32_t *cnt = nullptr;
  int cfg, splits;
  pick(M, N, K, GLU, c->cus, 1, cfg, splits);
  if (splits > 1 && dj_gemm_workspace(c, (size_t)splits * M * N, 1 << 16, &ws, &cnt) != DJ_OK) splits = 1;
  if (cfg < 0) return dj_fail(DJ_EINVAL, "decision.js: no matmul tile fits N = %d%s", N, GLU ? " (gated: N % 32 == 0)" : "");
  GemmArgs a;
  a.X = X; a.Wc = w->codes; a.Ws = (const uint32_t *)w->scales; a.Y = Y; a.ws = ws; a.counter = cnt;
  a.M = M; a.N = N; a.K = K; a.act = act;
  a.tiles_m = dj_cdiv(M, kCfgs[cfg].bm());
  a.tiles_n = N / kCfgs[cfg].bn();
  a.splits = splits;
  a.ksteps = (K / 64) / splits;
  if (splits > 1 && (long)a.tiles_m * a.tiles_n > (1 << 16)) {  // more tiles than counters: no split
    a.splits = 1;
    a.ksteps = K / 64;
  }
  launch_index<BITS, GLU>(cfg, c->stream, a);
  *name = names[BITS == 4 ? 0 : BITS == 8 ? 1 : 2][GLU][cfg];
  *splits_out = a.splits;
  return DJ_OK;
}

int dj_launch_gemm(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int glu_act, const char **name,
                   int *splits) {
  const bool glu = glu_act >= 0;
  const int bits = (w->layout & DJ_W_DIRECT) ? 16 : w->bits;
  if (bits == 8) return glu ? launch_bits<8, true>(c, X, w, Y, M, glu_act, name, splits) : launch_bits<8, false>(c, X, w, Y, M, 0, name, splits);
  if (bits == 4) return glu ? launch_bits<4, true>(c, X, w, Y, M, glu_act, name, splits) : launch_bits<4, false>(c, X, w, Y, M, 0, name, splits);
  return glu ? launch_bits<16, true>(c, X, w, Y, M, glu_act, name, splits) : launch_bits<16, false>(c, X, w, Y, M, 0, name, splits);
}

extern "C" int dj_matmul(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M) {
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == DJ_W_MFMA, "decision.js: matmul needs an MFMA-tiled weight (DJ_W_MFMA)");
  DJ_REQUIRE(X && Y && M >= 0, "decision.js: matmul: bad arguments");
  DJ_OP_BEGIN(rec, "matmul");
  const char *name = "matmul";
  int splits = 1;
  if (M > 0) {
    int st = dj_launch_gemm(rec->ctx, X, w, Y, M, -1, &name, &splits);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]%s", M, w->N, w->K, splits > 1 ? (splits == 2 ? "/k2" : splits == 4 ? "/k4" : "/k8") : "");
  return dj_op_end(rec, name, shape);
}

extern "C" int dj_matmul_glu(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *H, int M, int act) {
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == DJ_W_MFMA_GLU, "decision.js: matmul_glu needs a fused w1|w3 weight (DJ_W_MFMA_GLU)");
  DJ_REQUIRE(X && H && M >= 0 && (act == DJ_ACT_SILU || act == DJ_ACT_GELU_TANH), "decision.js: matmul_glu: bad arguments");
  DJ_OP_BEGIN(rec, "matmul_glu");
  const char *name = "matmul_glu";
  int splits = 1;
  if (M > 0) {
    int st = dj_launch_gemm(rec->ctx, X, w, H, M, act, &name, &splits);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]%s", M, w->N, w->K, splits > 1 ? (splits == 2 ? "/k2" : splits == 4 ? "/k4" : "/k8") : "");
  return dj_op_end(rec, name, shape);
}
