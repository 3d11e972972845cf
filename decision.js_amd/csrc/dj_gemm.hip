// GEMM on gfx950 f16 MFMA (v_mfma_f32_16x16x32_f16), f32 accumulation:
//   Y[M, N] = X[M, K] . W^T, X f16 row-major, W one of
//     q8 / q4  quantized in blocks of 32 along K with an f16 scale each (kept quantized in HBM), or
//     f16      the same weights dequantized once at load ("direct weights", the reference's directWeights
//              option, gpu.ts:16-20, 114-133) — bit-identical f16 values, twice the bytes of q8.
// Weights are repacked at load (dj_runtime.hip) into 16-column x 64-K blocks in MFMA lane order (1 KB q8,
// 512 B q4, 2 KB f16) with 16 scale words per block. Quantized codes become f16 in registers by the exponent
// trick: 0x6400 | code is exactly 1024 + code; minus (1024 + zero point), times the group scale — one RNE
// rounding, the reference's f16 dequantization (kernels.ts:20, 296, 541).
//
// Per workgroup: WM x WN waves, each computing FM x FN 16x16 fragments. Operands reach LDS without passing
// through registers: global_load_lds (16 bytes per lane; 4 for scales) fills a ring of NS stages, each one
// 64-K step of the tile (X rows XOR-swizzled in 16-byte chunks, weight blocks and scales as stored), NS - 1
// steps ahead of the MFMAs, so several steps of HBM/L2 latency are in flight per wave. Every vector-memory
// instruction in the loop is one of these, the same number per step, so "this step has landed" is an exact
// s_waitcnt vmcnt count (smaller in the tail, where no further steps are issued); a bare s_barrier (no fence,
// which would drain every outstanding load) then publishes the stage to the other waves.
//
// Split-K (grid y = S): each split stores its f32 partial tile in its own workspace slice with plain stores;
// k_splitk_sum, the next kernel on the stream, adds the slices in split order (deterministic) and runs the
// epilogue. No workgroup waits for another: on MI355X a device-scope release from each workgroup writes back
// its XCD's L2, which measured 130-290 ns per workgroup, serialized, and made a fenced last-arriver reduction
// slower than no split at all; a kernel boundary publishes the slices once.
//
// Epilogues: plain f16 store, or the gated MLP (SiLU / tanh-GELU) on a [w1; w3] weight whose 16-column
// blocks were interleaved at load so a lane holds a gate value and its up value side by side
// (MATMUL_SWIGLU, kernels.ts:591-599; GELU_MUL, eg2-kernels.ts:165-177).
#include <math.h>
#include <algorithm>
#include <type_traits>
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

// Gated activations on the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32: ~1 ulp f32 each, as WGSL's exp
// on a GPU), 5-7 VALU operations per value instead of ~30 for a libm exp and an IEEE division — the GLU epilogue
// runs 32 of them per lane with one wave per SIMD. Limits: a -> -inf gives a * rcp(inf) = -0, a -> +inf gives a.
__device__ __forceinline__ float act_silu(float a) {
  return a * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * a));
}
__device__ __forceinline__ float act_gelu_tanh(float x) {
  const float u = fminf(fmaxf(0.7978845608f * (x + 0.044715f * x * x * x), -15.0f), 15.0f);
  const float e = __builtin_amdgcn_exp2f(2.8853900817779268f * u);  // exp(2u), e in [e^-30, e^30]
  return 0.5f * x * (1.0f + (e - 1.0f) * __builtin_amdgcn_rcpf(e + 1.0f));
}

// GELU with the Abramowitz & Stegun 7.1.26 erf (|error| < 1.5e-7) of Laya's GELU_MUL (encoder-kernels.ts:30-40),
// its reciprocal and exp on the hardware units
__device__ __forceinline__ float act_gelu_erf(float x) {
  const float z = 0.70710678f * x, az = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * az);
  const float y = 1.0f - ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) *
                             t * __builtin_amdgcn_exp2f(-1.4426950408889634f * z * z);
  return 0.5f * x * (1.0f + (z >= 0.0f ? y : -y));
}

struct GemmArgs {
  const uint16_t *X;
  const uint8_t *Wc;
  const uint32_t *Ws;
  uint16_t *Y;
  float *ws;          // split-K workspace [S, M, N] f32 (N physical columns: a gated weight's interleaved blocks)
  int M, N, K, act, tiles_m, tiles_n, splits, ksteps;  // ksteps: 64-K steps per split
  // q/k norm + RoPE epilogue (EPI 2; the tile is one 128-wide head): norm weights, the forward's per-token
  // (cos, sin) table [M, rot / 2], heads layout
  const uint16_t *qn, *kn;
  const float2 *rtab;
  int heads, kv, vnorm, rot;
  float eps;
  // residual epilogue (plain products, dj_matmul_residual): R += f16(acc) in place, XW = f16(R * nw * XW_SCALE),
  // SS[m, n / 32] = the unrounded sums squared over each 32-column block. Y is not written.
  uint16_t *resid;
  const uint16_t *nw;
  uint16_t *xw;
  float *ssout;
  // row norm (dj_matmul_normed): every accumulator row times 1 / (XW_SCALE sqrt(sum_b ssin[m, b] / Hn + neps))
  // over Hn / 32 <= 32 blocks before any other epilogue step
  const float *ssin;
  int Hn;
  float neps;
};

// The pre-scale of a residual epilogue's XW (and its inverse in the row norm): XW = R * w / 4 keeps |XW| < 65504
// for norm weights up to 4 at any f16 residual value.
constexpr float XW_SCALE = 0.25f;


// Ring of LDS stages, each holding one 64-K step of the tile: A (BM rows x 128 bytes, XOR-swizzled 16-byte
// chunks), the NB weight blocks of B in their global lane order, and (quantized B) each block's 16 scale words.
// WK = 2: two K wave sets split every paired-ring step pair (a step each), each set accumulating the whole
// WM x WN wave tile; the sets' partial tiles are added through LDS at the end. Against a wave row twice as
// wide on the same A rows, a wave reads half the A fragments per MFMA, and the per-pair chain (barrier,
// fragment reads, dequantization, MFMAs) is one step long.
template <int BITS, int WM, int WN, int FM, int FN, int RING, int WK = 1>
struct GemmShape {
  static constexpr int NW = WM * WN * WK, NT = NW * 64;
  static constexpr int BM = WM * FM * 16, BN = WN * FN * 16, NB = BN / 16;
  static constexpr int CB = BITS == 8 ? 1024 : BITS == 4 ? 512 : 2048;  // bytes per 16x64 weight block
  static constexpr int A_BYTES = BM * 128;
  static constexpr int B_BYTES = (NB * CB + 1023) / 1024 * 1024;      // whole 1 KB DMA rows
  static constexpr int S_BYTES = BITS == 16 ? 0 : NW * 256;           // one 256-byte DMA row per wave
  static constexpr int STAGE = A_BYTES + B_BYTES + S_BYTES;
  // ring depth (NS - 1 steps in flight): RING, or 0 = the deepest of 4 / 3 that fits. Shallower rings leave
  // LDS for more workgroups per CU, which on MI355X hides more latency than a deeper ring does.
  // (a RING deeper than LDS holds, e.g. for the twice-as-large f16 weight blocks, is cut to what fits)
  static constexpr int NS_FIT = 160 * 1024 / STAGE;
  // RING < 0: a paired ring of -RING stages (steps land, and the workgroup synchronizes, two at a time), cut to
  // the even depth LDS holds; where that is under 4 (f16 weight blocks on wide tiles) a plain 2-stage ring
  static constexpr int NS_PAIR = -RING < (NS_FIT & ~1) ? -RING : (NS_FIT & ~1);
  static constexpr bool PAIRED = RING < 0 && NS_PAIR >= 4;
  static constexpr int NS = PAIRED ? NS_PAIR : RING < 0 ? 2 : RING ? (RING < NS_FIT ? RING : NS_FIT)
                                                                     : 4 * STAGE <= 160 * 1024 ? 4 : 3;
  static constexpr int TA = A_BYTES / 1024, IA = (TA + NW - 1) / NW; // 16-byte-per-lane DMAs per wave and step
  static constexpr int TB = B_BYTES / 1024, IB = (TB + NW - 1) / NW;
  static constexpr int IS = BITS == 16 ? 0 : 1;                       // 4-byte-per-lane DMA (scales)
  static constexpr int I = IA + IB + IS;                              // vector-memory ops per wave and step
  static_assert(A_BYTES % 1024 == 0, "A stage must split into whole 1 KB rows");
  static_assert(NB <= 4 * NW, "scale rows cover 4 blocks per wave");
  static_assert(NS >= 2 && (NS - 2) * I < 64, "vmcnt range");
  static_assert(!PAIRED || (NS % 2 == 0 && NS >= 4 && (NS / 2 - 2) * 2 * I < 64), "paired ring");
  static_assert(NS * STAGE <= 160 * 1024, "LDS");
  // LDS: the ring, or the K wave sets' partial tiles where those are larger (they reuse the ring's bytes)
  static constexpr int RED = (WK - 1) * BM * BN * 4, SMEM = NS * STAGE > RED ? NS * STAGE : RED;
  static_assert(SMEM <= 160 * 1024, "LDS for the partial tiles");
  // waves per SIMD that LDS allows (workgroups per CU x waves per workgroup / 4 SIMDs): the register budget
  // the compiler may use without costing occupancy. Left to itself it squeezes a 128x128 tile to 120 VGPRs
  // to reach 4 waves per SIMD that LDS never grants, serializing the fragment reads (9-15% slower at 1536 x
  // 2048 x 11008, measured).
  static constexpr int WG_PER_CU = 160 * 1024 / SMEM;
  static constexpr int WPE_RAW = WG_PER_CU * NW / 4;
  static constexpr int WPE = WPE_RAW < 1 ? 1 : WPE_RAW > 8 ? 8 : WPE_RAW;
  // MFMA loop order: weight fragment outermost where LDS holds occupancy to <= 3 waves per SIMD (up to 168
  // VGPRs free: every A fragment of the step is read ahead, 110 vs 127 us at 1536 x 2048 x 11008 on
  // 128x128n); row fragment outermost otherwise (the register-lean order: 128x256 on 8 waves keeps 4 waves
  // per SIMD at 116 VGPRs, where the other order's 136 cost 14-17% at 86016 rows).
};

// wait_vm_barrier with at most n (clamped to [0, MAXN]) steps of I DMAs each left in flight; n is
// wave-uniform, so this is a scalar branch to one immediate
template <int I, int MAXN>
__device__ __forceinline__ void wait_steps_barrier(int n) {
  if constexpr (MAXN <= 0) {
    wait_vm_barrier<0>();
  } else {
    if (n >= MAXN) wait_vm_barrier<MAXN * I>();
    else wait_steps_barrier<I, MAXN - 1>(n);
  }
}

// wait_vm with at most n (clamped to [0, MAXN]) steps of I DMAs each left in flight (no barrier)
template <int I, int MAXN>
__device__ __forceinline__ void wait_steps(int n) {
  if constexpr (MAXN <= 0) {
    wait_vm<0>();
  } else {
    if (n >= MAXN) wait_vm<MAXN * I>();
    else wait_steps<I, MAXN - 1>(n);
  }
}

// EPI: 0 plain store, 1 gated MLP, 2 QK_NORM_ROPE on a qkv weight (kernels.ts:86-112) before the store, 3 plain
// product into the residual epilogue (dj_matmul_residual); 4 + (0, 1 or 2): that epilogue after the row norm of
// dj_matmul_normed (every accumulator row times 1 / (XW_SCALE rms) from the producer's partial sums)
template <int BITS, int WM, int WN, int FM, int FN, int RING, int EPI, int WK>
__global__ __launch_bounds__(WM *WN *WK * 64)
__attribute__((amdgpu_waves_per_eu(1, GemmShape<BITS, WM, WN, FM, FN, RING, WK>::WPE))) void k_gemm(GemmArgs g) {
  using S = GemmShape<BITS, WM, WN, FM, FN, RING, WK>;
  static_assert(WK == 1 || (WK == 2 && S::PAIRED), "K wave sets take a paired ring's steps");
  constexpr int BASE = EPI & 3;
  constexpr bool GLU = BASE == 1, ROPE = BASE == 2, RES = EPI == 3, RN = (EPI & 4) != 0;
  static_assert(!RN || WK == 1 || !ROPE, "the row norm's scales are shared through a workgroup barrier: every wave "
                                         "live (K wave sets share the epilogue, except on RoPE tiles)");
  static_assert(!RES || FN % 2 == 0, "the residual epilogue sums 32-column blocks (fragment pairs)");
  constexpr int NW = S::NW, BM = S::BM, NB = S::NB, CB = S::CB, NS = S::NS;
  constexpr int A_BYTES = S::A_BYTES, B_BYTES = S::B_BYTES, STAGE = S::STAGE;
  // the row norm's per-row scales sit past the ring
  constexpr int RN_OFF = S::SMEM, RN_BYTES = RN ? (BM * 4 + 1023) / 1024 * 1024 : 0;
  static_assert(S::SMEM + RN_BYTES <= 160 * 1024, "LDS for the row norm's scales");
  static_assert(!RN || BM <= S::NT, "a lane per row for the row norm");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[S::SMEM + RN_BYTES];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wk = wave / (WM * WN), wm = (wave % (WM * WN)) / WN, wn = wave % WN;
  // Two K wave sets share the epilogue by fragment rows: set 0 takes i < FH, set 1 the rest (a RoPE tile needs
  // whole heads: set 0 alone).
  constexpr bool KSPLIT = WK > 1 && !ROPE;
  constexpr int FH = (FM + 1) / 2;
  auto mine = [&](int i) { return !KSPLIT || ((i < FH) == (wk == 0)); };
  int tm, tn;
  map_tile(blockIdx.x, g.tiles_m, g.tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * (WN * FN * 16);
  const int M = g.M, K = g.K, KT = g.K >> 6;
  const int kbeg = blockIdx.y * g.ksteps;  // this split's first 64-K step
  const int KS = g.ksteps;

  f4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

  // The accumulator layout: lane l holds output row l % 16 of each 16x16 fragment and its columns 4 (l / 16)..+3.
  const int mrow = m0 + wm * FM * 16 + (lane & 15), c4 = 4 * (lane >> 4);
  const int N = g.N;
  // Epilogue inputs loaded before the ring starts (their loads are older than the ring's DMAs, so the ring's
  // exact counter waits only get stricter). Row norm: lane r < BM of the workgroup loads row m0 + r's nb = Hn /
  // 32 partial sums (nb <= 32, a multiple of 4: whole 16-byte loads), waits for them alone once the prologue's
  // DMAs are issued, and leaves the row's scale in LDS for the epilogue. Residual: the tile's stream values and
  // norm weights, into registers.
  f4 rnp[RN ? 8 : 1];
  if constexpr (RN) {
    const int nb4 = g.Hn >> 7;
    const f4 *src = (const f4 *)(g.ssin + (size_t)min(m0 + tid, M - 1) * (g.Hn >> 5));
#pragma unroll
    for (int c = 0; c < 8; ++c) rnp[c] = (f4){0.f, 0.f, 0.f, 0.f};
    if (tid < BM) {
#pragma unroll
      for (int c = 0; c < 8; ++c)
        if (c < nb4) rnp[c] = src[c];
    }
  }
  h4 rx[RES ? FM : 1][RES ? FN : 1], rw[RES ? FN : 1];
  if (RES && (KSPLIT || wk == 0)) {  // each wave set its own epilogue rows
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * FN * 16 + j * 16 + c4;
      rw[j] = *(const h4 *)(g.nw + n);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        if (mine(i)) rx[i][j] = *(const h4 *)(g.resid + (size_t)min(mrow + i * 16, M - 1) * N + n);
    }
  }

  // Per-lane DMA sources at step 0 of the split (a step adds 128 bytes to A, one block to B and scales).
  // A row q (1 KB = 8 rows of the tile): lane L fills LDS chunk L of it = row 8q + L/8, physical chunk L%8,
  // which holds logical chunk (L%8) ^ (row % 8).
  // Waves past the last row (BM not a multiple of 8 NW) repeat it: same bytes, same place.
  const uint16_t *asrc[S::IA];
  int adst[S::IA];
#pragma unroll
  for (int i = 0; i < S::IA; ++i) {
    const int q = min(wave * S::IA + i, S::TA - 1), r = 8 * q + (lane >> 3), c = (lane & 7) ^ (r & 7);
    asrc[i] = g.X + (size_t)min(m0 + r, M - 1) * K + (size_t)kbeg * 64 + c * 8;
    adst[i] = __builtin_amdgcn_readfirstlane(q * 1024);
  }
  const int nb0 = n0 >> 4;  // the tile's first weight block row
  const uint8_t *bsrc[S::IB];
  int bdst[S::IB];
#pragma unroll
  for (int i = 0; i < S::IB; ++i) {
    const int q = min(wave + NW * i, S::TB - 1);  // waves past the last row repeat it (same bytes, same place)
    int j, off;
    if constexpr (BITS == 8) { j = q; off = lane * 16; }
    else if constexpr (BITS == 4) { j = min(2 * q + (lane >> 5), NB - 1); off = (lane & 31) * 16; }
    else { j = q >> 1; off = (q & 1) * 1024 + lane * 16; }
    bsrc[i] = g.Wc + ((size_t)(nb0 + j) * KT + kbeg) * CB + off;
    bdst[i] = __builtin_amdgcn_readfirstlane(A_BYTES + q * 1024);
  }
  const uint32_t *ssrc = nullptr;
  if constexpr (S::IS) {
    const int j = min(wave * 4 + (lane >> 4), NB - 1);
    ssrc = g.Ws + ((size_t)(nb0 + j) * KT + kbeg) * 16 + (lane & 15);
  }

  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int kt, int slot) {
    const uint32_t st = lds0 + slot * STAGE;
#pragma unroll
    for (int i = 0; i < S::IA; ++i) dma16(asrc[i] + kt * 64, st + adst[i]);
#pragma unroll
    for (int i = 0; i < S::IB; ++i) dma16(bsrc[i] + (size_t)kt * CB, st + bdst[i]);
    if constexpr (S::IS) dma4(ssrc + kt * 16, st + A_BYTES + B_BYTES + wv * 256);
  };

  // Fragments of one step in registers: A (FM x 2 k-halves of 16 rows x 32 K), raw B and scale words.
#define DJ_READ(step, A_, R_, P_)                                                                        \
  {                                                                                                      \
    const uint8_t *st_ = smem + ((step) % NS) * STAGE;                                                   \
    const u32x4 *As_ = (const u32x4 *)st_;                                                               \
    _Pragma("unroll") for (int i = 0; i < FM; ++i) _Pragma("unroll") for (int s = 0; s < 2; ++s) {       \
      const int r = wm * FM * 16 + i * 16 + (lane & 15), ch = s * 4 + (lane >> 4);                       \
      A_[i][s] = __builtin_bit_cast(h8, As_[r * 8 + (ch ^ (r & 7))]);                                    \
    }                                                                                                    \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) {                                                     \
      const int jb = wn * FN + j;                                                                        \
      if constexpr (BITS == 8) R_[j].v = *(const u32x4 *)(st_ + A_BYTES + jb * CB + lane * 16);          \
      else if constexpr (BITS == 4) R_[j].v = *(const u32x2 *)(st_ + A_BYTES + jb * CB + lane * 8);      \
      else {                                                                                             \
        R_[j].v0 = *(const u32x4 *)(st_ + A_BYTES + jb * CB + lane * 32);                                \
        R_[j].v1 = *(const u32x4 *)(st_ + A_BYTES + jb * CB + lane * 32 + 16);                           \
      }                                                                                                  \
      P_[j] = S::IS ? *(const uint32_t *)(st_ + A_BYTES + B_BYTES + jb * 64 + (lane & 15) * 4) : 0u;     \
    }                                                                                                    \
  }
#define DJ_MMA(A_, R_, P_)                                                                               \
  _Pragma("unroll") for (int s = 0; s < 2; ++s) {                                                        \
    h8 bf[FN];                                                                                           \
    _Pragma("unroll") for (int j = 0; j < FN; ++j) bf[j] = dequant<BITS>(R_[j], s, P_[j]);               \
    if constexpr (S::WPE <= 3) {                                                                         \
      _Pragma("unroll") for (int j = 0; j < FN; ++j)                                                     \
        _Pragma("unroll") for (int i = 0; i < FM; ++i) acc[i][j] = MFMA16(bf[j], A_[i][s], acc[i][j]);   \
    } else {                                                                                             \
      _Pragma("unroll") for (int i = 0; i < FM; ++i)                                                     \
        _Pragma("unroll") for (int j = 0; j < FN; ++j) acc[i][j] = MFMA16(bf[j], A_[i][s], acc[i][j]);   \
    }                                                                                                    \
  }

  // Steps are issued only while they exist: before the wait for step t, steps up to min(t + NS - 3, KS - 1)
  // have been issued (min(NS - 2, KS - 1) for t = 0), so min(NS - 3, KS - 1 - t) later steps may still be in
  // flight — the full ring depth until the tail, then exact counts (no re-loads of the last step to wait for).
  // prologue: steps 0 .. NS-2 in flight (paired ring: pairs 0 .. NS/2-2, steps 0 .. NS-3)
  constexpr int PRO = S::PAIRED ? NS - 2 : NS - 1;
#pragma unroll
  for (int p = 0; p < PRO; ++p)
    if (p < KS) issue(p, p);
  if constexpr (RN) {
    // the row sums have landed (older than the prologue's DMAs, which stay in flight): the row's scale
    // 1 / (XW_SCALE rms) into LDS, read by the epilogue after its barrier
    wait_steps<S::I, PRO>(min(PRO, KS));
    f4 p = rnp[0];
#pragma unroll
    for (int c = 1; c < 8; ++c) p += rnp[c];
    const float ssum = (p[0] + p[1]) + (p[2] + p[3]);
    if (tid < BM)
      ((float *)(smem + RN_OFF))[tid] = rsqrtf(ssum * (1.0f / (float)g.Hn) + g.neps) * (1.0f / XW_SCALE);
  }

  if constexpr (S::PAIRED && WK > 1) {
    // Paired ring with two K wave sets: the pair's waits, barrier and DMAs as below; set wk then reads and
    // multiplies step 2 kp + wk only (an odd count's last step: set 0).
    constexpr int NP = NS / 2;
    const int KP = KS / 2;
    for (int kp = 0; kp < KP; ++kp) {
      wait_steps_barrier<S::I, NS - 4>(min(NS - 4, KS - 2 * kp - 2));
      const int nx = kp + NP - 1;
      if (2 * nx < KS) issue(2 * nx, (2 * nx) % NS);
      if (2 * nx + 1 < KS) issue(2 * nx + 1, (2 * nx + 1) % NS);
      h8 a0[FM][2];
      RawB<BITS> r0[FN];
      uint32_t p0[FN];
      DJ_READ(2 * kp + wk, a0, r0, p0);
      DJ_MMA(a0, r0, p0);
    }
    if (KS & 1) {  // the last step alone: every DMA has been issued; all of them land, then the barrier
      wait_vm_barrier<0>();
      if (wk == 0) {
        h8 a0[FM][2];
        RawB<BITS> r0[FN];
        uint32_t p0[FN];
        DJ_READ(KS - 1, a0, r0, p0);
        DJ_MMA(a0, r0, p0);
      }
    }
  } else if constexpr (S::PAIRED) {
    // Paired ring (NP = NS / 2 pairs of stages): steps land two at a time, so the counter wait and the
    // workgroup barrier come once per 128 K. At pair p: steps 2p + 2 .. 2p + NS - 3 may still be in flight; after
    // the barrier every wave is done with pair p-1, whose stages take pair p+NP-1. Both steps' fragments are read
    // before the first MFMA. An odd step count issues its last step alone, and computes it after the pairs.
    constexpr int NP = NS / 2;
    const int KP = KS / 2;
    h8 a0[FM][2], a1[FM][2];
    RawB<BITS> r0[FN], r1[FN];
    uint32_t p0[FN], p1[FN];
    for (int kp = 0; kp < KP; ++kp) {
      // steps issued so far: min(KS, NS - 2 + 2 kp); steps 0 .. 2 kp + 1 must have landed
      wait_steps_barrier<S::I, NS - 4>(min(NS - 4, KS - 2 * kp - 2));
      const int nx = kp + NP - 1;
      if (2 * nx < KS) issue(2 * nx, (2 * nx) % NS);
      if (2 * nx + 1 < KS) issue(2 * nx + 1, (2 * nx + 1) % NS);
      DJ_READ(2 * kp, a0, r0, p0);
      DJ_READ(2 * kp + 1, a1, r1, p1);
      DJ_MMA(a0, r0, p0);
      DJ_MMA(a1, r1, p1);
    }
    if (KS & 1) {  // the last step alone
      wait_vm_barrier<0>();
      DJ_READ(KS - 1, a0, r0, p0);
      DJ_MMA(a0, r0, p0);
    }
  } else if constexpr (NS == 2) {
    // two stages: read a step's fragments right after its barrier, then compute it
    for (int kt = 0; kt < KS; ++kt) {
      // this wave's DMAs of step kt are done (nothing later is in flight); after the barrier every wave's
      // are, and every wave has finished reading step kt-1's stage, which is refilled next
      wait_vm_barrier<0>();
      if (kt + 1 < KS) issue(kt + 1, (kt + 1) % NS);
      h8 fa[FM][2];
      RawB<BITS> fr[FN];
      uint32_t fp[FN];
      DJ_READ(kt, fa, fr, fp);
      DJ_MMA(fa, fr, fp);
    }
  } else {
    // three or more stages: step k+1's fragments are read into the other register set while step k's MFMAs
    // run, so LDS latency overlaps the matrix work. At half-step k: step k+1 has landed, and after the barrier
    // every wave is done with step k-1 (read at k-2, used at k-1), whose stage takes step k+NS-1.
    h8 a0[FM][2], a1[FM][2];
    RawB<BITS> r0[FN], r1[FN];
    uint32_t p0[FN], p1[FN];
    wait_steps_barrier<S::I, NS - 2>(min(NS - 2, KS - 1));
    DJ_READ(0, a0, r0, p0);
    int kt = 0;
    for (; kt + 2 <= KS; kt += 2) {
      wait_steps_barrier<S::I, NS - 3>(KS - 2 - kt);
      if (kt + NS - 1 < KS) issue(kt + NS - 1, (kt + NS - 1) % NS);
      DJ_READ(kt + 1, a1, r1, p1);
      DJ_MMA(a0, r0, p0);
      wait_steps_barrier<S::I, NS - 3>(KS - 3 - kt);
      if (kt + NS < KS) issue(kt + NS, (kt + NS) % NS);
      DJ_READ(kt + 2, a0, r0, p0);  // kt + 2 == KS: a stale stage, read and unused
      DJ_MMA(a1, r1, p1);
    }
    if (kt < KS) DJ_MMA(a0, r0, p0);  // odd step count: the last step's fragments are in set 0
  }
#undef DJ_READ
#undef DJ_MMA
  wait_vm<0>();  // the clamped tail DMAs land before the wave moves on

  if constexpr (WK > 1) {
    // The K wave sets' partial tiles meet in the (now idle) ring. Split epilogue: each set leaves the fragments
    // the other one stores and adds the other's to its own (a + b == b + a: the same bits as one set adding
    // both). Otherwise sets 1 .. WK-1 leave theirs and set 0 adds them in set order and runs the epilogue alone.
    f4 *part = (f4 *)smem;
    constexpr int FR = FM * FN;  // fragments per wave
    __syncthreads();  // every DMA has landed and every wave is past its last fragment read
    if constexpr (KSPLIT) {
      static_assert(WK == 2, "the split epilogue pairs two wave sets");
#pragma unroll
      for (int i = 0; i < FM; ++i)
        if (!mine(i))
#pragma unroll
          for (int j = 0; j < FN; ++j) part[((wm * WN + wn) * FR + i * FN + j) * 64 + lane] = acc[i][j];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < FM; ++i)
        if (mine(i))
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] += part[((wm * WN + wn) * FR + i * FN + j) * 64 + lane];
    } else {
      if (wk > 0) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            part[(((wk - 1) * WM * WN + wm * WN + wn) * FR + i * FN + j) * 64 + lane] = acc[i][j];
      }
      __syncthreads();
      if (wk > 0) return;
#pragma unroll
      for (int k = 0; k < WK - 1; ++k)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] += part[((k * WM * WN + wm * WN + wn) * FR + i * FN + j) * 64 + lane];
    }
  }

  // The MFMAs take the weight fragment as their first operand, so each accumulator holds a 16x16 block of
  // Y^T: lane l has output row l%16 of the block and its 4 consecutive columns 4(l/16)..+3 — one 8-byte f16
  // (16-byte f32) store instead of four scattered 2-byte ones.
  if constexpr (RN) {  // row norm: the consumer side of a residual epilogue
    const float *scale = (const float *)(smem + RN_OFF);
    __syncthreads();  // every row's scale is in LDS
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const float rs = scale[wm * FM * 16 + i * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] *= rs;
    }
  }
  if (g.splits > 1) {
    // this split's partial tile, f32, into its slice; k_splitk_sum finishes the product
    float *slice = g.ws + (size_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int m = mrow + i * 16, n = n0 + wn * FN * 16 + j * 16 + c4;
        if (mine(i) && m < M) *(f4 *)(slice + (size_t)m * N + n) = acc[i][j];
      }
    return;
  }

  if constexpr (ROPE) {
    // The tile is one head of a qkv product (BN = D = 128, tile column n0 = head * 128). q and k heads (and v
    // heads with vnorm): the f16-rounded tile goes to LDS (the ring is free: every DMA has landed), then
    // LPH lanes per row run QK_NORM_ROPE's arithmetic (norm_rope_lane, shared with k_qk_norm_rope, cos/sin from
    // the forward's table) and store the row. Other v heads take the plain store below.
    // rows padded to 136 halves (272 bytes) so neighbouring rows start on different LDS banks
    constexpr int RS = 136;
    static_assert(BM * RS * 2 <= NS * STAGE, "the f16 tile fits the ring");
    const int hh = n0 >> 7;
    const bool isQ = hh < g.heads, isK = !isQ && hh < g.heads + g.kv;
    if (isQ || isK || g.vnorm) {
      uint16_t *tile = (uint16_t *)smem;
      __syncthreads();  // every wave is past its last fragment read
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          h4 v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = (_Float16)acc[i][j][r];
          *(h4 *)(tile + (wm * FM * 16 + i * 16 + (lane & 15)) * RS + wn * FN * 16 + j * 16 + c4) = v;
        }
      __syncthreads();
      const uint16_t *nw = isQ ? g.qn : isK ? g.kn : nullptr;
      const bool norm = isQ ? g.qn != nullptr : isK ? g.kn != nullptr : true;
      auto rows = [&](auto lph) {
        constexpr int LPH = decltype(lph)::value, RPP = S::NT / LPH, PASSES = (BM + RPP - 1) / RPP;
        const int rot = g.rot, half = rot / 2, npl = rot / 16, ntl = (128 - rot) / 8;
        const int sub = tid % LPH;
        const bool pl = sub < npl, tl = !pl && sub < npl + ntl;
        const int d0 = pl ? 8 * sub : rot + 8 * (sub - npl);
        h8 wx = {}, wy = {};
        if (nw && (pl || tl)) {
          wx = *(const h8 *)(nw + d0);
          if (pl) wy = *(const h8 *)(nw + half + d0);
        }
        // every pass's row values and angles are loaded before the first is computed, so their latencies
        // overlap (a lane group's rows are r0, r0 + RPP, ...; rows past BM or M are skipped as a group)
        h8 xs[PASSES], ys[PASSES];
        float2 cs[PASSES][8];
#pragma unroll
        for (int q = 0; q < PASSES; ++q) {
          const int r = tid / LPH + q * RPP, m = m0 + r;
          xs[q] = h8{};
          ys[q] = h8{};
          if (r < BM && m < M) {
            if (pl || tl) xs[q] = *(const h8 *)(tile + r * RS + d0);
            if (pl) ys[q] = *(const h8 *)(tile + r * RS + half + d0);
            if (pl && (isQ || isK)) {
              const float4 *c4p = (const float4 *)(g.rtab + (size_t)m * half + d0);
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float4 v = c4p[i];
                cs[q][2 * i] = make_float2(v.x, v.y);
                cs[q][2 * i + 1] = make_float2(v.z, v.w);
              }
            }
          }
        }
#pragma unroll
        for (int q = 0; q < PASSES; ++q) {
          const int r = tid / LPH + q * RPP, m = m0 + r;
          if (r >= BM || m >= M) continue;
          const h8x2 o = norm_rope_lane<LPH>(xs[q], ys[q], wx, wy, nw != nullptr, norm, isQ || isK, pl, 128, g.eps,
                                             [&](int i) { return cs[q][i]; });
          uint16_t *z = g.Y + (size_t)m * N + (size_t)hh * 128;
          if (pl) {
            *(h8 *)(z + d0) = o.x;
            *(h8 *)(z + half + d0) = o.y;
          } else if (tl) {
            *(h8 *)(z + d0) = o.x;
          }
        }
      };
      // the standalone kernel's lane counts: 8 lanes for a fully rotated head, 16 for a partial rotation
      if (g.rot == 128) rows(std::integral_constant<int, 8>{});
      else rows(std::integral_constant<int, 16>{});
      return;
    }
  }

  if constexpr (RES) {
    {
      // residual epilogue: per 32-column block (fragments j, j + 1) the lane's 8 values, then the row's four
      // lanes added, written by the first of them
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (!mine(i)) continue;
        const int m = mrow + i * 16;
#pragma unroll
        for (int j = 0; j < FN; j += 2) {
          float part = 0.f;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int n = n0 + wn * FN * 16 + (j + h) * 16 + c4;
            const h4 x = rx[i][j + h], w = rw[j + h];
            h4 xo, xwo;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float v = (float)x[r] + (float)(_Float16)acc[i][j + h][r];
              part += v * v;
              xo[r] = (_Float16)v;
              xwo[r] = (_Float16)((float)xo[r] * (float)w[r] * XW_SCALE);
            }
            if (m < M) {
              *(h4 *)(g.resid + (size_t)m * N + n) = xo;
              *(h4 *)(g.xw + (size_t)m * N + n) = xwo;
            }
          }
          part += __shfl_xor(part, 16);
          part += __shfl_xor(part, 32);
          if (m < M && lane < 16) g.ssout[(size_t)m * (N >> 5) + ((n0 + wn * FN * 16 + j * 16) >> 5)] = part;
        }
      }
      return;
    }
  }
  if constexpr (!GLU) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int m = mrow + i * 16, n = n0 + wn * FN * 16 + j * 16 + c4;
        h4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (_Float16)acc[i][j][r];
        if (mine(i) && m < M) *(h4 *)(g.Y + (size_t)m * N + n) = v;
      }
  } else {
    const int I = N >> 1;
    const int wb0 = nb0 + wn * FN;
    // The activation is chosen once, outside the unrolled fragments, and every value is formed before the
    // first store: a per-value switch (or a store guard between values) puts each value's exp / rcp chain in
    // a branch region of its own, and the chains then run one after another instead of interleaved.
    auto gated = [&](auto act) {
      h4 v[FM][FN / 2];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; j += 2)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float a = (float)(_Float16)acc[i][j][r], b = (float)(_Float16)acc[i][j + 1][r];
            v[i][j / 2][r] = (_Float16)(act(a) * b);
          }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; j += 2) {
          const int m = mrow + i * 16;
          const int col = ((wb0 + j) >> 1) * 16 + c4;  // physical block p even -> w1 block p / 2
          if (mine(i) && m < M) *(h4 *)(g.Y + (size_t)m * I + col) = v[i][j / 2];
        }
    };
    if (g.act == DJ_ACT_SILU) gated([](float a) { return act_silu(a); });
    else if (g.act == DJ_ACT_GELU_TANH) gated([](float a) { return act_gelu_tanh(a); });
    else gated([](float a) { return act_gelu_erf(a); });
  }
}

// Split-K finish: Y = epilogue(sum over splits of the f32 slices, in split order — the same bits whatever the
// schedule). Plain: 4 outputs per thread. Gated: output column c = 16 q + o takes its gate from physical column
// 32 q + o and its up value from 32 q + 16 + o (the load-time block interleave), each rounded to f16 first, as
// the tiled epilogue does.
template <bool GLU>
__global__ __launch_bounds__(256) void k_splitk_sum(const float *__restrict__ ws, int splits, int M, int N, int act,
                                                    uint16_t *__restrict__ Y, uint16_t *__restrict__ R,
                                                    const uint16_t *__restrict__ nw, uint16_t *__restrict__ XW,
                                                    float *__restrict__ SS) {
  const int NO = GLU ? N / 2 : N;  // output columns
  const long e = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= (long)M * NO) return;  // whole 8-thread groups (M N is a multiple of 32 where R is given)
  const int m = (int)(e / NO), c = (int)(e % NO);
  const size_t slice = (size_t)M * N;
  if constexpr (!GLU) {
    const float *p = ws + (size_t)m * N + c;
    f4 s = *(const f4 *)p;
    for (int k = 1; k < splits; ++k) s += *(const f4 *)(p + k * slice);
    if (R) {  // the residual epilogue of the tiled kernel; 8 consecutive threads hold one 32-column block
      const h4 x = *(const h4 *)(R + e), w = *(const h4 *)(nw + c);
      h4 xo, xwo;
      float part = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (float)x[r] + (float)(_Float16)s[r];
        part += v * v;
        xo[r] = (_Float16)v;
        xwo[r] = (_Float16)((float)xo[r] * (float)w[r] * XW_SCALE);
      }
      *(h4 *)(R + e) = xo;
      *(h4 *)(XW + e) = xwo;
      part += __shfl_xor(part, 1);
      part += __shfl_xor(part, 2);
      part += __shfl_xor(part, 4);
      if ((c & 31) == 0) SS[(size_t)m * (N >> 5) + (c >> 5)] = part;
      return;
    }
    h4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = (_Float16)s[r];
    *(h4 *)(Y + e) = v;
  } else {
    const float *p = ws + (size_t)m * N + (c >> 4) * 32 + (c & 15);
    f4 a = *(const f4 *)p, b = *(const f4 *)(p + 16);
    for (int k = 1; k < splits; ++k) {
      a += *(const f4 *)(p + k * slice);
      b += *(const f4 *)(p + k * slice + 16);
    }
    h4 v;
    auto gated = [&](auto fn) {  // the activation chosen once (the four values' chains interleave)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (_Float16)(fn((float)(_Float16)a[r]) * (float)(_Float16)b[r]);
    };
    if (act == DJ_ACT_SILU) gated([](float x) { return act_silu(x); });
    else if (act == DJ_ACT_GELU_TANH) gated([](float x) { return act_gelu_tanh(x); });
    else gated([](float x) { return act_gelu_erf(x); });
    *(h4 *)(Y + (size_t)m * NO + c) = v;
  }
}

// ---------------------------------------------------------------- skinny M (GEMV-style, M <= 64)
// The skinny products' accumulation: KW waves take the KS 64-K steps from k0 round-robin (wave w: steps w,
// w + KW, ...; BATCH of them loaded at once), each into its own accumulators (blocks of Y^T: weight fragment
// first).
template <int BITS, int MT, int CB, bool WIDE, int BATCH>
__device__ __forceinline__ void gemv_accumulate(const GemmArgs &g, f4 (&acc)[MT][CB], int wave, int lane, int KW, int nb0,
                                                int k0, int KS) {
  constexpr int CBYTES = BITS == 8 ? 1024 : BITS == 4 ? 512 : 2048;
  const int M = g.M, K = g.K, KT = K >> 6;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};
  const uint16_t *xr[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) xr[i] = g.X + (size_t)min(16 * i + (lane & 15), M - 1) * K + (lane >> 4) * 8;

  for (int kb = wave; kb < KS; kb += KW * BATCH) {
    h8 a[BATCH][MT][2];
    RawB<BITS> b[BATCH][CB];
    uint32_t sp[BATCH][CB];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      // past the end: skipped (WIDE, wave-uniform) or the last step re-loaded; neither is accumulated
      if (WIDE && kb + q * KW >= KS) break;
      const int kt = k0 + min(kb + q * KW, KS - 1);
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int s = 0; s < 2; ++s) a[q][i][s] = *(const h8 *)(xr[i] + kt * 64 + s * 32);
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const size_t blk = (size_t)(nb0 + j) * KT + kt;
        if constexpr (BITS == 8) b[q][j].v = *(const u32x4 *)(g.Wc + blk * CBYTES + lane * 16);
        else if constexpr (BITS == 4) b[q][j].v = *(const u32x2 *)(g.Wc + blk * CBYTES + lane * 8);
        else {
          b[q][j].v0 = *(const u32x4 *)(g.Wc + blk * CBYTES + lane * 32);
          b[q][j].v1 = *(const u32x4 *)(g.Wc + blk * CBYTES + lane * 32 + 16);
        }
        sp[q][j] = BITS == 16 ? 0u : g.Ws[blk * 16 + (lane & 15)];
      }
    }
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      if (kb + q * KW < KS) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int j = 0; j < CB; ++j) {
            const h8 bf = dequant<BITS>(b[q][j], s, sp[q][j]);
#pragma unroll
            for (int i = 0; i < MT; ++i) acc[i][j] = MFMA16(bf, a[q][i][s], acc[i][j]);
          }
      }
    }
  }
}

// Below a few dozen rows the product is bound by streaming the weights, and a tile grid has too few
// workgroups to keep HBM busy. Measured (graph replay, q8): 0.85 TB/s at M = 1 and 0.4-0.6 TB/s at M = 32
// on 1536-2048-wide weights, 2-3x the tiled kernel; the limit is that each workgroup re-reads X from L2
// (M / 8.5 times the weight bytes at 16 columns per workgroup). Here a workgroup owns CB 16-column weight blocks (CB = 2 for a gated weight:
// its gate and up blocks) and all of K; its KW waves take the 64-K steps round-robin. A wave loads BATCH
// steps at once — weight blocks (16 bytes per lane, already in MFMA lane order), scale words and the X
// fragments (L2-resident) — straight into registers, then runs their MFMAs; with up to 16 waves per
// workgroup that keeps enough weight bytes in flight. The waves' partial tiles are added through LDS in wave
// order (deterministic), and wave 0 runs the same epilogue as the tiled kernel.
//
// MAXW is the most waves a launch may use. MAXW = 16: 128 VGPRs per lane, so a batch stages about 80 VGPRs
// (3 steps at M = 32) and past-the-end steps re-load the last one. MAXW = 8 (the default launch): two waves
// per SIMD, 256 VGPRs per lane, so a batch stages about 176 VGPRs (9 steps at M = 32: all of a 4608-long K
// over 8 waves in one round trip) and loads past the end are skipped, not repeated.
template <int BITS, int MT, int CB, bool GLU, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void k_gemv(GemmArgs g) {
  // steps per load batch: the staging budget above over the VGPRs of one step (X fragments 8 MT, weight
  // blocks 4 or 8 and a scale word per block)
  constexpr bool WIDE = MAXW <= 8;
  constexpr int PER_STEP = 8 * MT + (BITS == 16 ? 8 : 5) * CB;
  constexpr int BUDGET = WIDE ? 176 : 80, BMAX = WIDE ? 12 : 8;
  constexpr int BATCH = BUDGET / PER_STEP < 1 ? 1 : BUDGET / PER_STEP > BMAX ? BMAX : BUDGET / PER_STEP;
  __shared__ f4 red[(MAXW - 1) * MT * CB * 64];
  // `wave` through readfirstlane: the batch guards below must be scalar branches. As vector compares they
  // become EXEC-masked regions, and an MFMA runs whatever EXEC says, so a skipped slot would still add its
  // (unloaded) registers into the accumulator.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, KW = blockDim.x >> 6;
  const int nb0 = blockIdx.x * CB;
  const int M = g.M;
  // split along K (gridDim.y > 1): this workgroup takes the KS steps from k0 and leaves f32 partials
  const int KS = g.ksteps, k0 = blockIdx.y * KS;

  f4 acc[MT][CB];
  gemv_accumulate<BITS, MT, CB, WIDE, BATCH>(g, acc, wave, lane, KW, nb0, k0, KS);

  // partial tiles of waves 1.. through LDS, added by wave 0 in wave order
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) red[(((wave - 1) * MT + i) * CB + j) * 64 + lane] = acc[i][j];
  }
  __syncthreads();
  if (wave > 0) return;
  for (int w = 1; w < KW; ++w)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) acc[i][j] += red[(((w - 1) * MT + i) * CB + j) * 64 + lane];

  // accumulators hold blocks of Y^T (weight fragment first): lane l has row 16 i + l%16 and the 4 consecutive
  // columns 4(l/16)..+3 of a 16-column block, one 8-byte store
  const int N = g.N, c4 = 4 * (lane >> 4);
  if (gridDim.y > 1) {  // a K split: f32 partial rows [split][M][N], summed in split order by the consumer
    if constexpr (!GLU) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          const int m = 16 * i + (lane & 15), n = (nb0 + j) * 16 + c4;
          if (m < M) *(f4 *)(g.ws + ((size_t)blockIdx.y * M + m) * N + n) = acc[i][j];
        }
    }
    return;
  }
  if constexpr (!GLU) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const int m = 16 * i + (lane & 15), n = (nb0 + j) * 16 + c4;
        h4 v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (_Float16)acc[i][j][r];
        if (m < M) *(h4 *)(g.Y + (size_t)m * N + n) = v;
      }
  } else {
    static_assert(!GLU || CB == 2, "a gated weight pairs gate and up blocks");
    const int I = N >> 1, col = (nb0 >> 1) * 16 + c4;  // block pair (2p, 2p + 1) -> w1/w3 block p
    // the activation chosen once and every value formed before the stores (as the tiled epilogue)
    auto gated = [&](auto fn) {
      h4 v[MT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          v[i][r] = (_Float16)(fn((float)(_Float16)acc[i][0][r]) * (float)(_Float16)acc[i][1][r]);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = 16 * i + (lane & 15);
        if (m < M) *(h4 *)(g.Y + (size_t)m * I + col) = v[i];
      }
    };
    if (g.act == DJ_ACT_SILU) gated([](float x) { return act_silu(x); });
    else if (g.act == DJ_ACT_GELU_TANH) gated([](float x) { return act_gelu_tanh(x); });
    else gated([](float x) { return act_gelu_erf(x); });
  }
}

// Waves per workgroup for the skinny kernel: about two steps each, 4..8 waves on the wide-batch form.
// DJ_GEMV_WAVES=<n> (1..16) forces the count (tuning sweeps; above 8 the 16-wave form runs).
static int gemv_waves(int KT) {
  const char *s = getenv("DJ_GEMV_WAVES");
  const int forced = s ? atoi(s) : 0;
  if (forced >= 1 && forced <= 16) return forced;
  return KT / 2 < 4 ? 4 : KT / 2 > 8 ? 8 : KT / 2;
}

template <int BITS, bool GLU, int MAXW>
static void launch_gemv_w(hipStream_t s, GemmArgs a, int waves) {
  constexpr int CB = GLU ? 2 : 1;
  const dim3 grid(a.N / 16 / CB, a.splits), block(64 * waves);
  if (a.M <= 16) k_gemv<BITS, 1, CB, GLU, MAXW><<<grid, block, 0, s>>>(a);
  else if (a.M <= 32) k_gemv<BITS, 2, CB, GLU, MAXW><<<grid, block, 0, s>>>(a);
  else k_gemv<BITS, 4, CB, GLU, MAXW><<<grid, block, 0, s>>>(a);
}

template <int BITS, bool GLU>
static void launch_gemv(hipStream_t s, GemmArgs a) {
  const int waves = gemv_waves(a.ksteps);
  if (waves <= 8) launch_gemv_w<BITS, GLU, 8>(s, a, waves);
  else launch_gemv_w<BITS, GLU, 16>(s, a, waves);
}

// ---------------------------------------------------------------- dispatch

// Tile configurations: waves along M and N, 16x16 fragments per wave along M and N, ring, K wave sets.
struct GemmCfg {
  const char *tag;
  int wm, wn, fm, fn, ring, wk;
  int bm() const { return wm * fm * 16; }
  int bn() const { return wn * fn * 16; }
};
// tag "<BM>x<BN>[s<ring>]": waves along M and N, 16x16 fragments per wave along M and N, LDS ring depth;
// "n": one wave row (every wave spans all BM rows and owns distinct columns, so no two waves dequantize the
// same weight fragment)
#define DJ_GEMM_CFGS(X)                                                                                    \
  X(0, "256x128", 2, 2, 8, 4, 0, 1) X(1, "128x128", 2, 2, 4, 4, 0, 1) X(2, "128x64", 2, 2, 4, 2, 0, 1)              \
  X(3, "64x128", 2, 2, 2, 4, 0, 1) X(4, "64x64", 2, 2, 2, 2, 0, 1) X(5, "32x128", 1, 4, 2, 2, 0, 1)                 \
  X(6, "128x32", 4, 1, 2, 2, 0, 1) X(7, "128x16", 4, 1, 2, 1, 0, 1) X(8, "32x64", 1, 4, 2, 1, 0, 1)                 \
  X(9, "64x32", 2, 2, 2, 1, 0, 1) X(10, "128x128s2", 2, 2, 4, 4, 2, 1) X(11, "128x128s3", 2, 2, 4, 4, 3, 1)         \
  X(12, "256x128s2", 2, 2, 8, 4, 2, 1) X(13, "128x256", 2, 2, 4, 8, 0, 1) X(14, "128x256s2", 2, 2, 4, 8, 2, 1)      \
  X(15, "64x64s2", 2, 2, 2, 2, 2, 1) X(16, "32x128s2", 1, 4, 2, 2, 2, 1) X(17, "64x128s2", 2, 2, 2, 4, 2, 1)        \
  X(18, "128x64s2", 2, 2, 4, 2, 2, 1) X(19, "128x128n", 1, 4, 8, 2, 2, 1) X(20, "128x128n3", 1, 4, 8, 2, 3, 1)        \
  X(21, "64x128n", 1, 4, 4, 2, 2, 1) X(22, "128x256n", 1, 4, 8, 4, 2, 1) X(23, "64x256n", 1, 4, 4, 4, 2, 1)        \
  X(24, "144x128n", 1, 4, 9, 2, 2, 1) X(25, "144x64n", 1, 4, 9, 1, 2, 1) X(26, "96x128n", 1, 4, 6, 2, 2, 1)         \
  X(27, "48x128n", 1, 4, 3, 2, 2, 1) X(28, "144x128n4", 1, 4, 9, 2, 4, 1) X(29, "144x128n5", 1, 4, 9, 2, 5, 1)        \
  X(30, "144x64n4", 1, 4, 9, 1, 4, 1) X(31, "144x64n6", 1, 4, 9, 1, 6, 1) X(32, "128x128n4", 1, 4, 8, 2, 4, 1)        \
  X(33, "128x128n6", 1, 4, 8, 2, 6, 1) X(34, "64x128n4", 1, 4, 4, 2, 4, 1) X(35, "64x128n6", 1, 4, 4, 2, 6, 1)        \
  X(36, "144x128w8", 1, 8, 9, 1, 2, 1) X(37, "144x128w8r3", 1, 8, 9, 1, 3, 1) X(38, "128x128w8", 2, 4, 4, 2, 2, 1)     \
  X(39, "64x128w8", 1, 8, 4, 1, 2, 1) X(40, "32x64w8", 2, 4, 1, 1, 0, 1) X(41, "128x256w8", 1, 8, 8, 2, 2, 1)          \
  X(42, "128x128w8r3", 2, 4, 4, 2, 3, 1) X(43, "64x128w8r4", 1, 8, 4, 1, 4, 1)                                    \
  X(44, "32x64p4", 1, 4, 2, 1, -4, 1) X(45, "32x64p6", 1, 4, 2, 1, -6, 1) X(46, "128x128np4", 1, 4, 8, 2, -4, 1)      \
  X(47, "128x256w8p4", 1, 8, 8, 2, -4, 1) X(48, "64x128np4", 1, 4, 4, 2, -4, 1) X(49, "144x64np4", 1, 4, 9, 1, -4, 1)      \
  X(50, "144x128np4", 1, 4, 9, 2, -4, 1) X(51, "48x64k2", 1, 2, 3, 2, -4, 2)        \
  X(52, "64x64k2", 1, 2, 4, 2, -4, 2) X(53, "80x64k2", 1, 2, 5, 2, -4, 2) X(54, "96x64k2", 1, 2, 6, 2, -4, 2)        \
  X(55, "64x128k2", 1, 4, 4, 2, -4, 2) X(56, "80x64k2p8", 1, 2, 5, 2, -8, 2) X(57, "96x64k2p8", 1, 2, 6, 2, -8, 2)
#define DJ_CFG_ROW(i, tag, wm, wn, fm, fn, ring, wk) {tag, wm, wn, fm, fn, ring, wk},
static const GemmCfg kCfgs[] = {DJ_GEMM_CFGS(DJ_CFG_ROW)};
static const int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// Whether a tile's LDS holds the row norm's sums past its ring (EPI 4-6) for these weight bits.
template <int BITS, int WM, int WN, int FM, int FN, int RING, int WK>
constexpr bool rn_fits_cfg() {
  return GemmShape<BITS, WM, WN, FM, FN, RING, WK>::SMEM + (WM * FM * 16 * 4 + 1023) / 1024 * 1024 <= 160 * 1024 &&
         WM * FM * 16 <= WM * WN * WK * 64;
}
template <int BITS>
static bool rn_fits(int i) {
  switch (i) {
#define DJ_RN_CASE(i, tag, wm, wn, fm, fn, ring, wk) \
  case i: return rn_fits_cfg<BITS, wm, wn, fm, fn, ring, wk>();
    DJ_GEMM_CFGS(DJ_RN_CASE)
#undef DJ_RN_CASE
  }
  return false;
}

// The tiles built with the folded-norm epilogues (EPI 3-6): every tile the policy picks for a product of more
// than 64 rows on the decoders' shapes, including the small-grid fallbacks; the rest are sweep-only tiles, not
// built in those forms (cfg_fits keeps the policy off them there).
constexpr bool fused_cfg(int i) {
  switch (i) {
    case 1: case 4: case 5: case 8: case 15: case 16: case 19: case 21: case 24: case 25: case 41: case 44: case 46:
    case 47: case 50: case 51: case 52: case 53: case 54: case 55: case 56: case 57:
      return true;
    default:
      return false;
  }
}

template <int BITS, int WM, int WN, int FM, int FN, int RING, int EPI, int WK, bool FZ>
static void launch_cfg(hipStream_t s, GemmArgs a) {
  constexpr int BASE = EPI & 3;
  if constexpr (((BASE == 1 || EPI == 3) && FN % 2 != 0) ||
                (BASE == 2 && (WN * FN * 16 != 128 || WM * FM * 16 > 144 || WK > 1)) ||
                (WK > 1 && !GemmShape<BITS, WM, WN, FM, FN, RING, WK>::PAIRED) || (EPI >= 3 && !FZ) ||
                ((EPI & 4) && !rn_fits_cfg<BITS, WM, WN, FM, FN, RING, WK>())) {
    return;  // never picked (cfg_fits): a gated tile and the residual epilogue need fragment pairs, a RoPE tile
             // is one 128-wide head of at most 144 rows (its epilogue holds every row pass in registers) on one
             // set of waves, K wave sets need their paired ring, the folded-norm forms exist for fused_cfg tiles
  } else {
    dim3 grid(a.tiles_m * a.tiles_n, a.splits);
    k_gemm<BITS, WM, WN, FM, FN, RING, EPI, WK><<<grid, WM * WN * WK * 64, 0, s>>>(a);
  }
}

template <int BITS, int EPI>
static void launch_index(int i, hipStream_t s, GemmArgs a) {
#define DJ_CFG_CASE(i, tag, wm, wn, fm, fn, ring, wk) \
  case i: launch_cfg<BITS, wm, wn, fm, fn, ring, EPI, wk, fused_cfg(i)>(s, a); break;
  switch (i) { DJ_GEMM_CFGS(DJ_CFG_CASE) }
#undef DJ_CFG_CASE
}

// A K wave set tile needs its paired ring: at least 4 stages of its shape in LDS for these weight bits (a
// 128x256 tile of direct f16 weights holds only 3).
static bool ksets_fit(const GemmCfg &c, int bits) {
  if (c.wk == 1) return true;
  const int nw = c.wm * c.wn * c.wk, cb = bits == 8 ? 1024 : bits == 4 ? 512 : 2048;
  const int stage = c.bm() * 128 + (c.bn() / 16 * cb + 1023) / 1024 * 1024 + (bits == 16 ? 0 : nw * 256);
  return std::min(-c.ring, (160 * 1024 / stage) & ~1) >= 4;
}

// epi (the kernel's EPI): 0 plain, 1 gated (gate/up fragment pairs), 2 RoPE (one 128-wide head per tile, <= 144
// rows), 3 plain with the residual epilogue (32-column blocks: fragment pairs); + 4: the row norm first. The
// folded-norm forms (3-6) exist for fused_cfg tiles only.
static bool cfg_fits(const GemmCfg &c, int N, int K, int epi, int bits) {
  const int base = epi & 3;
  return ksets_fit(c, bits) && N % c.bn() == 0 && ((base != 1 && epi != 3) || c.fn % 2 == 0) &&
         (base != 2 || (c.bn() == 128 && c.bm() <= 144 && c.wk == 1)) && (epi < 3 || fused_cfg((int)(&c - kCfgs))) &&
         (!(epi & 4) || (bits == 8    ? rn_fits<8>((int)(&c - kCfgs))
                         : bits == 4 ? rn_fits<4>((int)(&c - kCfgs))
                                     : rn_fits<16>((int)(&c - kCfgs)))) &&
         (c.ring >= 0 || K / 64 >= 2);  // a paired ring takes 64-K steps two at a time (an odd count's last
                                         // step alone)
}

// Picks (tile, splits). DJ_GEMM_TILE=<tag> and DJ_GEMM_SPLITK=<n> force them (tuning sweeps). Otherwise, from
// sweeps on MI355X with warm clocks (q8; M 1152-86016; the decoders' N and K), first rule that fits:
//   128x256w8p4 when its tiles fill one round (0.75-1 per CU): one 8-wave workgroup per CU, so the paired
//               4-stage ring costs no occupancy (the 1152-row GLU: 216 tiles, 18.3-18.9 us against 19.5-21.8
//               for 128x128n),
//   128x256w8   when it gives >= 8 tiles per CU (large M: 950-980 TFLOP/s at 86016 rows, 3-8% over 128x128n;
//               at 1536 rows the 3B GLU's 1032 tiles ran 3% slower than 128x128n),
//   128x128n    when it gives >= 1.5 tiles per CU, or >= 0.5 per CU when K >= 4096 (few long tiles beat many
//               short ones: 3B's w2) — on the paired 4-stage ring (128x128np4) where those fill one round: the
//               3B w2 (192 tiles at 1536 rows) takes its weights cold from HBM in the forward, and the deeper ring
//               took the 3B ticket from 12.35 to 11.76 ms (same box),
//   144x64n     when it gives >= 2 tiles per CU (1152-row qkv: 8 x 64 = 512 tiles, two per CU: 15-16 us
//               against 17-18 for 64x128n),
//   64x128n     when it gives >= 2 tiles per CU,
//   K wave set tiles (two wave sets, K / 64 even, K >= 2048; plain products, and residual ones from K = 1024,
//               where the 32x64 tiles cannot hold the epilogue's 32-column sums): 80x64k2p8 or 96x64k2p8 where
//               their tiles make one round at one workgroup per CU (0.75-1 per CU: the 8-stage paired ring keeps three pairs
//               of weight blocks in flight, which is what products on weights cold in HBM wait for), else the one of
//               48x64k2 / 64x64k2 / 80x64k2 / 96x64k2 (4 stages) whose grid is nearest 1.5 per CU, where that is
//               1-3 per CU (below one per CU, e.g. the 0.8B state's 8-question pass at 256 rows, it measured
//               slower in the forward than the rules below; so did K = 1024, Laya's 1152 x 3072 / 1024 x 1024
//               products on weights cold in HBM: 2.875 vs 2.818 ms per Laya ticket). In the ticket's forward (T = 1152, same box): 80x64k2p8 for o_proj / w2, 2.534 ms
//               per ticket, against 2.63 for 32x64p4 and for 48x64k2 (alone with weights cold in HBM, w2 16.8-18.0
//               vs 19.3-20.5 us; with weights in the MALL 48x64k2 is the faster, 15.8-17.5 us, which the forward
//               does not see). Alone, MALL-resident weights, against 32x64p4: 1152 x 2048 x 1024 10.2 vs 13.6 us,
//               1536 x 2048 x 2048 q4 19.7 vs 28.0, 1280 x 1024 x 3584 18.5 vs 23.2, 576 x 1024 x 2048 10.8 vs
//               10.8 (15.8 for the 128x16 the rules below gave it),
//   32x64p4     when it gives >= 2 tiles per CU (the paired 4-stage ring, K / 64 even), else 32x64,
//   32x128s2    the same for gated weights (a GLU tile needs gate/up fragment pairs),
//   else the tile with the most workgroups, split along K when even that leaves most CUs idle (skinny M).
static void pick(int M, int N, int K, int epi, int bits, int cus, size_t ws_floats, int &cfg, int &splits) {
  const bool ws_ok = ws_floats > 0;
  const char *force = getenv("DJ_GEMM_TILE");
  const char *fs = getenv("DJ_GEMM_SPLITK");
  cfg = -1;
  splits = 1;
  if (force)
    for (int i = 0; i < kNumCfgs; ++i)
      if (!strcmp(force, kCfgs[i].tag) && cfg_fits(kCfgs[i], N, K, epi, bits)) cfg = i;
  auto tiles = [&](int i) { return (long)dj_cdiv(M, kCfgs[i].bm()) * (N / kCfgs[i].bn()); };
  // the qkv product with the RoPE epilogue: 144x128 on a paired 4-stage ring where its tiles fill one round (one
  // workgroup per CU, so the deeper ring costs no occupancy; the 1152-row qkv, 256 tiles: 2.628 -> 2.616 ms
  // per ticket, same box)
  if (cfg < 0 && (epi & 3) == 2 && cfg_fits(kCfgs[50], N, K, epi, bits) && tiles(50) >= 0.75 * cus && tiles(50) <= cus) cfg = 50;
  // long K on at most one round of tiles (0.25-1 per CU): 128x128n split 4 ways along K (alone on cold weights,
  // the summing kernel included: the 3B w2, 1536 x 2048 x 11008 q4, 92.9 us against 107.0 on the paired ring;
  // the 0.8B prefill's w2, 1024 x 1536 x 4608 q8, 32.8 against 36.6); below that, 64x128n split 4 ways at
  // 0.1-0.25 tiles per CU (the 0.8B 8-question pass's w2, 256 x 1536 x 4608: 19.7 against 23.8 on 32x64);
  // DJ_GEMM_LONGK_SPLIT=1 keeps the paired ring unsplit
  const char *kss = getenv("DJ_GEMM_KSETS");  // DJ_GEMM_KSETS=0: no K wave set tiles (A/B sweeps)
  const bool ksets_off = kss && atoi(kss) == 0;
  const char *kst = getenv("DJ_GEMM_KSET_TILE");
  const char *kmk = getenv("DJ_GEMM_KSET_MINK");  // the plain products' least K for the K wave set tiles
  const int kset_mink = kmk ? atoi(kmk) : 2048;
  const char *lks = getenv("DJ_GEMM_LONGK_SPLIT");
  // A K wave set tile on the 8-stage ring that makes one round (0.75-1 tiles per CU) takes long-K products up to
  // K = 8192 ahead of the split (the omni trunk's 1152 x 1024 x 4608 w2: 25-27 against 29.8 us alone, its ticket
  // 1.933 -> 1.898 ms; fewer rows, e.g. the 0.8B prefill's 1024 x 1536 x 4608 at 312 tiles, keep the split,
  // which measured faster in its forward). DJ_GEMM_LONGK_KSET=0 keeps the split everywhere.
  const char *lkk = getenv("DJ_GEMM_LONGK_KSET");
  bool longk_kset = !(lkk && atoi(lkk) == 0) && K <= 8192 && !ksets_off;
  if (longk_kset) {
    bool round = false;
    for (int i : {56, 57})
      round = round || (cfg_fits(kCfgs[i], N, K, epi, bits) && tiles(i) >= 0.75 * cus && tiles(i) <= cus);
    longk_kset = round;
  }
  const int longk = lks ? atoi(lks) : 4;
  int rule_splits = 0;
  if (cfg < 0) {
    static const struct { int cfg; double per_cu; int min_k; double max_per_cu; int ks; } rules[] = {
        {47, 0.75, 0, 1.0, 0}, {41, 8.0, 0, 1e9, 0}, {19, 1.5, 0, 1e9, 0}, {19, 0.25, 4096, 1.0, -1}, {19, 0.5, 4096, 1e9, 0},
        {21, 0.1, 4096, 0.25, -1},
        {25, 2.0, 0, 1e9, 0}, {24, 1.0, 0, 1e9, 0}, {21, 2.0, 0, 1e9, 0}, {-2, 1.0, 0, 3.0, 0}, {44, 2.0, 0, 1e9, 0},
        {8, 2.0, 0, 1e9, 0}, {16, 2.0, 0, 1e9, 0}};
    for (const auto &r : rules) {
      if (r.cfg == -2) {  // the K wave set family (see above)
        if ((epi & 3) == 1 || (epi & 3) == 2 || ksets_off || K < (epi == 3 ? 1024 : kset_mink)) continue;
        int best = -1;
        for (int i : {56, 57})  // one round of one-workgroup-per-CU tiles on the 8-stage ring, most tiles first
          if (best < 0 && cfg_fits(kCfgs[i], N, K, epi, bits) && tiles(i) >= 0.75 * cus && tiles(i) <= cus) best = i;
        if (best < 0) {  // else the 4-stage tile nearest 1.5 per CU, within the rule's bounds
          for (int i : {51, 52, 53, 54})
            if (cfg_fits(kCfgs[i], N, K, epi, bits) &&
                (best < 0 || std::abs(tiles(i) - 1.5 * cus) < std::abs(tiles(best) - 1.5 * cus)))
              best = i;
          if (best >= 0 && (tiles(best) < r.per_cu * cus || tiles(best) > r.max_per_cu * cus)) best = -1;
        }
        if (kst)  // DJ_GEMM_KSET_TILE=<tag>: this rule's tile (A/B sweeps inside a forward)
          for (int i = 0; i < kNumCfgs; ++i)
            if (!strcmp(kst, kCfgs[i].tag) && cfg_fits(kCfgs[i], N, K, epi, bits)) best = i;
        if (best >= 0) {
          cfg = best;
          break;
        }
        continue;
      }
      if (cfg_fits(kCfgs[r.cfg], N, K, epi, bits) && K >= r.min_k && tiles(r.cfg) >= r.per_cu * cus &&
          tiles(r.cfg) <= r.max_per_cu * cus) {
        // a residual epilogue in the split's summing kernel costs more than the K wave set tiles save: never split
        if (r.ks < 0 && (epi == 3 || longk_kset)) continue;
        if (r.ks < 0) {  // a long-K rule: the split where it divides K and fits the workspace; else what the rules
                         // chose before it (the paired ring at 0.5-1 per CU, otherwise the rules below)
          if (longk > 1 && ws_ok && (epi & 3) != 2 && (K / 64) % longk == 0 && (size_t)longk * M * N <= ws_floats) {
            rule_splits = longk;
          } else if (r.cfg == 19 && tiles(19) >= 0.5 * cus && cfg_fits(kCfgs[46], N, K, epi, bits)) {
            cfg = 46;
            break;
          } else {
            continue;
          }
        }
        cfg = r.cfg;
        break;
      }
    }
    if (cfg < 0) {  // nothing fills the chip: the tile with the most workgroups among those no taller than
                    // the rows need (a 128-row tile on 32 rows does 4x the matrix work: 25 us against 9 for
                    // 32x64 on M = 32, 1536 x 4608)
      static const int small[] = {8, 5, 4, 7, 9, 15, 16};  // 32x64, 32x128, 64x64, 128x16, 64x32, ...
      const int need = std::max(32, (M + 15) / 16 * 16);
      long best = -1;
      for (int pass = 0; pass < 2 && cfg < 0; ++pass)
        for (int i : small)
          if (cfg_fits(kCfgs[i], N, K, epi, bits) && (pass || kCfgs[i].bm() <= need) && tiles(i) > best) {
            cfg = i;
            best = tiles(i);
          }
    }
  }
  if (cfg < 0) return;
  const int KT = K / 64;
  if (fs) {
    splits = atoi(fs);
  } else if (rule_splits) {
    splits = rule_splits;
  } else {
    const long t = tiles(cfg);
    while (t * splits * 4 < cus && KT % (splits * 2) == 0 && KT / (splits * 2) >= 4) splits *= 2;
  }
  if (splits < 1 || KT % splits || !ws_ok || (epi & 3) == 2 || kCfgs[cfg].ring < 0) splits = 1;
}

// Profile labels "matmul[_glu|_rope]_<q4|q8|f16>_<tile>", built when the library loads.
static const struct GemmNames {
  char v[3][3][kNumCfgs][40];
  GemmNames() {
    static const char *const epi[3] = {"", "_glu", "_rope"};
    for (int b = 0; b < 3; ++b)
      for (int e = 0; e < 3; ++e)
        for (int i = 0; i < kNumCfgs; ++i)
          snprintf(v[b][e][i], 40, "matmul%s_%s_%s", epi[e], b == 0 ? "q4" : b == 1 ? "q8" : "f16", kCfgs[i].tag);
  }
} kNames;

static const char *const kGemvNames[3][2] = {{"matmul_q4_gemv", "matmul_glu_q4_gemv"},
                                             {"matmul_q8_gemv", "matmul_glu_q8_gemv"},
                                             {"matmul_f16_gemv", "matmul_glu_f16_gemv"}};

// launcher state: the split-K workspace lives in the context
int dj_gemm_workspace(dj_ctx *c, size_t need_floats, float **ws);

// fx: the residual epilogue or the row norm (GemmArgs' fields of those; tiled kernel only)
template <int BITS, bool GLU>
static int launch_bits(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int act, const char **name,
                       int *splits_out, const GemmArgs *fx = nullptr, bool split_ok = true) {
  const int N = w->N, K = w->K;
  const char *force = getenv("DJ_GEMM_TILE");
  // skinny M: the GEMV-style kernel on weights up to 4096 outputs wide, and on any weight for M <= 16 (M = 1
  // GLU 9216 x 1536: 6.8 us against 9.5-10.1 for tiles). At 17-64 rows wider weights give the tiled kernel
  // enough workgroups (M = 32 GLU 9216 x 1536: 9.8-10.3 against 13.3 us), measured on MI355X. (Long K stays
  // here: M = 32, 1536 x 4608 took 10.0 + 4.6 us tiled with split-K and its sum inside the 0.8B decoder's
  // forward, against about 12 for this kernel.)
  const bool skinny = !fx && M <= 64 && N % (GLU ? 32 : 16) == 0 &&
                      (force ? !strcmp(force, "gemv") : M <= 16 || N <= 4096);
  if (skinny) {
    GemmArgs a{};
    a.X = X; a.Wc = w->codes; a.Ws = (const uint32_t *)w->scales; a.Y = Y;
    a.M = M; a.N = N; a.K = K; a.act = act;
    a.splits = 1; a.ksteps = K / 64;
    launch_gemv<BITS, GLU>(c->stream, a);
    *name = kGemvNames[BITS == 4 ? 0 : BITS == 8 ? 1 : 2][GLU];
    *splits_out = 1;
    return DJ_OK;
  }
  float *ws = nullptr;
  int cfg, splits;
  const bool res = fx && fx->resid;
  const int epi = (GLU ? 1 : res ? 3 : 0) | (fx && fx->ssin ? 4 : 0);
  pick(M, N, K, epi, BITS, c->cus, c->gemm_ws && split_ok ? c->gemm_ws_floats : 0, cfg, splits);
  if (splits > 1 && dj_gemm_workspace(c, (size_t)splits * M * N, &ws) != DJ_OK) splits = 1;
  if (cfg < 0)
    return dj_fail(DJ_EINVAL, "decision.js: no matmul tile fits N = %d%s", N,
                   GLU ? " (gated: N % 32 == 0)" : res ? " (residual: N % 32 == 0)" : "");
  const char *label = kNames.v[BITS == 4 ? 0 : BITS == 8 ? 1 : 2][GLU][cfg];
  GemmArgs a{};
  a.X = X; a.Wc = w->codes; a.Ws = (const uint32_t *)w->scales; a.Y = Y; a.ws = ws;
  a.M = M; a.N = N; a.K = K; a.act = act;
  a.tiles_m = dj_cdiv(M, kCfgs[cfg].bm());
  a.tiles_n = N / kCfgs[cfg].bn();
  a.splits = splits;
  a.ksteps = (K / 64) / splits;
  if (fx) {
    a.resid = fx->resid; a.nw = fx->nw; a.xw = fx->xw; a.ssout = fx->ssout;
    a.ssin = fx->ssin; a.Hn = fx->Hn; a.neps = fx->neps;
  }
  switch (epi) {
    case 0: launch_index<BITS, 0>(cfg, c->stream, a); break;
    case 1: launch_index<BITS, 1>(cfg, c->stream, a); break;
    case 3: launch_index<BITS, 3>(cfg, c->stream, a); break;
    case 4: launch_index<BITS, 4>(cfg, c->stream, a); break;
    default: launch_index<BITS, 5>(cfg, c->stream, a); break;
  }
  if (splits > 1) {
    const long n4 = (long)M * (GLU ? N / 2 : N) / 4;
    k_splitk_sum<GLU><<<(unsigned)dj_cdiv(n4, 256), 256, 0, c->stream>>>(ws, splits, M, N, act, Y, a.resid, a.nw, a.xw,
                                                                           a.ssout);
  }
  *name = label;
  *splits_out = a.splits;
  return DJ_OK;
}

// The qkv product with QK_NORM_ROPE as its epilogue (one head per tile). Returns 1 with nothing launched where
// that does not apply: skinny M (the GEMV kernel serves those rows), no 128-wide tile fits, or more than two
// tiles per CU. The epilogue holds every row pass's values and angles in registers at once (256 VGPRs: one
// wave per SIMD), which pays where the grid is about one wave of tiles and the saved kernel is a large share
// (T = 1152: 3.00 against 3.10 ms per ticket), and costs where occupancy hides the loads (T = 86147: 118.6
// against 108.2 ms per forward), measured on MI355X.
template <int BITS>
static int launch_rope_bits(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Z, int M, GemmArgs a,
                            const char **name) {
  const int N = w->N, K = w->K;
  if (M <= 64) return 1;
  int cfg, splits;
  pick(M, N, K, a.ssin ? 6 : 2, BITS, c->cus, 0, cfg, splits);
  if (cfg < 0 || (long)dj_cdiv(M, kCfgs[cfg].bm()) * (N / 128) > 2L * c->cus) return 1;
  a.X = X; a.Wc = w->codes; a.Ws = (const uint32_t *)w->scales; a.Y = Z; a.ws = nullptr;
  a.M = M; a.N = N; a.K = K; a.act = 0;
  a.tiles_m = dj_cdiv(M, kCfgs[cfg].bm());
  a.tiles_n = N / 128;
  a.splits = 1;
  a.ksteps = K / 64;
  if (a.ssin) launch_index<BITS, 6>(cfg, c->stream, a);
  else launch_index<BITS, 2>(cfg, c->stream, a);
  *name = kNames.v[BITS == 4 ? 0 : BITS == 8 ? 1 : 2][2][cfg];
  return 0;
}

static __global__ __launch_bounds__(256) void k_rownorm_apply(int M, int H, const uint16_t *__restrict__ XW,
                                                              const float *__restrict__ SS, float eps,
                                                              uint16_t *__restrict__ O);
static int qkv_rope_impl(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Z, int M, int heads, int kv, int D,
                         const uint16_t *qn, const uint16_t *kn, int vnorm, const int32_t *pos, int pos_stride, float eps,
                         float theta, int rot, int mode, const float *tab, const float *SS, int H, float neps);
static int launch_gemm_fx(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int glu_act,
                          const char **name, int *splits, const GemmArgs *fx, bool split_ok = true);

extern "C" int dj_matmul_qkv_rope(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Z, int M, int heads, int kv,
                                  int D, const uint16_t *qn, const uint16_t *kn, int vnorm, const int32_t *pos,
                                  int pos_stride, float eps, float theta, int rot, int mode, const float *tab) {
  return qkv_rope_impl(rec, X, w, Z, M, heads, kv, D, qn, kn, vnorm, pos, pos_stride, eps, theta, rot, mode, tab, nullptr,
                       0, 0.f);
}

extern "C" int dj_matmul_qkv_rope_normed(dj_rec *rec, const uint16_t *XW, const dj_weight *w, uint16_t *Z, int M,
                                         int heads, int kv, int D, const uint16_t *qn, const uint16_t *kn, int vnorm,
                                         const int32_t *pos, int pos_stride, float eps, float theta, int rot, int mode,
                                         const float *tab, const float *SS, int H, float norm_eps) {
  DJ_REQUIRE(SS && H > 0 && H % 32 == 0 && H <= 2048 && w && w->K == H,
             "decision.js: matmul_qkv_rope_normed: bad norm arguments (H %d must be the weight's K, a multiple of 32, "
             "at most 2048)", H);
  return qkv_rope_impl(rec, XW, w, Z, M, heads, kv, D, qn, kn, vnorm, pos, pos_stride, eps, theta, rot, mode, tab, SS, H,
                       norm_eps);
}

static int qkv_rope_impl(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Z, int M, int heads, int kv, int D,
                         const uint16_t *qn, const uint16_t *kn, int vnorm, const int32_t *pos, int pos_stride, float eps,
                         float theta, int rot, int mode, const float *tab, const float *SS, int H, float neps) {
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == DJ_W_MFMA, "decision.js: matmul_qkv_rope needs an MFMA-tiled weight (DJ_W_MFMA)");
  DJ_REQUIRE(mode == DJ_ROPE_POW_NEG || mode == DJ_ROPE_INV_POW, "decision.js: matmul_qkv_rope: unknown rope mode");
  DJ_REQUIRE(X && Z && pos && tab && M >= 0 && heads > 0 && kv > 0 && D > 0 && D <= 512 &&
                 w->N == (heads + 2 * kv) * D && rot > 0 && rot <= D && rot % 16 == 0 && (D - rot) % 8 == 0,
             "decision.js: matmul_qkv_rope: bad arguments (N %d for %d + 2 x %d heads of %d, rot %d)", w->N, heads, kv,
             D, rot);
  DJ_OP_BEGIN(rec, SS ? "matmul_qkv_rope_normed" : "matmul_qkv_rope");
  const char *name = "matmul_qkv_rope";
  if (M > 0) {
    GemmArgs a{};
    a.qn = qn; a.kn = kn; a.rtab = (const float2 *)tab;
    a.heads = heads; a.kv = kv; a.vnorm = vnorm; a.rot = rot; a.eps = eps;
    a.ssin = SS; a.Hn = H; a.neps = neps;
    // skinny or wide rows (or H / 32 sums not in whole 16-byte loads): the normalized rows first (in the
    // workspace), then the plain form
    if (SS && (M <= 64 || H > 1024 || H % 128)) {
      float *ws = nullptr;
      DJ_REQUIRE(dj_gemm_workspace(rec->ctx, ((size_t)M * H + 1) / 2, &ws) == DJ_OK,
                 "decision.js: matmul_qkv_rope_normed: %d x %d rows exceed the workspace", M, H);
      k_rownorm_apply<<<(unsigned)dj_cdiv((long)M * (H / 32), 256), 256, 0, rec->ctx->stream>>>(M, H, X, SS, neps,
                                                                                               (uint16_t *)ws);
      X = (const uint16_t *)ws;
      a.ssin = nullptr;
    }
    const int bits = (w->layout & DJ_W_DIRECT) ? 16 : w->bits;
    int st = 1;
    if (D == 128)
      st = bits == 8 ? launch_rope_bits<8>(rec->ctx, X, w, Z, M, a, &name)
           : bits == 4 ? launch_rope_bits<4>(rec->ctx, X, w, Z, M, a, &name)
                       : launch_rope_bits<16>(rec->ctx, X, w, Z, M, a, &name);
    if (st == 1) {  // the product, then the standalone kernel (its angles computed as the table's were)
      int splits = 1;
      st = launch_gemm_fx(rec->ctx, X, w, Z, M, -1, &name, &splits, a.ssin ? &a : nullptr, !SS);
      if (st) return st;
      dj_launch_qk_norm_rope(rec->ctx->stream, M, heads, kv, D, w->N, Z, qn, kn, vnorm, pos, pos_stride, eps, theta, rot,
                             mode);
    }
  }
  char shape[48];  // (+rownorm: the normalized-rows form, so profiles tell it from the plain op)
  snprintf(shape, sizeof shape, "[%dx%dx%d]%s", M, w->N, w->K, SS ? "+rownorm" : "");
  return dj_op_end(rec, name, shape);
}

// split_ok = false: no split-K (the caller keeps its own data in the workspace)
static int launch_gemm_fx(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int glu_act,
                          const char **name, int *splits, const GemmArgs *fx, bool split_ok) {
  const bool glu = glu_act >= 0;
  const int bits = (w->layout & DJ_W_DIRECT) ? 16 : w->bits;
  if (bits == 8) return glu ? launch_bits<8, true>(c, X, w, Y, M, glu_act, name, splits, fx, split_ok) : launch_bits<8, false>(c, X, w, Y, M, 0, name, splits, fx, split_ok);
  if (bits == 4) return glu ? launch_bits<4, true>(c, X, w, Y, M, glu_act, name, splits, fx, split_ok) : launch_bits<4, false>(c, X, w, Y, M, 0, name, splits, fx, split_ok);
  return glu ? launch_bits<16, true>(c, X, w, Y, M, glu_act, name, splits, fx, split_ok) : launch_bits<16, false>(c, X, w, Y, M, 0, name, splits, fx, split_ok);
}

int dj_launch_gemm(dj_ctx *c, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M, int glu_act, const char **name,
                   int *splits) {
  return launch_gemm_fx(c, X, w, Y, M, glu_act, name, splits, nullptr);
}

// K splits for a held skinny product (1: not worth holding): two, where the 64-K steps divide evenly into
// splits of >= 8 and the grid stays within two workgroups per CU. Measured on the 0.8B decoder's question
// alone (M = 32; one box, two runs each): 2 splits 1.182 ms, 3-4 splits (w2 4, o_proj 3) 1.273 ms, no holding
// 1.274 ms — more splits make the GEMV no faster and the norm reads more partials. DJ_GEMV_SPLIT=0 turns
// holding off; DJ_GEMV_SPLIT=<n> forces n where it divides.
static int gemv_split_count(int M, int N, int K, int cus, size_t ws_floats) {
  const int KT = K / 64;
  const char *f = getenv("DJ_GEMV_SPLIT");
  if (f) {
    const int n = atoi(f);
    return n >= 2 && KT % n == 0 && (size_t)n * M * N <= ws_floats ? n : 1;
  }
  const int S = 2;
  return KT % S == 0 && KT / S >= 8 && (long)(N / 16) * S <= 2L * cus && (size_t)S * M * N <= ws_floats ? S : 1;
}

// A product the recorder may hold back by one op: plain (not gated), on the skinny kernel's rows, with a K
// split worth taking, and no forced tile (sweeps time what they issue).
static bool holdable(dj_rec *rec, const dj_weight *w, int M) {
  if (!rec || !rec->ctx || rec->ctx->active != rec || rec->replay || rec->error || getenv("DJ_GEMM_TILE")) return false;
  const int N = w->N, K = w->K;
  const bool skinny = M >= 1 && M <= 64 && N % 16 == 0 && (M <= 16 || N <= 4096);
  return skinny && gemv_split_count(M, N, K, rec->ctx->cus, rec->ctx->gemm_ws_floats) > 1;
}

static int matmul_now(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M);

extern "C" int dj_matmul(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M) {
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == DJ_W_MFMA, "decision.js: matmul needs an MFMA-tiled weight (DJ_W_MFMA)");
  DJ_REQUIRE(X && Y && M >= 0, "decision.js: matmul: bad arguments");
  if (holdable(rec, w, M)) {
    if (int st = dj_release_held(rec)) return st;  // one product held at a time
    rec->held.X = X;
    rec->held.w = w;
    rec->held.Y = Y;
    rec->held.M = M;
    rec->holding = true;
    return DJ_OK;
  }
  return matmul_now(rec, X, w, Y, M);
}

int dj_release_held(dj_rec *rec) {
  if (!rec || !rec->holding) return DJ_OK;
  rec->holding = false;
  return matmul_now(rec, rec->held.X, rec->held.w, rec->held.Y, rec->held.M);
}

int dj_take_held_split(dj_rec *rec, const uint16_t *Y, int T, int H, const float **parts, int *S) {
  *parts = nullptr;
  *S = 1;
  if (!rec || !rec->ctx || rec->ctx->active != rec || !rec->holding || rec->held.Y != Y || rec->held.M != T ||
      rec->held.w->N != H)
    return DJ_OK;
  rec->holding = false;
  dj_ctx *c = rec->ctx;
  const dj_weight *w = rec->held.w;
  const int M = T, N = w->N, K = w->K;
  const int splits = gemv_split_count(M, N, K, c->cus, c->gemm_ws_floats);
  if (splits < 2) return matmul_now(rec, rec->held.X, w, rec->held.Y, M);
  DJ_OP_BEGIN(rec, "matmul");
  GemmArgs a{};
  a.X = rec->held.X; a.Wc = w->codes; a.Ws = (const uint32_t *)w->scales; a.Y = rec->held.Y; a.ws = c->gemm_ws;
  a.M = M; a.N = N; a.K = K; a.act = 0;
  a.splits = splits; a.ksteps = (K / 64) / splits;
  const int bits = (w->layout & DJ_W_DIRECT) ? 16 : w->bits;  // direct weights: f16 blocks
  if (bits == 8) launch_gemv<8, false>(c->stream, a);
  else if (bits == 4) launch_gemv<4, false>(c->stream, a);
  else launch_gemv<16, false>(c->stream, a);
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]/k%d+norm", M, N, K, splits);
  if (int st = dj_op_end(rec, kGemvNames[bits == 4 ? 0 : bits == 8 ? 1 : 2][0], shape)) return st;
  *parts = c->gemm_ws;
  *S = splits;
  return DJ_OK;
}

static int matmul_now(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *Y, int M) {
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

// ---------------------------------------------------------------- residual + norm folded into the products
// Skinny rows (the GEMV kernel has no such epilogues): the same outputs by a small kernel after a plain product
// (dj_matmul_residual), or before it (dj_matmul_normed). One thread per (row, 32-column block).
__global__ __launch_bounds__(256) void k_residual_parts(int M, int N, const uint16_t *__restrict__ Y,
                                                        uint16_t *__restrict__ R, const uint16_t *__restrict__ nw,
                                                        uint16_t *__restrict__ XW, float *__restrict__ SS) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long)M * (N / 32)) return;
  const int m = (int)(t / (N / 32)), c0 = (int)(t % (N / 32)) * 32;
  const size_t base = (size_t)m * N + c0;
  float part = 0.f;
  for (int k = 0; k < 32; k += 8) {
    const h8 x = *(const h8 *)(R + base + k), y = *(const h8 *)(Y + base + k), w = *(const h8 *)(nw + c0 + k);
    h8 xo, xwo;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float v = (float)x[r] + (float)y[r];
      part += v * v;
      xo[r] = (_Float16)v;
      xwo[r] = (_Float16)((float)xo[r] * (float)w[r] * XW_SCALE);
    }
    *(h8 *)(R + base + k) = xo;
    *(h8 *)(XW + base + k) = xwo;
  }
  SS[(size_t)m * (N / 32) + c0 / 32] = part;
}

static __global__ __launch_bounds__(256) void k_rownorm_apply(int M, int H, const uint16_t *__restrict__ XW,
                                                              const float *__restrict__ SS, float eps,
                                                              uint16_t *__restrict__ O) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  const int nb = H / 32;
  if (t >= (long)M * nb) return;
  const int m = (int)(t / nb), c0 = (int)(t % nb) * 32;
  float s = 0.f;
  for (int b = 0; b < nb; ++b) s += SS[(size_t)m * nb + b];
  const float rs = (1.0f / sqrtf(s / (float)H + eps)) * (1.0f / XW_SCALE);
  for (int k = 0; k < 32; k += 8) {
    const h8 x = *(const h8 *)(XW + (size_t)m * H + c0 + k);
    h8 o;
#pragma unroll
    for (int r = 0; r < 8; ++r) o[r] = (_Float16)((float)x[r] * rs);
    *(h8 *)(O + (size_t)m * H + c0 + k) = o;
  }
}

extern "C" int dj_matmul_residual(dj_rec *rec, const uint16_t *X, const dj_weight *w, int M, uint16_t *R,
                                  const uint16_t *nw, uint16_t *XW, float *SS) {
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == DJ_W_MFMA, "decision.js: matmul_residual needs an MFMA-tiled weight (DJ_W_MFMA)");
  DJ_REQUIRE(X && R && nw && XW && SS && M >= 0 && w->N % 32 == 0,
             "decision.js: matmul_residual: bad arguments (N %d must be a multiple of 32)", w->N);
  DJ_OP_BEGIN(rec, "matmul_residual");
  const char *name = "matmul_residual";
  int splits = 1;
  const int N = w->N;
  if (M > 0 && M <= 64) {  // skinny rows: the plain product into the workspace, then the epilogue's arithmetic
    float *ws = nullptr;
    DJ_REQUIRE(dj_gemm_workspace(rec->ctx, ((size_t)M * N + 1) / 2, &ws) == DJ_OK,
               "decision.js: matmul_residual: %d x %d rows exceed the workspace", M, N);
    int st = launch_gemm_fx(rec->ctx, X, w, (uint16_t *)ws, M, -1, &name, &splits, nullptr, false);
    if (st) return st;
    k_residual_parts<<<(unsigned)dj_cdiv((long)M * (N / 32), 256), 256, 0, rec->ctx->stream>>>(M, N, (const uint16_t *)ws,
                                                                                              R, nw, XW, SS);
  } else if (M > 0) {
    GemmArgs fx{};
    fx.resid = R; fx.nw = nw; fx.xw = XW; fx.ssout = SS;
    int st = launch_gemm_fx(rec->ctx, X, w, nullptr, M, -1, &name, &splits, &fx);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]%s+residual", M, w->N, w->K, splits > 1 ? (splits == 2 ? "/k2" : splits == 4 ? "/k4" : "/k8") : "");
  return dj_op_end(rec, name, shape);
}

extern "C" int dj_matmul_normed(dj_rec *rec, const uint16_t *XW, const dj_weight *w, uint16_t *Y, int M, int act,
                                const float *SS, int H, float eps) {
  const bool glu = act >= 0;
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == (glu ? DJ_W_MFMA_GLU : DJ_W_MFMA),
             "decision.js: matmul_normed needs %s", glu ? "a fused w1|w3 weight (DJ_W_MFMA_GLU)" : "an MFMA-tiled weight (DJ_W_MFMA)");
  DJ_REQUIRE(XW && Y && SS && M >= 0 && H > 0 && H % 32 == 0 && H <= 2048 && w->K == H &&
                 (act < 0 || act == DJ_ACT_SILU || act == DJ_ACT_GELU_TANH || act == DJ_ACT_GELU_ERF),
             "decision.js: matmul_normed: bad arguments (H %d must be the weight's K, a multiple of 32, at most 2048)", H);
  DJ_OP_BEGIN(rec, glu ? "matmul_glu_normed" : "matmul_normed");
  const char *name = "matmul_normed";
  int splits = 1;
  // skinny or wide rows (or H / 32 sums not in whole 16-byte loads): the normalized rows first, then the product
  if (M > 0 && (M <= 64 || H > 1024 || H % 128)) {
    float *ws = nullptr;
    DJ_REQUIRE(dj_gemm_workspace(rec->ctx, ((size_t)M * H + 1) / 2, &ws) == DJ_OK,
               "decision.js: matmul_normed: %d x %d rows exceed the workspace", M, H);
    k_rownorm_apply<<<(unsigned)dj_cdiv((long)M * (H / 32), 256), 256, 0, rec->ctx->stream>>>(M, H, XW, SS, eps,
                                                                                             (uint16_t *)ws);
    int st = launch_gemm_fx(rec->ctx, (const uint16_t *)ws, w, Y, M, act, &name, &splits, nullptr, false);
    if (st) return st;
  } else if (M > 0) {
    GemmArgs fx{};
    fx.ssin = SS; fx.Hn = H; fx.neps = eps;
    int st = launch_gemm_fx(rec->ctx, XW, w, Y, M, act, &name, &splits, &fx);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[%dx%dx%d]%s+rownorm", M, w->N, w->K, splits > 1 ? (splits == 2 ? "/k2" : splits == 4 ? "/k4" : "/k8") : "");
  return dj_op_end(rec, name, shape);
}

extern "C" int dj_matmul_glu(dj_rec *rec, const uint16_t *X, const dj_weight *w, uint16_t *H, int M, int act) {
  DJ_REQUIRE(w && (w->layout & ~DJ_W_DIRECT) == DJ_W_MFMA_GLU, "decision.js: matmul_glu needs a fused w1|w3 weight (DJ_W_MFMA_GLU)");
  DJ_REQUIRE(X && H && M >= 0 && (act == DJ_ACT_SILU || act == DJ_ACT_GELU_TANH || act == DJ_ACT_GELU_ERF),
             "decision.js: matmul_glu: bad arguments");
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
