// Attention over per-query key ranges on gfx950 MFMA (flash-attention style, online softmax).
//
// Each query t reads two key ranges rng[t] = (a0, a1, b0, b1): rows [a0, a1) of source A and [b0, b1) of
// source B. That one form covers every mask of the reference: the causal forest of ATTENTION (a trunk token
// sees earlier trunk tokens, a branch token the whole trunk and its own branch up to itself,
// kernels.ts:133-136), the bidirectional segment or window of the encoders (eg2-kernels.ts:128-145), the
// trunk + branch ranges of attention256 (d3-kernels.ts:207-223), and a kept prefix KV (source A = the
// cache) in the shared-state mode.
//
// A workgroup takes 64 queries of one head (4 waves x 16; with KG = 2 key groups, 8 waves, each group scoring
// one half of every key tile with its own running max and sum, merged through LDS at the end). K/V tiles of
// 64 keys of the block's union range are staged in LDS: K row-major (XOR-swizzled 16-byte chunks), V
// transposed. Per wave and tile:
//   S^T[key, q] = K . Q^T       (A = K from LDS, B = Q held in registers; the accumulator puts query
//                                l % 16 in lane l, so the softmax row reduction is 2 shuffles)
//   O^T[d, q]  += V^T . P^T     (P^T is the S^T accumulator itself, rounded to f16; the key order inside
//                                each 32-key MFMA step is permuted to match, and V^T is read to match)
// Scores, the running max (m0 = -1e30) and the row sums are f32; the output is f16(acc / l), as the reference.
#include <math.h>
#include <algorithm>
#include <stdio.h>
#include <stdlib.h>
#include "dj_internal.h"

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)
typedef short s4 __attribute__((ext_vector_type(4)));

// LDS layout of one ring stage: K tile then V tile, 64 keys x D halves each, row-major (2D bytes per key) with
// 16-byte chunks XOR-swizzled per row. K: chunk c of key r at c ^ (r & KSW) (conflict-free 16-byte MFMA reads of
// 16 keys x one chunk). V: chunk c at c ^ vswz(r), chosen so the transposing reads below (4 keys x 2 chunks per
// 16 lanes) hit distinct banks.
template <int D, int RING, int KG, int HG>
struct AttnShape {
  static_assert(KG == 1 || HG == 1, "key groups and head groups are not combined");
  static constexpr int NW = 4 * KG * HG;                        // waves per workgroup
  static constexpr int CH = D / 8;                              // 16-byte chunks per key row
  static constexpr int KSW = CH >= 16 ? 15 : 7;
  static constexpr int TILE = 64 * 2 * D;                       // bytes of K (or V) per 64-key tile
  static constexpr int STAGE = 2 * TILE;
  // ring depth: RING, or 0 = 4 stages where they fit in 128 KB, else 2
  static constexpr int NS = RING ? RING : 4 * STAGE <= 128 * 1024 ? 4 : 2;
  static constexpr int IK = TILE / 1024 / NW;                   // 1 KB DMAs per wave per tile, K (and V)
  static_assert(TILE % (1024 * NW) == 0, "a tile must split into whole 1 KB DMAs per wave");
  static constexpr int I = 2 * IK;                              // vector-memory ops per wave per tile
  static_assert((NS - 2) * I < 64, "vmcnt range");
  __device__ static int vswz(int r) { return D >= 128 ? 2 * (r & 7) : 2 * ((r >> 1) & 3); }
};

// Max and sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lanes that hold one query's scores in an MFMA
// accumulator) by gfx950's VALU lane swaps: permlane32_swap(v, v) leaves (v[l], v[l ^ 32]) in its two results,
// permlane16_swap(v, v) (v[l], v[l ^ 16]). The sum adds the l ^ 16 partner first, then the l ^ 32 one.
__device__ __forceinline__ float xmax4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xsum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Min / max over the 16 lanes of each row by DPP (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror:
// each step combines disjoint lane sets), and over the whole wave by the two row-swapping permlanes after it.
template <bool MAX>
__device__ __forceinline__ int minmax(int a, int b) { return MAX ? max(a, b) : min(a, b); }
template <bool MAX>
__device__ __forceinline__ int row_reduce(int v) {
  v = minmax<MAX>(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));
  v = minmax<MAX>(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));
  v = minmax<MAX>(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));
  return minmax<MAX>(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));
}
template <bool MAX>
__device__ __forceinline__ int wave_reduce(int v) {
  v = row_reduce<MAX>(v);
  const auto a = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  v = minmax<MAX>((int)a[0], (int)a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return minmax<MAX>((int)b[0], (int)b[1]);
}

// The sum of squares of one row for QK_NORM_ROPE, from the lanes holding its 8-lane layout's lanes g and g + 4
// (lo = that layout's v_g, hi = v_{g+4}; the partners holding v_{3-g}, v_{7-g} at lane ^ X3 and the next pair
// at lane ^ X1), added in that layout's order ((v0 + v7) + (v2 + v5)) + ((v1 + v6) + (v3 + v4)), so the row's
// 1 / rms has the bits the standalone kernel computes.
template <int X3, int X1>
__device__ __forceinline__ float qkn_row_sum(float lo, float hi, int g) {
  const float plo = __shfl_xor(lo, X3, 64), phi = __shfl_xor(hi, X3, 64);  // v_{3-g}, v_{7-g}
  const float a = lo + phi, b = hi + plo;                                    // u_g, u_{3-g} (u_i = v_i + v_{7-i})
  const float pa = __shfl_xor(a, X1, 64), pb = __shfl_xor(b, X1, 64);        // u_{g^1}, u_{3-(g^1)}
  const float w02 = (g & 1) ? pa + b : a + pb, w13 = (g & 1) ? a + pb : pa + b;
  return w02 + w13;
}

// Normalizes and rotates the two rotation-pair sets one lane holds of a 128-dim row: x0 / y0 = dims 8g..+7 and
// 64 + 8g..+7, x1 / y1 = dims 32 + 8g..+7 and 96 + 8g..+7 (QKN's layout; lanes X3 / X1 apart as above).
template <int X3, int X1>
__device__ __forceinline__ void qkn_row(h8 &x0, h8 &y0, h8 &x1, h8 &y1, int g, const uint16_t *nw, const float2 *cs,
                                        float eps) {
  const bool w = nw != nullptr;
  h8 w0 = {}, w1 = {}, w2 = {}, w3 = {};
  if (w) {
    w0 = *(const h8 *)(nw + 8 * g);
    w1 = *(const h8 *)(nw + 32 + 8 * g);
    w2 = *(const h8 *)(nw + 64 + 8 * g);
    w3 = *(const h8 *)(nw + 96 + 8 * g);
  }
  const float inv = norm_inv(qkn_row_sum<X3, X1>(pair_sumsq(x0, y0), pair_sumsq(x1, y1), g), w, 128, eps);
  const h8x2 lo = norm_rope_pairs(x0, y0, w0, w2, w, true, inv, [&](int i) { return cs[8 * g + i]; });
  const h8x2 hi = norm_rope_pairs(x1, y1, w1, w3, w, true, inv, [&](int i) { return cs[32 + 8 * g + i]; });
  x0 = lo.x;
  y0 = lo.y;
  x1 = hi.x;
  y1 = hi.y;
}

template <int D, int RING, int KG, int HG, bool QKN = false>
__global__ __launch_bounds__(256 * KG * HG) void k_attn(int T, int heads, int kv, const uint16_t *__restrict__ Q, int q_stride,
                                              dj_kv_src A, dj_kv_src B, const int4 *__restrict__ rng, float scale,
                                              uint16_t *__restrict__ O, dj_attn_gate gate, int splits,
                                              float *__restrict__ part, dj_attn_qkn qkn) {
  static_assert(!QKN || (D == 128 && KG == 1 && HG == 1), "q/k norm folded in: 128-dim heads, one head of 4 waves");
  using S = AttnShape<D, RING, KG, HG>;
  constexpr int KW = 64 / KG;          // keys of each tile this wave scores (KG key groups split a tile)
  constexpr int NB = KW / 16;          // 16-key blocks of S^T per wave and tile
  constexpr int NT = KW / 32;          // 32-key MFMA steps of P V per wave and tile
  constexpr int NS_ = D / 32;  // MFMA k-steps over the head dim
  constexpr int NDB = D / 16;  // 16-row blocks of O^T
  constexpr bool PRE_V = D <= 128;  // V^T fragments read ahead of the scores (register budget)
  constexpr int CH = S::CH, KSW = S::KSW, TILE = S::TILE, STAGE = S::STAGE, NS = S::NS;
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int kg = KG > 1 ? wave >> 2 : 0, wq = wave & 3;  // key group; which 16 queries of the block
  // head group: HG query heads that share one KV head, 4 waves each, staging every K/V tile once
  // Workgroups dispatch in linear order (x fastest); take (query block, head group) from that order with the
  // query block descending outermost, so later blocks — the longer key ranges of a causal sequence — start
  // first, and the workgroups past one per CU are the short first blocks of a sequence (longest first).
  const int lin = blockIdx.x + blockIdx.y * gridDim.x;
  const int qb = gridDim.x - 1 - lin / gridDim.y, hgi = lin % gridDim.y;
  const int h = hgi * HG + (HG > 1 ? wave >> 2 : 0), q0 = qb * 64;
  const int kvh = h / (heads / kv);

  // Q fragments first: nothing below depends on them until the first MFMA
  const int qi = q0 + wq * 16 + c16;
  const int qc = min(qi, T - 1);
  h8 qf[NS_];
#pragma unroll
  for (int s = 0; s < NS_; ++s) qf[s] = *(const h8 *)(Q + (size_t)qc * q_stride + (size_t)h * D + s * 32 + g * 8);
  // raw query rows (QKN): lane (c16, g) holds chunks g, 4 + g, 8 + g, 12 + g of its query, i.e. the rotation
  // pairs of QK_NORM_ROPE's 8-lane layout's lanes g and g + 4; the query's four lanes are 16 apart
  if constexpr (QKN) qkn_row<48, 16>(qf[0], qf[2], qf[1], qf[3], g, qkn.qn, qkn.tab + (size_t)qc * 64, qkn.eps);

  // The block's key span per source: lane l reads query q0 + l's ranges, the wave reduces them (every wave
  // does the same, so no LDS and no barrier before the first K/V loads).
  const bool lv = q0 + lane < T;
  const int4 rl = rng[min(q0 + lane, T - 1)];
  int blo[2] = {lv && rl.x < rl.y ? rl.x : INT_MAX, lv && rl.z < rl.w ? rl.z : INT_MAX};
  int bhi[2] = {lv && rl.x < rl.y ? rl.y : INT_MIN, lv && rl.z < rl.w ? rl.w : INT_MIN};
  // this lane's query ranges, and the wave's own span (a tile outside it is skipped by the wave)
  const int src_lane = wq * 16 + c16;
  const int4 rq = {__shfl(rl.x, src_lane, 64), __shfl(rl.y, src_lane, 64), __shfl(rl.z, src_lane, 64),
                   __shfl(rl.w, src_lane, 64)};
  int wlo[2] = {qi < T && rq.x < rq.y ? rq.x : INT_MAX, qi < T && rq.z < rq.w ? rq.z : INT_MAX};
  int whi[2] = {qi < T && rq.x < rq.y ? rq.y : INT_MIN, qi < T && rq.z < rq.w ? rq.w : INT_MIN};
  // keys every live query of the wave sees: [max low, min high) (a query past T does not constrain it)
  int wl2[2] = {qi < T ? rq.x : INT_MIN, qi < T ? rq.z : INT_MIN};
  int wh2[2] = {qi < T ? rq.y : INT_MAX, qi < T ? rq.w : INT_MAX};
  // (every row of 16 lanes holds the same 16 queries of the wave, so a row reduction is the wave's value)
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    blo[s] = wave_reduce<false>(blo[s]);
    bhi[s] = wave_reduce<true>(bhi[s]);
    wlo[s] = row_reduce<false>(wlo[s]);
    whi[s] = row_reduce<true>(whi[s]);
    wl2[s] = row_reduce<true>(wl2[s]);
    wh2[s] = row_reduce<false>(wh2[s]);
  }
  const int loA = max(__builtin_amdgcn_readfirstlane(blo[0]), 0), hiA = min(__builtin_amdgcn_readfirstlane(bhi[0]), A.rows);
  const int loB = max(__builtin_amdgcn_readfirstlane(blo[1]), 0), hiB = min(__builtin_amdgcn_readfirstlane(bhi[1]), B.rows);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    wlo[s] = __builtin_amdgcn_readfirstlane(wlo[s]);
    whi[s] = __builtin_amdgcn_readfirstlane(whi[s]);
    wl2[s] = __builtin_amdgcn_readfirstlane(wl2[s]);
    wh2[s] = __builtin_amdgcn_readfirstlane(wh2[s]);
  }
  const int ntA = hiA > loA ? (hiA - loA + 63) / 64 : 0, ntB = hiB > loB ? (hiB - loB + 63) / 64 : 0;
  const int ntiles = ntA + ntB;
  // split-KV (grid z = splits, small grids): this workgroup takes tiles [j0, j1) of the block's sequence
  const int split = blockIdx.z;
  const int j0 = (int)((long)ntiles * split / splits), j1 = (int)((long)ntiles * (split + 1) / splits);
  const int nloc = j1 - j0;

  // Per-lane DMA source offsets inside a tile: 1 KB DMA q of this wave covers LDS bytes [q KB, q KB + 1 KB) of
  // the K (or V) tile; lane L fills 16 bytes at key row r, physical chunk p, i.e. logical chunk p ^ swizzle(r).
  int krow[S::IK], kch[S::IK], vch[S::IK];
#pragma unroll
  for (int i = 0; i < S::IK; ++i) {
    const int off = (wave * S::IK + i) * 1024 + lane * 16;
    krow[i] = off / (2 * D);
    const int p = (off % (2 * D)) / 16;
    kch[i] = p ^ (krow[i] & KSW);
    vch[i] = p ^ S::vswz(krow[i]);
  }
  // The Q fragments must have landed before the first DMA is issued: the compiler's own wait for them, placed
  // at their first use inside the loop, would count only its own loads and drain the DMA ring every tile. An
  // empty asm that reads them pins that wait here (volatile asm keeps its order with the DMA asm below).
#pragma unroll
  for (int s = 0; s < NS_; ++s) asm volatile("" : "+v"(qf[s]));
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int j, int slot) {
    const bool sb = j >= ntA;
    const uint16_t *base = sb ? B.base : A.base;
    const int stride = sb ? B.stride : A.stride, hi = sb ? hiB : hiA;
    const int k0 = sb ? loB + (j - ntA) * 64 : loA + j * 64;
    const uint16_t *kb = base + (sb ? B.k_col : A.k_col) + (size_t)kvh * D;
    const uint16_t *vb = base + (sb ? B.v_col : A.v_col) + (size_t)kvh * D;
    const uint32_t st = lds0 + slot * STAGE;
#pragma unroll
    for (int i = 0; i < S::IK; ++i) {
      const size_t row = (size_t)min(k0 + krow[i], hi - 1) * stride;  // rows past the range: its last row
      dma16(kb + row + kch[i] * 8, st + (wv * S::IK + i) * 1024);
      dma16(vb + row + vch[i] * 8, st + TILE + (wv * S::IK + i) * 1024);
    }
  };
  if (nloc > 0) {
#pragma unroll
    for (int p = 0; p < NS - 1; ++p) issue(j0 + min(p, nloc - 1), p);  // a short range re-loads its last tile
  }

  // V^T fragment of 32-key step t, dims 16 db..+15 (A operand of O^T += V^T P^T), by two transposing reads:
  // within 16 lanes, lane i points at key 32t + 4g + i/4, dims 16db + 4(i%4)..+3, and receives dim 16db + i of
  // keys 32t + 4g + 0..3 (then the same 16 keys on), the key order of the S^T accumulator that became P^T
  auto read_vt = [&](const uint8_t *vt, int t, int db) -> h8 {
    const int key = 32 * t + 4 * g + (c16 >> 2);
    const int c = 2 * db + ((c16 & 3) >> 1), half8 = (c16 & 1) * 8;
    const uint8_t *p0 = vt + key * (2 * D) + ((c ^ S::vswz(key)) * 16) + half8;
    const uint8_t *p1 = vt + (key + 16) * (2 * D) + ((c ^ S::vswz(key + 16)) * 16) + half8;
    const h4 lo = __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)p0));
    const h4 hi4 = __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)p1));
    return (h8){lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
  };

  f4 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (f4){0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, lsum = 0.f;  // running max in log2 units of the scaled scores
  const float sl = scale * LOG2E;

  for (int jj = 0; jj < nloc; ++jj) {
    // tile jj landed for this wave once at most the NS-2 later tiles' DMAs remain; after the barrier for every
    // wave, and every wave is done with tile jj-1's stage, which is refilled next
    wait_vm_barrier<(NS - 2) * S::I>();
    if constexpr (!QKN) issue(j0 + min(jj + NS - 1, nloc - 1), (jj + NS - 1) % NS);
    const int j = j0 + jj;
    const uint8_t *st = smem + (jj % NS) * STAGE;
    const u32x4 *Ks = (const u32x4 *)st;
    const bool sb = j >= ntA;
    const int k0 = sb ? loB + (j - ntA) * 64 : loA + j * 64, hi = sb ? hiB : hiA;
    if constexpr (QKN) {
      if (sb) {
        // source B's raw key rows, normalized and rotated in LDS before any wave reads them: 4 lanes a row,
        // lane sub taking chunks sub, 4 + sub, 8 + sub, 12 + sub (the query fragments' layout, lanes 1 apart).
        // Before the next tile's DMA is issued, so the waits for the weights and angles count no DMA.
        const int kr = tid >> 2, sub = tid & 3;
        uint8_t *row = smem + (jj % NS) * STAGE + kr * (2 * D);
        h8 *c0 = (h8 *)(row + ((sub ^ (kr & KSW)) * 16)), *c1 = (h8 *)(row + (((4 + sub) ^ (kr & KSW)) * 16));
        h8 *c2 = (h8 *)(row + (((8 + sub) ^ (kr & KSW)) * 16)), *c3 = (h8 *)(row + (((12 + sub) ^ (kr & KSW)) * 16));
        h8 x0 = *c0, x1 = *c1, y0 = *c2, y1 = *c3;
        qkn_row<3, 1>(x0, y0, x1, y1, sub, qkn.kn, qkn.tab + (size_t)min(k0 + kr, hi - 1) * 64, qkn.eps);
        *c0 = x0;
        *c1 = x1;
        *c2 = y0;
        *c3 = y1;
        __syncthreads();
      }
      issue(j0 + min(jj + NS - 1, nloc - 1), (jj + NS - 1) % NS);
    }
    const int qlo = sb ? rq.z : rq.x, qhi = sb ? rq.w : rq.y;
    const int kb0 = k0 + KW * kg;  // this wave's keys of the tile: [kb0, kb0 + KW)
    if (kb0 < whi[sb] && kb0 + KW > wlo[sb]) {
      // Every K fragment of the tile (and at D <= 128 every V^T fragment) is read from LDS before the first
      // MFMA, so a tile waits for one LDS latency instead of one per MFMA pair; V needs no score, so its reads
      // run under the QK^T MFMAs and the softmax. The scheduling barrier keeps the compiler from sinking the
      // reads back to their uses.
      h8 kf[NB][NS_];
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) {
        const int r = 16 * (NB * kg + bb) + c16;
#pragma unroll
        for (int s = 0; s < NS_; ++s) kf[bb][s] = __builtin_bit_cast(h8, Ks[r * CH + ((4 * s + g) ^ (r & KSW))]);
      }
      const uint8_t *vt = st + TILE;
      h8 vf[PRE_V ? NT : 1][NDB];
      if constexpr (PRE_V) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int db = 0; db < NDB; ++db) vf[tt][db] = read_vt(vt, NT * kg + tt, db);
      }
      __builtin_amdgcn_sched_barrier(0);
      // S^T[key, q] = K . Q^T: A = 16 keys x 32 dims of K, B = the query fragment
      f4 sc[NB];
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) sc[bb] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS_; ++s)
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) sc[bb] = MFMA16(kf[bb][s], qf[s], sc[bb]);
      // Tiles that every query of the wave sees whole (all but the diagonal ones of a causal block) skip the
      // per-key mask.
      const bool whole = kb0 >= wl2[sb] && kb0 + KW <= wh2[sb] && kb0 + KW <= hi;
      // The max is taken on the raw scores (the scale is positive, so it commutes) and scaled once; the exp2
      // argument below is one fma per score.
      float tmax = -INFINITY;
      if (whole) {
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
          for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[bb][r]);
      } else {
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int kk = kb0 + 16 * bb + 4 * g + r;
            const bool ok = kk >= qlo && kk < qhi && kk < hi;
            sc[bb][r] = ok ? sc[bb][r] : -INFINITY;
            tmax = fmaxf(tmax, sc[bb][r]);
          }
      }
      tmax = xmax4(tmax) * sl;
      // Lazy rescaling: the reference point m moves (and O, l are rescaled) only when some query's maximum
      // has grown by more than 8 (log2 units); otherwise p = exp2(s - m) <= 2^8 stays exact enough in f16
      // and O / l is unchanged. The first live tile always moves m off -1e30.
      if (__builtin_amdgcn_ballot_w64(tmax > m + 8.0f) != 0) {
        const float mn = fmaxf(m, tmax);
        const float corr = __builtin_amdgcn_exp2f(m - mn);
        lsum *= corr;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[db] *= corr;
        m = mn;
      }
      float ps = 0.f;
      h8 pf[NT];
#pragma unroll
      for (int bb = 0; bb < NB; ++bb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[bb][r], sl, -m));  // exp2(-inf) = 0: masked
          ps += p;
          pf[bb >> 1][(bb & 1) * 4 + r] = (_Float16)p;
        }
      lsum += ps;
      // O^T[d, q] += V^T . P^T: A = V^T (16 dims x keys {32t + 4g + 0..3, 32t + 16 + 4g + 0..3}, read_vt), B = P^T
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          o[db] = MFMA16(PRE_V ? vf[PRE_V ? tt : 0][db] : read_vt(vt, NT * kg + tt, db), pf[tt], o[db]);
    }
  }
  wait_vm<0>();  // the clamped tail DMAs land before the wave ends

  if constexpr (KG > 1) {
    // key group 1 hands its (m, l, O) to group 0 through LDS (the ring is free: every DMA has landed and every
    // wave is past its last read), which merges them: M = max, both rescaled to it
    f4 *xo = (f4 *)smem;
    float *xml = (float *)(smem + 4 * NDB * 64 * sizeof(f4));
    __syncthreads();
    if (kg == 1) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) xo[(wq * NDB + db) * 64 + lane] = o[db];
      xml[(wq * 64 + lane) * 2] = m;
      xml[(wq * 64 + lane) * 2 + 1] = lsum;
    }
    __syncthreads();
    if (kg == 1) return;
    const float m1 = xml[(wq * 64 + lane) * 2], l1 = xml[(wq * 64 + lane) * 2 + 1];
    const float mm = fmaxf(m, m1);
    const float c0 = __builtin_amdgcn_exp2f(m - mm), c1 = __builtin_amdgcn_exp2f(m1 - mm);
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = o[db] * c0 + xo[(wq * NDB + db) * 64 + lane] * c1;
    lsum = lsum * c0 + l1 * c1;
    m = mm;
  }

  lsum = xsum4(lsum);
  if (splits > 1) {
    // partial of this split: unnormalized f32 O^T and (m, l) per query and head, merged by k_attn_combine
    if (qi < T) {
      const size_t row = ((size_t)split * T + qi) * heads + h;
      float *po = part + row * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db) *(f4 *)(po + 16 * db + 4 * g) = o[db];
      if (g == 0) {
        float *pml = part + (size_t)splits * T * heads * D + row * 2;
        pml[0] = m;
        pml[1] = lsum;
      }
    }
    return;
  }
  if (qi < T) {
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    uint16_t *orow = O + (size_t)qi * heads * D + (size_t)h * D;
    const uint16_t *grow = gate.g ? gate.g + (size_t)qi * gate.stride + (size_t)h * D : nullptr;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      h4 v;
      if (grow) {  // the output gate of d3's attention (d3-kernels.ts:232-236): acc / l / (1 + exp(-gate))
        const h4 gv = *(const h4 *)(grow + 16 * db + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (_Float16)(o[db][r] * inv / (1.0f + expf(-(float)gv[r])));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (_Float16)(o[db][r] * inv);
      }
      *(h4 *)(orow + 16 * db + 4 * g) = v;
    }
  }
}

// Merge of the split-KV partials of one (query, head): M = max m_s, L = sum l_s 2^(m_s - M),
// O = sum O_s 2^(m_s - M) / L, in split order (deterministic). A split that saw no key has l = 0.
// One wave per (query, head): lane s loads split s's (m, l), lane l owns D / 64 consecutive dims, and every
// partial of up to 16 splits is loaded before the first add, so the loads overlap; the sums then run in split
// order on values broadcast from lane s.
template <int DPL>
__global__ __launch_bounds__(256) void k_attn_combine(int T, int heads, int splits, const float *__restrict__ part,
                                                      uint16_t *__restrict__ O, dj_attn_gate gate) {
  constexpr int D = 64 * DPL, PRE = 16;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (pair >= T * heads) return;
  const int q = pair / heads, h = pair % heads;
  const size_t rs = (size_t)T * heads;  // rows per split
  const size_t row0 = (size_t)q * heads + h;
  const float *ml = part + (size_t)splits * rs * D;
  float ms = -1e30f, ls = 0.f;
  if (lane < splits) {
    ms = ml[(lane * rs + row0) * 2];
    ls = ml[(lane * rs + row0) * 2 + 1];
  }
  float M = ls > 0.f ? ms : -1e30f;
#pragma unroll
  for (int x = 1; x < 64; x <<= 1) M = fmaxf(M, __shfl_xor(M, x, 64));
  const float wl = ls > 0.f ? __builtin_amdgcn_exp2f(ms - M) : 0.f;
  float pv[PRE][DPL];
#pragma unroll
  for (int k = 0; k < PRE; ++k)
#pragma unroll
    for (int i = 0; i < DPL; ++i) pv[k][i] = k < splits ? part[(k * rs + row0) * D + lane * DPL + i] : 0.f;
  float L = 0.f, acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
#pragma unroll
  for (int k = 0; k < PRE; ++k) {
    const float l = __shfl(ls, k, 64), w = __shfl(wl, k, 64);
    if (k < splits && l > 0.f) {
      L += l * w;
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[i] += pv[k][i] * w;
    }
  }
  for (int k = PRE; k < splits; ++k) {
    const float l = __shfl(ls, k, 64), w = __shfl(wl, k, 64);
    if (l > 0.f) {
      L += l * w;
#pragma unroll
      for (int i = 0; i < DPL; ++i) acc[i] += part[(k * rs + row0) * D + lane * DPL + i] * w;
    }
  }
  uint16_t *o = O + row0 * D + lane * DPL;
  const uint16_t *gr = gate.g ? gate.g + (size_t)q * gate.stride + (size_t)h * D + lane * DPL : nullptr;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    float v = L > 0.f ? acc[i] / L : 0.f;
    if (gr) v = v / (1.0f + expf(-(float)__builtin_bit_cast(_Float16, gr[i])));
    o[i] = __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

// 512-dim heads (EmbeddingGemma 2's global layers, eg2-kernels.ts:98-163): a VALU form. A workgroup holds 16
// queries of one head, 16 lanes per query and 32 dims per lane (dims 8 part + 128 j .. +7, so the 16 lanes of a
// query read 256 consecutive bytes of a key row); key/value tiles of 16 rows x 512 dims in LDS; per tile the 16
// scores first (lane partials added over the 16 lanes), one online-softmax update, then P V. Both key ranges of
// each query (over sources A and B) are walked; a query's keys outside its ranges weigh zero.
constexpr int WD = 512, WQ = 16, WK = 16;
__global__ __launch_bounds__(256) void k_attn_wide(int T, int heads, int kv, const uint16_t *__restrict__ Q, int q_stride,
                                                   dj_kv_src A, dj_kv_src B, const int4 *__restrict__ rng, float scale,
                                                   uint16_t *__restrict__ O, dj_attn_gate gate) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[WK * WD];
  __shared__ __attribute__((aligned(16))) uint16_t vs[WK * WD];
  __shared__ int4 bounds;
  const int tid = threadIdx.x, qi = tid / 16, part = tid % 16;
  const int h = blockIdx.y, kvh = h / (heads / kv);
  const int q0 = blockIdx.x * WQ, t = min(q0 + qi, T - 1);
  const bool live = q0 + qi < T;
  float q[32];
  {
    const uint16_t *qr = Q + (size_t)t * q_stride + (size_t)h * WD + 8 * part;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const h8 v = *(const h8 *)(qr + 128 * j);
#pragma unroll
      for (int e = 0; e < 8; ++e) q[8 * j + e] = (float)v[e] * scale;
    }
  }
  const int4 r = rng[t];
  // the block's key span per source: min of starts, max of ends over its live queries
  if (tid == 0) bounds = make_int4(INT32_MAX, 0, INT32_MAX, 0);
  __syncthreads();
  if (part == 0 && live) {
    if (r.y > r.x) {
      atomicMin(&bounds.x, r.x);
      atomicMax(&bounds.y, r.y);
    }
    if (r.w > r.z) {
      atomicMin(&bounds.z, r.z);
      atomicMax(&bounds.w, r.w);
    }
  }
  __syncthreads();
  const int4 bd = bounds;
  float m = -1e30f, l = 0.f, acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
  for (int src = 0; src < 2; ++src) {
    const dj_kv_src X = src ? B : A;
    const int lo = src ? bd.z : bd.x, hi = src ? bd.w : bd.y;
    const int mylo = src ? r.z : r.x, myhi = src ? r.w : r.y;
    for (int k0 = lo; k0 < hi; k0 += WK) {
      // stage K and V rows k0 .. k0 + 15 (clamped to the source), 16 bytes per thread per pass
      for (int i = tid; i < WK * WD / 8; i += 256) {
        const int row = i / (WD / 8), c8 = (i % (WD / 8)) * 8;
        const int kr = min(max(k0 + row, 0), X.rows - 1);
        const uint16_t *base = X.base + (size_t)kr * X.stride;
        *(uint4 *)(ks + row * WD + c8) = *(const uint4 *)(base + X.k_col + kvh * WD + c8);
        *(uint4 *)(vs + row * WD + c8) = *(const uint4 *)(base + X.v_col + kvh * WD + c8);
      }
      __syncthreads();
      float sc[WK];
      float mb = m;
#pragma unroll
      for (int j = 0; j < WK; ++j) {
        float d = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const h8 kv8 = *(const h8 *)(ks + j * WD + 128 * c + 8 * part);
#pragma unroll
          for (int e = 0; e < 8; ++e) d += q[8 * c + e] * (float)kv8[e];
        }
        d = group_sum<16>(d);
        const int key = k0 + j;
        sc[j] = key >= mylo && key < myhi && key < hi ? d : -1e30f;
        mb = fmaxf(mb, sc[j]);
      }
      const float corr = expf(m - mb);
      l *= corr;
#pragma unroll
      for (int i = 0; i < 32; ++i) acc[i] *= corr;
#pragma unroll
      for (int j = 0; j < WK; ++j) {
        const float p = sc[j] > -1e29f ? expf(sc[j] - mb) : 0.f;
        l += p;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const h8 v8 = *(const h8 *)(vs + j * WD + 128 * c + 8 * part);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[8 * c + e] += p * (float)v8[e];
        }
      }
      m = mb;
      __syncthreads();
    }
  }
  if (!live) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  uint16_t *orow = O + (size_t)t * heads * WD + (size_t)h * WD + 8 * part;
  const uint16_t *grow = gate.g ? gate.g + (size_t)t * gate.stride + (size_t)h * WD + 8 * part : nullptr;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[8 * c + e] * inv;
      if (grow) v = v / (1.0f + expf(-(float)__builtin_bit_cast(_Float16, grow[128 * c + e])));
      o[e] = (_Float16)v;
    }
    *(h8 *)(orow + 128 * c) = o;
  }
}

// Launch with one workgroup shape; a shape whose K/V tile does not split into whole 1 KB DMAs per wave is never
// picked, nor one that would spill registers (the launcher falls back to HG 1 for them).
template <int D, int RING, int KG, int HG, bool QKN = false>
static void attn_launch(dim3 g3, hipStream_t s, int T, int heads, int kv, const uint16_t *Q, int q_stride,
                        dj_kv_src A, dj_kv_src B, const int4 *r4, float scale, uint16_t *O, dj_attn_gate gate, int splits,
                        float *part, dj_attn_qkn qkn = dj_attn_qkn{}) {
  if constexpr ((64 * 2 * D) % (1024 * 4 * KG * HG) == 0 && D * HG <= 256 &&  // (D 128 x HG 4 would spill)
                RING * 2 * (64 * 2 * D) <= 160 * 1024)
    k_attn<D, RING, KG, HG, QKN><<<g3, 256 * KG * HG, 0, s>>>(T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate,
                                                              splits, part, qkn);
}

// The split-KV plan of a launch: small grids (a short question against a long state: one query block per head)
// split each block's key tiles over up to 16 workgroups, their f32 partials (splits * T * heads * (D + 2) floats)
// in a workspace of ws_floats floats, merged by k_attn_combine; large grids run whole (1). Splits that do not fit
// the workspace are reduced until they do. DJ_ATTN_SPLITS=<n> forces the split count (tuning sweeps).
// Only long key sources are split: a 32-token question on a 1056-row kept state runs 14.1 us split against 25.0
// whole, while the encoder's 384-token layer (at most 4 tiles per block) runs 21.4 split against 15.9 whole, the
// merge costing as much as it saves (measured on MI355X).
static int attn_splits(int cus, int T, int heads, int D, const dj_kv_src &A, const dj_kv_src &B, size_t ws_floats) {
  const long grid = (long)dj_cdiv(T, 64) * heads;
  const char *force = getenv("DJ_ATTN_SPLITS");
  const int max_tiles = dj_cdiv(A.rows, 64) + dj_cdiv(B.rows, 64);
  if (!force && !(grid < cus && max_tiles >= 16)) return 1;
  int splits = force ? atoi(force) : (int)std::min<long>(std::min(16, max_tiles), dj_cdiv(2L * cus, grid));
  splits = std::max(1, std::min(splits, 64));
  while (splits > 1 && (size_t)splits * T * heads * (D + 2) > ws_floats) --splits;
  return splits;
}

int dj_launch_attention(dj_ctx *c, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride, dj_kv_src A,
                        dj_kv_src B, const int32_t *rng, float scale, uint16_t *O, float *ws, size_t ws_floats,
                        dj_attn_gate gate, const dj_attn_qkn *qkn) {
  hipStream_t s = c->stream;
  if (qkn && D != 128) return dj_fail(DJ_EINVAL, "decision.js: attention with q/k norm folded in: head dim %d (128)", D);
  if (D == WD) {  // 512-dim heads: the VALU form, whole
    k_attn_wide<<<dim3(dj_cdiv(T, WQ), heads), 256, 0, s>>>(T, heads, kv, Q, q_stride, A, B, (const int4 *)rng, scale, O,
                                                            gate);
    return DJ_OK;
  }
  const int qblocks = dj_cdiv(T, 64);
  const long grid = (long)qblocks * heads;
  const int4 *r4 = (const int4 *)rng;
  int splits = ws ? attn_splits(c->cus, T, heads, D, A, B, ws_floats) : 1;
  float *part = splits > 1 ? ws : nullptr;
  // Ring depth: two stages for 4-wave workgroups (two workgroups fit per CU and hide each other's latency:
  // 13.6 vs 18.0 us with a 4-stage ring, one workgroup per CU, at T = 1152, D 128 causal; 504 vs 719 us at
  // 86016), and the deepest that fits 128 KB for head groups.
  // key groups per workgroup: one. Two (8 waves, each scoring half of every key tile, merged in LDS) measured
  // slower at D 128 (32.7 vs 30.3 us at 1 x 1152, 46.8 vs 42.5 at 16 x 384) and mixed at D 256 (35.1 vs 37.6
  // us at 2 x 1024 causal, 8 heads, but 23.5 vs 20.5 us in the encoder's 384-token layer). DJ_ATTN_KG=2
  // selects them (tuning sweeps; covered by the attention tests).
  const char *kgs = getenv("DJ_ATTN_KG");
  const int kg = kgs ? atoi(kgs) : 1;
  // head groups: HG query heads sharing a KV head in one workgroup (4 HG waves) stage each K/V tile once, which
  // halves (HG 2) the workgroups and the K/V reads and leaves LDS for a 4-stage ring (one workgroup per CU).
  // DJ_ATTN_HG=<1|2|4> forces it (tuning sweeps).
  const char *hgs = getenv("DJ_ATTN_HG");
  // By default only large grids take them (the 192-sequence batch: 592 vs 616 us); at a ticket's few hundred
  // workgroups the 4-wave form is faster (14.3 vs 15.1 us at 3 x 384, 11.0 vs 14.7 at 1 x 384; MI355X).
  int hg = hgs ? atoi(hgs) : (splits == 1 && (heads / kv) % 2 == 0 && grid >= 16L * c->cus ? 2 : 1);
  if (kg > 1 || (hg != 1 && hg != 2 && hg != 4) || (heads / kv) % hg || (128 * D) % (4096 * hg) || D * hg > 256) hg = 1;
  // DJ_ATTN_RING=<3|4> deepens the 4-wave form's ring (tuning sweeps; at D 256 a stage is 64 KB, so 2)
  const char *rs = getenv("DJ_ATTN_RING");
  const int ring = rs && D <= 128 ? atoi(rs) : 2;
  const dim3 g3(qblocks, heads / hg, splits);
#define DJ_ATTN_CASE(DD)                                                                                              \
  case DD:                                                                                                            \
    if (kg > 1) attn_launch<DD, 2, 2, 1>(g3, s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate, splits, part);         \
    else if (hg == 2) attn_launch<DD, 0, 1, 2>(g3, s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate, splits, part);   \
    else if (hg == 4) attn_launch<DD, 0, 1, 4>(g3, s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate, splits, part);   \
    else if (ring == 3) attn_launch<DD, 3, 1, 1>(g3, s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate, splits, part); \
    else if (ring == 4) attn_launch<DD, 4, 1, 1>(g3, s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate, splits, part); \
    else attn_launch<DD, 2, 1, 1>(g3, s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate, splits, part);                \
    break;
  if (qkn)  // q/k norm folded in: the 4-wave, 2-stage form (the form a short question's split launch takes)
    attn_launch<128, 2, 1, 1, true>(dim3(qblocks, heads, splits), s, T, heads, kv, Q, q_stride, A, B, r4, scale, O, gate,
                                    splits, part, *qkn);
  else
    switch (D) {
      DJ_ATTN_CASE(64)
      DJ_ATTN_CASE(128)
      DJ_ATTN_CASE(256)
      default: return dj_fail(DJ_EINVAL, "decision.js: attention head dim %d (64, 128 or 256)", D);
    }
#undef DJ_ATTN_CASE
  if (splits > 1) {
    const unsigned blocks = (unsigned)dj_cdiv((long)T * heads, 4);
    if (D == 64) k_attn_combine<1><<<blocks, 256, 0, s>>>(T, heads, splits, part, O, gate);
    else if (D == 128) k_attn_combine<2><<<blocks, 256, 0, s>>>(T, heads, splits, part, O, gate);
    else k_attn_combine<4><<<blocks, 256, 0, s>>>(T, heads, splits, part, O, gate);
  }
  return DJ_OK;
}

static bool src_ok(const dj_kv_src &s, int kv, int D) {
  return s.base && s.rows > 0 && s.stride % 8 == 0 && s.k_col % 8 == 0 && s.v_col % 8 == 0 && s.k_col >= 0 &&
         s.v_col >= 0 && s.k_col + kv * D <= s.stride && s.v_col + kv * D <= s.stride;
}

extern "C" int dj_attention(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride, dj_kv_src A,
                            dj_kv_src B, const int32_t *rng, float scale, uint16_t *O) {
  DJ_REQUIRE(Q && rng && O && T >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && q_stride % 8 == 0 &&
                 q_stride >= heads * D,
             "decision.js: attention: bad arguments (heads %d, kv %d, q_stride %d)", heads, kv, q_stride);
  DJ_REQUIRE(D == 64 || D == 128 || D == 256 || D == 512, "decision.js: attention head dim %d (64, 128, 256 or 512)", D);
  DJ_REQUIRE(scale > 0.f, "decision.js: attention: the score scale must be positive (got %g)", (double)scale);
  DJ_REQUIRE(src_ok(A, kv, D) && src_ok(B, kv, D), "decision.js: attention: bad key/value source");
  DJ_OP_BEGIN(rec, "attention");
  if (T > 0) {
    int st = dj_launch_attention(rec->ctx, T, heads, kv, D, Q, q_stride, A, B, rng, scale, O, rec->ctx->gemm_ws,
                                 rec->ctx->gemm_ws_floats);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[T%d h%d kv%d D%d]", T, heads, kv, D);
  return dj_op_end(rec, "attention", shape);
}

extern "C" int dj_attention_gated(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride,
                                  dj_kv_src A, dj_kv_src B, const int32_t *rng, float scale, const uint16_t *G,
                                  int g_stride, uint16_t *O) {
  DJ_REQUIRE(Q && rng && O && G && T >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && q_stride % 8 == 0 &&
                 q_stride >= heads * D && g_stride % 8 == 0 && g_stride >= heads * D && ((uintptr_t)G & 7) == 0,
             "decision.js: attention_gated: bad arguments (heads %d, kv %d, q_stride %d, g_stride %d)", heads, kv,
             q_stride, g_stride);
  DJ_REQUIRE(D == 64 || D == 128 || D == 256 || D == 512, "decision.js: attention head dim %d (64, 128, 256 or 512)", D);
  DJ_REQUIRE(scale > 0.f, "decision.js: attention: the score scale must be positive (got %g)", (double)scale);
  DJ_REQUIRE(src_ok(A, kv, D) && src_ok(B, kv, D), "decision.js: attention: bad key/value source");
  DJ_OP_BEGIN(rec, "attention_gated");
  if (T > 0) {
    int st = dj_launch_attention(rec->ctx, T, heads, kv, D, Q, q_stride, A, B, rng, scale, O, rec->ctx->gemm_ws,
                                 rec->ctx->gemm_ws_floats, dj_attn_gate{G, g_stride});
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[T%d h%d kv%d D%d]", T, heads, kv, D);
  return dj_op_end(rec, "attention_gated", shape);
}

extern "C" int dj_attention_qk_rope(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride,
                                    dj_kv_src A, dj_kv_src B, const int32_t *rng, float scale, const uint16_t *qn,
                                    const uint16_t *kn, float eps, const float *tab, int rot, uint16_t *O) {
  DJ_REQUIRE(Q && rng && O && tab && T >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && q_stride % 8 == 0 &&
                 q_stride >= heads * D,
             "decision.js: attention_qk_rope: bad arguments (heads %d, kv %d, q_stride %d)", heads, kv, q_stride);
  DJ_REQUIRE(D == 128 && rot == 128, "decision.js: attention_qk_rope: head dim %d, rot %d (128 and 128)", D, rot);
  DJ_REQUIRE(scale > 0.f, "decision.js: attention: the score scale must be positive (got %g)", (double)scale);
  DJ_REQUIRE(src_ok(A, kv, D) && src_ok(B, kv, D) && B.rows == T,
             "decision.js: attention_qk_rope: bad key/value source (source B must be the %d query rows)", T);
  DJ_OP_BEGIN(rec, "attention_qk_rope");
  if (T > 0) {
    const dj_attn_qkn q{qn, kn, (const float2 *)tab, eps};
    int st = dj_launch_attention(rec->ctx, T, heads, kv, D, Q, q_stride, A, B, rng, scale, O, rec->ctx->gemm_ws,
                                 rec->ctx->gemm_ws_floats, dj_attn_gate{nullptr, 0}, &q);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[T%d h%d kv%d D%d]", T, heads, kv, D);
  return dj_op_end(rec, "attention_qk_rope", shape);
}

// ---------------------------------------------------------------- the entry point that allocates nothing

// Split-KV partials of dj_attention_noalloc: 8 MiB of f32 per GPU, held until the process ends. Every call on
// a GPU shares that GPU's array (calls that overlap on one GPU race); every partial is written before it is
// read, so nothing needs clearing. Host code never uses this name as an address: dj_attn_scratch_init takes the
// device's own address of the array with hipGetSymbolAddress.
constexpr size_t kScratchFloats = (size_t)2 << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

int dj_attn_scratch_init(dj_ctx *c) {  // with c's device current (dj_init)
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return dj_fail(DJ_EHIP, "decision.js: the attention scratch has no device address (%s)", hipGetErrorString(e));
  c->attn_scratch = (float *)p;
  return DJ_OK;
}

extern "C" int dj_attention_noalloc(dj_rec *rec, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride,
                                    dj_kv_src A, dj_kv_src B, const int32_t *rng, float scale, uint16_t *O) {
  DJ_REQUIRE(Q && rng && O && T >= 0 && heads > 0 && kv > 0 && heads % kv == 0 && q_stride % 8 == 0 &&
                 q_stride >= heads * D,
             "decision.js: attention: bad arguments (heads %d, kv %d, q_stride %d)", heads, kv, q_stride);
  DJ_REQUIRE(D == 64 || D == 128 || D == 256 || D == 512, "decision.js: attention head dim %d (64, 128, 256 or 512)", D);
  DJ_REQUIRE(scale > 0.f, "decision.js: attention: the score scale must be positive (got %g)", (double)scale);
  DJ_REQUIRE(src_ok(A, kv, D) && src_ok(B, kv, D), "decision.js: attention: bad key/value source");
  DJ_REQUIRE(rec && rec->ctx && rec->ctx->attn_scratch, "decision.js: dj_attention_noalloc: no recorder or scratch");
  // the plan dj_attention takes; refused (not shrunk) where its partials exceed the scratch, so both entry
  // points always compute the same thing
  const int splits = D == WD ? 1 : attn_splits(rec->ctx->cus, T, heads, D, A, B, rec->ctx->gemm_ws ? rec->ctx->gemm_ws_floats : 0);
  const size_t need = splits > 1 ? (size_t)splits * T * heads * (D + 2) : 0;
  DJ_REQUIRE(need <= kScratchFloats,
             "decision.js: dj_attention_noalloc: T %d x %d heads of %d dims split %d ways needs %.1f MB of scratch, "
             "more than its %.1f MB (use dj_attention)",
             T, heads, D, splits, need * 4 / 1e6, kScratchFloats * 4 / 1e6);
  DJ_OP_BEGIN(rec, "attention_noalloc");
  if (T > 0) {
    int st = dj_launch_attention(rec->ctx, T, heads, kv, D, Q, q_stride, A, B, rng, scale, O, rec->ctx->attn_scratch,
                                 kScratchFloats);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[T%d h%d kv%d D%d]/k%d", T, heads, kv, D, splits);
  return dj_op_end(rec, "attention_noalloc", shape);
}
