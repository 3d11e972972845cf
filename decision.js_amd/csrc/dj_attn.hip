// Attention over per-query key ranges on gfx950 MFMA (flash-attention style, online softmax).
//
// Each query t reads two key ranges rng[t] = (a0, a1, b0, b1): rows [a0, a1) of source A and [b0, b1) of
// source B. That one form covers every mask of the reference: the causal forest of ATTENTION (a trunk token
// sees earlier trunk tokens, a branch token the whole trunk and its own branch up to itself,
// kernels.ts:133-136), the bidirectional segment or window of the encoders (eg2-kernels.ts:128-145), the
// trunk + branch ranges of attention256 (d3-kernels.ts:207-223), and a kept prefix KV (source A = the
// cache) in the shared-state mode.
//
// A workgroup takes 64 queries of one head (4 waves x 16). K/V tiles of 64 keys of the block's union range
// are staged in LDS: K row-major (XOR-swizzled 16-byte chunks), V transposed. Per wave and tile:
//   S^T[key, q] = K . Q^T       (A = K from LDS, B = Q held in registers; the accumulator puts query
//                                l % 16 in lane l, so the softmax row reduction is 2 shuffles)
//   O^T[d, q]  += V^T . P^T     (P^T is the S^T accumulator itself, rounded to f16; the key order inside
//                                each 32-key MFMA step is permuted to match, and V^T is read to match)
// Scores, the running max (m0 = -1e30) and the row sums are f32; the output is f16(acc / l), as the reference.
#include <math.h>
#include <stdio.h>
#include "dj_internal.h"

#define MFMA16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16((a), (b), (c), 0, 0, 0)

// Global -> register staging of one K/V tile (64 keys) of the flattened tile sequence: tiles of source A first,
// then of source B. Rows past the range end are clamped to its last row (read, then masked).
#define DJ_ATTN_LOAD(j)                                                                                      \
  {                                                                                                          \
    const bool sb_ = (j) >= ntA;                                                                             \
    const uint16_t *kb_ = sb_ ? kbB : kbA, *vb_ = sb_ ? vbB : vbA;                                           \
    const int st_ = sb_ ? B.stride : A.stride, hi_ = sb_ ? hiB : hiA;                                        \
    const int k0_ = sb_ ? loB + ((j) - ntA) * 64 : loA + (j) * 64;                                           \
    _Pragma("unroll") for (int i = 0; i < KC; ++i) {                                                         \
      const int c = tid + 256 * i, r = c / CH, ch = c % CH;                                                  \
      kr[i] = *(const u32x4 *)(kb_ + (size_t)min(k0_ + r, hi_ - 1) * st_ + ch * 8);                          \
    }                                                                                                        \
    _Pragma("unroll") for (int i = 0; i < VI; ++i) {                                                         \
      const int it = tid + 256 * i, r0 = 2 * (it & 31), ch = it >> 5;                                        \
      vr[2 * i] = *(const u32x4 *)(vb_ + (size_t)min(k0_ + r0, hi_ - 1) * st_ + ch * 8);                     \
      vr[2 * i + 1] = *(const u32x4 *)(vb_ + (size_t)min(k0_ + r0 + 1, hi_ - 1) * st_ + ch * 8);             \
    }                                                                                                        \
  }

template <int D>
__global__ __launch_bounds__(256) void k_attn(int T, int heads, int kv, const uint16_t *__restrict__ Q, int q_stride,
                                              dj_kv_src A, dj_kv_src B, const int4 *__restrict__ rng, float scale,
                                              uint16_t *__restrict__ O) {
  constexpr int NS = D / 32;   // MFMA k-steps over the head dim
  constexpr int NDB = D / 16;  // 16-row blocks of O^T
  constexpr int CH = D / 8;    // 16-byte chunks per K row
  constexpr int KC = CH / 4;   // K chunks staged per thread and tile
  constexpr int VI = CH / 8;   // V chunk pairs (two adjacent keys) staged per thread and tile
  constexpr int SW = CH >= 16 ? 15 : 7;
  constexpr int VS = 68;       // V^T row stride in halves: 64 keys + 4 (conflict-free 8-byte reads)
  constexpr float LOG2E = 1.4426950408889634f;
  __shared__ u32x4 Ks[64 * CH];
  __shared__ uint32_t Vt[D * VS / 2];
  __shared__ int bounds[4];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int h = blockIdx.y, q0 = blockIdx.x * 64;
  const int kvh = h / (heads / kv);

  if (tid == 0) {
    bounds[0] = INT_MAX; bounds[1] = INT_MIN; bounds[2] = INT_MAX; bounds[3] = INT_MIN;
  }
  __syncthreads();
  if (tid < 64 && q0 + tid < T) {
    const int4 r = rng[q0 + tid];
    if (r.x < r.y) { atomicMin(&bounds[0], r.x); atomicMax(&bounds[1], r.y); }
    if (r.z < r.w) { atomicMin(&bounds[2], r.z); atomicMax(&bounds[3], r.w); }
  }
  __syncthreads();
  const int loA = max(bounds[0], 0), hiA = min(bounds[1], A.rows);
  const int loB = max(bounds[2], 0), hiB = min(bounds[3], B.rows);
  const int ntA = hiA > loA ? (hiA - loA + 63) / 64 : 0, ntB = hiB > loB ? (hiB - loB + 63) / 64 : 0;
  const uint16_t *kbA = A.base + A.k_col + (size_t)kvh * D, *vbA = A.base + A.v_col + (size_t)kvh * D;
  const uint16_t *kbB = B.base + B.k_col + (size_t)kvh * D, *vbB = B.base + B.v_col + (size_t)kvh * D;

  const int qi = q0 + wave * 16 + c16;
  const int qc = min(qi, T - 1);
  h8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = *(const h8 *)(Q + (size_t)qc * q_stride + (size_t)h * D + s * 32 + g * 8);
  const int4 rq = rng[qc];
  // the wave's own key span per source (a tile outside it is skipped by the wave; queries past T see nothing)
  int wlo[2] = {qi < T && rq.x < rq.y ? rq.x : INT_MAX, qi < T && rq.z < rq.w ? rq.z : INT_MAX};
  int whi[2] = {qi < T && rq.x < rq.y ? rq.y : INT_MIN, qi < T && rq.z < rq.w ? rq.w : INT_MIN};
#pragma unroll
  for (int x = 1; x < 16; x <<= 1)
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      wlo[s] = min(wlo[s], __shfl_xor(wlo[s], x, 64));
      whi[s] = max(whi[s], __shfl_xor(whi[s], x, 64));
    }
  wlo[0] = __builtin_amdgcn_readfirstlane(wlo[0]); whi[0] = __builtin_amdgcn_readfirstlane(whi[0]);
  wlo[1] = __builtin_amdgcn_readfirstlane(wlo[1]); whi[1] = __builtin_amdgcn_readfirstlane(whi[1]);

  f4 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (f4){0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, lsum = 0.f;  // running max in log2 units of the scaled scores
  const float sl = scale * LOG2E;
  const uint16_t *vt16 = (const uint16_t *)Vt;

  u32x4 kr[KC], vr[2 * VI];
  const int ntiles = ntA + ntB;
  if (ntiles > 0) DJ_ATTN_LOAD(0);
  for (int j = 0; j < ntiles; ++j) {
    // registers -> LDS: K row-major (chunk ch of row r at ch ^ (r & SW)), V transposed (Vt[d][key])
#pragma unroll
    for (int i = 0; i < KC; ++i) {
      const int c = tid + 256 * i, r = c / CH, ch = c % CH;
      Ks[r * CH + (ch ^ (r & SW))] = kr[i];
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) {
      const int it = tid + 256 * i, r0 = 2 * (it & 31), ch = it >> 5;
      uint32_t *dst = Vt + (((ch * 8) * VS + r0) >> 1);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t a = vr[2 * i][w], b = vr[2 * i + 1][w];
        dst[(2 * w) * (VS / 2)] = (a & 0xffffu) | (b << 16);          // d = 8ch + 2w: (key r0, key r0+1)
        dst[(2 * w + 1) * (VS / 2)] = (a >> 16) | (b & 0xffff0000u);  // d = 8ch + 2w + 1
      }
    }
    __syncthreads();
    if (j + 1 < ntiles) DJ_ATTN_LOAD(j + 1);  // in flight while this tile is computed

    const bool sb = j >= ntA;
    const int k0 = sb ? loB + (j - ntA) * 64 : loA + j * 64, hi = sb ? hiB : hiA;
    const int qlo = sb ? rq.z : rq.x, qhi = sb ? rq.w : rq.y;
    if (k0 < whi[sb] && k0 + 64 > wlo[sb]) {
      f4 sc[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        sc[b] = (f4){0.f, 0.f, 0.f, 0.f};
        const int r = 16 * b + c16;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const h8 kf = __builtin_bit_cast(h8, Ks[r * CH + ((4 * s + g) ^ (r & SW))]);
          sc[b] = MFMA16(kf, qf[s], sc[b]);
        }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kk = k0 + 16 * b + 4 * g + r;
          const bool ok = kk >= qlo && kk < qhi && kk < hi;
          const float v = ok ? sc[b][r] * sl : -INFINITY;
          sc[b][r] = v;
          tmax = fmaxf(tmax, v);
        }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mn = fmaxf(m, tmax);
      const float corr = __builtin_amdgcn_exp2f(m - mn);
      float ps = 0.f;
      h8 pf[2];
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(sc[b][r] - mn);  // exp2(-inf) = 0 for masked keys
          ps += p;
          pf[b >> 1][(b & 1) * 4 + r] = (_Float16)p;
        }
      lsum = lsum * corr + ps;
      m = mn;
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] *= corr;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t *vrow = vt16 + (size_t)(16 * db + c16) * VS + 32 * t + 4 * g;
          const u32x2 lo8 = *(const u32x2 *)vrow, hi8 = *(const u32x2 *)(vrow + 16);
          const h8 vf = __builtin_bit_cast(h8, (u32x4){lo8.x, lo8.y, hi8.x, hi8.y});
          o[db] = MFMA16(vf, pf[t], o[db]);
        }
    }
    __syncthreads();
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (qi < T) {
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    uint16_t *orow = O + (size_t)qi * heads * D + (size_t)h * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      h4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (_Float16)(o[db][r] * inv);
      *(h4 *)(orow + 16 * db + 4 * g) = v;
    }
  }
}

int dj_launch_attention(hipStream_t s, int T, int heads, int kv, int D, const uint16_t *Q, int q_stride, dj_kv_src A,
                        dj_kv_src B, const int32_t *rng, float scale, uint16_t *O) {
  dim3 grid(dj_cdiv(T, 64), heads);
  const int4 *r4 = (const int4 *)rng;
  switch (D) {
    case 64: k_attn<64><<<grid, 256, 0, s>>>(T, heads, kv, Q, q_stride, A, B, r4, scale, O); break;
    case 128: k_attn<128><<<grid, 256, 0, s>>>(T, heads, kv, Q, q_stride, A, B, r4, scale, O); break;
    case 256: k_attn<256><<<grid, 256, 0, s>>>(T, heads, kv, Q, q_stride, A, B, r4, scale, O); break;
    default: return dj_fail(DJ_EINVAL, "decision.js: attention head dim %d (64, 128 or 256)", D);
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
  DJ_REQUIRE(D == 64 || D == 128 || D == 256, "decision.js: attention head dim %d (64, 128 or 256)", D);
  DJ_REQUIRE(src_ok(A, kv, D) && src_ok(B, kv, D), "decision.js: attention: bad key/value source");
  DJ_OP_BEGIN(rec, "attention");
  if (T > 0) {
    int st = dj_launch_attention(rec->ctx->stream, T, heads, kv, D, Q, q_stride, A, B, rng, scale, O);
    if (st) return st;
  }
  char shape[48];
  snprintf(shape, sizeof shape, "[T%d h%d kv%d D%d]", T, heads, kv, D);
  return dj_op_end(rec, "attention", shape);
}
