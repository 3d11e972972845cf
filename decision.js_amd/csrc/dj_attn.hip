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

template <int D>
__global__ __launch_bounds__(256) void k_attn(int T, int heads, int kv, const uint16_t *__restrict__ Q, int q_stride,
                                              dj_kv_src A, dj_kv_src B, const int4 *__restrict__ rng, float scale,
                                              uint16_t *__restrict__ O) {
  constexpr int NS = D / 32;   // MFMA k-steps over the head dim
  constexpr int NDB = D / 16;  // 16-row blocks of O^T
  constexpr int CH = D / 8;    // 16-byte chunks per K row
  constexpr int SW = CH >= 16 ? 15 : 7;
  constexpr int VS = 68;       // V^T row stride in halves: 64 keys + 4 (conflict-free 8-byte reads)
  __shared__ uint4 Ks[64 * CH];
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

  const int qi = q0 + wave * 16 + c16;
  const int qc = min(qi, T - 1);
  h8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = *(const h8 *)(Q + (size_t)qc * q_stride + (size_t)h * D + s * 32 + g * 8);
  const int4 rq = rng[qc];

  f4 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (f4){0.f, 0.f, 0.f, 0.f};
  float m = -1e30f, lsum = 0.f;
  const uint16_t *vt16 = (const uint16_t *)Vt;

  for (int src = 0; src < 2; ++src) {
    const dj_kv_src S = src ? B : A;
    const int lo = max(bounds[2 * src], 0), hi = min(bounds[2 * src + 1], S.rows);
    const int qlo = src ? rq.z : rq.x, qhi = src ? rq.w : rq.y;
    const uint16_t *kbase = S.base + S.k_col + (size_t)kvh * D;
    const uint16_t *vbase = S.base + S.v_col + (size_t)kvh * D;
    for (int k0 = lo; k0 < hi; k0 += 64) {
      // K tile, row-major, chunk ch of row r at (ch ^ (r & SW))
      for (int c = tid; c < 64 * CH; c += 256) {
        const int r = c / CH, ch = c % CH;
        const int row = min(k0 + r, hi - 1);
        Ks[r * CH + (ch ^ (r & SW))] = *(const uint4 *)(kbase + (size_t)row * S.stride + ch * 8);
      }
      // V tile transposed: Vt[d][key], two keys per 32-bit store
      for (int it = tid; it < 32 * CH; it += 256) {
        const int kp = it & 31, ch = it >> 5, r0 = 2 * kp;
        const int row0 = min(k0 + r0, hi - 1), row1 = min(k0 + r0 + 1, hi - 1);
        // integer lanes, not vector elements: a bit_cast of an f16 vector element read element 0 only
        const uint4 v0 = *(const uint4 *)(vbase + (size_t)row0 * S.stride + ch * 8);
        const uint4 v1 = *(const uint4 *)(vbase + (size_t)row1 * S.stride + ch * 8);
        const uint32_t a[4] = {v0.x, v0.y, v0.z, v0.w}, b[4] = {v1.x, v1.y, v1.z, v1.w};
        uint32_t *dst = Vt + (((ch * 8) * VS + r0) >> 1);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          dst[(2 * w) * (VS / 2)] = (a[w] & 0xffffu) | (b[w] << 16);          // d = 8ch + 2w: (key r0, key r0+1)
          dst[(2 * w + 1) * (VS / 2)] = (a[w] >> 16) | (b[w] & 0xffff0000u);  // d = 8ch + 2w + 1
        }
      }
      __syncthreads();

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
          const float v = ok ? sc[b][r] * scale : -INFINITY;
          sc[b][r] = v;
          tmax = fmaxf(tmax, v);
        }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mn = fmaxf(m, tmax);
      const float corr = expf(m - mn);
      float ps = 0.f;
      h8 pf[2];
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = sc[b][r] == -INFINITY ? 0.f : expf(sc[b][r] - mn);
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
          const uint2 lo8 = *(const uint2 *)vrow, hi8 = *(const uint2 *)(vrow + 16);
          const h8 vf = __builtin_bit_cast(h8, (uint4){lo8.x, lo8.y, hi8.x, hi8.y});
          o[db] = MFMA16(vf, pf[t], o[db]);
        }
      __syncthreads();
    }
  }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (qi < T) {
    const float inv = 1.0f / lsum;
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
