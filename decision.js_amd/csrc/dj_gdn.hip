// d3-lite's Gated DeltaNet mixer after the in-projection (gdnLayer, d3-kernels.ts:9-149), one workgroup per
// (sequence, head): 512 threads = 128 rows of the f32 state S [v 128 x k 128] x 4 lanes, each lane holding 32
// of a row's k columns (the row's float4 chunks j*4 + lane, so the 4 lanes of a row read neighbouring 16-byte
// chunks of the shared q and k vectors). Per chunk of C tokens:
//  1. the causal 4-tap conv + SiLU of the head's q, k and v channels (zero before the sequence start; rounded to
//     f16, the stored activation it stands for), q and k L2-normalised (q also by 128^-1/2), the gates
//     decay = exp(-exp(A_log) softplus(a + dt_bias)) and beta = sigmoid(b), all into LDS;
//  2. the delta rule per token, on the old state in one pass: r = S k, p = S q, kq = k . q; delta = beta (v -
//     decay r); o = decay p + kq delta; S <- decay S + delta k^T (o replaces v in LDS);
//  3. the gated RMSNorm, y = f16(o / rms(o) * w * silu(z)).
// A sequence is span a then span b (a shared trunk, rescanned by each question, then the question; or the
// whole sequence and nothing): span a's outputs are written only when its flag (bit 31 of its length) is set.
#include <math.h>
#include "dj_internal.h"

namespace {

constexpr int C = 32;       // tokens per chunk
constexpr int DK = 128;     // key / value head dim
constexpr int NT = 512;     // threads: 128 rows x 4 lanes

__device__ __forceinline__ float hf(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

struct Span {
  uint32_t a0, alen, b0, blen;
  bool write_a;
  __device__ __forceinline__ uint32_t len() const { return alen + blen; }
  __device__ __forceinline__ uint32_t row(uint32_t v) const { return v < alen ? a0 + v : b0 + v - alen; }
};

__global__ __launch_bounds__(NT) void k_gdn(int T, int LH, int stride, const uint4 *__restrict__ spans,
                                            const uint16_t *__restrict__ Z, const uint16_t *__restrict__ Wc,
                                            const uint16_t *__restrict__ Alog, const uint16_t *__restrict__ dtb,
                                            const uint16_t *__restrict__ gw, float eps, uint16_t *__restrict__ Y) {
  __shared__ __attribute__((aligned(16))) float qs[C * DK];
  __shared__ __attribute__((aligned(16))) float ks[C * DK];
  __shared__ __attribute__((aligned(16))) float vs[C * DK];  // v, then o
  __shared__ float2 gs[C];                                    // (decay, beta)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = blockIdx.x % LH;
  const uint4 sp = spans[blockIdx.x / LH];
  const Span S{sp.x, sp.y & 0x7fffffffu, sp.z, sp.w, (sp.y >> 31) != 0};
  const uint32_t end = S.len();
  const int QK = LH * DK;
  const int row = tid >> 2, part = tid & 3;
  f4 st[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) st[j] = f4{0.f, 0.f, 0.f, 0.f};

  // phase-1 roles: threads 0..383 own one conv channel (q, k, v of this head), 384..511 the gates
  const int cc = tid < 3 * DK ? tid : 0;
  const int gch = (cc / DK) * QK + h * DK + cc % DK;
  float w4[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) w4[j] = hf(Wc[(size_t)gch * 4 + j]);
  const float negA = -expf(hf(Alog[h])), dt = hf(dtb[h]);
  auto input = [&](uint32_t v) -> float {  // channel gch at sequence index v (the caller checks v >= 0)
    const uint32_t r = S.row(v);
    return r < (uint32_t)T ? hf(Z[(size_t)r * stride + gch]) : 0.f;
  };

  for (uint32_t t0 = 0; t0 < end; t0 += C) {
    const int n = (int)min((uint32_t)C, end - t0);
    // 1. conv + SiLU (f16-rounded), gates
    if (tid < 3 * DK) {
      float xm3 = t0 >= 3 ? input(t0 - 3) : 0.f, xm2 = t0 >= 2 ? input(t0 - 2) : 0.f, xm1 = t0 >= 1 ? input(t0 - 1) : 0.f;
      float *dst = cc < DK ? qs : cc < 2 * DK ? ks : vs;
      const int d = cc % DK;
      for (int c = 0; c < n; ++c) {
        const float x0 = input(t0 + c);
        const float y = w4[0] * xm3 + w4[1] * xm2 + w4[2] * xm1 + w4[3] * x0;
        dst[c * DK + d] = (float)(_Float16)silu(y);
        xm3 = xm2;
        xm2 = xm1;
        xm1 = x0;
      }
    } else {
      const int c = tid - 3 * DK;
      if (c < n) {
        const uint32_t r = S.row(t0 + c);
        float b = 0.f, a = dt;
        if (r < (uint32_t)T) {
          const uint16_t *zr = Z + (size_t)r * stride + 4 * QK;
          b = hf(zr[h]);
          a += hf(zr[LH + h]);
        }
        const float sp = a > 20.f ? a : logf(1.0f + expf(a));
        gs[c] = make_float2(expf(negA * sp), 1.0f / (1.0f + expf(-b)));
      }
    }
    __syncthreads();
    // q and k L2 norms: one wave per (token, q or k) vector, 2 values per lane
    for (int k = wave; k < 2 * n; k += NT / 64) {
      float *vec = (k & 1 ? ks : qs) + (k >> 1) * DK;
      const float a = vec[lane], b = vec[lane + 64];
      const float inv = 1.0f / sqrtf(group_sum<64>(a * a + b * b) + 1e-6f) * (k & 1 ? 1.0f : 0.08838834764831845f);
      vec[lane] = a * inv;
      vec[lane + 64] = b * inv;
    }
    __syncthreads();
    // 2. the delta rule, token by token
    for (int c = 0; c < n; ++c) {
      const float2 g = gs[c];
      const f4 *k4 = (const f4 *)(ks + c * DK), *q4 = (const f4 *)(qs + c * DK);
      f4 kk[8];
      float r = 0.f, p = 0.f, kq = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kk[j] = k4[j * 4 + part];
        const f4 qq = q4[j * 4 + part];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r += st[j][e] * kk[j][e];
          p += st[j][e] * qq[e];
          kq += kk[j][e] * qq[e];
        }
      }
      r += __shfl_xor(r, 1, 64);
      p += __shfl_xor(p, 1, 64);
      kq += __shfl_xor(kq, 1, 64);
      r += __shfl_xor(r, 2, 64);
      p += __shfl_xor(p, 2, 64);
      kq += __shfl_xor(kq, 2, 64);
      const float delta = (vs[c * DK + row] - g.x * r) * g.y;
      const float o = g.x * p + kq * delta;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) st[j][e] = st[j][e] * g.x + kk[j][e] * delta;
      if (part == 0) vs[c * DK + row] = o;  // the row's 4 lanes (one wave) have read v above
    }
    __syncthreads();
    // 3. gated RMSNorm, one wave per token
    for (int c = wave; c < n; c += NT / 64) {
      const uint32_t v = t0 + c;
      const uint32_t r = S.row(v);
      if ((v < S.alen && !S.write_a) || r >= (uint32_t)T) continue;
      const float a = vs[c * DK + lane], b = vs[c * DK + lane + 64];
      const float inv = 1.0f / sqrtf(group_sum<64>(a * a + b * b) / (float)DK + eps);
      const uint16_t *z = Z + (size_t)r * stride + 3 * QK + h * DK;
      uint16_t *y = Y + (size_t)r * QK + h * DK;
      const float z0 = hf(z[lane]), z1 = hf(z[lane + 64]);
      y[lane] = __builtin_bit_cast(uint16_t, (_Float16)(a * inv * hf(gw[lane]) * silu(z0)));
      y[lane + 64] = __builtin_bit_cast(uint16_t, (_Float16)(b * inv * hf(gw[lane + 64]) * silu(z1)));
    }
    __syncthreads();
  }
}

}  // namespace

extern "C" int dj_gdn(dj_rec *rec, int T, int nspans, const uint32_t *spans, int LH, int stride, const uint16_t *Z,
                      const uint16_t *conv_w, const uint16_t *A_log, const uint16_t *dt_bias, const uint16_t *gnorm,
                      float eps, uint16_t *Y) {
  DJ_REQUIRE(Z && spans && conv_w && A_log && dt_bias && gnorm && Y && T >= 0 && nspans >= 0 && LH > 0,
             "decision.js: gdn: bad arguments");
  DJ_REQUIRE(stride >= 4 * LH * DK + 2 * LH, "decision.js: gdn: in-projection rows of %d values hold fewer than "
             "q | k | v | z | b | a (%d)", stride, 4 * LH * DK + 2 * LH);
  DJ_REQUIRE((long)nspans * LH < (1L << 31), "decision.js: gdn: %d sequences x %d heads is too large", nspans, LH);
  DJ_OP_BEGIN(rec, "gdn");
  if (nspans > 0 && T > 0)
    k_gdn<<<(unsigned)(nspans * LH), NT, 0, rec->ctx->stream>>>(T, LH, stride, (const uint4 *)spans, Z, conv_w, A_log,
                                                                 dt_bias, gnorm, eps, Y);
  return dj_op_end(rec, "gdn");
}
