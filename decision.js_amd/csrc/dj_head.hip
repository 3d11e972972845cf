// d1-omni's decision head and marker scorer (kernels.ts:186-283): question-type rows added to the trunk output,
// bias + activation in place, residual + LayerNorm, the rows at the option markers, and the scorer's last
// Linear(H, 1). All HBM-bound and small: elementwise ops take 8 halves per lane (one 16-byte load), row ops one
// wave per row with shuffle reductions (no shared memory).
#include <math.h>
#include "dj_internal.h"

namespace {

__device__ __forceinline__ float hf(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }

// Abramowitz & Stegun 7.1.26 (|error| < 1.5e-7), the erf of BIAS_ACT's GELU (kernels.ts:210-214)
__device__ __forceinline__ float erf_as(float x) {
  const float t = 1.0f / (1.0f + 0.3275911f * fabsf(x));
  const float y = 1.0f - ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
                          0.254829592f) * t * expf(-x * x);
  return x >= 0.0f ? y : -y;
}

// Xo[t, :] = f16(f32(Xi[t, :]) + f32(E[idx[t], :])); 8 columns per lane (H % 8 == 0)
__global__ __launch_bounds__(256) void k_add_rows(int T, int H, const uint16_t *__restrict__ Xi, const uint32_t *__restrict__ idx,
                                                  int rows, const uint16_t *__restrict__ E, uint16_t *__restrict__ Xo) {
  const int per = H >> 3;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)T * per) return;
  const int t = (int)(i / per), k0 = (int)(i % per) * 8;
  uint32_t r = idx[t];
  if (r >= (uint32_t)rows) r = rows - 1;
  const h8 x = *(const h8 *)(Xi + (size_t)t * H + k0), e = *(const h8 *)(E + (size_t)r * H + k0);
  h8 o;
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = (_Float16)((float)x[k] + (float)e[k]);
  *(h8 *)(Xo + (size_t)t * H + k0) = o;
}

// Y[t, n] = f16(act(f32(Y[t, n]) + f32(b[n]))) in place; act 0 none, 1 ReLU, 2 GELU (erf); 8 columns per lane
__global__ __launch_bounds__(256) void k_bias_act(int T, int N, uint16_t *__restrict__ Y, const uint16_t *__restrict__ b,
                                                  int act) {
  const int per = N >> 3;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)T * per) return;
  const int t = (int)(i / per), n0 = (int)(i % per) * 8;
  h8 y = *(h8 *)(Y + (size_t)t * N + n0);
  const h8 bb = *(const h8 *)(b + n0);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float v = (float)y[k] + (float)bb[k];
    if (act == 1) v = fmaxf(v, 0.0f);
    if (act == 2) v = 0.5f * v * (1.0f + erf_as(v * 0.70710678f));
    y[k] = (_Float16)v;
  }
  *(h8 *)(Y + (size_t)t * N + n0) = y;
}

// One wave per row: if add, X += Y (stored f16; the sums use the unrounded value, as ADD_LAYERNORM keeps v in a
// register); mean and E[x^2] in f32; var = max(E[x^2] - mean^2, 0); O = f16((f32(X) - mean) * inv * w + b), with
// X the stored f16 row.
__global__ __launch_bounds__(256) void k_add_layernorm(int T, int H, int add, float eps, uint16_t *__restrict__ X,
                                                       const uint16_t *__restrict__ Yr, const uint16_t *__restrict__ W,
                                                       const uint16_t *__restrict__ Bb, uint16_t *__restrict__ O) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  uint16_t *x = X + (size_t)t * H;
  float a = 0.f, q = 0.f;
  for (int k0 = lane * 8; k0 < H; k0 += 512) {
    h8 v = *(const h8 *)(x + k0);
    float f[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = (float)v[k];
    if (add) {
      const h8 y = *(const h8 *)(Yr + (size_t)t * H + k0);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        f[k] += (float)y[k];
        v[k] = (_Float16)f[k];
      }
      *(h8 *)(x + k0) = v;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      a += f[k];
      q += f[k] * f[k];
    }
  }
  a = group_sum<64>(a);
  q = group_sum<64>(q);
  const float mean = a / (float)H;
  const float inv = 1.0f / sqrtf(fmaxf(q / (float)H - mean * mean, 0.0f) + eps);
  for (int k0 = lane * 8; k0 < H; k0 += 512) {
    const h8 v = *(const h8 *)(x + k0), w = *(const h8 *)(W + k0), b = *(const h8 *)(Bb + k0);
    h8 o;
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] = (_Float16)(((float)v[k] - mean) * inv * (float)w[k] + (float)b[k]);
    *(h8 *)(O + (size_t)t * H + k0) = o;
  }
}

// G[m, :] = X[rows[m], :] (rows clamped to [0, T))
__global__ __launch_bounds__(256) void k_gather_rows(int M, int H, int T, const uint16_t *__restrict__ X,
                                                     const uint32_t *__restrict__ rows, uint16_t *__restrict__ G) {
  const int per = H >> 3;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)M * per) return;
  const int m = (int)(i / per), k0 = (int)(i % per) * 8;
  uint32_t r = rows[m];
  if (r >= (uint32_t)T) r = T - 1;
  *(h8 *)(G + (size_t)m * H + k0) = *(const h8 *)(X + (size_t)r * H + k0);
}

// out[m] = sum_k f32(Y[m, k]) f32(w[k]) + f32(b[0]), one wave per row
__global__ __launch_bounds__(256) void k_score(int M, int H, const uint16_t *__restrict__ Y, const uint16_t *__restrict__ w,
                                               const uint16_t *__restrict__ b, float *__restrict__ out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + wave;
  if (m >= M) return;
  float d = 0.f;
  for (int k0 = lane * 8; k0 < H; k0 += 512) {
    const h8 y = *(const h8 *)(Y + (size_t)m * H + k0), ww = *(const h8 *)(w + k0);
#pragma unroll
    for (int k = 0; k < 8; ++k) d += (float)y[k] * (float)ww[k];
  }
  d = group_sum<64>(d);
  if (lane == 0) out[m] = d + hf(b[0]);
}

}  // namespace

extern "C" int dj_add_rows(dj_rec *rec, int T, int H, const uint16_t *Xi, const uint32_t *idx, const uint16_t *E, int rows,
                           uint16_t *Xo) {
  DJ_REQUIRE(Xi && idx && E && Xo && T >= 0 && H > 0 && H % 8 == 0 && rows > 0,
             "decision.js: add_rows: bad arguments (H %d must be a multiple of 8)", H);
  DJ_OP_BEGIN(rec, "add_rows");
  const long n = (long)T * (H / 8);
  if (n > 0) k_add_rows<<<(unsigned)dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(T, H, Xi, idx, rows, E, Xo);
  return dj_op_end(rec, "add_rows");
}

extern "C" int dj_bias_act(dj_rec *rec, int T, int N, uint16_t *Y, const uint16_t *b, int act) {
  DJ_REQUIRE(Y && b && T >= 0 && N > 0 && N % 8 == 0 && act >= 0 && act <= 2,
             "decision.js: bias_act: bad arguments (N %d must be a multiple of 8, act 0..2)", N);
  DJ_OP_BEGIN(rec, "bias_act");
  const long n = (long)T * (N / 8);
  if (n > 0) k_bias_act<<<(unsigned)dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(T, N, Y, b, act);
  return dj_op_end(rec, "bias_act");
}

extern "C" int dj_add_layernorm(dj_rec *rec, int T, int H, int add, float eps, uint16_t *X, const uint16_t *Y,
                                const uint16_t *w, const uint16_t *b, uint16_t *O) {
  DJ_REQUIRE(X && w && b && O && (!add || Y) && T >= 0 && H > 0 && H % 8 == 0,
             "decision.js: add_layernorm: bad arguments (H %d must be a multiple of 8)", H);
  DJ_OP_BEGIN(rec, "add_layernorm");
  if (T > 0) k_add_layernorm<<<(unsigned)dj_cdiv(T, 4), 256, 0, rec->ctx->stream>>>(T, H, add, eps, X, Y, w, b, O);
  return dj_op_end(rec, "add_layernorm");
}

extern "C" int dj_gather_rows(dj_rec *rec, int M, int H, int T, const uint16_t *X, const uint32_t *rows, uint16_t *G) {
  DJ_REQUIRE(X && rows && G && M >= 0 && T > 0 && H > 0 && H % 8 == 0,
             "decision.js: gather_rows: bad arguments (H %d must be a multiple of 8)", H);
  DJ_OP_BEGIN(rec, "gather_rows");
  const long n = (long)M * (H / 8);
  if (n > 0) k_gather_rows<<<(unsigned)dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(M, H, T, X, rows, G);
  return dj_op_end(rec, "gather_rows");
}

extern "C" int dj_score(dj_rec *rec, int M, int H, const uint16_t *Y, const uint16_t *w, const uint16_t *b, float *out) {
  DJ_REQUIRE(Y && w && b && out && M >= 0 && H > 0 && H % 8 == 0,
             "decision.js: score: bad arguments (H %d must be a multiple of 8)", H);
  DJ_OP_BEGIN(rec, "score");
  if (M > 0) k_score<<<(unsigned)dj_cdiv(M, 4), 256, 0, rec->ctx->stream>>>(M, H, Y, w, b, out);
  return dj_op_end(rec, "score");
}
