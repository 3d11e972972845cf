// EmbeddingGemma 2's per-layer-embedding mix and its pooled projection (eg2-kernels.ts:179-228).
#include <math.h>
#include "dj_internal.h"

namespace {

__device__ __forceinline__ float hf(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }

// gelu of eg2-kernels.ts:9-13: tanh form, its argument clamped to +-15; exp and the division in IEEE f32
__device__ __forceinline__ float gelu_tanh(float x) {
  const float u = fminf(fmaxf(0.7978845608f * (x + 0.044715f * x * x * x), -15.0f), 15.0f);
  const float e = expf(2.0f * u);
  return 0.5f * x * (1.0f + (e - 1.0f) / (e + 1.0f));
}

// One wave per row of P values (P % 8 == 0, chunks of 8 per lane): O = f16(gelu(G) * E / rms(E) * w), the sum of
// squares of E in f32.
__global__ __launch_bounds__(256) void k_ple_mix(int T, int P, const uint16_t *__restrict__ G, const uint16_t *__restrict__ E,
                                                 const uint16_t *__restrict__ W, float eps, uint16_t *__restrict__ O) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (t >= T) return;
  const uint16_t *e = E + (size_t)t * P, *g = G + (size_t)t * P;
  float ss = 0.f;
  for (int k = lane * 8; k < P; k += 512) {
    const h8 v = *(const h8 *)(e + k);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (float)v[i] * (float)v[i];
  }
  const float inv = 1.0f / sqrtf(group_sum<64>(ss) / (float)P + eps);
  for (int k = lane * 8; k < P; k += 512) {
    const h8 v = *(const h8 *)(e + k), gv = *(const h8 *)(g + k), w = *(const h8 *)(W + k);
    h8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (_Float16)(gelu_tanh((float)gv[i]) * (float)v[i] * inv * (float)w[i]);
    *(h8 *)(O + (size_t)t * P + k) = o;
  }
}

// out[s, n] = sum_k mean[s, k] * W[n, k] in f32, W f16 [N, H]: one wave per (sequence, 4 outputs), the pooled row
// read as float4s, lane partials added by the row sums (fixed order).
__global__ __launch_bounds__(256) void k_project_f16(int S, int H, int N, const float *__restrict__ mean,
                                                     const uint16_t *__restrict__ W, float *__restrict__ out) {
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int groups = (N + 3) / 4;
  if (wave >= S * groups) return;
  const int s = wave / groups, n0 = (wave % groups) * 4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = lane * 4; k < H; k += 256) {
    const float4 m = *(const float4 *)(mean + (size_t)s * H + k);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (n0 + j >= N) break;
      const uint16_t *w = W + (size_t)(n0 + j) * H + k;
      acc[j] += m.x * hf(w[0]) + m.y * hf(w[1]) + m.z * hf(w[2]) + m.w * hf(w[3]);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float v = group_sum<64>(acc[j]);
    if (lane == 0 && n0 + j < N) out[(size_t)s * N + n0 + j] = v;
  }
}

}  // namespace

extern "C" int dj_ple_mix(dj_rec *rec, int T, int P, const uint16_t *G, const uint16_t *E, const uint16_t *w, float eps,
                          uint16_t *O) {
  DJ_REQUIRE(G && E && w && O && T >= 0 && P > 0 && P % 8 == 0,
             "decision.js: ple_mix: bad arguments (P %d must be a multiple of 8)", P);
  DJ_OP_BEGIN(rec, "ple_mix");
  if (T > 0) k_ple_mix<<<(unsigned)dj_cdiv(T, 4), 256, 0, rec->ctx->stream>>>(T, P, G, E, w, eps, O);
  return dj_op_end(rec, "ple_mix");
}

extern "C" int dj_pool_project(dj_rec *rec, int T, int S, int H, int N, const uint16_t *X, const uint32_t *seqs,
                               const uint16_t *W, float *out) {
  DJ_REQUIRE(X && seqs && W && out && T > 0 && S >= 0 && H > 0 && H % 4 == 0 && N > 0,
             "decision.js: pool_project: bad arguments (H %d must be a multiple of 4)", H);
  float *mean = nullptr;
  DJ_REQUIRE(dj_gemm_workspace(rec->ctx, (size_t)S * H, &mean) == DJ_OK,
             "decision.js: pool_project: %d sequences x %d values exceed the workspace", S, H);
  DJ_OP_BEGIN(rec, "pool_project");
  if (S > 0) {
    dj_launch_mean_pool(rec->ctx->stream, T, S, H, X, seqs, mean);
    k_project_f16<<<(unsigned)dj_cdiv((long)S * ((N + 3) / 4), 4), 256, 0, rec->ctx->stream>>>(S, H, N, mean, W, out);
  }
  return dj_op_end(rec, "pool_project");
}
