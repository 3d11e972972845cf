// Memory-bound kernels of the scoring path and their C-ABI entry points: embedding gather, residual +
// RMSNorm, sandwich norm, q/k(/v) norm + RoPE, KV store, answer-row logits, readout, pooling, the small
// f32 dense head, and the copy used by snapshots. One wave (64 lanes) owns a row wherever a row is
// reduced, so reductions are shuffles, not shared-memory trees.
#include <math.h>
#include "dj_internal.h"

#define WAVE 64

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ _Float16 u2h(uint16_t u) { return __builtin_bit_cast(_Float16, u); }
__device__ __forceinline__ uint16_t h2u(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }
__device__ __forceinline__ float hf(uint16_t u) { return (float)u2h(u); }

// ---------------------------------------------------------------- gather (kernels.ts:6-21, 292-296)
// X = f16(f16(code) - f16(zp)) * scale: both operands are f16, the product is rounded once (RNE).
template <int BITS>
__global__ void k_gather(const uint32_t *__restrict__ ids, int T, int H, int V, const uint8_t *__restrict__ codes,
                         const uint16_t *__restrict__ scales, uint16_t *__restrict__ X) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = H / 8;
  if (i >= (long)T * per) return;
  const int t = (int)(i / per), k0 = (int)(i % per) * 8;
  uint32_t row = ids[t];
  if (row >= (uint32_t)V) row = V - 1;
  const _Float16 s = u2h(scales[(size_t)row * (H / 32) + k0 / 32]);
  const _Float16 zp = BITS == 8 ? (_Float16)128.0f : (_Float16)8.0f;
  h8 out;
  if (BITS == 8) {
    const uint2 raw = *(const uint2 *)(codes + (size_t)row * H + k0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t c = ((j < 4 ? raw.x : raw.y) >> (8 * (j & 3))) & 255u;
      out[j] = ((_Float16)(float)c - zp) * s;
    }
  } else {
    const uint32_t raw = *(const uint32_t *)(codes + (size_t)row * (H / 2) + k0 / 2);
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = ((_Float16)(float)((raw >> (4 * j)) & 15u) - zp) * s;
  }
  *(h8 *)(X + (size_t)t * H + k0) = out;
}

extern "C" int dj_gather_q(dj_rec *rec, const uint32_t *ids, int T, const dj_weight *e, uint16_t *X) {
  DJ_REQUIRE(e && e->layout == DJ_W_PLAIN, "decision.js: gather needs a plain (untiled) embedding");
  DJ_REQUIRE(ids && X && T >= 0 && e->K % 32 == 0, "decision.js: gather: bad arguments");
  DJ_OP_BEGIN(rec, "gather_q");
  if (T > 0) {
    const long n = (long)T * (e->K / 8);
    if (e->bits == 8)
      k_gather<8><<<dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(ids, T, e->K, e->N, e->codes, (const uint16_t *)e->scales, X);
    else
      k_gather<4><<<dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(ids, T, e->K, e->N, e->codes, (const uint16_t *)e->scales, X);
  }
  return dj_op_end(rec, "gather_q");
}

// ---------------------------------------------------------------- residual + RMSNorm (kernels.ts:23-46)
// One wave per row, 8 halves per lane per chunk; NC = ceil(H / 512) chunks per lane stay in registers
// between the sum of squares and the scaling (NC = 0: rows too long for that, re-read from memory).
// PARTS: Y arrives as S f32 partial slices of a product split along K (P, `slice` floats apart).
template <int NC, bool PARTS>
__global__ __launch_bounds__(256) void k_add_rmsnorm(int T, int H, int add, float eps, uint16_t *__restrict__ X,
                                                     const uint16_t *__restrict__ Y, const uint16_t *__restrict__ W,
                                                     uint16_t *__restrict__ O, const float *__restrict__ P, int S,
                                                     size_t slice, uint16_t *__restrict__ YW) {
  const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  if (row >= T) return;
  const size_t base = (size_t)row * H;
  constexpr int R = NC > 0 ? NC : 1;
  h8 xs[R];
  float ss = 0.f;
  auto step = [&](int k, h8 &x) {
    x = *(const h8 *)(X + base + k);
    if (add) {
      h8 y;
      if constexpr (PARTS) {  // Y is a K-split product: its f32 partials added in split order, rounded to f16
        const float *p = P + base + k;
        f4 lo = *(const f4 *)p, hi = *(const f4 *)(p + 4);
        for (int s = 1; s < S; ++s) {
          lo += *(const f4 *)(p + s * slice);
          hi += *(const f4 *)(p + s * slice + 4);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          y[j] = (_Float16)lo[j];
          y[j + 4] = (_Float16)hi[j];
        }
        *(h8 *)(YW + base + k) = y;  // the product's own output
      } else {
        y = *(const h8 *)(Y + base + k);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = (float)x[j] + (float)y[j];
        ss += v * v;  // the unrounded sum, as the reference squares v before storing it
        x[j] = (_Float16)v;
      }
      *(h8 *)(X + base + k) = x;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += (float)x[j] * (float)x[j];
    }
  };
  auto scale_out = [&](int k, const h8 &x, const h8 &w, float inv) {
    h8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (_Float16)((float)x[j] * inv * (float)w[j]);
    *(h8 *)(O + base + k) = o;
  };
  // the norm weight chunks are loaded with the row, so the only memory latency after the reduction is the store
  h8 ws[R];
  if (NC > 0) {
#pragma unroll
    for (int c = 0; c < R; ++c)
      if (lane * 8 + c * WAVE * 8 < H) {
        ws[c] = *(const h8 *)(W + lane * 8 + c * WAVE * 8);
        step(lane * 8 + c * WAVE * 8, xs[c]);
      }
  } else {
    for (int k = lane * 8; k < H; k += WAVE * 8) step(k, xs[0]);
  }
  const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)H + eps);
  if (NC > 0) {
#pragma unroll
    for (int c = 0; c < R; ++c)
      if (lane * 8 + c * WAVE * 8 < H) scale_out(lane * 8 + c * WAVE * 8, xs[c], ws[c], inv);
  } else {
    for (int k = lane * 8; k < H; k += WAVE * 8) scale_out(k, *(const h8 *)(X + base + k), *(const h8 *)(W + k), inv);
  }
}

// Chunks of 8 halves per lane for a row of H (H % 8 == 0): 1..8 in registers, 0 = re-read.
static int row_chunks(int H) {
  const int nc = dj_cdiv(H / 8, WAVE);
  return nc <= 8 ? nc : 0;
}

#define DJ_ROW_DISPATCH(KERNEL, H, grid, stream, ...)                          \
  switch (row_chunks(H)) {                                                     \
    case 1: KERNEL<1><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 2: KERNEL<2><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 3: KERNEL<3><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 4: KERNEL<4><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 5: KERNEL<5><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 6: KERNEL<6><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 7: KERNEL<7><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 8: KERNEL<8><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    default: KERNEL<0><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;          \
  }

// row kernels templated on (chunks, bool)
#define DJ_ROW_DISPATCH_B(KERNEL, B, H, grid, stream, ...)                        \
  switch (row_chunks(H)) {                                                        \
    case 1: KERNEL<1, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 2: KERNEL<2, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 3: KERNEL<3, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 4: KERNEL<4, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 5: KERNEL<5, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 6: KERNEL<6, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 7: KERNEL<7, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    case 8: KERNEL<8, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;           \
    default: KERNEL<0, B><<<grid, 256, 0, stream>>>(__VA_ARGS__); break;          \
  }

extern "C" int dj_add_rmsnorm(dj_rec *rec, int T, int H, int add, float eps, uint16_t *X, const uint16_t *Y,
                              const uint16_t *W, uint16_t *O) {
  DJ_REQUIRE(X && W && O && (Y || !add) && T >= 0 && H > 0 && H % 8 == 0,
             "decision.js: add_rmsnorm: bad arguments (H = %d must be a multiple of 8)", H);
  // a skinny product of Y held by the recorder runs split along K now, and this kernel sums its partials
  const float *parts = nullptr;
  int S = 1;
  if (add && T > 0)
    if (int st = dj_take_held_split(rec, Y, T, H, &parts, &S)) return st;
  DJ_OP_BEGIN(rec, "add_rmsnorm");
  if (T > 0) {
    if (parts)
      DJ_ROW_DISPATCH_B(k_add_rmsnorm, true, H, dj_cdiv(T, 4), rec->ctx->stream, T, H, add, eps, X, Y, W, O, parts, S,
                        (size_t)T * H, const_cast<uint16_t *>(Y))
    else
      DJ_ROW_DISPATCH_B(k_add_rmsnorm, false, H, dj_cdiv(T, 4), rec->ctx->stream, T, H, add, eps, X, Y, W, O, nullptr, 1,
                        (size_t)0, nullptr)
  }
  return dj_op_end(rec, "add_rmsnorm");
}

// ---------------------------------------------------------------- sandwich (eg2-kernels.ts:15-48)
// Same row layout as add_rmsnorm: the residual chunks stay in registers across the two reductions.
template <int NC>
__global__ __launch_bounds__(256) void k_sandwich(int T, int H, float eps, float scale, uint16_t *__restrict__ X,
                                                  const uint16_t *__restrict__ Y, const uint16_t *__restrict__ W1,
                                                  const uint16_t *__restrict__ W2, uint16_t *__restrict__ O) {
  const int row = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  if (row >= T) return;
  const size_t base = (size_t)row * H;
  constexpr int R = NC > 0 ? NC : 1;
  h8 xs[R], ys[R];
  auto live = [&](int c) { return lane * 8 + c * WAVE * 8 < H; };
  float iy = 0.f;
  if (Y) {
    float ss = 0.f;
    auto sq = [&](const h8 &y) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += (float)y[j] * (float)y[j];
    };
    if (NC > 0) {
#pragma unroll
      for (int c = 0; c < R; ++c)
        if (live(c)) { ys[c] = *(const h8 *)(Y + base + lane * 8 + c * WAVE * 8); sq(ys[c]); }
    } else {
      for (int k = lane * 8; k < H; k += WAVE * 8) sq(*(const h8 *)(Y + base + k));
    }
    iy = 1.0f / sqrtf(wave_sum(ss) / (float)H + eps);
  }
  float ss2 = 0.f;
  auto mix = [&](int k, const h8 &y, h8 &x) {
    x = *(const h8 *)(X + base + k);
    if (Y) {
      const h8 w1 = *(const h8 *)(W1 + k);
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (_Float16)(((float)x[j] + (float)y[j] * iy * (float)w1[j]) * scale);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = (_Float16)((float)x[j] * scale);
    }
    *(h8 *)(X + base + k) = x;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss2 += (float)x[j] * (float)x[j];  // the stored residual, as the next block reads it
  };
  if (NC > 0) {
#pragma unroll
    for (int c = 0; c < R; ++c)
      if (live(c)) mix(lane * 8 + c * WAVE * 8, ys[c], xs[c]);
  } else {
    for (int k = lane * 8; k < H; k += WAVE * 8) {
      h8 y = {};
      if (Y) y = *(const h8 *)(Y + base + k);
      mix(k, y, xs[0]);
    }
  }
  if (!W2) return;
  const float ix = 1.0f / sqrtf(wave_sum(ss2) / (float)H + eps);
  auto out = [&](int k, const h8 &x) {
    const h8 w2 = *(const h8 *)(W2 + k);
    h8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (_Float16)((float)x[j] * ix * (float)w2[j]);
    *(h8 *)(O + base + k) = o;
  };
  if (NC > 0) {
#pragma unroll
    for (int c = 0; c < R; ++c)
      if (live(c)) out(lane * 8 + c * WAVE * 8, xs[c]);
  } else {
    for (int k = lane * 8; k < H; k += WAVE * 8) out(k, *(const h8 *)(X + base + k));
  }
}

extern "C" int dj_sandwich(dj_rec *rec, int T, int H, float eps, float scale, uint16_t *X, const uint16_t *Y,
                           const uint16_t *W1, const uint16_t *W2, uint16_t *O) {
  DJ_REQUIRE(X && (W1 || !Y) && (O || !W2) && T >= 0 && H > 0 && H % 8 == 0, "decision.js: sandwich: bad arguments");
  DJ_OP_BEGIN(rec, "sandwich");
  if (T > 0) DJ_ROW_DISPATCH(k_sandwich, H, dj_cdiv(T, 4), rec->ctx->stream, T, H, eps, scale, X, Y, W1, W2, O);
  return dj_op_end(rec, "sandwich");
}

// ---------------------------------------------------------------- q/k(/v) norm + RoPE
// One workgroup per token; LPH lanes per head (a power of two). Lane s < rot/16 owns the 8 rotation pairs
// (d, d + rot/2), d = 8s..8s+7 (two 16-byte loads); the next (D - rot)/8 lanes own 8 unrotated dims each.
// cos/sin of the token's rot/2 angles are computed once into LDS (rope_cs).
template <int LPH>
__global__ __launch_bounds__(256) void k_qk_norm_rope(int T, int heads, int kv, int D, int stride, uint16_t *__restrict__ Z,
                                                      const uint16_t *__restrict__ qn, const uint16_t *__restrict__ kn,
                                                      int vnorm, const int32_t *__restrict__ pos, int pos_stride, float eps,
                                                      float theta, int rot, int mode) {
  __shared__ float2 tab[256];  // (cos, sin) of rotation pair i < rot / 2
  const int t = blockIdx.x;
  const int per = heads + kv + (vnorm ? kv : 0);
  const int sub = threadIdx.x % LPH, grp = threadIdx.x / LPH;
  const int half = rot / 2, npl = rot / 16, ntl = (D - rot) / 8;
  const bool pl = sub < npl, tl = !pl && sub < npl + ntl;
  const int d0 = pl ? 8 * sub : rot + 8 * (sub - npl);  // first owned dim
  constexpr int HPP = 256 / LPH;                        // heads per pass
  // this lane's values of a head and the head's norm weights (q or k); the first head's are loaded before the
  // table is built
  h8 x = {}, y = {}, wx = {}, wy = {};
  auto load = [&](int hh) {
    if (pl || tl) {
      const uint16_t *z = Z + (size_t)t * stride + (size_t)hh * D;
      x = *(const h8 *)(z + d0);
      if (pl) y = *(const h8 *)(z + half + d0);
      const uint16_t *nw = hh < heads ? qn : hh < heads + kv ? kn : nullptr;
      if (nw) {
        wx = *(const h8 *)(nw + d0);
        if (pl) wy = *(const h8 *)(nw + half + d0);
      }
    }
  };
  int hh = grp;
  if (hh < per) load(hh);
  if ((int)threadIdx.x < half) tab[threadIdx.x] = rope_cs((float)pos[(size_t)t * pos_stride], threadIdx.x, rot, theta, mode);
  __syncthreads();
  for (; hh < per; hh += HPP) {
    uint16_t *z = Z + (size_t)t * stride + (size_t)hh * D;
    if (hh != grp) load(hh);
    const bool isQ = hh < heads, isK = !isQ && hh < heads + kv;
    const uint16_t *nw = isQ ? qn : isK ? kn : nullptr;
    const bool norm = isQ ? qn != nullptr : isK ? kn != nullptr : true;  // v heads only come with vnorm
    const h8x2 o = norm_rope_lane<LPH>(x, y, wx, wy, nw != nullptr, norm, isQ || isK, pl, D, eps,
                                       [&](int i) { return tab[d0 + i]; });
    if (pl) {
      *(h8 *)(z + d0) = o.x;
      *(h8 *)(z + half + d0) = o.y;
    } else if (tl) {
      *(h8 *)(z + d0) = o.x;
    }
  }
}

static int qk_rope_check(int heads, int kv, int D, int stride, int rot) {
  DJ_REQUIRE(heads > 0 && kv > 0 && D > 0 && D <= 512 && rot > 0 && rot <= D && rot % 16 == 0 && (D - rot) % 8 == 0 &&
                 stride % 8 == 0 && stride >= (heads + 2 * kv) * D,
             "decision.js: qk_norm_rope: unsupported shape (D %d, rot %d, stride %d)", D, rot, stride);
  return DJ_OK;
}

int dj_launch_qk_norm_rope(hipStream_t s, int T, int heads, int kv, int D, int stride, uint16_t *Z, const uint16_t *qn,
                           const uint16_t *kn, int vnorm, const int32_t *pos, int pos_stride, float eps, float theta, int rot,
                           int mode) {
  const int lanes = rot / 16 + (D - rot) / 8;
#define DJ_ROPE_LAUNCH(L) \
  k_qk_norm_rope<L><<<T, 256, 0, s>>>(T, heads, kv, D, stride, Z, qn, kn, vnorm, pos, pos_stride, eps, theta, rot, mode)
  if (lanes <= 4) DJ_ROPE_LAUNCH(4);
  else if (lanes <= 8) DJ_ROPE_LAUNCH(8);
  else if (lanes <= 16) DJ_ROPE_LAUNCH(16);
  else if (lanes <= 32) DJ_ROPE_LAUNCH(32);
  else DJ_ROPE_LAUNCH(64);
#undef DJ_ROPE_LAUNCH
  return DJ_OK;
}

extern "C" int dj_qk_norm_rope(dj_rec *rec, int T, int heads, int kv, int D, int stride, uint16_t *Z, const uint16_t *qn,
                               const uint16_t *kn, int vnorm, const int32_t *pos, int pos_stride, float eps, float theta,
                               int rot, int mode) {
  DJ_REQUIRE(Z && pos && T >= 0, "decision.js: qk_norm_rope: bad arguments");
  if (int st = qk_rope_check(heads, kv, D, stride, rot)) return st;
  DJ_REQUIRE(mode == DJ_ROPE_POW_NEG || mode == DJ_ROPE_INV_POW, "decision.js: qk_norm_rope: unknown rope mode");
  DJ_OP_BEGIN(rec, "qk_norm_rope");
  if (T > 0)
    dj_launch_qk_norm_rope(rec->ctx->stream, T, heads, kv, D, stride, Z, qn, kn, vnorm, pos, pos_stride, eps, theta, rot,
                           mode);
  return dj_op_end(rec, "qk_norm_rope");
}

// ---------------------------------------------------------------- RoPE table (one per forward)
__global__ __launch_bounds__(256) void k_rope_table(int T, const int32_t *__restrict__ pos, int pos_stride, float theta,
                                                    int rot, int mode, float2 *__restrict__ tab) {
  const int half = rot / 2;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)T * half) return;
  const int t = (int)(i / half), j = (int)(i % half);
  tab[i] = rope_cs((float)pos[(size_t)t * pos_stride], j, rot, theta, mode);
}

extern "C" int dj_rope_table(dj_rec *rec, int T, const int32_t *pos, int pos_stride, float theta, int rot, int mode,
                             float *tab) {
  DJ_REQUIRE(pos && tab && T >= 0 && rot > 0 && rot % 16 == 0 && rot <= 512, "decision.js: rope_table: bad arguments");
  DJ_REQUIRE(mode == DJ_ROPE_POW_NEG || mode == DJ_ROPE_INV_POW, "decision.js: rope_table: unknown rope mode");
  DJ_OP_BEGIN(rec, "rope_table");
  if (T > 0)
    k_rope_table<<<dj_cdiv((long)T * (rot / 2), 256), 256, 0, rec->ctx->stream>>>(T, pos, pos_stride, theta, rot, mode,
                                                                                 (float2 *)tab);
  return dj_op_end(rec, "rope_table");
}

// ---------------------------------------------------------------- KV store (kept prefix of a shared state)
__global__ void k_kv_store(int T, int width, const uint16_t *__restrict__ Z, int stride, int k_col, uint16_t *__restrict__ C,
                           int row0) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per = width / 8;
  if (i >= (long)T * per) return;
  const int t = (int)(i / per), c = (int)(i % per) * 8;
  *(h8 *)(C + (size_t)(row0 + t) * width + c) = *(const h8 *)(Z + (size_t)t * stride + k_col + c);
}

extern "C" int dj_kv_store(dj_rec *rec, int T, int kv, int D, const uint16_t *Z, int stride, int k_col, uint16_t *C, int row0) {
  const int width = 2 * kv * D;
  DJ_REQUIRE(Z && C && T >= 0 && row0 >= 0 && width % 8 == 0 && k_col % 8 == 0 && stride % 8 == 0 &&
                 k_col + width <= stride,
             "decision.js: kv_store: bad arguments");
  DJ_OP_BEGIN(rec, "kv_store");
  const long n = (long)T * (width / 8);
  if (n > 0) k_kv_store<<<dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(T, width, Z, stride, k_col, C, row0);
  return dj_op_end(rec, "kv_store");
}

// ---------------------------------------------------------------- block reduction helper (256 threads)
__device__ __forceinline__ float block_sum256(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x / WAVE;
  __syncthreads();
  if ((threadIdx.x % WAVE) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// ---------------------------------------------------------------- answer-row logits (kernels.ts:149-185)
// normed = f32(X) * inv * f32(w) (kept in f32), dot with (f32(code) - zp) * f32(scale), all in f32. Workgroup
// (leaf, g) forms its leaf's normed row in LDS, then wave w scores id 4 g + w: lane l takes 8 consecutive k per
// 512-wide pass (one 8-byte q8 or 4-byte q4 load), the wave adds the lanes' sums — the ids in parallel, each a
// single round trip, instead of one id after another behind two barriers.
template <int BITS>
__global__ __launch_bounds__(256) void k_leaf_logits(int T, int H, int nIds, float eps, const uint16_t *__restrict__ X,
                                                     const uint32_t *__restrict__ leaves, const uint16_t *__restrict__ W,
                                                     const uint32_t *__restrict__ ids, int V, const uint8_t *__restrict__ codes,
                                                     const uint16_t *__restrict__ scales, float *__restrict__ out) {
  extern __shared__ float normed[];
  __shared__ float red[4];
  const int leaf = blockIdx.x, wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  uint32_t r = leaves[leaf];
  if (r >= (uint32_t)T) r = T - 1;
  const size_t row = (size_t)r * H;
  float ss = 0.f;
  for (int k = threadIdx.x; k < H; k += 256) {
    const float v = hf(X[row + k]);
    ss += v * v;
  }
  const float inv = 1.0f / sqrtf(block_sum256(ss, red) / (float)H + eps);
  for (int k = threadIdx.x; k < H; k += 256) normed[k] = hf(X[row + k]) * inv * hf(W[k]);
  __syncthreads();
  const int j = blockIdx.y * 4 + wave;
  if (j >= nIds) return;
  uint32_t id = ids[(size_t)leaf * nIds + j];
  if (id >= (uint32_t)V) id = V - 1;
  const float zp = BITS == 8 ? 128.f : 8.f;
  float dot = 0.f;
  for (int k0 = lane * 8; k0 < H; k0 += WAVE * 8) {
    const float sc = hf(scales[(size_t)id * (H / 32) + k0 / 32]);
    if constexpr (BITS == 8) {
      const uint2 raw = *(const uint2 *)(codes + (size_t)id * H + k0);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t c = ((q < 4 ? raw.x : raw.y) >> (8 * (q & 3))) & 255u;
        dot += normed[k0 + q] * ((float)c - zp) * sc;
      }
    } else {
      const uint32_t raw = *(const uint32_t *)(codes + (size_t)id * (H / 2) + k0 / 2);
#pragma unroll
      for (int q = 0; q < 8; ++q) dot += normed[k0 + q] * ((float)((raw >> (4 * q)) & 15u) - zp) * sc;
    }
  }
  dot = wave_sum(dot);
  if (lane == 0) out[(size_t)leaf * nIds + j] = dot;
}

extern "C" int dj_leaf_logits(dj_rec *rec, int T, int L, int H, int nIds, float eps, const uint16_t *X, const uint32_t *leaves,
                              const uint16_t *W, const uint32_t *ids, const dj_weight *e, float *out) {
  DJ_REQUIRE(e && e->layout == DJ_W_PLAIN && e->K == H, "decision.js: leaf_logits needs the plain embedding [V, %d]", H);
  DJ_REQUIRE(X && leaves && W && ids && out && T > 0 && L >= 0 && nIds >= 0 && H % 32 == 0 && H <= 16384,
             "decision.js: leaf_logits: bad arguments");
  DJ_OP_BEGIN(rec, "leaf_logits");
  if (L > 0 && nIds > 0) {
    const size_t sh = (size_t)H * 4;
    if (e->bits == 8)
      k_leaf_logits<8><<<dim3(L, dj_cdiv(nIds, 4)), 256, sh, rec->ctx->stream>>>(T, H, nIds, eps, X, leaves, W, ids, e->N, e->codes,
                                                         (const uint16_t *)e->scales, out);
    else
      k_leaf_logits<4><<<dim3(L, dj_cdiv(nIds, 4)), 256, sh, rec->ctx->stream>>>(T, H, nIds, eps, X, leaves, W, ids, e->N, e->codes,
                                                         (const uint16_t *)e->scales, out);
  }
  return dj_op_end(rec, "leaf_logits");
}

// ---------------------------------------------------------------- readout (d3-kernels.ts:242-260)
__global__ __launch_bounds__(256) void k_readout(int T, int H, const uint16_t *__restrict__ X, const float *__restrict__ R,
                                                 int codes, const uint32_t *__restrict__ pairs, float *__restrict__ out) {
  __shared__ float red[4];
  const int k = blockIdx.x;
  uint32_t r = pairs[2 * k], c = pairs[2 * k + 1];
  if (r >= (uint32_t)T) r = T - 1;
  if (c >= (uint32_t)codes) c = codes - 1;
  float s = 0.f;
  for (int d = threadIdx.x; d < H; d += 256) s += hf(X[(size_t)r * H + d]) * R[(size_t)c * H + d];
  s = block_sum256(s, red);
  if (threadIdx.x == 0) out[k] = s;
}

extern "C" int dj_readout(dj_rec *rec, int T, int P, int H, const uint16_t *X, const float *R, int codes, const uint32_t *pairs,
                          float *out) {
  DJ_REQUIRE(X && R && pairs && out && T > 0 && P >= 0 && H > 0 && codes > 0, "decision.js: readout: bad arguments");
  DJ_OP_BEGIN(rec, "readout");
  if (P > 0) k_readout<<<P, 256, 0, rec->ctx->stream>>>(T, H, X, R, codes, pairs, out);
  return dj_op_end(rec, "readout");
}

// ---------------------------------------------------------------- LFM2 short conv (kernels.ts:62-84)
// One lane per (token, 8 channels): the token's C chunk and, for each of its three taps, the tapped token's B
// and U chunks (16-byte loads of Z's [B | C | U] rows; consecutive lanes take consecutive chunks of one row),
// conv = w0 (B U)[tap0] + w1 (B U)[tap1] + w2 (B U)[tap2] in f32 (a tap < 0 reads zero), Y = f16(C conv).
// HBM-bound: at most 3 Z rows read and one H-wide row written per token.
__global__ __launch_bounds__(256) void k_short_conv(int T, int H, const uint16_t *__restrict__ Z,
                                                    const uint16_t *__restrict__ Wc, const int4 *__restrict__ taps,
                                                    uint16_t *__restrict__ Y) {
  const int chunks = H >> 3;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)T * chunks) return;
  const int t = (int)(i / chunks), c0 = (int)(i % chunks) * 8;
  const int4 tp = taps[t];
  const int tt[3] = {tp.x, tp.y, tp.z};
  // the chunk's 24 tap weights: Wc [H, 3] row-major, channels c0 .. c0 + 7
  h8 w8[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) w8[q] = *(const h8 *)(Wc + (size_t)c0 * 3 + 8 * q);
  float conv[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) conv[k] = 0.f;
  const size_t row = (size_t)3 * H;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int s = tt[j];
    if (s < 0 || s >= T) continue;  // no token there: that tap reads zero
    const h8 b = *(const h8 *)(Z + (size_t)s * row + c0);
    const h8 u = *(const h8 *)(Z + (size_t)s * row + 2 * H + c0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int wi = k * 3 + j;  // channel c0 + k, tap j
      const float w = (float)w8[wi >> 3][wi & 7];
      conv[k] += w * ((float)b[k] * (float)u[k]);
    }
  }
  const h8 c = *(const h8 *)(Z + (size_t)t * row + H + c0);
  h8 y;
#pragma unroll
  for (int k = 0; k < 8; ++k) y[k] = (_Float16)((float)c[k] * conv[k]);
  *(h8 *)(Y + (size_t)t * H + c0) = y;
}

extern "C" int dj_short_conv(dj_rec *rec, int T, int H, const uint16_t *Z, const uint16_t *w, const int32_t *taps,
                             uint16_t *Y) {
  DJ_REQUIRE(Z && w && taps && Y && T >= 0 && H > 0 && H % 8 == 0,
             "decision.js: short_conv: bad arguments (H %d must be a multiple of 8)", H);
  DJ_OP_BEGIN(rec, "short_conv");
  const long n = (long)T * (H / 8);
  if (n > 0) k_short_conv<<<(unsigned)dj_cdiv(n, 256), 256, 0, rec->ctx->stream>>>(T, H, Z, w, (const int4 *)taps, Y);
  return dj_op_end(rec, "short_conv");
}

// ---------------------------------------------------------------- mean pooling (eg2-kernels.ts:202-219)
// One workgroup per (sequence, 64 columns): lane = column, the 4 waves take every 4th token (8 loads in
// flight each), then wave 0 adds the 4 partial sums in wave order (deterministic) and divides.
__global__ __launch_bounds__(256) void k_mean_pool(int T, int H, const uint16_t *__restrict__ X, const uint32_t *__restrict__ seqs,
                                                   float *__restrict__ out) {
  __shared__ float red[3][64];
  const int s = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = blockIdx.y * 64 + lane;
  uint32_t a = seqs[2 * s], b = seqs[2 * s + 1];
  if (b > (uint32_t)T) b = T;
  if (a > b) a = b;
  float acc = 0.f;
  if (k < H) {
#pragma unroll 8
    for (uint32_t t = a + wave; t < b; t += 4) acc += hf(X[(size_t)t * H + k]);
  }
  if (wave > 0) red[wave - 1][lane] = acc;
  __syncthreads();
  if (wave == 0 && k < H) {
    for (int w = 0; w < 3; ++w) acc += red[w][lane];
    out[(size_t)s * H + k] = acc / (float)(b - a);
  }
}

void dj_launch_mean_pool(hipStream_t s, int T, int S, int H, const uint16_t *X, const uint32_t *seqs, float *out) {
  k_mean_pool<<<dim3(S, dj_cdiv(H, 64)), 256, 0, s>>>(T, H, X, seqs, out);
}

extern "C" int dj_mean_pool(dj_rec *rec, int T, int S, int H, const uint16_t *X, const uint32_t *seqs, float *out) {
  DJ_REQUIRE(X && seqs && out && T > 0 && S >= 0 && H > 0, "decision.js: mean_pool: bad arguments");
  DJ_OP_BEGIN(rec, "mean_pool");
  if (S > 0) dj_launch_mean_pool(rec->ctx->stream, T, S, H, X, seqs, out);
  return dj_op_end(rec, "mean_pool");
}

// ---------------------------------------------------------------- small f32 dense (pooled head)
// One wave per output column: lane l takes 4 consecutive k (one 4-byte q8 / 2-byte q4 code load, one scale,
// a float4 of each input row) every 256 k, rows in chunks of 16 kept in registers; lane partials are then
// added by a butterfly (fixed order: deterministic).
template <int BITS>
__global__ __launch_bounds__(256) void k_dense_f32(int M, int N, int K, const float *__restrict__ in, const uint8_t *__restrict__ codes,
                                                   const uint16_t *__restrict__ scales, float *__restrict__ out) {
  constexpr int MR = 16;
  const int n = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  if (n >= N) return;
  const float zp = BITS == 8 ? 128.f : 8.f;
  for (int m0 = 0; m0 < M; m0 += MR) {
    float acc[MR];
#pragma unroll
    for (int i = 0; i < MR; ++i) acc[i] = 0.f;
#pragma unroll 2
    for (int k = 4 * lane; k < K; k += 4 * WAVE) {
      uint32_t c4;
      if constexpr (BITS == 8) {
        c4 = *(const uint32_t *)(codes + (size_t)n * K + k);
      } else {
        const uint32_t p = *(const uint16_t *)(codes + (size_t)n * (K / 2) + k / 2);  // nibbles k..k+3, low first
        c4 = (p & 15u) | ((p >> 4 & 15u) << 8) | ((p >> 8 & 15u) << 16) | ((p >> 12 & 15u) << 24);
      }
      const float sc = hf(scales[(size_t)n * (K / 32) + k / 32]);
      float w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = ((float)((c4 >> (8 * j)) & 255u) - zp) * sc;
#pragma unroll
      for (int i = 0; i < MR; ++i)
        if (m0 + i < M) {
          const float4 x = *(const float4 *)(in + (size_t)(m0 + i) * K + k);
          acc[i] += x.x * w[0] + x.y * w[1] + x.z * w[2] + x.w * w[3];
        }
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      const float v = wave_sum(acc[i]);
      if (lane == 0 && m0 + i < M) out[(size_t)(m0 + i) * N + n] = v;
    }
  }
}

extern "C" int dj_dense_f32(dj_rec *rec, int M, const float *in, const dj_weight *w, float *out) {
  DJ_REQUIRE(w && w->layout == DJ_W_PLAIN, "decision.js: dense_f32 needs a plain weight");
  DJ_REQUIRE(w->K % 32 == 0, "decision.js: dense_f32: K = %d must be a multiple of 32", w->K);
  DJ_REQUIRE(in && out && M >= 0, "decision.js: dense_f32: bad arguments");
  DJ_OP_BEGIN(rec, "dense_f32");
  if (M > 0) {
    if (w->bits == 8)
      k_dense_f32<8><<<dj_cdiv(w->N, 4), 256, 0, rec->ctx->stream>>>(M, w->N, w->K, in, w->codes, (const uint16_t *)w->scales, out);
    else
      k_dense_f32<4><<<dj_cdiv(w->N, 4), 256, 0, rec->ctx->stream>>>(M, w->N, w->K, in, w->codes, (const uint16_t *)w->scales, out);
  }
  return dj_op_end(rec, "dense_f32");
}

// ---------------------------------------------------------------- copy (snapshots; a kernel, so it can be captured)
__global__ void k_copy(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src, size_t bytes) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i + 16 <= bytes) {
    *(uint4 *)(dst + i) = *(const uint4 *)(src + i);
  } else {
    for (size_t j = i; j < bytes; ++j) dst[j] = src[j];
  }
}

int dj_launch_copy(hipStream_t s, void *dst, const void *src, size_t bytes) {
  if (!bytes) return DJ_OK;
  DJ_REQUIRE(((uintptr_t)dst | (uintptr_t)src) % 16 == 0, "decision.js: snapshot buffers must be 16-byte aligned");
  k_copy<<<dj_cdiv((long)((bytes + 15) / 16), 256), 256, 0, s>>>((uint8_t *)dst, (const uint8_t *)src, bytes);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return dj_fail(DJ_EHIP, "decision.js: snapshot copy: %s", hipGetErrorString(e));
  return DJ_OK;
}
