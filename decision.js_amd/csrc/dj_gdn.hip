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

constexpr int C = 64;       // tokens per chunk
constexpr int DK = 128;     // key / value head dim
constexpr int NT = 512;     // threads: 128 rows x 4 lanes

__device__ __forceinline__ float hf(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
// SiLU on the hardware exp2 and reciprocal (about 1 f32 ulp each): for the conv outputs, which are rounded to
// f16 right after
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

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

// ---------------------------------------------------------------- the row-split form
// The same recurrence with the 128 state rows of a head split over RS = 4 workgroups of 32 rows (256 threads:
// 8 lanes per row, 16 k columns each): 4x the workgroups of the form above and half the multiply-adds per lane
// and token (k . q is formed once per token in the prep phase); the chunk's inputs are loaded with all threads,
// 16 bytes per load, while the previous chunk's recurrence runs, and the conv reads them from LDS. The gated
// RMSNorm needs a token's 128 outputs, so the scan writes them (f32, unrounded) to a workspace and k_gdn_norm
// finishes them. (16 lanes per row, twice the waves: 110 against ~60 us for the recurrence of 3 x 384 tokens x
// 16 heads, the lane reductions and register moves outweighing the shorter rows; MI355X.)
constexpr int RW = 32;             // state rows per workgroup
constexpr int RS = DK / RW;        // workgroups per (sequence, head)
constexpr int LPR = 8;             // lanes per row
constexpr int NT2 = RW * LPR;      // 256 threads
constexpr int XW = 2 * DK + RW;    // f16 inputs per token staged: q | k | this workgroup's v rows
constexpr int PPR = XW / 8;        // 16-byte pieces per staged row

__global__ __launch_bounds__(NT2) void k_gdn_scan(int T, int LH, int stride, const uint4 *__restrict__ spans,
                                                  const uint16_t *__restrict__ Z, const uint16_t *__restrict__ Wc,
                                                  const uint16_t *__restrict__ Alog, const uint16_t *__restrict__ dtb,
                                                  float *__restrict__ Ob) {
  constexpr int PIECES = (C + 3) * PPR;              // 16-byte pieces staged per chunk
  constexpr int PPT = (PIECES + NT2 - 1) / NT2;      // per thread
  __shared__ __attribute__((aligned(16))) uint16_t xin[(C + 3) * XW];  // sequence indices t0-3 .. t0+C-1
  __shared__ __attribute__((aligned(16))) float qs[C * DK];
  __shared__ __attribute__((aligned(16))) float ks[C * DK];
  __shared__ float vs[C * RW];   // v, then o
  __shared__ float4 gs[C];       // (decay, beta, k . q, -)
  const int tid = threadIdx.x;
  const int rs = blockIdx.x % RS, h = (blockIdx.x / RS) % LH;
  const uint4 sp = spans[blockIdx.x / (RS * LH)];
  const Span S{sp.x, sp.y & 0x7fffffffu, sp.z, sp.w, (sp.y >> 31) != 0};
  const uint32_t end = S.len();
  const int QK = LH * DK;
  const int row = tid / LPR, part = tid % LPR;
  f4 st[4] = {};  // k columns 4 part + 32 j .. +3, j = 0..3

  // conv roles: threads 0..255 a q or k channel; threads 0..15 also one of this workgroup's v channels
  const int qk_ch = (tid < DK ? 0 : QK) + h * DK + tid % DK;
  const int v_ch = 2 * QK + h * DK + rs * RW + (tid % RW);
  float wq[4], wv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    wq[j] = hf(Wc[(size_t)qk_ch * 4 + j]);
    wv[j] = hf(Wc[(size_t)v_ch * 4 + j]);
  }
  const float negA = -expf(hf(Alog[h])), dt = hf(dtb[h]);

  // the staged inputs of the chunk at t0: rows t0-3 .. t0+C-1, PPR 16-byte pieces each (q and k of this head: 32,
  // this workgroup's v rows: 4); zero before the sequence and past its end; and the raw gate inputs (b, a)
  // The loads are unconditional (a piece with no token reads row 0 and is zeroed when staged), so they stay in
  // flight until stage() or the gates need them.
  uint4 pre[PPT];
  uint32_t ok = 0;  // bit q: piece q holds a token's values
  uint16_t pb = 0, pa = 0;
  bool gok = false;
  auto fetch = [&](uint32_t t0) {
    ok = 0;
#pragma unroll
    for (int q = 0; q < PPT; ++q) {
      const int i = tid + q * NT2;
      const int lr = i / PPR, pc = i % PPR;
      const long v = (long)t0 + lr - 3;
      const uint32_t r = v >= 0 && v < (long)end ? S.row((uint32_t)v) : 0xffffffffu;
      const bool good = i < PIECES && r < (uint32_t)T;
      ok |= (uint32_t)good << q;
      const uint16_t *zr = Z + (size_t)(good ? r : 0) * stride;
      const int col = pc < 16 ? h * DK + pc * 8 : pc < 32 ? QK + h * DK + (pc - 16) * 8 : 2 * QK + h * DK + rs * RW + (pc - 32) * 8;
      pre[q] = *(const uint4 *)(zr + (i < PIECES ? col : 0));
    }
    const uint32_t r = t0 + (tid % C) < end ? S.row(t0 + tid % C) : 0xffffffffu;
    gok = tid < C && r < (uint32_t)T;
    const uint16_t *zr = Z + (size_t)(gok ? r : 0) * stride + 4 * QK;
    pb = zr[h];
    pa = zr[LH + h];
  };
  auto stage = [&]() {
#pragma unroll
    for (int q = 0; q < PPT; ++q) {
      const int i = tid + q * NT2;
      if (i < PIECES) *(uint4 *)(xin + (i / PPR) * XW + (i % PPR) * 8) = (ok >> q) & 1 ? pre[q] : uint4{0u, 0u, 0u, 0u};
    }
  };
  fetch(0);
  stage();

  for (uint32_t t0 = 0; t0 < end; t0 += C) {
    const int n = (int)min((uint32_t)C, end - t0);
    if (tid < n) {  // the gates of token t0 + tid
      const float b = gok ? hf(pb) : 0.f, a = (gok ? hf(pa) : 0.f) + dt;
      const float spl = a > 20.f ? a : logf(1.0f + expf(a));
      gs[tid] = make_float4(expf(negA * spl), 1.0f / (1.0f + expf(-b)), 0.f, 0.f);
    }
    __syncthreads();
    // 1. conv + SiLU, rounded to f16: a thread per q / k channel over the chunk's tokens, the v channels' (token,
    //    channel) pairs spread over all threads
    {
      float *dst = (tid < DK ? qs : ks) + tid % DK;
#pragma unroll 8
      for (int c = 0; c < n; ++c) {
        const uint16_t *x = xin + c * XW + tid;
        const float y = wq[0] * hf(x[0]) + wq[1] * hf(x[XW]) + wq[2] * hf(x[2 * XW]) + wq[3] * hf(x[3 * XW]);
        dst[c * DK] = (float)(_Float16)silu_fast(y);
      }
      for (int i = tid; i < n * RW; i += NT2) {
        const int c = i / RW, ch = i % RW;
        const uint16_t *x = xin + c * XW + 2 * DK + ch;
        const float w0 = __shfl(wv[0], ch, 64), w1 = __shfl(wv[1], ch, 64), w2 = __shfl(wv[2], ch, 64),
                    w3 = __shfl(wv[3], ch, 64);
        const float y = w0 * hf(x[0]) + w1 * hf(x[XW]) + w2 * hf(x[2 * XW]) + w3 * hf(x[3 * XW]);
        vs[c * RW + ch] = (float)(_Float16)silu_fast(y);
      }
    }
    __syncthreads();
    // q and k L2 norms and k . q: 16 lanes per token (8 of its q and k values each), 16 tokens at a time
    for (int c = tid / 16; c < n; c += NT2 / 16) {
      const int l = tid % 16;
      f4 *q = (f4 *)(qs + c * DK), *k = (f4 *)(ks + c * DK);
      const f4 qa = q[l], qb = q[l + 16], ka = k[l], kb = k[l + 16];
      float sq = 0.f, sk = 0.f, qk = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sq += qa[e] * qa[e] + qb[e] * qb[e];
        sk += ka[e] * ka[e] + kb[e] * kb[e];
        qk += qa[e] * ka[e] + qb[e] * kb[e];
      }
      sq = group_sum<16>(sq);
      sk = group_sum<16>(sk);
      qk = group_sum<16>(qk);
      const float iq = rsqrtf(sq + 1e-6f) * 0.08838834764831845f, ik = rsqrtf(sk + 1e-6f);
      q[l] = qa * iq;
      q[l + 16] = qb * iq;
      k[l] = ka * ik;
      k[l + 16] = kb * ik;
      if (l == 0) gs[c].z = qk * iq * ik;
    }
    __syncthreads();
    // the next chunk's inputs load while the recurrence runs (xin is not read again in this chunk)
    const bool more = t0 + C < end;
    if (more) fetch(t0 + C);
    // 2. the delta rule on this workgroup's 32 rows, two tokens per step with their LDS operands read a token
    //    ahead into alternating register sets
    {
      struct Tok {
        f4 k[4], q[4];
        float4 g;
        float v;
      };
      auto ld = [&](int c, Tok &t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          t.k[j] = *(const f4 *)(ks + c * DK + 4 * part + 32 * j);
          t.q[j] = *(const f4 *)(qs + c * DK + 4 * part + 32 * j);
        }
        t.g = gs[c];
        t.v = vs[c * RW + row];
      };
      auto step = [&](int c, const Tok &t) {
        // four partial sums each (short dependency chains; the next token waits on this one's sums)
        float r4[4] = {}, p4[4] = {};
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            r4[e] += st[j][e] * t.k[j][e];
            p4[e] += st[j][e] * t.q[j][e];
          }
        float r = (r4[0] + r4[1]) + (r4[2] + r4[3]), p = (p4[0] + p4[1]) + (p4[2] + p4[3]);
        r = group_sum<LPR>(r);
        p = group_sum<LPR>(p);
        const float delta = (t.v - t.g.x * r) * t.g.y;
        const float o = t.g.x * p + t.g.z * delta;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) st[j][e] = st[j][e] * t.g.x + t.k[j][e] * delta;
        if (part == 0) vs[c * RW + row] = o;  // token c's v was read (a token ahead) by the row's lanes
      };
      // the look-ahead loads are unconditional (past the chunk's end they reread its last token), so the
      // compiler's wait before a step counts only the older loads
      Tok A, B;
      ld(0, A);
      for (int c = 0; c < n; c += 2) {
        ld(min(c + 1, n - 1), B);
        step(c, A);
        if (c + 1 >= n) break;
        ld(min(c + 2, n - 1), A);
        step(c + 1, B);
      }
    }
    if (more) stage();
    __syncthreads();
    // 3. the outputs, unnormalised, to the workspace
    for (int i = tid; i < n * RW; i += NT2) {
      const int c = i / RW, k = i % RW;
      const uint32_t v = t0 + c;
      const uint32_t r = S.row(v);
      if ((v < S.alen && !S.write_a) || r >= (uint32_t)T) continue;
      Ob[((size_t)r * LH + h) * DK + rs * RW + k] = vs[c * RW + k];
    }
  }
}

// The gated RMSNorm of the scan's outputs: one wave per (token, head).
__global__ __launch_bounds__(256) void k_gdn_norm(int T, int LH, int stride, const uint16_t *__restrict__ Z,
                                                  const float *__restrict__ Ob, const uint16_t *__restrict__ gw, float eps,
                                                  uint16_t *__restrict__ Y) {
  const long pair = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (pair >= (long)T * LH) return;
  const int r = (int)(pair / LH), h = (int)(pair % LH);
  const float *o = Ob + (size_t)pair * DK;
  const float a = o[lane], b = o[lane + 64];
  const float inv = 1.0f / sqrtf(group_sum<64>(a * a + b * b) / (float)DK + eps);
  const int QK = LH * DK;
  const uint16_t *z = Z + (size_t)r * stride + 3 * QK + h * DK;
  uint16_t *y = Y + (size_t)r * QK + h * DK;
  y[lane] = __builtin_bit_cast(uint16_t, (_Float16)(a * inv * hf(gw[lane]) * silu(hf(z[lane]))));
  y[lane + 64] = __builtin_bit_cast(uint16_t, (_Float16)(b * inv * hf(gw[lane + 64]) * silu(hf(z[lane + 64]))));
}

}  // namespace

extern "C" int dj_gdn(dj_rec *rec, int T, int nspans, const uint32_t *spans, int LH, int stride, const uint16_t *Z,
                      const uint16_t *conv_w, const uint16_t *A_log, const uint16_t *dt_bias, const uint16_t *gnorm,
                      float eps, uint16_t *Y) {
  DJ_REQUIRE(Z && spans && conv_w && A_log && dt_bias && gnorm && Y && T >= 0 && nspans >= 0 && LH > 0,
             "decision.js: gdn: bad arguments");
  DJ_REQUIRE(stride >= 4 * LH * DK + 2 * LH, "decision.js: gdn: in-projection rows of %d values hold fewer than "
             "q | k | v | z | b | a (%d)", stride, 4 * LH * DK + 2 * LH);
  DJ_REQUIRE((long)nspans * LH * 8 < (1L << 31), "decision.js: gdn: %d sequences x %d heads is too large", nspans, LH);
  DJ_REQUIRE(((uintptr_t)Z & 15) == 0 && stride % 8 == 0, "decision.js: gdn: Z must be 16-byte aligned with rows of a "
             "multiple of 8 values (stride %d)", stride);
  DJ_OP_BEGIN(rec, "gdn");
  if (nspans > 0 && T > 0) {
    // the row-split scan (8x the workgroups) when its f32 outputs fit the context workspace; else one workgroup
    // per (sequence, head) with the norm inside. DJ_GDN_FORM=1 forces the latter (tests, sweeps).
    float *ws = nullptr;
    const char *form = getenv("DJ_GDN_FORM");
    const bool split = !(form && atoi(form) == 1) && dj_gemm_workspace(rec->ctx, (size_t)T * LH * DK, &ws) == DJ_OK;
    hipStream_t s = rec->ctx->stream;
    if (split) {
      k_gdn_scan<<<(unsigned)(nspans * LH * RS), NT2, 0, s>>>(T, LH, stride, (const uint4 *)spans, Z, conv_w, A_log,
                                                             dt_bias, ws);
      k_gdn_norm<<<(unsigned)dj_cdiv((long)T * LH, 4), 256, 0, s>>>(T, LH, stride, Z, ws, gnorm, eps, Y);
    } else {
      k_gdn<<<(unsigned)(nspans * LH), NT, 0, s>>>(T, LH, stride, (const uint4 *)spans, Z, conv_w, A_log, dt_bias, gnorm,
                                                   eps, Y);
    }
  }
  return dj_op_end(rec, "gdn");
}
