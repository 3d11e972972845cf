/* oracle.c — plain-C restatement of the integer/byte parts of decision.js's scoring path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (ctypes) to cross-check the numpy restatement in oracle/ref.py
 * and the GPU kernels. It is not part of the product and is never linked into libdj.so.
 *
 *   o_f32_to_f16    IEEE binary32 -> binary16, round to nearest even (what WGSL's f16() and numpy do)
 *   o_f16_to_f32    binary16 -> binary32 (gpu.ts:285-292, f16ToF32)
 *   o_dequant       q8/q4 codes + f16 scales -> f16 weights: f16(f16(code) - f16(zp)) * scale
 *                   (kernels.ts:20, 296, 541; the f16 multiply's single RNE rounding)
 *   o_quantize8     export_common.py:90-97 (f32 division, round half to even, clamp +-127, zp 128)
 *   o_pack_forest   d1-3b-engine.ts:46-72 (ids, pos, meta, leaves)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint16_t o_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) return (uint16_t)(sign | (absx > 0x7f800000u ? 0x7e00u : 0x7c00u)); /* NaN / inf */
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
  if (absx < 0x33000000u) return (uint16_t)sign;               /* < 2^-25: rounds to 0 */
  const int e = (int)(absx >> 23) - 127;
  uint32_t mant = (absx & 0x7fffffu) | 0x800000u; /* 24 significant bits */
  int shift;                                      /* bits to drop from the 24-bit significand */
  uint32_t base;
  if (e < -14) { /* subnormal half: value = m * 2^-24 */
    shift = 13 + (-14 - e);
    base = 0;
  } else {
    shift = 13;
    base = (uint32_t)(e + 15) << 10;
    mant &= 0x7fffffu; /* the implicit bit is carried by the exponent field */
    mant |= 0;
  }
  uint32_t q, rem, half;
  if (e < -14) {
    q = mant >> shift;
    rem = mant & ((1u << shift) - 1);
    half = 1u << (shift - 1);
  } else {
    q = mant >> 13;
    rem = mant & 0x1fffu;
    half = 0x1000u;
  }
  uint32_t h = base + q;
  if (rem > half || (rem == half && (q & 1u))) h += 1; /* a carry into the exponent is correct rounding */
  return (uint16_t)(sign | h);
}

float o_f16_to_f32(uint16_t h) {
  const int s = (h & 0x8000) ? -1 : 1, e = (h >> 10) & 31, f = h & 1023;
  if (e == 0) return s * ldexpf((float)f, -24);
  if (e == 31) return f ? NAN : s * INFINITY;
  return s * ldexpf(1.0f + f / 1024.0f, e - 15);
}

/* out[n * K + k] = f16 weight; codes: bits 8 -> [N, K] bytes, bits 4 -> [N, K/2] bytes (low nibble first). */
void o_dequant(const uint8_t *codes, const uint16_t *scales, int N, int K, int bits, uint16_t *out) {
  const float zp = bits == 8 ? 128.0f : 8.0f;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k) {
      uint32_t c;
      if (bits == 8)
        c = codes[(size_t)n * K + k];
      else
        c = (codes[(size_t)n * (K / 2) + k / 2] >> ((k & 1) * 4)) & 15u;
      const float q = (float)c - zp;                         /* exact: f16(code) - f16(zp) */
      const float s = o_f16_to_f32(scales[(size_t)n * (K / 32) + k / 32]);
      out[(size_t)n * K + k] = o_f32_to_f16(q * s);          /* the f32 product of two f16 values is exact */
    }
}

void o_quantize8(const float *w, int N, int K, uint8_t *codes, uint16_t *scales) {
  for (int n = 0; n < N; ++n)
    for (int g = 0; g < K / 32; ++g) {
      const float *b = w + (size_t)n * K + g * 32;
      float amax = 0.0f;
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(b[i]));
      uint16_t sh = o_f32_to_f16(amax / 127.0f);
      float s = o_f16_to_f32(sh);
      if (s == 0.0f) { s = 1.0f; sh = 0x3c00; } /* an all-zero block: scale 1, codes 0 */
      scales[(size_t)n * (K / 32) + g] = sh;
      for (int i = 0; i < 32; ++i) {
        float q = nearbyintf(b[i] / s); /* default rounding mode: half to even, as torch.round */
        if (q > 127.0f) q = 127.0f;
        if (q < -127.0f) q = -127.0f;
        codes[(size_t)n * K + g * 32 + i] = (uint8_t)(int)(q + 128.0f);
      }
    }
}

/* trees: ntrees entries of (trunk length, branch count); tok: every token id, trees in order, each tree's
 * trunk then its branches; blen: every branch length in order. Outputs sized by the caller. Returns T. */
int o_pack_forest(int ntrees, const int32_t *trees, const uint32_t *tok, const int32_t *blen, uint32_t *ids,
                  int32_t *pos, int32_t *meta, uint32_t *leaves, int *L) {
  int t = 0, bi = 0, nl = 0;
  const uint32_t *src = tok;
  for (int r = 0; r < ntrees; ++r) {
    const int p = trees[2 * r], nb = trees[2 * r + 1];
    int total = p;
    for (int b = 0; b < nb; ++b) total += blen[bi + b];
    const int start = t;
    for (int i = 0; i < p; ++i, ++t) {
      ids[t] = *src++;
      pos[t] = i;
      meta[4 * t] = start; meta[4 * t + 1] = start + total; meta[4 * t + 2] = -1; meta[4 * t + 3] = i;
    }
    for (int b = 0; b < nb; ++b) {
      const int n = blen[bi++];
      for (int o = 0; o < n; ++o, ++t) {
        ids[t] = *src++;
        pos[t] = p + o;
        meta[4 * t] = start; meta[4 * t + 1] = start + total; meta[4 * t + 2] = b; meta[4 * t + 3] = p + o;
      }
      leaves[nl++] = (uint32_t)(t - 1);
    }
  }
  *L = nl;
  return t;
}
