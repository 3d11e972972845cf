// The runtime half of libdj.so: device context, buffers, quantized weights and their MFMA repack,
// the forward recorder (optionally captured into a cached HIP graph), timers and per-kernel profiling.
// It stands where src/gpu.ts stands in the reference (requestDevice, loadWeights, GpuEngine, recorder).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <algorithm>
#include "dj_internal.h"

// ---------------------------------------------------------------- errors (gpu.ts:260, d1.ts:68)

static thread_local std::string g_err;

int dj_fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

extern "C" const char *dj_last_error(void) { return g_err.c_str(); }
extern "C" int dj_abi_version(void) { return DJ_ABI_VERSION; }

// ---------------------------------------------------------------- device

extern "C" int dj_init(int ordinal, dj_ctx **out) {
  DJ_REQUIRE(out, "decision.js: dj_init: null output");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return dj_fail(DJ_EHIP, "decision.js: no HIP device is available (%s)", e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  DJ_REQUIRE(ordinal >= 0 && ordinal < n, "decision.js: device %d out of range (%d devices)", ordinal, n);
  DJ_HIP(hipSetDevice(ordinal));
  hipDeviceProp_t p;
  DJ_HIP(hipGetDeviceProperties(&p, ordinal));
  dj_ctx *c = new dj_ctx();
  c->device = ordinal;
  c->cus = p.multiProcessorCount;
  // default priority only: streams of other priorities have hung on these boxes
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return dj_fail(DJ_EHIP, "decision.js: hipStreamCreate failed");
  }
  DJ_HIP(hipEventCreate(&c->t0));
  DJ_HIP(hipEventCreate(&c->t1));
  // this device's address of the static attention scratch (dj_attention_noalloc), taken with the device current
  if (int st = dj_attn_scratch_init(c)) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return st;
  }
  // DJ_FAULT_INJECT=<op>[:<n>]: the op fails (before launching anything) every time, or its next n times
  if (const char *f = getenv("DJ_FAULT_INJECT")) {
    c->fault_op = f;
    const size_t colon = c->fault_op.find(':');
    if (colon != std::string::npos) {
      c->fault_left = atol(c->fault_op.c_str() + colon + 1);
      c->fault_op.resize(colon);
    }
  }
  // split-K / split-KV workspace: 64 MiB of f32 partials (every slice is written before it is read)
  const size_t ws_floats = (size_t)16 << 20;
  if (hipMalloc((void **)&c->gemm_ws, ws_floats * 4) == hipSuccess) c->gemm_ws_floats = ws_floats;
  *out = c;
  return DJ_OK;
}

int dj_gemm_workspace(dj_ctx *c, size_t need_floats, float **ws) {
  if (!c->gemm_ws || need_floats > c->gemm_ws_floats) return DJ_ENOMEM;
  *ws = c->gemm_ws;
  return DJ_OK;
}

extern "C" int dj_device_info(dj_ctx *ctx, char *name, size_t cap, int *cus, size_t *total) {
  DJ_REQUIRE(ctx, "decision.js: null context");
  hipDeviceProp_t p;
  DJ_HIP(hipGetDeviceProperties(&p, ctx->device));
  if (name && cap) snprintf(name, cap, "%s", p.gcnArchName);
  if (cus) *cus = p.multiProcessorCount;
  if (total) *total = p.totalGlobalMem;
  return DJ_OK;
}

static void free_graph(dj_graph_entry &g) {
  if (g.exec) (void)hipGraphExecDestroy(g.exec);
  for (void *p : g.staging) (void)hipFree(p);
  g.exec = nullptr;
  g.staging.clear();
}

static void free_graphs(dj_ctx *c) {
  for (auto &kv : c->graphs) free_graph(kv.second);
  c->graphs.clear();
}

// Most graphs a context keeps (DJ_GRAPH_CAP, default 64): a long-running host that sees many shapes or many
// shared states holds a bounded number of graph execs and snapshot staging buffers.
static size_t graph_cap() {
  const char *e = getenv("DJ_GRAPH_CAP");
  const long n = e ? atol(e) : 64;
  return n >= 1 ? (size_t)n : 1;
}

// Makes room for one more graph: evicts least recently used entries until fewer than the cap remain. Called
// with the stream drained (every forward waits for its work in dj_rec_finish), so no evicted exec is running.
static void evict_graphs(dj_ctx *c, uint64_t keep) {
  const size_t cap = graph_cap();
  while (c->graphs.size() >= cap) {
    auto victim = c->graphs.end();
    for (auto it = c->graphs.begin(); it != c->graphs.end(); ++it)
      if (it->first != keep && (victim == c->graphs.end() || it->second.last_use < victim->second.last_use)) victim = it;
    if (victim == c->graphs.end()) break;
    free_graph(victim->second);
    c->graphs.erase(victim);
  }
}

extern "C" int dj_destroy(dj_ctx *c) {
  if (!c) return DJ_OK;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  free_graphs(c);
  for (dj_weight *w : c->weights) {
    (void)hipFree(w->codes);
    (void)hipFree(w->scales);
    delete w;
  }
  for (auto &kv : c->buffers) (void)hipFree(kv.first);
  if (c->gemm_ws) (void)hipFree(c->gemm_ws);
  if (c->pinned) (void)hipHostFree(c->pinned);
  for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
  (void)hipEventDestroy(c->t0);
  (void)hipEventDestroy(c->t1);
  (void)hipStreamDestroy(c->stream);
  delete c;
  return DJ_OK;
}

// ---------------------------------------------------------------- buffers

extern "C" int dj_buf_alloc(dj_ctx *c, size_t bytes, void **dev) {
  DJ_REQUIRE(c && dev, "decision.js: dj_buf_alloc: null argument");
  size_t n = std::max<size_t>(256, (bytes + 255) & ~(size_t)255);
  void *p = nullptr;
  if (hipMalloc(&p, n) != hipSuccess)
    return dj_fail(DJ_ENOMEM, "decision.js: the GPU could not allocate %.1f MB", n / 1e6);
  c->buffers[p] = n;
  *dev = p;
  return DJ_OK;
}

extern "C" int dj_buf_free(dj_ctx *c, void *dev) {
  DJ_REQUIRE(c, "decision.js: null context");
  if (!dev) return DJ_OK;
  auto it = c->buffers.find(dev);
  DJ_REQUIRE(it != c->buffers.end(), "decision.js: dj_buf_free: %p is not a buffer of this context", dev);
  if (int st = dj_settle(c)) return st;
  DJ_HIP(hipStreamSynchronize(c->stream));
  DJ_HIP(hipFree(dev));
  c->buffers.erase(it);
  return DJ_OK;
}

extern "C" int dj_buf_write(dj_ctx *c, void *dev, const void *host, size_t bytes) {
  DJ_REQUIRE(c && (dev || !bytes) && (host || !bytes), "decision.js: dj_buf_write: null argument");
  DJ_REQUIRE(!c->active || !c->active->capturing, "decision.js: dj_buf_write while a graph is captured");
  if (!bytes) return DJ_OK;
  if (int st = dj_settle(c)) return st;
  DJ_HIP(hipStreamSynchronize(c->stream));
  DJ_HIP(hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice));
  return DJ_OK;
}

extern "C" int dj_buf_read(dj_ctx *c, void *host, const void *dev, size_t bytes) {
  DJ_REQUIRE(c && (dev || !bytes) && (host || !bytes), "decision.js: dj_buf_read: null argument");
  DJ_REQUIRE(!c->active || !c->active->capturing, "decision.js: dj_buf_read while a graph is captured");
  if (!bytes) return DJ_OK;
  if (int st = dj_settle(c)) return st;
  DJ_HIP(hipStreamSynchronize(c->stream));
  DJ_HIP(hipMemcpy(host, dev, bytes, hipMemcpyDeviceToHost));
  return DJ_OK;
}

extern "C" int dj_buf_copy(dj_ctx *c, void *dst, const void *src, size_t bytes) {
  DJ_REQUIRE(c && (dst || !bytes) && (src || !bytes), "decision.js: dj_buf_copy: null argument");
  if (int st = dj_settle(c)) return st;
  return dj_launch_copy(c->stream, dst, src, bytes);
}

extern "C" int dj_upload(dj_ctx *c, void *dev, const void *host, size_t bytes) {
  DJ_REQUIRE(c && (dev || !bytes) && (host || !bytes), "decision.js: dj_upload: null argument");
  DJ_REQUIRE(!c->active || !c->active->capturing,
             "decision.js: dj_upload while a graph is captured (upload before dj_rec_begin)");
  if (!bytes) return DJ_OK;
  if (int st = dj_settle(c)) return st;
  size_t need = (bytes + 255) & ~(size_t)255;
  if (c->pinned_used + need > c->pinned_cap) {
    DJ_HIP(hipStreamSynchronize(c->stream));  // every earlier upload has landed: the arena is free again
    c->pinned_used = 0;
    if (need > c->pinned_cap) {
      if (c->pinned) DJ_HIP(hipHostFree(c->pinned));
      c->pinned = nullptr;
      size_t cap = std::max<size_t>(need, 4 << 20);
      if (hipHostMalloc((void **)&c->pinned, cap, hipHostMallocDefault) != hipSuccess) {
        c->pinned_cap = 0;
        return dj_fail(DJ_ENOMEM, "decision.js: pinned staging of %zu bytes failed", cap);
      }
      c->pinned_cap = cap;
    }
  }
  uint8_t *stage = c->pinned + c->pinned_used;
  memcpy(stage, host, bytes);
  c->pinned_used += need;
  DJ_HIP(hipMemcpyAsync(dev, stage, bytes, hipMemcpyHostToDevice, c->stream));
  return DJ_OK;
}

// ---------------------------------------------------------------- weights

// MFMA block layout (the B operand of v_mfma_f32_16x16x32_f16, two k-steps of 32 per block):
// block (nb, kb) covers rows 16nb..16nb+15 and k 64kb..64kb+63. Lane l (n = l % 16, g = l / 16) owns,
// for k-step s in {0, 1}, the 8 codes k = 64kb + 32s + 8g + j (j < 8).
//  q8: 1024 bytes per block, lane l at byte 16l: [s0 j0..7][s1 j0..7], one code per byte.
//  q4:  512 bytes per block, lane l at byte 8l: one u32 per k-step; code j at bits 4(j/2) + 16(j%2)
//       (so ((w >> 4i) & 0x000F000F) is the f16 pair (j = 2i, 2i+1) once or'ed with 0x6400).
// Scales: block (nb, kb) holds 16 u32, lane l % 16 reads (scale[n][2kb] | scale[n][2kb+1] << 16).
// DJ_W_DIRECT: 2048 bytes per block, lane l at byte 32l: the 16 dequantized f16 weights of the same k
// positions ([s0 j0..7][s1 j0..7]); no scales.
// DJ_W_MFMA_GLU: physical row block p maps to w1 block p/2 (p even) or w3 block p/2 (p odd).
static inline int src_row_block(int p, int N, int layout) {
  if ((layout & ~DJ_W_DIRECT) != DJ_W_MFMA_GLU) return p;
  int half = N / 32;  // row blocks per half
  return (p & 1) ? half + (p >> 1) : (p >> 1);
}

// IEEE binary32 -> binary16, round to nearest even (the f16 conversions of the GPU and of numpy).
static uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (a < 0x33000000u) return (uint16_t)sign;
  const int e = (int)(a >> 23) - 127;
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const int shift = e < -14 ? -1 - e : 13;  // significand bits dropped
  const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
  uint32_t h = e < -14 ? q : (((uint32_t)(e + 15) << 10) + (q & 0x3ffu));
  if (rem > half || (rem == half && (q & 1u))) h += 1;
  return (uint16_t)(sign | h);
}

static float f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31, f = h & 1023;
  float v;
  if (e == 0) {
    v = ldexpf((float)f, -24);
  } else if (e == 31) {
    v = f ? NAN : INFINITY;
  } else {
    v = ldexpf((float)(f | 1024), (int)e - 25);
  }
  uint32_t x;
  memcpy(&x, &v, 4);
  x |= s;
  memcpy(&v, &x, 4);
  return v;
}

static int repack_mfma(const uint8_t *codes, const uint16_t *scales, int N, int K, int bits, int layout,
                       std::vector<uint8_t> &oc, std::vector<uint32_t> &os) {
  const int NB = N / 16, KB = K / 64, G = K / 32;
  const bool direct = (layout & DJ_W_DIRECT) != 0;
  const size_t blk = direct ? 2048 : bits == 8 ? 1024 : 512;
  oc.assign((size_t)NB * KB * blk, 0);
  os.assign(direct ? 16 : (size_t)NB * KB * 16, 0);
  const size_t row_bytes = (size_t)K * bits / 8;
  const float zp = bits == 8 ? 128.0f : 8.0f;
  for (int p = 0; p < NB; ++p) {
    const int sb = src_row_block(p, N, layout);
    for (int kb = 0; kb < KB; ++kb) {
      uint8_t *dst = oc.data() + ((size_t)p * KB + kb) * blk;
      for (int l = 0; l < 64; ++l) {
        const int n = sb * 16 + (l & 15), g = l >> 4;
        const uint8_t *row = codes + (size_t)n * row_bytes;
        for (int s = 0; s < 2; ++s) {
          const int k0 = kb * 64 + s * 32 + g * 8;
          if (direct) {
            // (f16(code) - f16(zp)) * scale, rounded once: exact f32 product of two f16 values, then RNE
            const float sc = f16_to_f32(scales[(size_t)n * G + k0 / 32]);
            uint16_t hv[8];
            for (int j = 0; j < 8; ++j) {
              const int k = k0 + j;
              const uint32_t c = bits == 8 ? row[k] : (row[k >> 1] >> ((k & 1) * 4)) & 15u;
              hv[j] = f32_to_f16(((float)c - zp) * sc);
            }
            memcpy(dst + l * 32 + s * 16, hv, 16);
          } else if (bits == 8) {
            memcpy(dst + l * 16 + s * 8, row + k0, 8);
          } else {
            uint32_t w = 0;
            for (int j = 0; j < 8; ++j) {
              const int k = k0 + j;
              const uint32_t c = (row[k >> 1] >> ((k & 1) * 4)) & 15u;
              w |= c << (4 * (j >> 1) + 16 * (j & 1));
            }
            memcpy(dst + l * 8 + s * 4, &w, 4);
          }
        }
      }
      for (int i = 0; i < 16 && !direct; ++i) {
        const int n = sb * 16 + i;
        os[((size_t)p * KB + kb) * 16 + i] =
            (uint32_t)scales[(size_t)n * G + 2 * kb] | ((uint32_t)scales[(size_t)n * G + 2 * kb + 1] << 16);
      }
    }
  }
  return DJ_OK;
}

extern "C" int dj_weight_q(dj_ctx *c, const void *codes, const void *scales, int N, int K, int bits, int layout,
                           dj_weight **out) {
  DJ_REQUIRE(c && codes && scales && out, "decision.js: dj_weight_q: null argument");
  DJ_REQUIRE(bits == 8 || bits == 4, "decision.js: weights must be q8 or q4, got %d bits", bits);
  DJ_REQUIRE(N > 0 && K > 0 && K % 32 == 0, "decision.js: weight [%d, %d]: K must be a multiple of 32", N, K);
  const int base = layout & ~DJ_W_DIRECT;
  DJ_REQUIRE(base >= DJ_W_PLAIN && base <= DJ_W_MFMA_GLU && (base != DJ_W_PLAIN || layout == DJ_W_PLAIN),
             "decision.js: unknown weight layout %d", layout);
  if (layout != DJ_W_PLAIN) {
    DJ_REQUIRE(N % 16 == 0 && K % 64 == 0, "decision.js: MFMA weight [%d, %d] needs N %% 16 == 0 and K %% 64 == 0", N, K);
    DJ_REQUIRE(base != DJ_W_MFMA_GLU || N % 32 == 0, "decision.js: fused w1|w3 [%d, %d] needs N %% 32 == 0", N, K);
  }
  dj_weight *w = new dj_weight();
  w->N = N; w->K = K; w->bits = bits; w->layout = layout;
  const size_t plain_codes = (size_t)N * K * bits / 8, plain_scales = (size_t)N * (K / 32) * 2;
  std::vector<uint8_t> oc;
  std::vector<uint32_t> os;
  const void *up_c = codes, *up_s = scales;
  w->code_bytes = plain_codes;
  w->scale_bytes = plain_scales;
  if (layout != DJ_W_PLAIN) {
    repack_mfma((const uint8_t *)codes, (const uint16_t *)scales, N, K, bits, layout, oc, os);
    up_c = oc.data();
    up_s = os.data();
    w->code_bytes = oc.size();
    w->scale_bytes = os.size() * 4;
  }
  if (hipMalloc((void **)&w->codes, w->code_bytes) != hipSuccess ||
      hipMalloc(&w->scales, w->scale_bytes) != hipSuccess) {
    (void)hipFree(w->codes);
    delete w;
    return dj_fail(DJ_ENOMEM, "decision.js: the GPU could not hold weight [%d, %d] (%.1f MB)", N, K,
                   (plain_codes + plain_scales) / 1e6);
  }
  DJ_HIP(hipMemcpy(w->codes, up_c, w->code_bytes, hipMemcpyHostToDevice));
  DJ_HIP(hipMemcpy(w->scales, up_s, w->scale_bytes, hipMemcpyHostToDevice));
  c->weights.push_back(w);
  *out = w;
  return DJ_OK;
}

extern "C" int dj_weight_free(dj_ctx *c, dj_weight *w) {
  DJ_REQUIRE(c, "decision.js: null context");
  if (!w) return DJ_OK;
  auto it = std::find(c->weights.begin(), c->weights.end(), w);
  DJ_REQUIRE(it != c->weights.end(), "decision.js: dj_weight_free: not a weight of this context");
  if (int st = dj_settle(c)) return st;
  DJ_HIP(hipStreamSynchronize(c->stream));
  (void)hipFree(w->codes);
  (void)hipFree(w->scales);
  c->weights.erase(it);
  delete w;
  return DJ_OK;
}

extern "C" size_t dj_weight_bytes(const dj_weight *w) { return w ? w->code_bytes + w->scale_bytes : 0; }

// ---------------------------------------------------------------- recorder and graphs

extern "C" int dj_rec_begin(dj_ctx *c, uint64_t key, dj_rec **out, int *replay) {
  DJ_REQUIRE(c && out, "decision.js: dj_rec_begin: null argument");
  DJ_REQUIRE(!c->active, "decision.js: a forward is already being recorded on this context");
  dj_rec *r = new dj_rec();
  r->ctx = c;
  r->key = key;
  if (key) {
    auto it = c->graphs.find(key);
    if (it != c->graphs.end()) {
      r->replay = true;
      it->second.last_use = ++c->graph_clock;
    } else {
      hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed);
      if (e != hipSuccess) {
        delete r;
        return dj_fail(DJ_EHIP, "decision.js: hipStreamBeginCapture: %s", hipGetErrorString(e));
      }
      r->capturing = true;
    }
  }
  if (replay) *replay = r->replay ? 1 : 0;
  c->active = r;
  *out = r;
  return DJ_OK;
}

static hipEvent_t pool_event(dj_ctx *c) {
  if (!c->event_pool.empty()) {
    hipEvent_t e = c->event_pool.back();
    c->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  (void)hipEventCreate(&e);
  return e;
}

int dj_op_begin(dj_rec *rec, const char *name) {
  if (!rec || !rec->ctx) return -dj_fail(DJ_ESTATE, "decision.js: %s: no recorder", name);
  dj_ctx *c = rec->ctx;
  if (c->active != rec) return -dj_fail(DJ_ESTATE, "decision.js: %s: recorder is not active", name);
  if (rec->holding) {  // the held product runs first, in the order the ops were issued
    const int st = dj_release_held(rec);
    if (st) return -st;
  }
  if (rec->replay) return 1;
  if (!c->fault_op.empty() && c->fault_left != 0 && (c->fault_op == name || c->fault_op == "*")) {
    if (c->fault_left > 0) c->fault_left--;
    return -dj_fail(DJ_EINJECT, "decision.js: fault injected in %s (DJ_FAULT_INJECT)", name);
  }
  if (c->profiling && !rec->capturing) {
    dj_prof_slot s{name, pool_event(c), pool_event(c)};
    (void)hipEventRecord(s.a, c->stream);
    c->prof_pending.push_back(s);
  }
  return 0;
}

int dj_op_end(dj_rec *rec, const char *name, const char *detail) {
  dj_ctx *c = rec->ctx;
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    rec->error = DJ_EHIP;
    return dj_fail(DJ_EHIP, "decision.js: launching %s: %s", name, hipGetErrorString(e));
  }
  if (c->profiling && !rec->capturing && !c->prof_pending.empty()) {
    dj_prof_slot &s = c->prof_pending.back();
    s.name = detail ? std::string(name) + detail : std::string(name);  // the launcher may refine the name
    (void)hipEventRecord(s.b, c->stream);
  }
  return DJ_OK;
}

int dj_settle(dj_ctx *c) { return c->active ? dj_release_held(c->active) : DJ_OK; }

extern "C" int dj_rec_snapshot(dj_rec *rec, const void *dev, size_t bytes, void *host) {
  DJ_REQUIRE(rec && rec->ctx && host, "decision.js: dj_rec_snapshot: null argument");
  dj_ctx *c = rec->ctx;
  DJ_REQUIRE(c->active == rec, "decision.js: dj_rec_snapshot: recorder is not active");
  if (int st = dj_release_held(rec)) return st;
  if (rec->replay) {
    auto &g = c->graphs[rec->key];
    DJ_REQUIRE(rec->snap_index < g.staging.size() && g.staging_bytes[rec->snap_index] == bytes,
               "decision.js: replayed forward asks for a snapshot the captured one did not take");
    rec->snaps.push_back({g.staging[rec->snap_index], bytes, host});
    rec->snap_index++;
    return DJ_OK;
  }
  DJ_REQUIRE(dev, "decision.js: dj_rec_snapshot: null device pointer");
  void *stage = nullptr;
  DJ_HIP(hipMalloc(&stage, std::max<size_t>(bytes, 16)));
  int s = dj_launch_copy(c->stream, stage, dev, bytes);
  if (s) {
    (void)hipFree(stage);
    return s;
  }
  rec->snaps.push_back({stage, bytes, host});
  return DJ_OK;
}

static void drain_profile(dj_ctx *c) {
  for (auto &s : c->prof_pending) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, s.a, s.b) == hipSuccess) {
      auto it = c->prof.find(s.name);
      if (it == c->prof.end()) {
        c->prof_order.push_back(s.name);
        c->prof[s.name] = {ms, 1};
      } else {
        it->second.first += ms;
        it->second.second += 1;
      }
    }
    c->event_pool.push_back(s.a);
    c->event_pool.push_back(s.b);
  }
  c->prof_pending.clear();
}

extern "C" int dj_rec_finish(dj_rec *r) {
  DJ_REQUIRE(r && r->ctx, "decision.js: dj_rec_finish: null recorder");
  dj_ctx *c = r->ctx;
  DJ_REQUIRE(c->active == r, "decision.js: dj_rec_finish: recorder is not active");
  if (int st = dj_release_held(r)) {
    if (!r->error) r->error = st;
  }
  c->active = nullptr;
  int status = DJ_OK;
  std::string msg;
  auto fail = [&](int code, const std::string &m) {
    if (!status) { status = code; msg = m; }
  };
  if (r->error) fail(r->error, g_err);
  if (r->capturing) {
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &graph);
    if (e != hipSuccess) fail(DJ_EHIP, std::string("decision.js: hipStreamEndCapture: ") + hipGetErrorString(e));
    if (!status) {
      dj_graph_entry ge;
      e = hipGraphInstantiate(&ge.exec, graph, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        fail(DJ_EHIP, std::string("decision.js: hipGraphInstantiate: ") + hipGetErrorString(e));
      } else {
        for (auto &s : r->snaps) {
          ge.staging.push_back(s.staging);
          ge.staging_bytes.push_back(s.bytes);
        }
        ge.last_use = ++c->graph_clock;
        evict_graphs(c, r->key);
        c->graphs[r->key] = ge;
        e = hipGraphLaunch(ge.exec, c->stream);
        if (e != hipSuccess) fail(DJ_EHIP, std::string("decision.js: hipGraphLaunch: ") + hipGetErrorString(e));
      }
    }
    if (graph) (void)hipGraphDestroy(graph);
    if (status) {  // the staging buffers belong to no graph: free them below
      c->graphs.erase(r->key);
    }
  } else if (r->replay && !status) {
    auto it = c->graphs.find(r->key);
    if (it == c->graphs.end()) {
      fail(DJ_ESTATE, "decision.js: replayed graph vanished");
    } else {
      hipError_t e = hipGraphLaunch(it->second.exec, c->stream);
      if (e != hipSuccess) fail(DJ_EHIP, std::string("decision.js: hipGraphLaunch: ") + hipGetErrorString(e));
    }
  }
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) fail(DJ_EHIP, std::string("decision.js: the forward failed on the GPU: ") + hipGetErrorString(e));
  c->pinned_used = 0;
  if (c->profiling) drain_profile(c);
  for (auto &s : r->snaps) {
    if (!status) {
      e = hipMemcpy(s.host, s.staging, s.bytes, hipMemcpyDeviceToHost);
      if (e != hipSuccess) fail(DJ_EHIP, std::string("decision.js: snapshot readback: ") + hipGetErrorString(e));
    }
  }
  const bool owned_by_graph = r->key && !status && (r->capturing || r->replay);
  if (!owned_by_graph)
    for (auto &s : r->snaps) (void)hipFree(s.staging);
  delete r;
  if (status) return dj_fail(status, "%s", msg.c_str());
  return DJ_OK;
}

extern "C" int dj_rec_abort(dj_rec *r) {
  DJ_REQUIRE(r && r->ctx, "decision.js: dj_rec_abort: null recorder");
  dj_ctx *c = r->ctx;
  DJ_REQUIRE(c->active == r, "decision.js: dj_rec_abort: recorder is not active");
  c->active = nullptr;
  r->holding = false;  // a held product is dropped, never launched
  if (r->capturing) {  // the partial capture becomes no graph
    hipGraph_t graph = nullptr;
    (void)hipStreamEndCapture(c->stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
  }
  (void)hipStreamSynchronize(c->stream);  // ops already launched run to their end; their results are dropped
  c->pinned_used = 0;
  if (c->profiling) drain_profile(c);
  if (!r->replay)  // a replay's snapshots are the cached graph's own staging buffers
    for (auto &s : r->snaps) (void)hipFree(s.staging);
  delete r;
  (void)hipGetLastError();
  return DJ_OK;
}

extern "C" int dj_graph_clear(dj_ctx *c) {
  DJ_REQUIRE(c, "decision.js: null context");
  DJ_REQUIRE(!c->active, "decision.js: dj_graph_clear during a forward");
  DJ_HIP(hipStreamSynchronize(c->stream));
  free_graphs(c);
  return DJ_OK;
}

extern "C" int dj_graph_drop(dj_ctx *c, uint64_t key) {
  DJ_REQUIRE(c, "decision.js: null context");
  DJ_REQUIRE(!c->active, "decision.js: dj_graph_drop during a forward");
  auto it = c->graphs.find(key);
  if (it == c->graphs.end()) return DJ_OK;
  DJ_HIP(hipStreamSynchronize(c->stream));
  free_graph(it->second);
  c->graphs.erase(it);
  return DJ_OK;
}

extern "C" int dj_graph_count(dj_ctx *c, int *n) {
  DJ_REQUIRE(c && n, "decision.js: dj_graph_count: null argument");
  *n = (int)c->graphs.size();
  return DJ_OK;
}

// ---------------------------------------------------------------- timers and profiling

extern "C" int dj_timer_begin(dj_ctx *c) {
  DJ_REQUIRE(c, "decision.js: null context");
  if (int st = dj_settle(c)) return st;
  DJ_HIP(hipEventRecord(c->t0, c->stream));
  return DJ_OK;
}

extern "C" int dj_timer_end(dj_ctx *c, float *ms) {
  DJ_REQUIRE(c && ms, "decision.js: null argument");
  if (int st = dj_settle(c)) return st;
  DJ_HIP(hipEventRecord(c->t1, c->stream));
  DJ_HIP(hipEventSynchronize(c->t1));
  DJ_HIP(hipEventElapsedTime(ms, c->t0, c->t1));
  return DJ_OK;
}

extern "C" int dj_profile_enable(dj_ctx *c, int on) {
  DJ_REQUIRE(c, "decision.js: null context");
  c->profiling = on != 0;
  return DJ_OK;
}

extern "C" int dj_profile_get(dj_ctx *c, dj_profile_entry *out, int cap, int *n) {
  DJ_REQUIRE(c && n, "decision.js: null argument");
  int k = 0;
  for (const std::string &name : c->prof_order) {
    if (out && k < cap) {
      auto &v = c->prof[name];
      snprintf(out[k].name, sizeof out[k].name, "%s", name.c_str());
      out[k].ms = v.first;
      out[k].launches = v.second;
    }
    ++k;
  }
  *n = k;
  return DJ_OK;
}

extern "C" int dj_profile_reset(dj_ctx *c) {
  DJ_REQUIRE(c, "decision.js: null context");
  c->prof.clear();
  c->prof_order.clear();
  return DJ_OK;
}
