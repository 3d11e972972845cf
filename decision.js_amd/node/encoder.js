"use strict";
/* The EmbeddingGemma-shaped bidirectional encoder engine on the Node host (Eg2Engine, eg2-engine.ts): every
 * text one sequence, many packed on one token axis, one recorded forward; then mean pooling and the configured
 * head (Linear hidden->width, Linear width->embed_dim, in f32) and L2 normalisation. The same steps as
 * decision_js_amd/encoder.py, which the tests hold the two hosts to. */
const { lib, kvSrc } = require("./dj");
const { loadWeights } = require("./format");
const { GpuEngine, layoutFor } = require("./engine");

/** Eg2Engine.embed's packing (eg2-engine.ts:74-86): per token meta (start, end, -1, i) and its key range on
 * the global layers [start, end) and, with a window, on the sliding layers [max(start, t-w), min(end, t+w+1));
 * per sequence (start, end). */
function packEncoder(seqs, window) {
  const T = seqs.reduce((a, s) => a + s.length, 0), S = seqs.length;
  const ids = new Uint32Array(T), meta = new Int32Array(T * 4), full = new Int32Array(T * 4), ranges = new Uint32Array(S * 2);
  const slide = window === undefined ? null : new Int32Array(T * 4);
  let off = 0;
  seqs.forEach((s, k) => {
    for (let i = 0; i < s.length; ++i) {
      const t = off + i;
      ids[t] = s[i];
      meta.set([off, off + s.length, -1, i], 4 * t);
      full[4 * t] = off;
      full[4 * t + 1] = off + s.length;
      if (slide) {
        slide[4 * t] = Math.max(off, t - window);
        slide[4 * t + 1] = Math.min(off + s.length, t + window + 1);
      }
    }
    ranges[2 * k] = off;
    ranges[2 * k + 1] = off + s.length;
    off += s.length;
  });
  return { ids, meta, full, slide, ranges, T, S };
}

/** The cosine prior of Eg2Head.logits (eg2-head.ts:82-84, 97): cos(option, state + question). */
function cosineLogits(s, q, opts) {
  const anchor = Array.from(s, (v, i) => v + q[i]);
  const an = Math.max(Math.hypot(...anchor), 1e-12);
  return opts.map((o) => {
    const on = Math.max(Math.hypot(...o), 1e-12);
    let d = 0;
    for (let i = 0; i < o.length; ++i) d += (o[i] / on) * anchor[i];
    return d / an;
  });
}

class EncoderEngine extends GpuEngine {
  static async load(base, opts) {
    opts = opts || {};
    const direct = !!(opts.directWeights || opts.direct_weights);
    const { ctx, m, w, host } = await loadWeights(base, opts, layoutFor(direct));
    if (m.config.model !== "eg2-encoder" && m.config.model !== "eg2") throw new Error(`decision.js: ${base} is not an encoder model (${m.config.model})`);
    const e = new EncoderEngine(ctx, m, w, opts);
    e.host = host; // the decision head's f32 tensors, kept on the host (eg2-engine.ts:46-50)
    return e;
  }

  constructor(ctx, m, w, opts) {
    super(ctx, m, w, opts);
    const c = m.config;
    Object.assign(this, { H: c.hidden, I: c.intermediate, h: c.heads, kv: c.kv_heads, D: c.head_dim, eps: c.eps, theta: c.rope_theta });
    this.layers = c.layers;
    this.stride = (this.h + 2 * this.kv) * this.D;
    this.scalars = c.layer_scalars || new Array(this.layers).fill(1);
    this.scale = c.attention_scale === undefined ? 1 : c.attention_scale;
    this.width = c.head_width;
    this.E = c.embed_dim;
    this.capacity = 0;
    this.seqCapacity = 0;
    this.host = {};
  }

  ensure(T, S) {
    if (T <= this.capacity && S <= this.seqCapacity) return;
    const cap = Math.ceil(Math.max(T, this.capacity, 256) / 64) * 64, scap = Math.max(S, this.seqCapacity, 64);
    const H = this.H;
    this.alloc({ x: cap * H * 2, normed: cap * H * 2, o: cap * H * 2, z: cap * this.stride * 2, y: cap * this.h * this.D * 2,
      h: cap * this.I * 2, ids: cap * 4, meta: cap * 16, rng: cap * 16, seqs: scap * 8, pooled: scap * H * 4,
      h1: scap * this.width * 4, emb: scap * this.E * 4 });
    this.capacity = cap;
    this.seqCapacity = scap;
  }

  /** The normalized embedding of every token sequence: Float32Array per sequence. */
  async embed(seqs) {
    const pk = packEncoder(seqs);
    const { T, S } = pk;
    this.ensure(T, S);
    const B = this.bufs;
    B.ids.upload(pk.ids);
    B.meta.upload(pk.meta);
    B.rng.upload(pk.full);
    B.seqs.upload(pk.ranges);
    const rec = this.ctx.recorder(this.key(["embed", T, S]));
    const ei = rec.record(() => this.recordEmbed(rec, T, S)); // aborted on an error
    const got = await rec.finish();
    this.stats.forwards += 1;
    this.stats.tokens += T;
    const e = got[ei];
    const embeddings = [];
    for (let s = 0; s < S; ++s) {
      const v = e.subarray(s * this.E, (s + 1) * this.E);
      let ss = 0;
      for (const x of v) ss += x * x;
      const n = Math.max(Math.sqrt(ss), 1e-12);
      embeddings.push(Float32Array.from(v, (x) => x / n));
    }
    return { embeddings };
  }

  /** The encoder's ops (eg2-engine.ts:103-129 without per-layer embeddings), pooling and head; returns the
   * embeddings' snapshot index. */
  recordEmbed(rec, T, S) {
    const B = this.bufs, w = this.w, L = lib();
    const { H, h, kv, D, eps } = this;
    if (!rec.replay) {
      const z = B.z.ptr, src = kvSrc(z, T, this.stride, h * D, (h + kv) * D), ptr = (n) => w[n].ptr;
      rec.gatherQ(B.ids.ptr, T, w.embed, B.x.ptr);
      rec.sandwich(T, H, eps, 1, B.x.ptr, 0n, 0n, ptr("layers.0.input_layernorm"), B.normed.ptr);
      for (let i = 0; i < this.layers; ++i) {
        const p = `layers.${i}.`;
        rec.matmul(B.normed.ptr, w[p + "qkv"], z, T);
        rec.qkNormRope(T, h, kv, D, this.stride, z, ptr(p + "q_norm"), ptr(p + "k_norm"), true, B.meta.at(12), 4, eps, this.theta, D,
          L.ROPE_INV_POW);
        rec.attention(T, h, kv, D, z, this.stride, src, src, B.rng.ptr, this.scale, B.y.ptr);
        rec.matmul(B.y.ptr, w[p + "o"], B.o.ptr, T);
        rec.sandwich(T, H, eps, 1, B.x.ptr, B.o.ptr, ptr(p + "post_attention_layernorm"), ptr(p + "pre_feedforward_layernorm"), B.normed.ptr);
        rec.matmulGlu(B.normed.ptr, w[p + "gu"], B.h.ptr, T, L.ACT_GELU_TANH);
        rec.matmul(B.h.ptr, w[p + "down"], B.o.ptr, T);
        const nxt = i + 1 < this.layers ? `layers.${i + 1}.input_layernorm` : "final_norm";
        rec.sandwich(T, H, eps, this.scalars[i], B.x.ptr, B.o.ptr, ptr(p + "post_feedforward_layernorm"), ptr(nxt), B.normed.ptr);
      }
      rec.meanPool(T, S, H, B.normed.ptr, B.seqs.ptr, B.pooled.ptr);
      rec.denseF32(S, B.pooled.ptr, w["head.dense1"], B.h1.ptr);
      rec.denseF32(S, B.h1.ptr, w["head.dense2"], B.emb.ptr);
    }
    return rec.snapshot(B.emb.ptr, Float32Array, S * this.E);
  }
}

module.exports = { EncoderEngine, packEncoder, cosineLogits };
