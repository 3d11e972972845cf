"use strict";
/* EmbeddingGemma 2 as shipped, Node host (Eg2Engine, src/eg2-engine.ts): the bidirectional Gemma text encoder with
 * per-layer embeddings — sandwich norms, q/k/v norms + RoPE with each layer type's head width and theta (a window
 * on the sliding layers), the tanh-GELU MLP, the per-layer embedding with the layer scalar — then the pooled
 * f16 projection, the first embed_dim values L2-normalised. The same steps as decision_js_amd/eg2.py, which the
 * tests hold the two hosts to. */
const { lib, kvSrc } = require("./dj");
const { loadWeights } = require("./format");
const { GpuEngine, layoutFor } = require("./engine");
const { packEncoder } = require("./encoder");

class Eg2Engine extends GpuEngine {
  static async load(base, opts) {
    opts = opts || {};
    const direct = !!(opts.directWeights || opts.direct_weights);
    const { ctx, m, w, host } = await loadWeights(base, opts, layoutFor(direct));
    const c = m.config;
    if (c.model !== "eg2" || !("ple" in c)) throw new Error(`decision.js: ${base} is not an EmbeddingGemma 2 export (${c.model})`);
    const bad = c.layer_types.filter((t) => t !== "sliding_attention" && t !== "full_attention");
    if (bad.length) throw new Error(`decision.js: unsupported layer types ${JSON.stringify(Array.from(new Set(bad)).sort())}`);
    for (const t of new Set(c.layer_types)) {
      if (![64, 128, 256, 512].includes(c.head_dim[t])) throw new Error(`decision.js: ${t} heads of ${c.head_dim[t]} dims (64, 128, 256 or 512)`);
    }
    const e = new Eg2Engine(ctx, m, w, opts);
    e.host = host; // the decision head's f32 tensors (eg2-engine.ts:46-50)
    return e;
  }

  constructor(ctx, m, w, opts) {
    super(ctx, m, w, opts);
    const c = m.config;
    Object.assign(this, { H: c.hidden, I: c.intermediate, h: c.heads, P: c.ple, eps: c.eps, types: c.layer_types });
    this.layers = c.layers;
    this.N = c.embedding_dim;
    this.E = c.embed_dim;
    this.scalars = c.layer_scalars || new Array(this.layers).fill(1);
    this.qkvW = Math.max(...this.types.map((t) => (this.h + 2 * c.kv_heads[t]) * c.head_dim[t]));
    this.attW = Math.max(...this.types.map((t) => this.h * c.head_dim[t]));
    this.capacity = 0;
    this.seqCapacity = 0;
    this.host = {};
  }

  ensure(T, S) {
    if (T <= this.capacity && S <= this.seqCapacity) return;
    const cap = Math.ceil(Math.max(T, this.capacity, 256) / 64) * 64, scap = Math.max(S, this.seqCapacity, 64);
    const { H, P } = this;
    this.alloc({ x: cap * H * 2, xe: cap * H * 2, normed: cap * H * 2, o: cap * H * 2, z: cap * this.qkvW * 2,
      y: cap * this.attW * 2, h: cap * this.I * 2, gate: cap * P * 2, e: cap * P * 2, mix: cap * P * 2, ids: cap * 4,
      meta: cap * 16, full: cap * 16, slide: cap * 16, seqs: scap * 8, emb: scap * this.N * 4 });
    this.capacity = cap;
    this.seqCapacity = scap;
  }

  /** The normalized embedding of every token sequence: Float32Array (embed_dim) per sequence. */
  async embed(seqs) {
    const pk = packEncoder(seqs, this.m.config.window);
    const { T, S } = pk;
    if (T === 0) return { embeddings: seqs.map(() => new Float32Array(this.E)) };
    this.ensure(T, S);
    const B = this.bufs;
    B.ids.upload(pk.ids);
    B.meta.upload(pk.meta);
    B.full.upload(pk.full);
    B.slide.upload(pk.slide);
    B.seqs.upload(pk.ranges);
    const rec = this.ctx.recorder(this.key(["eg2", T, S, false]));
    const ei = rec.record(() => { // aborted on an error
      if (!rec.replay) this.recordEmbed(rec, T, S);
      return rec.snapshot(B.emb.ptr, Float32Array, S * this.N);
    });
    const got = await rec.finish();
    this.stats.forwards += 1;
    this.stats.tokens += T;
    const e = got[ei];
    const embeddings = [];
    for (let s = 0; s < S; ++s) {
      const v = e.subarray(s * this.N, s * this.N + this.E);
      let ss = 0;
      for (const x of v) ss += x * x;
      const n = Math.max(Math.sqrt(ss), 1e-12);
      embeddings.push(Float32Array.from(v, (x) => x / n));
    }
    return { embeddings };
  }

  /** The layer loop of eg2-engine.ts:103-131, then POOL_PROJECT. */
  recordEmbed(rec, T, S) {
    const B = this.bufs, w = this.w, L = lib(), c = this.m.config;
    const { H, h, eps, P } = this;
    const z = B.z.ptr, ptr = (n) => w[n].ptr;
    rec.gatherQ(B.ids.ptr, T, w.embed, B.x.ptr);
    rec.gatherQ(B.ids.ptr, T, w.embed, B.xe.ptr); // the copy each layer projects its own embedding from
    rec.sandwich(T, H, eps, 1, B.x.ptr, 0n, 0n, ptr("layers.0.input_layernorm"), B.normed.ptr);
    this.types.forEach((t, i) => {
      const p = `layers.${i}.`, D = c.head_dim[t], kv = c.kv_heads[t];
      const stride = (h + 2 * kv) * D, src = kvSrc(z, T, stride, h * D, (h + kv) * D);
      rec.matmul(B.normed.ptr, w[p + "qkv"], z, T);
      rec.qkNormRope(T, h, kv, D, stride, z, ptr(p + "q_norm"), ptr(p + "k_norm"), true, B.meta.at(12), 4, eps, c.rope_theta[t], D,
        L.ROPE_INV_POW);
      rec.attention(T, h, kv, D, z, stride, src, src, (t === "full_attention" ? B.full : B.slide).ptr, 1, B.y.ptr);
      rec.matmul(B.y.ptr, w[p + "o"], B.o.ptr, T);
      rec.sandwich(T, H, eps, 1, B.x.ptr, B.o.ptr, ptr(p + "post_attention_layernorm"), ptr(p + "pre_feedforward_layernorm"), B.normed.ptr);
      rec.matmulGlu(B.normed.ptr, w[p + "gu"], B.h.ptr, T, L.ACT_GELU_TANH);
      rec.matmul(B.h.ptr, w[p + "down"], B.o.ptr, T);
      rec.sandwich(T, H, eps, 1, B.x.ptr, B.o.ptr, ptr(p + "post_feedforward_layernorm"), 0n, 0n);
      rec.matmul(B.x.ptr, w[p + "ple_gate"], B.gate.ptr, T);
      rec.matmul(B.xe.ptr, w[p + "ple_in"], B.e.ptr, T);
      rec.pleMix(T, P, B.gate.ptr, B.e.ptr, ptr("ple.norm"), eps, B.mix.ptr);
      rec.matmul(B.mix.ptr, w[p + "ple_proj"], B.o.ptr, T);
      const nxt = i + 1 < this.layers ? `layers.${i + 1}.input_layernorm` : "final_norm";
      rec.sandwich(T, H, eps, this.scalars[i], B.x.ptr, B.o.ptr, ptr(p + "ple_norm"), ptr(nxt), B.normed.ptr);
    });
    rec.poolProject(T, S, H, this.N, B.normed.ptr, B.seqs.ptr, ptr("projection"), B.emb.ptr);
  }
}

module.exports = { Eg2Engine };
