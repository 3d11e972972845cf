"use strict";
/* Laya's engine on the Node host (LayaEngine, src/laya-engine.ts): a ModernBERT encoder (bias-free LayerNorms,
 * RoPE attention over the whole sequence on the global layers and a +-window on the others, the erf-GELU GeGLU
 * MLP; layer 0 reads the stream without an attention norm), then d1-omni's decision head and scorer. The same
 * steps as decision_js_amd/laya.py, which the tests hold the two hosts to (identical logits through the same
 * library). */
const { kvSrc, lib } = require("./dj");
const { loadWeights } = require("./format");
const { layoutFor } = require("./engine");
const { OmniEngine, packOmni } = require("./omni");

/** LayaEngine.logits's packing (laya-engine.ts:57-66): packOmni's arrays plus each token's window
 * [max(start, t - window), min(end, t + window + 1)) for the local layers. */
function packLaya(seqs, window) {
  const pk = packOmni(seqs);
  const win = new Int32Array(pk.T * 4);
  for (let t = 0; t < pk.T; ++t) {
    win[4 * t] = Math.max(pk.rng[4 * t], t - window);
    win[4 * t + 1] = Math.min(pk.rng[4 * t + 1], t + window + 1);
  }
  pk.win = win;
  return pk;
}

const INPUTS = ["ids", "pos", "qtype", "rng", "win", "markers"];

class LayaEngine extends OmniEngine {
  static async load(base, opts) {
    opts = opts || {};
    const direct = !!(opts.directWeights || opts.direct_weights);
    const { ctx, m, w } = await loadWeights(base, opts, layoutFor(direct));
    const c = m.config;
    if (c.model !== "laya") throw new Error(`decision.js: ${base} is not a Laya export (${c.model})`);
    const bad = c.layer_types.filter((t) => t !== "full_attention" && t !== "sliding_attention");
    if (bad.length) throw new Error(`decision.js: unsupported layer types ${JSON.stringify(Array.from(new Set(bad)).sort())}`);
    for (const t of new Set(c.layer_types)) if (!(t in c.rope_theta)) throw new Error(`decision.js: no rope_theta for ${t} layers`);
    if (c.hidden % c.heads || ![64, 128, 256].includes(c.hidden / c.heads))
      throw new Error(`decision.js: encoder width ${c.hidden} / ${c.heads} heads (64, 128 or 256 per head)`);
    if (c.hidden % c.head_heads || ![64, 128, 256].includes(c.hidden / c.head_heads))
      throw new Error(`decision.js: head width ${c.hidden} / ${c.head_heads} heads (64, 128 or 256 per head)`);
    return new LayaEngine(ctx, m, w, opts);
  }

  constructor(ctx, m, w, opts) {
    // OmniEngine's constructor reads the decoder's kv_heads and head_dim: Laya's heads are all full width
    super(ctx, { ...m, config: { ...m.config, kv_heads: m.config.heads, head_dim: m.config.hidden / m.config.heads } }, w, opts);
    this.m = m;
    const c = m.config;
    Object.assign(this, { stride: 3 * c.hidden, conv: false, eps: c.eps, window: c.window, theta: null });
    this.zeros = ctx.array(new Uint16Array(c.hidden)); // the bias of the bias-free LayerNorms
  }

  /** Activation buffers for T tokens and M markers (laya-engine.ts:38-47: grown, never shrunk). */
  ensure(T, M = 0) {
    if (T <= this.capacity && M <= this.markerCapacity) return;
    const cap = Math.ceil(Math.max(T, this.capacity, 256) / 64) * 64;
    const mcap = Math.max(M, this.markerCapacity, 64);
    const H = this.H;
    this.alloc({ x: cap * H * 2, normed: cap * H * 2, o: cap * H * 2, z: cap * 3 * H * 2, y: cap * H * 2,
      h: cap * Math.max(this.I, this.ff) * 2, ids: cap * 4, pos: cap * 4, qtype: cap * 4, rng: cap * 16, win: cap * 16,
      markers: mcap * 4, g: mcap * H * 2, gf: mcap * H * 2, out: mcap * 4 });
    this.capacity = cap;
    this.markerCapacity = mcap;
  }

  pack(seqs) {
    return packLaya(seqs, this.window);
  }

  get inputs() {
    return INPUTS;
  }

  /** The encoder (laya-engine.ts:99-115); its output lands in B.normed as the head expects. */
  recordLayers(rec, T, B) {
    const w = this.w, L = lib(), c = this.m.config;
    const { H, h, D, eps } = this;
    const z = B.z.ptr, src = kvSrc(z, T, 3 * H, H, 2 * H), zeros = this.zeros.ptr;
    rec.gatherQ(B.ids.ptr, T, w.embed, B.normed.ptr);
    rec.addLayernorm(T, H, false, eps, B.normed.ptr, B.o.ptr, w.embed_norm.ptr, zeros, B.x.ptr);
    this.types.forEach((t, i) => {
      const p = `layers.${i}.`;
      let inp = B.x.ptr;
      if (w[p + "attn_norm"]) { // adds the previous layer's MLP output (every layer but the first)
        rec.addLayernorm(T, H, true, eps, B.x.ptr, B.o.ptr, w[p + "attn_norm"].ptr, zeros, B.normed.ptr);
        inp = B.normed.ptr;
      }
      rec.matmul(inp, w[p + "qkv"], z, T);
      rec.qkNormRope(T, h, h, D, 3 * H, z, 0n, 0n, false, B.pos.ptr, 1, eps, c.rope_theta[t], D, L.ROPE_POW_NEG);
      rec.attention(T, h, h, D, z, 3 * H, src, src, (t === "full_attention" ? B.rng : B.win).ptr, 1 / Math.sqrt(D), B.y.ptr);
      rec.matmul(B.y.ptr, w[p + "o"], B.o.ptr, T);
      rec.addLayernorm(T, H, true, eps, B.x.ptr, B.o.ptr, w[p + "mlp_norm"].ptr, zeros, B.normed.ptr);
      rec.matmulGlu(B.normed.ptr, w[p + "wi"], B.h.ptr, T, L.ACT_GELU_ERF);
      rec.matmul(B.h.ptr, w[p + "wo"], B.o.ptr, T);
    });
    rec.addLayernorm(T, H, true, eps, B.x.ptr, B.o.ptr, w.final_norm.ptr, zeros, B.normed.ptr);
  }

  destroy() {
    if (this.zeros) this.zeros.free();
    this.zeros = null;
    super.destroy();
  }
}

module.exports = { LayaEngine, packLaya };
