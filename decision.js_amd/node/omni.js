"use strict";
/* d1-omni's engine on the Node host (D1OmniEngine, src/omni-engine.ts): the bidirectional LFM2 trunk (the
 * decoder's layer loop on centred taps and whole-sequence key ranges), then the decision head — the
 * question-type row added, pre-norm transformer layers with biases, the last residual under the scorer's
 * LayerNorm — and at each option marker Linear + GELU + Linear(H, 1). The same steps as
 * decision_js_amd/omni.py, which the tests hold the two hosts to (identical logits through the same library). */
const { kvSrc, lib } = require("./dj");
const { loadWeights } = require("./format");
const { DecoderEngine, layoutFor } = require("./engine");

const QTYPES = { choice: 0, score: 1, noul: 2 }; // omni-engine.ts:18

/** D1OmniEngine.logits's packing (omni-engine.ts:62-75). seqs: [{ids, markers, type}]. Per token: id, position
 * within its sequence, question type, the centred short-conv taps (t-1, t, t+1; -1 past either end of its
 * sequence) and its key range [start, end); per option marker its row on the packed axis. */
function packOmni(seqs) {
  const T = seqs.reduce((a, s) => a + s.ids.length, 0);
  const ids = new Uint32Array(T), pos = new Uint32Array(T), qtype = new Uint32Array(T);
  const taps = new Int32Array(T * 4), rng = new Int32Array(T * 4), markers = [];
  let off = 0;
  for (const s of seqs) {
    if (!(s.type in QTYPES)) throw new Error(`decision.js: question type ${JSON.stringify(s.type)} (choice, score or noul)`);
    const start = off, end = off + s.ids.length;
    for (const m of s.markers) {
      if (!(m >= 0 && m < s.ids.length)) throw new Error(`decision.js: a marker outside its sequence of ${s.ids.length} tokens`);
      markers.push(start + m);
    }
    for (let i = 0; i < s.ids.length; ++i, ++off) {
      ids[off] = s.ids[i];
      pos[off] = i;
      qtype[off] = QTYPES[s.type];
      taps.set([off > start ? off - 1 : -1, off, off + 1 < end ? off + 1 : -1, 0], 4 * off);
      rng.set([start, end, 0, 0], 4 * off);
    }
  }
  return { ids, pos, qtype, taps, rng, markers: Uint32Array.from(markers), T, M: markers.length };
}

/** The calibration temperature of a question (omni-engine.ts:22-26). */
function temperature(config, type, options) {
  const k = options <= 2 ? "2" : options <= 5 ? "3-5" : options <= 10 ? "6-10" : "11+";
  const t = config.temperatures || {};
  return t[`${type}:${k}`] !== undefined ? t[`${type}:${k}`] : t[type] !== undefined ? t[type] : 1;
}

const INPUTS = ["ids", "pos", "qtype", "rng", "taps", "markers"];

class OmniEngine extends DecoderEngine {
  static async load(base, opts) {
    opts = opts || {};
    const direct = !!(opts.directWeights || opts.direct_weights);
    const { ctx, m, w } = await loadWeights(base, opts, layoutFor(direct));
    const c = m.config;
    if (c.model !== "d1-omni" && !("head_layers" in c)) throw new Error(`decision.js: ${base} is not a d1-omni model (${c.model})`);
    const bad = (c.layer_types || []).filter((t) => t !== "full_attention" && t !== "conv");
    if (bad.length) throw new Error(`decision.js: unsupported layer types ${JSON.stringify(Array.from(new Set(bad)).sort())}`);
    if (c.hidden % c.head_heads || ![64, 128, 256].includes(c.hidden / c.head_heads))
      throw new Error(`decision.js: head width ${c.hidden} / ${c.head_heads} heads (64, 128 or 256 per head)`);
    return new OmniEngine(ctx, m, w, opts);
  }

  constructor(ctx, m, w, opts) {
    super(ctx, m, w, opts);
    const c = m.config;
    Object.assign(this, { hh: c.head_heads, ff: c.head_ff, lnEps: c.ln_eps, headLayers: c.head_layers });
    this.Dh = this.H / this.hh;
    this.typeRows = m.tensors["head.type_emb"].shape[0];
    this.markerCapacity = 0;
  }

  /** Activation buffers for T tokens and M markers (omni-engine.ts:44-52: grown, never shrunk). */
  ensure(T, M = 0) {
    if (T <= this.capacity && M <= this.markerCapacity) return;
    const cap = Math.ceil(Math.max(T, this.capacity, 256) / 64) * 64;
    const mcap = Math.max(M, this.markerCapacity, 64);
    const H = this.H;
    const zw = Math.max(this.stride, 3 * H), yw = Math.max(this.h * this.D, H);
    this.alloc({ x: cap * H * 2, normed: cap * H * 2, o: cap * H * 2, z: cap * zw * 2, y: cap * yw * 2,
      h: cap * Math.max(this.I, this.ff) * 2, ids: cap * 4, pos: cap * 4, qtype: cap * 4, rng: cap * 16, taps: cap * 16,
      rope: cap * (this.D / 2) * 8, markers: mcap * 4, g: mcap * H * 2, gf: mcap * H * 2, out: mcap * 4, ...this.normBufs(cap) });
    this.capacity = cap;
    this.markerCapacity = mcap;
  }

  /** Raw marker logits per sequence ([seq][marker], before the temperature); with `debug` also the trunk's
   * output and the head's stream before the scorer (f16 bits, [T * H]). */
  async logits(seqs, debug = false) {
    const pk = this.pack(seqs);
    if (pk.T === 0) return { logits: seqs.map(() => []), debug: {} };
    const { T, M } = pk;
    this.ensure(T, M);
    const B = this.bufs;
    for (const k of this.inputs) if (pk[k].length) B[k].upload(pk[k]);
    const rec = this.ctx.recorder(this.key(["omni", T, M, !!debug]));
    const snaps = {};
    const oi = rec.record(() => { // aborted on an error; a replay returns its snapshots in the order taken
      if (!rec.replay) this.recordLayers(rec, T, B, null, null);
      if (debug) snaps.trunk = rec.snapshot(B.normed.ptr, Uint16Array, T * this.H);
      if (!rec.replay) this.recordHead(rec, T, M, B);
      if (debug) snaps.head = rec.snapshot(B.x.ptr, Uint16Array, T * this.H);
      return M ? rec.snapshot(B.out.ptr, Float32Array, M) : -1;
    });
    const got = await this.finish(rec, T);
    const out = oi >= 0 ? got[oi] : new Float32Array(0);
    let k = 0;
    const logits = seqs.map((s) => Array.from(out.subarray(k, (k += s.markers.length))));
    const dbg = {};
    for (const [n, i] of Object.entries(snaps)) dbg[n] = got[i];
    return { logits, debug: dbg };
  }

  pack(seqs) {
    return packOmni(seqs);
  }

  get inputs() {
    return INPUTS;
  }

  /** The decision head and scorer (omni-engine.ts:125-147). */
  recordHead(rec, T, M, B) {
    const w = this.w, L = lib();
    const { H, hh, Dh, lnEps } = this;
    const z = B.z.ptr, src = kvSrc(z, T, 3 * H, H, 2 * H);
    rec.addRows(T, H, B.normed.ptr, B.qtype.ptr, w["head.type_emb"].ptr, this.typeRows, B.x.ptr);
    for (let i = 0; i < this.headLayers; ++i) {
      const p = `head.${i}.`;
      // i > 0: the residual first takes the previous layer's FFN output
      rec.addLayernorm(T, H, i > 0, lnEps, B.x.ptr, B.o.ptr, w[p + "norm1"].ptr, w[p + "norm1_bias"].ptr, B.normed.ptr);
      rec.matmul(B.normed.ptr, w[p + "in_proj"], z, T);
      rec.biasAct(T, 3 * H, z, w[p + "in_proj_bias"].ptr, L.BIAS_NONE);
      rec.attention(T, hh, hh, Dh, z, 3 * H, src, src, B.rng.ptr, 1 / Math.sqrt(Dh), B.y.ptr);
      rec.matmul(B.y.ptr, w[p + "out_proj"], B.o.ptr, T);
      rec.biasAct(T, H, B.o.ptr, w[p + "out_proj_bias"].ptr, L.BIAS_NONE);
      rec.addLayernorm(T, H, true, lnEps, B.x.ptr, B.o.ptr, w[p + "norm2"].ptr, w[p + "norm2_bias"].ptr, B.normed.ptr);
      rec.matmul(B.normed.ptr, w[p + "linear1"], B.h.ptr, T);
      rec.biasAct(T, this.ff, B.h.ptr, w[p + "linear1_bias"].ptr, L.BIAS_RELU);
      rec.matmul(B.h.ptr, w[p + "linear2"], B.o.ptr, T);
      rec.biasAct(T, H, B.o.ptr, w[p + "linear2_bias"].ptr, L.BIAS_NONE);
    }
    // the last residual add, under the scorer's LayerNorm
    rec.addLayernorm(T, H, this.headLayers > 0, lnEps, B.x.ptr, B.o.ptr, w["scorer.norm"].ptr, w["scorer.norm_bias"].ptr, B.normed.ptr);
    if (M) {
      rec.gatherRows(M, H, T, B.normed.ptr, B.markers.ptr, B.g.ptr);
      rec.matmul(B.g.ptr, w["scorer.fc"], B.gf.ptr, M);
      rec.biasAct(M, H, B.gf.ptr, w["scorer.fc_bias"].ptr, L.BIAS_GELU_ERF);
      rec.score(M, H, B.gf.ptr, w["scorer.out"].ptr, w["scorer.out_bias"].ptr, B.out.ptr);
    }
  }
}

module.exports = { OmniEngine, packOmni, temperature, QTYPES };
