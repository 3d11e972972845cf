"use strict";
/* d3-lite's engine on its shipped layout, Node host (D3Engine, src/d3-engine.ts): Gated DeltaNet layers (`in`,
 * gdn, `out`) with a gated attention layer every few (fused q | k | v | gate, q/k RMSNorm + partial RoPE,
 * attentionGated, `o`), SwiGLU, the final norm and READOUT at each question's last token. The same steps as
 * decision_js_amd/d3.py, which the tests hold the two hosts to (identical logits through the same library). */
const { kvSrc, lib } = require("./dj");
const { loadWeights } = require("./format");
const { DecoderEngine, layoutFor, packShared } = require("./engine");

/** The DeltaNet scans of D3Engine.logits's packing (d3-engine.ts:89) on packShared's rows: per question (a start,
 * a length | write_a << 31, b start, b length); a shared trunk is span a, written by the group's first question. */
function gdnSpans(seqs, groups) {
  const sizes = groups || seqs.map(() => 1);
  const out = new Uint32Array(seqs.length * 4);
  let si = 0, off = 0;
  for (const n of sizes) {
    const group = seqs.slice(si, si + n);
    let P = 0;
    if (n > 1) {
      const lim = Math.min(...group.map((s) => s.ids.length)) - 1;
      while (P < lim && group.every((s) => s.ids[P] === group[0].ids[P])) P++;
    }
    const ts = off;
    off += P;
    group.forEach((s, b) => {
      const L = s.ids.length - P;
      out.set(P ? [ts, (P | (b === 0 ? 0x80000000 : 0)) >>> 0, off, L] : [off, (L | 0x80000000) >>> 0, 0, 0], 4 * (si + b));
      off += L;
    });
    si += n;
  }
  return out;
}

class D3Engine extends DecoderEngine {
  static async load(base, opts) {
    opts = opts || {};
    const direct = !!(opts.directWeights || opts.direct_weights);
    const { ctx, m, w } = await loadWeights(base, opts, layoutFor(direct));
    const c = m.config;
    if (c.model !== "d3" || !("linear_heads" in c)) throw new Error(`decision.js: ${base} is not a d3-lite export (${c.model})`);
    const bad = c.layer_types.filter((t) => t !== "linear_attention" && t !== "full_attention");
    if (bad.length) throw new Error(`decision.js: unsupported layer types ${JSON.stringify(Array.from(new Set(bad)).sort())}`);
    if (c.linear_key_dim !== 128 || c.linear_value_dim !== 128 || (c.conv_kernel || 4) !== 4)
      throw new Error(`decision.js: the DeltaNet kernel takes 128-wide key and value heads and 4 conv taps (got ${c.linear_key_dim}, ${c.linear_value_dim}, ${c.conv_kernel})`);
    if (![64, 128, 256].includes(c.head_dim) || !(c.rotary_dim > 0 && c.rotary_dim <= c.head_dim) || c.rotary_dim % 16)
      throw new Error(`decision.js: attention heads of ${c.head_dim} with ${c.rotary_dim} rotary dims`);
    return new D3Engine(ctx, m, w, opts);
  }

  constructor(ctx, m, w, opts) {
    super(ctx, m, w, opts);
    const c = m.config;
    Object.assign(this, { LH: c.linear_heads, rows: c.linear_rows, rot: c.rotary_dim });
    this.astride = (2 * this.h + 2 * this.kv) * this.D;
    this.codes = m.tensors.readout.shape[0];
    this.seqCapacity = 0;
  }

  ensure(T, P = 0, S = 0) {
    if (T <= this.capacity && P <= this.leafCapacity && S <= this.seqCapacity) return;
    const cap = Math.ceil(Math.max(T, this.capacity, 256) / 64) * 64;
    const pcap = Math.max(P, this.leafCapacity, 1024), scap = Math.max(S, this.seqCapacity, 64);
    const H = this.H;
    this.alloc({ x: cap * H * 2, normed: cap * H * 2, o: cap * H * 2, z: cap * Math.max(this.rows, this.astride) * 2,
      y: cap * Math.max(this.LH * 128, this.h * this.D) * 2, h: cap * this.I * 2, ids: cap * 4, pos: cap * 4, rng: cap * 16,
      spans: scap * 16, leafIds: pcap * 8, out: pcap * 4 });
    this.capacity = cap;
    this.leafCapacity = pcap;
    this.seqCapacity = scap;
  }

  /** Code logits per question ([seq][its options codes], before the temperature; D3Engine.logits). */
  async logitsD3(seqs, groups) {
    const pk = packShared(seqs, groups), spans = gdnSpans(seqs, groups);
    const { T, P } = pk, S = seqs.length;
    if (T === 0) return seqs.map(() => []);
    this.ensure(T, P, S);
    const B = this.bufs;
    B.ids.upload(pk.ids);
    B.pos.upload(pk.pos);
    B.rng.upload(pk.rng);
    B.spans.upload(spans);
    if (P) B.leafIds.upload(pk.pairs);
    const rec = this.ctx.recorder(this.key(["d3lite", T, P, S, false]));
    const oi = rec.record(() => { // aborted on an error
      if (!rec.replay) {
        this.recordD3(rec, T, S, B);
        if (P) rec.readout(T, P, this.H, B.normed.ptr, this.w.readout.ptr, this.codes, B.leafIds.ptr, B.out.ptr);
      }
      return P ? rec.snapshot(B.out.ptr, Float32Array, P) : -1;
    });
    const got = await this.finish(rec, T);
    const out = oi >= 0 ? got[oi] : new Float32Array(0);
    let k = 0;
    return seqs.map((s) => Array.from(out.subarray(k, (k += s.options))));
  }

  /** The layer loop of d3-engine.ts:109-131. */
  recordD3(rec, T, S, B) {
    const w = this.w, L = lib();
    const { H, h, kv, D, eps, astride: A } = this;
    const z = B.z.ptr, src = kvSrc(z, T, A, h * D, (h + kv) * D);
    rec.gatherQ(B.ids.ptr, T, w.embed, B.x.ptr);
    this.types.forEach((t, i) => {
      const p = `layers.${i}.`;
      rec.addRmsnorm(T, H, i > 0, eps, B.x.ptr, B.o.ptr, w[p + "input_norm"].ptr, B.normed.ptr); // adds the last MLP
      if (t === "linear_attention") {
        rec.matmul(B.normed.ptr, w[p + "in"], z, T);
        rec.gdn(T, S, B.spans.ptr, this.LH, this.rows, z, w[p + "conv"].ptr, w[p + "A_log"].ptr, w[p + "dt_bias"].ptr,
          w[p + "gnorm"].ptr, eps, B.y.ptr);
        rec.matmul(B.y.ptr, w[p + "out"], B.o.ptr, T);
      } else {
        rec.matmul(B.normed.ptr, w[p + "qkvg"], z, T);
        rec.qkNormRope(T, h, kv, D, A, z, w[p + "q_norm"].ptr, w[p + "k_norm"].ptr, false, B.pos.ptr, 1, eps, this.theta, this.rot,
          L.ROPE_POW_NEG);
        rec.attentionGated(T, h, kv, D, z, A, src, src, B.rng.ptr, 1 / Math.sqrt(D), B.z.at((h + 2 * kv) * D * 2), A, B.y.ptr);
        rec.matmul(B.y.ptr, w[p + "o"], B.o.ptr, T);
      }
      rec.addRmsnorm(T, H, true, eps, B.x.ptr, B.o.ptr, w[p + "post_norm"].ptr, B.normed.ptr);
      rec.matmulGlu(B.normed.ptr, w[p + "w13"], B.h.ptr, T, L.ACT_SILU);
      rec.matmul(B.h.ptr, w[p + "w2"], B.o.ptr, T);
    });
    rec.addRmsnorm(T, H, true, eps, B.x.ptr, B.o.ptr, w.final_norm.ptr, B.normed.ptr);
  }
}

module.exports = { D3Engine, gdnSpans };
