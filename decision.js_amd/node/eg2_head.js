"use strict";
/* The decision head of the EmbeddingGemma 2 typed-decision model (Eg2Head, eg2-head.ts:44-100) on the Node host,
 * in f32 storage with double arithmetic, as the reference's host code:
 *   f = LayerNorm(field([S, Q, S*Q]) + type)        S, Q, O: the state, question and option embeddings, projected
 *   logit_i = prior * cos(o_i, s + q) + gate * (joint * cos(f, LayerNorm(O_i)) + residual([f, On, f*On, |f - On|]))
 * The projections of a text depend on that text only and are cached with it (4096 per cache, oldest first).
 * decision_js_amd/eg2_head.py is the same head on the Python host; the tests hold the two to each other. */
const QTYPES = ["choice", "score", "noul"];
const CACHE = 4096;

/** y = W[:, from:from+cols] x + b for W [out, stride] row-major, stored f32 (eg2-head.ts:11-20). */
function linear(W, b, x, out, from = 0, cols = x.length, stride = x.length) {
  const y = new Float32Array(out);
  for (let o = 0; o < out; o++) {
    let s = b ? b[o] : 0;
    const r = o * stride + from;
    for (let k = 0; k < cols; k++) s += W[r + k] * x[k];
    y[o] = s;
  }
  return y;
}

/** Abramowitz & Stegun 7.1.26, |error| < 1.5e-7. */
function erf(x) {
  const t = 1 / (1 + 0.3275911 * Math.abs(x));
  const y = 1 - ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t * Math.exp(-x * x);
  return x >= 0 ? y : -y;
}
const gelu = (x) => 0.5 * x * (1 + erf(x / Math.SQRT2));

function layerNorm(x, w, b, eps) {
  let m = 0, v = 0;
  for (const a of x) m += a;
  m /= x.length;
  for (const a of x) v += (a - m) * (a - m);
  const inv = 1 / Math.sqrt(v / x.length + eps);
  return x.map((a, i) => (a - m) * inv * w[i] + b[i]);
}

const dot = (a, b) => {
  let s = 0;
  for (let i = 0; i < a.length; i++) s += a[i] * b[i];
  return s;
};
const norm = (a) => Math.sqrt(dot(a, a));

class Eg2Head {
  /** `config` the manifest config (its `head`: width, ln_eps, prior_scale, joint_scale, gate, residual_bias);
   * `t` the head's f32 tensors by name (the manifest's `host` list). */
  constructor(config, t) {
    this.h = config.head;
    this.W = config.head.width;
    this.t = t;
    this.projS = new Map();
    this.projQ = new Map();
    this.terms = new Map();
  }

  cached(map, key, make) {
    let v = map.get(key);
    if (v === undefined) {
      if (map.size >= CACHE) map.delete(map.keys().next().value); // the oldest text first
      map.set(key, (v = make()));
    }
    return v;
  }

  /** The raw logit of every option: s, q, opts are [key, normalized embedding] of the state, question, options. */
  logits(type, s, q, opts) {
    const { t, W, h } = this;
    const S = this.cached(this.projS, s[0], () => linear(t["head.state_proj.weight"], t["head.state_proj.bias"], s[1], W));
    const Q = this.cached(this.projQ, q[0], () => linear(t["head.question_proj.weight"], t["head.question_proj.bias"], q[1], W));
    const fin = new Float32Array(3 * W);
    fin.set(S, 0);
    fin.set(Q, W);
    for (let i = 0; i < W; i++) fin[2 * W + i] = S[i] * Q[i];
    const f1 = linear(t["head.field.0.weight"], t["head.field.0.bias"], fin, W).map(gelu);
    const f2 = linear(t["head.field.3.weight"], t["head.field.3.bias"], f1, W);
    const type0 = QTYPES.indexOf(type) * W, emb = t["head.type_emb.weight"];
    for (let i = 0; i < W; i++) f2[i] += emb[type0 + i];
    const f = layerNorm(f2, t["head.field_norm.weight"], t["head.field_norm.bias"], h.ln_eps);
    const fNorm = norm(f);
    const R0 = t["head.residual.0.weight"], rb = t["head.residual.0.bias"], R3 = t["head.residual.3.weight"];
    const rf = linear(R0, rb, f, W, 0, W, 4 * W);
    const anchor = new Float32Array(s[1].length);
    for (let i = 0; i < anchor.length; i++) anchor[i] = s[1][i] + q[1][i];
    const an = Math.max(norm(anchor), 1e-12);
    return opts.map(([key, e]) => {
      const o = this.cached(this.terms, key, () => {
        const O = linear(t["head.option_proj.weight"], t["head.option_proj.bias"], e, W);
        const on = layerNorm(O, t["head.option_norm.weight"], t["head.option_norm.bias"], h.ln_eps);
        const en = Math.max(norm(e), 1e-12);
        return { o: Float32Array.from(e, (v) => v / en), on, onNorm: norm(on), r: linear(R0, undefined, on, W, W, W, 4 * W) };
      });
      const prod = new Float32Array(W), diff = new Float32Array(W);
      for (let i = 0; i < W; i++) {
        prod[i] = f[i] * o.on[i];
        diff[i] = Math.abs(f[i] - o.on[i]);
      }
      const rm = linear(R0, undefined, prod, W, 2 * W, W, 4 * W), ra = linear(R0, undefined, diff, W, 3 * W, W, 4 * W);
      let res = h.residual_bias;
      for (let i = 0; i < W; i++) res += R3[i] * gelu(rf[i] + o.r[i] + rm[i] + ra[i]);
      const joint = h.joint_scale * dot(f, o.on) / Math.max(fNorm * o.onNorm, 1e-8);
      const prior = h.prior_scale * dot(o.o, anchor) / an;
      return prior + h.gate * (joint + res);
    });
  }
}

module.exports = { Eg2Head, QTYPES };
