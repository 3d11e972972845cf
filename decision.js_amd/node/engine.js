"use strict";
/* The causal decoder engine on the Node host (D13BEngine, d1-3b-engine.ts; shared state after d3-engine.ts):
 * forest packing on the host, the per-layer op sequence on a Recorder of the native library, answer-set
 * logits at each branch's last token. The same steps as decision_js_amd/engine.py, which the tests hold the
 * two hosts to (identical logits through the same library). */
const { Context, kvSrc, lib } = require("./dj");
const { loadWeights } = require("./format");

/** Device layout of a quantized tensor: the embedding (gathered, read as the LM head) stays plain, fused
 * gated-MLP inputs are interleaved for the GLU epilogue, other linears are repacked for the MFMA GEMM
 * (directWeights: dequantized once to f16 — gpu.ts:16-20, 114-133). */
function layoutFor(direct) {
  return (name) => {
    const L = lib();
    if (name === "embed" || name.startsWith("head.dense")) return L.W_PLAIN;
    const base = name.endsWith("w13") || name.endsWith(".gu") || name.endsWith(".wi") ? L.W_MFMA_GLU : L.W_MFMA;
    return direct ? base | L.W_DIRECT : base;
  };
}

/** Forest packing of D13BEngine.run (d1-3b-engine.ts:46-72): each tree's trunk once, each branch
 * continuing it; per token ids (u32), pos (branch positions continue after the trunk), and the attention key
 * ranges (a0, a1, b0, b1) equal to the forest mask of kernels.ts:135 — a trunk token i sees
 * [start, start+i+1), a branch token the trunk [start, start+P) and its branch up to itself; leaves = each
 * branch's last token; leafIds = the flattened option groups, zero-padded to nIds. */
function packForest(trees) {
  let T = 0;
  for (const t of trees) T += t.trunk.length + t.branches.reduce((a, b) => a + b.length, 0);
  const ids = new Uint32Array(T), pos = new Int32Array(T), rng = new Int32Array(T * 4), taps = new Int32Array(T * 4);
  const leaves = [], leafGroups = [];
  let off = 0;
  for (const tr of trees) {
    const start = off, P = tr.trunk.length;
    for (let i = 0; i < P; ++i, ++off) {
      ids[off] = tr.trunk[i];
      pos[off] = i;
      rng[4 * off] = start;
      rng[4 * off + 1] = start + i + 1;
      // the short conv's taps (d1-3b-engine.ts:56-64): trunk tokens i-2, i-1, i
      taps.set([i >= 2 ? start + i - 2 : -1, i >= 1 ? start + i - 1 : -1, start + i, 0], 4 * off);
    }
    tr.branches.forEach((br, b) => {
      const b0 = off;
      for (let o = 0; o < br.length; ++o, ++off) {
        ids[off] = br[o];
        pos[off] = P + o;
        rng.set([start, start + P, b0, off + 1], 4 * off);
        // back j tokens: within the branch, else into the end of the trunk, else none
        const back = (j) => (o - j >= 0 ? off - j : P + o - j >= 0 ? start + P + o - j : -1);
        taps.set([back(2), back(1), off, 0], 4 * off);
      }
      leaves.push(off - 1);
      leafGroups.push([].concat(...tr.groups[b]));
    });
  }
  const L = leaves.length;
  const nIds = leafGroups.reduce((a, g) => Math.max(a, g.length), 0);
  const leafIds = new Uint32Array(Math.max(L * nIds, 1));
  leafGroups.forEach((g, k) => leafIds.set(g, k * nIds));
  return { ids, pos, rng, taps, leaves: Uint32Array.from(leaves), leafIds, nIds, T, L };
}

/** The common token prefix of a request's sequences, leaving at least one token per sequence (d3-engine.ts:76-80). */
function commonPrefix(seqs) {
  if (seqs.length < 2) return 0;
  const lim = Math.min(...seqs.map((s) => s.length)) - 1;
  let P = 0;
  while (P < lim && seqs.every((s) => s[P] === seqs[0][P])) ++P;
  return P;
}

/** D3Engine.logits's packing (d3-engine.ts:67-93): seqs [{ids, options}], groups (sequences per request,
 * consecutive; undefined: each alone). A request's common prefix is laid once as a trunk whose tokens see the
 * trunk; each question's remaining tokens see the trunk and themselves; without a prefix a sequence sees
 * itself. Positions are indices within the original sequence; pairs = (the question's last row, code k). */
function packShared(seqs, groups) {
  const sizes = groups || seqs.map(() => 1);
  if (sizes.reduce((a, b) => a + b, 0) !== seqs.length) throw new Error(`decision.js: groups cover ${sizes.reduce((a, b) => a + b, 0)} sequences, ${seqs.length} given`);
  const ids = [], pos = [], rng = [], pairs = [];
  let si = 0;
  for (const n of sizes) {
    const group = seqs.slice(si, si + n);
    si += n;
    const P = n > 1 ? commonPrefix(group.map((s) => s.ids)) : 0;
    const ts = ids.length;
    for (let i = 0; i < P; ++i) {
      ids.push(group[0].ids[i]);
      pos.push(i);
      rng.push(ts, ts + P, 0, 0);
    }
    for (const s of group) {
      const bs = ids.length, be = bs + s.ids.length - P;
      for (let i = P; i < s.ids.length; ++i) {
        ids.push(s.ids[i]);
        pos.push(i);
        if (P) rng.push(ts, ts + P, bs, be);
        else rng.push(bs, be, 0, 0);
      }
      for (let k = 0; k < s.options; ++k) pairs.push(be - 1, k);
    }
  }
  return { ids: Uint32Array.from(ids), pos: Int32Array.from(pos), rng: Int32Array.from(rng), pairs: Uint32Array.from(pairs),
    T: ids.length, P: pairs.length / 2 };
}

/** Readout of d1-3b-engine.ts:112-121: each option scores the max over its token group. */
function groupMax(out, nIds, trees) {
  const scores = [];
  let leaf = 0;
  for (const tr of trees) {
    const perQ = [];
    for (const groups of tr.groups) {
      let j = 0;
      const s = [];
      for (const g of groups) {
        let best = -Infinity;
        for (let k = 0; k < g.length; ++k) best = Math.max(best, out[leaf * nIds + j + k]);
        s.push(best);
        j += g.length;
      }
      perQ.push(s);
      ++leaf;
    }
    scores.push(perQ);
  }
  return scores;
}

// Graph keys come from one process-wide counter: every distinct forward (its exact key string, on any engine)
// gets its own 64-bit number, so two forwards never share a cached graph and a dropped key is never reused.
let nextGraphKey = 0n;
let stateSerial = 0;

class GpuEngine {
  constructor(ctx, m, w, opts) {
    this.ctx = ctx;
    this.m = m;
    this.w = w;
    this.opts = opts || {};
    this.graphs = this.opts.graphs === undefined ? true : !!this.opts.graphs;
    this.stats = { forwards: 0, tokens: 0 };
    this.bufs = {};
    this.gen = 0;
    this.keys = new Map(); // key string -> 0n after its first use, its graph key from the second use on
    this.stateKeys = new Map(); // shared state serial -> graph keys of the forwards reading its K/V
    this.ownsCtx = !this.opts.device;
  }
  /** Frees every weight and buffer (gpu.ts:108-110). */
  destroy() {
    for (const b of Object.values(this.bufs)) b.free();
    this.bufs = {};
    for (const v of Object.values(this.w)) v.free();
    this.w = {};
    if (this.ownsCtx) this.ctx.close();
  }
  alloc(spec) {
    for (const b of Object.values(this.bufs)) b.free();
    this.bufs = {};
    for (const [k, n] of Object.entries(spec)) this.bufs[k] = this.ctx.alloc(n);
    this.gen += 1;
    this.ctx.graphClear();
  }
  // The graph key of a forward, from its second use on: the first forward with a key runs eagerly (0n), the
  // second captures the graph, later ones replay it (capturing costs more than launching once). `state`: the
  // serial of the shared state whose K/V the forward reads (its graphs are dropped with the state). The library
  // keeps at most DJ_GRAPH_CAP graphs; forgetting a key string here only costs a new capture.
  key(parts, state) {
    if (!this.graphs) return 0n;
    const t = JSON.stringify([this.gen, state === undefined ? null : state].concat(parts));
    let k = this.keys.get(t);
    if (k === undefined) {
      if (this.keys.size >= 4096) this.keys.clear();
      this.keys.set(t, 0n);
      return 0n;
    }
    if (k === 0n) {
      k = ++nextGraphKey;
      this.keys.set(t, k);
      if (state !== undefined) {
        if (!this.stateKeys.has(state)) this.stateKeys.set(state, []);
        this.stateKeys.get(state).push(k);
      }
    }
    return k;
  }
  /** Frees a shared state's kept K/V and drops the graphs captured against it (they point at its memory). */
  freeState(st) {
    for (const k of this.stateKeys.get(st.serial) || []) this.ctx.graphDrop(k);
    this.stateKeys.delete(st.serial);
    for (const t of Array.from(this.keys.keys())) if (JSON.parse(t)[1] === st.serial) this.keys.delete(t);
    st.free();
  }
}

class SharedState {
  constructor(P, cache, ids) {
    this.P = P;
    this.cache = cache;
    this.ids = ids;
    this.serial = ++stateSerial;
  }
  free() {
    this.cache.free();
  }
}

const INPUTS = ["ids", "pos", "rng", "leaves", "leafIds"];

class DecoderEngine extends GpuEngine {
  static async load(base, opts) {
    opts = opts || {};
    const direct = !!(opts.directWeights || opts.direct_weights);
    const { ctx, m, w } = await loadWeights(base, opts, layoutFor(direct));
    const model = m.config.model;
    if (model !== "decoder" && model !== "d1-3b" && model !== "d3") throw new Error(`decision.js: ${base} is not a decoder (${model})`);
    const bad = (m.config.layer_types || []).filter((t) => t !== "full_attention" && t !== "conv");
    if (bad.length) throw new Error(`decision.js: unsupported layer types ${JSON.stringify(Array.from(new Set(bad)).sort())} (attention and LFM2 conv layers run here)`);
    return new DecoderEngine(ctx, m, w, opts);
  }

  constructor(ctx, m, w, opts) {
    super(ctx, m, w, opts);
    const c = m.config;
    Object.assign(this, { H: c.hidden, I: c.intermediate, h: c.heads, kv: c.kv_heads, D: c.head_dim, eps: c.eps, theta: c.rope_theta });
    this.layers = c.layers !== undefined ? c.layers : (c.layer_types || []).length;
    this.types = c.layer_types || new Array(this.layers).fill("full_attention");
    this.conv = this.types.includes("conv");
    this.stride = (this.h + 2 * this.kv) * this.D;
    this.capacity = 0;
    this.leafCapacity = 0;
    // the residual + RMSNorm between products folded into them on forwards of fusedRows rows (as the Python
    // host): opts.fusedNorms, else DJ_FUSED_NORMS=0/1, else the class's fusedDefault
    const fo = this.opts.fusedNorms !== undefined ? this.opts.fusedNorms : this.opts.fused_norms;
    const env = process.env.DJ_FUSED_NORMS;
    const want = fo !== undefined ? !!fo : env !== undefined ? env !== "0" : this.constructor.fusedDefault;
    this.fusedNorms = want && this.H % 128 === 0 && this.H <= 1024;
    // a short question on a kept state (up to 64 rows): q/k norm + RoPE in the attention kernel
    // (dj_attention_qk_rope) after a plain qkv product: opts.qkAttention, else DJ_ATTN_QK_ROPE=0/1, else on
    const qo = this.opts.qkAttention !== undefined ? this.opts.qkAttention : this.opts.qk_attention;
    const qenv = process.env.DJ_ATTN_QK_ROPE;
    this.qkAttention = (qo !== undefined ? !!qo : qenv !== undefined ? qenv !== "0" : true) && this.D === 128;
  }

  /** The folded norms' buffers: the norm-weighted residual rows and their per-32-column sums of squares. */
  normBufs(cap) {
    return this.fusedNorms ? { xw: cap * this.H * 2, ss: cap * (this.H / 32) * 4 } : {};
  }

  /** Activation buffers, grown and never shrunk, capacity rounded to 64 rows (d1-3b-engine.ts:33-42). */
  ensure(T, L = 0, nIds = 0) {
    if (T <= this.capacity && L * Math.max(nIds, 1) <= this.leafCapacity) return;
    let cap = Math.max(T, this.capacity, 256);
    cap = Math.ceil(cap / 64) * 64;
    const lcap = Math.max(L * Math.max(nIds, 1), this.leafCapacity, 1024);
    const { H, I } = this;
    const zw = Math.max(this.stride, this.conv ? 3 * H : 0), yw = Math.max(this.h * this.D, this.conv ? H : 0);
    this.alloc({ x: cap * H * 2, normed: cap * H * 2, o: cap * H * 2, z: cap * zw * 2, y: cap * yw * 2,
      h: cap * I * 2, ids: cap * 4, pos: cap * 4, rng: cap * 16, taps: cap * 16, rope: cap * (this.D / 2) * 8,
      leaves: lcap * 4, leafIds: lcap * 4, out: lcap * 4, ...this.normBufs(cap) });
    this.capacity = cap;
    this.leafCapacity = lcap;
  }

  /** The per-layer loop (d1-3b-engine.ts:88-105) on the recorder; on more than 64 rows the norms between
   * products are folded into them (dj_matmul_residual / dj_matmul_normed), as the Python host does. */
  recordLayers(rec, T, B, kvA, kvStore) {
    const w = this.w, L = lib();
    const { H, h, kv, D, eps } = this;
    const z = B.z.ptr;
    const src = kvSrc(z, T, this.stride, h * D, (h + kv) * D);
    const ptr = (name) => (w[name] ? w[name].ptr : 0n);
    rec.gatherQ(B.ids.ptr, T, w.embed, B.x.ptr);
    rec.addRmsnorm(T, H, false, eps, B.x.ptr, B.o.ptr, ptr("layers.0.operator_norm"), B.normed.ptr);
    // the RoPE angles of this forward, once; every layer's qkv product applies q/k norm + RoPE with them
    rec.ropeTable(T, B.pos.ptr, 1, this.theta, D, B.rope.ptr, L.ROPE_POW_NEG);
    const [lo, hi] = this.constructor.fusedRows;
    const fused = this.fusedNorms && T >= lo && T <= hi && !!B.xw;
    let pending = false; // the next product reads B.xw / B.ss (a folded norm) instead of B.normed
    const qkAttention = this.qkAttention && T <= 64 && !!kvA && !kvStore && !fused;
    for (let i = 0; i < this.layers; ++i) {
      const p = `layers.${i}.`;
      let second;
      if (this.types[i] === "conv") { // LFM2 short conv (d1-3b-engine.ts:90-93)
        if (pending) rec.matmulNormed(B.xw.ptr, w[p + "in_proj"], z, T, -1, B.ss.ptr, H, eps);
        else rec.matmul(B.normed.ptr, w[p + "in_proj"], z, T);
        rec.shortConv(T, H, z, ptr(p + "conv"), B.taps.ptr, B.y.ptr);
        second = w[p + "out_proj"];
      } else if (qkAttention) { // the kept state's keys are rotated already; the question's own are raw
        rec.matmul(B.normed.ptr, w[p + "qkv"], z, T);
        rec.attentionQkRope(T, h, kv, D, z, this.stride, kvA(i), src, B.rng.ptr, 1 / Math.sqrt(D), ptr(p + "q_norm"),
          ptr(p + "k_norm"), eps, B.rope.ptr, B.y.ptr);
        second = w[p + "o_proj"];
      } else {
        if (pending)
          rec.matmulQkvRopeNormed(B.xw.ptr, w[p + "qkv"], z, T, h, kv, D, ptr(p + "q_norm"), ptr(p + "k_norm"), false, B.pos.ptr, 1,
            eps, this.theta, B.rope.ptr, B.ss.ptr, H, eps, D, L.ROPE_POW_NEG);
        else
          rec.matmulQkvRope(B.normed.ptr, w[p + "qkv"], z, T, h, kv, D, ptr(p + "q_norm"), ptr(p + "k_norm"), false, B.pos.ptr, 1,
            eps, this.theta, B.rope.ptr, D, L.ROPE_POW_NEG);
        if (kvStore) rec.kvStore(T, kv, D, z, this.stride, h * D, kvStore.at(i * T * 2 * kv * D * 2), 0);
        rec.attention(T, h, kv, D, z, this.stride, kvA ? kvA(i) : src, src, B.rng.ptr, 1 / Math.sqrt(D), B.y.ptr);
        second = w[p + "o_proj"];
      }
      if (fused) {
        rec.matmulResidual(B.y.ptr, second, T, B.x.ptr, ptr(p + "ffn_norm"), B.xw.ptr, B.ss.ptr);
        rec.matmulNormed(B.xw.ptr, w[p + "w13"], B.h.ptr, T, L.ACT_SILU, B.ss.ptr, H, eps);
      } else {
        rec.matmul(B.y.ptr, second, B.o.ptr, T);
        rec.addRmsnorm(T, H, true, eps, B.x.ptr, B.o.ptr, ptr(p + "ffn_norm"), B.normed.ptr);
        rec.matmulGlu(B.normed.ptr, w[p + "w13"], B.h.ptr, T, L.ACT_SILU);
      }
      const last = i + 1 === this.layers;
      if (fused && !last) {
        rec.matmulResidual(B.h.ptr, w[p + "w2"], T, B.x.ptr, ptr(`layers.${i + 1}.operator_norm`), B.xw.ptr, B.ss.ptr);
        pending = true;
      } else {
        rec.matmul(B.h.ptr, w[p + "w2"], B.o.ptr, T);
        rec.addRmsnorm(T, H, true, eps, B.x.ptr, B.o.ptr, ptr(last ? "final_norm" : `layers.${i + 1}.operator_norm`), B.normed.ptr);
        pending = false;
      }
    }
  }

  async finish(rec, T) {
    const got = await rec.finish();
    this.stats.forwards += 1;
    this.stats.tokens += T;
    return got;
  }

  /** Option scores for every question of every tree: [tree][question][option], plus the raw logits. */
  async run(trees) {
    const pk = packForest(trees);
    if (pk.T === 0) return { scores: trees.map(() => []), logits: new Float32Array(0) };
    const { T, L, nIds } = pk;
    this.ensure(T, L, nIds);
    const B = this.bufs;
    B.ids.upload(pk.ids);
    B.pos.upload(pk.pos);
    B.rng.upload(pk.rng);
    B.taps.upload(pk.taps);
    if (L) {
      B.leaves.upload(pk.leaves);
      B.leafIds.upload(pk.leafIds);
    }
    const rec = this.ctx.recorder(this.key(["run", T, L, nIds]));
    const oi = rec.record(() => { // aborted on an error
      if (!rec.replay) {
        this.recordLayers(rec, T, B, null, null);
        if (L && nIds) rec.leafLogits(T, L, this.H, nIds, this.eps, B.x.ptr, B.leaves.ptr, this.w.final_norm.ptr, B.leafIds.ptr, this.w.embed, B.out.ptr);
      }
      return L && nIds ? rec.snapshot(B.out.ptr, Float32Array, L * nIds) : -1;
    });
    const got = await this.finish(rec, T);
    const out = oi >= 0 ? got[oi] : new Float32Array(0);
    return { scores: groupMax(out, nIds, trees), logits: out };
  }

  /** d3's code logits per question ([seq][its options codes], before the temperature; D3Engine.logits,
   * d3-engine.ts:67-139): packShared's ranges on every layer, the final norm, then READOUT of each question's
   * last row against the model's f32 `readout` matrix [codes, hidden] (d3-kernels.ts:242-260). */
  noConv(what) {
    if (this.conv) throw new Error(`decision.js: ${what} is not available for models with LFM2 conv layers (their taps would need each state's last conv inputs): use run()`);
  }

  async logitsD3(seqs, groups) {
    if (!this.w.readout) throw new Error("decision.js: this model has no code readout (a d3 export's `readout` matrix)");
    this.noConv("d3's code readout");
    const pk = packShared(seqs, groups);
    const { T, P } = pk;
    if (T === 0) return seqs.map(() => []);
    this.ensure(T, P, 2); // leafIds holds the pairs (2 u32 each), out the P logits
    const B = this.bufs;
    B.ids.upload(pk.ids);
    B.pos.upload(pk.pos);
    B.rng.upload(pk.rng);
    if (P) B.leafIds.upload(pk.pairs);
    const R = this.w.readout, codes = this.m.tensors.readout.shape[0];
    const rec = this.ctx.recorder(this.key(["d3", T, P]));
    const oi = rec.record(() => { // aborted on an error
      if (!rec.replay) {
        this.recordLayers(rec, T, B, null, null);
        if (P) rec.readout(T, P, this.H, B.normed.ptr, R.ptr, codes, B.leafIds.ptr, B.out.ptr);
      }
      return P ? rec.snapshot(B.out.ptr, Float32Array, P) : -1;
    });
    const got = await this.finish(rec, T);
    const out = oi >= 0 ? got[oi] : new Float32Array(0);
    let k = 0;
    return seqs.map((s) => Array.from(out.subarray(k, (k += s.options))));
  }

  /** Runs the state alone (causal) and keeps every layer's K/V rows on the device. */
  async prefill(trunk) {
    const P = trunk.length;
    if (P === 0) throw new Error("decision.js: an empty state has nothing to prefill");
    this.noConv("a kept shared state");
    this.ensure(P);
    const B = this.bufs;
    const pos = new Int32Array(P), rng = new Int32Array(P * 4);
    for (let i = 0; i < P; ++i) {
      pos[i] = i;
      rng[4 * i + 1] = i + 1;
    }
    B.ids.upload(Uint32Array.from(trunk));
    B.pos.upload(pos);
    B.rng.upload(rng);
    const cache = this.ctx.alloc(this.layers * P * 2 * this.kv * this.D * 2);
    try {
      const rec = this.ctx.recorder(0n); // the cache pointer is new each time: no graph
      rec.record(() => this.recordLayers(rec, P, B, null, cache));
      await this.finish(rec, P);
    } catch (e) {
      cache.free();
      throw e;
    }
    return new SharedState(P, cache, trunk.slice());
  }

  /** Scores of each branch continuing a prefilled state (its K/V reused; positions continue after it). */
  async runShared(state, branches, groups) {
    const P = state.P;
    const T = branches.reduce((a, b) => a + b.length, 0);
    if (T === 0) return branches.map(() => []);
    const ids = new Uint32Array(T), pos = new Int32Array(T), rng = new Int32Array(T * 4);
    const leaves = [], leafGroups = [];
    let off = 0;
    branches.forEach((br, b) => {
      const b0 = off;
      for (let o = 0; o < br.length; ++o, ++off) {
        ids[off] = br[o];
        pos[off] = P + o;
        rng.set([0, P, b0, off + 1], 4 * off);
      }
      leaves.push(off - 1);
      leafGroups.push([].concat(...groups[b]));
    });
    const L = leaves.length, nIds = leafGroups.reduce((a, g) => Math.max(a, g.length), 0);
    const leafIds = new Uint32Array(L * nIds);
    leafGroups.forEach((g, k) => leafIds.set(g, k * nIds));
    this.ensure(T, L, nIds);
    const B = this.bufs;
    B.ids.upload(ids);
    B.pos.upload(pos);
    B.rng.upload(rng);
    B.leaves.upload(Uint32Array.from(leaves));
    B.leafIds.upload(leafIds);
    const width = 2 * this.kv * this.D;
    const rec = this.ctx.recorder(this.key(["shared", T, L, nIds], state.serial));
    const oi = rec.record(() => {
      if (!rec.replay) {
        this.recordLayers(rec, T, B, (i) => kvSrc(state.cache.at(i * P * width * 2), P, width, 0, this.kv * this.D), null);
        rec.leafLogits(T, L, this.H, nIds, this.eps, B.x.ptr, B.leaves.ptr, this.w.final_norm.ptr, B.leafIds.ptr, this.w.embed, B.out.ptr);
      }
      return rec.snapshot(B.out.ptr, Float32Array, L * nIds);
    });
    const out = (await this.finish(rec, T))[oi];
    return groupMax(out, nIds, [{ groups }])[0];
  }
}

// where the folded norms pay (measured: a 3 x 384-id ticket gains, an 86k-row batch loses)
DecoderEngine.fusedDefault = true;
DecoderEngine.fusedRows = [65, 8192];

module.exports = { packForest, packShared, commonPrefix, groupMax, GpuEngine, SharedState, DecoderEngine, layoutFor, Context };
