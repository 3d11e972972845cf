"use strict";
/* The Decision API of decision.js (d1.ts:38-227) on the Node host: D1.load, systemOne, systemOneBatch,
 * probabilities, probabilitiesBatch, destroy — the reference's names, argument meaning and error behaviour —
 * over the MI355X library. Calls are serialised on one queue (d1.ts:112-119): one forward in flight per
 * engine, and a failed call does not wedge the queue.
 *
 * Text-to-ids is upstream of the scoring path: `prompt` turns states and questions into token ids. The
 * default takes them already tokenized — a state is a list of ids; a question is the reference's question
 * plus `ids` (its tokens) and `options` (one token-id group per option, [yes, no] for a noul; each option
 * scores its best token, d1-3b-engine.ts:112-121); for EmbeddingGemma 2, `option_ids` (one token-id list per
 * option text, in the model's order: a noul as [no, yes], eg2-prompt.ts:27-33); for d1-omni, `markers` (each
 * option's marker position within the question's ids, in the model's order: a noul as [false, true]); for
 * Laya the same markers, the question's ids laid out as laya-prompt.ts does and read before the state's. */
const { DecoderEngine } = require("./engine");
const { EncoderEngine, cosineLogits } = require("./encoder");
const { OmniEngine, temperature: omniTemperature } = require("./omni");
const { LayaEngine } = require("./laya");
const { D3Engine } = require("./d3");
const { Eg2Engine } = require("./eg2");
const { criterion } = require("./py");
const { Eg2Head } = require("./eg2_head");
const { fileFetch } = require("./format");
const Q = require("./questions");

/** gpu.ts:294-297: max-subtracted exp (f64). */
function softmax(s) {
  const m = Math.max(...s);
  const e = s.map((x) => Math.exp(x - m));
  const z = e.reduce((a, b) => a + b, 0);
  return e.map((x) => x / z);
}

const idPrompt = {
  trunk: (state) => Array.from(state.ids || state, Number),
  branch: (q) => Array.from(q.ids, Number),
  readoutIds: (q) => {
    if (q.options.length !== Q.nOptions(q)) throw new Q.QuestionError(`decision.js: ${q.options.length} option groups for a ${q.type} with ${Q.nOptions(q)} options`);
    return q.options.map((g) => Array.from(g, Number));
  },
  // the encoder: state, question and each option are texts of their own (eg2-prompt.ts renders them)
  texts: (state, q) => [Array.from(state.ids || state, Number), Array.from(q.ids, Number), q.option_ids.map((o) => Array.from(o, Number))],
  // d1-omni: one sequence per question over its state (omni-prompt.ts:33-51 on ids), markers shifted past the state
  sequence: (state, q) => {
    const trunk = Array.from(state.ids || state, Number), ids = Array.from(q.ids, Number), markers = Array.from(q.markers, Number);
    if (markers.length !== Q.nOptions(q)) throw new Q.QuestionError(`decision.js: ${markers.length} markers for a ${q.type} with ${Q.nOptions(q)} options`);
    if (markers.some((m) => !(m >= 0 && m < ids.length))) throw new Q.QuestionError("decision.js: a marker outside the question's ids");
    return { ids: trunk.concat(ids), markers: markers.map((m) => trunk.length + m), type: q.type };
  },
  // Laya: the question's ids first ([CLS] question [SEP], [MASK] and tokens per option, [SEP]), then the state's
  // (laya-prompt.ts:27-56 on ids), the whole cut to maxLen; every option marker must fit
  sequenceLaya: (state, q, maxLen = 512) => {
    const trunk = Array.from(state.ids || state, Number), ids = Array.from(q.ids, Number), markers = Array.from(q.markers, Number);
    if (markers.length !== Q.nOptions(q)) throw new Q.QuestionError(`decision.js: ${markers.length} markers for a ${q.type} with ${Q.nOptions(q)} options`);
    if (markers.some((m) => !(m >= 0 && m < ids.length))) throw new Q.QuestionError("decision.js: a marker outside the question's ids");
    const fit = markers.filter((m) => m < maxLen).length;
    if (fit !== markers.length) throw new Q.QuestionError(`decision.js: only ${fit} of the ${markers.length} option markers fit in ${maxLen} tokens`);
    return { ids: ids.concat(trunk).slice(0, maxLen), markers, type: q.type };
  },
};

/** BatchOptions (d1.ts:33-35): {onProgress(done, total)}; a bare function is taken as that callback. */
const onProgressOf = (opts) => (typeof opts === "function" ? opts : opts && opts.onProgress);

/** The reference's ModelKind (d1.ts:17, 63-64) for a manifest: laya, d3, eg2 by name; d1-3b for a causal
 * decoder without marker heads (run as d1-3B's forest); else d1-omni. */
function kindOf(config) {
  const model = config && config.model;
  if (model === "laya") return "laya";
  if (model === "eg2" || model === "eg2-encoder") return "eg2";
  if (model === "d3") return "d3";
  if (model === "decoder" || model === "d1-3b" || !("head_layers" in (config || {}))) return "d1-3b";
  return "d1-omni";
}

class D1 {
  /** A model in the decision.js format at `base` (manifest.json + weights.bin). opts (LoadOptions, d1.ts:19-28;
   * gpu.ts:13-27): fetch (a Range-capable fetch; local files by default), device, onProgress, directWeights,
   * graphs, tokensPerPass (the reference's defaults: 4096 for d1-3b, 8192 otherwise), shareState, workflow,
   * prompt. */
  static async load(base, opts) {
    opts = Object.assign({}, opts || {});
    if (!base.endsWith("/")) base += "/";
    opts.fetch = opts.fetch || fileFetch();
    const manifest = await (await opts.fetch(`${base}manifest.json`)).json();
    const kind = kindOf(manifest.config);
    const engine = kind === "eg2" ? await ("ple" in manifest.config ? Eg2Engine : EncoderEngine).load(base, opts) // shipped / configs[0]
      : kind === "d1-omni" ? await OmniEngine.load(base, opts)
      : kind === "laya" ? await LayaEngine.load(base, opts)
      : kind === "d3" && "linear_heads" in manifest.config ? await D3Engine.load(base, opts) // the shipped d3-lite
      : await DecoderEngine.load(base, opts);
    return new D1(kind, engine, opts);
  }

  constructor(kind, engine, opts) {
    this.kind = kind;
    this.engine = engine;
    this.tokenizer = null; // text-to-ids is upstream of this build: `prompt` takes token ids
    this.prompt = opts.prompt || idPrompt;
    this.tokensPerPass = opts.tokensPerPass || (kind === "d1-3b" ? 4096 : 8192);
    this.shareState = !!opts.shareState; // can be switched between calls (d1.ts:51-52)
    this.workflow = opts.workflow || ""; // EmbeddingGemma 2: for a prompt that renders states (d1.ts:53-54)
    this.states = new Map(); // shareState: prefilled states by their ids, oldest dropped first
    this.embeddings = new Map(); // eg2: normalized embeddings of the texts seen so far (d1.ts:44)
    this.eg2Head = null;
    this.queue = Promise.resolve();
  }

  systemOne(state, questions) {
    return this.systemOneBatch([[state, questions]]).then((r) => r[0]);
  }

  systemOneBatch(requests, opts = {}) {
    return this.enqueue(async () => {
      const done = await this.runAll(requests.map(([s, qs]) => [s, Object.values(qs)]), onProgressOf(opts));
      const legend = this.kind === "d1-3b" ? String : criterion; // d1.ts:91
      return requests.map(([, qs], r) => {
        const names = Object.keys(qs), answers = {};
        names.forEach((n, j) => (answers[n] = Q.answer(qs[n], done[r].probs[j], legend)));
        return { answers, usage: { input_tokens: done[r].tokens, output_tokens: 0 } };
      });
    });
  }

  probabilities(state, questions) {
    return this.enqueue(async () => (await this.runAll([[state, Array.from(questions)]]))[0].probs);
  }

  probabilitiesBatch(requests, opts = {}) {
    return this.enqueue(async () => (await this.runAll(requests.map(([s, qs]) => [s, Array.from(qs)]), onProgressOf(opts))).map((r) => r.probs));
  }

  destroy() {
    for (const st of this.states.values()) this.engine.freeState(st);
    this.states.clear();
    this.engine.destroy();
  }

  enqueue(fn) {
    const run = this.queue.then(fn, fn);
    this.queue = run.then(() => undefined, () => undefined);
    return run;
  }

  async runAll(requests, onProgress) {
    for (const [, qs] of requests) qs.forEach(Q.checkQuestion);
    if (this.kind === "eg2") return this.runEg2(requests, onProgress);
    if (this.kind === "d3") return this.runD3(requests, onProgress);
    if (this.kind === "d1-omni" || this.kind === "laya") return this.runOmni(requests, onProgress);
    return this.shareState ? this.runShared(requests, onProgress) : this.runDecoder(requests, onProgress);
  }

  /** Whole requests per pass up to the token budget; a pass always takes at least one (d1.ts:217-219). */
  *passes(sizes) {
    let i = 0;
    while (i < sizes.length) {
      let j = i, used = 0;
      do {
        used += sizes[j++];
      } while (j < sizes.length && used + sizes[j] <= this.tokensPerPass);
      yield [i, j];
      i = j;
    }
  }

  /** run3B (d1.ts:211-226): a forest per request (the state as trunk, each question a branch). */
  async runDecoder(requests, onProgress) {
    const p = this.prompt;
    const trees = requests.map(([s, qs]) => ({ trunk: p.trunk(s), branches: qs.map(p.branch), groups: qs.map(p.readoutIds) }));
    const sizes = trees.map((t) => t.trunk.length + t.branches.reduce((a, b) => a + b.length, 0));
    const out = sizes.map((n) => ({ probs: [], tokens: n }));
    for (const [i, j] of this.passes(sizes)) {
      const { scores } = await this.engine.run(trees.slice(i, j));
      scores.forEach((perQ, r) => (out[i + r].probs = perQ.map(softmax)));
      if (onProgress) onProgress(j, trees.length);
    }
    return out;
  }

  /** Shared state: each request's state prefilled once and its K/V kept (reused by later calls on the same
   * state); the questions then run against it. */
  async runShared(requests, onProgress) {
    const p = this.prompt, out = [];
    for (let k = 0; k < requests.length; ++k) {
      const [s, qs] = requests[k];
      const trunk = p.trunk(s), key = trunk.join(",");
      let st = this.states.get(key);
      if (!st) {
        if (this.states.size >= 64) {
          const oldest = this.states.keys().next().value;
          this.engine.freeState(this.states.get(oldest));
          this.states.delete(oldest);
        }
        st = await this.engine.prefill(trunk);
        this.states.set(key, st);
      }
      const branches = qs.map(p.branch);
      const scores = await this.engine.runShared(st, branches, qs.map(p.readoutIds));
      out.push({ probs: scores.map(softmax), tokens: trunk.length + branches.reduce((a, b) => a + b.length, 0) });
      if (onProgress) onProgress(k + 1, requests.length);
    }
    return out;
  }

  /** runD3 (d1.ts:150-169): one sequence per question (the state's ids, then the question's), its first
   * n-options codes read at its last token; with shareState a request's common prefix (the state) is read once
   * for all its questions. Softmax at the model's temperature; a noul is read as [false, true], reversed. */
  async runD3(requests, onProgress) {
    const p = this.prompt, temp = this.engine.m.config.temperature === undefined ? 1 : this.engine.m.config.temperature;
    const seqs = requests.map(([s, qs]) => qs.map((q) => ({ ids: p.trunk(s).concat(p.branch(q)), options: Q.nOptions(q) })));
    const sizes = seqs.map((g) => g.reduce((a, x) => a + x.ids.length, 0));
    const out = sizes.map((n) => ({ probs: [], tokens: n }));
    for (const [i, j] of this.passes(sizes)) {
      const logits = await this.engine.logitsD3([].concat(...seqs.slice(i, j)), this.shareState ? seqs.slice(i, j).map((g) => g.length) : undefined);
      let k = 0;
      for (let r = i; r < j; ++r) {
        out[r].probs = requests[r][1].map((q) => {
          const pr = softmax(logits[k++].map((v) => v / temp));
          return q.type === "noul" ? pr.reverse() : pr;
        });
      }
      if (onProgress) onProgress(j, requests.length);
    }
    return out;
  }

  /** runEncoder (d1.ts:121-147) for d1-omni and Laya: one sequence per question (the state read anew for each;
   * Laya's puts the question first, cut to max_len), whole requests per pass up to the token budget; marker
   * logits over the question's temperature (type and option-count bucket), softmax, a noul read as
   * [false, true] and reversed to [yes, no]. */
  async runOmni(requests, onProgress) {
    const p = this.prompt, c = this.engine.m.config;
    const seqs = requests.map(([s, qs]) => qs.map((q) => (this.kind === "laya" ? p.sequenceLaya(s, q, c.max_len) : p.sequence(s, q))));
    const sizes = seqs.map((g) => g.reduce((a, x) => a + x.ids.length, 0));
    const out = sizes.map((n) => ({ probs: [], tokens: n }));
    for (const [i, j] of this.passes(sizes)) {
      const { logits } = await this.engine.logits([].concat(...seqs.slice(i, j)));
      let k = 0;
      for (let r = i; r < j; ++r) {
        out[r].probs = requests[r][1].map((q) => {
          const t = omniTemperature(c, q.type, Q.nOptions(q));
          const pr = softmax(logits[k++].map((v) => v / t));
          return q.type === "noul" ? pr.reverse() : pr;
        });
      }
      if (onProgress) onProgress(j, requests.length);
    }
    return out;
  }

  /** runEg2 (d1.ts:172-204): every distinct text (state, question, option) embedded once and cached, in passes
   * of at most tokensPerPass tokens; then the head on the host — the learned decision head when the model has
   * one (eg2-head.ts), else the cosine prior — and a softmax at the type's temperature. */
  async runEg2(requests, onProgress) {
    const p = this.prompt, c = this.engine.m.config;
    if (!this.eg2Head && c.head && Object.keys(this.engine.host).length) this.eg2Head = new Eg2Head(c, this.engine.host);
    const asked = requests.map(([s, qs]) => qs.map((q) => p.texts(s, q)));
    const todo = new Map(), tokens = requests.map(() => 0);
    asked.forEach((perQ, r) => {
      for (const [st, qi, opts] of perQ) {
        for (const t of [st, qi, ...opts]) {
          const key = t.join(",");
          if (this.embeddings.has(key) || todo.has(key)) continue;
          todo.set(key, t);
          tokens[r] += t.length;
        }
      }
    });
    const keys = Array.from(todo.keys());
    for (const [i, j] of keys.length ? this.passes(keys.map((k) => todo.get(k).length)) : []) {
      const { embeddings } = await this.engine.embed(keys.slice(i, j).map((k) => todo.get(k)));
      embeddings.forEach((e, k) => this.remember(keys[i + k], e));
      if (onProgress) onProgress(j, keys.length);
    }
    const temps = c.temperatures || {};
    const emb = (t) => [t.join(","), this.embeddings.get(t.join(","))];
    return requests.map(([, qs], r) => ({
      probs: qs.map((q, k) => {
        const [st, qi, opts] = asked[r][k];
        const z = this.eg2Head ? this.eg2Head.logits(q.type, emb(st), emb(qi), opts.map(emb))
          : cosineLogits(emb(st)[1], emb(qi)[1], opts.map((o) => emb(o)[1]));
        const tau = temps[q.type] === undefined ? 1 : temps[q.type];
        const pr = softmax(z.map((v) => v / tau));
        return q.type === "noul" ? pr.reverse() : pr; // the model reads a noul as [no, yes]
      }),
      tokens: tokens[r],
    }));
  }

  remember(key, e) {
    if (this.embeddings.size >= 8192) this.embeddings.delete(this.embeddings.keys().next().value); // the oldest text first (d1.ts:207)
    this.embeddings.set(key, e);
  }
}

module.exports = { D1, Decision: D1, softmax, idPrompt, kindOf };
