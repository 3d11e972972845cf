"use strict";
/* The Decision API of decision.js (d1.ts:38-227) on the Node host: D1.load, systemOne, systemOneBatch,
 * probabilities, probabilitiesBatch, destroy — the reference's names, argument meaning and error behaviour —
 * over the MI355X library. Calls are serialised on one queue (d1.ts:112-119): one forward in flight per
 * engine, and a failed call does not wedge the queue.
 *
 * Text-to-ids is upstream of the scoring path: `prompt` turns states and questions into token ids. The
 * default takes them already tokenized — a state is a list of ids; a question is the reference's question
 * plus `ids` (its tokens) and `options` (one token-id group per option, [yes, no] for a noul; each option
 * scores its best token, d1-3b-engine.ts:112-121). */
const { DecoderEngine } = require("./engine");
const { loadManifestSync } = require("./format");
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
};

class D1 {
  /** A model in the decision.js format at `base` (manifest.json + weights.bin). opts: fetch, device,
   * onProgress, directWeights, graphs, tokensPerPass (default 131072), shareState, prompt. */
  static async load(base, opts) {
    opts = opts || {};
    const model = opts.fetch ? null : loadManifestSync(base).config.model;
    if (model !== null && model !== "decoder" && model !== "d1-3b") {
      throw new Error(`decision.js: the Node host runs the causal decoders; ${base} is a ${model} model (use the Python host for encoders)`);
    }
    const engine = await DecoderEngine.load(base, opts);
    return new D1(engine, opts);
  }

  constructor(engine, opts) {
    this.engine = engine;
    this.prompt = opts.prompt || idPrompt;
    this.tokensPerPass = opts.tokensPerPass || 131072;
    this.shareState = !!opts.shareState;
    this.states = new Map(); // shareState: prefilled states by their ids, oldest dropped first
    this.queue = Promise.resolve();
  }

  systemOne(state, questions) {
    return this.systemOneBatch([[state, questions]]).then((r) => r[0]);
  }

  systemOneBatch(requests, onProgress) {
    return this.enqueue(async () => {
      const done = await this.runAll(requests.map(([s, qs]) => [s, Object.values(qs)]), onProgress);
      return requests.map(([, qs], r) => {
        const names = Object.keys(qs), answers = {};
        names.forEach((n, j) => (answers[n] = Q.answer(qs[n], done[r].probs[j])));
        return { answers, usage: { input_tokens: done[r].tokens, output_tokens: 0 } };
      });
    });
  }

  probabilities(state, questions) {
    return this.enqueue(async () => (await this.runAll([[state, Array.from(questions)]]))[0].probs);
  }

  probabilitiesBatch(requests, onProgress) {
    return this.enqueue(async () => (await this.runAll(requests.map(([s, qs]) => [s, Array.from(qs)]), onProgress)).map((r) => r.probs));
  }

  destroy() {
    for (const st of this.states.values()) st.free();
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
          this.states.get(oldest).free();
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
}

module.exports = { D1, softmax, idPrompt };
