"use strict";
/* Test driver for the Node host: one JSON request on stdin, one JSON result on stdout (tests/test_node.py
 * compares it with the Python host and the oracle). */
const path = require("path");
const root = path.join(__dirname, "..", "..", "decision.js_amd", "node");
const host = require(root);

const typed = (a) => Array.from(a);

async function main(req) {
  switch (req.cmd) {
    case "exports":
      return Object.keys(host.dj.lib());
    case "pack": {
      const pk = host.packForest(req.trees);
      return { ids: typed(pk.ids), pos: typed(pk.pos), rng: typed(pk.rng), taps: typed(pk.taps), leaves: typed(pk.leaves), leafIds: typed(pk.leafIds), nIds: pk.nIds, T: pk.T, L: pk.L };
    }
    case "groupmax":
      return host.groupMax(req.out, req.nIds, req.trees);
    case "answer":
      return req.items.map(([q, probs]) => {
        try {
          host.questions.checkQuestion(q);
          return host.questions.answer(q, probs);
        } catch (e) {
          return { error: e.message };
        }
      });
    case "graphkeys": {
      // graph keys handed out over a sequence of forwards, then a shared state freed (no device: key() reads
      // only the engine's own state; a stand-in context records the dropped graphs)
      const { GpuEngine } = require(path.join(root, "engine"));
      const dropped = [];
      const e = new GpuEngine({ graphDrop: (k) => dropped.push(String(k)) }, {}, {}, { graphs: req.graphs });
      const keys = req.seq.map(([parts, st]) => String(e.key(parts, st === null ? undefined : st)));
      e.freeState({ serial: req.free, free: () => undefined });
      const again = req.seq.find(([, st]) => st === req.free);
      return { keys, dropped, after: String(e.key(again[0], req.free)) };
    }
    case "d3": {
      const d = await host.Decision.load(req.model, req.opts || {});
      try {
        const reqs = req.batch.map(([s, qs]) => [s, Object.values(qs)]);
        const out = { kind: d.kind };
        out.plain = await d.probabilitiesBatch(reqs);
        d.shareState = true;
        out.shared = await d.probabilitiesBatch(reqs);
        return out;
      } finally {
        d.destroy();
      }
    }
    case "question": {
      // one short question on a prefilled state, through DecoderEngine.runShared: its scores on three runs
      // (eager, capture, replay)
      const e = await host.DecoderEngine.load(req.model, req.opts || {});
      try {
        const st = await e.prefill(req.state);
        const runs = [];
        for (let k = 0; k < 3; ++k) runs.push(await e.runShared(st, req.branches, req.groups));
        e.freeState(st);
        return { qkAttention: e.qkAttention, runs };
      } finally {
        e.destroy();
      }
    }
    case "logits": {
      const e = await host.DecoderEngine.load(req.model, req.opts || {});
      try {
        return { logits: typed((await e.run(req.trees)).logits) };
      } finally {
        e.destroy();
      }
    }
    case "packshared": {
      const pk = host.packShared(req.seqs, req.groups === null ? undefined : req.groups);
      return { ids: typed(pk.ids), pos: typed(pk.pos), rng: typed(pk.rng), pairs: typed(pk.pairs), T: pk.T, P: pk.P };
    }
    case "gdnspans":
      return typed(host.gdnSpans(req.seqs, req.groups === null ? undefined : req.groups));
    case "packomni": {
      const pk = host.packOmni(req.seqs);
      const out = { T: pk.T, M: pk.M };
      for (const k of ["ids", "pos", "qtype", "taps", "rng", "markers"]) out[k] = typed(pk[k]);
      return out;
    }
    case "packlaya": {
      const pk = host.packLaya(req.seqs, req.window);
      const out = { T: pk.T, M: pk.M };
      for (const k of ["ids", "pos", "qtype", "rng", "win", "markers"]) out[k] = typed(pk[k]);
      return out;
    }
    case "layaprompt":
      return req.calls.map(([state, q, maxLen]) => {
        try {
          return require(path.join(root, "d1")).idPrompt.sequenceLaya(state, q, maxLen);
        } catch (e) {
          return { error: e.message };
        }
      });
    case "omni": {
      const d = await host.Decision.load(req.model, req.opts || {});
      try {
        const out = { kind: d.kind };
        out.batch = await d.systemOneBatch(req.batch);
        out.logits = (await d.engine.logits(req.seqs)).logits;
        return out;
      } finally {
        d.destroy();
      }
    }
    case "packenc": {
      const pk = host.packEncoder(req.seqs);
      return { ids: typed(pk.ids), meta: typed(pk.meta), full: typed(pk.full), ranges: typed(pk.ranges), T: pk.T, S: pk.S };
    }
    case "eg2head": {
      // the learned head on given tensors and embeddings (no device)
      const t = {};
      for (const [k, v] of Object.entries(req.tensors)) t[k] = Float32Array.from(v);
      const head = new host.Eg2Head(req.config, t);
      return req.calls.map(([type, s, q, opts]) => head.logits(type, [s[0], Float32Array.from(s[1])], [q[0], Float32Array.from(q[1])],
        opts.map(([k, e]) => [k, Float32Array.from(e)])));
    }
    case "kinds":
      return req.configs.map((c) => {
        try {
          return require(path.join(root, "d1")).kindOf(c);
        } catch (e) {
          return { error: e.message };
        }
      });
    case "encode": {
      const d = await host.Decision.load(req.model, req.opts || {});
      try {
        const out = { kind: d.kind, tokensPerPass: d.tokensPerPass };
        const seen = [];
        out.batch = await d.systemOneBatch(req.batch, { onProgress: (a, b) => seen.push([a, b]) });
        out.progress = seen;
        out.again = await d.systemOneBatch(req.batch); // every text cached: no forward
        out.embeddings = (await d.engine.embed(req.texts)).embeddings.map(typed);
        return out;
      } finally {
        d.destroy();
      }
    }
    case "fault": {
      // the test sets DJ_FAULT_INJECT=<op>:1 in this process's environment: the first forward fails
      const d = await host.D1.load(req.model, req.opts || {});
      try {
        const out = {};
        try {
          await d.probabilities(req.state, Object.values(req.questions));
        } catch (e) {
          out.error = e.message;
        }
        out.after = await d.probabilities(req.state, Object.values(req.questions));
        out.again = await d.probabilities(req.state, Object.values(req.questions));
        return out;
      } finally {
        d.destroy();
      }
    }
    case "passes": {
      const d = Object.create(host.D1.prototype);
      d.tokensPerPass = req.budget;
      return Array.from(d.passes(req.sizes));
    }
    case "load": {
      try {
        const d = await host.D1.load(req.model, req.opts || {});
        d.destroy();
        return { ok: true };
      } catch (e) {
        return { error: e.message };
      }
    }
    case "decide": {
      const d = await host.D1.load(req.model, req.opts || {});
      try {
        const out = { one: await d.systemOne(req.state, req.questions) };
        out.probs = await d.probabilities(req.state, Object.values(req.questions));
        out.again = await d.systemOne(req.state, req.questions); // a replayed graph
        try {
          await d.systemOne(req.state, { bad: { type: "choice", instructions: "x", criteria: { a: 1 } } });
        } catch (e) {
          out.badError = e.message;
        }
        out.afterError = await d.systemOne(req.state, req.questions); // the queue is not wedged
        if (req.batch) {
          d.tokensPerPass = req.budget;
          const seen = [];
          out.batch = await d.systemOneBatch(req.batch, { onProgress: (a, b) => seen.push([a, b]) }); // BatchOptions
          const seenP = [];
          out.probsBatch = await d.probabilitiesBatch(req.batch.map(([s, qs]) => [s, Object.values(qs)]), { onProgress: (a, b) => seenP.push([a, b]) });
          out.progressP = seenP;
          out.progress = seen;
        }
        if (req.shared) {
          d.shareState = true;
          out.shared = await d.systemOne(req.state, req.questions);
          out.shared2 = await d.systemOne(req.state, req.questions);
        }
        out.logits = typed((await d.engine.run(req.trees)).logits);
        return out;
      } finally {
        d.destroy();
      }
    }
    default:
      throw new Error(`unknown command ${req.cmd}`);
  }
}

let input = "";
process.stdin.on("data", (c) => (input += c));
process.stdin.on("end", () => {
  main(JSON.parse(input)).then(
    (r) => process.stdout.write(JSON.stringify(r)),
    (e) => {
      process.stderr.write(String(e && e.stack ? e.stack : e));
      process.exit(1);
    });
});
