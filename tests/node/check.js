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
      return { ids: typed(pk.ids), pos: typed(pk.pos), rng: typed(pk.rng), leaves: typed(pk.leaves), leafIds: typed(pk.leafIds), nIds: pk.nIds, T: pk.T, L: pk.L };
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
      // graph keys handed out over a sequence of forwards (no device: key() reads only the engine's own state)
      const { GpuEngine } = require(path.join(root, "engine"));
      const e = new GpuEngine(null, {}, {}, { graphs: req.graphs });
      return req.seq.map((parts) => String(e.key(...parts)));
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
          out.batch = await d.systemOneBatch(req.batch, (a, b) => seen.push([a, b]));
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
