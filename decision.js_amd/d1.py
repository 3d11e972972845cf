"""The Decision API of decision.js (src/d1.ts): load, system_one, system_one_batch, probabilities,
probabilities_batch, destroy — same names (snake_case), argument meaning and error behaviour.

Text-to-ids (prompts, tokenizers) is upstream of the scoring path and not part of this build; a `prompt`
object turns states and questions into token ids. The default, IdPrompt, takes them already tokenized:
  state:     a list of token ids
  question:  the reference's question dict plus "ids" (its token ids) and "options" (one token-id group per
             option, [yes, no] for a noul: each option scores its best token, d1-3b-engine.ts:112-121);
             for EmbeddingGemma 2, "option_ids" (one token-id list per option text, in the model's order: a
             noul as [no, yes], eg2-prompt.ts:27-33); for d1-omni, "markers" (the position of each option's
             marker within the question's ids, in the model's order: a noul as [false, true],
             omni-prompt.ts:18-27); for Laya the same markers, the question's ids laid out as
             laya-prompt.ts does ([CLS] question [SEP], [MASK] and tokens per option, [SEP]) and read
             before the state's
"""
import json
import threading

import numpy as np

from . import questions as Q
from .eg2 import Eg2Engine
from .eg2_head import Eg2Head
from .encoder import EncoderEngine, cosine_logits
from .d3 import D3Engine
from .engine import DecoderEngine
from .laya import LayaEngine
from .omni import OmniEngine, temperature as omni_temperature


def _on_progress(opts):
    """BatchOptions.onProgress (d1.ts:33-35): opts is {"on_progress": f} (or "onProgress"); a bare callable is
    taken as that callback."""
    if opts is None or callable(opts):
        return opts
    return opts.get("on_progress") or opts.get("onProgress")


def softmax(s):
    """gpu.ts:294-297: max-subtracted exp in float64."""
    s = np.asarray(s, dtype=np.float64)
    e = np.exp(s - s.max())
    return list(e / e.sum())


class IdPrompt:
    """Pre-tokenized states and questions (see the module docstring)."""

    def trunk(self, state):
        return [int(t) for t in (state["ids"] if isinstance(state, dict) else state)]

    def branch(self, q):
        return [int(t) for t in q["ids"]]

    def readout_ids(self, q):
        groups = q["options"]
        if len(groups) != Q.n_options(q):
            raise Q.QuestionError(f"decision.js: {len(groups)} option groups for a {q['type']} with {Q.n_options(q)} options")
        return [[int(t) for t in g] for g in groups]

    def texts(self, state, q):
        return self.trunk(state), self.branch(q), [[int(t) for t in o] for o in q["option_ids"]]

    def sequence(self, state, q):
        """d1-omni's sequence of one question over one state (omni-prompt.ts:33-51 on ids): the state's ids, then
        the question's; its markers shifted past the state."""
        trunk, ids = self.trunk(state), self.branch(q)
        markers = [int(m) for m in q["markers"]]
        if len(markers) != Q.n_options(q):
            raise Q.QuestionError(f"decision.js: {len(markers)} markers for a {q['type']} with {Q.n_options(q)} options")
        if any(not 0 <= m < len(ids) for m in markers):
            raise Q.QuestionError("decision.js: a marker outside the question's ids")
        return {"ids": trunk + ids, "markers": [len(trunk) + m for m in markers], "type": q["type"]}

    def sequence_laya(self, state, q, max_len=512):
        """Laya's sequence of one question over one state (laya-prompt.ts:27-56 on ids): the question's ids first
        ([CLS] question [SEP], each option's [MASK] and tokens, [SEP]; `markers` index them), then the state's (its
        tokens and closing [SEP], cut to fit by the caller as laya-prompt.ts does), the whole cut to max_len tokens;
        every option marker must fit."""
        trunk, ids = self.trunk(state), self.branch(q)
        markers = [int(m) for m in q["markers"]]
        if len(markers) != Q.n_options(q):
            raise Q.QuestionError(f"decision.js: {len(markers)} markers for a {q['type']} with {Q.n_options(q)} options")
        if any(not 0 <= m < len(ids) for m in markers):
            raise Q.QuestionError("decision.js: a marker outside the question's ids")
        fit = [m for m in markers if m < max_len]
        if len(fit) != len(markers):
            raise Q.QuestionError(f"decision.js: only {len(fit)} of the {len(markers)} option markers fit in {max_len} tokens")
        return {"ids": (ids + trunk)[:max_len], "markers": markers, "type": q["type"]}


def criterion(v):
    """The legend text of a score level for every kind but d1-3b (omni-prompt.ts:16: the text, else Python's
    json.dumps of it)."""
    return v if isinstance(v, str) else json.dumps(v, ensure_ascii=False)


def _kind(config):
    """The reference's ModelKind of a manifest (d1.ts:63-64)."""
    model = config.get("model")
    if model == "laya":
        return "laya"
    if model in ("eg2-encoder", "eg2"):
        return "eg2"
    if model == "d3":
        return "d3"
    if model in ("decoder", "d1-3b") or "head_layers" not in config:
        return "d1-3b"
    return "d1-omni"


class Decision:
    """D1 (d1.ts:38-227): a model and the serial queue of its calls. `kind` is the reference's ModelKind
    (d1.ts:17): "d1-3b" for the causal decoders (run as d1-3B's forest), "d3" for the code readout, "d1-omni"
    and "laya" for the marker-head encoders, "eg2" for EmbeddingGemma 2."""

    def __init__(self, kind, engine, prompt, tokens_per_pass, share_state=False, workflow=""):
        self.kind, self.engine, self.prompt = kind, engine, prompt
        self.tokens_per_pass = tokens_per_pass
        self.share_state = share_state  # d3-lite's shareState; can be switched between calls (d1.ts:51-52)
        self.workflow = workflow  # EmbeddingGemma 2's LoadOptions.workflow, for a prompt that renders states
        self._lock = threading.Lock()  # one call at a time on the GPU (d1.ts:112-119)
        self._states = {}  # share_state: prefilled states by their ids (oldest dropped first)
        self._embeddings = {}  # encoder: normalized embeddings of the texts seen so far (d1.ts:44, 206-209)
        self._head = None  # encoder: the learned decision head, when the model has one (d1.ts:174)

    @classmethod
    def load(cls, base: str, opts: dict = None):
        """A model in the decision.js format at `base` (manifest.json + weights.bin). opts: device,
        on_progress, share_state, tokens_per_pass, workflow, graphs, prompt, direct_weights
        (LoadOptions.directWeights, gpu.ts:20). The kind comes from manifest.config.model (d1.ts:63-64)."""
        opts = dict(opts or {})
        from .fmt import load_manifest
        config = load_manifest(base if base.endswith("/") else base + "/")["config"]
        kind = _kind(config)
        d3 = D3Engine if "linear_heads" in config else DecoderEngine  # the shipped d3-lite, or its attention-only form
        eg2 = Eg2Engine if "ple" in config else EncoderEngine  # the shipped EmbeddingGemma 2, or the configs[0] form
        engine = {"d1-3b": DecoderEngine, "d3": d3, "eg2": eg2, "d1-omni": OmniEngine, "laya": LayaEngine}[kind].load(base, opts)
        # the reference's defaults (d1.ts:78): 4096 tokens per pass for d1-3B, 8192 otherwise; pass a larger
        # tokens_per_pass to pack more requests into one forward (MI355X activations take ~25 KB per token)
        tpp = opts.get("tokens_per_pass") or opts.get("tokensPerPass") or (4096 if kind == "d1-3b" else 8192)
        return cls(kind, engine, opts.get("prompt") or IdPrompt(), tpp,
                   bool(opts.get("share_state", opts.get("shareState"))), opts.get("workflow", ""))

    # ---- the public calls (d1.ts:81-110)
    def system_one(self, state, questions: dict):
        return self.system_one_batch([(state, questions)])[0]

    def system_one_batch(self, requests, opts=None):
        """Many (state, {name: question}) requests packed into as few forwards as fit; opts: BatchOptions."""
        done = self._run([(s, list(qs.values())) for s, qs in requests], _on_progress(opts))
        legend = str if self.kind == "d1-3b" else criterion  # d1.ts:91
        out = []
        for (s, qs), d in zip(requests, done):
            names = list(qs.keys())
            out.append({"answers": {n: Q.answer(qs[n], d["probs"][j], legend) for j, n in enumerate(names)},
                        "usage": {"input_tokens": d["tokens"], "output_tokens": 0}})
        return out

    def probabilities(self, state, qs):
        return self._run([(state, list(qs))], None)[0]["probs"]

    def probabilities_batch(self, requests, opts=None):
        return [r["probs"] for r in self._run([(s, list(qs)) for s, qs in requests], _on_progress(opts))]

    def destroy(self):
        for st in self._states.values():
            self.engine.free_state(st)
        self._states = {}
        self.engine.destroy()

    # ---- internals
    def _run(self, requests, on_progress):
        for _, qs in requests:
            for q in qs:
                Q.check_question(q)
        with self._lock:  # a failed call releases the lock: the queue does not wedge (d1.ts:117)
            if self.kind == "d1-3b":
                return self._run_shared(requests, on_progress) if self.share_state else self._run_decoder(requests, on_progress)
            if self.kind == "d3":
                return self._run_d3(requests, on_progress)
            if self.kind in ("d1-omni", "laya"):
                return self._run_omni(requests, on_progress)
            return self._run_encoder(requests, on_progress)

    def _passes(self, sizes):
        """Whole requests per pass up to the token budget; a pass always takes at least one (d1.ts:217-219)."""
        i = 0
        while i < len(sizes):
            j, used = i, 0
            while True:
                used += sizes[j]
                j += 1
                if not (j < len(sizes) and used + sizes[j] <= self.tokens_per_pass):
                    break
            yield i, j
            i = j

    def _run_decoder(self, requests, on_progress):
        """run3B (d1.ts:211-226): a forest per request (the state as trunk, each question a branch)."""
        p = self.prompt
        trees = [{"trunk": p.trunk(s), "branches": [p.branch(q) for q in qs], "groups": [p.readout_ids(q) for q in qs]}
                 for s, qs in requests]
        sizes = [len(t["trunk"]) + sum(len(b) for b in t["branches"]) for t in trees]
        out = [{"probs": [], "tokens": n} for n in sizes]
        for i, j in self._passes(sizes):
            scores = self.engine.run(trees[i:j])["scores"]
            for r, per_q in enumerate(scores):
                out[i + r]["probs"] = [softmax(s) for s in per_q]
            if on_progress:
                on_progress(j, len(trees))
        return out

    def _run_d3(self, requests, on_progress):
        """runD3 (d1.ts:150-169): one sequence per question (the state's ids then the question's), its first
        n-options codes read at its last token; with share_state each request's common prefix (the state) is
        read once for all its questions (D3Engine's groups). Softmax at the model's temperature; a noul is read
        as [false, true] and reversed to [yes, no]."""
        p = self.prompt
        seqs = [[{"ids": p.trunk(s) + p.branch(q), "options": Q.n_options(q)} for q in qs] for s, qs in requests]
        sizes = [sum(len(x["ids"]) for x in g) for g in seqs]
        temp = float(self.engine.m["config"].get("temperature", 1.0))
        out = [{"probs": [], "tokens": n} for n in sizes]
        for i, j in self._passes(sizes):
            flat = [x for g in seqs[i:j] for x in g]
            logits = self.engine.logits_d3(flat, [len(g) for g in seqs[i:j]] if self.share_state else None)
            k = 0
            for r in range(i, j):
                probs = []
                for q in requests[r][1]:
                    pr = softmax(np.asarray(logits[k], dtype=np.float64) / temp)
                    probs.append(pr[::-1] if q.get("type") == "noul" else pr)
                    k += 1
                out[r]["probs"] = probs
            if on_progress:
                on_progress(j, len(requests))
        return out

    def _run_omni(self, requests, on_progress):
        """runEncoder (d1.ts:121-147) for d1-omni and Laya: one sequence per question (the state read anew for
        each; Laya's puts the question first, cut to max_len), whole requests per pass up to the token budget;
        each question's marker logits divided by its temperature (omni-prompt.ts temperatureKey: type and
        option-count bucket), softmax, a noul read as [false, true] and reversed to [yes, no]."""
        c = self.engine.m["config"]
        if self.kind == "laya":
            seqs = [[self.prompt.sequence_laya(s, q, c["max_len"]) for q in qs] for s, qs in requests]
        else:
            seqs = [[self.prompt.sequence(s, q) for q in qs] for s, qs in requests]
        sizes = [sum(len(x["ids"]) for x in g) for g in seqs]
        out = [{"probs": [], "tokens": n} for n in sizes]
        for i, j in self._passes(sizes):
            logits = self.engine.logits([x for g in seqs[i:j] for x in g])["logits"]
            k = 0
            for r in range(i, j):
                probs = []
                for q in requests[r][1]:
                    t = omni_temperature(c, q["type"], Q.n_options(q))
                    pr = softmax(np.asarray(logits[k], dtype=np.float64) / t)
                    probs.append(pr[::-1] if q["type"] == "noul" else pr)
                    k += 1
                out[r]["probs"] = probs
            if on_progress:
                on_progress(j, len(requests))
        return out

    def _run_shared(self, requests, on_progress):
        """Shared state: each request's state is prefilled once and its K/V kept (reused by later calls on the
        same state); the questions then run against it."""
        p = self.prompt
        out = []
        for k, (s, qs) in enumerate(requests):
            trunk = p.trunk(s)
            key = tuple(trunk)
            st = self._states.get(key)
            if st is None:
                if len(self._states) >= 64:
                    old = next(iter(self._states))
                    self.engine.free_state(self._states.pop(old))
                st = self._states[key] = self.engine.prefill(trunk)
            branches = [p.branch(q) for q in qs]
            scores = self.engine.run_shared(st, branches, [p.readout_ids(q) for q in qs])
            out.append({"probs": [softmax(x) for x in scores], "tokens": len(trunk) + sum(len(b) for b in branches)})
            if on_progress:
                on_progress(k + 1, len(requests))
        return out

    def _run_encoder(self, requests, on_progress):
        """runEg2 (d1.ts:172-204): every distinct text embedded once (cached), then the head on the host."""
        p = self.prompt
        asked = [[p.texts(s, q) for q in qs] for s, qs in requests]
        todo, tokens = {}, [0] * len(requests)
        for r, per_q in enumerate(asked):
            for st, qi, opts in per_q:
                for t in [st, qi, *opts]:
                    key = tuple(t)
                    if key in self._embeddings or key in todo:
                        continue
                    todo[key] = t
                    tokens[r] += len(t)
        texts = list(todo.values())
        sizes = [len(t) for t in texts]
        for i, j in self._passes(sizes) if texts else []:
            emb = self.engine.embed(texts[i:j])["embeddings"]
            for k, e in enumerate(emb):
                self._remember(tuple(texts[i + k]), e)
            if on_progress:
                on_progress(j, len(texts))
        c = self.engine.m["config"]
        if self._head is None and c.get("head") and self.engine.host:
            self._head = Eg2Head(c, self.engine.host)
        temps = c.get("temperatures", {})
        emb = lambda t: (tuple(t), self._embeddings[tuple(t)])  # noqa: E731
        out = []
        for r, (s, qs) in enumerate(requests):
            probs = []
            for q, (st, qi, opts) in zip(qs, asked[r]):
                if self._head is not None:  # the learned head (eg2-head.ts:64-99)
                    z = self._head.logits(q["type"], emb(st), emb(qi), [emb(o) for o in opts])
                else:  # the cosine prior alone (the configured dense head has no learned scorer)
                    z = cosine_logits(emb(st)[1], emb(qi)[1], [emb(o)[1] for o in opts])
                t = float(temps.get(q["type"], 1.0))
                pr = softmax(np.asarray(z, dtype=np.float64) / t)
                probs.append(pr[::-1] if q["type"] == "noul" else pr)  # the model reads a noul as [no, yes]
            out.append({"probs": probs, "tokens": tokens[r]})
        return out

    def _remember(self, key, e):
        if len(self._embeddings) >= 8192:
            self._embeddings.pop(next(iter(self._embeddings)))  # the oldest text first (d1.ts:207)
        self._embeddings[key] = e
