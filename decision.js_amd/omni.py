"""d1-omni's engine (D1OmniEngine, src/omni-engine.ts) on libdj.so: a bidirectional LFM2 trunk (centred 3-tap
short convolutions and GQA attention over each whole sequence), then the decision head — the question-type
row added to every token, pre-norm transformer layers with biases, the last residual under the scorer's
LayerNorm — and at each option marker Linear + GELU + Linear(H, 1). One question is one sequence; many are
packed on one token axis and recorded as one forward.
"""
import math

import numpy as np

from . import _dj
from .engine import DecoderEngine, load_weights

QTYPES = {"choice": 0, "score": 1, "noul": 2}  # omni-engine.ts:18


def pack_omni(seqs):
    """D1OmniEngine.logits's packing (omni-engine.ts:62-75). seqs: [{"ids", "markers", "type"}]. Per token: id,
    position within its sequence, question type, the centred short-conv taps (t-1, t, t+1; -1 past either end of
    its sequence, never into a neighbour) and its key range [start, end) (every token sees its whole sequence);
    per option marker: its row on the packed axis."""
    n = [len(s["ids"]) for s in seqs]
    T = sum(n)
    starts = np.cumsum([0] + n[:-1]).astype(np.int64) if seqs else np.zeros(0, np.int64)
    seq_of = np.repeat(np.arange(len(seqs)), n)
    start = starts[seq_of] if T else np.zeros(0, np.int64)
    end = start + np.repeat(np.array(n, dtype=np.int64), n) if T else np.zeros(0, np.int64)
    t = np.arange(T, dtype=np.int64)
    ids = np.array([x for s in seqs for x in s["ids"]], dtype=np.uint32)
    taps = np.zeros((T, 4), dtype=np.int32)
    taps[:, 0] = np.where(t > start, t - 1, -1)
    taps[:, 1] = t
    taps[:, 2] = np.where(t + 1 < end, t + 1, -1)
    rng = np.zeros((T, 4), dtype=np.int32)
    rng[:, 0], rng[:, 1] = start, end
    for k, s in enumerate(seqs):
        if s["type"] not in QTYPES:
            raise ValueError(f"decision.js: question type {s['type']!r} (choice, score or noul)")
        if any(not 0 <= m < n[k] for m in s["markers"]):
            raise ValueError(f"decision.js: a marker outside its sequence of {n[k]} tokens")
    qtype = np.repeat(np.array([QTYPES[s["type"]] for s in seqs], dtype=np.uint32), n)
    markers = np.array([starts[k] + m for k, s in enumerate(seqs) for m in s["markers"]], dtype=np.uint32)
    return {"ids": ids, "pos": (t - start).astype(np.uint32), "qtype": qtype, "taps": taps, "rng": rng,
            "markers": markers, "T": T, "M": len(markers)}


def temperature(config, qtype, options):
    """The calibration temperature of a question (omni-engine.ts:22-26): "<type>:<bucket>" for buckets 2, 3-5,
    6-10, 11+, else "<type>", else 1."""
    k = "2" if options <= 2 else "3-5" if options <= 5 else "6-10" if options <= 10 else "11+"
    temps = config.get("temperatures", {})
    return float(temps.get(f"{qtype}:{k}", temps.get(qtype, 1.0)))


class OmniEngine(DecoderEngine):
    """The trunk is DecoderEngine's layer loop on the omni packing (centred taps, whole-sequence key ranges);
    the head and scorer follow omni-engine.ts:125-147 with dj_add_rows / dj_add_layernorm / dj_bias_act /
    dj_gather_rows / dj_score around the q8/q4 products."""

    @classmethod
    def load(cls, base: str, opts: dict = None):
        ctx, m, w = load_weights(base, opts)
        c = m["config"]
        if c.get("model") != "d1-omni" and "head_layers" not in c:
            raise ValueError(f"decision.js: {base} is not a d1-omni model ({c.get('model')})")
        bad = sorted({t for t in c.get("layer_types", []) if t not in ("full_attention", "conv")})
        if bad:
            raise ValueError(f"decision.js: unsupported layer types {bad}")
        if c["hidden"] % c["head_heads"] or c["hidden"] // c["head_heads"] not in (64, 128, 256):
            raise ValueError(f"decision.js: head width {c['hidden']} / {c['head_heads']} heads (64, 128 or 256 per head)")
        return cls(ctx, m, w, opts)

    def __init__(self, ctx, m, w, opts=None):
        super().__init__(ctx, m, w, opts)
        c = m["config"]
        self.hh, self.ff, self.ln_eps = c["head_heads"], c["head_ff"], c["ln_eps"]
        self.head_layers = c["head_layers"]
        self.Dh = self.H // self.hh
        self.type_rows = int(w["head.type_emb"].host.shape[0])
        self.marker_capacity = 0

    def ensure(self, T: int, M: int = 0, n_ids: int = 0):
        """Activation buffers for T tokens and M markers (omni-engine.ts:44-52: grown, never shrunk)."""
        if T <= self.capacity and M <= self.marker_capacity:
            return
        cap = (max(T, self.capacity, 256) + 63) // 64 * 64
        mcap = max(M, self.marker_capacity, 64)
        H = self.H
        zw = max(self.stride, 3 * H)  # qkv rows, a conv layer's [B | C | U], or the head's q | k | v
        yw = max(self.h * self.D, H)
        self._alloc({"x": cap * H * 2, "normed": cap * H * 2, "o": cap * H * 2, "z": cap * zw * 2, "y": cap * yw * 2,
                     "h": cap * max(self.I, self.ff) * 2, "ids": cap * 4, "pos": cap * 4, "qtype": cap * 4,
                     "rng": cap * 16, "taps": cap * 16, "rope": cap * (self.D // 2) * 8,
                     "markers": mcap * 4, "g": mcap * H * 2, "gf": mcap * H * 2, "out": mcap * 4, **self._norm_bufs(cap)})
        self.capacity, self.marker_capacity = cap, mcap

    INPUTS = ("ids", "pos", "qtype", "rng", "taps", "markers")

    def logits(self, seqs, debug=False):
        """Raw marker logits per sequence ([seq][marker], before the temperature), and with `debug` the trunk's
        output (after the final norm) and the head's residual stream before the scorer, f16 [T, H]."""
        pk = pack_omni(seqs)
        if pk["T"] == 0:
            return {"logits": [[] for _ in seqs], "debug": {}}
        return self._forward_omni(pk, seqs, debug, None)

    def stage(self, seqs):
        """Packs `seqs` and keeps the packed inputs in device memory (the benchmark's resident inputs)."""
        pk = pack_omni(seqs)
        return {"pk": pk, "seqs": seqs, "bufs": {k: self.ctx.array(pk[k]) for k in self.INPUTS if len(pk[k])}}

    def run_staged(self, st):
        return self._forward_omni(st["pk"], st["seqs"], False, st["bufs"])

    def _forward_omni(self, pk, seqs, debug, staged):
        T, M = pk["T"], pk["M"]
        self.ensure(T, M)
        B = self._bufs
        for k in self.INPUTS:
            if not len(pk[k]):
                continue
            if staged is not None:
                B[k].copy_from(staged[k])
            else:
                B[k].upload(pk[k])
        snaps = {}
        with self.ctx.recorder(self._key("omni", T, M, bool(debug))) as rec:  # aborted on an error
            # a replay returns the captured snapshots in the order they were taken: take them in that order
            if not rec.replay:
                self._layers(rec, T, B)
            if debug:
                snaps["trunk"] = rec.snapshot(B["normed"], T * self.H * 2, np.float16, (T, self.H))
            if not rec.replay:
                self._head(rec, T, M, B)
            if debug:
                snaps["head"] = rec.snapshot(B["x"], T * self.H * 2, np.float16, (T, self.H))
            oi = rec.snapshot(B["out"], max(M, 1) * 4, np.float32, (max(M, 1),)) if M else None
        got = self._finish(rec, T)
        out = got[oi] if oi is not None else np.zeros(0, np.float32)
        res, k = [], 0
        for s in seqs:
            res.append([float(v) for v in out[k:k + len(s["markers"])]])
            k += len(s["markers"])
        return {"logits": res, "debug": {n: got[i] for n, i in snaps.items()}}

    def _head(self, rec, T, M, B):
        """The decision head and scorer (omni-engine.ts:125-147)."""
        w, H, hh, Dh, ln = self.w, self.H, self.hh, self.Dh, self.ln_eps
        z = B["z"]
        src = _dj.kv_src(z, T, 3 * H, H, 2 * H)
        rec.add_rows(T, H, B["normed"], B["qtype"], w["head.type_emb"], self.type_rows, B["x"])
        for i in range(self.head_layers):
            p = f"head.{i}."
            # i > 0: the residual first takes the previous layer's FFN output
            rec.add_layernorm(T, H, i > 0, ln, B["x"], B["o"], w[p + "norm1"], w[p + "norm1_bias"], B["normed"])
            rec.matmul(B["normed"], w[p + "in_proj"], z, T)
            rec.bias_act(T, 3 * H, z, w[p + "in_proj_bias"], _dj.BIAS_NONE)
            rec.attention(T, hh, hh, Dh, z, 3 * H, src, src, B["rng"], 1.0 / math.sqrt(Dh), B["y"])
            rec.matmul(B["y"], w[p + "out_proj"], B["o"], T)
            rec.bias_act(T, H, B["o"], w[p + "out_proj_bias"], _dj.BIAS_NONE)
            rec.add_layernorm(T, H, True, ln, B["x"], B["o"], w[p + "norm2"], w[p + "norm2_bias"], B["normed"])
            rec.matmul(B["normed"], w[p + "linear1"], B["h"], T)
            rec.bias_act(T, self.ff, B["h"], w[p + "linear1_bias"], _dj.BIAS_RELU)
            rec.matmul(B["h"], w[p + "linear2"], B["o"], T)
            rec.bias_act(T, H, B["o"], w[p + "linear2_bias"], _dj.BIAS_NONE)
        # the last residual add, under the scorer's LayerNorm
        rec.add_layernorm(T, H, self.head_layers > 0, ln, B["x"], B["o"], w["scorer.norm"], w["scorer.norm_bias"], B["normed"])
        if M:
            rec.gather_rows(M, H, T, B["normed"], B["markers"], B["g"])
            rec.matmul(B["g"], w["scorer.fc"], B["gf"], M)
            rec.bias_act(M, H, B["gf"], w["scorer.fc_bias"], _dj.BIAS_GELU_ERF)
            rec.score(M, H, B["gf"], w["scorer.out"], w["scorer.out_bias"], B["out"])

    def probabilities(self, seqs):
        """Calibrated probabilities per sequence in option order (omni-engine.ts:151-158; a noul as [false, true],
        as the model reads it)."""
        from .d1 import softmax
        out = []
        for s, z in zip(seqs, self.logits(seqs)["logits"]):
            t = temperature(self.m["config"], s["type"], len(z))
            out.append(softmax(np.asarray(z, dtype=np.float64) / t))
        return out
