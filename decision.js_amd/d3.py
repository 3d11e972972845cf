"""d3-lite's engine on its shipped layout (D3Engine, src/d3-engine.ts) over libdj.so: a Qwen3.5-shaped backbone of
Gated DeltaNet layers (the `in` product, dj_gdn, the `out` product) with a gated attention layer every few
(the fused q | k | v | gate product, q/k RMSNorm + partial RoPE, dj_attention_gated, the `o` product), SwiGLU
MLPs, the final norm and the code readout at each question's last token. One question is one sequence (with
`groups`, a request's common prefix is read once); many are packed on one token axis and recorded as one
forward. Manifests of the attention-only form (no `linear_heads`) run on DecoderEngine.logits_d3.
"""
import math

import numpy as np

from . import _dj
from .engine import DecoderEngine, load_weights, pack_shared


def gdn_spans(seqs, groups=None):
    """The DeltaNet scans of D3Engine.logits's packing (d3-engine.ts:89), on pack_shared's row layout: per question
    (a start, a length | write_a << 31, b start, b length). With a shared prefix the trunk is span a (written by
    the group's first question only) and the question's own tokens span b; without one the sequence is span a
    (written) and b is empty. [S, 4] u32."""
    sizes = groups if groups is not None else [1] * len(seqs)
    out = np.zeros((len(seqs), 4), dtype=np.uint32)
    si = off = 0
    for n in sizes:
        group = seqs[si:si + n]
        P = 0
        if n > 1:
            lim = min(len(s["ids"]) for s in group) - 1
            first = group[0]["ids"]
            while P < lim and all(s["ids"][P] == first[P] for s in group):
                P += 1
        ts = off
        off += P
        for b, s in enumerate(group):
            L = len(s["ids"]) - P
            out[si + b] = (ts, P | (1 << 31 if b == 0 else 0), off, L) if P else (off, L | (1 << 31), 0, 0)
            off += L
        si += n
    return out


class D3Engine(DecoderEngine):
    """The layer loop of d3-engine.ts:109-131."""

    @classmethod
    def load(cls, base: str, opts: dict = None):
        ctx, m, w = load_weights(base, opts)
        c = m["config"]
        if c.get("model") != "d3" or "linear_heads" not in c:
            raise ValueError(f"decision.js: {base} is not a d3-lite export ({c.get('model')})")
        bad = sorted({t for t in c["layer_types"] if t not in ("linear_attention", "full_attention")})
        if bad:
            raise ValueError(f"decision.js: unsupported layer types {bad}")
        if c["linear_key_dim"] != 128 or c["linear_value_dim"] != 128 or c.get("conv_kernel", 4) != 4:
            raise ValueError("decision.js: the DeltaNet kernel takes 128-wide key and value heads and 4 conv taps "
                             f"(got {c['linear_key_dim']}, {c['linear_value_dim']}, {c.get('conv_kernel')})")
        if c["head_dim"] not in (64, 128, 256) or not 0 < c["rotary_dim"] <= c["head_dim"] or c["rotary_dim"] % 16:
            raise ValueError(f"decision.js: attention heads of {c['head_dim']} with {c['rotary_dim']} rotary dims")
        return cls(ctx, m, w, opts)

    def __init__(self, ctx, m, w, opts=None):
        super().__init__(ctx, m, w, opts)
        c = m["config"]
        self.LH, self.rows, self.rot = c["linear_heads"], c["linear_rows"], c["rotary_dim"]
        self.astride = (2 * self.h + 2 * self.kv) * self.D  # q | k | v | gate heads
        self.codes = int(w["readout"].host.shape[0])
        self.seq_capacity = 0

    def ensure(self, T: int, P: int = 0, S: int = 0):
        """Buffers for T tokens, P (row, code) pairs and S scans (grown, never shrunk)."""
        if T <= self.capacity and P <= self.leaf_capacity and S <= self.seq_capacity:
            return
        cap = (max(T, self.capacity, 256) + 63) // 64 * 64
        pcap = max(P, self.leaf_capacity, 1024)
        scap = max(S, self.seq_capacity, 64)
        H = self.H
        self._alloc({"x": cap * H * 2, "normed": cap * H * 2, "o": cap * H * 2, "z": cap * max(self.rows, self.astride) * 2,
                     "y": cap * max(self.LH * 128, self.h * self.D) * 2, "h": cap * self.I * 2, "ids": cap * 4,
                     "pos": cap * 4, "rng": cap * 16, "spans": scap * 16, "leaf_ids": pcap * 8, "out": pcap * 4})
        self.capacity, self.leaf_capacity, self.seq_capacity = cap, pcap, scap

    def logits_d3(self, seqs, groups=None, debug=False):
        """Code logits per question ([seq][its `options` codes], before the temperature), as D3Engine.logits: the
        sequences packed by pack_shared (a request's common prefix read once when `groups` is given), the DeltaNet
        scans from gdn_spans, the attention on pack_shared's key ranges, READOUT against the f32 `readout` matrix.
        With `debug`, the returned dict form also holds the final normed hidden state (f16 [T, H])."""
        pk = pack_shared(seqs, groups)
        spans = gdn_spans(seqs, groups)
        T, P, S = pk["T"], pk["P"], len(spans)
        if T == 0:
            return {"logits": [[] for _ in seqs], "debug": {}} if debug else [[] for _ in seqs]
        self.ensure(T, P, S)
        B = self._bufs
        B["ids"].upload(pk["ids"])
        B["pos"].upload(pk["pos"])
        B["rng"].upload(pk["rng"])
        B["spans"].upload(spans)
        if P:
            B["leaf_ids"].upload(pk["pairs"].reshape(-1))
        with self.ctx.recorder(self._key("d3lite", T, P, S, bool(debug))) as rec:  # aborted on an error
            if not rec.replay:
                self._layers_d3(rec, T, S, B)
                if P:
                    rec.readout(T, P, self.H, B["normed"], self.w["readout"], self.codes, B["leaf_ids"], B["out"])
            di = rec.snapshot(B["normed"], T * self.H * 2, np.float16, (T, self.H)) if debug else None
            oi = rec.snapshot(B["out"], max(P, 1) * 4, np.float32, (max(P, 1),)) if P else None
        got = self._finish(rec, T)
        out = got[oi] if oi is not None else np.zeros(0, np.float32)
        res, k = [], 0
        for s in seqs:
            res.append([float(v) for v in out[k:k + s["options"]]])
            k += s["options"]
        return {"logits": res, "debug": {"final": got[di]}} if debug else res

    def _layers_d3(self, rec, T, S, B):
        w, H, h, kv, D, eps = self.w, self.H, self.h, self.kv, self.D, self.eps
        z, A = B["z"], self.astride
        src = _dj.kv_src(z, T, A, h * D, (h + kv) * D)
        rec.gather_q(B["ids"], T, w["embed"], B["x"])
        for i, t in enumerate(self.types):
            p = f"layers.{i}."
            rec.add_rmsnorm(T, H, i > 0, eps, B["x"], B["o"], w[p + "input_norm"], B["normed"])  # adds the last MLP
            if t == "linear_attention":
                rec.matmul(B["normed"], w[p + "in"], z, T)
                rec.gdn(T, S, B["spans"], self.LH, self.rows, z, w[p + "conv"], w[p + "A_log"], w[p + "dt_bias"],
                        w[p + "gnorm"], eps, B["y"])
                rec.matmul(B["y"], w[p + "out"], B["o"], T)
            else:
                rec.matmul(B["normed"], w[p + "qkvg"], z, T)
                rec.qk_norm_rope(T, h, kv, D, A, z, w[p + "q_norm"], w[p + "k_norm"], False, B["pos"], 1, eps,
                                 self.theta, self.rot, _dj.ROPE_POW_NEG)
                rec.attention_gated(T, h, kv, D, z, A, src, src, B["rng"], 1.0 / math.sqrt(D), z.at((h + 2 * kv) * D * 2),
                                    A, B["y"])
                rec.matmul(B["y"], w[p + "o"], B["o"], T)
            rec.add_rmsnorm(T, H, True, eps, B["x"], B["o"], w[p + "post_norm"], B["normed"])
            rec.matmul_glu(B["normed"], w[p + "w13"], B["h"], T, _dj.ACT_SILU)
            rec.matmul(B["h"], w[p + "w2"], B["o"], T)
        rec.add_rmsnorm(T, H, True, eps, B["x"], B["o"], w["final_norm"], B["normed"])

    def run(self, trees, debug_layers=()):
        raise ValueError("decision.js: d3-lite reads codes at each question's last token: use logits_d3")

    def prefill(self, trunk):
        raise ValueError("decision.js: d3-lite shares a request's prefix through logits_d3's groups")
