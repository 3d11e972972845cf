"""EmbeddingGemma 2 as shipped (Eg2Engine, src/eg2-engine.ts) on libdj.so: a bidirectional Gemma text encoder with
per-layer embeddings — sandwich RMSNorms, q/k/v norms + RoPE with each layer type's head width and theta
(256-dim heads within a +-window on the sliding layers, 512-dim heads over the whole text on the global ones),
the tanh-GELU MLP, and after every layer the per-layer embedding (gelu(x W_gate) * rmsnorm(xe W_in) through
W_proj) with the layer scalar — then the mean of each text's rows times the f16 embedding projection, the first
embed_dim values L2-normalised. Every text is one sequence; many are packed on one token axis and recorded as
one forward. The learned decision head runs on the host (eg2_head.py).
"""
import numpy as np

from . import _dj, fmt
from .encoder import pack_encoder
from .engine import GpuEngine, load_weights


class Eg2Engine(GpuEngine):
    """The layer loop of eg2-engine.ts:103-131."""

    @classmethod
    def load(cls, base: str, opts: dict = None):
        ctx, m, w = load_weights(base, opts)
        c = m["config"]
        if c.get("model") != "eg2" or "ple" not in c:
            raise ValueError(f"decision.js: {base} is not an EmbeddingGemma 2 export ({c.get('model')})")
        bad = sorted({t for t in c["layer_types"] if t not in ("sliding_attention", "full_attention")})
        if bad:
            raise ValueError(f"decision.js: unsupported layer types {bad}")
        for t in set(c["layer_types"]):
            if c["head_dim"][t] not in (64, 128, 256, 512):
                raise ValueError(f"decision.js: {t} heads of {c['head_dim'][t]} dims (64, 128, 256 or 512)")
        eng = cls(ctx, m, w, opts)
        # the decision head's f32 tensors stay on the host (Eg2Engine.load, eg2-engine.ts:46-50)
        tf = fmt.TensorFile(base if base.endswith("/") else base + "/")
        eng.host = {name: np.array(tf.tensor(info), dtype=np.float32) for name, info in m.get("host", {}).items()}
        return eng

    def __init__(self, ctx, m, w, opts=None):
        super().__init__(ctx, m, w, opts)
        c = m["config"]
        self.H, self.I, self.h, self.P = c["hidden"], c["intermediate"], c["heads"], c["ple"]
        self.layers, self.eps, self.types = c["layers"], c["eps"], c["layer_types"]
        self.N, self.E = c["embedding_dim"], c["embed_dim"]
        self.scalars = c.get("layer_scalars", [1.0] * self.layers)
        self.qkv_w = max((self.h + 2 * c["kv_heads"][t]) * c["head_dim"][t] for t in self.types)
        self.att_w = max(self.h * c["head_dim"][t] for t in self.types)
        self.capacity = self.seq_capacity = 0
        self.host = {}

    def ensure(self, T, S):
        if T <= self.capacity and S <= self.seq_capacity:
            return
        cap = (max(T, self.capacity, 256) + 63) // 64 * 64
        scap = max(S, self.seq_capacity, 64)
        H, P = self.H, self.P
        self._alloc({"x": cap * H * 2, "xe": cap * H * 2, "normed": cap * H * 2, "o": cap * H * 2,
                     "z": cap * self.qkv_w * 2, "y": cap * self.att_w * 2, "h": cap * self.I * 2, "gate": cap * P * 2,
                     "e": cap * P * 2, "mix": cap * P * 2, "ids": cap * 4, "meta": cap * 16, "full": cap * 16,
                     "slide": cap * 16, "seqs": scap * 8, "emb": scap * self.N * 4})
        self.capacity, self.seq_capacity = cap, scap

    def embed(self, seqs, debug=False):
        """The normalized embedding of every token sequence (f32 [S, embed_dim]); with `debug` also the final
        norm's output (f16 [T, H])."""
        c = self.m["config"]
        pk = pack_encoder(seqs, c["window"])
        T, S = pk["T"], pk["S"]
        if T == 0:
            return {"embeddings": np.zeros((S, self.E), np.float32), "debug": {}}
        self.ensure(T, S)
        B = self._bufs
        B["ids"].upload(pk["ids"])
        B["meta"].upload(pk["meta"])
        B["full"].upload(pk["full"])
        B["slide"].upload(pk["slide"])
        B["seqs"].upload(pk["ranges"])
        with self.ctx.recorder(self._key("eg2", T, S, bool(debug))) as rec:  # aborted on an error
            if not rec.replay:
                self._record(rec, T, S, B)
            di = rec.snapshot(B["normed"], T * self.H * 2, np.float16, (T, self.H)) if debug else None
            ei = rec.snapshot(B["emb"], S * self.N * 4, np.float32, (S, self.N))
        got = rec.finish()
        self.stats["forwards"] += 1
        self.stats["tokens"] += T
        e = got[ei][:, :self.E].astype(np.float64)
        n = np.maximum(np.sqrt((e * e).sum(-1, keepdims=True)), 1e-12)
        return {"embeddings": (e / n).astype(np.float32), "debug": {"final": got[di]} if debug else {}}

    def _record(self, rec, T, S, B):
        c, w = self.m["config"], self.w
        H, h, eps, P = self.H, self.h, self.eps, self.P
        z = B["z"]
        rec.gather_q(B["ids"], T, w["embed"], B["x"])
        rec.gather_q(B["ids"], T, w["embed"], B["xe"])  # the copy each layer projects its own embedding from
        rec.sandwich(T, H, eps, 1.0, B["x"], None, None, w["layers.0.input_layernorm"], B["normed"])
        for i, t in enumerate(self.types):
            p, D, kv = f"layers.{i}.", c["head_dim"][t], c["kv_heads"][t]
            stride = (h + 2 * kv) * D
            src = _dj.kv_src(z, T, stride, h * D, (h + kv) * D)
            # attention: x += post_norm(o(attn(rope(norm(q)), rope(norm(k)), norm(v))))
            rec.matmul(B["normed"], w[p + "qkv"], z, T)
            rec.qk_norm_rope(T, h, kv, D, stride, z, w[p + "q_norm"], w[p + "k_norm"], True, B["meta"].at(12), 4, eps,
                             c["rope_theta"][t], D, _dj.ROPE_INV_POW)
            rec.attention(T, h, kv, D, z, stride, src, src, B["full" if t == "full_attention" else "slide"], 1.0, B["y"])
            rec.matmul(B["y"], w[p + "o"], B["o"], T)
            rec.sandwich(T, H, eps, 1.0, B["x"], B["o"], w[p + "post_attention_layernorm"], w[p + "pre_feedforward_layernorm"],
                         B["normed"])
            # MLP: x += post_norm(down(gelu(gate) up))
            rec.matmul_glu(B["normed"], w[p + "gu"], B["h"], T, _dj.ACT_GELU_TANH)
            rec.matmul(B["h"], w[p + "down"], B["o"], T)
            rec.sandwich(T, H, eps, 1.0, B["x"], B["o"], w[p + "post_feedforward_layernorm"], None, None)
            # per-layer embedding: x = (x + norm(proj(gelu(gate(x)) * norm(embedding slice)))) * layer scalar
            rec.matmul(B["x"], w[p + "ple_gate"], B["gate"], T)
            rec.matmul(B["xe"], w[p + "ple_in"], B["e"], T)
            rec.ple_mix(T, P, B["gate"], B["e"], w["ple.norm"], eps, B["mix"])
            rec.matmul(B["mix"], w[p + "ple_proj"], B["o"], T)
            nxt = f"layers.{i + 1}.input_layernorm" if i + 1 < self.layers else "final_norm"
            rec.sandwich(T, H, eps, float(self.scalars[i]), B["x"], B["o"], w[p + "ple_norm"], w[nxt], B["normed"])
        rec.pool_project(T, S, H, self.N, B["normed"], B["seqs"], w["projection"], B["emb"])
