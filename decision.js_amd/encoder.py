"""The EmbeddingGemma-shaped bidirectional encoder engine (Eg2Engine, src/eg2-engine.ts) on libdj.so:
every text one sequence, many packed on one token axis, one recorded forward; then mean pooling and the
configured head (Linear hidden->width, Linear width->embed_dim, in f32) and L2 normalisation.
"""
import numpy as np

from . import _dj, fmt
from .engine import GpuEngine, load_weights


def pack_encoder(seqs, window=None):
    """Eg2Engine.embed's packing (eg2-engine.ts:74-86): per token meta (start, end, -1, i) and its key range
    on the global layers [start, end) (and on windowed layers [max(start, t-w), min(end, t+w+1))); per
    sequence (start, end)."""
    T = sum(len(s) for s in seqs)
    ids = np.empty(T, dtype=np.uint32)
    meta = np.empty((T, 4), dtype=np.int32)
    full = np.zeros((T, 4), dtype=np.int32)
    slide = np.zeros((T, 4), dtype=np.int32) if window is not None else None
    ranges = np.empty((len(seqs), 2), dtype=np.uint32)
    off = 0
    for k, s in enumerate(seqs):
        n = len(s)
        i = np.arange(n, dtype=np.int32)
        ids[off:off + n] = s
        meta[off:off + n] = np.stack([np.full(n, off), np.full(n, off + n), np.full(n, -1), i], 1)
        full[off:off + n, 0], full[off:off + n, 1] = off, off + n
        if window is not None:
            t = off + i
            slide[off:off + n, 0] = np.maximum(off, t - window)
            slide[off:off + n, 1] = np.minimum(off + n, t + window + 1)
        ranges[k] = (off, off + n)
        off += n
    return {"ids": ids, "meta": meta, "full": full, "slide": slide, "ranges": ranges, "T": T, "S": len(seqs)}


class EncoderEngine(GpuEngine):
    """Layers (eg2-engine.ts:103-129, without per-layer embeddings): qkv -> q/k/v RMSNorm + RoPE ->
    bidirectional attention (scale 1) -> o -> sandwich -> gate|up with the tanh-GELU epilogue -> down ->
    sandwich (times the layer scalar)."""

    @classmethod
    def load(cls, base: str, opts: dict = None):
        ctx, m, w = load_weights(base, opts)
        if m["config"].get("model") != "eg2-encoder":
            raise ValueError(f"decision.js: {base} is not an encoder model ({m['config'].get('model')})")
        eng = cls(ctx, m, w, opts)
        # the decision head's f32 tensors stay on the host (Eg2Engine.load, eg2-engine.ts:46-50)
        tf = fmt.TensorFile(base if base.endswith("/") else base + "/")
        eng.host = {name: np.array(tf.tensor(info), dtype=np.float32) for name, info in m.get("host", {}).items()}
        return eng

    def __init__(self, ctx, m, w, opts=None):
        super().__init__(ctx, m, w, opts)
        c = m["config"]
        self.H, self.I, self.h, self.kv, self.D = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"]
        self.layers, self.eps, self.theta = c["layers"], c["eps"], c["rope_theta"]
        self.stride = (self.h + 2 * self.kv) * self.D
        self.scalars = c.get("layer_scalars", [1.0] * self.layers)
        self.scale = c.get("attention_scale", 1.0)
        self.width, self.E = c["head_width"], c["embed_dim"]
        self.capacity = self.seq_capacity = 0
        self.host = {}

    def ensure(self, T, S):
        if T <= self.capacity and S <= self.seq_capacity:
            return
        cap = (max(T, self.capacity, 256) + 63) // 64 * 64
        scap = max(S, self.seq_capacity, 64)
        H = self.H
        self._alloc({"x": cap * H * 2, "normed": cap * H * 2, "o": cap * H * 2, "z": cap * self.stride * 2,
                     "y": cap * self.h * self.D * 2, "h": cap * self.I * 2, "ids": cap * 4, "meta": cap * 16,
                     "rng": cap * 16, "seqs": scap * 8, "pooled": scap * H * 4, "h1": scap * self.width * 4,
                     "emb": scap * self.E * 4})
        self.capacity, self.seq_capacity = cap, scap

    def embed(self, seqs, debug_layers=()):
        """The normalized embedding of every token sequence (f32 [S, embed_dim]), plus debug hidden states."""
        pk = pack_encoder(seqs)
        T, S = pk["T"], pk["S"]
        self.ensure(T, S)
        B = self._bufs
        B["ids"].upload(pk["ids"])
        B["meta"].upload(pk["meta"])
        B["rng"].upload(pk["full"])
        B["seqs"].upload(pk["ranges"])
        debug_layers = tuple(sorted(set(debug_layers)))
        with self.ctx.recorder(self._key("embed", T, S, debug_layers)) as rec:  # aborted on an error
            snaps = self._record(rec, T, S, debug_layers)
            ei = rec.snapshot(B["emb"], S * self.E * 4, np.float32, (S, self.E))
        got = rec.finish()
        self.stats["forwards"] += 1
        self.stats["tokens"] += T
        e = got[ei].astype(np.float64)
        n = np.maximum(np.sqrt((e * e).sum(-1, keepdims=True)), 1e-12)
        return {"embeddings": (e / n).astype(np.float32), "debug": {i: got[k] for i, k in snaps.items()}}

    def _record(self, rec, T, S, debug_layers):
        """The encoder's ops on the recorder (eg2-engine.ts:103-129 without per-layer embeddings), then pooling
        and the head; returns the debug snapshots' indices."""
        B, w = self._bufs, self.w
        H, h, kv, D, eps = self.H, self.h, self.kv, self.D, self.eps
        snaps = {}
        if not rec.replay:
            z = B["z"]
            src = _dj.kv_src(z, T, self.stride, h * D, (h + kv) * D)
            rec.gather_q(B["ids"], T, w["embed"], B["x"])
            rec.sandwich(T, H, eps, 1.0, B["x"], None, None, w["layers.0.input_layernorm"], B["normed"])
            for i in range(self.layers):
                p = f"layers.{i}."
                if i in debug_layers:
                    snaps[i] = rec.snapshot(B["x"], T * H * 2, np.float16, (T, H))
                rec.matmul(B["normed"], w[p + "qkv"], z, T)
                rec.qk_norm_rope(T, h, kv, D, self.stride, z, w[p + "q_norm"], w[p + "k_norm"], True,
                                 B["meta"].at(12), 4, eps, self.theta, D, _dj.ROPE_INV_POW)
                rec.attention(T, h, kv, D, z, self.stride, src, src, B["rng"], self.scale, B["y"])
                rec.matmul(B["y"], w[p + "o"], B["o"], T)
                rec.sandwich(T, H, eps, 1.0, B["x"], B["o"], w[p + "post_attention_layernorm"], w[p + "pre_feedforward_layernorm"], B["normed"])
                rec.matmul_glu(B["normed"], w[p + "gu"], B["h"], T, _dj.ACT_GELU_TANH)
                rec.matmul(B["h"], w[p + "down"], B["o"], T)
                nxt = f"layers.{i + 1}.input_layernorm" if i + 1 < self.layers else "final_norm"
                rec.sandwich(T, H, eps, float(self.scalars[i]), B["x"], B["o"], w[p + "post_feedforward_layernorm"], w[nxt], B["normed"])
            rec.mean_pool(T, S, H, B["normed"], B["seqs"], B["pooled"])
            rec.dense_f32(S, B["pooled"], w["head.dense1"], B["h1"])
            rec.dense_f32(S, B["h1"], w["head.dense2"], B["emb"])
        else:
            for i in debug_layers:
                snaps[i] = rec.snapshot(B["x"], T * H * 2, np.float16, (T, H))
        return snaps


def cosine_logits(state_e, question_e, option_es):
    """The cosine prior of Eg2Head.logits (eg2-head.ts:82-84, 97): cos(option, state + question)."""
    anchor = state_e.astype(np.float64) + question_e.astype(np.float64)
    an = max(float(np.sqrt((anchor * anchor).sum())), 1e-12)
    out = []
    for o in option_es:
        o = o.astype(np.float64)
        on = o / max(float(np.sqrt((o * o).sum())), 1e-12)
        out.append(float((on * anchor).sum() / an))
    return out
