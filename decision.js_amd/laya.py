"""Laya's engine (LayaEngine, src/laya-engine.ts) on libdj.so: a ModernBERT encoder — the embedding rows under a
bias-free LayerNorm; per layer RoPE attention (layer 0 reads the stream itself, later layers a bias-free
LayerNorm of it) over the whole sequence on the global layers and a +-window on the others, then LayerNorm and
the GeGLU MLP (erf GELU) — then d1-omni's decision head and scorer at each option marker. One question is one
sequence; many are packed on one token axis and recorded as one forward.
"""
import math

import numpy as np

from . import _dj
from .engine import GpuEngine, load_weights
from .omni import OmniEngine, pack_omni


def pack_laya(seqs, window):
    """LayaEngine.logits's packing (laya-engine.ts:57-66): pack_omni's ids, positions, question types, whole-
    sequence key ranges and marker rows, plus each token's window [max(start, t - window), min(end, t + window
    + 1)) for the local layers."""
    pk = pack_omni(seqs)
    t = np.arange(pk["T"], dtype=np.int64)
    win = np.zeros((pk["T"], 4), dtype=np.int32)
    win[:, 0] = np.maximum(pk["rng"][:, 0], t - window)
    win[:, 1] = np.minimum(pk["rng"][:, 1], t + window + 1)
    pk["win"] = win
    return pk


class LayaEngine(OmniEngine):
    """The encoder loop of laya-engine.ts:99-115 with dj_add_layernorm (a zero bias for the bias-free norms),
    dj_qk_norm_rope (no norms: plain RoPE over the whole head, pow(theta, -2d/D) per layer type), dj_attention
    on the sequence or window ranges at 1/sqrt(D), and the erf-GELU GLU epilogue on the Wi product; the head
    is OmniEngine's."""

    @classmethod
    def load(cls, base: str, opts: dict = None):
        ctx, m, w = load_weights(base, opts)
        c = m["config"]
        if c.get("model") != "laya":
            raise ValueError(f"decision.js: {base} is not a Laya export ({c.get('model')})")
        bad = sorted({t for t in c["layer_types"] if t not in ("full_attention", "sliding_attention")})
        if bad:
            raise ValueError(f"decision.js: unsupported layer types {bad}")
        for t in set(c["layer_types"]):
            if t not in c["rope_theta"]:
                raise ValueError(f"decision.js: no rope_theta for {t} layers")
        if c["hidden"] % c["heads"] or c["hidden"] // c["heads"] not in (64, 128, 256):
            raise ValueError(f"decision.js: encoder width {c['hidden']} / {c['heads']} heads (64, 128 or 256 per head)")
        if c["hidden"] % c["head_heads"] or c["hidden"] // c["head_heads"] not in (64, 128, 256):
            raise ValueError(f"decision.js: head width {c['hidden']} / {c['head_heads']} heads (64, 128 or 256 per head)")
        return cls(ctx, m, w, opts)

    def __init__(self, ctx, m, w, opts=None):
        GpuEngine.__init__(self, ctx, m, w, opts)
        c = m["config"]
        self.H, self.I, self.h = c["hidden"], c["intermediate"], c["heads"]
        self.kv, self.D = self.h, self.H // self.h
        self.layers, self.types = c["layers"], c["layer_types"]
        self.conv, self.eps, self.window = False, c["eps"], c["window"]
        self.stride = 3 * self.H
        self.capacity = self.leaf_capacity = self.marker_capacity = 0
        self.hh, self.ff, self.ln_eps = c["head_heads"], c["head_ff"], c["ln_eps"]
        self.head_layers = c["head_layers"]
        self.Dh = self.H // self.hh
        self.type_rows = int(w["head.type_emb"].host.shape[0])
        self.zeros = ctx.array(np.zeros(self.H, dtype=np.float16))  # the bias of the bias-free LayerNorms

    def ensure(self, T: int, M: int = 0, n_ids: int = 0):
        """Activation buffers for T tokens and M markers (laya-engine.ts:38-47: grown, never shrunk)."""
        if T <= self.capacity and M <= self.marker_capacity:
            return
        cap = (max(T, self.capacity, 256) + 63) // 64 * 64
        mcap = max(M, self.marker_capacity, 64)
        H = self.H
        self._alloc({"x": cap * H * 2, "normed": cap * H * 2, "o": cap * H * 2, "z": cap * 3 * H * 2, "y": cap * H * 2,
                     "h": cap * max(self.I, self.ff) * 2, "ids": cap * 4, "pos": cap * 4, "qtype": cap * 4,
                     "rng": cap * 16, "win": cap * 16, "markers": mcap * 4, "g": mcap * H * 2, "gf": mcap * H * 2,
                     "out": mcap * 4})
        self.capacity, self.marker_capacity = cap, mcap

    INPUTS = ("ids", "pos", "qtype", "rng", "win", "markers")

    def logits(self, seqs, debug=False):
        """Raw marker logits per sequence ([seq][marker], before the temperature), and with `debug` the encoder's
        output (after final_norm) and the head's residual stream before the scorer, f16 [T, H]."""
        pk = pack_laya(seqs, self.window)
        if pk["T"] == 0:
            return {"logits": [[] for _ in seqs], "debug": {}}
        return self._forward_omni(pk, seqs, debug, None)

    def stage(self, seqs):
        """Packs `seqs` and keeps the packed inputs in device memory (the benchmark's resident inputs)."""
        pk = pack_laya(seqs, self.window)
        return {"pk": pk, "seqs": seqs, "bufs": {k: self.ctx.array(pk[k]) for k in self.INPUTS if len(pk[k])}}

    def _layers(self, rec, T, B):
        """The encoder (laya-engine.ts:99-115); its output lands in B["normed"] as the head expects."""
        c, w = self.m["config"], self.w
        H, h, D, eps, zeros = self.H, self.h, self.D, self.eps, self.zeros
        z = B["z"]
        src = _dj.kv_src(z, T, 3 * H, H, 2 * H)
        rec.gather_q(B["ids"], T, w["embed"], B["normed"])
        rec.add_layernorm(T, H, False, eps, B["normed"], B["o"], w["embed_norm"], zeros, B["x"])
        for i, t in enumerate(self.types):
            p = f"layers.{i}."
            inp = B["x"]
            if p + "attn_norm" in w:  # adds the previous layer's MLP output (every layer but the first)
                rec.add_layernorm(T, H, True, eps, B["x"], B["o"], w[p + "attn_norm"], zeros, B["normed"])
                inp = B["normed"]
            rec.matmul(inp, w[p + "qkv"], z, T)
            rec.qk_norm_rope(T, h, h, D, 3 * H, z, None, None, False, B["pos"], 1, eps, c["rope_theta"][t], D,
                             _dj.ROPE_POW_NEG)
            rec.attention(T, h, h, D, z, 3 * H, src, src, B["rng" if t == "full_attention" else "win"],
                          1.0 / math.sqrt(D), B["y"])
            rec.matmul(B["y"], w[p + "o"], B["o"], T)
            rec.add_layernorm(T, H, True, eps, B["x"], B["o"], w[p + "mlp_norm"], zeros, B["normed"])
            rec.matmul_glu(B["normed"], w[p + "wi"], B["h"], T, _dj.ACT_GELU_ERF)
            rec.matmul(B["h"], w[p + "wo"], B["o"], T)
        rec.add_layernorm(T, H, True, eps, B["x"], B["o"], w["final_norm"], zeros, B["normed"])

    def destroy(self):
        if self.zeros is not None:
            self.zeros.free()
            self.zeros = None
        super().destroy()
