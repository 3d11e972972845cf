"""The decision head of the EmbeddingGemma 2 typed-decision model (Eg2Head, eg2-head.ts:44-100), on the host.

    f = LayerNorm(field([S, Q, S*Q]) + type)        S, Q, O: the state, question and option embeddings, projected
    logit_i = prior * cos(o_i, s + q) + gate * (joint * cos(f, LayerNorm(O_i)) + residual([f, On, f*On, |f - On|]))

Arithmetic as the reference's host code: float64 operations on float32-stored vectors (every linear output,
GELU and LayerNorm result is stored as f32, as its Float32Arrays are; dots, norms and the final logit stay
f64). The projections of a text depend on that text only, so they are cached with it (4096 texts per cache,
the oldest dropped first): a question asked of many states costs only its field and its options' residuals.
"""
import math

import numpy as np

F32, F64 = np.float32, np.float64
QTYPES = ["choice", "score", "noul"]  # eg2-head.ts:8
CACHE = 4096  # eg2-head.ts:56


def _linear(W, b, x, out, frm=0, cols=None, stride=None):
    """y = W[:, frm:frm+cols] x + b for W [out, stride] row-major (eg2-head.ts:11-20), stored f32."""
    cols = len(x) if cols is None else cols
    stride = len(x) if stride is None else stride
    Wm = np.asarray(W, F32).reshape(out, stride)[:, frm:frm + cols].astype(F64)
    y = Wm @ np.asarray(x, F32).astype(F64)
    if b is not None:
        y = y + np.asarray(b, F32).astype(F64)
    return y.astype(F32)


def _erf(x):
    """Abramowitz & Stegun 7.1.26 (|error| < 1.5e-7), as eg2-head.ts:23-27."""
    x = np.asarray(x, F64)
    t = 1.0 / (1.0 + 0.3275911 * np.abs(x))
    y = 1.0 - ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t * np.exp(-x * x)
    return np.where(x >= 0, y, -y)


def _gelu(x):
    """Exact (erf) GELU with the A&S erf, eg2-head.ts:22; stored f32."""
    x = np.asarray(x, F32).astype(F64)
    return (0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))).astype(F32)


def _layer_norm(x, w, b, eps):
    """eg2-head.ts:29-36: mean and variance in f64, output stored f32."""
    x = np.asarray(x, F32).astype(F64)
    m = x.sum() / len(x)
    v = ((x - m) ** 2).sum()
    inv = 1.0 / math.sqrt(v / len(x) + eps)
    return ((x - m) * inv * np.asarray(w, F32) + np.asarray(b, F32)).astype(F32)


def _dot(a, b):
    return float(np.asarray(a, F32).astype(F64) @ np.asarray(b, F32).astype(F64))


def _norm(a):
    return math.sqrt(_dot(a, a))


class Eg2Head:
    """Eg2Head (eg2-head.ts:44-100): `config` the manifest config (its "head" entry: width, ln_eps, prior_scale,
    joint_scale, gate, residual_bias), `t` the head's f32 tensors by name (the manifest's "host" list)."""

    def __init__(self, config: dict, t: dict):
        self.h = config["head"]
        self.W = int(self.h["width"])
        self.t = {k: np.asarray(v, F32).reshape(-1) for k, v in t.items()}
        self.projS, self.projQ, self.terms = {}, {}, {}

    @staticmethod
    def _cached(cache: dict, key, make):
        v = cache.get(key)
        if v is None:
            if len(cache) >= CACHE:
                cache.pop(next(iter(cache)))  # the oldest text first (eg2-head.ts:56)
            v = cache[key] = make()
        return v

    def logits(self, qtype: str, s, q, opts):
        """The raw logit of every option. s, q: (key, normalized embedding) of the state and the question;
        opts: [(key, normalized embedding)] of the options (eg2-head.ts:64-99)."""
        t, W, h = self.t, self.W, self.h
        S = self._cached(self.projS, s[0], lambda: _linear(t["head.state_proj.weight"], t.get("head.state_proj.bias"), s[1], W))
        Q = self._cached(self.projQ, q[0], lambda: _linear(t["head.question_proj.weight"], t.get("head.question_proj.bias"), q[1], W))
        fin = np.concatenate([S, Q, (S.astype(F64) * Q.astype(F64)).astype(F32)])
        f1 = _gelu(_linear(t["head.field.0.weight"], t.get("head.field.0.bias"), fin, W))
        f2 = _linear(t["head.field.3.weight"], t.get("head.field.3.bias"), f1, W)
        ti = QTYPES.index(qtype) * W
        f2 = (f2.astype(F64) + t["head.type_emb.weight"][ti:ti + W].astype(F64)).astype(F32)
        f = _layer_norm(f2, t["head.field_norm.weight"], t["head.field_norm.bias"], h["ln_eps"])
        f_norm = _norm(f)
        R0, rb, R3 = t["head.residual.0.weight"], t["head.residual.0.bias"], t["head.residual.3.weight"]
        # the residual's first layer W [f, On, f*On, |f - On|] = W_f f + W_o On + W_m (f*On) + W_a |f - On|
        rf = _linear(R0, rb, f, W, 0, W, 4 * W)
        anchor = (np.asarray(s[1], F32).astype(F64) + np.asarray(q[1], F32).astype(F64)).astype(F32)
        an = max(_norm(anchor), 1e-12)
        out = []
        for key, e in opts:
            def make(e=e):
                O = _linear(t["head.option_proj.weight"], t.get("head.option_proj.bias"), e, W)
                on = _layer_norm(O, t["head.option_norm.weight"], t["head.option_norm.bias"], h["ln_eps"])
                ev = np.asarray(e, F32)
                return {"o": (ev.astype(F64) / max(_norm(ev), 1e-12)).astype(F32), "on": on, "on_norm": _norm(on),
                        "r": _linear(R0, None, on, W, W, W, 4 * W)}
            o = self._cached(self.terms, key, make)
            prod = (f.astype(F64) * o["on"].astype(F64)).astype(F32)
            diff = np.abs(f.astype(F64) - o["on"].astype(F64)).astype(F32)
            rm = _linear(R0, None, prod, W, 2 * W, W, 4 * W)
            ra = _linear(R0, None, diff, W, 3 * W, W, 4 * W)
            pre = (rf.astype(F64) + o["r"].astype(F64) + rm.astype(F64) + ra.astype(F64))
            res = float(h["residual_bias"]) + float(R3[:W].astype(F64) @ (0.5 * pre * (1.0 + _erf(pre / math.sqrt(2.0)))))
            joint = h["joint_scale"] * _dot(f, o["on"]) / max(f_norm * o["on_norm"], 1e-8)
            prior = h["prior_scale"] * _dot(o["o"], anchor) / an
            out.append(prior + h["gate"] * (joint + res))
        return out
