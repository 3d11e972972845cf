"""The learned EmbeddingGemma 2 decision head on the host (decision_js_amd/eg2_head.py, after eg2-head.ts:44-100),
pinned on the CPU against a float64 restatement from torch library routines (F.linear, F.layer_norm, exact erf
F.gelu, F.cosine_similarity) of the head's formula:

    f = LayerNorm(field([S, Q, S*Q]) + type)       S, Q, O the projected state, question and option embeddings
    logit_i = prior cos(o_i, s + q) + gate (joint cos(f, LN(O_i)) + residual([f, On, f*On, |f - On|]))

plus its caches (one projection per text, the oldest of 4096 dropped first) and mistakes planted in it."""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")
F = torch.nn.functional

W, E = 48, 32
CFG = {"head": {"width": W, "ln_eps": 1e-5, "prior_scale": 2.5, "joint_scale": 4.0, "gate": 0.7, "residual_bias": -0.2}}


def _tensors(seed=0):
    from decision_js_amd import synth
    rng = np.random.default_rng(seed)
    t = {}
    for name, shape in synth.head_plan({"learned_head": {"width": W}, "embed_dim": E}):
        if name.endswith("norm.weight"):
            t[name] = (1 + 0.2 * rng.standard_normal(shape)).astype(np.float32)
        else:
            t[name] = (rng.standard_normal(shape) / math.sqrt(shape[-1])).astype(np.float32)
    return t


def _unit(rng):
    v = rng.standard_normal(E)
    return (v / np.linalg.norm(v)).astype(np.float32)


def _torch_head(t, qtype, s, q, opts):
    h = CFG["head"]
    T = {k: torch.from_numpy(v.astype(np.float64)) for k, v in t.items()}
    lin = lambda x, p, bias=True: F.linear(x, T[p + ".weight"], T[p + ".bias"] if bias else None)  # noqa: E731
    s, q = torch.from_numpy(s.astype(np.float64)), torch.from_numpy(q.astype(np.float64))
    S, Q = lin(s, "head.state_proj"), lin(q, "head.question_proj")
    f = lin(F.gelu(lin(torch.cat([S, Q, S * Q]), "head.field.0")), "head.field.3")
    f = f + T["head.type_emb.weight"][["choice", "score", "noul"].index(qtype)]
    f = F.layer_norm(f, (W,), T["head.field_norm.weight"], T["head.field_norm.bias"], h["ln_eps"])
    out = []
    for o in opts:
        o = torch.from_numpy(o.astype(np.float64))
        On = F.layer_norm(lin(o, "head.option_proj"), (W,), T["head.option_norm.weight"], T["head.option_norm.bias"], h["ln_eps"])
        r = F.gelu(F.linear(torch.cat([f, On, f * On, (f - On).abs()]), T["head.residual.0.weight"], T["head.residual.0.bias"]))
        res = float(T["head.residual.3.weight"].reshape(-1) @ r) + h["residual_bias"]
        joint = h["joint_scale"] * float(F.cosine_similarity(f, On, dim=0, eps=1e-8))
        prior = h["prior_scale"] * float(F.cosine_similarity(o, s + q, dim=0, eps=1e-12))
        out.append(prior + h["gate"] * (joint + res))
    return out


def _check(head_cls=None):
    from decision_js_amd.eg2_head import Eg2Head
    head_cls = head_cls or Eg2Head
    t = _tensors()
    rng = np.random.default_rng(1)
    head = head_cls(CFG, t)
    for qtype in ("choice", "score", "noul"):
        s, q = _unit(rng), _unit(rng)
        opts = [_unit(rng) for _ in range(4)]
        got = head.logits(qtype, ("s" + qtype, s), ("q" + qtype, q), [(f"o{qtype}{i}", o) for i, o in enumerate(opts)])
        want = _torch_head(t, qtype, s, q, opts)
        # f32 storage of the reference's vectors against float64 throughout: ~1e-6 relative
        assert np.abs(np.array(got) - np.array(want)).max() < 1e-4 * max(1.0, np.abs(want).max()), (got, want)


def test_eg2_head_matches_library_restatement(pkg):
    _check()


def test_planted_head_type_embedding_slip_is_caught(pkg, monkeypatch):
    from decision_js_amd import eg2_head
    monkeypatch.setattr(eg2_head, "QTYPES", ["score", "choice", "noul"])  # the type rows in the wrong order
    with pytest.raises(AssertionError):
        _check()


def test_planted_head_residual_order_slip_is_caught(pkg, monkeypatch):
    from decision_js_amd import eg2_head
    orig = eg2_head._linear

    def slip(Wt, b, x, out, frm=0, cols=None, stride=None):
        # the product and |difference| blocks of the residual's first layer swapped
        if stride is not None and stride == 4 * out and frm in (2 * out, 3 * out):
            frm = 5 * out - frm
        return orig(Wt, b, x, out, frm, cols, stride)
    monkeypatch.setattr(eg2_head, "_linear", slip)
    with pytest.raises(AssertionError):
        _check()


def test_planted_head_layernorm_slip_is_caught(pkg, monkeypatch):
    from decision_js_amd import eg2_head
    orig = eg2_head._layer_norm
    monkeypatch.setattr(eg2_head, "_layer_norm", lambda x, w, b, eps: orig(x, w, b * 0, eps))  # bias dropped
    with pytest.raises(AssertionError):
        _check()


def test_erf_within_published_bound(pkg):
    """A&S 7.1.26 against math.erf: |error| < 1.5e-7 over [-6, 6] (the bound eg2-head.ts:23 states)."""
    from decision_js_amd.eg2_head import _erf
    x = np.linspace(-6, 6, 24001)
    assert np.abs(_erf(x) - np.array([math.erf(v) for v in x])).max() < 1.5e-7


def test_head_caches_one_projection_per_text(pkg):
    """Projections are cached by text: a state, question or option seen again is not projected again, and the
    caches keep the newest 4096 texts (eg2-head.ts:53-62)."""
    from decision_js_amd import eg2_head
    calls = []
    orig = eg2_head._linear

    def spy(*a, **k):
        calls.append(a[3])
        return orig(*a, **k)
    head = eg2_head.Eg2Head(CFG, _tensors())
    rng = np.random.default_rng(2)
    s, q, o = _unit(rng), _unit(rng), [_unit(rng) for _ in range(3)]
    eg2_head._linear = spy
    try:
        a = head.logits("choice", ("s", s), ("q", q), [(str(i), v) for i, v in enumerate(o)])
        n_first = len(calls)
        calls.clear()
        b = head.logits("choice", ("s", s), ("q", q), [(str(i), v) for i, v in enumerate(o)])
    finally:
        eg2_head._linear = orig
    assert a == b
    # second call: field (2) + residual f-part (1) + per option prod and diff (2 each); no projections
    assert len(calls) == 3 + 2 * 3 < n_first
    for i in range(eg2_head.CACHE + 10):
        head._cached(head.projS, ("x", i), lambda: np.zeros(1, np.float32))
    assert len(head.projS) == eg2_head.CACHE and ("x", 0) not in head.projS and ("x", eg2_head.CACHE + 9) in head.projS
