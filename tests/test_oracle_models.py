"""Pins the oracle's whole forwards and the parts of its kernels the single-op checks leave open (CPU only).

* decoder_forward (oracle/ref.py) against `transformers`' Qwen3Model (QK-norm, the configs[1] / configs[4] form)
  and Qwen2Model with zero q/k/v biases (no QK-norm, q4: the configs[2] form), random-init architectures built
  offline and loaded with the oracle's own f16-dequantized weights, run in float64. The library's layer wiring
  is independent of ours: which norm weight sits where, which half of w13 is the gate, GQA, the final norm and
  the tied head (d1-3b-engine.ts:86-106; LEAF_LOGITS kernels.ts:149-185).
* encoder_forward against a float64 restatement built from torch library routines (F.rms_norm,
  F.scaled_dot_product_attention, F.gelu(approximate="tanh"), RoPE as a complex rotation), following
  Eg2Engine.embed (eg2-engine.ts:103-139) without per-layer embeddings.
* qk_norm_rope's norm half (q with qn, k with kn, plain v-norm; kernels.ts:100-104, eg2-kernels.ts:76-81),
  gelu_tanh (eg2-kernels.ts:9-13) against erf-GELU and torch's tanh GELU, attention over kept K/V rows
  (the shared-state mode) against the concatenated-rows form, and the shared trunk invariant of the causal
  decoder (d3-engine.ts:67-93) on the oracle itself.

Each check comes with mistakes planted in the oracle that it must catch.
"""
import math

import numpy as np
import pytest

from oracle import ref

torch = pytest.importorskip("torch")
F = torch.nn.functional

TINY_DEC = dict(layers=2, hidden=64, intermediate=96, heads=4, kv_heads=2, head_dim=16, vocab=512)
TINY_ENC = dict(layers=2, hidden=64, intermediate=96, heads=2, kv_heads=1, head_dim=32, vocab=512, head_width=128,
                embed_dim=64)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.float64)))


def _rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


# ---------------------------------------------------------------- decoder_forward vs transformers

@pytest.fixture(scope="module")
def tiny_decoders(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("dec")
    # unit-gain weights (std 1/sqrt(hidden)): every branch moves the residual stream as much as the embedding
    q3 = synth.generate(synth.reduced("qwen3-0.6b-q8", **TINY_DEC), str(d / "qwen3"), norm_std=0.1, std=0.125)
    q2 = synth.generate(synth.reduced("qwen2.5-3b-q4", **TINY_DEC), str(d / "qwen2"), norm_std=0.1, std=0.125)
    return {"qwen3": q3, "qwen2": q2}


def _hf_decoder(model: ref.Model):
    """A transformers Qwen3Model (QK-norm) or Qwen2Model (none) holding the oracle model's f16 weights."""
    tr = pytest.importorskip("transformers")
    c = model.c
    H, I, h, kv, D = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"]
    common = dict(vocab_size=c["vocab"], hidden_size=H, intermediate_size=I, num_hidden_layers=c["layers"],
                  num_attention_heads=h, num_key_value_heads=kv, rms_norm_eps=c["eps"], rope_theta=c["rope_theta"],
                  max_position_embeddings=4096, tie_word_embeddings=True)
    if c.get("qk_norm"):
        cfg = tr.Qwen3Config(head_dim=D, attention_bias=False, **common)
        m = tr.Qwen3Model(cfg)
    else:
        assert H // h == D
        cfg = tr.Qwen2Config(**common)
        m = tr.Qwen2Model(cfg)
    m.config._attn_implementation = "eager"
    m = m.to(torch.float64).eval()
    sd = {"embed_tokens.weight": _t(model.w16("embed")), "norm.weight": _t(model.t["final_norm"])}
    for i in range(c["layers"]):
        p, q = f"layers.{i}.", f"layers.{i}."
        qkv = model.w16(p + "qkv")
        sd[q + "self_attn.q_proj.weight"] = _t(qkv[:h * D])
        sd[q + "self_attn.k_proj.weight"] = _t(qkv[h * D:(h + kv) * D])
        sd[q + "self_attn.v_proj.weight"] = _t(qkv[(h + kv) * D:])
        sd[q + "self_attn.o_proj.weight"] = _t(model.w16(p + "o_proj"))
        w13 = model.w16(p + "w13")
        sd[q + "mlp.gate_proj.weight"] = _t(w13[:I])
        sd[q + "mlp.up_proj.weight"] = _t(w13[I:])
        sd[q + "mlp.down_proj.weight"] = _t(model.w16(p + "w2"))
        sd[q + "input_layernorm.weight"] = _t(model.t[p + "operator_norm"])
        sd[q + "post_attention_layernorm.weight"] = _t(model.t[p + "ffn_norm"])
        if c.get("qk_norm"):
            sd[q + "self_attn.q_norm.weight"] = _t(model.t[p + "q_norm"])
            sd[q + "self_attn.k_norm.weight"] = _t(model.t[p + "k_norm"])
        else:
            for n in ("q", "k", "v"):
                sd[q + f"self_attn.{n}_proj.bias"] = torch.zeros_like(m.state_dict()[q + f"self_attn.{n}_proj.bias"])
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def _forest(rng, V):
    trunk = [int(x) for x in rng.integers(0, V, 21)]
    branches = [[int(x) for x in rng.integers(0, V, n)] for n in (9, 1, 14)]
    groups = [[[int(a)] for a in rng.choice(V, n, replace=False)] for n in (2, 3, 5)]
    return {"trunk": trunk, "branches": branches, "groups": groups}


def _compare_decoder(path, model=None):
    """The oracle's forest forward (float64 accumulation, f16 storage points) against the library model run on
    each trunk + branch sequence alone: the residual stream after layer 0 and the final normed hidden state at
    every token within 5e-3 relative L2 (f16 rounding of the stored activations is ~1e-3), and the answer
    logits (normed leaf row . f32-dequantized embedding rows) within 5e-3 of their scale."""
    model = model or ref.Model(path)
    c = model.c
    rng = np.random.default_rng(11)
    tree = _forest(rng, c["vocab"])
    ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest([tree])
    mask = ref.ranges_mask(ref.forest_ranges(meta), len(ids))
    logits, _, dbg = ref.decoder_forward(model, ids, pos, mask, leaves, leaf_ids, n_ids, acc=np.float64,
                                         debug_layers=(0, c["layers"] - 1))
    hf = _hf_decoder(ref.Model(path))  # the library side always reads the untouched file
    ec, es, eb = model.t["embed"]
    E32 = ref.dequant_f32(ec, es, eb).astype(np.float64)
    P = len(tree["trunk"])
    off = P
    for b, br in enumerate(tree["branches"]):
        seq = tree["trunk"] + br
        rows = list(range(P)) + list(range(off, off + len(br)))
        off += len(br)
        with torch.no_grad():
            out = hf(input_ids=torch.tensor([seq]), output_hidden_states=True)
        layer0 = out.hidden_states[1][0].numpy()
        final = out.last_hidden_state[0].numpy()
        assert _rel_l2(dbg[0][rows], layer0) < 5e-3, f"branch {b}: residual after layer 0"
        x = dbg[c["layers"] - 1][rows].astype(np.float64)  # the oracle's last residual, normed here in float64
        normed = x / np.sqrt((x * x).mean(-1, keepdims=True) + c["eps"]) * model.t["final_norm"].astype(np.float64)
        assert _rel_l2(normed, final) < 5e-3, f"branch {b}: final hidden state"
        want = final[-1] @ E32[leaf_ids[b * n_ids:(b + 1) * n_ids]].T
        got = logits[b * n_ids:(b + 1) * n_ids].astype(np.float64)
        assert np.abs(got - want).max() < 5e-3 * np.abs(want).max(), f"branch {b}: answer logits"


@pytest.mark.parametrize("name", ["qwen3", "qwen2"])
def test_decoder_forward_matches_transformers(tiny_decoders, name):
    _compare_decoder(tiny_decoders[name])


def _planted(path, mutate):
    model = ref.Model(path)
    mutate(model)
    with pytest.raises(AssertionError):
        _compare_decoder(path, model)


def test_planted_decoder_norm_swap_is_caught(tiny_decoders):
    def swap(m):
        t = m.t
        t["layers.1.operator_norm"], t["layers.1.ffn_norm"] = t["layers.1.ffn_norm"], t["layers.1.operator_norm"]
    _planted(tiny_decoders["qwen3"], swap)


def test_planted_decoder_qk_norm_swap_is_caught(tiny_decoders):
    def swap(m):
        t = m.t
        t["layers.0.q_norm"], t["layers.0.k_norm"] = t["layers.0.k_norm"], t["layers.0.q_norm"]
    _planted(tiny_decoders["qwen3"], swap)


def test_planted_decoder_final_norm_slip_is_caught(tiny_decoders):
    def drop(m):
        m.t["final_norm"] = np.ones_like(m.t["final_norm"])
    _planted(tiny_decoders["qwen2"], drop)


def test_planted_decoder_gate_up_swap_is_caught(tiny_decoders, monkeypatch):
    orig = ref.silu_mul
    monkeypatch.setattr(ref, "silu_mul", lambda a, b, acc=np.float32: orig(b, a, acc))
    with pytest.raises(AssertionError):
        _compare_decoder(tiny_decoders["qwen3"])


def test_planted_decoder_gqa_slip_is_caught(tiny_decoders, monkeypatch):
    """Query head h reading kv head h % kv instead of h / (heads / kv)."""
    orig = ref.attention

    def slip(Z, heads, kv, D, mask, scale, acc=np.float32, q_stride=None, kv_rows=None):
        q = Z[:, :heads * D].reshape(len(Z), heads, D)
        perm = [h % kv * (heads // kv) + h // kv for h in range(heads)]  # inverse of the grouping
        Z2 = Z.copy()
        Z2[:, :heads * D] = q[:, perm].reshape(len(Z), -1)
        out = orig(Z2, heads, kv, D, mask, scale, acc, q_stride, kv_rows).reshape(len(Z), heads, D)
        inv = np.argsort(perm)
        return out[:, inv].reshape(len(Z), -1)
    monkeypatch.setattr(ref, "attention", slip)
    with pytest.raises(AssertionError):
        _compare_decoder(tiny_decoders["qwen3"])


# ---------------------------------------------------------------- shared state (kept K/V) on the oracle

def test_shared_state_equals_forest_on_oracle(tiny_decoders):
    """A state prefilled once with its K/V kept, then each question run alone against the kept rows
    (kv_prefix), gives the same answer logits as the forest that packs state + questions in one forward: the
    causal invariant of d3-engine.ts:67-93, on the oracle's kv_rows path."""
    model = ref.Model(tiny_decoders["qwen3"])
    rng = np.random.default_rng(13)
    tree = _forest(rng, model.c["vocab"])
    ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest([tree])
    mask = ref.ranges_mask(ref.forest_ranges(meta), len(ids))
    want, _, _ = ref.decoder_forward(model, ids, pos, mask, leaves, leaf_ids, n_ids, acc=np.float64)
    P = len(tree["trunk"])
    st = np.array(tree["trunk"], np.uint32)
    _, kept, _ = ref.decoder_forward(model, st, np.arange(P, dtype=np.int32), np.tril(np.ones((P, P), bool)), [], None, 0,
                                     acc=np.float64, keep_kv=True)
    for b, br in enumerate(tree["branches"]):
        n = len(br)
        qmask = np.concatenate([np.ones((n, P), bool), np.tril(np.ones((n, n), bool))], axis=1)
        lid = leaf_ids[b * n_ids:(b + 1) * n_ids]
        got, _, _ = ref.decoder_forward(model, np.array(br, np.uint32), np.arange(P, P + n, dtype=np.int32), qmask,
                                        [n - 1], lid, n_ids, acc=np.float64, kv_prefix=kept)
        assert np.abs(got - want[b * n_ids:(b + 1) * n_ids]).max() < 1e-9


def test_attention_kv_rows_equals_concatenated_rows():
    """attention() over separate kept rows [k | v] equals attention over the same keys laid in Z itself."""
    rng = np.random.default_rng(14)
    h, kv, D, P, T = 4, 2, 8, 6, 5
    prefix = rng.standard_normal((P, (h + 2 * kv) * D)).astype(np.float16)
    Z = rng.standard_normal((T, (h + 2 * kv) * D)).astype(np.float16)
    rows = np.concatenate([prefix[:, h * D:], Z[:, h * D:]])
    mask = np.concatenate([np.ones((T, P), bool), np.tril(np.ones((T, T), bool))], axis=1)
    mask[2, 1] = False
    got = ref.attention(Z, h, kv, D, mask, 0.4, np.float64, kv_rows=rows)
    # the same keys as rows of one [P + T] array, queries at the last T rows
    full = np.concatenate([prefix, Z])
    fmask = np.zeros((P + T, P + T), bool)
    fmask[P:] = mask
    fmask[:P, 0] = True
    want = ref.attention(full, h, kv, D, fmask, 0.4, np.float64)[P:]
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # and a slip that drops the kept rows (queries see only their own rows) differs
    bad = ref.attention(Z, h, kv, D, mask[:, P:], 0.4, np.float64)
    assert not np.array_equal(got.view(np.uint16), bad.view(np.uint16))


# ---------------------------------------------------------------- qk_norm_rope: the norm half

def _check_qkv_norm_rope(mode, vnorm):
    """Per head: q * rsqrt(mean q^2 + eps) * qn, k likewise with kn, v plain-normed when vnorm (else untouched),
    then RoPE as multiplication by exp(i pos f_d) on the (d, d + D/2) pairs of q and k, in float64."""
    rng = np.random.default_rng(15)
    T, h, kv, D, eps, theta = 4, 3, 1, 16, 1e-6, 1e4
    Z = (rng.standard_normal((T, (h + 2 * kv) * D)) * 3).astype(np.float16)
    qn = (1 + rng.standard_normal(D) * 0.3).astype(np.float16)
    kn = (1 + rng.standard_normal(D) * 0.3).astype(np.float16)
    pos = np.array([0, 3, 17, 250], np.int32)
    got = ref.qk_norm_rope(Z, h, kv, D, pos, qn, kn, vnorm, eps, theta, mode=mode, acc=np.float64).astype(np.float64)
    z = Z.astype(np.float64).reshape(T, h + 2 * kv, D)
    g = got.reshape(T, h + 2 * kv, D)
    d = np.arange(D // 2)
    f = theta ** (-2.0 * d / D) if mode == 0 else 1.0 / theta ** (2.0 * d / D)
    for t in range(T):
        for j in range(h + 2 * kv):
            v = z[t, j]
            r = v / math.sqrt((v * v).mean() + eps)
            if j < h:
                r = r * qn.astype(np.float64)
            elif j < h + kv:
                r = r * kn.astype(np.float64)
            else:
                want = r if vnorm else v
                assert np.abs(g[t, j] - want).max() <= 2 ** -10 * np.abs(want).max()
                continue
            c = (r[:D // 2] + 1j * r[D // 2:]) * np.exp(1j * pos[t] * f)
            want = np.concatenate([c.real, c.imag])
            assert np.abs(g[t, j] - want).max() <= 2 ** -9 * np.abs(want).max()


@pytest.mark.parametrize("mode,vnorm", [(0, False), (1, True)])
def test_qkv_norm_rope_closed_form(mode, vnorm):
    _check_qkv_norm_rope(mode, vnorm)


def test_planted_qk_norm_weight_swap_is_caught(monkeypatch):
    orig = ref.qk_norm_rope
    monkeypatch.setattr(ref, "qk_norm_rope", lambda Z, h, kv, D, pos, qn=None, kn=None, *a, **k: orig(Z, h, kv, D, pos, kn, qn, *a, **k))
    with pytest.raises(AssertionError):
        _check_qkv_norm_rope(0, False)


def test_planted_vnorm_slip_is_caught(monkeypatch):
    orig = ref.qk_norm_rope
    monkeypatch.setattr(ref, "qk_norm_rope", lambda Z, h, kv, D, pos, qn=None, kn=None, vnorm=False, *a, **k: orig(Z, h, kv, D, pos, qn, kn, False, *a, **k))
    with pytest.raises(AssertionError):
        _check_qkv_norm_rope(1, True)


# ---------------------------------------------------------------- gelu_tanh

def _check_gelu(fn):
    """The tanh GELU against (1) torch's F.gelu(approximate="tanh") in float64 (the same formula, a library
    routine) to 1e-12 wherever the +-15 clamp is inactive, and (2) the exact erf GELU within the tanh form's
    approximation error, below 5e-4 everywhere (the tanh form's largest deviation is 4.73e-4, near |x| = 2.2);
    saturated at the clamp."""
    x = np.concatenate([np.linspace(-8, 8, 4001), [-30.0, -20.0, 20.0, 30.0]])
    got = fn(x)
    lib = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    inner = np.abs(0.7978845608 * (x + 0.044715 * x ** 3)) < 15
    assert np.abs(got[inner] - lib[inner]).max() < 1e-9
    from scipy.special import erf
    exact = 0.5 * x * (1 + erf(x / math.sqrt(2)))
    assert np.abs(got - exact).max() < 5e-4


def test_gelu_tanh_vs_library_and_erf():
    _check_gelu(ref.gelu_tanh)


def test_planted_gelu_dropped_cubic_is_caught():
    def slip(x):
        u = np.clip(0.7978845608 * x, -15.0, 15.0)
        e = np.exp(2.0 * u)
        return 0.5 * x * (1.0 + (e - 1.0) / (e + 1.0))
    with pytest.raises(AssertionError):
        _check_gelu(slip)


# ---------------------------------------------------------------- encoder_forward vs a torch-library restatement

@pytest.fixture(scope="module")
def tiny_encoder(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("enc")
    return synth.generate(synth.reduced("eg2-encoder-q8", **TINY_ENC), str(d / "eg2"), norm_std=0.1, std=0.125)


def _torch_encoder(model: ref.Model, seqs):
    """Each text alone, float64, library routines: embedding rows (sqrt(H) folded in) -> rms_norm(input_layernorm)
    -> per layer [qkv, q/k rms_norm with weights and plain v rms_norm, RoPE exp(i pos / theta^(2d/D)),
    bidirectional SDPA (scale 1, GQA), o, x += rms_norm(o) post_attention_layernorm, rms_norm(x)
    pre_feedforward_layernorm, gate|up, gelu_tanh(gate) up, down, x = (x + rms_norm(o) post_ff) * scalar, rms_norm(x)
    with the next layer's input norm or final_norm] -> mean over the text -> dense1, dense2 (f32-dequantized) ->
    L2 normalisation."""
    c = model.c
    H, I, h, kv, D, eps, theta = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["eps"], c["rope_theta"]
    L = c["layers"]

    def W(name):
        return _t(model.w16(name))

    def nw(name):
        return _t(model.t[name])

    def rms(x, w=None):
        return F.rms_norm(x, (x.shape[-1],), weight=w, eps=eps)

    E = W("embed")
    out = []
    for s in seqs:
        n = len(s)
        x = E[torch.tensor(s)]
        normed = rms(x, nw("layers.0.input_layernorm"))
        ang = torch.arange(n, dtype=torch.float64)[:, None] / theta ** (torch.arange(D // 2, dtype=torch.float64) * 2 / D)
        rot = torch.polar(torch.ones_like(ang), ang)
        for i in range(L):
            p = f"layers.{i}."
            z = normed @ W(p + "qkv").T
            q = rms(z[:, :h * D].reshape(n, h, D), nw(p + "q_norm"))
            k = rms(z[:, h * D:(h + kv) * D].reshape(n, kv, D), nw(p + "k_norm"))
            v = rms(z[:, (h + kv) * D:].reshape(n, kv, D))

            def rope(a):
                cplx = torch.complex(a[..., :D // 2], a[..., D // 2:]) * rot[:, None, :]
                return torch.cat([cplx.real, cplx.imag], -1)
            q, k = rope(q), rope(k)
            k = k.repeat_interleave(h // kv, dim=1)
            v = v.repeat_interleave(h // kv, dim=1)
            y = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), scale=1.0)
            y = y.transpose(0, 1).reshape(n, h * D)
            o = y @ W(p + "o").T
            x = x + rms(o, nw(p + "post_attention_layernorm"))
            normed = rms(x, nw(p + "pre_feedforward_layernorm"))
            gu = normed @ W(p + "gu").T
            o = (F.gelu(gu[:, :I], approximate="tanh") * gu[:, I:]) @ W(p + "down").T
            x = (x + rms(o, nw(p + "post_feedforward_layernorm"))) * c.get("layer_scalars", [1.0] * L)[i]
            normed = rms(x, nw(f"layers.{i + 1}.input_layernorm" if i + 1 < L else "final_norm"))
        pooled = normed.mean(0)
        d1 = _t(ref.dequant_f32(*model.t["head.dense1"]))
        d2 = _t(ref.dequant_f32(*model.t["head.dense2"]))
        e = (pooled @ d1.T) @ d2.T
        out.append((e / e.norm()).numpy())
    return np.stack(out)


def _compare_encoder(path, model=None):
    model = model or ref.Model(path)
    rng = np.random.default_rng(16)
    seqs = [[int(x) for x in rng.integers(0, model.c["vocab"], n)] for n in (23, 8, 1, 12)]
    got = ref.encoder_forward(model, seqs, acc=np.float64)
    want = _torch_encoder(ref.Model(path), seqs)  # the untouched file
    for i in range(len(seqs)):
        assert _rel_l2(got[i], want[i]) < 5e-3, f"text {i}"


def test_encoder_forward_matches_library_restatement(tiny_encoder):
    _compare_encoder(tiny_encoder)


def test_planted_encoder_sandwich_swap_is_caught(tiny_encoder):
    model = ref.Model(tiny_encoder)
    t = model.t
    p = "layers.1."
    t[p + "post_attention_layernorm"], t[p + "pre_feedforward_layernorm"] = t[p + "pre_feedforward_layernorm"], t[p + "post_attention_layernorm"]
    with pytest.raises(AssertionError):
        _compare_encoder(tiny_encoder, model)


def test_planted_encoder_gate_up_swap_is_caught(tiny_encoder, monkeypatch):
    orig = ref.gelu_mul
    monkeypatch.setattr(ref, "gelu_mul", lambda a, b, acc=np.float32: orig(b, a, acc))
    with pytest.raises(AssertionError):
        _compare_encoder(tiny_encoder)


def test_planted_encoder_rope_position_slip_is_caught(tiny_encoder, monkeypatch):
    """RoPE at twice the position within the text (a stride slip; a constant offset per text would be invisible,
    since bidirectional RoPE scores depend only on position differences)."""
    orig = ref.pack_encoder

    def slip(seqs, window=None):
        ids, meta, full, slide, ranges = orig(seqs, window)
        meta = meta.copy()
        meta[:, 3] = 2 * meta[:, 3]
        return ids, meta, full, slide, ranges
    monkeypatch.setattr(ref, "pack_encoder", slip)
    with pytest.raises(AssertionError):
        _compare_encoder(tiny_encoder)


# ---------------------------------------------------------------- LFM2 short conv (d1-3B's conv layers)

def _check_short_conv(fn=None):
    """SHORT_CONV against an element-by-element float64 loop: y[t, c] = C[t, c] * sum_j w[c, j] * B[s_j, c] *
    U[s_j, c] over the three taps s_j of token t (a tap < 0 contributes nothing), with Z = [B | C | U]."""
    fn = fn or ref.short_conv
    rng = np.random.default_rng(40)
    T, H = 7, 16
    Z = rng.standard_normal((T, 3 * H)).astype(np.float16)
    w = rng.standard_normal((H, 3)).astype(np.float16)
    taps = np.array([[-1, -1, 0, 0], [-1, 0, 1, 0], [0, 1, 2, 0], [1, 2, 3, 0], [-1, -1, 4, 0], [1, 2, 5, 0], [-1, 5, 6, 0]],
                    np.int32)
    got = fn(Z, H, w, taps, np.float64).astype(np.float64)
    z = Z.astype(np.float64)
    for t in range(T):
        for c in range(H):
            conv = sum(float(w[c, j]) * z[taps[t, j], c] * z[taps[t, j], 2 * H + c] for j in range(3) if taps[t, j] >= 0)
            want = z[t, H + c] * conv
            assert abs(got[t, c] - want) <= 2 ** -10 * abs(want) + 1e-6


def test_short_conv_closed_form():
    _check_short_conv()


def test_planted_short_conv_slips_are_caught():
    """Taps applied in reverse order, and C and U swapped in the [B | C | U] split."""
    with pytest.raises(AssertionError):
        _check_short_conv(lambda Z, H, w, taps, acc: ref.short_conv(Z, H, w[:, ::-1].copy(), taps, acc))

    def swapped(Z, H, w, taps, acc):
        Z2 = Z.copy()
        Z2[:, H:2 * H], Z2[:, 2 * H:] = Z[:, 2 * H:], Z[:, H:2 * H]
        return ref.short_conv(Z2, H, w, taps, acc)
    with pytest.raises(AssertionError):
        _check_short_conv(swapped)


def _check_forest_taps(fn=None):
    """Brute force: a token's taps are the packed rows of the two tokens before it and itself in its own
    sequence (its tree's trunk, then its branch), -1 past the sequence's start."""
    fn = fn or ref.forest_taps
    rng = np.random.default_rng(41)
    for _ in range(10):
        trees = [{"trunk": [0] * int(rng.integers(0, 4)), "branches": [[0] * int(rng.integers(1, 4)) for _ in range(rng.integers(0, 3))],
                  "groups": []} for _ in range(3)]
        taps = fn(trees)
        rows, off = [], 0
        for tr in trees:
            trunk = list(range(off, off + len(tr["trunk"])))
            rows += [trunk[:i + 1] for i in range(len(trunk))]
            off += len(trunk)
            for br in tr["branches"]:
                own = list(range(off, off + len(br)))
                rows += [trunk + own[:o + 1] for o in range(len(br))]
                off += len(br)
        assert len(taps) == len(rows)
        for t, seq in enumerate(rows):
            want = ([-1, -1] + seq)[-3:]
            assert list(taps[t, :3]) == want, (t, seq, taps[t])


def test_forest_taps_brute_force():
    _check_forest_taps()


def test_planted_forest_taps_slip_is_caught():
    """Branch taps that reach back into the previous branch (packed order) instead of the trunk."""
    def slip(trees):
        taps, n = [], 0
        for tr in trees:
            L = len(tr["trunk"]) + sum(len(b) for b in tr["branches"])
            for i in range(L):
                taps.append((n + i - 2 if i >= 2 else -1, n + i - 1 if i >= 1 else -1, n + i, 0))
            n += L
        return np.array(taps, dtype=np.int32).reshape(-1, 4)
    with pytest.raises(AssertionError):
        _check_forest_taps(slip)


TINY_LFM2 = dict(layers=3, hidden=64, intermediate=96, heads=4, kv_heads=2, head_dim=16, vocab=512,
                 layer_types=["conv", "full_attention", "conv"])


@pytest.fixture(scope="module")
def tiny_lfm2(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("lfm2")
    return synth.generate(synth.reduced("lfm2-d1-3b-q4", **TINY_LFM2), str(d / "lfm2"), norm_std=0.1, std=0.125)


def _hf_lfm2(model: ref.Model):
    """A transformers Lfm2Model holding the oracle model's f16 weights (float64)."""
    tr = pytest.importorskip("transformers")
    c = model.c
    H, I, h, kv = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"]
    cfg = tr.Lfm2Config(vocab_size=c["vocab"], hidden_size=H, intermediate_size=I, num_hidden_layers=c["layers"],
                        num_attention_heads=h, num_key_value_heads=kv, norm_eps=c["eps"], rope_theta=c["rope_theta"],
                        layer_types=c["layer_types"], conv_L_cache=3, conv_bias=False, block_auto_adjust_ff_dim=False,
                        max_position_embeddings=4096, tie_word_embeddings=True)
    m = tr.Lfm2Model(cfg)
    m.config._attn_implementation = "eager"
    m = m.to(torch.float64).eval()
    sd = {"embed_tokens.weight": _t(model.w16("embed")), "embedding_norm.weight": _t(model.t["final_norm"])}
    D = c["head_dim"]
    for i, t in enumerate(c["layer_types"]):
        p = f"layers.{i}."
        w13 = model.w16(p + "w13")
        sd[p + "feed_forward.w1.weight"] = _t(w13[:I])
        sd[p + "feed_forward.w3.weight"] = _t(w13[I:])
        sd[p + "feed_forward.w2.weight"] = _t(model.w16(p + "w2"))
        sd[p + "operator_norm.weight"] = _t(model.t[p + "operator_norm"])
        sd[p + "ffn_norm.weight"] = _t(model.t[p + "ffn_norm"])
        if t == "conv":
            sd[p + "conv.in_proj.weight"] = _t(model.w16(p + "in_proj"))
            sd[p + "conv.out_proj.weight"] = _t(model.w16(p + "out_proj"))
            sd[p + "conv.conv.weight"] = _t(model.t[p + "conv"]).reshape(H, 1, 3)
        else:
            qkv = model.w16(p + "qkv")
            sd[p + "self_attn.q_proj.weight"] = _t(qkv[:h * D])
            sd[p + "self_attn.k_proj.weight"] = _t(qkv[h * D:(h + kv) * D])
            sd[p + "self_attn.v_proj.weight"] = _t(qkv[(h + kv) * D:])
            sd[p + "self_attn.out_proj.weight"] = _t(model.w16(p + "o_proj"))
            sd[p + "self_attn.q_layernorm.weight"] = _t(model.t[p + "q_norm"])
            sd[p + "self_attn.k_layernorm.weight"] = _t(model.t[p + "k_norm"])
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def _compare_lfm2(path, model=None):
    """The oracle's forest forward with conv layers (forest taps) against Lfm2Model on each trunk + branch
    alone: the final normed hidden state within 5e-3 relative L2 and the answer logits within 5e-3 of scale."""
    model = model or ref.Model(path)
    c = model.c
    rng = np.random.default_rng(42)
    tree = _forest(rng, c["vocab"])
    ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest([tree])
    mask = ref.ranges_mask(ref.forest_ranges(meta), len(ids))
    logits, _, dbg = ref.decoder_forward(model, ids, pos, mask, leaves, leaf_ids, n_ids, acc=np.float64,
                                         debug_layers=(c["layers"] - 1,), taps=ref.forest_taps([tree]))
    hf = _hf_lfm2(ref.Model(path))
    ec, es, eb = model.t["embed"]
    E32 = ref.dequant_f32(ec, es, eb).astype(np.float64)
    P, off = len(tree["trunk"]), len(tree["trunk"])
    for b, br in enumerate(tree["branches"]):
        rows = list(range(P)) + list(range(off, off + len(br)))
        off += len(br)
        with torch.no_grad():
            final = hf(input_ids=torch.tensor([tree["trunk"] + br])).last_hidden_state[0].numpy()
        x = dbg[c["layers"] - 1][rows].astype(np.float64)
        normed = x / np.sqrt((x * x).mean(-1, keepdims=True) + c["eps"]) * model.t["final_norm"].astype(np.float64)
        assert _rel_l2(normed, final) < 5e-3, f"branch {b}: final hidden state"
        want = final[-1] @ E32[leaf_ids[b * n_ids:(b + 1) * n_ids]].T
        got = logits[b * n_ids:(b + 1) * n_ids].astype(np.float64)
        assert np.abs(got - want).max() < 5e-3 * np.abs(want).max(), f"branch {b}: answer logits"


def test_lfm2_forward_matches_transformers(tiny_lfm2):
    _compare_lfm2(tiny_lfm2)


def test_planted_lfm2_tap_order_slip_is_caught(tiny_lfm2):
    def flip(m):
        m.t["layers.0.conv"] = np.ascontiguousarray(m.t["layers.0.conv"].reshape(-1, 3)[:, ::-1])
    model = ref.Model(tiny_lfm2)
    flip(model)
    with pytest.raises(AssertionError):
        _compare_lfm2(tiny_lfm2, model)


def test_planted_lfm2_branch_taps_slip_is_caught(tiny_lfm2, monkeypatch):
    """Branch tokens whose conv taps restart at the branch (the trunk not continued)."""
    orig = ref.forest_taps

    def slip(trees):
        taps = orig(trees).copy()
        P = len(trees[0]["trunk"])
        off = P
        for br in trees[0]["branches"]:
            for o in range(len(br)):
                for j in (1, 2):
                    if o - j < 0:
                        taps[off + o, 2 - j] = -1
            off += len(br)
        return taps
    monkeypatch.setattr(ref, "forest_taps", slip)
    with pytest.raises(AssertionError):
        _compare_lfm2(tiny_lfm2)


# ---------------------------------------------------------------- d1-omni: trunk, head and scorer

TINY_OMNI = dict(layers=3, hidden=64, intermediate=96, heads=4, kv_heads=2, head_dim=16, vocab=512,
                 layer_types=["conv", "full_attention", "conv"], head_layers=2, head_heads=4, head_ff=128)


@pytest.fixture(scope="module")
def tiny_omni(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("omni")
    return synth.generate(synth.reduced("d1-omni-q8", **TINY_OMNI), str(d / "omni"), norm_std=0.1, std=0.125)


def _omni_seqs(rng, V):
    return [{"ids": [int(x) for x in rng.integers(0, V, n)], "markers": m, "type": t}
            for n, m, t in ((23, [5, 9, 14], "choice"), (11, [2, 7], "noul"), (17, [0, 4, 8, 12, 16], "score"))]


def _torch_omni(model: ref.Model, monkeypatch):
    """The d1-omni forward from library modules, float64: transformers' Lfm2Model as the trunk, made
    bidirectional the way d1-omni reads it (an all-zero additive attention mask; the short conv centred: its
    causal conv replaced by F.conv1d with padding 1, a cross-correlation whose taps 0, 1, 2 read t-1, t, t+1),
    then torch.nn.TransformerEncoderLayer(norm_first=True, ReLU) for each head layer and
    Sequential(LayerNorm, Linear, GELU, Linear(H, 1)) as the scorer (export-omni.py:70-90)."""
    from transformers.models.lfm2 import modeling_lfm2
    monkeypatch.setattr(modeling_lfm2, "causal_conv1d_fn",
                        lambda x, w, b=None, seq_idx=None, **kw: F.conv1d(x, w.unsqueeze(1), b, padding=1, groups=x.shape[1]))
    trunk = _hf_lfm2(model)
    c = model.c
    H, hh, ff, ln = c["hidden"], c["head_heads"], c["head_ff"], c["ln_eps"]
    layers = []
    for i in range(c["head_layers"]):
        p = f"head.{i}."
        lay = torch.nn.TransformerEncoderLayer(H, hh, ff, dropout=0.0, activation="relu", layer_norm_eps=ln,
                                               batch_first=True, norm_first=True).to(torch.float64).eval()
        sd = {"self_attn.in_proj_weight": model.w16(p + "in_proj"), "self_attn.in_proj_bias": model.t[p + "in_proj_bias"],
              "self_attn.out_proj.weight": model.w16(p + "out_proj"), "self_attn.out_proj.bias": model.t[p + "out_proj_bias"],
              "linear1.weight": model.w16(p + "linear1"), "linear1.bias": model.t[p + "linear1_bias"],
              "linear2.weight": model.w16(p + "linear2"), "linear2.bias": model.t[p + "linear2_bias"],
              "norm1.weight": model.t[p + "norm1"], "norm1.bias": model.t[p + "norm1_bias"],
              "norm2.weight": model.t[p + "norm2"], "norm2.bias": model.t[p + "norm2_bias"]}
        lay.load_state_dict({k: _t(v) for k, v in sd.items()})
        layers.append(lay)
    scorer = torch.nn.Sequential(torch.nn.LayerNorm(H, eps=ln), torch.nn.Linear(H, H), torch.nn.GELU(),
                                 torch.nn.Linear(H, 1)).to(torch.float64).eval()
    scorer.load_state_dict({"0.weight": _t(model.t["scorer.norm"]), "0.bias": _t(model.t["scorer.norm_bias"]),
                            "1.weight": _t(model.w16("scorer.fc")), "1.bias": _t(model.t["scorer.fc_bias"]),
                            "3.weight": _t(model.t["scorer.out"]).reshape(1, H), "3.bias": _t(model.t["scorer.out_bias"][:1])})
    type_emb = _t(model.t["head.type_emb"])

    def run(seq):
        T = len(seq["ids"])
        with torch.no_grad():
            mask = {"full_attention": torch.zeros(1, 1, T, T, dtype=torch.float64), "conv": None}
            x = trunk(input_ids=torch.tensor([seq["ids"]]), attention_mask=mask).last_hidden_state
            t = x.clone()
            h = x + type_emb[["choice", "score", "noul"].index(seq["type"])]
            for lay in layers:
                h = lay(h)
            return t[0].numpy(), h[0].numpy(), scorer(h)[0, seq["markers"], 0].numpy()
    return run


def _compare_omni(path, monkeypatch, model=None):
    """The oracle's packed omni forward (float64 accumulation, f16 storage points) against the library modules
    on each sequence alone: trunk output and the head's stream within 5e-3 relative L2, the marker logits within
    1e-2 of their scale."""
    model = model or ref.Model(path)
    seqs = _omni_seqs(np.random.default_rng(5), model.c["vocab"])
    logits, dbg = ref.omni_forward(model, seqs, acc=np.float64)
    run = _torch_omni(ref.Model(path), monkeypatch)  # the library side always reads the untouched file
    off, k = 0, 0
    for s in seqs:
        n, m = len(s["ids"]), len(s["markers"])
        trunk, head, want = run(s)
        assert _rel_l2(dbg["trunk"][off:off + n], trunk) < 5e-3, f"{s['type']}: trunk"
        assert _rel_l2(dbg["head"][off:off + n], head) < 5e-3, f"{s['type']}: head stream"
        got = logits[k:k + m].astype(np.float64)
        assert np.abs(got - want).max() < 1e-2 * max(np.abs(want).max(), 1e-3), f"{s['type']}: marker logits"
        off += n
        k += m


def test_omni_forward_matches_library_modules(tiny_omni, monkeypatch):
    _compare_omni(tiny_omni, monkeypatch)


def test_planted_omni_causal_taps_slip_is_caught(tiny_omni, monkeypatch):
    """The decoder's causal taps (t-2, t-1, t) in place of d1-omni's centred ones."""
    orig = ref.pack_omni

    def slip(seqs):
        pk = orig(seqs)
        t = pk["taps"]
        pk["taps"] = np.stack([np.where(t[:, 0] >= 0, t[:, 0] - 1, -1), t[:, 0], t[:, 1], t[:, 3]], 1).astype(np.int32)
        pk["taps"][pk["taps"][:, 0] < np.repeat(pk["rng"][:, 0], 1), 0] = -1
        return pk
    monkeypatch.setattr(ref, "pack_omni", slip)
    with pytest.raises(AssertionError):
        _compare_omni(tiny_omni, monkeypatch)


def test_planted_omni_taps_across_sequences_slip_is_caught(tiny_omni, monkeypatch):
    """Centred taps that read the neighbouring sequence's edge token."""
    orig = ref.pack_omni

    def slip(seqs):
        pk = orig(seqs)
        T = pk["T"]
        t = np.arange(T)
        pk["taps"][:, 0] = t - 1
        pk["taps"][:, 2] = np.where(t + 1 < T, t + 1, -1)
        return pk
    monkeypatch.setattr(ref, "pack_omni", slip)
    with pytest.raises(AssertionError):
        _compare_omni(tiny_omni, monkeypatch)


@pytest.mark.parametrize("slip", ["relu_gelu_swapped", "no_in_proj_bias", "post_norm_scorer", "type_rows"])
def test_planted_omni_head_slips_are_caught(tiny_omni, monkeypatch, slip):
    """ReLU and GELU swapped; the fused in_proj bias dropped; the scorer's LayerNorm read before the last
    residual add; the question-type rows in the wrong order."""
    if slip == "relu_gelu_swapped":
        orig = ref.bias_act
        monkeypatch.setattr(ref, "bias_act", lambda Y, b, act=0, acc=np.float32: orig(Y, b, {1: 2, 2: 1}.get(act, act), acc))
    elif slip == "no_in_proj_bias":
        orig = ref.bias_act
        fused = 3 * TINY_OMNI["hidden"]
        monkeypatch.setattr(ref, "bias_act", lambda Y, b, act=0, acc=np.float32: orig(Y, b * 0 if b.shape[0] == fused else b, act, acc))
    elif slip == "post_norm_scorer":
        orig = ref.add_layernorm
        calls = {"n": 0}

        def ln(X, Y, w, b, eps, add=True, acc=np.float32):
            calls["n"] += 1
            if calls["n"] % (2 * TINY_OMNI["head_layers"] + 1) == 0:  # the scorer's: normalise X before adding Y
                Xn, O = orig(X, Y, w, b, eps, add, acc)
                return Xn, orig(X, None, w, b, eps, False, acc)[1]
            return orig(X, Y, w, b, eps, add, acc)
        monkeypatch.setattr(ref, "add_layernorm", ln)
    else:
        orig = ref.pack_omni

        def rows(seqs):
            pk = orig(seqs)
            pk["qtype"] = np.array([{0: 1, 1: 0}.get(int(q), int(q)) for q in pk["qtype"]], dtype=np.uint32)
            return pk
        monkeypatch.setattr(ref, "pack_omni", rows)
    with pytest.raises(AssertionError):
        _compare_omni(tiny_omni, monkeypatch)


def test_erf_as_error_bound():
    """BIAS_ACT's erf (A&S 7.1.26) within its published 1.5e-7 of erf on [-6, 6]; a changed coefficient is caught."""
    x = np.linspace(-6, 6, 24001)
    exact = np.array([math.erf(v) for v in x])
    assert np.abs(ref.erf_as(x) - exact).max() < 1.5e-7
    bad = 1.0 - ((((1.061405429 * (t := 1.0 / (1.0 + 0.3275911 * np.abs(x))) - 1.453152027) * t + 1.421413741) * t
                  - 0.284496736) * t + 0.254829592 * 1.001) * t * np.exp(-x * x)
    assert np.abs(np.where(x >= 0, bad, -bad) - exact).max() > 1.5e-7


def test_add_layernorm_matches_torch_layer_norm():
    """ADD_LAYERNORM (kernels.ts:224-255) in float64 against F.layer_norm of X + Y (the variance as
    E[x^2] - mean^2 agrees with the two-pass form to rounding); the stored sum is f16(X + Y)."""
    rng = np.random.default_rng(3)
    X = (rng.standard_normal((9, 192)) * 2 + 0.5).astype(np.float16)
    Y = rng.standard_normal((9, 192)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(192)).astype(np.float16)
    b = (0.1 * rng.standard_normal(192)).astype(np.float16)
    for add in (False, True):
        Xn, O = ref.add_layernorm(X, Y, w, b, 1e-5, add=add, acc=np.float64)
        v = X.astype(np.float64) + (Y.astype(np.float64) if add else 0)
        assert np.array_equal(Xn, v.astype(np.float16))
        want = F.layer_norm(_t(Xn.astype(np.float64)), (192,), _t(w), _t(b), 1e-5).numpy()
        assert np.abs(O.astype(np.float64) - want).max() < 2e-3 * np.abs(want).max()
        assert np.abs(O.astype(np.float64) - want).max() <= np.abs(want).max() * 2.0 ** -10  # one f16 rounding


# ---------------------------------------------------------------- d3-lite: Gated DeltaNet and gated attention

TINY_D3 = dict(layers=4, hidden=128, intermediate=192, heads=2, kv_heads=1, head_dim=64, rotary_dim=16, vocab=512,
               layer_types=["linear_attention", "linear_attention", "full_attention", "linear_attention"],
               linear_heads=2, linear_rows=1056, codes=["A", "B", "C", "D", "E"])


@pytest.fixture(scope="module")
def tiny_d3(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("d3")
    return synth.generate(synth.reduced("d3-lite-q8", **TINY_D3), str(d / "d3"), norm_std=0.1, std=0.09)


def _hf_qwen35(model: ref.Model):
    """A transformers Qwen3_5TextModel holding the oracle model's weights (float64): zero-centred norms get the
    file's folded weight minus one, the fused q | k | v | gate rows go back to per-head [q; gate] rows, the
    DeltaNet's `in` rows split into in_proj_qkv / z / b / a (export-d3.py:66-100)."""
    tr = pytest.importorskip("transformers")
    c = model.c
    H, I, h, kv, D, LH = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["linear_heads"]
    cfg = tr.Qwen3_5TextConfig(vocab_size=c["vocab"], hidden_size=H, intermediate_size=I, num_hidden_layers=len(c["layer_types"]),
                               num_attention_heads=h, num_key_value_heads=kv, head_dim=D, linear_num_key_heads=LH,
                               linear_num_value_heads=LH, linear_key_head_dim=128, linear_value_head_dim=128,
                               linear_conv_kernel_dim=4, layer_types=c["layer_types"], rms_norm_eps=c["eps"],
                               rope_parameters={"rope_theta": c["rope_theta"], "rope_type": "default",
                                                "partial_rotary_factor": c["rotary_dim"] / D})
    m = tr.Qwen3_5TextModel(cfg)
    m.config._attn_implementation = "eager"
    m = m.to(torch.float64).eval()
    QK = LH * 128
    one = lambda name: _t(model.t[name].astype(np.float64) - 1.0)  # noqa: E731  (1 + w folded at export)
    sd = {"embed_tokens.weight": _t(model.w16("embed")), "norm.weight": one("final_norm")}
    for i, t in enumerate(c["layer_types"]):
        p = f"layers.{i}."
        sd[p + "input_layernorm.weight"] = one(p + "input_norm")
        sd[p + "post_attention_layernorm.weight"] = one(p + "post_norm")
        w13 = model.w16(p + "w13")
        sd[p + "mlp.gate_proj.weight"], sd[p + "mlp.up_proj.weight"] = _t(w13[:I]), _t(w13[I:])
        sd[p + "mlp.down_proj.weight"] = _t(model.w16(p + "w2"))
        if t == "linear_attention":
            w = model.w16(p + "in")
            q = p + "linear_attn."
            sd[q + "in_proj_qkv.weight"] = _t(w[:3 * QK])
            sd[q + "in_proj_z.weight"] = _t(w[3 * QK:4 * QK])
            sd[q + "in_proj_b.weight"] = _t(w[4 * QK:4 * QK + LH])
            sd[q + "in_proj_a.weight"] = _t(w[4 * QK + LH:4 * QK + 2 * LH])
            sd[q + "conv1d.weight"] = _t(model.t[p + "conv"]).reshape(3 * QK, 1, 4)
            sd[q + "A_log"] = _t(model.t[p + "A_log"])
            sd[q + "dt_bias"] = _t(model.t[p + "dt_bias"])
            sd[q + "norm.weight"] = _t(model.t[p + "gnorm"])
            sd[q + "out_proj.weight"] = _t(model.w16(p + "out"))
        else:
            w = model.w16(p + "qkvg")
            qw, kw, vw, gw = w[:h * D], w[h * D:(h + kv) * D], w[(h + kv) * D:(h + 2 * kv) * D], w[(h + 2 * kv) * D:]
            q = p + "self_attn."
            sd[q + "q_proj.weight"] = _t(np.concatenate([qw.reshape(h, D, H), gw.reshape(h, D, H)], 1).reshape(2 * h * D, H))
            sd[q + "k_proj.weight"], sd[q + "v_proj.weight"] = _t(kw), _t(vw)
            sd[q + "o_proj.weight"] = _t(model.w16(p + "o"))
            sd[q + "q_norm.weight"], sd[q + "k_norm.weight"] = one(p + "q_norm"), one(p + "k_norm")
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def _d3_seqs(rng, V):
    state = [int(x) for x in rng.integers(0, V, 37)]
    return [{"ids": state + [int(x) for x in rng.integers(0, V, n)], "options": k} for n, k in ((9, 3), (1, 2), (15, 5))]


def _compare_d3(path, model=None, groups=None):
    """The oracle's d3-lite forward (float64 accumulation, f16 storage points) against Qwen3_5TextModel on each
    sequence alone with d3's noncausal attention (an all-zero additive mask; the DeltaNet is causal by its
    recurrence): the final normed hidden state within 5e-3 relative L2 and the code logits within 1e-2 of their
    scale. With `groups` the shared prefix is read once: the DeltaNet still scans it in front of each question,
    and the attention sees the trunk and the question; the library model runs the same on trunk + question,
    the trunk tokens attending only to the trunk."""
    model = model or ref.Model(path)
    c = model.c
    seqs = _d3_seqs(np.random.default_rng(9), c["vocab"])
    logits, normed = ref.d3_forward(model, seqs, groups, acc=np.float64)
    hf = _hf_qwen35(ref.Model(path))
    R = model.t["readout"].astype(np.float64)
    ids, meta, rng, pairs = ref.pack_shared(seqs, groups)
    k = 0
    for s in seqs:
        n = len(s["ids"])
        if groups is None:
            mask = torch.zeros(1, 1, n, n, dtype=torch.float64)
            rows = None
        else:  # trunk of 37 shared: its tokens see the trunk only
            P = 37
            mask = torch.zeros(1, 1, n, n, dtype=torch.float64)
            mask[0, 0, :P, P:] = -1e30
            rows = None
        with torch.no_grad():
            final = hf(input_ids=torch.tensor([s["ids"]]), attention_mask={"full_attention": mask, "linear_attention": None}).last_hidden_state[0].numpy()
        last = int(pairs[k][0])
        got_last = normed[last].astype(np.float64)
        assert _rel_l2(got_last, final[-1]) < 5e-3, "final hidden state at the readout row"
        want = final[-1] @ R[:s["options"]].T
        got = logits[k:k + s["options"]].astype(np.float64)
        assert np.abs(got - want).max() < 1e-2 * max(np.abs(want).max(), 1e-3), "code logits"
        k += s["options"]
    if groups is None:  # every row of the first sequence (rows 0..n-1 of the packing)
        n0 = len(seqs[0]["ids"])
        with torch.no_grad():
            final = hf(input_ids=torch.tensor([seqs[0]["ids"]]),
                       attention_mask={"full_attention": torch.zeros(1, 1, n0, n0, dtype=torch.float64),
                                       "linear_attention": None}).last_hidden_state[0].numpy()
        assert _rel_l2(normed[:n0], final) < 5e-3


def test_d3_forward_matches_transformers(tiny_d3):
    _compare_d3(tiny_d3)


def test_d3_forward_shared_prefix_matches_transformers(tiny_d3):
    _compare_d3(tiny_d3, groups=[3])


def test_d3_spans_match_oracle_and_packing(pkg):
    """gdn_spans (the product path) == the oracle's d3_spans bit for bit, and every scan's rows are exactly its
    question's tokens of pack_shared's layout, trunk first."""
    from decision_js_amd import d3
    rng = np.random.default_rng(4)
    for groups in ([3, 1, 2], None, [1, 1, 1, 1, 1, 1], [6]):
        seqs = []
        for g in (groups or [1] * 6):
            state = [int(x) for x in rng.integers(0, 9, rng.integers(0, 6))]
            for _ in range(g):
                seqs.append({"ids": state + [int(x) for x in rng.integers(0, 9, rng.integers(1, 5))], "options": 2})
        seqs = seqs[:6] if groups is None else seqs
        got = d3.gdn_spans(seqs, groups)
        assert np.array_equal(got, ref.d3_spans(seqs, groups))
        ids = ref.pack_shared(seqs, groups)[0]
        for s, (a0, aw, b0, bl) in zip(seqs, got):
            rows = list(range(a0, a0 + (aw & 0x7fffffff))) + list(range(b0, b0 + bl))
            assert [int(ids[r]) for r in rows] == s["ids"]


@pytest.mark.parametrize("slip", ["conv_taps_reversed", "decay_after_update", "no_q_scale", "no_gate", "full_rotary"])
def test_planted_d3_slips_are_caught(tiny_d3, monkeypatch, slip):
    """The conv taps in reverse order; the decay applied after the delta update; q not scaled by 128^-1/2; the
    attention's output gate dropped; RoPE over the whole head instead of rotary_dim."""
    model = ref.Model(tiny_d3)
    if slip == "conv_taps_reversed":
        for i, t in enumerate(model.c["layer_types"]):
            if t == "linear_attention":
                model.t[f"layers.{i}.conv"] = np.ascontiguousarray(model.t[f"layers.{i}.conv"][:, ::-1])
    elif slip == "decay_after_update":
        def gdn(Z, spans, LH, conv_w, A_log, dt_bias, gnorm, eps, acc=np.float32):
            # the same as ref.gdn with S <- S + delta k^T applied before S <- decay S
            return _gdn_variant(Z, spans, LH, conv_w, A_log, dt_bias, gnorm, eps, acc, decay_last=True)
        monkeypatch.setattr(ref, "gdn", gdn)
    elif slip == "no_q_scale":
        def gdn(Z, spans, LH, conv_w, A_log, dt_bias, gnorm, eps, acc=np.float32):
            return _gdn_variant(Z, spans, LH, conv_w, A_log, dt_bias, gnorm, eps, acc, q_scale=1.0)
        monkeypatch.setattr(ref, "gdn", gdn)
    elif slip == "no_gate":
        orig = ref.attention
        monkeypatch.setattr(ref, "attention", lambda *a, gate=None, **k: orig(*a, **k))
    else:
        model.c["rotary_dim"] = model.c["head_dim"]
    with pytest.raises(AssertionError):
        _compare_d3(tiny_d3, model)


def _gdn_variant(Z, spans, LH, conv_w, A_log, dt_bias, gnorm, eps, acc, decay_last=False, q_scale=None):
    """ref.gdn with one step changed (planted slips only)."""
    T, QK = Z.shape[0], LH * 128
    Y = np.zeros((T, QK), dtype=np.float16)
    W = conv_w.astype(acc).reshape(3 * QK, 4)
    for a0, aw, b0, bl in np.asarray(spans, dtype=np.int64):
        alen, write_a = int(aw) & 0x7fffffff, (int(aw) >> 31) & 1
        rows = list(range(a0, a0 + alen)) + list(range(b0, b0 + bl))
        n = len(rows)
        X = Z[rows].astype(acc)
        for h in range(LH):
            ch = np.concatenate([np.arange(128) + h * 128, QK + np.arange(128) + h * 128, 2 * QK + np.arange(128) + h * 128])
            x = np.concatenate([np.zeros((3, len(ch)), dtype=acc), X[:, ch]])
            y = sum(W[ch][:, j][None, :] * x[j:j + n] for j in range(4))
            y = (y / (1.0 + np.exp(-y))).astype(np.float16).astype(acc)
            q, k, v = y[:, :128], y[:, 128:256], y[:, 256:]
            q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) * (q_scale if q_scale is not None else 1 / np.sqrt(128.0))
            k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
            a = X[:, 4 * QK + LH + h] + acc(dt_bias[h])
            dec = np.exp(-np.exp(acc(A_log[h])) * np.where(a > 20, a, np.log1p(np.exp(np.minimum(a, 20)))))
            beta = 1.0 / (1.0 + np.exp(-X[:, 4 * QK + h]))
            S = np.zeros((128, 128), dtype=acc)
            o = np.zeros((n, 128), dtype=acc)
            for t in range(n):
                if not decay_last:
                    S = dec[t] * S
                delta = beta[t] * (v[t] - S @ k[t])
                S = S + np.outer(delta, k[t])
                if decay_last:
                    S = dec[t] * S
                o[t] = S @ q[t]
            inv = 1.0 / np.sqrt((o * o).mean(-1, keepdims=True) + eps)
            z = X[:, 3 * QK + h * 128:3 * QK + (h + 1) * 128]
            out = (o * inv * gnorm.astype(acc) * (z / (1.0 + np.exp(-z)))).astype(np.float16)
            for i, r in enumerate(rows):
                if i < alen and not write_a:
                    continue
                Y[r, h * 128:(h + 1) * 128] = out[i]
    return Y


# ---------------------------------------------------------------- EmbeddingGemma 2 as shipped (per-layer embeddings)

TINY_EG2 = dict(layers=3, hidden=64, intermediate=96, heads=2, vocab=512, window=3,
                layer_types=["sliding_attention", "full_attention", "sliding_attention"],
                head_dim={"sliding_attention": 32, "full_attention": 64}, kv_heads={"sliding_attention": 1, "full_attention": 2},
                rope_theta={"sliding_attention": 1e4, "full_attention": 1e6}, ple=32, embedding_dim=48, embed_dim=40,
                learned_head={"width": 16}, layer_scalars=[0.9, 1.1, 0.8])


@pytest.fixture(scope="module")
def tiny_eg2(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("eg2")
    return synth.generate(synth.reduced("eg2-q8", **TINY_EG2), str(d / "eg2"), norm_std=0.1, std=0.125)


def _torch_eg2(model: ref.Model, seqs):
    """Each text alone, float64, library routines (export-eg2.py's layout; eg2-engine.ts:72-139): embedding rows
    (sqrt(H) folded in) as the residual stream and as the per-layer embeddings' source; per layer q/k/v
    F.rms_norm (q, k weighted, v plain), RoPE as a complex rotation by pos / theta^(2d/D) of the layer type, SDPA at
    scale 1 with a boolean mask |i - j| <= window on the sliding layers (GQA by repeat), post-attention norm into the
    residual, pre-FF norm, gelu_tanh(gate) up, down, post-FF norm into the residual; then gelu_tanh(x ple_gate^T) *
    rms_norm(xe ple_in^T, ple.norm), ple_proj, ple_norm into the residual, times the layer scalar; the next
    layer's input norm (final_norm last); the mean over the text, the projection, the first embed_dim values
    L2-normalised."""
    c = model.c
    H, I, h, eps, win = c["hidden"], c["intermediate"], c["heads"], c["eps"], c["window"]

    def W(name):
        return _t(model.w16(name))

    def nw(name):
        return _t(model.t[name])

    def rms(x, w=None):
        return F.rms_norm(x, (x.shape[-1],), weight=w, eps=eps)

    E = W("embed")
    out = []
    for s in seqs:
        n = len(s)
        x = E[torch.tensor(s)]
        xe = x.clone()
        normed = rms(x, nw("layers.0.input_layernorm"))
        pos = torch.arange(n, dtype=torch.float64)
        for i, t in enumerate(c["layer_types"]):
            p, D, kv, theta = f"layers.{i}.", c["head_dim"][t], c["kv_heads"][t], c["rope_theta"][t]
            ang = pos[:, None] / theta ** (torch.arange(D // 2, dtype=torch.float64) * 2 / D)
            rot = torch.polar(torch.ones_like(ang), ang)
            z = normed @ W(p + "qkv").T
            q = rms(z[:, :h * D].reshape(n, h, D), nw(p + "q_norm"))
            k = rms(z[:, h * D:(h + kv) * D].reshape(n, kv, D), nw(p + "k_norm"))
            v = rms(z[:, (h + kv) * D:].reshape(n, kv, D))

            def rope(a):
                cplx = torch.complex(a[..., :D // 2], a[..., D // 2:]) * rot[:, None, :]
                return torch.cat([cplx.real, cplx.imag], -1)
            q, k = rope(q), rope(k).repeat_interleave(h // kv, dim=1)
            v = v.repeat_interleave(h // kv, dim=1)
            mask = None
            if t == "sliding_attention":
                mask = (pos[:, None] - pos[None, :]).abs() <= win
            y = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), attn_mask=mask, scale=1.0)
            o = y.transpose(0, 1).reshape(n, h * D) @ W(p + "o").T
            x = x + rms(o, nw(p + "post_attention_layernorm"))
            gu = rms(x, nw(p + "pre_feedforward_layernorm")) @ W(p + "gu").T
            o = (F.gelu(gu[:, :I], approximate="tanh") * gu[:, I:]) @ W(p + "down").T
            x = x + rms(o, nw(p + "post_feedforward_layernorm"))
            mix = F.gelu(x @ W(p + "ple_gate").T, approximate="tanh") * rms(xe @ W(p + "ple_in").T, nw("ple.norm"))
            x = (x + rms(mix @ W(p + "ple_proj").T, nw(p + "ple_norm"))) * c["layer_scalars"][i]
            normed = rms(x, nw(f"layers.{i + 1}.input_layernorm" if i + 1 < len(c["layer_types"]) else "final_norm"))
        e = (normed.mean(0) @ nw("projection").T)[:c["embed_dim"]]
        out.append((e / e.norm()).numpy())
    return np.stack(out)


def _compare_eg2(path, model=None):
    model = model or ref.Model(path)
    rng = np.random.default_rng(19)
    seqs = [[int(x) for x in rng.integers(0, model.c["vocab"], n)] for n in (23, 8, 1, 12)]
    got, _ = ref.eg2_forward(model, seqs, acc=np.float64)
    want = _torch_eg2(ref.Model(path), seqs)  # the untouched file
    for i in range(len(seqs)):
        assert _rel_l2(got[i], want[i]) < 5e-3, f"text {i}"


def test_eg2_forward_matches_library_restatement(tiny_eg2):
    _compare_eg2(tiny_eg2)


@pytest.mark.parametrize("slip", ["window_exclusive", "stream_normed_after_mlp", "ple_operands_swapped",
                                  "no_layer_scalar", "truncate_from_end"])
def test_planted_eg2_slips_are_caught(tiny_eg2, monkeypatch, slip):
    """The window's edge excluded; the residual stream RMS-normalised after the MLP (what the PLE gate reads);
    PLE_MIX's gate and embedding swapped; the layer scalar dropped; the embedding truncated to its last embed_dim
    values."""
    model = ref.Model(tiny_eg2)
    if slip == "window_exclusive":
        orig = ref.pack_encoder

        def pe(seqs, window=None):
            return orig(seqs, None if window is None else window - 1)
        monkeypatch.setattr(ref, "pack_encoder", pe)
    elif slip == "stream_normed_after_mlp":
        orig_s = ref.sandwich

        def sw(X, Y, w1, w2, eps, scale, acc=np.float32):
            Xn, O = orig_s(X, Y, w1, w2, eps, scale, acc)
            if w2 is None and Y is not None:  # the post-FF sandwich: a normalised stream
                a = Xn.astype(acc)
                Xn = (a / np.sqrt((a * a).mean(-1, keepdims=True) + eps)).astype(np.float16)
            return Xn, O
        monkeypatch.setattr(ref, "sandwich", sw)
    elif slip == "ple_operands_swapped":
        orig = ref.ple_mix
        monkeypatch.setattr(ref, "ple_mix", lambda G, E, w, eps, acc=np.float32: orig(E, G, w, eps, acc))
    elif slip == "no_layer_scalar":
        model.c["layer_scalars"] = [1.0] * len(model.c["layer_types"])
    else:
        orig_pp = ref.pool_project
        monkeypatch.setattr(ref, "pool_project", lambda X, ranges, W: np.ascontiguousarray(orig_pp(X, ranges, W)[:, ::-1]))
    with pytest.raises(AssertionError):
        _compare_eg2(tiny_eg2, model)


def test_ple_mix_and_pool_project_closed_forms():
    """PLE_MIX element by element in float64 (torch's tanh GELU, the row's RMS); POOL_PROJECT as the explicit
    mean then product (a 3 x 5 output from a 5 x 8 projection: a transposed operand fails)."""
    rng = np.random.default_rng(12)
    G, E = rng.standard_normal((4, 16)).astype(np.float16), rng.standard_normal((4, 16)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(16)).astype(np.float16)
    got = ref.ple_mix(G, E, w, 1e-6, np.float64).astype(np.float64)
    e = E.astype(np.float64)
    want = F.gelu(_t(G), approximate="tanh").numpy() * e / np.sqrt((e * e).mean(-1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.abs(got - want).max() <= 2 ** -10 * np.abs(want).max() + 1e-6
    X = rng.standard_normal((9, 8)).astype(np.float16)
    W = rng.standard_normal((5, 8)).astype(np.float16)
    ranges = np.array([(0, 4), (4, 5), (5, 9)], dtype=np.uint32)
    out = ref.pool_project(X, ranges, W)
    assert out.shape == (3, 5)
    for s, (a, b) in enumerate(ranges):
        m = X[a:b].astype(np.float64).mean(0)
        assert np.allclose(out[s], W.astype(np.float64) @ m, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- Laya: ModernBERT encoder + d1-omni's head

TINY_LAYA = dict(layers=4, hidden=64, intermediate=96, heads=4, vocab=512, window=3,
                 layer_types=["full_attention", "sliding_attention", "sliding_attention", "full_attention"],
                 head_layers=2, head_heads=4, head_ff=128)


@pytest.fixture(scope="module")
def tiny_laya(pkg, tmp_path_factory):
    from decision_js_amd import synth
    d = tmp_path_factory.mktemp("laya")
    return synth.generate(synth.reduced("laya-q8", **TINY_LAYA), str(d / "laya"), norm_std=0.1, std=0.125)


def _torch_laya(model: ref.Model):
    """transformers' ModernBertModel (bias-free LayerNorms, RoPE per layer type, GeGLU with the erf GELU) holding the
    oracle model's weights, float64, run with d1-omni-style per-sequence masks (all keys on the global layers,
    |i - j| <= window on the others); then the head modules of _torch_omni's construction."""
    tr = pytest.importorskip("transformers")
    c = model.c
    H, I, h = c["hidden"], c["intermediate"], c["heads"]
    cfg = tr.ModernBertConfig(vocab_size=c["vocab"], hidden_size=H, intermediate_size=I, num_hidden_layers=c["layers"],
                              num_attention_heads=h, layer_types=c["layer_types"], local_attention=2 * c["window"],
                              norm_eps=c["eps"], norm_bias=False, hidden_activation="gelu", pad_token_id=0,
                              bos_token_id=None, eos_token_id=None, cls_token_id=None, sep_token_id=None,
                              rope_parameters={t: {"rope_type": "default", "rope_theta": th} for t, th in c["rope_theta"].items()})
    m = tr.ModernBertModel(cfg)
    m.config._attn_implementation = "eager"
    m = m.to(torch.float64).eval()
    sd = {"embeddings.tok_embeddings.weight": _t(model.w16("embed")), "embeddings.norm.weight": _t(model.t["embed_norm"]),
          "final_norm.weight": _t(model.t["final_norm"])}
    for i in range(c["layers"]):
        p = f"layers.{i}."
        if i > 0:
            sd[p + "attn_norm.weight"] = _t(model.t[p + "attn_norm"])
        sd[p + "mlp_norm.weight"] = _t(model.t[p + "mlp_norm"])
        sd[p + "attn.Wqkv.weight"], sd[p + "attn.Wo.weight"] = _t(model.w16(p + "qkv")), _t(model.w16(p + "o"))
        sd[p + "mlp.Wi.weight"], sd[p + "mlp.Wo.weight"] = _t(model.w16(p + "wi")), _t(model.w16(p + "wo"))
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m


def _torch_marker_head(model: ref.Model):
    c = model.c
    H, hh, ff, ln = c["hidden"], c["head_heads"], c["head_ff"], c["ln_eps"]
    layers = []
    for i in range(c["head_layers"]):
        p = f"head.{i}."
        lay = torch.nn.TransformerEncoderLayer(H, hh, ff, dropout=0.0, activation="relu", layer_norm_eps=ln,
                                               batch_first=True, norm_first=True).to(torch.float64).eval()
        sd = {"self_attn.in_proj_weight": model.w16(p + "in_proj"), "self_attn.in_proj_bias": model.t[p + "in_proj_bias"],
              "self_attn.out_proj.weight": model.w16(p + "out_proj"), "self_attn.out_proj.bias": model.t[p + "out_proj_bias"],
              "linear1.weight": model.w16(p + "linear1"), "linear1.bias": model.t[p + "linear1_bias"],
              "linear2.weight": model.w16(p + "linear2"), "linear2.bias": model.t[p + "linear2_bias"],
              "norm1.weight": model.t[p + "norm1"], "norm1.bias": model.t[p + "norm1_bias"],
              "norm2.weight": model.t[p + "norm2"], "norm2.bias": model.t[p + "norm2_bias"]}
        lay.load_state_dict({k: _t(v) for k, v in sd.items()})
        layers.append(lay)
    scorer = torch.nn.Sequential(torch.nn.LayerNorm(H, eps=ln), torch.nn.Linear(H, H), torch.nn.GELU(),
                                 torch.nn.Linear(H, 1)).to(torch.float64).eval()
    scorer.load_state_dict({"0.weight": _t(model.t["scorer.norm"]), "0.bias": _t(model.t["scorer.norm_bias"]),
                            "1.weight": _t(model.w16("scorer.fc")), "1.bias": _t(model.t["scorer.fc_bias"]),
                            "3.weight": _t(model.t["scorer.out"]).reshape(1, H), "3.bias": _t(model.t["scorer.out_bias"][:1])})
    return layers, scorer, _t(model.t["head.type_emb"])


def _compare_laya(path, model=None):
    """The oracle's packed Laya forward against ModernBertModel + the head modules on each sequence alone: encoder
    output and head stream within 5e-3 relative L2, marker logits within 1e-2 of their scale."""
    model = model or ref.Model(path)
    seqs = _omni_seqs(np.random.default_rng(6), model.c["vocab"])
    logits, dbg = ref.laya_forward(model, seqs, acc=np.float64)
    fresh = ref.Model(path)
    enc = _torch_laya(fresh)
    layers, scorer, type_emb = _torch_marker_head(fresh)
    w = fresh.c["window"]
    off = k = 0
    for s in seqs:
        n, m = len(s["ids"]), len(s["markers"])
        pos = torch.arange(n)
        slide = torch.zeros(1, 1, n, n, dtype=torch.float64).masked_fill((pos[:, None] - pos[None, :]).abs() > w, -1e30)
        with torch.no_grad():
            x = enc(input_ids=torch.tensor([s["ids"]]), attention_mask={"full_attention": torch.zeros(1, 1, n, n, dtype=torch.float64),
                                                                      "sliding_attention": slide}).last_hidden_state
            trunk = x[0].numpy().copy()
            hx = x + type_emb[["choice", "score", "noul"].index(s["type"])]
            for lay in layers:
                hx = lay(hx)
            want = scorer(hx)[0, s["markers"], 0].numpy()
        assert _rel_l2(dbg["trunk"][off:off + n], trunk) < 5e-3, f"{s['type']}: encoder output"
        assert _rel_l2(dbg["head"][off:off + n], hx[0].numpy()) < 5e-3, f"{s['type']}: head stream"
        got = logits[k:k + m].astype(np.float64)
        assert np.abs(got - want).max() < 1e-2 * max(np.abs(want).max(), 1e-3), f"{s['type']}: marker logits"
        off += n
        k += m


def test_laya_forward_matches_modernbert(tiny_laya):
    _compare_laya(tiny_laya)


@pytest.mark.parametrize("slip", ["global_on_every_layer", "theta_swapped", "window_plus_one", "attn_norm_on_layer0"])
def test_planted_laya_slips_are_caught(tiny_laya, slip):
    """Every layer global (no windows); the global and local RoPE thetas swapped; the window one key wider;
    layer 0's attention reading a normed stream (ModernBERT's layer 0 has no attention norm). (The tanh GELU in
    place of erf moves the outputs by less than f16's rounding: test_gelu_erf_mul_matches_torch pins it.)"""
    model = ref.Model(tiny_laya)
    if slip == "global_on_every_layer":
        model.c["layer_types"] = ["full_attention"] * len(model.c["layer_types"])
    elif slip == "theta_swapped":
        th = model.c["rope_theta"]
        model.c["rope_theta"] = {"full_attention": th["sliding_attention"], "sliding_attention": th["full_attention"]}
    elif slip == "window_plus_one":
        model.c["window"] += 1
    else:
        model.t["layers.0.attn_norm"] = np.full(model.c["hidden"], 0.5, dtype=np.float16)
    with pytest.raises(AssertionError):
        _compare_laya(tiny_laya, model)


def test_gelu_erf_mul_matches_torch():
    """gelu_erf_mul against torch's exact-erf GELU times b in f64: within one f16 rounding of the product (the erf
    approximation adds < 1.5e-7 absolute), over inputs where the tanh form differs from erf by up to 4.7e-4."""
    a = np.linspace(-6, 6, 4001).astype(np.float16)
    b = np.random.default_rng(2).uniform(0.5, 4, a.shape).astype(np.float16)
    got = ref.gelu_erf_mul(a, b, np.float64).astype(np.float64)
    want = (F.gelu(torch.from_numpy(a.astype(np.float64)), approximate="none") * torch.from_numpy(b.astype(np.float64))).numpy()
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert (np.abs(got - want) <= 0.5 * ulp + 1e-6).all()
