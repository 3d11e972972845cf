"""Pins the oracle (CPU only): golden vectors from the reference's own quantizer, brute force over every
q8/q4 code and every f16 scale, two independent restatements (numpy and C), float64 textbook forms, and
mistakes planted in the oracle that these checks must catch."""
import math
import os

import numpy as np
import pytest

from oracle import cref, ref

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module", autouse=True)
def built_oracle():
    if not os.path.exists(cref.LIB):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.dirname(cref.HERE) + "/oracle"], check=True)


# ---------------------------------------------------------------- f16 and dequantization

def test_f16_rounding_c_matches_numpy():
    rng = np.random.default_rng(0)
    L = cref.lib()
    xs = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 20000),
                         np.array([65504, 65519.99, 65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0, -0.0, 1e-45], np.float32)])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L.o_f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", [8, 4])
def test_dequant_brute_force_all_codes_all_scales(bits):
    """Every code x every finite f16 scale: numpy restatement == C restatement == RNE(code * scale) in float64."""
    ncodes = 256 if bits == 8 else 16
    scales = np.arange(65536, dtype=np.uint16).view(np.float16)
    scales = scales[np.isfinite(scales)]  # every finite f16, subnormals and signs included
    N, K = len(scales), max(ncodes, 32)
    c_full = np.tile((np.arange(K) % ncodes).astype(np.uint8), (N, 1))  # row n: every code, all under scale n
    s_full = np.repeat(scales[:, None], K // 32, axis=1)
    stored = c_full if bits == 8 else (c_full[:, 0::2] | (c_full[:, 1::2] << 4)).astype(np.uint8)
    got_np = ref.dequant_f16(stored, s_full, bits)
    got_c = cref.dequant(stored, s_full, N, K, bits)
    zp = 128 if bits == 8 else 8
    with np.errstate(over="ignore", invalid="ignore"):
        want = ((c_full.astype(np.float64) - zp) * np.repeat(s_full.astype(np.float64), 32, axis=1)).astype(np.float16)
    assert np.array_equal(got_np.view(np.uint16), want.view(np.uint16))
    assert np.array_equal(got_c.view(np.uint16), want.view(np.uint16))


def test_planted_dequant_mistake_is_caught(monkeypatch):
    """A dequantization with the wrong zero point (a plausible slip) fails the closed-form check."""
    orig = ref.unpack_codes
    monkeypatch.setattr(ref, "unpack_codes", lambda c, b: orig(c, b).astype(np.int32) + (1 if b == 8 else 0))
    codes = np.arange(256, dtype=np.uint8).reshape(8, 32)
    s = np.full((8, 1), 0.01, dtype=np.float16)
    got = ref.dequant_f16(codes, s, 8)
    want = ((codes.astype(np.float64) - 128) * 0.01).astype(np.float16)
    assert not np.array_equal(got.view(np.uint16), want.view(np.uint16))


# ---------------------------------------------------------------- quantizers (the format, export_common.py)

def test_quantize4_matches_reference_golden(pkg):
    """fmt.quantize4 against vectors written by the reference's own export_common.quantize4
    (tests/golden/make_q4_golden.py), including an all-zero block, near-ties and constant blocks."""
    from decision_js_amd import fmt
    g = np.load(os.path.join(HERE, "golden", "q4_golden.npz"))
    codes, scales, deq = fmt.quantize4(g["w"])
    assert np.array_equal(codes.reshape(-1), g["codes4"].reshape(-1))
    assert np.array_equal(scales.view(np.uint16), g["scales4"].view(np.uint16))
    assert np.array_equal(deq.astype(np.float32), g["deq4"])


def test_linspace_matches_torch(pkg):
    torch = pytest.importorskip("torch")
    from decision_js_amd import fmt
    assert np.array_equal(fmt._linspace_f32(0.6, 1.15, 23), torch.linspace(0.6, 1.15, 23).numpy())


def test_quantize8_closed_form(pkg):
    from decision_js_amd import fmt
    rng = np.random.default_rng(3)
    w = rng.standard_normal((64, 256)).astype(np.float32) * 0.02
    w[0, :32] = 0
    w[1, :32] = np.linspace(-1, 1, 32)
    codes, scales, deq = fmt.quantize8(w)
    c_codes, c_scales = cref.quantize8(w)
    assert np.array_equal(codes, c_codes) and np.array_equal(scales.view(np.uint16), c_scales.view(np.uint16))
    b = w.reshape(64, 8, 32)
    s = scales.astype(np.float32)
    assert s[0, 0] == 1.0 and np.all(codes[0, :32] == 128)
    assert np.array_equal(scales, (np.abs(b).max(-1) / np.float32(127)).astype(np.float16)[:, :] * (s != 1) + (s == 1) * np.float16(1))
    assert codes.min() >= 1 and codes.max() <= 255
    assert np.all(np.abs(deq - w) <= np.repeat(s, 32, axis=1) / 2 + 1e-9)


# ---------------------------------------------------------------- packing

def _trees(rng, n=5):
    out = []
    for _ in range(n):
        out.append({"trunk": [int(x) for x in rng.integers(0, 100, rng.integers(0, 20))],
                    "branches": [[int(x) for x in rng.integers(0, 100, rng.integers(1, 9))] for _ in range(rng.integers(0, 4))],
                    "groups": []})
        out[-1]["groups"] = [[[1, 2], [3]] for _ in out[-1]["branches"]]
    return out


def test_forest_packing_numpy_c_and_mask():
    rng = np.random.default_rng(4)
    for _ in range(20):
        trees = _trees(rng)
        ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest(trees)
        cids, cpos, cmeta, cleaves = cref.pack_forest(trees)
        assert np.array_equal(ids, cids) and np.array_equal(pos, cpos) and np.array_equal(meta, cmeta)
        assert np.array_equal(leaves, cleaves)
        T = len(ids)
        if T:
            assert np.array_equal(ref.ranges_mask(ref.forest_ranges(meta), T), ref.forest_mask(meta))
            # invariants: positions restart per tree and continue after the trunk; leaves end branches
            for t in range(T):
                s, e, b, p = meta[t]
                assert pos[t] == p and s <= t < e
                if b == -1:
                    assert p == t - s
            for l in leaves:
                assert l == len(ids) - 1 or meta[l + 1][2] != meta[l][2] or meta[l + 1][0] != meta[l][0]


def test_planted_mask_mistake_is_caught():
    """A forest mask that lets trunk tokens see later trunk tokens (a dropped causal term) is caught."""
    meta = ref.pack_forest([{"trunk": [1, 2, 3], "branches": [[4, 5]], "groups": [[[1]]]}])[2]
    good = ref.forest_mask(meta)
    bad = good.copy()
    bad[0, 1] = True
    assert not np.array_equal(ref.ranges_mask(ref.forest_ranges(meta), len(meta)), bad)


def test_shared_prefix_packing():
    """d3-engine.ts:67-93: the common prefix laid once; each question's rows see the trunk and themselves."""
    seqs = [{"ids": [1, 2, 3, 4, 5, 6], "options": 2}, {"ids": [1, 2, 3, 9, 9], "options": 3}, {"ids": [7, 7], "options": 2}]
    ids, meta, rng, pairs = ref.pack_shared(seqs, groups=[2, 1])
    assert list(ids) == [1, 2, 3, 4, 5, 6, 9, 9, 7, 7]
    assert [tuple(r) for r in rng[:3]] == [(0, 3, 0, 0)] * 3
    assert tuple(rng[3]) == (0, 3, 3, 6) and tuple(rng[6]) == (0, 3, 6, 8)
    assert tuple(rng[8]) == (8, 10, 0, 0)
    assert [tuple(p) for p in pairs] == [(5, 0), (5, 1), (7, 0), (7, 1), (7, 2), (9, 0), (9, 1)]
    # the prefix always leaves a token per question
    ids2, _, _, _ = ref.pack_shared([{"ids": [1, 2], "options": 2}, {"ids": [1, 2, 3], "options": 2}], groups=[2])
    assert list(ids2) == [1, 2, 2, 3]


def test_encoder_packing_windows():
    ids, meta, full, slide, ranges = ref.pack_encoder([[5] * 10, [6] * 3], window=2)
    assert tuple(full[4]) == (0, 10, 0, 0) and tuple(slide[4]) == (2, 7, 0, 0) and tuple(slide[11]) == (10, 13, 0, 0)
    assert [tuple(r) for r in ranges] == [(0, 10), (10, 13)] and meta[12][3] == 2


# ---------------------------------------------------------------- float kernels against float64 textbook forms

def test_rmsnorm_closed_form():
    rng = np.random.default_rng(5)
    X, Y = (rng.standard_normal((7, 64)) * 3).astype(np.float16), rng.standard_normal((7, 64)).astype(np.float16)
    w = (1 + rng.standard_normal(64) * 0.1).astype(np.float16)
    Xn, O = ref.add_rmsnorm(X, Y, w, 1e-6, add=True, acc=np.float64)
    v = X.astype(np.float64) + Y.astype(np.float64)
    assert np.array_equal(Xn, v.astype(np.float16))
    want = Xn.astype(np.float64) / np.sqrt((v ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.abs(O.astype(np.float64) - want).max() <= 2 ** -10 * np.abs(want).max()


@pytest.mark.parametrize("mode", [0, 1])
def test_rope_is_a_rotation(mode):
    """RoPE without norms equals multiplying (a + ib) by exp(i pos theta^(-2d/D)) (closed form), and keeps
    each pair's norm."""
    rng = np.random.default_rng(6)
    T, h, kv, D = 5, 2, 1, 16
    Z = rng.standard_normal((T, (h + 2 * kv) * D)).astype(np.float16)
    pos = np.array([0, 1, 7, 300, 1000], dtype=np.int32)
    out = ref.qk_norm_rope(Z, h, kv, D, pos, None, None, False, 1e-6, 1e4, mode=mode, acc=np.float64).astype(np.float64)
    z = Z.astype(np.float64).reshape(T, h + 2 * kv, D)
    d = np.arange(D // 2)
    freq = 1e4 ** (-2.0 * d / D)
    ang = pos[:, None].astype(np.float64) * freq[None, :]
    c = (z[:, :h + kv, :D // 2] + 1j * z[:, :h + kv, D // 2:]) * np.exp(1j * ang)[:, None, :]
    o = out.reshape(T, h + 2 * kv, D)
    assert np.abs(o[:, :h + kv, :D // 2] - c.real).max() < 2e-3 and np.abs(o[:, :h + kv, D // 2:] - c.imag).max() < 2e-3
    assert np.array_equal(o[:, h + kv:], z[:, h + kv:])  # v untouched


def test_planted_rope_sign_mistake_is_caught(monkeypatch):
    orig = ref.inv_freq
    monkeypatch.setattr(ref, "inv_freq", lambda theta, rot, mode=0: -orig(theta, rot, mode))
    with pytest.raises(AssertionError):
        test_rope_is_a_rotation(0)


def test_attention_vs_brute_force():
    rng = np.random.default_rng(7)
    T, h, kv, D = 9, 4, 2, 8
    Z = rng.standard_normal((T, (h + 2 * kv) * D)).astype(np.float16)
    mask = np.tril(np.ones((T, T), dtype=bool))
    mask[5, :3] = False
    got = ref.attention(Z, h, kv, D, mask, 0.3, np.float64).astype(np.float64)
    z = Z.astype(np.float64)
    for t in range(T):
        for hh in range(h):
            q = z[t, hh * D:(hh + 1) * D]
            g = hh // (h // kv)
            ks = [k for k in range(T) if mask[t, k]]
            s = np.array([0.3 * q @ z[k, (h + g) * D:(h + g + 1) * D] for k in ks])
            p = np.exp(s - s.max())
            o = sum(pk * z[k, (h + kv + g) * D:(h + kv + g + 1) * D] for pk, k in zip(p, ks)) / p.sum()
            assert np.abs(got[t, hh * D:(hh + 1) * D] - o).max() < 2e-3


def test_glu_and_softmax_forms():
    a = np.array([-20, -1, 0, 0.5, 3, 30], dtype=np.float16)
    b = np.ones(6, dtype=np.float16)
    s = ref.silu_mul(a, b, np.float64).astype(np.float64)
    assert np.allclose(s, a.astype(np.float64) / (1 + np.exp(-a.astype(np.float64))), rtol=1e-3, atol=1e-6)
    gg = ref.gelu_tanh(np.array([-30.0, 0.0, 30.0]))
    assert abs(gg[0]) < 1e-10 and gg[1] == 0 and abs(gg[2] - 30) < 1e-9  # saturated at the +-15 clamp
    p = ref.softmax([1000.0, 1000.0, -1000.0])
    assert abs(p[0] - 0.5) < 1e-12 and p[2] == 0 and abs(sum(p) - 1) < 1e-12


def test_leaf_logits_brute_force():
    rng = np.random.default_rng(8)
    from decision_js_amd import fmt  # noqa: F401  (package import for the session)
    V, H = 40, 64
    w = rng.standard_normal((V, H)).astype(np.float32) * 0.1
    codes, scales = cref.quantize8(w)
    X = rng.standard_normal((6, H)).astype(np.float16)
    nw = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    out = ref.leaf_logits(X, [2, 5], nw, np.array([3, 9, 0, 39], np.uint32), 2, codes, scales, 8, 1e-6, np.float64)
    for l, row in enumerate([2, 5]):
        x = X[row].astype(np.float64)
        nrm = x / math.sqrt((x ** 2).mean() + 1e-6) * nw
        for j in range(2):
            r = [3, 9, 0, 39][2 * l + j]
            e = (codes[r].astype(np.float64) - 128) * np.repeat(scales[r].astype(np.float64), 32)
            assert abs(out[2 * l + j] - nrm @ e) < 1e-9


def test_group_max_readout():
    out = np.array([1, 5, 2, 0, 0, 7, 8, 9, 0], dtype=np.float32)
    assert ref.group_max(out, 3, [[[10, 11], [12]], [[1], [2], [3]], [[4]]]) == [[5.0, 2.0], [0.0, 0.0, 7.0], [8.0]]


# ---------------------------------------------------------------- the encoder's tail (eg2-kernels.ts, eg2-head.ts)

def _check_sandwich(scale=0.5):
    """SANDWICH against an element-by-element float64 loop: x' = f16((x + y / rms(y) * w1) * scale),
    O = f16(x' / rms(x') * w2); rms(v) = sqrt(mean(v^2) + eps). Also rms-scale invariance in Y (Y and 4Y give
    the same result) and the no-residual form x' = f16(x * scale)."""
    rng = np.random.default_rng(17)
    H, eps = 48, 1e-6
    X = (rng.standard_normal((5, H)) * 2).astype(np.float16)
    Y = rng.standard_normal((5, H)).astype(np.float16)
    w1, w2 = [(1 + rng.standard_normal(H) * 0.2).astype(np.float16) for _ in range(2)]
    Xn, O = ref.sandwich(X, Y, w1, w2, eps, scale, acc=np.float64)
    for r in range(5):
        y = [float(v) for v in Y[r]]
        iy = 1.0 / math.sqrt(sum(v * v for v in y) / H + eps)
        xs = [np.float16((float(X[r, k]) + y[k] * iy * float(w1[k])) * scale) for k in range(H)]
        ix = 1.0 / math.sqrt(sum(float(v) * float(v) for v in xs) / H + eps)
        for k in range(H):
            assert abs(float(Xn[r, k]) - float(xs[k])) <= 2 ** -10 * abs(float(xs[k])) + 1e-7
            want = float(xs[k]) * ix * float(w2[k])
            assert abs(float(O[r, k]) - want) <= 2 ** -10 * abs(want) + 1e-7
    Xn4, O4 = ref.sandwich(X, (Y.astype(np.float32) * 4).astype(np.float16), w1, w2, eps, scale, acc=np.float64)
    assert np.abs(Xn4.astype(np.float64) - Xn.astype(np.float64)).max() <= 2 ** -9 * np.abs(Xn.astype(np.float64)).max()
    Xs, none = ref.sandwich(X, None, None, None, eps, scale, acc=np.float64)
    assert none is None and np.array_equal(Xs, (X.astype(np.float64) * scale).astype(np.float16))


def test_sandwich_closed_form():
    _check_sandwich()


def test_planted_sandwich_mistake_is_caught(monkeypatch):
    orig = ref.sandwich
    # the layer scalar applied to the norm branch only, not to the residual sum
    monkeypatch.setattr(ref, "sandwich", lambda X, Y, w1, w2, eps, scale, acc=np.float32:
                        orig(X.astype(np.float64) / scale if Y is not None else X, Y, w1, w2, eps, scale, acc))
    with pytest.raises(AssertionError):
        _check_sandwich()


def test_mean_pool_readout_dense_brute_force():
    """mean_pool, readout and dense_f32 against explicit loops: the mean of each token range (a one-token
    range is that row; constant rows pool to the constant), out[k] = X[row] . R[code], and out[m, n] =
    sum_k in[m, k] * w[n, k] with w the dequantized weight — a 3 x 5 output from a 5 x 64 weight, so a
    transposed operand cannot pass."""
    rng = np.random.default_rng(23)
    T, H = 20, 16
    X = rng.standard_normal((T, H)).astype(np.float16)
    X[12:15] = np.float16(0.75)
    ranges = [(0, 7), (7, 8), (12, 15), (8, 20)]
    pooled = ref.mean_pool(X, np.array(ranges, dtype=np.uint32))
    for s, (a, b) in enumerate(ranges):
        for k in range(H):
            want = sum(float(X[t, k]) for t in range(a, b)) / (b - a)
            assert abs(float(pooled[s, k]) - want) <= 1e-6 * (1 + abs(want))
    assert np.array_equal(pooled[1], X[7].astype(np.float32)) and np.all(pooled[2] == np.float32(0.75))
    R = rng.standard_normal((6, H)).astype(np.float32)
    pairs = [(3, 5), (0, 0), (19, 2)]
    got = ref.readout(X, R, pairs)
    for i, (r, c) in enumerate(pairs):
        assert abs(float(got[i]) - sum(float(X[r, k]) * float(R[c, k]) for k in range(H))) <= 1e-5
    for bits in (8, 4):
        w = (rng.standard_normal((5, 64)) * 0.05).astype(np.float32)
        from decision_js_amd import fmt
        codes, scales = (fmt.quantize8 if bits == 8 else fmt.quantize4)(w)[:2]
        W = ref.dequant_f32(codes, scales, bits).astype(np.float64)
        inp = rng.standard_normal((3, 64)).astype(np.float32)
        out = ref.dense_f32(inp, codes, scales, bits)
        assert out.shape == (3, 5) and out.dtype == np.float32
        for m in range(3):
            for n in range(5):
                want = sum(float(inp[m, k]) * W[n, k] for k in range(64))
                assert abs(float(out[m, n]) - want) <= 1e-5 * (1 + abs(want))


def test_cosine_scores_closed_forms():
    """cos(option, state + question): an option along the anchor scores 1 whatever its length, the opposite
    direction -1, an orthogonal one 0; the anchor is the sum of the two embeddings, not either alone."""
    s = np.array([1.0, 0.0, 0.0, 0.0], dtype=np.float32)
    q = np.array([0.0, 1.0, 0.0, 0.0], dtype=np.float32)
    opts = [np.array([3.0, 3.0, 0, 0], np.float32), np.array([-1.0, -1.0, 0, 0], np.float32),
            np.array([0, 0, 2.0, 0], np.float32), np.array([1.0, 0, 0, 0], np.float32)]
    got = ref.cosine_scores(s, q, opts)
    assert abs(got[0] - 1) < 1e-12 and abs(got[1] + 1) < 1e-12 and abs(got[2]) < 1e-12
    assert abs(got[3] - 1 / math.sqrt(2)) < 1e-12


def test_encoder_texts_embed_independently(pkg, tmp_path):
    """Texts packed into one encoder pass attend only within themselves: each text's embedding equals the
    one it gets alone (a segment, window or position slip in the packing or the mask breaks this), and
    embeddings are unit vectors."""
    from decision_js_amd import synth
    mdir = synth.generate(synth.reduced("eg2-encoder-q8", layers=1, vocab=512), str(tmp_path / "enc"), seed=0)
    model = ref.Model(mdir)
    rng = np.random.default_rng(29)
    seqs = [[int(x) for x in rng.integers(0, 512, n)] for n in (37, 5, 1, 20)]
    # float64 accumulation: numpy's blocking differs with the number of rows, and f32 sums in another order
    # move the result by ~2e-5 (measured), which would hide nothing a mask slip does (O(1e-2) and up)
    together = ref.encoder_forward(model, seqs, acc=np.float64)
    assert np.allclose(np.linalg.norm(together.astype(np.float64), axis=1), 1, atol=1e-6)
    for i, s in enumerate(seqs):
        alone = ref.encoder_forward(model, [s], acc=np.float64)
        assert np.abs(alone[0].astype(np.float64) - together[i].astype(np.float64)).max() < 1e-6


def test_planted_encoder_mask_leak_is_caught(pkg, tmp_path, monkeypatch):
    orig = ref.pack_encoder

    def leaky(seqs, window=None):
        ids, meta, full, slide, ranges = orig(seqs, window)
        full = full.copy()
        full[:, 0], full[:, 1] = 0, len(ids)  # every text attends to the whole batch
        return ids, meta, full, slide, ranges
    monkeypatch.setattr(ref, "pack_encoder", leaky)
    with pytest.raises(AssertionError):
        test_encoder_texts_embed_independently(pkg, tmp_path)
