"""numpy restatement of decision.js's scoring path (test infrastructure: see oracle/__init__.py).

Precision contract of the reference: activations stored as f16 at the points the WGSL kernels store them,
every reduction in f32 (kernels.ts:1). Functions take an `acc` dtype (float32 by default; float64 for the
checks that want a tighter reference).
"""
import math

import numpy as np

F16, F32, F64 = np.float16, np.float32, np.float64


def f16(x):
    return np.asarray(x).astype(F16)


# ---------------------------------------------------------------- weights (export_common.py, kernels.ts)

def dequant_f16(codes: np.ndarray, scales: np.ndarray, bits: int) -> np.ndarray:
    """f16 weights [N, K] as the GEMM / gather use them: (f16(code) - f16(zp)) * scale rounded once to f16
    (kernels.ts:20, 296, 319, 321, 541). The f32 product of two f16 values is exact, so rounding it to f16
    is the f16 multiply's RNE result."""
    q = unpack_codes(codes, bits).astype(F32) - (128.0 if bits == 8 else 8.0)
    s = np.repeat(scales.astype(F32), 32, axis=1)
    with np.errstate(over="ignore", invalid="ignore"):  # huge scales overflow to inf, as in f16 hardware
        return (q * s).astype(F16)


def dequant_f32(codes, scales, bits) -> np.ndarray:
    """f32 weights as LEAF_LOGITS reads them: (f32(code) - zp) * f32(scale) (kernels.ts:177-178)."""
    q = unpack_codes(codes, bits).astype(F32) - (128.0 if bits == 8 else 8.0)
    return q * np.repeat(scales.astype(F32), 32, axis=1)


def unpack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """u8 codes [N, K] from the stored bytes (q4: low nibble first, export_common.py:87)."""
    if bits == 8:
        return codes
    lo, hi = codes & 15, codes >> 4
    return np.stack([lo, hi], axis=-1).reshape(codes.shape[0], -1)


def gather(ids, codes, scales, bits):
    """GATHER_Q8 / GATHER_Q4 (kernels.ts:6-21, 292-296): rows of the f16-dequantized embedding."""
    ids = np.minimum(np.asarray(ids, dtype=np.int64), codes.shape[0] - 1)
    return dequant_f16(codes[ids], scales[ids], bits)


# ---------------------------------------------------------------- norms

def add_rmsnorm(X, Y, w, eps, add=True, acc=F32):
    """ADD_RMSNORM (kernels.ts:23-46): v = f32(X) + f32(Y), X <- f16(v); the sum of squares of the unrounded
    v; O = f16(f32(X_f16) * inv * f32(w)). Returns (X_new, O)."""
    x = X.astype(acc)
    if add:
        x = x + Y.astype(acc)
    ss = (x * x).sum(-1, keepdims=True, dtype=acc)
    Xn = x.astype(F16)
    inv = (1.0 / np.sqrt(ss / X.shape[-1] + eps)).astype(acc)
    O = (Xn.astype(acc) * inv * w.astype(acc)).astype(F16)
    return Xn, O


def sandwich(X, Y, w1, w2, eps, scale, acc=F32):
    """SANDWICH (eg2-kernels.ts:15-48): X = f16((X + rmsnorm(Y) w1) * scale); O = f16(rmsnorm(f16 X) w2)."""
    H = X.shape[-1]
    x = X.astype(acc)
    if Y is not None:
        y = Y.astype(acc)
        iy = 1.0 / np.sqrt((y * y).sum(-1, keepdims=True) / H + eps)
        x = x + y * iy * w1.astype(acc)
    Xn = (x * acc(scale)).astype(F16)
    if w2 is None:
        return Xn, None
    a = Xn.astype(acc)
    ix = 1.0 / np.sqrt((a * a).sum(-1, keepdims=True) / H + eps)
    return Xn, (a * ix * w2.astype(acc)).astype(F16)


# ---------------------------------------------------------------- matmul and gated MLP

def matmul(X, W16, acc=F32):
    """Y = f16(X . W^T) with W the f16-dequantized weight; f32 (or f64) accumulation (kernels.ts:441-520
    portable path; the matrix-unit path adds f16 partials every 128 K, kernels.ts:301-302)."""
    return (X.astype(acc) @ W16.astype(acc).T).astype(F16)


def silu_mul(a16, b16, acc=F32):
    """SILU_MUL (kernels.ts:48-60) / MATMUL_SWIGLU (kernels.ts:597): f16(a / (1 + exp(-a)) * b), a, b the
    f16 matmul outputs."""
    a, b = a16.astype(acc), b16.astype(acc)
    return (a / (1.0 + np.exp(-a)) * b).astype(F16)


def gelu_tanh(x):
    """gelu of eg2-kernels.ts:9-13: tanh form with the argument clamped to +-15."""
    u = np.clip(0.7978845608 * (x + 0.044715 * x * x * x), -15.0, 15.0)
    e = np.exp(2.0 * u)
    return 0.5 * x * (1.0 + (e - 1.0) / (e + 1.0))


def gelu_mul(a16, b16, acc=F32):
    """GELU_MUL (eg2-kernels.ts:165-177): f16(gelu(a) * b)."""
    return (gelu_tanh(a16.astype(acc)) * b16.astype(acc)).astype(F16)


# ---------------------------------------------------------------- q/k norm + rope

def inv_freq(theta, rot, mode=0):
    """Angle per position of dim pair d: pow(theta, -2d/rot) (kernels.ts:106) or 1/pow(theta, 2d/rot)
    (eg2-kernels.ts:86), in f32."""
    d = np.arange(rot // 2, dtype=F32)
    ex = (F32(2) * d) / F32(rot)
    if mode == 0:
        return np.power(F32(theta), -ex).astype(F32)
    return (F32(1) / np.power(F32(theta), ex)).astype(F32)


def qk_norm_rope(Z, heads, kv, D, pos, qn=None, kn=None, vnorm=False, eps=1e-6, theta=1e6, rot=None, mode=0, acc=F32):
    """QK_NORM_ROPE (kernels.ts:86-112) generalised (QK_NORM_ROPE_256 d3-kernels.ts:151-178, ROPE
    encoder-kernels.ts:5-23, QKV_NORM_ROPE eg2-kernels.ts:50-96): per head RMSNorm over D times the weight
    (q with qn, k with kn, v plain when vnorm), then rotate-half RoPE on the first `rot` dims; the normed value
    is not rounded before RoPE. Z [T, (heads + 2kv) D] f16; returns a new array."""
    rot = D if rot is None else rot
    T = Z.shape[0]
    Z = Z.copy()
    x = Z[:, :(heads + 2 * kv) * D].reshape(T, heads + 2 * kv, D).astype(acc)
    out = x.copy()

    def norm(v, w):
        inv = 1.0 / np.sqrt((v * v).sum(-1, keepdims=True) / D + eps)
        v = v * inv
        return v * w.astype(acc) if w is not None else v

    if qn is not None:
        out[:, :heads] = norm(x[:, :heads], qn)
    if kn is not None:
        out[:, heads:heads + kv] = norm(x[:, heads:heads + kv], kn)
    if vnorm:
        out[:, heads + kv:] = norm(x[:, heads + kv:], None)
    f = inv_freq(theta, rot, mode)
    ang = (np.asarray(pos, dtype=F32)[:, None] * f[None, :]).astype(F32)  # f32 angle, as the kernels
    c, s = np.cos(ang.astype(F64)).astype(acc), np.sin(ang.astype(F64)).astype(acc)
    half = rot // 2
    for sl in (slice(0, heads), slice(heads, heads + kv)):
        a = out[:, sl, :half].copy()
        b = out[:, sl, half:rot].copy()
        out[:, sl, :half] = a * c[:, None, :] - b * s[:, None, :]
        out[:, sl, half:rot] = b * c[:, None, :] + a * s[:, None, :]
    Z[:, :(heads + 2 * kv) * D] = out.reshape(T, -1).astype(F16)
    return Z


# ---------------------------------------------------------------- packing (host side of the engines)

def pack_forest(trees):
    """D13BEngine.run's packing (d1-3b-engine.ts:46-72): per token ids, pos (branch positions continue after
    the trunk), meta (treeStart, treeEnd, branch or -1, pos); leaves = each branch's last token; leafIds =
    the flattened answer groups, zero-padded to nIds. trees: [{"trunk", "branches", "groups"}]."""
    ids, pos, meta, leaves, leaf_ids = [], [], [], [], []
    for tr in trees:
        start = len(ids)
        total = len(tr["trunk"]) + sum(len(b) for b in tr["branches"])
        p = len(tr["trunk"])
        for i, t in enumerate(tr["trunk"]):
            ids.append(t); pos.append(i); meta.append((start, start + total, -1, i))
        for b, br in enumerate(tr["branches"]):
            for o, t in enumerate(br):
                ids.append(t); pos.append(p + o); meta.append((start, start + total, b, p + o))
            leaves.append(len(ids) - 1)
            leaf_ids.append([x for g in tr["groups"][b] for x in g])
    L = len(leaves)
    n_ids = max((len(x) for x in leaf_ids), default=0)
    flat = np.zeros(L * n_ids, dtype=np.uint32)
    for i, g in enumerate(leaf_ids):
        flat[i * n_ids:i * n_ids + len(g)] = g
    return (np.array(ids, dtype=np.uint32), np.array(pos, dtype=np.int32), np.array(meta, dtype=np.int32).reshape(-1, 4),
            np.array(leaves, dtype=np.uint32), flat, n_ids)


def forest_taps(trees):
    """The short conv's taps of D13BEngine.run (d1-3b-engine.ts:56-64): per token the rows its three taps read
    (-1: none), causal over the forest: a trunk token i reads trunk tokens i-2, i-1, i; a branch token reads back
    through its own branch and then into the end of its trunk. [T, 4] i32 (the 4th unused, 0)."""
    taps, n = [], 0
    for tr in trees:
        start, p = n, len(tr["trunk"])
        for i in range(p):
            taps.append((start + i - 2 if i >= 2 else -1, start + i - 1 if i >= 1 else -1, start + i, 0))
        n += p
        for br in tr["branches"]:
            for o in range(len(br)):
                t = n + o

                def back(j):
                    if o - j >= 0:
                        return t - j
                    return start + p + (o - j) if p + (o - j) >= 0 else -1
                taps.append((back(2), back(1), t, 0))
            n += len(br)
    return np.array(taps, dtype=np.int32).reshape(-1, 4)


def short_conv(Z, H, w, taps, acc=F32):
    """SHORT_CONV (kernels.ts:62-84): Z [T, 3H] = [B | C | U]; conv = sum_j w[c, j] * f32(B[tap_j]) * f32(U[tap_j])
    (a tap < 0 reads zero); Y = f16(f32(C) * conv)."""
    Z = Z.astype(acc)
    B, C, U = Z[:, :H], Z[:, H:2 * H], Z[:, 2 * H:3 * H]
    bu = B * U
    conv = np.zeros((Z.shape[0], H), dtype=acc)
    w = w.astype(acc).reshape(H, 3)
    for j in range(3):
        tj = taps[:, j]
        ok = tj >= 0
        conv[ok] += w[:, j][None, :] * bu[tj[ok]]
    return (C * conv).astype(F16)


def forest_mask(meta, bidir=False):
    """Boolean [T, T] key mask of ATTENTION (kernels.ts:133-136): key k in [start, end) of the query's tree,
    and (bidir or (k is a trunk token and (the query is a branch token or pos_k <= pos_q)) or (same branch,
    not the trunk, pos_k <= pos_q))."""
    T = meta.shape[0]
    m = np.zeros((T, T), dtype=bool)
    for t in range(T):
        s, e, br, p = meta[t]
        for k in range(s, e):
            ks, ke, kb, kp = meta[k]
            ok = bidir or (kb == -1 and (br != -1 or kp <= p)) or (kb == br and br != -1 and kp <= p)
            m[t, k] = ok
    return m


def forest_ranges(meta):
    """The forest mask as two key ranges per query (a0, a1, b0, b1): a trunk token i sees [start, start+i+1);
    a branch token sees the trunk [start, start+P) and its own branch [branch start, itself]."""
    T = meta.shape[0]
    rng = np.zeros((T, 4), dtype=np.int32)
    t = 0
    while t < T:
        s, e = meta[t, 0], meta[t, 1]
        # the trunk: tokens of this tree with branch -1 come first
        P = 0
        while s + P < e and meta[s + P, 2] == -1:
            P += 1
        for i in range(P):
            rng[s + i] = (s, s + i + 1, 0, 0)
        k = s + P
        while k < e:
            b, bs = meta[k, 2], k
            while k < e and meta[k, 2] == b:
                rng[k] = (s, s + P, bs, k + 1)
                k += 1
        t = e
    return rng


def ranges_mask(rng, T_keys):
    m = np.zeros((rng.shape[0], T_keys), dtype=bool)
    for t, (a0, a1, b0, b1) in enumerate(rng):
        m[t, max(a0, 0):max(a1, 0)] = True
        m[t, max(b0, 0):max(b1, 0)] = True
    return m


def pack_shared(seqs, groups=None):
    """D3Engine.logits's packing (d3-engine.ts:67-93): per request group, the common id prefix P (at least one
    token left per question) laid once with rng [ts, ts+P); each question's rest with rng = trunk + itself
    (bidirectional within the ranges); pairs (last row, option k). seqs: [{"ids", "options"}]."""
    ids, meta, rng, pairs = [], [], [], []
    sizes = groups if groups is not None else [1] * len(seqs)
    si = 0
    for n in sizes:
        group = seqs[si:si + n]
        si += n
        P = 0
        if n > 1:
            lim = min(len(s["ids"]) for s in group) - 1
            while P < lim and all(s["ids"][P] == group[0]["ids"][P] for s in group):
                P += 1
        ts = len(ids)
        for i in range(P):
            ids.append(group[0]["ids"][i]); meta.append((ts, ts + P, -1, i)); rng.append((ts, ts + P, 0, 0))
        for s in group:
            bs = len(ids)
            be = bs + len(s["ids"]) - P
            for i in range(P, len(s["ids"])):
                ids.append(s["ids"][i]); meta.append((bs, be, -1, i))
                rng.append((ts if P else bs, ts + P if P else be, bs if P else 0, be if P else 0))
            for k in range(s["options"]):
                pairs.append((be - 1, k))
    return (np.array(ids, dtype=np.uint32), np.array(meta, dtype=np.int32).reshape(-1, 4), np.array(rng, dtype=np.int32).reshape(-1, 4),
            np.array(pairs, dtype=np.uint32).reshape(-1, 2))


def pack_encoder(seqs, window=None):
    """Eg2Engine.embed's packing (eg2-engine.ts:74-86): meta (start, end, -1, i), full range [start, end),
    window range [max(start, t-w), min(end, t+w+1)), and per sequence (start, end)."""
    ids, meta, full, slide, ranges = [], [], [], [], []
    for s in seqs:
        start, end = len(ids), len(ids) + len(s)
        for i, t_id in enumerate(s):
            t = start + i
            ids.append(t_id); meta.append((start, end, -1, i)); full.append((start, end, 0, 0))
            if window is not None:
                slide.append((max(start, t - window), min(end, t + window + 1), 0, 0))
        ranges.append((start, end))
    return (np.array(ids, dtype=np.uint32), np.array(meta, dtype=np.int32).reshape(-1, 4), np.array(full, dtype=np.int32).reshape(-1, 4),
            np.array(slide, dtype=np.int32).reshape(-1, 4) if window is not None else None, np.array(ranges, dtype=np.uint32).reshape(-1, 2))


# ---------------------------------------------------------------- attention

def attention(Z, heads, kv, D, mask, scale, acc=F32, q_stride=None, kv_rows=None, gate=None):
    """softmax(scale q.k) v over the allowed keys, per query and head (ATTENTION kernels.ts:114-147 and its
    tiled/eg2/d3 variants); f32 scores and sums, output f16(acc / l). mask [T, Tk] boolean. Z holds
    [q | k | v] rows; kv_rows (optional) is a separate [Tk, 2 kv D] array of [k | v] rows; gate (optional,
    [T, heads D]) multiplies the output by sigmoid(gate) before its f16 rounding (d3's attention256,
    d3-kernels.ts:232-236)."""
    T = Z.shape[0]
    q = Z[:, :heads * D].reshape(T, heads, D).astype(acc)
    if kv_rows is None:
        k = Z[:, heads * D:(heads + kv) * D].reshape(T, kv, D).astype(acc)
        v = Z[:, (heads + kv) * D:(heads + 2 * kv) * D].reshape(T, kv, D).astype(acc)
    else:
        k = kv_rows[:, :kv * D].reshape(-1, kv, D).astype(acc)
        v = kv_rows[:, kv * D:2 * kv * D].reshape(-1, kv, D).astype(acc)
    g = heads // kv
    out = np.zeros((T, heads, D), dtype=acc)
    for h in range(heads):
        s = (q[:, h, :] * acc(scale)) @ k[:, h // g, :].T
        s = np.where(mask, s, -np.inf)
        m = np.maximum(s.max(-1, keepdims=True), -1e30)
        p = np.where(mask, np.exp(s - m), 0.0)
        out[:, h, :] = (p @ v[:, h // g, :]) / p.sum(-1, keepdims=True)
    out = out.reshape(T, heads * D)
    if gate is not None:
        out = out / (1.0 + np.exp(-gate.astype(acc)))
    return out.astype(F16)


# ---------------------------------------------------------------- readouts

def leaf_logits(X, leaves, w, ids, n_ids, codes, scales, bits, eps, acc=F32):
    """LEAF_LOGITS (kernels.ts:149-185): normed = f32(X[leaf]) * inv * f32(w) (not rounded); dot with the
    f32-dequantized embedding rows of the leaf's ids; f32 out [L * nIds]."""
    L = len(leaves)
    out = np.zeros(L * n_ids, dtype=acc)
    for l in range(L):
        x = X[leaves[l]].astype(acc)
        inv = 1.0 / np.sqrt((x * x).sum(dtype=acc) / X.shape[1] + eps)
        normed = x * inv * w.astype(acc)
        for j in range(n_ids):
            r = int(ids[l * n_ids + j])
            e = dequant_f32(codes[r:r + 1], scales[r:r + 1], bits)[0].astype(acc)
            out[l * n_ids + j] = (normed * e).sum(dtype=acc)
    return out


def readout(X, R, pairs):
    """READOUT (d3-kernels.ts:242-260): out[k] = f32(X[row]) . R[code]."""
    return np.array([(X[r].astype(F32) * R[c]).sum(dtype=F32) for r, c in pairs], dtype=F32)


def mean_pool(X, ranges):
    """POOL_PROJECT's mean (eg2-kernels.ts:214-218), f32."""
    return np.stack([X[a:b].astype(F32).mean(0) for a, b in ranges])


def dense_f32(inp, codes, scales, bits):
    """f32 activations times the f32-dequantized weight (the pooled head)."""
    return (inp.astype(F32) @ dequant_f32(codes, scales, bits).T).astype(F32)


# ---------------------------------------------------------------- EmbeddingGemma 2 (eg2-kernels.ts, eg2-engine.ts)

def ple_mix(G, E, w, eps, acc=F32):
    """PLE_MIX (eg2-kernels.ts:179-200): f16(gelu_tanh(G) * E / sqrt(mean(E^2) + eps) * w)."""
    e = E.astype(acc)
    inv = 1.0 / np.sqrt((e * e).sum(-1, keepdims=True) / E.shape[-1] + eps)
    return (gelu_tanh(G.astype(acc)) * e * inv * w.astype(acc)).astype(F16)


def pool_project(X, ranges, W):
    """POOL_PROJECT (eg2-kernels.ts:202-228): the f32 mean of each sequence's rows, times the f16 projection W
    [N, H]^T, in f32."""
    return (mean_pool(X, ranges).astype(F32) @ W.astype(F32).T).astype(F32)


def eg2_forward(model: "Model", seqs, acc=F32, layers=None):
    """Eg2Engine.embed (eg2-engine.ts:72-139) on the shipped layout: two gathers of the (sqrt(hidden)-scaled)
    embedding (the residual stream x and the copy xe the per-layer embeddings read); per layer q/k/v RMSNorm +
    RoPE (rotate-half over the whole head, 1/theta^(2d/D) of the layer type's theta) -> bidirectional attention
    at scale 1 over the layer type's key ranges (the sequence, or +-window on the sliding layers) -> o ->
    sandwich -> gate|up with the tanh GELU -> down -> x += rmsnorm(.) w; then the per-layer embedding:
    gate = x . ple_gate^T, e = xe . ple_in^T, ple_proj(PLE_MIX(gate, e)) -> sandwich with ple_norm, the layer scalar
    and the next input norm (final_norm after the last); POOL_PROJECT; the first embed_dim values L2-normalised.
    Returns (embeddings f32 [S, embed_dim], final normed f16 [T, H])."""
    c = model.c
    H, I, h, eps, P = c["hidden"], c["intermediate"], c["heads"], c["eps"], c["ple"]
    L = c["layers"] if layers is None else layers
    ids, meta, full, slide, ranges = pack_encoder(seqs, c["window"])
    T = len(ids)
    masks = {"full_attention": ranges_mask(full, T), "sliding_attention": ranges_mask(slide, T)}
    ec, es, eb = model.t["embed"]
    x = gather(ids, ec, es, eb)
    xe = x.copy()
    x, normed = sandwich(x, None, None, model.t["layers.0.input_layernorm"], eps, 1.0, acc)
    scalars = c.get("layer_scalars", [1.0] * c["layers"])
    for i in range(L):
        p, t = f"layers.{i}.", c["layer_types"][i]
        D, kv = c["head_dim"][t], c["kv_heads"][t]
        z = matmul(normed, model.w16(p + "qkv"), acc)
        z = qk_norm_rope(z, h, kv, D, meta[:, 3], model.t[p + "q_norm"], model.t[p + "k_norm"], True, eps,
                         c["rope_theta"][t], mode=1, acc=acc)
        o = matmul(attention(z, h, kv, D, masks[t], 1.0, acc), model.w16(p + "o"), acc)
        x, normed = sandwich(x, o, model.t[p + "post_attention_layernorm"], model.t[p + "pre_feedforward_layernorm"], eps, 1.0, acc)
        gu = matmul(normed, model.w16(p + "gu"), acc)
        o = matmul(gelu_mul(gu[:, :I], gu[:, I:], acc), model.w16(p + "down"), acc)
        x, _ = sandwich(x, o, model.t[p + "post_feedforward_layernorm"], None, eps, 1.0, acc)
        g = matmul(x, model.w16(p + "ple_gate"), acc)
        e = matmul(xe, model.w16(p + "ple_in"), acc)
        o = matmul(ple_mix(g, e, model.t["ple.norm"], eps, acc), model.w16(p + "ple_proj"), acc)
        nxt = f"layers.{i + 1}.input_layernorm" if i + 1 < L else "final_norm"
        x, normed = sandwich(x, o, model.t[p + "ple_norm"], model.t[nxt], eps, float(scalars[i]), acc)
    out = pool_project(normed, ranges, model.t["projection"])[:, :c["embed_dim"]].astype(F64)
    n = np.maximum(np.sqrt((out * out).sum(-1, keepdims=True)), 1e-12)
    return (out / n).astype(F32), normed


# ---------------------------------------------------------------- d3-lite's Gated DeltaNet (d3-kernels.ts:9-149)

def d3_spans(seqs, groups=None):
    """The GDN scans of D3Engine.logits's packing (d3-engine.ts:89): per question (a start, a length | write_a <<
    31, b start, b length): with a shared prefix P, a = the trunk (written by the group's first question only)
    and b = the question's own tokens; without one, a = the whole sequence (written) and b empty. Rows follow
    pack_shared's layout. [S, 4] u32."""
    sizes = groups if groups is not None else [1] * len(seqs)
    spans, si, off = [], 0, 0
    for n in sizes:
        group = seqs[si:si + n]
        si += n
        P = 0
        if n > 1:
            lim = min(len(s["ids"]) for s in group) - 1
            while P < lim and all(s["ids"][P] == group[0]["ids"][P] for s in group):
                P += 1
        ts = off
        off += P
        for b, s in enumerate(group):
            bs, L = off, len(s["ids"]) - P
            off += L
            if P:
                spans.append((ts, P | (0x80000000 if b == 0 else 0), bs, L))
            else:
                spans.append((bs, L | 0x80000000, 0, 0))
    return np.array(spans, dtype=np.uint32).reshape(-1, 4)


def gdn(Z, spans, LH, conv_w, A_log, dt_bias, gnorm, eps, acc=F32):
    """gdnLayer (d3-kernels.ts:9-149) in its textbook form: for each scan and head, the causal 4-tap conv (tap 3
    the token itself, zero before the sequence start) + SiLU of the q, k, v channels, rounded to f16; q and k L2
    normalised (eps 1e-6 inside the root), q scaled by 128^-1/2; decay = exp(-exp(A_log) softplus(a + dt_bias))
    (softplus(x) = x past 20), beta = sigmoid(b); per token S <- decay S; delta = beta (v - S k); S <- S + delta
    k^T; o = S q (S [v, k] in acc); then y = f16(o / sqrt(mean(o^2) + eps) * gnorm * silu(z)). Z rows q | k | v |
    z (LH x 128 each) | b | a (LH each). Returns Y [T, LH 128] f16 (rows no scan writes stay 0)."""
    T = Z.shape[0]
    QK = LH * 128
    Y = np.zeros((T, QK), dtype=F16)
    W = conv_w.astype(acc).reshape(3 * QK, 4)
    for a0, aw, b0, bl in np.asarray(spans, dtype=np.int64):
        alen, write_a = int(aw) & 0x7fffffff, (int(aw) >> 31) & 1
        rows = list(range(a0, a0 + alen)) + list(range(b0, b0 + bl))
        n = len(rows)
        if n == 0:
            continue
        X = Z[rows].astype(acc)
        for h in range(LH):
            ch = np.concatenate([np.arange(128) + h * 128, QK + np.arange(128) + h * 128, 2 * QK + np.arange(128) + h * 128])
            x = np.concatenate([np.zeros((3, len(ch)), dtype=acc), X[:, ch]])
            w = W[ch]
            y = sum(w[:, j][None, :] * x[j:j + n] for j in range(4))
            y = (y / (1.0 + np.exp(-y))).astype(F16).astype(acc)
            q, k, v = y[:, :128], y[:, 128:256], y[:, 256:]
            q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(acc(128))
            k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
            b = X[:, 4 * QK + h]
            a = X[:, 4 * QK + LH + h] + acc(dt_bias[h])
            sp = np.where(a > 20, a, np.log1p(np.exp(np.minimum(a, 20))))
            dec = np.exp(-np.exp(acc(A_log[h])) * sp)
            beta = 1.0 / (1.0 + np.exp(-b))
            S = np.zeros((128, 128), dtype=acc)
            o = np.zeros((n, 128), dtype=acc)
            for t in range(n):
                S = dec[t] * S
                delta = beta[t] * (v[t] - S @ k[t])
                S = S + np.outer(delta, k[t])
                o[t] = S @ q[t]
            inv = 1.0 / np.sqrt((o * o).mean(-1, keepdims=True) + eps)
            z = X[:, 3 * QK + h * 128:3 * QK + (h + 1) * 128]
            out = (o * inv * gnorm.astype(acc) * (z / (1.0 + np.exp(-z)))).astype(F16)
            for i, r in enumerate(rows):
                if i < alen and not write_a:
                    continue
                Y[r, h * 128:(h + 1) * 128] = out[i]
    return Y


def d3_forward(model: "Model", seqs, groups=None, acc=F32):
    """D3Engine.logits (d3-engine.ts:67-139) on the shipped d3-lite layout: per layer the input RMSNorm (adding
    the previous MLP output), then a Gated DeltaNet mixer (`in` product, gdn on d3_spans, `out` product) or a
    gated attention layer (fused q | k | v | gate product, q/k RMSNorm over 256 with RoPE on the first
    `rotary_dim` dims at each token's position, attention over pack_shared's key ranges at 1/sqrt(head_dim),
    output times sigmoid(gate), `o` product), the post RMSNorm, SwiGLU; the final norm; READOUT at (row, code)
    pairs. Returns (code logits f32 [pairs], final normed hidden f16 [T, H])."""
    c = model.c
    H, I, h, kv, D, eps = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["eps"]
    LH = c["linear_heads"]
    ids, meta, rng, pairs = pack_shared(seqs, groups)
    spans = d3_spans(seqs, groups)
    T = len(ids)
    mask = ranges_mask(rng, T)
    stride = (2 * h + 2 * kv) * D
    ec, es, eb = model.t["embed"]
    x = gather(ids, ec, es, eb)
    o = None
    for i, t in enumerate(c["layer_types"]):
        p = f"layers.{i}."
        x, normed = add_rmsnorm(x, o, model.t[p + "input_norm"], eps, add=i > 0, acc=acc)
        if t == "linear_attention":
            z = matmul(normed, model.w16(p + "in"), acc)
            g = gdn(z, spans, LH, model.t[p + "conv"], model.t[p + "A_log"], model.t[p + "dt_bias"], model.t[p + "gnorm"],
                    eps, acc)
            o = matmul(g, model.w16(p + "out"), acc)
        else:
            z = matmul(normed, model.w16(p + "qkvg"), acc)
            z = qk_norm_rope(z, h, kv, D, meta[:, 3], model.t[p + "q_norm"], model.t[p + "k_norm"], False, eps,
                             c["rope_theta"], rot=c["rotary_dim"], acc=acc)
            y = attention(z, h, kv, D, mask, 1.0 / math.sqrt(D), acc, gate=z[:, (h + 2 * kv) * D:stride])
            o = matmul(y, model.w16(p + "o"), acc)
        x, normed = add_rmsnorm(x, o, model.t[p + "post_norm"], eps, acc=acc)
        ab = matmul(normed, model.w16(p + "w13"), acc)
        o = matmul(silu_mul(ab[:, :I], ab[:, I:], acc), model.w16(p + "w2"), acc)
    x, normed = add_rmsnorm(x, o, model.t["final_norm"], eps, acc=acc)
    return readout(normed, model.t["readout"], pairs), normed


# ---------------------------------------------------------------- d1-omni's decision head (kernels.ts:186-283)

def add_rows(X, idx, E, acc=F32):
    """ADD_ROWS (kernels.ts:188-201): f16(f32(X[t]) + f32(E[idx[t]])) (idx past the table: its last row)."""
    idx = np.minimum(np.asarray(idx, dtype=np.int64), E.shape[0] - 1)
    return (X.astype(acc) + E[idx].astype(acc)).astype(F16)


def erf_as(x):
    """erf of BIAS_ACT (kernels.ts:208-212): Abramowitz & Stegun 7.1.26, |error| < 1.5e-7."""
    x = np.asarray(x)
    t = 1.0 / (1.0 + 0.3275911 * np.abs(x))
    y = 1.0 - ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t * np.exp(-x * x)
    return np.where(x >= 0, y, -y)


def bias_act(Y, b, act=0, acc=F32):
    """BIAS_ACT (kernels.ts:203-222): f16(act(f32(Y) + f32(b))), act 0 none, 1 ReLU, 2 GELU with erf_as."""
    v = Y.astype(acc) + b.astype(acc)
    if act == 1:
        v = np.maximum(v, acc(0))
    elif act == 2:
        v = acc(0.5) * v * (acc(1) + erf_as(v * acc(0.70710678)).astype(acc))
    return v.astype(F16)


def add_layernorm(X, Y, w, b, eps, add=True, acc=F32):
    """ADD_LAYERNORM (kernels.ts:224-255): v = X (+ Y), X <- f16(v); mean and E[v^2] of the unrounded v;
    var = max(E[v^2] - mean^2, 0); O = f16((f32(X_f16) - mean) / sqrt(var + eps) * w + b). Returns (X_new, O)."""
    v = X.astype(acc)
    if add:
        v = v + Y.astype(acc)
    H = X.shape[-1]
    mean = v.sum(-1, keepdims=True, dtype=acc) / acc(H)
    var = np.maximum((v * v).sum(-1, keepdims=True, dtype=acc) / acc(H) - mean * mean, acc(0))
    Xn = v.astype(F16)
    inv = (1.0 / np.sqrt(var + eps)).astype(acc)
    return Xn, ((Xn.astype(acc) - mean) * inv * w.astype(acc) + b.astype(acc)).astype(F16)


def score(Y, w, b, acc=F32):
    """SCORE (kernels.ts:269-283): out[m] = Y[m] . w + b[0], f32."""
    return ((Y.astype(acc) @ w.astype(acc)) + acc(b[0])).astype(F32)


def pack_omni(seqs):
    """D1OmniEngine.logits's packing (omni-engine.ts:62-75): per token its id, its position in its sequence, its
    question type (choice 0, score 1, noul 2), the centred taps (t-1, t, t+1; -1 past either end of the
    sequence) and its key range [start, end) (bidirectional within the sequence); per option marker its row.
    seqs: [{"ids", "markers", "type"}]."""
    QT = {"choice": 0, "score": 1, "noul": 2}
    ids, pos, qtype, taps, rng, markers = [], [], [], [], [], []
    for s in seqs:
        start, end = len(ids), len(ids) + len(s["ids"])
        for i, tok in enumerate(s["ids"]):
            t = start + i
            ids.append(tok); pos.append(i); qtype.append(QT[s["type"]])
            taps.append((t - 1 if t > start else -1, t, t + 1 if t + 1 < end else -1, 0))
            rng.append((start, end, 0, 0))
        markers.extend(start + m for m in s["markers"])
    return {"ids": np.array(ids, dtype=np.uint32), "pos": np.array(pos, dtype=np.uint32),
            "qtype": np.array(qtype, dtype=np.uint32), "taps": np.array(taps, dtype=np.int32).reshape(-1, 4),
            "rng": np.array(rng, dtype=np.int32).reshape(-1, 4), "markers": np.array(markers, dtype=np.uint32), "T": len(ids)}


def omni_temperature(temps, qtype, options):
    """temperature() of omni-engine.ts:22-26 (prompt.py temperature_key): "<type>:<bucket>" with buckets 2,
    3-5, 6-10, 11+, else "<type>", else 1."""
    k = "2" if options <= 2 else "3-5" if options <= 5 else "6-10" if options <= 10 else "11+"
    return float(temps.get(f"{qtype}:{k}", temps.get(qtype, 1.0)))


def omni_forward(model: "Model", seqs, acc=F32, layers=None):
    """D1OmniEngine.logits (omni-engine.ts:55-149): the bidirectional LFM2 trunk (conv layers on the centred
    taps, attention layers with q/k norm + RoPE over the whole sequence, SwiGLU, final norm), then the head:
    the question-type row added, `head_layers` pre-norm transformer layers (LayerNorm with bias, fused
    in_proj + bias, attention over the sequence at scale 1/sqrt(D), out_proj + bias, LayerNorm, linear1 + bias
    + ReLU, linear2 + bias), the last residual with the scorer's LayerNorm, then at each marker Linear + bias +
    GELU (erf) and Linear(H, 1). Returns (marker logits f32 [M], {"trunk": f16 [T, H], "head": f16 [T, H]})."""
    c = model.c
    H, I, h, kv, D, eps = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["eps"]
    types = c["layer_types"]
    L = len(types) if layers is None else layers
    pk = pack_omni(seqs)
    T = pk["T"]
    mask = ranges_mask(pk["rng"], T)
    ec, es, eb = model.t["embed"]
    x = gather(pk["ids"], ec, es, eb)
    x, normed = add_rmsnorm(x, None, model.t["layers.0.operator_norm"], eps, add=False, acc=acc)
    for i in range(L):
        p = f"layers.{i}."
        if types[i] == "conv":
            z = matmul(normed, model.w16(p + "in_proj"), acc)
            o = matmul(short_conv(z, H, model.t[p + "conv"], pk["taps"], acc), model.w16(p + "out_proj"), acc)
        else:
            z = matmul(normed, model.w16(p + "qkv"), acc)
            z = qk_norm_rope(z, h, kv, D, pk["pos"], model.t[p + "q_norm"], model.t[p + "k_norm"], False, eps,
                             c["rope_theta"], acc=acc)
            o = matmul(attention(z, h, kv, D, mask, 1.0 / math.sqrt(D), acc), model.w16(p + "o_proj"), acc)
        x, normed = add_rmsnorm(x, o, model.t[p + "ffn_norm"], eps, acc=acc)
        ab = matmul(normed, model.w16(p + "w13"), acc)
        o = matmul(silu_mul(ab[:, :I], ab[:, I:], acc), model.w16(p + "w2"), acc)
        nxt = f"layers.{i + 1}.operator_norm" if i + 1 < L else "final_norm"
        x, normed = add_rmsnorm(x, o, model.t[nxt], eps, acc=acc)
    trunk = normed
    logits, x = marker_head(model, trunk, pk, mask, acc)
    return logits, {"trunk": trunk, "head": x}


def marker_head(model: "Model", trunk, pk, mask, acc=F32):
    """d1-omni's decision head and scorer on the trunk's output (omni-engine.ts:125-147, laya-engine.ts:114-138):
    the question-type row added, `head_layers` pre-norm layers (LayerNorm with bias, in_proj + bias, attention over
    the sequence at 1/sqrt(D), out_proj + bias, LayerNorm, linear1 + bias + ReLU, linear2 + bias), the last residual
    under the scorer's LayerNorm, then at each marker Linear + bias + GELU (erf) and Linear(H, 1). Returns (marker
    logits f32 [M], the head's residual stream f16 [T, H])."""
    c = model.c
    H = c["hidden"]
    hh, ln = c["head_heads"], c["ln_eps"]
    Dh = H // hh
    x = add_rows(trunk, pk["qtype"], model.t["head.type_emb"], acc)
    o = None
    for i in range(c["head_layers"]):
        p = f"head.{i}."
        x, n1 = add_layernorm(x, o, model.t[p + "norm1"], model.t[p + "norm1_bias"], ln, add=i > 0, acc=acc)
        z = bias_act(matmul(n1, model.w16(p + "in_proj"), acc), model.t[p + "in_proj_bias"], 0, acc)
        y = attention(z, hh, hh, Dh, mask, 1.0 / math.sqrt(Dh), acc)
        o = bias_act(matmul(y, model.w16(p + "out_proj"), acc), model.t[p + "out_proj_bias"], 0, acc)
        x, n2 = add_layernorm(x, o, model.t[p + "norm2"], model.t[p + "norm2_bias"], ln, acc=acc)
        f = bias_act(matmul(n2, model.w16(p + "linear1"), acc), model.t[p + "linear1_bias"], 1, acc)
        o = bias_act(matmul(f, model.w16(p + "linear2"), acc), model.t[p + "linear2_bias"], 0, acc)
    x, sn = add_layernorm(x, o, model.t["scorer.norm"], model.t["scorer.norm_bias"], ln, add=o is not None, acc=acc)
    g = sn[pk["markers"].astype(np.int64)]
    gf = bias_act(matmul(g, model.w16("scorer.fc"), acc), model.t["scorer.fc_bias"], 2, acc)
    return score(gf, model.t["scorer.out"], model.t["scorer.out_bias"], acc), x


def gelu_erf_mul(a16, b16, acc=F32):
    """GELU_MUL of encoder-kernels.ts:25-41: f16(0.5 a (1 + erf_as(a / sqrt 2)) b)."""
    a, b = a16.astype(acc), b16.astype(acc)
    return (acc(0.5) * a * (acc(1) + erf_as(a * acc(0.70710678)).astype(acc)) * b).astype(F16)


def laya_windows(rng, window):
    """The local layers' key ranges of laya-engine.ts:64: token t of a sequence [start, end) sees
    [max(start, t - window), min(end, t + window + 1)) (a per-token loop)."""
    out = np.zeros((len(rng), 4), dtype=np.int32)
    for t in range(len(rng)):
        out[t, 0] = max(int(rng[t, 0]), t - window)
        out[t, 1] = min(int(rng[t, 1]), t + window + 1)
    return out


def laya_forward(model: "Model", seqs, acc=F32):
    """LayaEngine.logits (laya-engine.ts:55-150): the ModernBERT encoder — the embedding rows under the bias-free
    embed_norm; per layer the attention input (layer 0: the stream itself; later layers: the bias-free attn_norm
    after adding the previous MLP output), fused qkv, RoPE on q and k over the whole 64-dim head (pow(theta,
    -2d/64) of the layer type's theta), attention at 1/8 over the sequence (global layers) or a +-window (the
    others), Wo, add + mlp_norm, Wi with the erf-GELU gate, Wo; the last MLP output added under final_norm — then
    d1-omni's head and scorer. Returns (marker logits f32 [M], {"trunk": f16 [T, H], "head": f16 [T, H]})."""
    c = model.c
    H, I, h, eps = c["hidden"], c["intermediate"], c["heads"], c["eps"]
    D = H // h
    pk = pack_omni(seqs)
    T = pk["T"]
    full = ranges_mask(pk["rng"], T)
    slide = ranges_mask(laya_windows(pk["rng"], c["window"]), T)
    zeros = np.zeros(H, dtype=F16)
    ec, es, eb = model.t["embed"]
    e = gather(pk["ids"], ec, es, eb)
    _, x = add_layernorm(e, None, model.t["embed_norm"], zeros, eps, add=False, acc=acc)
    o = None
    for i, lt in enumerate(c["layer_types"]):
        p = f"layers.{i}."
        inp = x
        if p + "attn_norm" in model.t:
            x, inp = add_layernorm(x, o, model.t[p + "attn_norm"], zeros, eps, add=o is not None, acc=acc)
        z = matmul(inp, model.w16(p + "qkv"), acc)
        z = qk_norm_rope(z, h, h, D, pk["pos"], None, None, False, eps, c["rope_theta"][lt], acc=acc)
        y = attention(z, h, h, D, full if lt == "full_attention" else slide, 1.0 / math.sqrt(D), acc)
        o = matmul(y, model.w16(p + "o"), acc)
        x, normed = add_layernorm(x, o, model.t[p + "mlp_norm"], zeros, eps, acc=acc)
        ab = matmul(normed, model.w16(p + "wi"), acc)
        o = matmul(gelu_erf_mul(ab[:, :I], ab[:, I:], acc), model.w16(p + "wo"), acc)
    x, trunk = add_layernorm(x, o, model.t["final_norm"], zeros, eps, acc=acc)
    logits, hx = marker_head(model, trunk, pk, full, acc)
    return logits, {"trunk": trunk, "head": hx}


# ---------------------------------------------------------------- host tail (gpu.ts, d1.ts, questions.ts)

def softmax(s):
    """softmax of gpu.ts:294-297 in float64."""
    s = np.asarray(s, dtype=F64)
    e = np.exp(s - s.max())
    return e / e.sum()


def group_max(out, n_ids, groups_per_leaf):
    """The readout of d1-3b-engine.ts:112-121: each option scores the max over its group."""
    scores = []
    for leaf, groups in enumerate(groups_per_leaf):
        j, s = 0, []
        for g in groups:
            s.append(max(float(out[leaf * n_ids + j + i]) for i in range(len(g))))
            j += len(g)
        scores.append(s)
    return scores


# ---------------------------------------------------------------- whole forwards

class Model:
    """A decision.js-format model read into host arrays (manifest config + tensors)."""

    def __init__(self, base):
        import json
        import os
        with open(os.path.join(base, "manifest.json")) as f:
            self.m = json.load(f)
        self.c = self.m["config"]
        mm = np.memmap(os.path.join(base, "weights.bin"), dtype=np.uint8, mode="r")
        self.t = {}
        for name, info in self.m["tensors"].items():
            raw = np.asarray(mm[info["offset"]:info["offset"] + info["bytes"]])
            if info["dtype"] in ("q4", "q8"):
                N, K = info["shape"]
                sc = np.asarray(mm[info["scales"]:info["scales"] + info["scales_bytes"]]).view(F16).reshape(N, K // 32)
                self.t[name] = (raw.reshape(N, -1), sc, 8 if info["dtype"] == "q8" else 4)
            else:
                self.t[name] = raw.view(F16 if info["dtype"] == "f16" else F32).reshape(info["shape"])
        self._w16 = {}

    def w16(self, name):
        if name not in self._w16:
            c, s, b = self.t[name]
            self._w16[name] = dequant_f16(c, s, b)
        return self._w16[name]


def decoder_forward(model: Model, ids, pos, mask, leaves, leaf_ids, n_ids, acc=F32, layers=None, kv_prefix=None,
                    keep_kv=False, debug_layers=(), pairs=None, taps=None):
    """The causal decoder forward of D13BEngine.run (d1-3b-engine.ts:86-106) on attention-only layers:
    gather -> rmsnorm -> per layer [qkv, qk-norm+rope, attention, o_proj, add+rmsnorm, w13+SwiGLU, w2,
    add+rmsnorm] -> LEAF_LOGITS at the leaves. kv_prefix: per-layer [P, 2 kv D] kept K/V rows that the mask's
    first P columns refer to (shared-state mode). pairs: (row, code) pairs of d3's READOUT (d3-engine.ts:128-131,
    d3-kernels.ts:242-260): the code logits of the final norm's f16 output against the model's f32 `readout`
    matrix replace the leaf logits. Returns (logits [L * nIds] or [pairs], per-layer K/V rows if keep_kv,
    debug {layer: x}). LFM2 conv layers (layer_types "conv", d1-3b-engine.ts:90-93) run in_proj, SHORT_CONV on
    `taps` (forest_taps) and out_proj in place of attention."""
    c = model.c
    H, I, h, kv, D, eps = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["eps"]
    L = c["layers"] if layers is None else layers
    types = c.get("layer_types", ["full_attention"] * L)
    ec, es, eb = model.t["embed"]
    x = gather(ids, ec, es, eb)
    T = x.shape[0]
    o = np.zeros_like(x)
    x, normed = add_rmsnorm(x, o, model.t["layers.0.operator_norm"], eps, add=False, acc=acc)
    kept, dbg = [], {}
    for i in range(L):
        p = f"layers.{i}."
        if types[i] == "conv":
            z = matmul(normed, model.w16(p + "in_proj"), acc)
            o = matmul(short_conv(z, H, model.t[p + "conv"], taps, acc), model.w16(p + "out_proj"), acc)
            if keep_kv:
                kept.append(None)
        else:
            z = matmul(normed, model.w16(p + "qkv"), acc)
            z = qk_norm_rope(z, h, kv, D, pos, model.t.get(p + "q_norm"), model.t.get(p + "k_norm"), False, eps,
                             c["rope_theta"], acc=acc)
            if keep_kv:
                kept.append(z[:, h * D:(h + 2 * kv) * D].copy())
            if kv_prefix is not None:
                rows = np.concatenate([kv_prefix[i], z[:, h * D:(h + 2 * kv) * D]])
                y = attention(z, h, kv, D, mask, 1.0 / math.sqrt(D), acc, kv_rows=rows)
            else:
                y = attention(z, h, kv, D, mask, 1.0 / math.sqrt(D), acc)
            o = matmul(y, model.w16(p + "o_proj"), acc)
        x, normed = add_rmsnorm(x, o, model.t[p + "ffn_norm"], eps, acc=acc)
        ab = matmul(normed, model.w16(p + "w13"), acc)
        hh = silu_mul(ab[:, :I], ab[:, I:], acc)
        o = matmul(hh, model.w16(p + "w2"), acc)
        nxt = f"layers.{i + 1}.operator_norm" if i + 1 < L else "final_norm"
        x, normed = add_rmsnorm(x, o, model.t[nxt], eps, acc=acc)
        if i in debug_layers:
            dbg[i] = x.copy()
    if pairs is not None:
        return readout(normed, model.t["readout"], pairs), kept, dbg
    logits = leaf_logits(x, leaves, model.t["final_norm"], leaf_ids, n_ids, ec, es, eb, eps, acc) if len(leaves) else None
    return logits, kept, dbg


def encoder_forward(model: Model, seqs, acc=F32, layers=None):
    """The EmbeddingGemma-shaped encoder (Eg2Engine.embed, eg2-engine.ts:103-139, without per-layer embeddings)
    and the configured head: sandwich norms, q/k/v norm + RoPE, bidirectional attention (scale 1), GeGLU
    (tanh), mean pool (f32), Linear 768->3072 -> Linear 3072->768 in f32, L2 normalisation."""
    c = model.c
    H, I, h, kv, D, eps = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["eps"]
    L = c["layers"] if layers is None else layers
    ids, meta, full, _, ranges = pack_encoder(seqs)
    mask = ranges_mask(full, len(ids))
    ec, es, eb = model.t["embed"]
    x = gather(ids, ec, es, eb)
    x, normed = sandwich(x, None, None, model.t["layers.0.input_layernorm"], eps, 1.0, acc)
    for i in range(L):
        p = f"layers.{i}."
        z = matmul(normed, model.w16(p + "qkv"), acc)
        z = qk_norm_rope(z, h, kv, D, meta[:, 3], model.t[p + "q_norm"], model.t[p + "k_norm"], True, eps,
                         c["rope_theta"], mode=1, acc=acc)
        y = attention(z, h, kv, D, mask, c.get("attention_scale", 1.0), acc)
        o = matmul(y, model.w16(p + "o"), acc)
        x, normed = sandwich(x, o, model.t[p + "post_attention_layernorm"], model.t[p + "pre_feedforward_layernorm"], eps, 1.0, acc)
        gu = matmul(normed, model.w16(p + "gu"), acc)
        hh = gelu_mul(gu[:, :I], gu[:, I:], acc)
        o = matmul(hh, model.w16(p + "down"), acc)
        nxt = f"layers.{i + 1}.input_layernorm" if i + 1 < L else "final_norm"
        x, normed = sandwich(x, o, model.t[p + "post_feedforward_layernorm"], model.t[nxt], eps,
                             c.get("layer_scalars", [1.0] * L)[i], acc)
    pooled = mean_pool(normed, ranges)
    d1c, d1s, d1b = model.t["head.dense1"]
    d2c, d2s, d2b = model.t["head.dense2"]
    e = dense_f32(dense_f32(pooled, d1c, d1s, d1b), d2c, d2s, d2b)
    n = np.maximum(np.sqrt((e.astype(F64) ** 2).sum(-1, keepdims=True)), 1e-12)
    return (e / n).astype(F32)


def cosine_scores(state_e, question_e, option_es):
    """The cosine prior of Eg2Head.logits (eg2-head.ts:82-84, 97): cos(option, state + question)."""
    anchor = state_e.astype(F64) + question_e.astype(F64)
    an = max(np.sqrt((anchor ** 2).sum()), 1e-12)
    out = []
    for o in option_es:
        o = o.astype(F64)
        on = o / max(np.sqrt((o ** 2).sum()), 1e-12)
        out.append(float((on * anchor).sum() / an))
    return out
