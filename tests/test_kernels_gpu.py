"""Kernel-level parity of libdj.so against the oracle (GPU). Every call goes through the C ABI."""
import math

import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu


def _dj():
    from decision_js_amd import _dj
    return _dj


def _fmt():
    from decision_js_amd import fmt
    return fmt


def rand_f16(rng, shape, std=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float16)


def f16_close(got, want, ulps=1.0, atol=1e-5):
    """|got - want| <= ulps * 2^-10 |want| + atol, elementwise; returns the worst ratio to the bound."""
    g, w = got.astype(np.float64), want.astype(np.float64)
    bound = ulps * 2.0 ** -10 * np.abs(w) + atol
    return float((np.abs(g - w) / bound).max())


def quant(rng, N, K, bits, std=0.02):
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32(std)
    return (_fmt().quantize8 if bits == 8 else _fmt().quantize4)(w)[:2]


def run(ctx, fn):
    rec = ctx.recorder()
    fn(rec)
    return rec.finish()


# ---------------------------------------------------------------- gather

@pytest.mark.parametrize("bits", [8, 4])
def test_gather_bit_exact(pkg, ctx, bits):
    dj = _dj()
    rng = np.random.default_rng(bits)
    V, H, T = 300, 1024, 257
    codes, scales = quant(rng, V, H, bits)
    # every code value in row 0 and extreme scales in row 1, to cover the whole table
    c = ref.unpack_codes(codes, bits).copy()
    c[0] = np.arange(H) % (256 if bits == 8 else 16)
    codes = c.astype(np.uint8) if bits == 8 else (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)
    scales[1] = np.array([6.1e-5, 65504.0 / 300, 1e-3, 0.5] * (H // 128), dtype=np.float16)
    ids = rng.integers(0, V, T).astype(np.uint32)
    ids[:3] = [0, 1, V + 50]  # an id past the vocabulary reads the last row
    E = ctx.weight_q(codes, scales, V, H, bits, dj.W_PLAIN)
    d_ids, X = ctx.array(ids), ctx.alloc(T * H * 2)
    run(ctx, lambda r: r.gather_q(d_ids, T, E, X))
    got = X.read(np.uint16, (T, H))
    want = ref.gather(ids, codes, scales, bits).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- norms

@pytest.mark.parametrize("H,add", [(1024, True), (1024, False), (768, True), (2048, True), (1536, True), (4160, True)])
def test_add_rmsnorm(pkg, ctx, H, add):
    rng = np.random.default_rng(H + add)
    T = 133
    X, Y = rand_f16(rng, (T, H)), rand_f16(rng, (T, H))
    w = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    dX, dY, dw, dO = ctx.array(X), ctx.array(Y), ctx.array(w), ctx.alloc(T * H * 2)
    run(ctx, lambda r: r.add_rmsnorm(T, H, add, 1e-6, dX, dY, dw, dO))
    Xn, O = ref.add_rmsnorm(X, Y, w, 1e-6, add=add, acc=np.float64)
    assert np.array_equal(dX.read(np.float16, (T, H)).view(np.uint16), Xn.view(np.uint16))  # f16(f32 sum): exact
    assert f16_close(dO.read(np.float16, (T, H)), O, ulps=1.0) <= 1.0


@pytest.mark.parametrize("with_y,with_w2,H", [(True, True, 768), (True, False, 768), (False, True, 768),
                                              (True, True, 2560), (True, True, 4160), (False, True, 4160)])
def test_sandwich(pkg, ctx, with_y, with_w2, H):
    rng = np.random.default_rng(7)
    T = 50
    X, Y = rand_f16(rng, (T, H)), rand_f16(rng, (T, H))
    w1, w2 = (1 + rng.standard_normal(H) * 0.1).astype(np.float16), (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    dX, dY, d1, d2, dO = ctx.array(X), ctx.array(Y), ctx.array(w1), ctx.array(w2), ctx.alloc(T * H * 2)
    run(ctx, lambda r: r.sandwich(T, H, 1e-6, 0.75, dX, dY if with_y else None, d1 if with_y else None, d2 if with_w2 else None, dO))
    Xn, O = ref.sandwich(X, Y if with_y else None, w1, w2 if with_w2 else None, 1e-6, 0.75, np.float64)
    assert f16_close(dX.read(np.float16, (T, H)), Xn, ulps=1.0) <= 1.0
    if with_w2:
        assert f16_close(dO.read(np.float16, (T, H)), O, ulps=2.0) <= 1.0


# ---------------------------------------------------------------- quantized matmul

@pytest.mark.parametrize("M,N,K,bits", [
    (384, 4096, 1024, 8), (384, 1024, 3072, 8), (1152, 6144, 1024, 8),  # the minimum slice's shapes
    (77, 1040, 128, 8), (2304, 256, 512, 8), (5, 1024, 1536, 8),
    (512, 2560, 2048, 4), (300, 2048, 11008, 4), (2100, 512, 256, 4), (33, 48, 64, 4),
    # skinny M (the GEMV-style kernel): one row, a single K step, 16/17/32/64 rows, long K in several batches
    (1, 2048, 1536, 8), (8, 1536, 64, 8), (16, 1536, 4608, 8), (17, 2048, 1536, 4), (32, 1536, 1536, 8),
    (64, 2560, 2048, 4), (32, 2048, 11008, 4),
    # long K on one round of 128x128 tiles: split 4 ways along K (K / 64 divisible by 4), else unsplit
    (1024, 2048, 4096, 4), (1152, 2560, 4352, 8), (1024, 2048, 4160, 8), (1024, 1536, 4608, 8),
    (256, 1536, 4608, 8), (256, 2048, 4160, 4),
])
@pytest.mark.parametrize("direct", [False, True])
def test_matmul(pkg, ctx, M, N, K, bits, direct):
    dj = _dj()
    rng = np.random.default_rng(M * 7 + N + K + bits)
    codes, scales = quant(rng, N, K, bits)
    W16 = ref.dequant_f16(codes, scales, bits)
    X = rand_f16(rng, (M, K))
    W = ctx.weight_q(codes, scales, N, K, bits, dj.W_MFMA | (dj.W_DIRECT if direct else 0))
    dX, dY = ctx.array(X), ctx.alloc(M * N * 2)
    ctx.profile_reset()
    ctx.profile(True)
    try:
        run(ctx, lambda r: r.matmul(dX, W, dY, M))
    finally:
        ctx.profile(False)
    labels = [name for name in ctx.profile_table() if name.startswith("matmul")]
    got = dY.read(np.float16, (M, N))
    want = ref.matmul(X, W16, np.float64)
    worst = f16_close(got, want, ulps=1.0, atol=2e-5)
    print(f"matmul {M}x{N}x{K} q{bits}: worst/bound {worst:.3f} via {labels}")
    assert worst <= 1.0
    # the long-K cases must take the path they are listed for: the 4-way split where K / 64 divides by 4,
    # unsplit (no split suffix) where it does not
    if (M, N, K) in LONGK_SPLIT:
        assert len(labels) == 1 and labels[0].endswith("/k4"), labels
    if (M, N, K) in LONGK_UNSPLIT:
        assert len(labels) == 1 and "/k" not in labels[0].split("]")[-1], labels


LONGK_SPLIT = {(1024, 2048, 4096), (1152, 2560, 4352), (1024, 1536, 4608), (256, 1536, 4608)}
LONGK_UNSPLIT = {(1024, 2048, 4160), (256, 2048, 4160)}


@pytest.mark.parametrize("bits,direct", [(8, False), (4, False), (8, True), (4, True)])
def test_matmul_weights_bit_exact(pkg, ctx, bits, direct):
    """X = identity: Y = W16^T exactly (one nonzero product per output), so the in-register dequantization
    must give the reference's f16 weights bit for bit."""
    dj = _dj()
    rng = np.random.default_rng(11 + bits)
    N, K = 384, 256
    codes, scales = quant(rng, N, K, bits, std=0.5)
    X = np.eye(K, dtype=np.float16)
    W = ctx.weight_q(codes, scales, N, K, bits, dj.W_MFMA | (dj.W_DIRECT if direct else 0))
    dX, dY = ctx.array(X), ctx.alloc(K * N * 2)
    run(ctx, lambda r: r.matmul(dX, W, dY, K))
    got = dY.read(np.uint16, (K, N))
    assert np.array_equal(got, np.ascontiguousarray(ref.dequant_f16(codes, scales, bits).T).view(np.uint16))


@pytest.mark.parametrize("M,I,K,bits,act", [(384, 3072, 1024, 8, 0), (70, 1152, 768, 8, 1), (2200, 1024, 512, 4, 0), (19, 64, 128, 8, 1),
                                             (32, 4608, 1536, 8, 0), (1, 1024, 2048, 4, 0), (64, 1152, 768, 8, 1),
                                             (1500, 2624, 1024, 8, 2), (33, 96, 64, 8, 2), (1, 2624, 1024, 4, 2)])
@pytest.mark.parametrize("direct", [False, True])
def test_matmul_glu(pkg, ctx, M, I, K, bits, act, direct):
    dj = _dj()
    rng = np.random.default_rng(M + I + K + act)
    codes, scales = quant(rng, 2 * I, K, bits)
    W16 = ref.dequant_f16(codes, scales, bits)
    X = rand_f16(rng, (M, K), std=2.0)
    W = ctx.weight_q(codes, scales, 2 * I, K, bits, dj.W_MFMA_GLU | (dj.W_DIRECT if direct else 0))
    dX, dH = ctx.array(X), ctx.alloc(M * I * 2)
    run(ctx, lambda r: r.matmul_glu(dX, W, dH, M, act))
    got = dH.read(np.float16, (M, I))
    ab = ref.matmul(X, W16, np.float64)
    want = (ref.silu_mul, ref.gelu_mul, ref.gelu_erf_mul)[act](ab[:, :I], ab[:, I:], np.float64)
    # a and b are f16 matmul outputs and may each differ from the oracle's by one f16 ulp (their own
    # rounding); propagate that through act(a) * b, plus one ulp of the result
    a, b = ab[:, :I].astype(np.float64), ab[:, I:].astype(np.float64)
    act_fn = ((lambda x: x / (1 + np.exp(-x))), ref.gelu_tanh, (lambda x: 0.5 * x * (1 + ref.erf_as(x * 0.70710678))))[act]
    act_a = act_fn(a)
    hstep = np.maximum(np.abs(a) * 1e-4, 1e-6)
    dact = (act_fn(a + hstep) - act_fn(a - hstep)) / (2 * hstep)
    u = 2.0 ** -10
    bound = u * (np.abs(dact * a * b) + np.abs(act_a * b)) + u * np.abs(want.astype(np.float64)) + 1e-5
    worst = float((np.abs(got.astype(np.float64) - want.astype(np.float64)) / bound).max())
    print(f"matmul_glu {M}x{I}x{K} q{bits} act{act}: worst/bound {worst:.3f}")
    assert worst <= 1.0


@pytest.mark.parametrize("tile,K,glu", [("32x64p4", 128, False), ("32x64p4", 64, False), ("32x64p4", 1088, False),
                                         ("32x64p4", 192, False), ("128x256w8p4", 128, True), ("128x256w8p4", 1088, True),
                                         ("128x128np4", 256, False), ("128x128np4", 320, False),
                                         ("80x64k2p8", 1088, False), ("48x64k2", 2624, False), ("96x64k2", 192, True)])
def test_matmul_paired_ring_edges(pkg, ctx, monkeypatch, tile, K, glu):
    """Paired-ring tiles take 64-K steps two at a time: one pair only (K = 128), and odd step counts (3, 5, 17,
    41), whose last step is issued alone and computed after the pairs (on K wave set tiles by the first set),
    including a count whose last step is issued in the prologue (K = 192); a single step (K = 64) is below the
    paired tiles and the policy picks another. All match the oracle; the forced tile is the one that ran."""
    dj = _dj()
    monkeypatch.setenv("DJ_GEMM_TILE", tile)
    rng = np.random.default_rng(K)
    M, N = 300, 1024
    codes, scales = quant(rng, N, K, 8)
    W16 = ref.dequant_f16(codes, scales, 8)
    W = ctx.weight_q(codes, scales, N, K, 8, dj.W_MFMA_GLU if glu else dj.W_MFMA)
    X = rand_f16(rng, (M, K))
    dX, dY = ctx.array(X), ctx.alloc(M * N * 2)
    ctx.profile_reset()
    ctx.profile(True)
    try:
        if glu:
            run(ctx, lambda r: r.matmul_glu(dX, W, dY, M, 0))
        else:
            run(ctx, lambda r: r.matmul(dX, W, dY, M))
    finally:
        ctx.profile(False)
    labels = [name for name in ctx.profile_table() if name.startswith("matmul")]
    assert (K >= 128) == all(f"_{tile}[" in name for name in labels), labels
    if glu:
        ab = ref.matmul(X, W16, np.float64)
        want = ref.silu_mul(ab[:, :N // 2], ab[:, N // 2:], np.float64)
        got = dY.read(np.float16, (M, N // 2))
        assert np.abs(got.astype(np.float64) - want.astype(np.float64)).max() < 2e-2
    else:
        want = ref.matmul(X, W16, np.float64)
        assert f16_close(dY.read(np.float16, (M, N)), want, ulps=1.0, atol=2e-5) <= 1.0


@pytest.mark.parametrize("tile,splits,glu", [("128x128", 4, False), ("64x64", 2, False), ("128x128", 2, True),
                                              ("256x128", 1, False), ("32x128", 8, False), ("128x128n", 4, True),
                                              ("32x64", 2, False), ("64x128n", 8, False), ("144x128n", 1, False),
                                              ("144x64n", 2, False), ("96x128n", 1, True), ("48x128n", 4, True),
                                              ("32x64p4", 1, False), ("32x64p6", 1, False), ("128x128np4", 1, True),
                                              ("64x128np4", 1, False), ("144x64np4", 2, False), ("128x256w8p4", 1, True),
                                              ("128x256w8p4", 1, False)])
def test_matmul_forced_tiles_and_split_k(pkg, ctx, monkeypatch, tile, splits, glu):
    """Every tile shape and the split-K path (f32 partial slices in a workspace, summed in split order by a
    second kernel that runs the epilogue) agree with the oracle; run twice on fresh inputs so a stale slice
    would show."""
    dj = _dj()
    monkeypatch.setenv("DJ_GEMM_TILE", tile)
    monkeypatch.setenv("DJ_GEMM_SPLITK", str(splits))
    rng = np.random.default_rng(splits)
    M, N, K = 300, 1024, 2048
    codes, scales = quant(rng, N, K, 8)
    W16 = ref.dequant_f16(codes, scales, 8)
    W = ctx.weight_q(codes, scales, N, K, 8, dj.W_MFMA_GLU if glu else dj.W_MFMA)
    for rep in range(2):
        X = rand_f16(rng, (M, K))
        dX, dY = ctx.array(X), ctx.alloc(M * N * 2)
        if glu:
            run(ctx, lambda r: r.matmul_glu(dX, W, dY, M, 0))
            ab = ref.matmul(X, W16, np.float64)
            want = ref.silu_mul(ab[:, :N // 2], ab[:, N // 2:], np.float64)
            got = dY.read(np.float16, (M, N // 2))
            assert np.abs(got.astype(np.float64) - want.astype(np.float64)).max() < 2e-2
        else:
            run(ctx, lambda r: r.matmul(dX, W, dY, M))
            want = ref.matmul(X, W16, np.float64)
            assert f16_close(dY.read(np.float16, (M, N)), want, ulps=1.0, atol=2e-5) <= 1.0


@pytest.mark.parametrize("tile", ["48x64k2", "64x64k2", "80x64k2", "96x64k2", "64x128k2", "80x64k2p8", "96x64k2p8"])
@pytest.mark.parametrize("bits,glu,K", [(8, False, 2048), (8, False, 128), (4, False, 3072), (16, False, 1024),
                                        (8, True, 1024), (4, True, 256)])
def test_matmul_k_wave_sets(pkg, ctx, monkeypatch, tile, bits, glu, K):
    """Tiles whose waves also split K (two wave sets, each taking one step of every paired-ring pair; the
    partial tiles are added through LDS in set order): q8, q4 and direct f16 weights, one pair only (K = 128),
    ragged rows (300), the gated epilogue; each within the product's one-ulp bound of the oracle, and
    bit-identical on a second run."""
    dj = _dj()
    monkeypatch.setenv("DJ_GEMM_TILE", tile)
    rng = np.random.default_rng(K + bits + glu)
    M, N = 300, 1024
    qb = 8 if bits == 16 else bits
    codes, scales = quant(rng, N, K, qb)
    W16 = ref.dequant_f16(codes, scales, qb)
    layout = (dj.W_MFMA_GLU if glu else dj.W_MFMA) | (dj.W_DIRECT if bits == 16 else 0)
    W = ctx.weight_q(codes, scales, N, K, qb, layout)
    X = rand_f16(rng, (M, K))
    dX = ctx.array(X)
    outs = []
    ctx.profile_reset()
    ctx.profile(True)
    try:
        for _ in range(2):
            dY = ctx.alloc(M * N * 2)
            if glu:
                run(ctx, lambda r: r.matmul_glu(dX, W, dY, M, 0))
                outs.append(dY.read(np.uint16, (M, N // 2)))
            else:
                run(ctx, lambda r: r.matmul(dX, W, dY, M))
                outs.append(dY.read(np.uint16, (M, N)))
    finally:
        ctx.profile(False)
    labels = [name for name in ctx.profile_table() if name.startswith("matmul")]
    assert labels and all(f"_{tile}[" in name for name in labels), labels  # the forced tile is the one that ran
    assert np.array_equal(outs[0], outs[1])
    ab = ref.matmul(X, W16, np.float64)
    if glu:
        want = ref.silu_mul(ab[:, :N // 2], ab[:, N // 2:], np.float64)
        got = outs[0].view(np.float16)
        assert np.abs(got.astype(np.float64) - want.astype(np.float64)).max() < 2e-2
    else:
        assert f16_close(outs[0].view(np.float16), ab, ulps=1.0, atol=2e-5) <= 1.0


@pytest.mark.parametrize("M,N,K,want", [(1152, 1024, 2048, "80x64k2p8"), (1152, 1024, 3072, "80x64k2p8"),
                                         (1536, 2048, 2048, "96x64k2"), (2304, 1024, 2048, "96x64k2"),
                                         (1536, 1024, 2048, "96x64k2p8"), (1152, 1024, 2624, "80x64k2p8"),
                                         (1152, 2048, 1024, "32x64p4")])
def test_matmul_policy_k_wave_sets(pkg, ctx, M, N, K, want):
    """The tile policy's K wave set rule (256 CUs, K >= 2048): one round of the 8-stage tiles where that fills
    0.75-1 per CU (the ticket's o_proj / w2), else the 4-stage tile whose grid is nearest 1.5 per CU, an odd
    64-K step count (Laya's 2624) included; K = 1024 keeps the paired 32x64p4."""
    dj = _dj()
    cus = ctx.info()["compute_units"]
    if cus != 256:
        pytest.skip(f"the rule's tile counts assume 256 CUs (this device: {cus})")
    rng = np.random.default_rng(M + N + K)
    codes, scales = quant(rng, N, K, 8)
    W = ctx.weight_q(codes, scales, N, K, 8, dj.W_MFMA)
    X = rand_f16(rng, (M, K))
    dX, dY = ctx.array(X), ctx.alloc(M * N * 2)
    ctx.profile_reset()
    ctx.profile(True)
    try:
        run(ctx, lambda r: r.matmul(dX, W, dY, M))
    finally:
        ctx.profile(False)
    labels = [name for name in ctx.profile_table() if name.startswith("matmul")]
    assert labels == [f"matmul_q8_{want}[{M}x{N}x{K}]"], labels
    want_y = ref.matmul(X, ref.dequant_f16(codes, scales, 8), np.float64)
    assert f16_close(dY.read(np.float16, (M, N)), want_y, ulps=1.0, atol=2e-5) <= 1.0


@pytest.mark.parametrize("M,H,K2,bits", [(1152, 1024, 2048, 8), (300, 1024, 3072, 8), (1536, 2048, 2048, 4), (40, 1024, 2048, 8),
                                        (1152, 1024, 1024, 8), (200, 768, 1536, 8)])
def test_matmul_residual_and_normed(pkg, ctx, M, H, K2, bits):
    """The residual add + RMSNorm folded into the products: dj_matmul_residual (R += f16(X W^T) in place, XW = f16(R w
    / 4), per-32-column sums of squares of the unrounded sums) and its consumers dj_matmul_normed (plain and gated)
    and dj_matmul_qkv_rope_normed against the separate ADD_RMSNORM of the oracle followed by the product: the new
    stream within one f16 rounding of the product's, XW bit-exact from it, the sums within 1e-5 relative, the
    consumers within 4-16 f16 ulps + 3e-3 of the unfused form (the norm's 1 / rms lands after the product's sum
    instead of before the input's f16 rounding, which moves the outputs by ~2.5e-4 rms); M = 40 takes the skinny
    rows' kernels."""
    dj = _dj()
    rng = np.random.default_rng(M + H + K2)
    eps = 1e-6
    cX, sX = quant(rng, H, K2, bits)  # the producer: o_proj / w2, K2 -> H
    W1 = ctx.weight_q(cX, sX, H, K2, bits, dj.W_MFMA)
    X = rand_f16(rng, (M, K2))
    R = rand_f16(rng, (M, H), std=0.5)
    nw = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    dX, dR, dnw = ctx.array(X), ctx.array(R), ctx.array(nw)
    dXW, dSS = ctx.alloc(M * H * 2), ctx.alloc(M * (H // 32) * 4)
    run(ctx, lambda r: r.matmul_residual(dX, W1, M, dR, dnw, dXW, dSS))
    Rn, XW, SS = dR.read(np.float16, (M, H)), dXW.read(np.float16, (M, H)), dSS.read(np.float32, (M, H // 32))
    y = ref.matmul(X, ref.dequant_f16(cX, sX, bits), np.float64)
    v = R.astype(np.float64) + y.astype(np.float64)
    ulp_y = np.spacing(np.abs(y).astype(np.float16)).astype(np.float64)
    assert (np.abs(Rn.astype(np.float64) - v) <= np.spacing(np.abs(v).astype(np.float16)).astype(np.float64) + ulp_y).all()
    want_xw = (Rn.astype(np.float32) * nw.astype(np.float32) * np.float32(0.25)).astype(np.float16)
    assert np.array_equal(XW.view(np.uint16), want_xw.view(np.uint16))
    ss_want = (v * v).reshape(M, H // 32, 32).sum(-1)
    assert np.abs(SS - ss_want).max() <= 1e-5 * ss_want.max() + 2 * (np.abs(v) * ulp_y).reshape(M, H // 32, 32).sum(-1).max()
    # the consumers against the unfused form on the same stream: O = f16(R_new inv w), then the product
    inv = 1.0 / np.sqrt(SS.astype(np.float64).sum(-1, keepdims=True) / H + eps)
    normed = (Rn.astype(np.float64) * inv * nw.astype(np.float64)).astype(np.float16)
    N2 = 1536
    c2, s2 = quant(rng, N2, H, bits)
    W16 = ref.dequant_f16(c2, s2, bits)
    W2, dY = ctx.weight_q(c2, s2, N2, H, bits, dj.W_MFMA), ctx.alloc(M * N2 * 2)
    run(ctx, lambda r: r.matmul_normed(dXW, W2, dY, M, -1, dSS, H, eps))
    # the A roundings differ by up to an f16 ulp per element: about 2.5e-4 rms on these 0.9-sized outputs
    assert f16_close(dY.read(np.float16, (M, N2)), ref.matmul(normed, W16, np.float64), ulps=4.0, atol=3e-3) <= 1.0
    W3, dG = ctx.weight_q(c2, s2, N2, H, bits, dj.W_MFMA_GLU), ctx.alloc(M * N2 // 2 * 2)
    run(ctx, lambda r: r.matmul_normed(dXW, W3, dG, M, dj.ACT_SILU, dSS, H, eps))
    ab = ref.matmul(normed, W16, np.float64)
    want_g = ref.silu_mul(ab[:, :N2 // 2], ab[:, N2 // 2:], np.float64)
    assert f16_close(dG.read(np.float16, (M, N2 // 2)), want_g, ulps=6.0, atol=3e-3) <= 1.0
    # qkv + RoPE on the normalized rows against the same op on the unfused rows (both on the GPU)
    heads, kv, D = H // 128, max(1, H // 512), 128
    N3 = (heads + 2 * kv) * D
    c3, s3 = quant(rng, N3, H, bits)
    W4 = ctx.weight_q(c3, s3, N3, H, bits, dj.W_MFMA)
    pos = ctx.array((np.arange(M) % 384).astype(np.int32))
    qn, kn = ctx.array(nw[:D].copy()), ctx.array(nw[D:2 * D].copy())
    tab, dZa, dZb, dN = ctx.alloc(M * 64 * 8), ctx.alloc(M * N3 * 2), ctx.alloc(M * N3 * 2), ctx.array(normed)

    def both(r):
        r.rope_table(M, pos, 1, 1e6, D, tab)
        r.matmul_qkv_rope(dN, W4, dZa, M, heads, kv, D, qn, kn, False, pos, 1, eps, 1e6, tab)
        r.matmul_qkv_rope_normed(dXW, W4, dZb, M, heads, kv, D, qn, kn, False, pos, 1, eps, 1e6, tab, dSS, H, eps)
    run(ctx, both)
    za, zb = dZa.read(np.float16, (M, N3)), dZb.read(np.float16, (M, N3))
    assert f16_close(zb, za, ulps=16.0, atol=4e-3) <= 1.0  # the q/k norm rescales the two roundings apart


@pytest.mark.parametrize("tile", ["80x64k2p8", "96x64k2p8", "48x64k2", "80x64k2"])
def test_matmul_normed_on_k_wave_sets(pkg, ctx, monkeypatch, tile):
    """The row norm on K wave set tiles (both sets share the epilogue, so the row scales' barrier sees every
    wave): dj_matmul_normed forced onto each such tile, and dj_matmul_residual on the same tile, against the
    oracle's ADD_RMSNORM then product, at the bounds of the untiled-K form."""
    dj = _dj()
    M, H, K2, N2, bits, eps = 1152, 1024, 2048, 1024, 8, 1e-6
    rng = np.random.default_rng(77)
    cX, sX = quant(rng, H, K2, bits)
    W1 = ctx.weight_q(cX, sX, H, K2, bits, dj.W_MFMA)
    X, R = rand_f16(rng, (M, K2)), rand_f16(rng, (M, H), std=0.5)
    nw = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    dX, dR, dnw = ctx.array(X), ctx.array(R), ctx.array(nw)
    dXW, dSS = ctx.alloc(M * H * 2), ctx.alloc(M * (H // 32) * 4)
    c2, s2 = quant(rng, N2, H, bits)
    W2, dY = ctx.weight_q(c2, s2, N2, H, bits, dj.W_MFMA), ctx.alloc(M * N2 * 2)
    monkeypatch.setenv("DJ_GEMM_TILE", tile)
    ctx.profile_reset()
    ctx.profile(True)
    try:
        run(ctx, lambda r: (r.matmul_residual(dX, W1, M, dR, dnw, dXW, dSS),
                            r.matmul_normed(dXW, W2, dY, M, -1, dSS, H, eps)))
    finally:
        ctx.profile(False)
    labels = [k for k in ctx.profile_table() if k.startswith("matmul")]
    assert labels and all(f"_{tile}[" in k for k in labels), labels
    Rn, SS = dR.read(np.float16, (M, H)), dSS.read(np.float32, (M, H // 32))
    v = R.astype(np.float64) + ref.matmul(X, ref.dequant_f16(cX, sX, bits), np.float64).astype(np.float64)
    assert np.abs(Rn.astype(np.float64) - v).max() <= 2 * np.spacing(np.abs(v).astype(np.float16)).max()
    inv = 1.0 / np.sqrt(SS.astype(np.float64).sum(-1, keepdims=True) / H + eps)
    normed = (Rn.astype(np.float64) * inv * nw.astype(np.float64)).astype(np.float16)
    want = ref.matmul(normed, ref.dequant_f16(c2, s2, bits), np.float64)
    assert f16_close(dY.read(np.float16, (M, N2)), want, ulps=4.0, atol=3e-3) <= 1.0


@pytest.mark.parametrize("waves", [1, 5, 8, 9, 16])
@pytest.mark.parametrize("M,N,K,bits,glu", [(1, 2048, 832, 8, False), (32, 1536, 4608, 8, False),
                                            (64, 512, 1024, 4, False), (17, 1024, 1536, 8, True),
                                            (5, 2048, 1536, 16, False), (16, 1024, 2048, 16, True)])
def test_gemv_wave_counts(pkg, ctx, monkeypatch, waves, M, N, K, bits, glu):
    """The skinny kernel at forced wave counts: 1-8 run the 8-wave form (batches of up to 12 K-steps, loads
    past the end skipped), 9-16 the 16-wave form (small batches, the last step re-loaded); K = 832 is 13 steps,
    which no count above 1 divides. Each matches the oracle to the product's one-ulp bound. bits 16: q8 weights
    loaded as direct f16 blocks (the 16-bit kernel)."""
    dj = _dj()
    monkeypatch.setenv("DJ_GEMV_WAVES", str(waves))
    rng = np.random.default_rng(waves * 31 + M + K)
    direct = bits == 16
    bits = 8 if direct else bits
    codes, scales = quant(rng, N, K, bits)
    W16 = ref.dequant_f16(codes, scales, bits)
    W = ctx.weight_q(codes, scales, N, K, bits, (dj.W_MFMA_GLU if glu else dj.W_MFMA) | (dj.W_DIRECT if direct else 0))
    X = rand_f16(rng, (M, K))
    dX, dY = ctx.array(X), ctx.alloc(M * N * 2)
    ab = ref.matmul(X, W16, np.float64)
    if glu:
        run(ctx, lambda r: r.matmul_glu(dX, W, dY, M, 0))
        want = ref.silu_mul(ab[:, :N // 2], ab[:, N // 2:], np.float64)
        assert np.abs(dY.read(np.float16, (M, N // 2)).astype(np.float64) - want.astype(np.float64)).max() < 2e-2
    else:
        run(ctx, lambda r: r.matmul(dX, W, dY, M))
        assert f16_close(dY.read(np.float16, (M, N)), ab, ulps=1.0, atol=2e-5) <= 1.0


def _held_case(ctx, rng, M, N, K, bits, direct):
    dj = _dj()
    codes, scales = quant(rng, N, K, bits)
    W16 = ref.dequant_f16(codes, scales, bits)
    W = ctx.weight_q(codes, scales, N, K, bits, dj.W_MFMA | (dj.W_DIRECT if direct else 0))
    X, Xr = rand_f16(rng, (M, K)), rand_f16(rng, (M, N))
    w = (1 + rng.standard_normal(N) * 0.1).astype(np.float16)
    return W, W16, X, Xr, w


@pytest.mark.parametrize("M,N,K,bits,direct", [(32, 1536, 4608, 8, False), (32, 1536, 1536, 8, False),
                                               (16, 1024, 2048, 4, False), (5, 2048, 1536, 8, False),
                                               (16, 2048, 1536, 8, False), (64, 512, 1024, 8, False),
                                               (5, 2048, 1536, 8, True), (32, 1536, 4608, 8, True)])
@pytest.mark.parametrize("split", [None, "0", "3", "4"])
def test_held_product_into_norm(pkg, ctx, monkeypatch, M, N, K, bits, direct, split):
    """matmul followed by the residual + RMSNorm of its output: on skinny rows the recorder holds the product
    and runs it split along K with the norm summing the f32 partials (split None: automatic, two; "0": holding
    off; "3", "4": forced where they divide the K steps). Either way the product buffer holds the product (one f16 ulp of float64), and x and the normed rows
    are the oracle's add_rmsnorm of that product: x bit-exact, the normed rows within one ulp. Direct (f16)
    weights at M = 5 have the largest load batch of the skinny kernel, whose slots are mostly empty here."""
    if split is not None:
        monkeypatch.setenv("DJ_GEMV_SPLIT", split)
    rng = np.random.default_rng(M * 13 + N + K + bits)
    W, W16, X, Xr, w = _held_case(ctx, rng, M, N, K, bits, direct)
    dX, dY, dx, dw, dO = ctx.array(X), ctx.alloc(M * N * 2), ctx.array(Xr), ctx.array(w), ctx.alloc(M * N * 2)

    def body(r):
        r.matmul(dX, W, dY, M)
        r.add_rmsnorm(M, N, True, 1e-6, dx, dY, dw, dO)

    for rep in range(2):  # twice: the second call reuses the workspace slices
        dx.upload(Xr)
        run(ctx, body)
        Y = dY.read(np.float16, (M, N))
        assert f16_close(Y, ref.matmul(X, W16, np.float64), ulps=1.0, atol=2e-5) <= 1.0
        xn, O = ref.add_rmsnorm(Xr, Y, w, 1e-6, add=True, acc=np.float64)
        assert np.array_equal(dx.read(np.float16, (M, N)).view(np.uint16), xn.view(np.uint16))
        assert f16_close(dO.read(np.float16, (M, N)), O, ulps=1.0) <= 1.0


@pytest.mark.parametrize("after", ["finish", "snapshot", "matmul", "other_norm", "copy"])
def test_held_product_released_in_order(pkg, ctx, after):
    """A held product that the next op does not consume runs first, in issue order: before another op,
    a snapshot of its output, the end of the forward, a norm of another buffer, or a buffer copy."""
    rng = np.random.default_rng(7)
    M, N, K = 32, 1536, 4608
    W, W16, X, Xr, w = _held_case(ctx, rng, M, N, K, 8, False)
    want = ref.matmul(X, W16, np.float64)
    dX, dY, dY2, dx, dw, dO = (ctx.array(X), ctx.alloc(M * N * 2), ctx.alloc(M * N * 2), ctx.array(Xr), ctx.array(w),
                               ctx.alloc(M * N * 2))
    dZ = ctx.alloc(M * N * 2)
    rec = ctx.recorder()
    rec.matmul(dX, W, dY, M)
    snap = None
    if after == "snapshot":
        snap = rec.snapshot(dY, M * N * 2, np.float16, (M, N))
    elif after == "matmul":  # a product reading the held one's output
        rec.matmul(dY, ctx.weight_q(*quant(rng, N, N, 8), N, N, 8, _dj().W_MFMA), dY2, M)
    elif after == "other_norm":
        rec.add_rmsnorm(M, N, True, 1e-6, dx, dZ, dw, dO)
    elif after == "copy":
        dY2.copy_from(dY)
    got = rec.finish()
    Y = got[snap] if snap is not None else dY.read(np.float16, (M, N))
    assert f16_close(Y, want, ulps=1.0, atol=2e-5) <= 1.0
    if after == "copy":
        assert np.array_equal(dY2.read(np.float16, (M, N)).view(np.uint16), Y.view(np.uint16))


def test_held_product_graph_replays(pkg, ctx):
    """The held product and its norm captured in a HIP graph: every replay (with eager work and reads in
    between) gives the bits of the eager run."""
    rng = np.random.default_rng(11)
    M, N, K = 32, 1536, 4608
    W, W16, X, Xr, w = _held_case(ctx, rng, M, N, K, 8, False)
    dX, dY, dx, dw, dO = ctx.array(X), ctx.alloc(M * N * 2), ctx.array(Xr), ctx.array(w), ctx.alloc(M * N * 2)

    def body(r):
        r.matmul(dX, W, dY, M)
        r.add_rmsnorm(M, N, True, 1e-6, dx, dY, dw, dO)

    dx.upload(Xr)
    run(ctx, body)
    eager = [b.read(np.float16, (M, N)).view(np.uint16).copy() for b in (dY, dx, dO)]
    for rep in range(4):
        dx.upload(Xr)
        dY.upload(np.zeros((M, N), np.float16))
        dO.upload(np.zeros((M, N), np.float16))
        rec = ctx.recorder(0x4E1D0)
        if not rec.replay:
            body(rec)
        rec.finish()
        for b, e in zip((dY, dx, dO), eager):
            assert np.array_equal(b.read(np.float16, (M, N)).view(np.uint16), e), f"replay {rep}"
        run(ctx, lambda r: r.add_rmsnorm(M, N, False, 1e-6, dx, None, dw, dO))  # eager work between replays
    ctx.graph_clear()  # the cached graph points at this test's buffers


# ---------------------------------------------------------------- q/k norm + rope

@pytest.mark.parametrize("heads,kv,D,qk,vnorm,mode,rot", [
    (16, 8, 128, True, False, 0, None), (16, 2, 128, False, False, 0, None), (12, 2, 128, True, False, 0, None),
    (3, 1, 256, True, True, 1, None), (8, 2, 256, True, False, 0, 64), (4, 4, 64, True, False, 0, None),
    (6, 2, 128, True, False, 1, 96), (5, 5, 512, False, True, 0, 256),
])
def test_qk_norm_rope(pkg, ctx, heads, kv, D, qk, vnorm, mode, rot):
    rng = np.random.default_rng(heads * D + kv)
    T = 97
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride))
    pos = rng.integers(0, 1100, T).astype(np.int32)
    pos[:4] = [0, 1, 65535, 131071]  # the position range of a full tokens-per-pass budget
    qn, kn = (1 + rng.standard_normal(D) * 0.1).astype(np.float16), (1 + rng.standard_normal(D) * 0.1).astype(np.float16)
    dZ, dpos, dq, dk = ctx.array(Z), ctx.array(pos), ctx.array(qn), ctx.array(kn)
    theta = 1e6 if mode == 0 else 1e4
    run(ctx, lambda r: r.qk_norm_rope(T, heads, kv, D, stride, dZ, dq if qk else None, dk if qk else None, vnorm, dpos, 1,
                                      1e-6, theta, rot, mode))
    want = ref.qk_norm_rope(Z, heads, kv, D, pos, qn if qk else None, kn if qk else None, vnorm, 1e-6, theta, rot, mode, np.float64)
    got = dZ.read(np.float16, (T, stride))
    worst = f16_close(got[4:], want[4:], ulps=2.0, atol=2e-4)
    print(f"qk_norm_rope h{heads} kv{kv} D{D}: worst/bound {worst:.3f}")
    assert worst <= 1.0
    assert f16_close(got[:2], want[:2], ulps=2.0, atol=2e-4) <= 1.0
    # at positions near 2^17 one ulp of an f32 frequency moves the f32 angle by pos * 2^-24 rad, so any two
    # correct implementations (this kernel, the oracle, the reference's pow) differ by |x| * that much
    r = D if rot is None else rot
    big = np.abs(got[2:4].astype(np.float64) - want[2:4])
    assert big.max() <= 8 * 131071 * 2.0 ** -24 * max(1.0, np.abs(want[2:4]).max()) + 4e-3
    # rotation keeps each pair's length: |(x, y)| before and after RoPE agree for the q and k heads
    g = got[2:4, :(heads + kv) * D].astype(np.float64).reshape(2, heads + kv, D)
    w = want[2:4, :(heads + kv) * D].reshape(2, heads + kv, D)
    ln = lambda a: np.hypot(a[..., :r // 2], a[..., r // 2:r])
    assert np.abs(ln(g) - ln(w)).max() <= 4e-3 * max(1.0, ln(w).max())


@pytest.mark.parametrize("M,heads,kv,D,qk,vnorm,rot,bits", [
    (300, 16, 8, 128, True, False, 128, 8),    # fused: one head per tile (144 / 128 / 64-row tiles)
    (1152, 16, 8, 128, True, False, 128, 8),   # the bench's qkv shape
    (8192, 16, 8, 128, True, False, 128, 8),   # more than two tiles per CU: the product, then the standalone kernel
    (1536, 16, 2, 128, True, False, 128, 4),   # q4, GQA 8:1
    (300, 12, 2, 128, False, True, 64, 8),     # partial rotation (16 lanes a row), no q/k weights, v norm
    (200, 6, 2, 128, True, False, 96, 8),
    (40, 16, 8, 128, True, False, 128, 8),     # skinny M: the product and the standalone kernel
    (300, 8, 4, 64, True, False, 64, 8),       # D 64: no 128-wide head tile, two kernels
])
def test_matmul_qkv_rope_matches_two_ops(pkg, ctx, monkeypatch, M, heads, kv, D, qk, vnorm, rot, bits):
    """dj_matmul_qkv_rope (the forward's RoPE table, norm + rotation in the product's epilogue where it fits)
    gives the same bits as dj_matmul followed by dj_qk_norm_rope (which computes its own angles), the plain
    product on a tile that sums K in step order (64x64: the K wave set tiles add two partial sums, a different
    rounding; the RoPE tile ignores the forced plain tile); and the table itself is the angles' cos and sin."""
    monkeypatch.setenv("DJ_GEMM_TILE", "64x64")
    dj = _dj()
    rng = np.random.default_rng(M + heads + D + rot)
    K = 1024
    N = (heads + 2 * kv) * D
    codes, scales = quant(rng, N, K, bits)
    W = ctx.weight_q(codes, scales, N, K, bits, dj.W_MFMA)
    X = rand_f16(rng, (M, K))
    pos = rng.integers(0, 3000, M).astype(np.int32)
    qn, kn = (1 + rng.standard_normal(D) * 0.1).astype(np.float16), (1 + rng.standard_normal(D) * 0.1).astype(np.float16)
    dX, dpos, dq, dk = ctx.array(X), ctx.array(pos), ctx.array(qn), ctx.array(kn)
    dZ1, dZ2, dtab = ctx.alloc(M * N * 2), ctx.alloc(M * N * 2), ctx.alloc(M * (rot // 2) * 8)
    theta, eps = 1e6, 1e-6

    def two(r):
        r.matmul(dX, W, dZ1, M)
        r.qk_norm_rope(M, heads, kv, D, N, dZ1, dq if qk else None, dk if qk else None, vnorm, dpos, 1, eps, theta, rot)

    def fused(r):
        r.rope_table(M, dpos, 1, theta, rot, dtab)
        r.matmul_qkv_rope(dX, W, dZ2, M, heads, kv, D, dq if qk else None, dk if qk else None, vnorm, dpos, 1, eps, theta,
                          dtab, rot)
    run(ctx, two)
    run(ctx, fused)
    a, b = dZ1.read(np.uint16, (M, N)), dZ2.read(np.uint16, (M, N))
    assert np.array_equal(a, b), f"{int((a != b).sum())} of {a.size} halves differ"
    tab = dtab.read(np.float32, (M, rot // 2, 2)).astype(np.float64)
    ang = pos[:, None].astype(np.float64) * ref.inv_freq(theta, rot, 0)[None, :]
    assert np.abs(tab[..., 0] - np.cos(ang)).max() < 2e-3 and np.abs(tab[..., 1] - np.sin(ang)).max() < 2e-3
    # and the fused result against the oracle (the product rounded to f16, then the op)
    want = ref.qk_norm_rope(ref.matmul(X, ref.dequant_f16(codes, scales, bits), np.float64), heads, kv, D, pos,
                            qn if qk else None, kn if qk else None, vnorm, eps, theta, rot, 0, np.float64)
    assert f16_close(b.view(np.float16), want, ulps=4.0, atol=2e-3) <= 1.0


# ---------------------------------------------------------------- attention

def _forest_case(rng, trunks_branches):
    trees = []
    for trunk, branches in trunks_branches:
        trees.append({"trunk": list(rng.integers(0, 1000, trunk)), "branches": [list(rng.integers(0, 1000, b)) for b in branches],
                      "groups": [[[1], [2]] for _ in branches]})
    ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest(trees)
    return meta, ref.forest_ranges(meta)


ATTN_FORMS = {"default": {}, "kg2": {"DJ_ATTN_KG": "2"}, "hg1": {"DJ_ATTN_HG": "1"}, "hg2": {"DJ_ATTN_HG": "2"},
              "hg4": {"DJ_ATTN_HG": "4"}}


@pytest.mark.parametrize("form", list(ATTN_FORMS))
@pytest.mark.parametrize("heads,kv,D", [(16, 8, 128), (16, 2, 128), (12, 2, 128), (3, 1, 256), (4, 2, 64), (8, 2, 256)])
def test_attention_forest(pkg, ctx, monkeypatch, heads, kv, D, form):
    """The forest mask through every workgroup form: one head and one key group (4 waves), two key groups (8
    waves, each scoring half of every key tile, merged through LDS), and head groups of 2 or 4 query heads
    sharing a KV head (8 or 16 waves staging each K/V tile once); a form that does not apply falls back."""
    for k, v in ATTN_FORMS[form].items():
        monkeypatch.setenv(k, v)
    dj = _dj()
    rng = np.random.default_rng(heads + kv + D)
    meta, rng4 = _forest_case(rng, [(100, [20, 37, 5]), (70, [64, 1]), (0, [90]), (130, [])])
    T = meta.shape[0]
    mask = ref.forest_mask(meta)
    assert np.array_equal(ref.ranges_mask(rng4, T), mask)
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride))
    dZ, drng, dO = ctx.array(Z), ctx.array(rng4), ctx.alloc(T * heads * D * 2)
    src = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    scale = 1.0 / math.sqrt(D)
    run(ctx, lambda r: r.attention(T, heads, kv, D, dZ, stride, src, src, drng, scale, dO))
    got = dO.read(np.float16, (T, heads * D)).astype(np.float64)
    want = ref.attention(Z, heads, kv, D, mask, scale, np.float64).astype(np.float64)
    err = np.abs(got - want).max()
    print(f"attention h{heads} kv{kv} D{D} T{T}: max abs err {err:.2e}")
    assert err < 4e-3


@pytest.mark.parametrize("form", list(ATTN_FORMS))
def test_attention_large_grid(pkg, ctx, monkeypatch, form):
    """A varlen batch of causal sequences large enough (>= 512 workgroups) for the two-stage K/V ring, and
    long enough that the lazy max-rescaling and the unmasked-tile path both run many times."""
    for k, v in ATTN_FORMS[form].items():
        monkeypatch.setenv(k, v)
    dj = _dj()
    rng = np.random.default_rng(41)
    heads, kv, D = 16, 8, 128
    meta, rng4 = _forest_case(rng, [(300, []), (450, []), (128, []), (700, []), (512, []), (300, [])])
    T = meta.shape[0]
    assert (T + 63) // 64 * heads >= 512
    mask = ref.forest_mask(meta)
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride), std=1.5)  # sharper softmax: the running max moves often
    dZ, drng, dO = ctx.array(Z), ctx.array(rng4), ctx.alloc(T * heads * D * 2)
    src = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    scale = 1.0 / math.sqrt(D)
    run(ctx, lambda r: r.attention(T, heads, kv, D, dZ, stride, src, src, drng, scale, dO))
    got = dO.read(np.float16, (T, heads * D)).astype(np.float64)
    want = ref.attention(Z, heads, kv, D, mask, scale, np.float64).astype(np.float64)
    err = np.abs(got - want).max()
    print(f"attention large grid T{T}: max abs err {err:.2e}")
    assert err < 4e-3


@pytest.mark.parametrize("D", [128, 256])
def test_attention_bidirectional_and_windows(pkg, ctx, D):
    dj = _dj()
    rng = np.random.default_rng(D)
    heads, kv = 3, 1
    seqs = [list(range(n)) for n in (256, 24, 24, 24, 8, 8, 8, 8, 8, 8, 8, 300)]
    ids, meta, full, slide, ranges = ref.pack_encoder(seqs, window=40)
    T = len(ids)
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride), std=0.5)
    dZ, dO = ctx.array(Z), ctx.alloc(T * heads * D * 2)
    src = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    for r4 in (full, slide):
        drng = ctx.array(r4)
        run(ctx, lambda r: r.attention(T, heads, kv, D, dZ, stride, src, src, drng, 1.0, dO))
        got = dO.read(np.float16, (T, heads * D)).astype(np.float64)
        want = ref.attention(Z, heads, kv, D, ref.ranges_mask(r4, T), 1.0, np.float64).astype(np.float64)
        assert np.abs(got - want).max() < 4e-3


@pytest.mark.parametrize("P,splits,hg", [(300, None, None), (1100, None, None), (300, 4, None), (1100, 16, None),
                                         (1100, 1, None), (1100, 4, 2), (1100, 1, 2), (300, None, 1)])
def test_attention_kept_prefix(pkg, ctx, monkeypatch, P, splits, hg):
    """Source A = a kept K/V cache (the shared state), source B = the current rows: same result as one pass.
    A 1100-row cache is split over workgroups by default (partials merged by k_attn_combine); the split count
    is also forced (4, 16) and turned off (1), alone and with head groups of 2 forced (or off)."""
    if splits is not None:
        monkeypatch.setenv("DJ_ATTN_SPLITS", str(splits))
    if hg is not None:
        monkeypatch.setenv("DJ_ATTN_HG", str(hg))
    dj = _dj()
    rng = np.random.default_rng(5 + P)
    heads, kv, D = 12, 2, 128
    branches = [32, 32, 17, 32]
    stride = (heads + 2 * kv) * D
    T = sum(branches)
    Zp = rand_f16(rng, (P, stride))
    Zb = rand_f16(rng, (T, stride))
    cache = np.ascontiguousarray(Zp[:, heads * D:(heads + 2 * kv) * D])
    rng4 = []
    s = 0
    for b in branches:
        for o in range(b):
            rng4.append((0, P, s, s + o + 1))
        s += b
    rng4 = np.array(rng4, dtype=np.int32)
    dZ, dC, drng, dO = ctx.array(Zb), ctx.array(cache), ctx.array(rng4), ctx.alloc(T * heads * D * 2)
    A = dj.kv_src(dC, P, 2 * kv * D, 0, kv * D)
    B = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    run(ctx, lambda r: r.attention(T, heads, kv, D, dZ, stride, A, B, drng, 1 / math.sqrt(D), dO))
    got = dO.read(np.float16, (T, heads * D)).astype(np.float64)
    kvrows = np.concatenate([cache, Zb[:, heads * D:(heads + 2 * kv) * D]])
    mask = np.zeros((T, P + T), dtype=bool)
    for t, (a0, a1, b0, b1) in enumerate(rng4):
        mask[t, a0:a1] = True
        mask[t, P + b0:P + b1] = True
    want = ref.attention(Zb, heads, kv, D, mask, 1 / math.sqrt(D), np.float64, kv_rows=kvrows).astype(np.float64)
    assert np.abs(got - want).max() < 4e-3


@pytest.mark.parametrize("T,P,qk,splits", [(32, 1056, True, None), (32, 1056, False, None), (17, 300, True, None),
                                           (64, 1100, True, 4), (64, 1100, True, 1), (1, 700, True, None)])
def test_attention_qk_rope_equals_norm_then_attention(pkg, ctx, monkeypatch, T, P, qk, splits):
    """dj_attention_qk_rope on raw q/k rows against a kept state == dj_qk_norm_rope on the rows then
    dj_attention, bit for bit (the same arithmetic in the same order, the row sums added in the standalone
    kernel's lane order), with and without norm weights, split over workgroups by default, forced to 4 and off;
    the rows keep their raw values. The result is also the oracle's attention of the oracle-normalized rows."""
    if splits is not None:
        monkeypatch.setenv("DJ_ATTN_SPLITS", str(splits))
    dj = _dj()
    rng = np.random.default_rng(T * 7 + P)
    heads, kv, D, theta = 12, 2, 128, 1e6
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride))
    cache = rand_f16(rng, (P, 2 * kv * D))  # a kept state's rotated K / V rows (any values)
    pos = (P + np.arange(T)).astype(np.int32)
    qn, kn = (1 + rng.standard_normal(D) * 0.1).astype(np.float16), (1 + rng.standard_normal(D) * 0.1).astype(np.float16)
    rng4 = np.array([(0, P, 0, t + 1) for t in range(T)], dtype=np.int32)  # the whole state, causal question
    dZ, dZ2, dC, drng, dpos = ctx.array(Z), ctx.array(Z), ctx.array(cache), ctx.array(rng4), ctx.array(pos)
    dq, dk = (ctx.array(qn), ctx.array(kn)) if qk else (None, None)
    dtab, dO1, dO2 = ctx.alloc(T * (D // 2) * 8), ctx.alloc(T * heads * D * 2), ctx.alloc(T * heads * D * 2)
    A = dj.kv_src(dC, P, 2 * kv * D, 0, kv * D)
    B1 = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    B2 = dj.kv_src(dZ2, T, stride, heads * D, (heads + kv) * D)
    scale = 1 / math.sqrt(D)

    def fused(r):
        r.rope_table(T, dpos, 1, theta, D, dtab)
        r.attention_qk_rope(T, heads, kv, D, dZ, stride, A, B1, drng, scale, dq, dk, 1e-6, dtab, dO1)

    def separate(r):
        r.qk_norm_rope(T, heads, kv, D, stride, dZ2, dq, dk, False, dpos, 1, 1e-6, theta)
        r.attention(T, heads, kv, D, dZ2, stride, A, B2, drng, scale, dO2)

    run(ctx, fused)
    run(ctx, separate)
    got, want = dO1.read(np.float16, (T, heads * D)), dO2.read(np.float16, (T, heads * D))
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64)).max()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), f"max |fused - separate| {diff:.3e}"
    assert np.array_equal(dZ.read(np.float16, (T, stride)).view(np.uint16), Z.view(np.uint16))  # rows kept raw
    Zn = ref.qk_norm_rope(Z, heads, kv, D, pos, qn if qk else None, kn if qk else None, False, 1e-6, theta, None, 0,
                          np.float64)
    kvrows = np.concatenate([cache, Zn[:, heads * D:(heads + 2 * kv) * D].astype(np.float16)])
    mask = np.zeros((T, P + T), dtype=bool)
    for t, (a0, a1, b0, b1) in enumerate(rng4):
        mask[t, a0:a1] = True
        mask[t, P + b0:P + b1] = True
    oracle = ref.attention(Zn.astype(np.float16), heads, kv, D, mask, scale, np.float64, kv_rows=kvrows)
    assert np.abs(got.astype(np.float64) - oracle).max() < 4e-3


def test_attention_qk_rope_refuses_other_shapes(pkg, ctx):
    """The folded form is 128-dim heads fully rotated, with source B the query rows: other shapes are refused
    before anything is launched."""
    dj = _dj()
    heads, kv, T = 4, 2, 8
    for D, rot, brows, msg in ((64, 64, T, "head dim"), (128, 64, T, "head dim"), (128, 128, T + 1, "source B")):
        stride = (heads + 2 * kv) * D
        dZ, dO, dtab = ctx.alloc((T + 1) * stride * 2), ctx.alloc(T * heads * D * 2), ctx.alloc(T * D * 8)
        drng = ctx.array(np.array([(0, 0, 0, t + 1) for t in range(T)], dtype=np.int32))
        src = dj.kv_src(dZ, brows, stride, heads * D, (heads + kv) * D)
        rec = ctx.recorder()
        try:
            with pytest.raises(dj.DJError, match=msg):
                rec.attention_qk_rope(T, heads, kv, D, dZ, stride, src, src, drng, 0.1, None, None, 1e-6, dtab, dO, rot=rot)
        finally:
            rec.finish()


def test_attention_rejects_nonpositive_scale(pkg, ctx):
    """The kernel takes the row max on raw scores (it commutes with a positive scale): a scale <= 0 is refused
    before anything is launched."""
    dj = _dj()
    heads, kv, D, T = 4, 2, 128, 8
    stride = (heads + 2 * kv) * D
    dZ, dO = ctx.alloc(T * stride * 2), ctx.alloc(T * heads * D * 2)
    drng = ctx.array(np.array([(0, t + 1, 0, 0) for t in range(T)], dtype=np.int32))
    src = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    for bad in (0.0, -0.5):
        rec = ctx.recorder()
        try:
            with pytest.raises(dj.DJError, match="score scale must be positive"):
                rec.attention(T, heads, kv, D, dZ, stride, src, src, drng, bad, dO)
        finally:
            rec.finish()  # the refused op launched nothing; the (empty) forward completes


def test_kv_store(pkg, ctx):
    rng = np.random.default_rng(3)
    heads, kv, D, T = 4, 2, 128, 70
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride))
    dZ, dC = ctx.array(Z), ctx.alloc((T + 10) * 2 * kv * D * 2)
    run(ctx, lambda r: r.kv_store(T, kv, D, dZ, stride, heads * D, dC, 10))
    got = dC.read(np.uint16, (T + 10, 2 * kv * D))[10:]
    assert np.array_equal(got, Z[:, heads * D:].view(np.uint16))


# ---------------------------------------------------------------- readouts

@pytest.mark.parametrize("bits,H", [(8, 1024), (4, 2048), (8, 1536)])
def test_leaf_logits(pkg, ctx, bits, H):
    dj = _dj()
    rng = np.random.default_rng(bits + H)
    V, T, L, n_ids = 500, 64, 5, 7
    codes, scales = quant(rng, V, H, bits)
    X = rand_f16(rng, (T, H), std=3.0)
    w = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    leaves = rng.integers(0, T, L).astype(np.uint32)
    ids = rng.integers(0, V, L * n_ids).astype(np.uint32)
    E = ctx.weight_q(codes, scales, V, H, bits, dj.W_PLAIN)
    dX, dl, dw, di, do = ctx.array(X), ctx.array(leaves), ctx.array(w), ctx.array(ids), ctx.alloc(L * n_ids * 4)
    run(ctx, lambda r: r.leaf_logits(T, L, H, n_ids, 1e-6, dX, dl, dw, di, E, do))
    got = do.read(np.float32, (L * n_ids,))
    want = ref.leaf_logits(X, leaves, w, ids, n_ids, codes, scales, bits, 1e-6, np.float64)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max() + 1e-6


def test_readout_pool_dense(pkg, ctx):
    dj = _dj()
    rng = np.random.default_rng(9)
    T, H, codes_n = 80, 768, 10
    X = rand_f16(rng, (T, H))
    R = rng.standard_normal((codes_n, H)).astype(np.float32)
    pairs = np.array([(5, 1), (79, 9), (0, 0), (40, 3)], dtype=np.uint32)
    dX, dR, dp, do = ctx.array(X), ctx.array(R), ctx.array(pairs), ctx.alloc(4 * 4)
    ranges = np.array([(0, 30), (30, 31), (31, 80)], dtype=np.uint32)
    dr, dpool = ctx.array(ranges), ctx.alloc(3 * H * 4)
    c, s = quant(rng, 96, H, 8)
    W = ctx.weight_q(c, s, 96, H, 8, dj.W_PLAIN)
    dd = ctx.alloc(3 * 96 * 4)

    def body(r):
        r.readout(T, 4, H, dX, dR, codes_n, dp, do)
        r.mean_pool(T, 3, H, dX, dr, dpool)
        r.dense_f32(3, dpool, W, dd)
    run(ctx, body)
    assert np.allclose(do.read(np.float32, (4,)), ref.readout(X, R, pairs), rtol=1e-5, atol=1e-4)
    pooled = ref.mean_pool(X, ranges)
    assert np.allclose(dpool.read(np.float32, (3, H)), pooled, rtol=1e-5, atol=1e-6)
    assert np.allclose(dd.read(np.float32, (3, 96)), ref.dense_f32(pooled, c, s, 8), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("bits", [8, 4])
def test_pooled_head_long_sequences_and_many_rows(pkg, ctx, bits):
    """mean_pool over a 256-token sequence (4 waves x 64 tokens each) and a 1-token one; dense_f32 with 20 rows
    (two register chunks of 16) over K = 3072 (12 steps of 256 per lane) and its 768-wide second layer."""
    dj = _dj()
    rng = np.random.default_rng(bits + 90)
    H = 768
    lens = [256] + [24] * 3 + [8] * 7 + [1] * 9
    T = sum(lens)
    X = rand_f16(rng, (T, H))
    starts = np.cumsum([0] + lens[:-1])
    ranges = np.array([(a, a + n) for a, n in zip(starts, lens)], dtype=np.uint32)
    M = len(lens)
    c1, s1 = quant(rng, 3072, H, bits)
    c2, s2 = quant(rng, H, 3072, bits)
    W1, W2 = ctx.weight_q(c1, s1, 3072, H, bits, dj.W_PLAIN), ctx.weight_q(c2, s2, H, 3072, bits, dj.W_PLAIN)
    dX, dr = ctx.array(X), ctx.array(ranges)
    dpool, dh, de = ctx.alloc(M * H * 4), ctx.alloc(M * 3072 * 4), ctx.alloc(M * H * 4)

    def body(r):
        r.mean_pool(T, M, H, dX, dr, dpool)
        r.dense_f32(M, dpool, W1, dh)
        r.dense_f32(M, dh, W2, de)
    run(ctx, body)
    pooled = ref.mean_pool(X, ranges)
    assert np.allclose(dpool.read(np.float32, (M, H)), pooled, rtol=1e-5, atol=1e-6)
    h = ref.dense_f32(pooled, c1, s1, bits)
    assert np.allclose(dh.read(np.float32, (M, 3072)), h, rtol=1e-4, atol=1e-5)
    e = ref.dense_f32(h, c2, s2, bits)
    assert np.allclose(de.read(np.float32, (M, H)), e, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- recorder: snapshots, graphs, errors

def test_graph_replay_matches_eager(pkg, ctx):
    """A captured forward replayed several times, with eager work and syncs in between, equals eager."""
    dj = _dj()
    rng = np.random.default_rng(21)
    T, H, N = 96, 1024, 2048
    codes, scales = quant(rng, N, H, 8)
    ec, es = quant(rng, 400, H, 8)
    W = ctx.weight_q(codes, scales, N, H, 8, dj.W_MFMA)
    E = ctx.weight_q(ec, es, 400, H, 8, dj.W_PLAIN)
    w = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    dw, dids = ctx.array(w), ctx.alloc(T * 4)
    dX, dO, dY = ctx.alloc(T * H * 2), ctx.alloc(T * H * 2), ctx.alloc(T * N * 2)

    def forward(key, ids):
        dids.write(ids)
        rec = ctx.recorder(key)
        rec.gather_q(dids, T, E, dX)
        rec.add_rmsnorm(T, H, False, 1e-6, dX, dX, dw, dO)
        rec.matmul(dO, W, dY, T)
        i = rec.snapshot(dY, T * N * 2, np.float16, (T, N))
        replay = rec.replay
        return rec.finish()[i], replay

    key = 0xD1_0001
    ctx.graph_clear()
    for it in range(4):
        ids = rng.integers(0, 400, T).astype(np.uint32)
        eager, _ = forward(0, ids)
        graph, replayed = forward(key, ids)
        assert replayed == (it > 0)
        assert np.array_equal(eager.view(np.uint16), graph.view(np.uint16))
    ctx.graph_clear()


def test_profile_and_timer(pkg, ctx):
    dj = _dj()
    rng = np.random.default_rng(2)
    codes, scales = quant(rng, 256, 256, 8)
    W = ctx.weight_q(codes, scales, 256, 256, 8, dj.W_MFMA)
    dX, dY = ctx.array(rand_f16(rng, (64, 256))), ctx.alloc(64 * 256 * 2)
    ctx.profile_reset()
    ctx.profile(True)
    ctx.timer_begin()
    for _ in range(3):
        run(ctx, lambda r: r.matmul(dX, W, dY, 64))
    ms = ctx.timer_end()
    ctx.profile(False)
    table = ctx.profile_table()
    assert ms > 0 and any(k.startswith("matmul_q8") and v[1] == 3 for k, v in table.items())


def test_errors_surface(pkg, ctx):
    dj = _dj()
    rng = np.random.default_rng(1)
    codes, scales = quant(rng, 64, 64, 8)
    W = ctx.weight_q(codes, scales, 64, 64, 8, dj.W_PLAIN)
    dX = ctx.alloc(64 * 64 * 2)
    rec = ctx.recorder()
    with pytest.raises(dj.DJError, match="decision.js: matmul needs an MFMA-tiled weight"):
        rec.matmul(dX, W, dX, 64)
    rec.finish()
    with pytest.raises(dj.DJError, match="K must be a multiple of 32"):
        ctx.weight_q(np.zeros((4, 40), np.uint8), np.zeros((4, 1), np.float16), 4, 40, 8, dj.W_PLAIN)


# ---------------------------------------------------------------- LFM2 short conv

@pytest.mark.parametrize("H", [2048, 64, 1536])
def test_short_conv(pkg, ctx, H):
    """dj_short_conv against a float64 closed form of SHORT_CONV (kernels.ts:62-84) on forest taps (causal,
    branches continuing their trunk), with taps of -1 and out of range (read as zero): within one f16 ulp of
    the float64 value plus the f32 accumulation's error."""
    rng = np.random.default_rng(H)
    trees = [{"trunk": [0] * 40, "branches": [[0] * 9, [0] * 1, [0] * 17], "groups": []},
             {"trunk": [], "branches": [[0] * 5], "groups": []}, {"trunk": [0] * 2, "branches": [], "groups": []}]
    taps = ref.forest_taps(trees)
    T = len(taps)
    taps[3, 0] = T + 5  # out of range: reads zero
    Z = rand_f16(rng, (T, 3 * H))
    w = rand_f16(rng, (H, 3), 0.5)
    dZ, dw, dT, dY = ctx.array(Z), ctx.array(w), ctx.array(taps), ctx.alloc(T * H * 2)
    run(ctx, lambda r: r.short_conv(T, H, dZ, dw, dT, dY))
    got = dY.read(np.float16, (T, H))
    t64 = taps.copy()
    t64[3, 0] = -1
    want = ref.short_conv(Z, H, w, t64, np.float64)
    z = Z.astype(np.float64)
    bu = np.abs(z[:, :H] * z[:, 2 * H:])
    # f32 rounding of the three products and sums, on the magnitude of the terms
    mag = np.abs(z[:, H:2 * H]) * sum(np.abs(w[:, j].astype(np.float64))[None, :] * np.where((t64[:, j] >= 0)[:, None], bu[t64[:, j]], 0) for j in range(3))
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert (err <= 2.0 ** -10 * np.abs(want.astype(np.float64)) + 4 * 2.0 ** -24 * mag + 1e-7).all()
    assert not np.isnan(got.astype(np.float32)).any()


# ---------------------------------------------------------------- d1-omni's decision head ops

def test_add_rows_bit_exact(pkg, ctx):
    """dj_add_rows against ADD_ROWS (kernels.ts:188-201): f16(f32 + f32) is exactly rounded, so bit for bit; a
    type index past the table reads its last row."""
    rng = np.random.default_rng(51)
    T, H = 301, 1024
    X, E = rand_f16(rng, (T, H)), rand_f16(rng, (3, H), 0.5)
    idx = rng.integers(0, 3, T).astype(np.uint32)
    idx[:2] = [7, 2]
    dX, di, dE, dO = ctx.array(X), ctx.array(idx), ctx.array(E), ctx.alloc(T * H * 2)
    run(ctx, lambda r: r.add_rows(T, H, dX, di, dE, 3, dO))
    assert np.array_equal(dO.read(np.uint16, (T, H)), ref.add_rows(X, idx, E).view(np.uint16))


@pytest.mark.parametrize("act", [0, 1, 2])
def test_bias_act(pkg, ctx, act):
    """dj_bias_act against BIAS_ACT (kernels.ts:203-222): no activation and ReLU bit for bit; GELU with the A&S
    erf within one f16 rounding of the float64 value (the erf's exp is libm's, not numpy's)."""
    rng = np.random.default_rng(60 + act)
    T, N = 77, 3072
    Y, b = rand_f16(rng, (T, N), 2.0), rand_f16(rng, (N,), 0.5)
    dY, db = ctx.array(Y), ctx.array(b)
    run(ctx, lambda r: r.bias_act(T, N, dY, db, act))
    got = dY.read(np.float16, (T, N))
    if act < 2:
        assert np.array_equal(got.view(np.uint16), ref.bias_act(Y, b, act).view(np.uint16))
    else:
        want = ref.bias_act(Y, b, 2, np.float64)
        assert f16_close(got, want, ulps=1.0, atol=2e-7) <= 1.0


@pytest.mark.parametrize("H,add", [(1024, True), (1024, False), (2048, True), (768, True)])
def test_add_layernorm(pkg, ctx, H, add):
    """dj_add_layernorm against ADD_LAYERNORM (kernels.ts:224-255): the stored sum bit for bit; the normalised
    output within one f16 ulp of the float64 value (rows with a large mean included: E[x^2] - mean^2)."""
    rng = np.random.default_rng(H + 7 * add)
    T = 131
    X, Y = rand_f16(rng, (T, H)), rand_f16(rng, (T, H))
    X[:5] += np.float16(6.0)
    w = (1 + rng.standard_normal(H) * 0.1).astype(np.float16)
    b = rand_f16(rng, (H,), 0.1)
    dX, dY, dw, db, dO = ctx.array(X), ctx.array(Y), ctx.array(w), ctx.array(b), ctx.alloc(T * H * 2)
    run(ctx, lambda r: r.add_layernorm(T, H, add, 1e-5, dX, dY, dw, db, dO))
    Xn, O = ref.add_layernorm(X, Y, w, b, 1e-5, add=add, acc=np.float64)
    assert np.array_equal(dX.read(np.uint16, (T, H)), Xn.view(np.uint16))
    assert f16_close(dO.read(np.float16, (T, H)), O, ulps=1.0, atol=1e-4) <= 1.0


def test_gather_rows_and_score(pkg, ctx):
    """dj_gather_rows (GATHER_ROWS, kernels.ts:257-267) bit for bit, rows past T clamped; dj_score (SCORE,
    kernels.ts:269-283) within f32 accumulation error of the float64 dot product plus the bias."""
    rng = np.random.default_rng(71)
    T, H, M = 500, 1024, 37
    X = rand_f16(rng, (T, H))
    rows = rng.integers(0, T, M).astype(np.uint32)
    rows[0] = T + 3
    w, b = rand_f16(rng, (H,), 0.05), np.array([0.3, 0.0], dtype=np.float16)
    dX, dr, dG, dw, db, dout = ctx.array(X), ctx.array(rows), ctx.alloc(M * H * 2), ctx.array(w), ctx.array(b), ctx.alloc(M * 4)
    run(ctx, lambda r: (r.gather_rows(M, H, T, dX, dr, dG), r.score(M, H, dG, dw, db, dout)))
    G = dG.read(np.float16, (M, H))
    assert np.array_equal(G.view(np.uint16), X[np.minimum(rows, T - 1)].view(np.uint16))
    want = ref.score(G, w, b, np.float64)
    mag = np.abs(G.astype(np.float64)) @ np.abs(w.astype(np.float64))
    assert (np.abs(dout.read(np.float32, (M,)) - want) <= 2.0 ** -18 * (mag + 0.3) + 1e-6).all()


def test_head_ops_refuse_bad_shapes(pkg, ctx):
    dj = _dj()
    buf = ctx.alloc(4096)
    rec = ctx.recorder()
    try:
        with pytest.raises(dj.DJError, match="multiple of 8"):
            rec.add_layernorm(2, 100, True, 1e-5, buf, buf, buf, buf, buf)
        with pytest.raises(dj.DJError, match="act 0..2"):
            rec.bias_act(2, 64, buf, buf, 3)
    finally:
        rec.abort()


# ---------------------------------------------------------------- d3-lite's mixers

@pytest.mark.parametrize("split", [False, True])
def test_attention_gated(pkg, ctx, split, monkeypatch):
    """dj_attention_gated (attention256, d3-kernels.ts:180-240): attention over d3's key ranges (a shared trunk +
    each question, noncausal within them) times sigmoid(gate), one f16 rounding, against the float64 oracle;
    with the split-KV plan forced the merge applies the gate."""
    if split:
        monkeypatch.setenv("DJ_ATTN_SPLITS", "3")
    dj = _dj()
    rng = np.random.default_rng(81)
    heads, kv, D = 8, 2, 256
    seqs = [{"ids": [1] * 40 + [int(x) for x in rng.integers(0, 9, n)], "options": 2} for n in (12, 1, 30)]
    ids, meta, r4, pairs = ref.pack_shared(seqs, [3])
    T = len(ids)
    stride = (2 * heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride))
    dZ, dr, dO = ctx.array(Z), ctx.array(r4), ctx.alloc(T * heads * D * 2)
    src = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    goff = (heads + 2 * kv) * D
    run(ctx, lambda r: r.attention_gated(T, heads, kv, D, dZ, stride, src, src, dr, 1 / 16, dZ.at(goff * 2), stride, dO))
    got = dO.read(np.float16, (T, heads * D)).astype(np.float64)
    want = ref.attention(Z, heads, kv, D, ref.ranges_mask(r4, T), 1 / 16, np.float64, gate=Z[:, goff:]).astype(np.float64)
    err = np.abs(got - want).max()
    print(f"gated attention T{T}: max abs err {err:.2e}")
    assert err < 4e-3


def _gdn_case(rng, LH, seqs, groups):
    ids, meta, r4, pairs = ref.pack_shared(seqs, groups)
    spans = ref.d3_spans(seqs, groups)
    T, QK = len(ids), LH * 128
    stride = 4 * QK + 2 * LH + 16
    Z = rand_f16(rng, (T, stride))
    conv = rand_f16(rng, (3 * QK, 4), 0.5)
    A_log = np.log(0.01 + 0.99 * rng.random(LH)).astype(np.float16)
    dt = rand_f16(rng, (LH,), 0.5)
    gn = (1 + 0.1 * rng.standard_normal(128)).astype(np.float16)
    return T, stride, spans, Z, conv, A_log, dt, gn


@pytest.mark.parametrize("form", ["split", "whole"])
@pytest.mark.parametrize("groups", [None, [3, 1], [4]])
def test_gdn(pkg, ctx, groups, form, monkeypatch):
    """dj_gdn (gdnLayer, d3-kernels.ts:9-149) against the oracle's textbook recurrence in float64: sequences longer
    than a 32-token chunk and of one token, a shared trunk rescanned by each question and written once; both forms
    (state rows split over 8 workgroups with the norm in a second kernel, and one workgroup per head). Bound: the f16 output within 3e-3 of the largest value (the state runs in f32 over
    up to 110 tokens; the conv rounding points are the oracle's)."""
    if form == "whole":
        monkeypatch.setenv("DJ_GDN_FORM", "1")
    rng = np.random.default_rng(90 + (0 if groups is None else sum(groups)))
    LH = 4
    state = [int(x) for x in rng.integers(0, 9, 45)]
    lens = (70, 1, 33, 5)
    seqs = [{"ids": (state if groups else []) + [int(x) for x in rng.integers(0, 9, n)], "options": 2} for n in lens]
    T, stride, spans, Z, conv, A_log, dt, gn = _gdn_case(rng, LH, seqs, groups)
    dZ, ds, dc, da, ddt, dg = (ctx.array(a) for a in (Z, spans, conv, A_log, dt, gn))
    Y0 = np.full((T, LH * 128), 7.0, dtype=np.float16)
    dY = ctx.array(Y0)
    run(ctx, lambda r: r.gdn(T, len(spans), ds, LH, stride, dZ, dc, da, ddt, dg, 1e-6, dY))
    got = dY.read(np.float16, (T, LH * 128)).astype(np.float64)
    want = ref.gdn(Z, spans, LH, conv, A_log, dt, gn, 1e-6, np.float64).astype(np.float64)
    err = np.abs(got - want).max()
    print(f"gdn groups {groups} T{T}: max abs err {err:.2e} (max |y| {np.abs(want).max():.2f})")
    assert err < 3e-3 * np.abs(want).max()
    assert not np.isnan(got).any()


def test_gdn_refuses_short_rows(pkg, ctx):
    dj = _dj()
    buf = ctx.alloc(4096)
    rec = ctx.recorder()
    try:
        with pytest.raises(dj.DJError, match="hold fewer than"):
            rec.gdn(4, 1, buf, 2, 100, buf, buf, buf, buf, buf, 1e-6, buf)
    finally:
        rec.abort()


# ---------------------------------------------------------------- EmbeddingGemma 2's per-layer embeddings

def test_ple_mix(pkg, ctx):
    """dj_ple_mix (PLE_MIX, eg2-kernels.ts:179-200) within one f16 ulp of the float64 oracle."""
    rng = np.random.default_rng(101)
    T, P = 133, 512
    G, E = rand_f16(rng, (T, P), 1.5), rand_f16(rng, (T, P))
    w = (1 + 0.1 * rng.standard_normal(P)).astype(np.float16)
    dG, dE, dw, dO = ctx.array(G), ctx.array(E), ctx.array(w), ctx.alloc(T * P * 2)
    run(ctx, lambda r: r.ple_mix(T, P, dG, dE, dw, 1e-6, dO))
    want = ref.ple_mix(G, E, w, 1e-6, np.float64)
    assert f16_close(dO.read(np.float16, (T, P)), want, ulps=1.0, atol=1e-6) <= 1.0


def test_pool_project(pkg, ctx):
    """dj_pool_project (POOL_PROJECT, eg2-kernels.ts:202-228): the f32 mean of each text's rows times the f16
    projection, within f32 rounding of the float64 product; one-token texts included."""
    rng = np.random.default_rng(102)
    H, N = 512, 768
    lens = [256, 24, 24, 1, 8, 40]
    T = sum(lens)
    X = rand_f16(rng, (T, H))
    W = rand_f16(rng, (N, H), 0.05)
    ranges = np.array([(sum(lens[:k]), sum(lens[:k + 1])) for k in range(len(lens))], dtype=np.uint32)
    dX, dr, dW, dout = ctx.array(X), ctx.array(ranges), ctx.array(W), ctx.alloc(len(lens) * N * 4)
    run(ctx, lambda r: r.pool_project(T, len(lens), H, N, dX, dr, dW, dout))
    got = dout.read(np.float32, (len(lens), N)).astype(np.float64)
    means = np.stack([X[a:b].astype(np.float64).mean(0) for a, b in ranges])
    want = means @ W.astype(np.float64).T
    mag = np.abs(means) @ np.abs(W.astype(np.float64)).T
    assert (np.abs(got - want) <= 2.0 ** -18 * mag + 1e-6).all()


@pytest.mark.parametrize("window", [None, 40])
def test_attention_512(pkg, ctx, window):
    """dj_attention with 512-dim heads (EmbeddingGemma 2's global layers; the windowed form too) against the float64
    oracle; GQA 4:2; texts of 1 to 300 tokens."""
    dj = _dj()
    rng = np.random.default_rng(103 + (window or 0))
    heads, kv, D = 4, 2, 512
    seqs = [list(range(n)) for n in (300, 24, 1, 8, 77)]
    ids, meta, full, slide, ranges = ref.pack_encoder(seqs, window=window)
    r4 = full if window is None else slide
    T = len(ids)
    stride = (heads + 2 * kv) * D
    Z = rand_f16(rng, (T, stride), 0.3)
    dZ, dr, dO = ctx.array(Z), ctx.array(r4), ctx.alloc(T * heads * D * 2)
    src = dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    run(ctx, lambda r: r.attention(T, heads, kv, D, dZ, stride, src, src, dr, 1.0, dO))
    got = dO.read(np.float16, (T, heads * D)).astype(np.float64)
    want = ref.attention(Z, heads, kv, D, ref.ranges_mask(r4, T), 1.0, np.float64).astype(np.float64)
    err = np.abs(got - want).max()
    print(f"attention D512 window {window}: max abs err {err:.2e}")
    assert err < 4e-3
