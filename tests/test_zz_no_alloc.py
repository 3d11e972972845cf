"""dj_attention_noalloc (the entry point that allocates nothing: its split-KV partials live in the library's
static device scratch) against dj_attention on the same inputs, through the C ABI: bit-identical outputs on two
calls in a row, the second with fewer queries and keys, each on a split-KV shape (a short question against a
long kept state); a call whose split plan needs more scratch than the array holds is refused with a clear
error, and nothing has been written to its output."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(ctx, rng, T, P, heads, kv, D):
    from decision_js_amd import _dj
    stride = (heads + 2 * kv) * D
    Z = (rng.standard_normal((T, stride)) * 0.5).astype(np.float16)
    cache = (rng.standard_normal((P, 2 * kv * D)) * 0.5).astype(np.float16)
    i = np.arange(T, dtype=np.int32)
    rngs = np.stack([np.zeros(T, np.int32), np.full(T, P, np.int32), np.zeros(T, np.int32), i + 1], 1)
    dZ, dC, dR = ctx.array(Z), ctx.array(cache), ctx.array(rngs)
    A = _dj.kv_src(dC, P, 2 * kv * D, 0, kv * D)
    B = _dj.kv_src(dZ, T, stride, heads * D, (heads + kv) * D)
    return dZ, dC, dR, A, B, stride


def _run(ctx, fn_name, T, heads, kv, D, dZ, stride, A, B, dR, out):
    rec = ctx.recorder()
    getattr(rec, fn_name)(T, heads, kv, D, dZ, stride, A, B, dR, 1.0 / np.sqrt(D), out)
    rec.finish()
    return out.read(np.uint16, (T, heads * D))


def test_attention_noalloc_matches_attention(pkg, ctx):
    rng = np.random.default_rng(21)
    ctx.profile_reset()
    for T, P, heads, kv, D in [(32, 1056, 12, 2, 128), (9, 700, 16, 8, 64)]:  # the second call smaller
        dZ, dC, dR, A, B, stride = _case(ctx, rng, T, P, heads, kv, D)
        out1, out2 = ctx.alloc(T * heads * D * 2), ctx.alloc(T * heads * D * 2)
        ctx.profile(True)
        try:
            want = _run(ctx, "attention", T, heads, kv, D, dZ, stride, A, B, dR, out1)
            got = _run(ctx, "attention_noalloc", T, heads, kv, D, dZ, stride, A, B, dR, out2)
        finally:
            ctx.profile(False)
        assert np.array_equal(got, want), (T, P, heads, kv, D)
        assert np.isfinite(got.view(np.float16)).all()
        for b in (dZ, dC, dR, out1, out2):
            b.free()
    # both shapes took the split-KV path (its combine kernel ran), so the scratch was used
    names = ctx.profile_table()
    assert sum(v[1] for k, v in names.items() if k.startswith("attention_noalloc")) == 2, names


def test_attention_noalloc_refuses_oversized_plans(pkg, ctx):
    from decision_js_amd import _dj
    rng = np.random.default_rng(22)
    # 40 queries x 64 heads of 256 dims against 4096 kept keys: the split plan (8 splits) needs ~21 MB of partials
    T, P, heads, kv, D = 40, 4096, 64, 4, 256
    dZ, dC, dR, A, B, stride = _case(ctx, rng, T, P, heads, kv, D)
    out = ctx.alloc(T * heads * D * 2)
    out.write(np.zeros(T * heads * D, np.uint16))
    rec = ctx.recorder()
    with pytest.raises(_dj.DJError, match="dj_attention_noalloc: .* scratch"):
        with rec:
            rec.attention_noalloc(T, heads, kv, D, dZ, stride, A, B, dR, 1.0 / np.sqrt(D), out)
    assert not out.read(np.uint16, (T * heads * D,)).any()
    # the context is free again (the failed recording was aborted) and the plain entry point handles the shape
    got = _run(ctx, "attention", T, heads, kv, D, dZ, stride, A, B, dR, out)
    assert np.isfinite(got.view(np.float16)).all()
    for b in (dZ, dC, dR, out):
        b.free()
