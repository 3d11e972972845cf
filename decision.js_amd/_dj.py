"""ctypes binding of libdj.so (include/dj.h): the C ABI the host engines call.

The library is built in-tree by decision.js_amd/csrc/build.py. Loading fails loudly when it is missing:
there is no CPU fallback on the product path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libdj.so")

DJ_OK, DJ_EINVAL, DJ_EHIP, DJ_ENOMEM, DJ_ESTATE, DJ_EINJECT = range(6)
W_PLAIN, W_MFMA, W_MFMA_GLU = 0, 1, 2
BIAS_NONE, BIAS_RELU, BIAS_GELU_ERF = 0, 1, 2
W_DIRECT = 16  # flag: f16 weights dequantized once at load (the reference's directWeights)
ACT_SILU, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2
ROPE_POW_NEG, ROPE_INV_POW = 0, 1


class DJError(RuntimeError):
    """A failed libdj call; str() is the library's "decision.js: ..." message."""

    def __init__(self, status: int, message: str):
        super().__init__(message or f"decision.js: error {status}")
        self.status = status


class KVSrc(C.Structure):
    _fields_ = [("base", C.c_void_p), ("rows", C.c_int), ("stride", C.c_int), ("k_col", C.c_int), ("v_col", C.c_int)]


class ProfileEntry(C.Structure):
    _fields_ = [("name", C.c_char * 96), ("ms", C.c_double), ("launches", C.c_int64)]


_P, _I, _F, _U64, _SZ = C.c_void_p, C.c_int, C.c_float, C.c_uint64, C.c_size_t

# name: argument types (all return int status unless listed in _RET)
SIGNATURES = {
    "dj_last_error": [],
    "dj_abi_version": [],
    "dj_init": [_I, C.POINTER(_P)],
    "dj_destroy": [_P],
    "dj_device_info": [_P, C.c_char_p, _SZ, C.POINTER(_I), C.POINTER(_SZ)],
    "dj_buf_alloc": [_P, _SZ, C.POINTER(_P)],
    "dj_buf_free": [_P, _P],
    "dj_buf_write": [_P, _P, _P, _SZ],
    "dj_buf_read": [_P, _P, _P, _SZ],
    "dj_weight_q": [_P, _P, _P, _I, _I, _I, _I, C.POINTER(_P)],
    "dj_weight_free": [_P, _P],
    "dj_weight_bytes": [_P],
    "dj_rec_begin": [_P, _U64, C.POINTER(_P), C.POINTER(_I)],
    "dj_upload": [_P, _P, _P, _SZ],
    "dj_buf_copy": [_P, _P, _P, _SZ],
    "dj_rec_snapshot": [_P, _P, _SZ, _P],
    "dj_rec_finish": [_P],
    "dj_rec_abort": [_P],
    "dj_graph_clear": [_P],
    "dj_graph_drop": [_P, _U64],
    "dj_graph_count": [_P, C.POINTER(_I)],
    "dj_timer_begin": [_P],
    "dj_timer_end": [_P, C.POINTER(_F)],
    "dj_profile_enable": [_P, _I],
    "dj_profile_get": [_P, C.POINTER(ProfileEntry), _I, C.POINTER(_I)],
    "dj_profile_reset": [_P],
    "dj_gather_q": [_P, _P, _I, _P, _P],
    "dj_add_rmsnorm": [_P, _I, _I, _I, _F, _P, _P, _P, _P],
    "dj_sandwich": [_P, _I, _I, _F, _F, _P, _P, _P, _P, _P],
    "dj_matmul": [_P, _P, _P, _P, _I],
    "dj_matmul_glu": [_P, _P, _P, _P, _I, _I],
    "dj_qk_norm_rope": [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P, _I, _F, _F, _I, _I],
    "dj_rope_table": [_P, _I, _P, _I, _F, _I, _I, _P],
    "dj_matmul_qkv_rope": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _F, _F, _I, _I, _P],
    "dj_matmul_residual": [_P, _P, _P, _I, _P, _P, _P, _P],
    "dj_matmul_normed": [_P, _P, _P, _P, _I, _I, _P, _I, _F],
    "dj_matmul_qkv_rope_normed": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _F, _F, _I, _I, _P, _P, _I, _F],
    "dj_attention": [_P, _I, _I, _I, _I, _P, _I, KVSrc, KVSrc, _P, _F, _P],
    "dj_attention_noalloc": [_P, _I, _I, _I, _I, _P, _I, KVSrc, KVSrc, _P, _F, _P],
    "dj_attention_qk_rope": [_P, _I, _I, _I, _I, _P, _I, KVSrc, KVSrc, _P, _F, _P, _P, _F, _P, _I, _P],
    "dj_attention_gated": [_P, _I, _I, _I, _I, _P, _I, KVSrc, KVSrc, _P, _F, _P, _I, _P],
    "dj_gdn": [_P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _P, _F, _P],
    "dj_ple_mix": [_P, _I, _I, _P, _P, _P, _F, _P],
    "dj_pool_project": [_P, _I, _I, _I, _I, _P, _P, _P, _P],
    "dj_kv_store": [_P, _I, _I, _I, _P, _I, _I, _P, _I],
    "dj_leaf_logits": [_P, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P],
    "dj_readout": [_P, _I, _I, _I, _P, _P, _I, _P, _P],
    "dj_short_conv": [_P, _I, _I, _P, _P, _P, _P],
    "dj_add_rows": [_P, _I, _I, _P, _P, _P, _I, _P],
    "dj_bias_act": [_P, _I, _I, _P, _P, _I],
    "dj_add_layernorm": [_P, _I, _I, _I, _F, _P, _P, _P, _P, _P],
    "dj_gather_rows": [_P, _I, _I, _I, _P, _P, _P],
    "dj_score": [_P, _I, _I, _P, _P, _P, _P],
    "dj_mean_pool": [_P, _I, _I, _I, _P, _P, _P],
    "dj_dense_f32": [_P, _I, _P, _P, _P],
}
_RET = {"dj_last_error": C.c_char_p, "dj_weight_bytes": _SZ}

_lib = None


def lib():
    """The loaded libdj.so (raises ImportError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"decision.js: {LIB_PATH} is missing; build it with `python decision.js_amd/csrc/build.py`")
        L = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RET.get(name, C.c_int)
        _lib = L
    return _lib


def check(status: int):
    if status != DJ_OK:
        raise DJError(status, lib().dj_last_error().decode(errors="replace"))


def ptr(x) -> int:
    """Device address of a DevBuf (plus byte offset), or a plain int."""
    if x is None:
        return None
    if isinstance(x, DevBuf):
        return x.ptr
    return int(x)


class DevBuf:
    """A device buffer owned by a Context (the reference's GPUBuffer)."""

    def __init__(self, ctx: "Context", nbytes: int, ptr_: int, owner: bool = True, base=None):
        self.ctx, self.nbytes, self.ptr, self.owner, self.base = ctx, nbytes, ptr_, owner, base

    def at(self, byte_offset: int, nbytes: int = None) -> "DevBuf":
        """A view starting `byte_offset` bytes in (not owning memory)."""
        n = self.nbytes - byte_offset if nbytes is None else nbytes
        if byte_offset < 0 or byte_offset + n > self.nbytes:
            raise ValueError("decision.js: buffer view out of range")
        return DevBuf(self.ctx, n, self.ptr + byte_offset, owner=False, base=self)

    def write(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError(f"decision.js: {arr.nbytes} bytes do not fit a {self.nbytes}-byte buffer")
        check(lib().dj_buf_write(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes))

    def upload(self, arr: np.ndarray):
        """Asynchronous write ordered with the queued ops (dj_upload)."""
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError(f"decision.js: {arr.nbytes} bytes do not fit a {self.nbytes}-byte buffer")
        check(lib().dj_upload(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes))

    def copy_from(self, src: "DevBuf", nbytes: int = None):
        """Asynchronous device->device copy on the context's stream (dj_buf_copy)."""
        n = src.nbytes if nbytes is None else nbytes
        if n > self.nbytes or n > src.nbytes:
            raise ValueError("decision.js: device copy larger than a buffer")
        check(lib().dj_buf_copy(self.ctx.h, self.ptr, src.ptr, n))

    def read(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("decision.js: read past the end of a buffer")
        check(lib().dj_buf_read(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.owner and self.ptr:
            check(lib().dj_buf_free(self.ctx.h, self.ptr))
        self.ptr = 0


class Weight:
    """A quantized weight on the device (the reference's Weight, gpu.ts:11)."""

    def __init__(self, ctx, handle, N, K, bits, layout):
        self.ctx, self.h, self.N, self.K, self.bits, self.layout = ctx, handle, N, K, bits, layout
        self.shape = [N, K]

    @property
    def nbytes(self) -> int:
        return int(lib().dj_weight_bytes(self.h))

    def free(self):
        if self.h:
            check(lib().dj_weight_free(self.ctx.h, self.h))
        self.h = None


class Context:
    """One device and its stream (dj_init)."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        check(lib().dj_init(ordinal, C.byref(h)))
        self.h = h.value
        self.closed = False

    def info(self):
        name = C.create_string_buffer(64)
        cus, mem = C.c_int(), C.c_size_t()
        check(lib().dj_device_info(self.h, name, 64, C.byref(cus), C.byref(mem)))
        return {"arch": name.value.decode(), "compute_units": cus.value, "memory": mem.value}

    def alloc(self, nbytes: int) -> DevBuf:
        p = C.c_void_p()
        check(lib().dj_buf_alloc(self.h, max(int(nbytes), 1), C.byref(p)))
        return DevBuf(self, int(nbytes), p.value)

    def array(self, arr: np.ndarray) -> DevBuf:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        b.write(arr)
        return b

    def weight_q(self, codes: np.ndarray, scales: np.ndarray, N: int, K: int, bits: int, layout: int) -> Weight:
        codes = np.ascontiguousarray(codes, dtype=np.uint8)
        scales = np.ascontiguousarray(scales).view(np.uint16)
        exp_codes = N * K * bits // 8
        if codes.nbytes != exp_codes or scales.nbytes != N * (K // 32) * 2:
            raise ValueError(f"decision.js: weight [{N}, {K}] q{bits}: {codes.nbytes} code bytes, {scales.nbytes} scale bytes")
        h = C.c_void_p()
        check(lib().dj_weight_q(self.h, codes.ctypes.data, scales.ctypes.data, N, K, bits, layout, C.byref(h)))
        return Weight(self, h.value, N, K, bits, layout)

    def graph_clear(self):
        check(lib().dj_graph_clear(self.h))

    def graph_drop(self, key: int):
        check(lib().dj_graph_drop(self.h, key))

    def graph_count(self) -> int:
        n = C.c_int()
        check(lib().dj_graph_count(self.h, C.byref(n)))
        return n.value

    # timing / profiling (gpu.ts:29-34, 185-197)
    def timer_begin(self):
        check(lib().dj_timer_begin(self.h))

    def timer_end(self) -> float:
        ms = C.c_float()
        check(lib().dj_timer_end(self.h, C.byref(ms)))
        return ms.value

    def profile(self, on: bool):
        check(lib().dj_profile_enable(self.h, 1 if on else 0))

    def profile_reset(self):
        check(lib().dj_profile_reset(self.h))

    def profile_table(self):
        n = C.c_int()
        check(lib().dj_profile_get(self.h, None, 0, C.byref(n)))
        arr = (ProfileEntry * max(n.value, 1))()
        check(lib().dj_profile_get(self.h, arr, n.value, C.byref(n)))
        return {arr[i].name.decode(): (arr[i].ms, arr[i].launches) for i in range(n.value)}

    def recorder(self, graph_key: int = 0) -> "Recorder":
        return Recorder(self, graph_key)

    def close(self):
        if not self.closed:
            check(lib().dj_destroy(self.h))
            self.closed = True


class Recorder:
    """One forward pass (gpu.ts recorder(): dispatch / matmul / swiglu / snapshot / finish)."""

    def __init__(self, ctx: Context, graph_key: int = 0):
        self.ctx = ctx
        h = C.c_void_p()
        rp = C.c_int()
        check(lib().dj_rec_begin(ctx.h, C.c_uint64(graph_key), C.byref(h), C.byref(rp)))
        self.h = h.value
        self.replay = bool(rp.value)
        self._snaps = []

    # ---- ops
    def gather_q(self, ids, T, embed: Weight, X):
        check(lib().dj_gather_q(self.h, ptr(ids), T, embed.h, ptr(X)))

    def add_rmsnorm(self, T, H, add, eps, X, Y, w, O):
        check(lib().dj_add_rmsnorm(self.h, T, H, 1 if add else 0, eps, ptr(X), ptr(Y), ptr(w), ptr(O)))

    def sandwich(self, T, H, eps, scale, X, Y, w1, w2, O):
        check(lib().dj_sandwich(self.h, T, H, eps, scale, ptr(X), ptr(Y), ptr(w1), ptr(w2), ptr(O)))

    def matmul(self, X, w: Weight, Y, M):
        check(lib().dj_matmul(self.h, ptr(X), w.h, ptr(Y), M))

    def matmul_glu(self, X, w: Weight, H, M, act=ACT_SILU):
        check(lib().dj_matmul_glu(self.h, ptr(X), w.h, ptr(H), M, act))

    def qk_norm_rope(self, T, heads, kv, D, stride, Z, qn, kn, vnorm, pos, pos_stride, eps, theta, rot=None, mode=ROPE_POW_NEG):
        check(lib().dj_qk_norm_rope(self.h, T, heads, kv, D, stride, ptr(Z), ptr(qn), ptr(kn), 1 if vnorm else 0,
                                    ptr(pos), pos_stride, eps, theta, D if rot is None else rot, mode))

    def rope_table(self, T, pos, pos_stride, theta, rot, tab, mode=ROPE_POW_NEG):
        check(lib().dj_rope_table(self.h, T, ptr(pos), pos_stride, theta, rot, mode, ptr(tab)))

    def matmul_qkv_rope(self, X, w: Weight, Z, M, heads, kv, D, qn, kn, vnorm, pos, pos_stride, eps, theta, tab, rot=None,
                        mode=ROPE_POW_NEG):
        check(lib().dj_matmul_qkv_rope(self.h, ptr(X), w.h, ptr(Z), M, heads, kv, D, ptr(qn), ptr(kn), 1 if vnorm else 0,
                                       ptr(pos), pos_stride, eps, theta, D if rot is None else rot, mode, ptr(tab)))

    def matmul_residual(self, X, w: Weight, M, R, nw, XW, SS):
        check(lib().dj_matmul_residual(self.h, ptr(X), w.h, M, ptr(R), ptr(nw), ptr(XW), ptr(SS)))

    def matmul_normed(self, XW, w: Weight, Y, M, act, SS, H, eps):
        """act: -1 plain, else a gated activation (ACT_*)."""
        check(lib().dj_matmul_normed(self.h, ptr(XW), w.h, ptr(Y), M, act, ptr(SS), H, eps))

    def matmul_qkv_rope_normed(self, XW, w: Weight, Z, M, heads, kv, D, qn, kn, vnorm, pos, pos_stride, eps, theta, tab,
                               SS, H, norm_eps, rot=None, mode=ROPE_POW_NEG):
        check(lib().dj_matmul_qkv_rope_normed(self.h, ptr(XW), w.h, ptr(Z), M, heads, kv, D, ptr(qn), ptr(kn),
                                              1 if vnorm else 0, ptr(pos), pos_stride, eps, theta,
                                              D if rot is None else rot, mode, ptr(tab), ptr(SS), H, norm_eps))

    def attention(self, T, heads, kv, D, Q, q_stride, A: KVSrc, B: KVSrc, rng, scale, O):
        check(lib().dj_attention(self.h, T, heads, kv, D, ptr(Q), q_stride, A, B, ptr(rng), scale, ptr(O)))

    def attention_qk_rope(self, T, heads, kv, D, Q, q_stride, A: KVSrc, B: KVSrc, rng, scale, qn, kn, eps, tab, O,
                          rot=None):
        check(lib().dj_attention_qk_rope(self.h, T, heads, kv, D, ptr(Q), q_stride, A, B, ptr(rng), scale, ptr(qn),
                                         ptr(kn), eps, ptr(tab), D if rot is None else rot, ptr(O)))

    def attention_gated(self, T, heads, kv, D, Q, q_stride, A: KVSrc, B: KVSrc, rng, scale, G, g_stride, O):
        check(lib().dj_attention_gated(self.h, T, heads, kv, D, ptr(Q), q_stride, A, B, ptr(rng), scale, ptr(G),
                                       g_stride, ptr(O)))

    def gdn(self, T, nspans, spans, LH, stride, Z, conv_w, A_log, dt_bias, gnorm, eps, Y):
        check(lib().dj_gdn(self.h, T, nspans, ptr(spans), LH, stride, ptr(Z), ptr(conv_w), ptr(A_log), ptr(dt_bias),
                           ptr(gnorm), eps, ptr(Y)))

    def ple_mix(self, T, P, G, E, w, eps, O):
        check(lib().dj_ple_mix(self.h, T, P, ptr(G), ptr(E), ptr(w), eps, ptr(O)))

    def pool_project(self, T, S, H, N, X, seqs, W, out):
        check(lib().dj_pool_project(self.h, T, S, H, N, ptr(X), ptr(seqs), ptr(W), ptr(out)))

    def attention_noalloc(self, T, heads, kv, D, Q, q_stride, A: KVSrc, B: KVSrc, rng, scale, O):
        check(lib().dj_attention_noalloc(self.h, T, heads, kv, D, ptr(Q), q_stride, A, B, ptr(rng), scale, ptr(O)))

    def kv_store(self, T, kv, D, Z, stride, k_col, cache, row0):
        check(lib().dj_kv_store(self.h, T, kv, D, ptr(Z), stride, k_col, ptr(cache), row0))

    def leaf_logits(self, T, L, H, nIds, eps, X, leaves, w, ids, embed: Weight, out):
        check(lib().dj_leaf_logits(self.h, T, L, H, nIds, eps, ptr(X), ptr(leaves), ptr(w), ptr(ids), embed.h, ptr(out)))

    def add_rows(self, T, H, Xi, idx, E, rows, Xo):
        check(lib().dj_add_rows(self.h, T, H, ptr(Xi), ptr(idx), ptr(E), rows, ptr(Xo)))

    def bias_act(self, T, N, Y, b, act=0):
        check(lib().dj_bias_act(self.h, T, N, ptr(Y), ptr(b), act))

    def add_layernorm(self, T, H, add, eps, X, Y, w, b, O):
        check(lib().dj_add_layernorm(self.h, T, H, 1 if add else 0, eps, ptr(X), ptr(Y), ptr(w), ptr(b), ptr(O)))

    def gather_rows(self, M, H, T, X, rows, G):
        check(lib().dj_gather_rows(self.h, M, H, T, ptr(X), ptr(rows), ptr(G)))

    def score(self, M, H, Y, w, b, out):
        check(lib().dj_score(self.h, M, H, ptr(Y), ptr(w), ptr(b), ptr(out)))

    def short_conv(self, T, H, Z, w, taps, Y):
        check(lib().dj_short_conv(self.h, T, H, ptr(Z), ptr(w), ptr(taps), ptr(Y)))

    def readout(self, T, P, H, X, R, codes, pairs, out):
        check(lib().dj_readout(self.h, T, P, H, ptr(X), ptr(R), codes, ptr(pairs), ptr(out)))

    def mean_pool(self, T, S, H, X, seqs, out):
        check(lib().dj_mean_pool(self.h, T, S, H, ptr(X), ptr(seqs), ptr(out)))

    def dense_f32(self, M, inp, w: Weight, out):
        check(lib().dj_dense_f32(self.h, M, ptr(inp), w.h, ptr(out)))

    # ---- readback
    def snapshot(self, src, nbytes: int, dtype, shape) -> int:
        host = np.empty(shape, dtype=dtype)
        if host.nbytes != nbytes:
            raise ValueError("decision.js: snapshot shape does not match its byte count")
        check(lib().dj_rec_snapshot(self.h, ptr(src), nbytes, host.ctypes.data))
        self._snaps.append(host)
        return len(self._snaps) - 1

    def finish(self):
        h, self.h = self.h, None
        check(lib().dj_rec_finish(h))
        return self._snaps

    def abort(self):
        """Ends a recording that failed (dj_rec_abort): nothing more runs and the context is free for the next
        forward. Its own status is not raised: the error being handled is the one to report."""
        if self.h is not None:
            h, self.h = self.h, None
            lib().dj_rec_abort(h)

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        if exc_type is not None:
            self.abort()
        return False


def kv_src(buf, rows, stride, k_col, v_col) -> KVSrc:
    return KVSrc(ptr(buf), rows, stride, k_col, v_col)


def exported_symbols():
    """The dj_* functions include/dj.h declares (for the ABI test)."""
    return sorted(SIGNATURES)
