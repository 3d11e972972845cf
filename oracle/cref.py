"""ctypes access to oracle/_build/liboracle.so, the C restatement (test infrastructure only)."""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")


def lib():
    L = C.CDLL(LIB)
    L.o_f32_to_f16.argtypes = [C.c_float]
    L.o_f32_to_f16.restype = C.c_uint16
    L.o_f16_to_f32.argtypes = [C.c_uint16]
    L.o_f16_to_f32.restype = C.c_float
    L.o_dequant.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
    L.o_quantize8.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    L.o_pack_forest.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.POINTER(C.c_int)]
    L.o_pack_forest.restype = C.c_int
    return L


def dequant(codes, scales, N, K, bits):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scales = np.ascontiguousarray(scales).view(np.uint16)
    out = np.empty((N, K), dtype=np.uint16)
    lib().o_dequant(codes.ctypes.data, scales.ctypes.data, N, K, bits, out.ctypes.data)
    return out.view(np.float16)


def quantize8(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    codes = np.empty((N, K), dtype=np.uint8)
    scales = np.empty((N, K // 32), dtype=np.uint16)
    lib().o_quantize8(w.ctypes.data, N, K, codes.ctypes.data, scales.ctypes.data)
    return codes, scales.view(np.float16)


def pack_forest(trees):
    tr = np.array([(len(t["trunk"]), len(t["branches"])) for t in trees], dtype=np.int32).reshape(-1)
    tok = np.array([x for t in trees for x in t["trunk"] + [y for b in t["branches"] for y in b]], dtype=np.uint32)
    blen = np.array([len(b) for t in trees for b in t["branches"]] or [0], dtype=np.int32)
    T = len(tok)
    ids, pos = np.empty(max(T, 1), np.uint32), np.empty(max(T, 1), np.int32)
    meta = np.empty((max(T, 1), 4), np.int32)
    leaves = np.empty(max(len(blen), 1), np.uint32)
    L = C.c_int()
    n = lib().o_pack_forest(len(trees), tr.ctypes.data, tok.ctypes.data, blen.ctypes.data, ids.ctypes.data, pos.ctypes.data,
                            meta.ctypes.data, leaves.ctypes.data, C.byref(L))
    return ids[:n], pos[:n], meta[:n], leaves[:L.value]
