"""The weights format of decision.js, unchanged: manifest.json + weights.bin.

Writer: the `Blob` of scripts/export_common.py:17-61 — tensors appended to weights.bin at 256-byte aligned
offsets; manifest {"format": "d1.js/1", "config", "tensors": {name: TensorInfo}, "bytes", "source"}, where
TensorInfo (gpu.ts:6) is {dtype: q4|q8|f16|f32, shape, offset, bytes[, scales, scales_bytes]}.
Quantizers: quantize8 (export_common.py:90-97) and quantize4 (export_common.py:64-87), restated in numpy.
Reader: `load_manifest` / `TensorFile` read what loadWeights fetches by Range requests (gpu.ts:57-88).
"""
import json
import os

import numpy as np

BLOCK = 32
FORMAT = "d1.js/1"


def quantize8(w: np.ndarray):
    """q8: scale = f16(absmax / 127) per 32-block (1 for an all-zero block), code = clamp(round(w / scale),
    -127, 127) + 128 (export_common.py:90-97). Returns (codes u8 [N, K], scales f16 [N, K/32], dequantized f32)."""
    n, k = w.shape
    blocks = np.asarray(w, dtype=np.float32).reshape(n, k // BLOCK, BLOCK)
    scale = (np.abs(blocks).max(-1) / np.float32(127)).astype(np.float16).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1), scale)
    codes = np.clip(np.round(blocks / scale[..., None]), -127, 127)
    deq = (codes * scale[..., None]).reshape(n, k)
    return (codes + 128).astype(np.uint8).reshape(n, k), scale.astype(np.float16), deq


def _linspace_f32(start: float, end: float, steps: int) -> np.ndarray:
    """torch.linspace(start, end, steps) in float32 (the candidates of export_common.py:72): step = (end -
    start) / (steps - 1) in f32; fma(step, i, start) for the first steps // 2 values and fma(-step, steps-1-i,
    end) for the rest, each rounded once (torch's CPU kernel). The fma is emulated exactly in float64."""
    st, en = np.float32(start), np.float32(end)
    step = np.float32((en - st) / np.float32(steps - 1))
    half = steps // 2
    out = np.empty(steps, dtype=np.float32)
    for i in range(steps):
        if i < half:
            out[i] = np.float32(np.float64(step) * i + np.float64(st))
        else:
            out[i] = np.float32(-np.float64(step) * (steps - 1 - i) + np.float64(en))
    return out


def quantize4(w: np.ndarray, rows: int = 8192):
    """q4: per 32-block, the scale among 46 candidates f16(absmax * f / d), f in linspace(0.6, 1.15, 23),
    d in (7, 8), with the least squared error; codes clamp(round(w / scale), -8, 7) + 8, two per byte, low
    nibble first (export_common.py:64-87). Returns (codes u8 [N, K/2], scales f16 [N, K/32], dequantized f32)."""
    if w.shape[0] > rows:
        parts = [quantize4(w[i:i + rows]) for i in range(0, w.shape[0], rows)]
        return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts]), np.concatenate([p[2] for p in parts])
    n, k = w.shape
    blocks = np.asarray(w, dtype=np.float32).reshape(n, k // BLOCK, BLOCK)
    amax = np.maximum(np.abs(blocks).max(-1), np.float32(1e-12))
    best_codes = best_scale = err = None
    for f in _linspace_f32(0.6, 1.15, 23):
        for d in (np.float32(7.0), np.float32(8.0)):
            scale = (amax * f / d).astype(np.float16).astype(np.float32)
            scale = np.where(scale == 0, np.float32(1), scale)
            codes = np.clip(np.round(blocks / scale[..., None]), -8, 7)
            e = ((codes * scale[..., None] - blocks) ** 2).sum(-1, dtype=np.float32)
            if err is None:
                best_codes, best_scale, err = codes, scale, e
            else:
                better = e < err
                best_codes = np.where(better[..., None], codes, best_codes)
                best_scale = np.where(better, scale, best_scale)
                err = np.minimum(e, err)
    deq = (best_codes * best_scale[..., None]).reshape(n, k)
    codes = (best_codes + 8).astype(np.uint8).reshape(n, k)
    return (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8), best_scale.astype(np.float16), deq


class Blob:
    """weights.bin + manifest.json writer (export_common.py:17-61), without the tokenizer copy (the synthetic
    models have no tokenizer)."""

    def __init__(self, out: str, config: dict, bits: int):
        os.makedirs(out, exist_ok=True)
        self.out, self.bits, self.offset = out, bits, 0
        self.f = open(os.path.join(out, "weights.bin"), "wb")
        self.manifest = {"format": FORMAT, "config": config, "tensors": {}}

    def put(self, raw: bytes) -> int:
        pad = (-self.offset) % 256
        self.f.write(b"\0" * pad)
        self.offset += pad
        start = self.offset
        self.f.write(raw)
        self.offset += len(raw)
        return start

    def quant(self, name: str, w: np.ndarray, bits: int = None) -> np.ndarray:
        bits = bits or self.bits
        codes, scales, deq = (quantize8 if bits == 8 else quantize4)(w)
        self.put_quant(name, codes, scales, list(w.shape), bits)
        return deq

    def put_quant(self, name: str, codes: np.ndarray, scales: np.ndarray, shape, bits: int):
        self.manifest["tensors"][name] = {"dtype": f"q{bits}", "shape": list(shape), "offset": self.put(codes.tobytes()),
                                          "bytes": codes.nbytes, "scales": self.put(scales.tobytes()), "scales_bytes": scales.nbytes}

    def f16(self, name: str, t: np.ndarray):
        a = np.asarray(t, dtype=np.float32).astype(np.float16)
        self.manifest["tensors"][name] = {"dtype": "f16", "shape": list(a.shape), "offset": self.put(a.tobytes()), "bytes": a.nbytes}

    def f32(self, name: str, t: np.ndarray):
        a = np.asarray(t, dtype=np.float32)
        self.manifest["tensors"][name] = {"dtype": "f32", "shape": list(a.shape), "offset": self.put(a.tobytes()), "bytes": a.nbytes}

    def host_f32(self, name: str, t: np.ndarray):
        """An f32 tensor read on the host, listed under the manifest's "host" (export-eg2.py:122-125: the
        EmbeddingGemma 2 decision head)."""
        self.f32(name, t)
        self.manifest.setdefault("host", {})[name] = self.manifest["tensors"].pop(name)

    def close(self, source: dict = None):
        self.f.close()
        self.manifest["bytes"] = self.offset
        self.manifest["source"] = source or {"repo": "synthetic", "revision": None}
        with open(os.path.join(self.out, "manifest.json"), "w") as f:
            json.dump(self.manifest, f)


def load_manifest(base: str) -> dict:
    with open(os.path.join(base, "manifest.json")) as f:
        m = json.load(f)
    if m.get("format") != FORMAT:
        raise ValueError(f"decision.js: {base}manifest.json is not a {FORMAT} manifest")
    return m


class TensorFile:
    """Byte ranges of weights.bin, as the reference's Range reads (gpu.ts:63-66), over a memory map."""

    def __init__(self, base: str):
        self.path = os.path.join(base, "weights.bin")
        self.mm = np.memmap(self.path, dtype=np.uint8, mode="r")

    def range(self, offset: int, nbytes: int) -> np.ndarray:
        data = self.mm[offset:offset + nbytes]
        if data.nbytes != nbytes:
            raise ValueError(f"decision.js: range read returned {data.nbytes} bytes, wanted {nbytes}")
        return data

    def tensor(self, info: dict):
        """(codes, scales) for q4/q8, else the array itself."""
        dt = info["dtype"]
        if dt in ("q4", "q8"):
            N, K = info["shape"]
            codes = self.range(info["offset"], info["bytes"])
            scales = self.range(info["scales"], info["scales_bytes"]).view(np.float16)
            return codes.reshape(N, -1), scales.reshape(N, K // BLOCK)
        raw = self.range(info["offset"], info["bytes"])
        return raw.view(np.float16 if dt == "f16" else np.float32).reshape(info["shape"])
