"""Seeded synthetic models in the decision.js format, shaped as the benchmark configurations.

Weights are N(0, 0.02) from numpy PCG64 with seed [0, crc32(tensor name)], quantized with fmt.quantize8 /
fmt.quantize4 (the exporters' encodings). Norm weights are 1.0 (an untrained model's init) unless
`norm_std` asks for 1 + N(0, norm_std) (the tests use that, so a wrong norm index cannot hide).
Layouts follow the exporters: fused qkv = [q; k; v] (export-3b.py:48), fused w13 = [w1; w3]
(export-3b.py:54) or gate|up (export-eg2.py:206), the tied embedding also read as the LM head (export-3b.py:34).
"""
import concurrent.futures as cf
import copy
import math
import os
import zlib

import numpy as np

from . import fmt

# The BASELINE.json configurations. Choices the configurations leave open are recorded in the config
# itself ("choices") and written to the manifest.
CONFIGS = {
    # Qwen3-0.6B-shaped causal decoder, q8 (the bench workload)
    "qwen3-0.6b-q8": dict(model="decoder", bits=8, layers=28, hidden=1024, intermediate=3072, heads=16, kv_heads=8,
                          head_dim=128, vocab=151936, eps=1e-6, rope_theta=1e6, qk_norm=True,
                          choices={"norm_weights": 1.0}),
    # Qwen2.5-3B-shaped causal decoder, q4. No QK-norm; theta and the absent qkv bias are choices.
    "qwen2.5-3b-q4": dict(model="decoder", bits=4, layers=36, hidden=2048, intermediate=11008, heads=16, kv_heads=2,
                          head_dim=128, vocab=151936, eps=1e-6, rope_theta=1e6, qk_norm=False,
                          choices={"norm_weights": 1.0, "rope_theta": "1e6 (not stated; Qwen2.5's)", "qkv_bias": "none"}),
    # ~0.8B q8 causal decoder for the shared-state case. QK-norm is a choice (Qwen3 family).
    "d3lite-0.8b-q8": dict(model="decoder", bits=8, layers=20, hidden=1536, intermediate=4608, heads=12, kv_heads=2,
                           head_dim=128, vocab=151936, eps=1e-6, rope_theta=1e6, qk_norm=True,
                           choices={"norm_weights": 1.0, "qk_norm": "yes (not stated)", "rope_theta": "1e6 (not stated)"}),
    # d3-lite's readout form (D3Engine.logits, d3-engine.ts:67-139) on attention-only layers of the configs[4]
    # shape: noncausal attention within each sequence (or trunk + question with a shared prefix), the final norm,
    # then code logits READOUT from an f32 [codes, hidden] matrix at each sequence's last token
    "d3-attn-0.8b-q8": dict(model="d3", bits=8, layers=20, hidden=1536, intermediate=4608, heads=12, kv_heads=2,
                            head_dim=128, vocab=151936, eps=1e-6, rope_theta=1e6, qk_norm=True,
                            codes=["A", "B", "C", "D", "E", "F", "G", "H"], temperature=1.0,
                            choices={"norm_weights": 1.0, "layers": "attention only (no Gated DeltaNet)"}),
    # d3-lite as shipped (D3Engine, d3-engine.ts; export-d3.py): a Qwen3.5-0.8B-shaped backbone, 18 Gated DeltaNet
    # layers and every fourth a gated attention layer with 256-dim heads (RoPE on the first 64 dims), the f32
    # code readout. The widths follow the published 803 MB q8 size (export-d3.py:56-60 names the keys); theta,
    # the gate parameters' ranges and the codes are choices.
    "d3-lite-q8": dict(model="d3", bits=8, layers=24, hidden=1024, intermediate=3584, heads=8, kv_heads=2, head_dim=256,
                       rotary_dim=64, vocab=248320, eps=1e-6, rope_theta=1e7,
                       layer_types=["full_attention" if i % 4 == 3 else "linear_attention" for i in range(24)],
                       linear_heads=16, linear_key_dim=128, linear_value_dim=128, conv_kernel=4, linear_rows=8320,
                       codes=["A", "B", "C", "D", "E", "F", "G", "H"], temperature=1.0,
                       choices={"norm_weights": 1.0, "rope_theta": "1e7 (not stated)",
                                "A_log": "log U(0.01, 1)", "dt_bias": "N(0, 0.5)", "conv taps": "N(0, 0.5)"}),
    # d1-3B's LFM2 backbone form (D13BEngine, d1-3b-engine.ts; export-3b.py): short-conv layers with attention
    # layers between them, 64-dim heads with q/k norm, q4 linears, f16 conv taps [H, 3]. Not a BASELINE config:
    # the layer pattern, widths and vocabulary are choices.
    "lfm2-d1-3b-q4": dict(model="d1-3b", bits=4, layers=30, hidden=2048, intermediate=8192, heads=32, kv_heads=8,
                          head_dim=64, vocab=65536, eps=1e-5, rope_theta=1e6, qk_norm=True,
                          layer_types=["full_attention" if i % 3 == 2 else "conv" for i in range(30)],
                          choices={"norm_weights": 1.0, "layer_types": "attention every third layer (not stated)",
                                   "intermediate": "8192 (not stated)", "vocab": "65536 (not stated)"}),
    # d1-omni's form (D1OmniEngine, omni-engine.ts; export-omni.py): a bidirectional LFM2 trunk shaped like
    # LFM2-350M (its published q8 size, 405 MB with the head, fits this shape) and the marker head. Not a BASELINE
    # config: the layer pattern, widths, head sizes and temperatures are choices.
    "d1-omni-q8": dict(model="d1-omni", bits=8, layers=16, hidden=1024, intermediate=4608, heads=16, kv_heads=8,
                       head_dim=64, vocab=65536, eps=1e-5, rope_theta=1e6, qk_norm=True,
                       layer_types=["conv", "conv", "full_attention", "conv", "conv", "full_attention", "conv", "conv",
                                    "full_attention", "conv", "full_attention", "conv", "full_attention", "conv",
                                    "full_attention", "conv"],
                       head_layers=2, head_heads=16, head_ff=4096, ln_eps=1e-5, max_length=16384,
                       temperatures={"choice": 1.1, "score": 0.9, "noul": 1.2, "choice:2": 1.05, "choice:3-5": 1.15,
                                     "score:6-10": 0.8, "noul:2": 1.25},
                       choices={"norm_weights": 1.0, "layer_types": "LFM2-350M's pattern (not stated)",
                                "head": "2 layers, 16 heads, ff 4096 (not stated)", "biases": "N(0, 0.1)",
                                "type_emb": "N(0, 0.5)", "temperatures": "synthetic"}),
    # EmbeddingGemma 2 as shipped (Eg2Engine, eg2-engine.ts; export-eg2.py): a 24-layer bidirectional Gemma text
    # encoder at hidden 512 with per-layer embeddings (PLE_MIX's 512-wide rows), 256-dim heads on the sliding
    # layers (a +-512-token window) and 512-dim heads on every sixth (global) layer, the f16 embedding projection
    # after mean pooling, and the learned decision head on the host. Heads, widths, thetas, the projection width
    # and the head width are choices (export-eg2.py writes them from the checkpoint).
    "eg2-q8": dict(model="eg2", bits=8, layers=24, hidden=512, intermediate=2048, heads=4, vocab=262144, eps=1e-6,
                   layer_types=["full_attention" if i % 6 == 5 else "sliding_attention" for i in range(24)], window=512,
                   head_dim={"sliding_attention": 256, "full_attention": 512},
                   kv_heads={"sliding_attention": 1, "full_attention": 1},
                   rope_theta={"sliding_attention": 1e4, "full_attention": 1e6}, ple=512, embedding_dim=768,
                   embed_dim=768, learned_head={"width": 256},
                   choices={"norm_weights": 1.0, "heads": "4 query / 1 kv per layer type (not stated)",
                            "intermediate": "2048 (not stated)", "rope_theta": "1e4 sliding, 1e6 global (not stated)",
                            "embedding_dim": "768 (not stated)", "layer_scalars": 1.0}),
    # Laya as shipped (LayaEngine, laya-engine.ts; export-laya.py): a ModernBERT-large-shaped encoder (bias-free
    # LayerNorms, RoPE, every third layer global and the others a +-64-token window, GeGLU with the erf GELU) and
    # d1-omni's decision head. The head sizes and temperatures are choices.
    "laya-q8": dict(model="laya", bits=8, layers=28, hidden=1024, intermediate=2624, heads=16, vocab=50368, eps=1e-5,
                    layer_types=["full_attention" if i % 3 == 0 else "sliding_attention" for i in range(28)], window=64,
                    rope_theta={"full_attention": 160000.0, "sliding_attention": 10000.0},
                    head_layers=2, head_heads=16, head_ff=4096, ln_eps=1e-5, max_len=512, head_max_len=192,
                    temperatures={"choice": 1.1, "score": 0.9, "noul": 1.2, "choice:3-5": 1.15},
                    choices={"norm_weights": 1.0, "head": "2 layers, 16 heads, ff 4096 (not stated)",
                             "biases": "N(0, 0.1)", "type_emb": "N(0, 0.5)", "temperatures": "synthetic"}),
    # EmbeddingGemma-shaped bidirectional encoder, q8, mean-pool + 768->3072->768 head
    "eg2-encoder-q8": dict(model="encoder", bits=8, layers=24, hidden=768, intermediate=1152, heads=3, kv_heads=1,
                           head_dim=256, vocab=262144, eps=1e-6, rope_theta=1e4, head_width=3072, embed_dim=768,
                           choices={"norm_weights": 1.0, "rope_theta": "1e4 (not stated)",
                                    "embed_scale": "sqrt(hidden) folded into the embedding (export-eg2.py:100)",
                                    "head": "Linear 768->3072, Linear 3072->768, no activation, q8, f32 on the GPU",
                                    "attention_scale": 1.0, "layer_scalars": 1.0, "window": "none (all layers global)"}),
}


def reduced(name: str, **over) -> dict:
    """A configuration with some fields replaced (tests use fewer layers and a smaller vocabulary)."""
    c = copy.deepcopy(CONFIGS[name])
    c.update(over)
    return c


def _rng(name: str, seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed, zlib.crc32(name.encode())]))


def normal(name: str, shape, std: float = 0.02, seed: int = 0) -> np.ndarray:
    return (_rng(name, seed).standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def _norm(name, n, norm_std, seed):
    if not norm_std:
        return np.ones(n, dtype=np.float32)
    return 1.0 + normal(name, (n,), norm_std, seed)


def tensor_plan(cfg: dict):
    """[(name, kind, shape)] of a configuration: kind q (quantized linear) or n (norm weight)."""
    if cfg["model"] == "eg2":
        return _eg2_plan(cfg)
    if cfg["model"] == "laya":
        return _laya_plan(cfg)
    H, I, h, kv, D, V, L = (cfg[k] for k in ("hidden", "intermediate", "heads", "kv_heads", "head_dim", "vocab", "layers"))
    plan = [("embed", "q", (V, H))]
    if cfg["model"] == "d3" and "linear_heads" in cfg:  # d3-lite as exported (export-d3.py:66-102)
        LH, QK, A = cfg["linear_heads"], cfg["linear_heads"] * 128, (2 * h + 2 * kv) * D
        plan += [("final_norm", "n", (H,)), ("readout", "r", (len(cfg["codes"]), H))]
        for i, t in enumerate(cfg["layer_types"]):
            p = f"layers.{i}."
            plan += [(p + "input_norm", "n", (H,)), (p + "post_norm", "n", (H,)), (p + "w13", "q", (2 * I, H)),
                     (p + "w2", "q", (H, I))]
            if t == "linear_attention":
                plan += [(p + "in", "q", (cfg["linear_rows"], H)), (p + "conv", "c", (3 * QK, 4)),
                         (p + "A_log", "alog", (LH,)), (p + "dt_bias", "b5", (LH,)), (p + "gnorm", "n", (128,)),
                         (p + "out", "q", (H, QK))]
            else:
                plan += [(p + "qkvg", "q", (A, H)), (p + "q_norm", "n", (D,)), (p + "k_norm", "n", (D,)),
                         (p + "o", "q", (H, h * D))]
    elif cfg["model"] in ("decoder", "d3", "d1-3b", "d1-omni"):
        plan.append(("final_norm", "n", (H,)))
        types = cfg.get("layer_types") or ["full_attention"] * L
        for i in range(L):
            p = f"layers.{i}."
            plan += [(p + "operator_norm", "n", (H,)), (p + "ffn_norm", "n", (H,)), (p + "w13", "q", (2 * I, H)),
                     (p + "w2", "q", (H, I))]
            if types[i] == "conv":  # LFM2 short conv (export-3b.py: in_proj, out_proj, conv taps [H, 3])
                plan += [(p + "in_proj", "q", (3 * H, H)), (p + "out_proj", "q", (H, H)), (p + "conv", "c", (H, 3))]
                continue
            plan += [(p + "qkv", "q", ((h + 2 * kv) * D, H)), (p + "o_proj", "q", (H, h * D))]
            if cfg.get("qk_norm"):
                plan += [(p + "q_norm", "n", (D,)), (p + "k_norm", "n", (D,))]
        if cfg["model"] == "d3":
            plan.append(("readout", "r", (len(cfg["codes"]), H)))  # f32 code matrix (d3-kernels.ts:242-260)
        if cfg["model"] == "d1-omni":  # the decision head and scorer (export-omni.py:70-90)
            plan += _marker_head_plan(cfg)
    else:
        for i in range(L):
            p = f"layers.{i}."
            plan += [(p + "qkv", "q", ((h + 2 * kv) * D, H)), (p + "q_norm", "n", (D,)), (p + "k_norm", "n", (D,)),
                     (p + "o", "q", (H, h * D)), (p + "gu", "q", (2 * I, H)), (p + "down", "q", (H, I))]
            for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm", "post_feedforward_layernorm"):
                plan.append((p + n, "n", (H,)))
        plan += [("final_norm", "n", (H,)), ("head.dense1", "q", (cfg["head_width"], H)),
                 ("head.dense2", "q", (cfg["embed_dim"], cfg["head_width"]))]
    return plan


def _marker_head_plan(cfg: dict):
    """d1-omni's decision head and scorer (export-omni.py:70-90, export-laya.py:80-101)."""
    H, F = cfg["hidden"], cfg["head_ff"]
    plan = [("head.type_emb", "e", (3, H))]
    for i in range(cfg["head_layers"]):
        p = f"head.{i}."
        plan += [(p + "in_proj", "q", (3 * H, H)), (p + "in_proj_bias", "b", (3 * H,)),
                 (p + "out_proj", "q", (H, H)), (p + "out_proj_bias", "b", (H,)),
                 (p + "linear1", "q", (F, H)), (p + "linear1_bias", "b", (F,)),
                 (p + "linear2", "q", (H, F)), (p + "linear2_bias", "b", (H,))]
        for nm in ("norm1", "norm2"):
            plan += [(p + nm, "n", (H,)), (p + nm + "_bias", "b", (H,))]
    plan += [("scorer.norm", "n", (H,)), ("scorer.norm_bias", "b", (H,)), ("scorer.fc", "q", (H, H)),
             ("scorer.fc_bias", "b", (H,)), ("scorer.out", "v", (H,)), ("scorer.out_bias", "s", (2,))]
    return plan


def _laya_plan(cfg: dict):
    """Laya's encoder (export-laya.py:70-79: no attention norm on layer 0) and the marker head."""
    H, I, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    plan = [("embed", "q", (V, H)), ("embed_norm", "n", (H,)), ("final_norm", "n", (H,))]
    for i in range(cfg["layers"]):
        p = f"layers.{i}."
        if i > 0:
            plan.append((p + "attn_norm", "n", (H,)))
        plan += [(p + "mlp_norm", "n", (H,)), (p + "qkv", "q", (3 * H, H)), (p + "o", "q", (H, H)),
                 (p + "wi", "q", (2 * I, H)), (p + "wo", "q", (H, I))]
    return plan + _marker_head_plan(cfg)


def _eg2_plan(cfg: dict):
    """The shipped EmbeddingGemma 2 layout (export-eg2.py:92-118)."""
    H, I, h, V, L, P = (cfg[k] for k in ("hidden", "intermediate", "heads", "vocab", "layers", "ple"))
    plan = [("embed", "q", (V, H)), ("ple.norm", "n", (P,)), ("final_norm", "n", (H,)),
            ("projection", "v", (cfg["embedding_dim"], H))]
    for i, t in enumerate(cfg["layer_types"]):
        p, D, kv = f"layers.{i}.", cfg["head_dim"][t], cfg["kv_heads"][t]
        plan += [(p + "ple_in", "q", (P, H)), (p + "qkv", "q", ((h + 2 * kv) * D, H)), (p + "q_norm", "n", (D,)),
                 (p + "k_norm", "n", (D,)), (p + "o", "q", (H, h * D)), (p + "gu", "q", (2 * I, H)), (p + "down", "q", (H, I)),
                 (p + "ple_gate", "q", (P, H)), (p + "ple_proj", "q", (H, P)), (p + "ple_norm", "n", (H,))]
        plan += [(p + n, "n", (H,)) for n in ("input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                                                  "post_feedforward_layernorm")]
    return plan


def head_plan(cfg: dict):
    """[(name, shape)] of the learned EmbeddingGemma 2 decision head (eg2-head.ts:64-99) on embed_dim inputs:
    state/question/option projections, the field MLP, the type embedding, two LayerNorms and the residual MLP."""
    W, E = cfg["learned_head"]["width"], cfg["embed_dim"]
    plan = []
    for p in ("state_proj", "question_proj", "option_proj"):
        plan += [(f"head.{p}.weight", (W, E)), (f"head.{p}.bias", (W,))]
    plan += [("head.field.0.weight", (W, 3 * W)), ("head.field.0.bias", (W,)), ("head.field.3.weight", (W, W)),
             ("head.field.3.bias", (W,)), ("head.type_emb.weight", (3, W)),
             ("head.field_norm.weight", (W,)), ("head.field_norm.bias", (W,)),
             ("head.option_norm.weight", (W,)), ("head.option_norm.bias", (W,)),
             ("head.residual.0.weight", (W, 4 * W)), ("head.residual.0.bias", (W,)), ("head.residual.3.weight", (1, W))]
    return plan


def manifest_config(cfg: dict) -> dict:
    c = {k: v for k, v in cfg.items() if k not in ("bits",)}
    if cfg["model"] == "eg2":  # export-eg2.py:68-80's keys
        c["layer_scalars"] = list(cfg.get("layer_scalars", [1.0] * cfg["layers"]))
        c.setdefault("prompt", "")
        c.setdefault("max_len", 8192)
        lh = c.pop("learned_head")
        c["question_types"] = ["choice", "score", "noul"]
        c["temperatures"] = dict(lh.get("temperatures", {"choice": 1.0, "score": 1.0, "noul": 1.0}))
        c["head"] = {"width": lh["width"], "ln_eps": 1e-5, "prior_scale": lh.get("prior_scale", 2.0),
                     "joint_scale": lh.get("joint_scale", 5.0), "gate": lh.get("gate", 0.6),
                     "residual_bias": lh.get("residual_bias", 0.1)}
        return c
    c["layer_types"] = list(cfg.get("layer_types") or ["full_attention"] * cfg["layers"])
    if cfg["model"] in ("decoder", "d3", "d1-3b", "d1-omni", "laya"):
        c["model"] = cfg["model"]
    else:
        c["model"] = "eg2-encoder"
        c["layer_scalars"] = [1.0] * cfg["layers"]
        c["attention_scale"] = 1.0
        c["embed_scale"] = math.sqrt(cfg["hidden"])
        lh = cfg.get("learned_head")
        if lh:  # the typed-decision head's scalars (export-eg2.py:80-84)
            c["question_types"] = ["choice", "score", "noul"]
            c["temperatures"] = dict(lh.get("temperatures", {"choice": 1.0, "score": 1.0, "noul": 1.0}))
            c["head"] = {"width": lh["width"], "ln_eps": 1e-5, "prior_scale": lh.get("prior_scale", 2.0),
                         "joint_scale": lh.get("joint_scale", 5.0), "gate": lh.get("gate", 0.6),
                         "residual_bias": lh.get("residual_bias", 0.1)}
            del c["learned_head"]
    return c


def _make(cfg, name, kind, shape, seed, norm_std, std):
    if kind == "n":
        return name, kind, _norm(name, shape[0], norm_std, seed), None
    if kind == "r":  # an f32 readout matrix, N(0, std)
        return name, kind, normal(name, shape, std, seed), None
    if kind == "c":  # f16 conv taps, N(0, 0.5): each tap moves its channel by about as much as the others
        return name, kind, normal(name, shape, 0.5, seed), None
    if kind == "alog":  # log of the DeltaNet decay rates, log U(0.01, 1): per-token decays of ~0.3 to ~1
        return name, kind, np.log(0.01 + 0.99 * _rng(name, seed).random(shape, dtype=np.float32)), None
    if kind == "b5":  # f16 biases, N(0, 0.5)
        return name, kind, normal(name, shape, 0.5, seed), None
    if kind == "b":  # f16 biases, N(0, 0.1)
        return name, kind, normal(name, shape, 0.1, seed), None
    if kind == "e":  # the f16 question-type rows, N(0, 0.5): each type moves the head's input visibly
        return name, kind, normal(name, shape, 0.5, seed), None
    if kind == "v":  # an f16 weight row (the scorer's last Linear(H, 1)), N(0, std)
        return name, kind, normal(name, shape, std, seed), None
    if kind == "s":  # the scorer's bias and a zero half (export-omni.py:90: one aligned word)
        return name, kind, np.array([normal(name, (1,), 0.1, seed)[0], 0.0], dtype=np.float32), None
    w = normal(name, shape, std, seed)
    if name == "embed" and cfg["model"] in ("encoder", "eg2"):
        w = w * np.float32(math.sqrt(cfg["hidden"]))  # Gemma's sqrt(hidden) embedding scale, folded in
    q = fmt.quantize8(w) if cfg["bits"] == 8 else fmt.quantize4(w)
    return name, kind, q[0], q[1]


def generate(cfg: dict, out: str, seed: int = 0, norm_std: float = 0.0, threads: int = 8, std: float = 0.02) -> str:
    """Writes manifest.json + weights.bin for `cfg` under `out`; returns `out`. Skips the work when a
    manifest with the same configuration and seed already exists there. `std` is the linear and embedding
    weights' standard deviation (the configurations' 0.02; tiny test models use ~1/sqrt(hidden) so that every
    layer's branches move the residual stream as much as the embedding does)."""
    mc = manifest_config(cfg)
    mc["synthetic"] = {"seed": seed, "norm_std": norm_std}
    if std != 0.02:
        mc["synthetic"]["std"] = std
    if os.path.exists(os.path.join(out, "manifest.json")):
        try:
            if fmt.load_manifest(out)["config"] == mc:
                return out
        except Exception:  # noqa: BLE001 (a broken earlier write: regenerate)
            pass
    blob = fmt.Blob(out, mc, cfg["bits"])
    plan = tensor_plan(cfg)
    with cf.ThreadPoolExecutor(max_workers=threads) as ex:
        futs = [ex.submit(_make, cfg, n, k, s, seed, norm_std, std) for n, k, s in plan]
        for (name, kind, shape), fut in zip(plan, futs):
            _, _, a, b = fut.result()
            if kind in ("n", "c", "b", "e", "v", "s", "alog", "b5"):
                blob.f16(name, a)
            elif kind == "r":
                blob.f32(name, a)
            else:
                blob.put_quant(name, a, b, shape, cfg["bits"])
    if cfg["model"] in ("encoder", "eg2") and cfg.get("learned_head"):
        # f32 host tensors; LayerNorm weights around 1, everything else N(0, 1/sqrt(fan-in))
        for name, shape in head_plan(cfg):
            if name.endswith("norm.weight"):
                blob.host_f32(name, 1.0 + normal(name, shape, 0.1, seed))
            else:
                blob.host_f32(name, normal(name, shape, 1.0 / math.sqrt(shape[-1]), seed))
    blob.close({"repo": "synthetic", "revision": None, "seed": seed})
    return out
