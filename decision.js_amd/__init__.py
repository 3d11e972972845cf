"""decision.js on MI355X: the scoring path of decision.js (Jacqkues/decision.js) on hand-written gfx950 HIP
kernels behind the C ABI of include/dj.h.

The directory name holds a dot, so Python imports it under the module name `decision_js_amd` through
`load()` below (tests, bench.py and __graft_entry__.py do this).

Modules
  _dj        ctypes binding of libdj.so (device, buffers, weights, recorder, ops)        ~ src/gpu.ts
  fmt        manifest.json + weights.bin reader/writer, quantize8 / quantize4            ~ scripts/export_common.py
  synth      seeded synthetic models shaped as the benchmark configurations
  engine     GpuEngine + the causal decoder engine (forest packing, shared-state KV)     ~ src/gpu.ts, d1-3b-engine.ts, d3-engine.ts
  encoder    the EmbeddingGemma-shaped encoder engine (configs[0] form)                   ~ src/eg2-engine.ts
  eg2        EmbeddingGemma 2 on its shipped layout (per-layer embeddings)                ~ src/eg2-engine.ts
  eg2_head   the learned EmbeddingGemma 2 decision head on the host                       ~ src/eg2-head.ts
  omni       d1-omni: bidirectional LFM2 trunk + marker head                              ~ src/omni-engine.ts
  laya       Laya: ModernBERT encoder + d1-omni's marker head                             ~ src/laya-engine.ts
  d3         d3-lite on its shipped layout (Gated DeltaNet + gated attention)             ~ src/d3-engine.ts
  questions  checkQuestion / answer                                                       ~ src/questions.ts
  d1         the Decision API (load, systemOne, systemOneBatch, probabilities)           ~ src/d1.ts
"""
import importlib.util
import os
import sys

NAME = "decision_js_amd"
PKG_DIR = os.path.dirname(os.path.abspath(__file__))


def load():
    """Imports this directory as the package `decision_js_amd` (idempotent) and returns it."""
    if NAME in sys.modules:
        return sys.modules[NAME]
    spec = importlib.util.spec_from_file_location(NAME, os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[NAME] = mod
    spec.loader.exec_module(mod)
    return mod
