"""Benchmark of the scoring path on one MI355X: decisions/s on 3-question tickets, p50 ms per ticket.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config qwen3-0.6b-q8] [--no-graphs] [--no-cpu]

Workload: the Qwen3-0.6B-shaped causal decoder, q8 per-32 groups, seeded
N(0, 0.02) weights; a ticket is 3 questions, each a 384-token prompt of random ids, packed as 3 sequences in
one forward; answer-set logits (sizes 2, 3, 5) at each sequence's last token, then softmax. A step is one
ticket. Its packed inputs are staged in HBM before the timed region; a step copies them into the engine's
buffers (device to device), runs the forward (a replayed HIP graph) and reads the 10 logits back.

The JSON line also carries:
  roofline      the dominant kernel (by GPU time in a profiled pass of the same tickets, HIP events around
                every op) against f16 dense MFMA peak: algorithmic FLOPs per launch (2 M N K) / its launch
                time, timed alone — the model's own weight, 50 launches in one HIP graph replayed between two
                HIP events on the engine's stream; traffic = HBM bytes per launch from the FETCH_SIZE and
                WRITE_SIZE counters (profiles/traffic.json, when it names the same kernel)
  cpu_baseline  the oracle (oracle/ref.py, numpy on the host cores) on one ticket of the same workload
  north_star    the two targets on their own workloads: configs[3]'s batched prefill GEMMs against dense f16
                peak, configs[4]'s single 32-token question against HBM bandwidth
  cpu_reference_probe  whether the reference's own CPU path (WGSL via Node WebGPU on lavapipe) can run here
"""
import argparse
import json
import math
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense f16 (no sparsity)
HBM_PEAK_GBS = 8000.0
METRIC = "decisions/sec (3-question tickets) on 1 MI355X; p50 ms per ticket"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def load_pkg():
    sys.path.insert(0, ROOT)
    import importlib.util
    name = "decision_js_amd"
    if name in sys.modules:
        return sys.modules[name]
    d = os.path.join(ROOT, "decision.js_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(d, "__init__.py"), submodule_search_locations=[d])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def make_tickets(n, V, seq_len=384, seed=1, answer_seed=3, sizes=(2, 3, 5)):
    """n tickets of 3 questions: token ids from PCG64 seed 1, answer sets (distinct ids) from seed 3."""
    ids_rng = np.random.Generator(np.random.PCG64(seed))
    ans_rng = np.random.Generator(np.random.PCG64(answer_seed))
    tickets = []
    for _ in range(n):
        trees = []
        for q in range(3):
            ans = ans_rng.choice(V, size=sizes[q], replace=False)
            trees.append({"trunk": [], "branches": [[int(x) for x in ids_rng.integers(0, V, seq_len)]],
                          "groups": [[[int(a)] for a in ans]]})
        tickets.append(trees)
    return tickets


def model_flops_bytes(c, T, seqs_len, causal=True, markers=0):
    """Appendix-B algorithmic work of one forward: 2 T sum(N K) over the linears plus 4 D h (allowed
    query-key pairs) per attention layer; bytes = quantized linear weights + gathered embedding rows. LFM2 conv
    layers count in_proj (3H x H) and out_proj (H x H); Laya's sliding layers count the pairs within their
    window; a d1-omni / Laya head counts its layers' in_proj (3H x H), out_proj, linear1/linear2 on every token
    and bidirectional attention, and the scorer's H x H product on `markers` rows."""
    H, I, h = c["hidden"], c["intermediate"], c["heads"]
    kv, D = c.get("kv_heads", h), c.get("head_dim", H // h)  # Laya: full-width heads
    types = c.get("layer_types") or ["full_attention"] * c["layers"]
    attn_nk, conv_nk, ffn_nk = (h + 2 * kv) * D * H + H * h * D, 4 * H * H, 2 * I * H + H * I
    nk = sum(conv_nk if t == "conv" else attn_nk for t in types) + len(types) * ffn_nk
    pairs = sum(n * (n + 1) // 2 if causal else n * n for n in seqs_len)
    w = c.get("window")
    # Laya's local layers: each token sees the keys within +-window of it in its sequence
    win_pairs = sum(sum(min(n, t + w + 1) - max(0, t - w) for t in range(n)) for n in seqs_len) if w else pairs
    flops = 2 * T * nk + 4 * D * h * sum(win_pairs if t == "sliding_attention" else pairs for t in types if t != "conv")
    wnk = nk
    if c.get("head_layers"):
        hl, ff = c["head_layers"], c["head_ff"]
        head_nk = hl * (4 * H * H + 2 * ff * H)
        bidir = sum(n * n for n in seqs_len)
        flops += 2 * T * head_nk + 4 * H * bidir * hl + 2 * markers * H * H
        wnk += head_nk + H * H
    qbytes = 1.0625 if c.get("bits", 8) == 8 else 0.5625
    return flops, wnk * qbytes + T * H * qbytes


def roofline_from_profile(table):
    """The dominant kernel by total GPU time in the profiled pass: (name, shape (M, N, K) or None, event ms)."""
    name, (ms, n) = max(table.items(), key=lambda kv: kv[1][0])
    m = re.search(r"\[(\d+)x(\d+)x(\d+)\]", name)
    return name, (tuple(map(int, m.groups())) if m else None), ms / n


def isolated_gemm_ms(eng, name, shape, reps=50, rounds=4):
    """That GEMM alone: the model's own weight of this shape, `reps` launches captured in one HIP graph and
    replayed `rounds` times between two HIP events on the engine's stream. Back-to-back launches in a graph
    leave no per-launch event overhead, so this is the kernel's own duration (what rocprofv3 reports). The
    fused qkv + q/k norm + RoPE product is timed as that op (layer 0's weight and norms, the RoPE table made
    once beforehand), not as a plain product of its shape, which would pick another tile; a product tagged
    +rownorm (the folded norm's consumer) or +residual (its producer) is timed in that form, on seeded rows,
    sums of squares and stream values."""
    from decision_js_amd import _dj
    M, N, K = shape
    glu = name.startswith("matmul_glu")
    rope = name.startswith("matmul_rope")
    rownorm, residual = name.endswith("+rownorm"), name.endswith("+residual")
    want = _dj.W_MFMA_GLU if glu else _dj.W_MFMA
    w = next((w for w in eng.w.values() if isinstance(w, _dj.Weight) and w.N == N and w.K == K
              and (w.layout & ~_dj.W_DIRECT) == want), None)
    if rope:  # the fused qkv + q/k norm + RoPE op itself, on layer 0's weights and norms
        w = eng.w.get("layers.0.qkv")
    if w is None or (rope and (w.N, w.K) != (N, K)):
        return None
    ctx = eng.ctx
    rng = np.random.default_rng(5)
    X = ctx.array((rng.standard_normal((M, K)) * 0.5).astype(np.float16))
    Y = ctx.alloc(M * (N // 2 if glu else N) * 2)
    key = 0x6A5EB0000 + (M * 131 + N * 7 + K) % 65521 + (1 << 20 if rope else 0) + (2 << 20 if rownorm else 0) \
        + (4 << 20 if residual else 0)
    if rownorm:  # per-32-column sums of squares of rows of about unit scale
        SS = ctx.array((rng.random((M, K // 32)) * 16 + 16).astype(np.float32))
    if residual:
        R = ctx.array(rng.standard_normal((M, N)).astype(np.float16))
        nw = ctx.array(np.ones(N, np.float16))
        XW, SS = ctx.alloc(M * N * 2), ctx.alloc(M * (N // 32) * 4)
    if rope:
        pos = ctx.array((np.arange(M) % 384).astype(np.int32))
        tab = ctx.alloc(M * (eng.D // 2) * 8)
        rec = ctx.recorder()
        rec.rope_table(M, pos, 1, eng.theta, eng.D, tab)  # the forward's angle table, made once outside the timing
        rec.finish()
        qn, kn = eng.w.get("layers.0.q_norm"), eng.w.get("layers.0.k_norm")

    def one(rec):
        if rope and rownorm:
            rec.matmul_qkv_rope_normed(X, w, Y, M, eng.h, eng.kv, eng.D, qn, kn, False, pos, 1, eng.eps, eng.theta, tab,
                                       SS, K, eng.eps)
        elif rope:
            rec.matmul_qkv_rope(X, w, Y, M, eng.h, eng.kv, eng.D, qn, kn, False, pos, 1, eng.eps, eng.theta, tab)
        elif rownorm:
            rec.matmul_normed(X, w, Y, M, _dj.ACT_SILU if glu else -1, SS, K, eng.eps)
        elif residual:
            rec.matmul_residual(X, w, M, R, nw, XW, SS)
        elif glu:
            rec.matmul_glu(X, w, Y, M)
        else:
            rec.matmul(X, w, Y, M)

    def run():
        rec = ctx.recorder(key)
        if not rec.replay:
            for _ in range(reps):
                one(rec)
        rec.finish()

    run()
    ctx.timer_begin()
    for _ in range(rounds):
        run()
    ms = ctx.timer_end() / (rounds * reps)
    X.free()
    Y.free()
    if rope:
        pos.free()
        tab.free()
    for b in ((SS,) if rownorm else (R, nw, XW, SS) if residual else ()):
        b.free()
    return ms


def cpu_baseline(model_dir, ticket, budget_s):
    """The oracle's forward (numpy, f32 accumulation, f16 storage points) on one ticket, on the host cores."""
    sys.path.insert(0, ROOT)
    from oracle import ref
    try:
        from threadpoolctl import threadpool_info
        cores = max((i.get("num_threads", 1) for i in threadpool_info()), default=os.cpu_count())
    except Exception:  # noqa: BLE001
        cores = os.cpu_count()
    model = ref.Model(model_dir)
    ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest(ticket)
    mask = ref.ranges_mask(ref.forest_ranges(meta), len(ids))
    done, t0 = 0, time.perf_counter()
    while True:
        ref.decoder_forward(model, ids, pos, mask, leaves, leaf_ids, n_ids)
        done += 1
        el = time.perf_counter() - t0
        if el > budget_s or done >= 3:
            break
    return {"value": round(3 * done / el, 4), "unit": "decisions/s", "cores": int(cores), "kind": "port",
            "sample": f"{done} ticket(s) of the same workload ({len(ticket)} x {len(ticket[0]['branches'][0])} tokens, all {model.c['layers']} layers) through "
                      f"oracle/ref.decoder_forward (numpy f32, CPU restatement of the reference path); {el:.1f} s"}


def calibration_copy(ctx, mib):
    """A plain device copy of `mib` MiB (the library's copy kernel), the known-size reference that scales the
    FETCH_SIZE / WRITE_SIZE counters of the same run."""
    src, dst = ctx.alloc(mib << 20), ctx.alloc(mib << 20)
    dst.copy_from(src)
    ctx.timer_begin()
    dst.copy_from(src)
    log(f"calibration copy {mib} MiB: {ctx.timer_end():.3f} ms")
    src.free()
    dst.free()


def _line(metric, value, unit, steps, warmup, ms, dtype, workload, roofline, extra=None):
    out = {"metric": metric, "value": round(value, 3), "unit": unit, "n_gpus": 1, "steps": steps, "warmup": warmup,
           "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
           "data": "synthetic", "config": {"workload": workload}, "roofline": roofline, "cpu_baseline": None}
    out.update(extra or {})
    return out


def _forward_fraction(cfg, T, seqs, ms, causal=True, markers=0):
    """Appendix-B roofline of a forward: achieved TFLOP/s (and weight GB/s) over the measured time."""
    flops, wbytes = model_flops_bytes(cfg, T, seqs, causal, markers)
    t_mfma, t_hbm = flops / (MFMA_F16_PEAK_TFLOPS * 1e12), wbytes / (HBM_PEAK_GBS * 1e9)
    s = ms * 1e-3
    if t_mfma >= t_hbm:
        a = flops / s / 1e12
        return {"bound": "mfma", "achieved": round(a, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(a / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None, "scope": "whole forward (Appendix B flops)"}
    a = wbytes / s / 1e9
    return {"bound": "hbm", "achieved": round(a, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(a / HBM_PEAK_GBS, 4),
            "traffic": None, "scope": "whole forward (quantized weight bytes)"}


def probe_reference_cpu_path(timeout=20):
    """The reference's own CPU path (its WGSL kernels through Node WebGPU/Dawn on a CPU Vulkan adapter) needs
    Node >= 18, a WebGPU binding and a Vulkan ICD such as lavapipe. Records what this host has, run before the
    GPU is touched (child processes only); nothing is installed."""
    import shutil
    import subprocess
    out = {}
    node = shutil.which("node")
    out["node"] = None
    if node:
        try:
            out["node"] = subprocess.run([node, "--version"], capture_output=True, text=True, timeout=timeout).stdout.strip()
        except Exception as e:  # noqa: BLE001
            out["node"] = f"error: {e}"
    icd = "/usr/share/vulkan/icd.d"
    out["vulkan_icds"] = sorted(os.listdir(icd)) if os.path.isdir(icd) else []
    out["webgpu_binding"] = False
    if node:
        try:
            r = subprocess.run([node, "-e", "require('webgpu')"], capture_output=True, text=True, timeout=timeout)
            out["webgpu_binding"] = r.returncode == 0
        except Exception:  # noqa: BLE001
            pass
    major = int(out["node"][1:].split(".")[0]) if out["node"] and out["node"].startswith("v") else 0
    out["runnable"] = bool(major >= 18 and out["vulkan_icds"] and out["webgpu_binding"])
    out["status"] = ("available" if out["runnable"] else
                     "unavailable: the reference's WGSL path needs Node >= 18, a WebGPU binding and a Vulkan ICD "
                     "(none installed here); cpu_baseline is this build's CPU restatement instead")
    return out


def batch_trees(cfg):
    """192 sequences of U[128, 768] random ids (lengths seed 2, ids seed 1, answer sets seed 3)."""
    lens_rng = np.random.Generator(np.random.PCG64(2))
    ids_rng = np.random.Generator(np.random.PCG64(1))
    ans_rng = np.random.Generator(np.random.PCG64(3))
    V = cfg["vocab"]
    lens = [int(x) for x in lens_rng.integers(128, 769, 192)]
    trees = [{"trunk": [], "branches": [[int(x) for x in ids_rng.integers(0, V, n)]],
              "groups": [[[int(a)] for a in ans_rng.choice(V, size=(2, 3, 5)[k % 3], replace=False)]]} for k, n in enumerate(lens)]
    return trees, lens


def batched_gemm_fraction(eng, cfg, st, T):
    """One configs[3] forward with every op timed on its own (HIP events on the engine's stream): the prefill
    GEMMs' FLOPs (2 T sum(N K) per layer) over their summed GPU time, against dense f16 peak."""
    graphs = eng.graphs
    eng.graphs = False
    eng.ctx.profile_reset()
    eng.ctx.profile(True)
    eng.run_staged(st)
    eng.ctx.profile(False)
    table = eng.ctx.profile_table()
    eng.graphs = graphs
    total = sum(v[0] for v in table.values())
    for k, (kms, cnt) in sorted(table.items(), key=lambda kv: -kv[1][0])[:8]:
        log(f"  {k:48s} {kms:8.3f} ms/forward  {100 * kms / total:5.1f}%  ({cnt} launches, {1e3 * kms / cnt:8.1f} us each)")
    gemm_ms = sum(v[0] for k, v in table.items() if k.startswith("matmul"))
    gemm_flops = 2.0 * T * sum(n * k for n, k in _linear_shapes(cfg)) * cfg["layers"]
    tf = gemm_flops / (gemm_ms * 1e-3) / 1e12
    return {"tokens": T, "gemm_ms": round(gemm_ms, 3), "forward_ms_events": round(total, 3), "gemm_tflops": round(tf, 1),
            "peak": MFMA_F16_PEAK_TFLOPS, "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "target": 0.60}


def question_alone(eng, cfg, state, branch, group, steps, warmup, per_op=True):
    """One 32-token question against a prefilled, kept state (configs[4]'s weight-streaming regime): GPU time
    per question (HIP events over `steps` replayed forwards) and its quantized weight bytes over that time."""
    stt = eng.prefill(state)
    try:
        for _ in range(warmup):
            eng.run_shared(stt, [branch], [group])
        eng.ctx.timer_begin()
        t1 = time.perf_counter()
        for _ in range(steps):
            eng.run_shared(stt, [branch], [group])
        wall = (time.perf_counter() - t1) / steps
        gpu = eng.ctx.timer_end() / steps
        if per_op:
            graphs = eng.graphs
            eng.graphs = False
            eng.ctx.profile_reset()
            eng.ctx.profile(True)
            eng.run_shared(stt, [branch], [group])
            eng.ctx.profile(False)
            table = eng.ctx.profile_table()
            eng.graphs = graphs
            total = sum(v[0] for v in table.values())
            log(f"question alone, per op (launched one at a time, {1e3 * total:.0f} us in all):")
            for k, (kms, cnt) in sorted(table.items(), key=lambda kv: -kv[1][0])[:10]:
                log(f"  {k:48s} {1e3 * kms:8.1f} us/question  {100 * kms / total:5.1f}%  ({cnt} launches, {1e3 * kms / cnt:6.1f} us each)")
    finally:
        eng.free_state(stt)
    roof = _forward_fraction(cfg, 32, [32], gpu)
    return wall, gpu, roof


def run_workload(args):
    """The BASELINE configs other than the metric's, one JSON line each (not the driver's bench line):
    batch   configs[3]: 192 sequences of U[128, 768] random ids (lengths seed 2) on the 0.6B q8 decoder, packed
            varlen into one forward; a step is that forward (192 decisions)
    shared  configs[4]: a 1024-id state prefilled once (K/V kept) and 8 questions of 32 ids against it on the
            ~0.8B q8 decoder; a step is prefill + 8 questions (8 decisions); also one question alone
    encoder configs[0]: 11 texts (1 x 256, 3 x 24, 7 x 8 ids) embedded in one forward of the EG2-shaped encoder,
            every question scoring all 7 options by cosine; a step is one ticket (3 decisions)"""
    from decision_js_amd import synth
    from decision_js_amd.engine import DecoderEngine
    steps, warmup = args.steps, args.warmup
    if args.workload == "batch":
        cfg = synth.CONFIGS["qwen3-0.6b-q8"]
        mdir = os.path.join(args.model_dir, "qwen3-0.6b-q8")
        synth.generate(cfg, mdir, seed=0, threads=16)
        eng = DecoderEngine.load(mdir, {"graphs": not args.no_graphs})
        trees, lens = batch_trees(cfg)
        st = eng.stage(trees)
        T = sum(lens)
        log(f"batch: 192 sequences, T = {T}")
        for _ in range(warmup):
            eng.run_staged(st)
        eng.ctx.timer_begin()
        t0 = time.perf_counter()
        for _ in range(steps):
            eng.run_staged(st)
        wall = time.perf_counter() - t0
        gpu_ms = eng.ctx.timer_end() / steps
        ms = 1e3 * wall / steps
        roof = _forward_fraction(cfg, T, lens, gpu_ms)
        g = batched_gemm_fraction(eng, cfg, st, T)
        roof["gemm_tflops"], roof["gemm_frac"] = g["gemm_tflops"], g["frac"]
        log(f"forward {gpu_ms:.2f} ms (GPU), {192 * steps / wall:.1f} decisions/s; GEMMs {roof['gemm_tflops']} TFLOP/s "
            f"({100 * roof['gemm_frac']:.1f}% of dense f16 peak)")
        out = _line("decisions/sec (config-4 batch: 192 sequences, one varlen forward) on 1 MI355X", 192 * steps / wall,
                    "decisions/s", steps, warmup, ms, "f16",
                    f"configs[3]: qwen3-0.6b-q8, 192 sequences of U[128,768] random ids (T={T}) in one forward", roof,
                    {"gpu_ms_per_step": round(gpu_ms, 3)})
        eng.free_staged(st)
        eng.destroy()
    elif args.workload == "shared":
        cfg = synth.CONFIGS["d3lite-0.8b-q8"]
        mdir = os.path.join(args.model_dir, "d3lite-0.8b-q8")
        synth.generate(cfg, mdir, seed=0, threads=16)
        eng = DecoderEngine.load(mdir, {"graphs": not args.no_graphs})
        ids_rng = np.random.Generator(np.random.PCG64(1))
        ans_rng = np.random.Generator(np.random.PCG64(3))
        V = cfg["vocab"]
        state = [int(x) for x in ids_rng.integers(0, V, 1024)]
        branches = [[int(x) for x in ids_rng.integers(0, V, 32)] for _ in range(8)]
        groups = [[[int(a)] for a in ans_rng.choice(V, size=(2, 3, 5)[k % 3], replace=False)] for k in range(8)]

        def unit():
            stt = eng.prefill(state)
            eng.run_shared(stt, branches, groups)
            eng.free_state(stt)

        for _ in range(warmup):
            unit()
        eng.ctx.timer_begin()
        t0 = time.perf_counter()
        for _ in range(steps):
            unit()
        wall = time.perf_counter() - t0
        gpu_ms = eng.ctx.timer_end() / steps
        ms = 1e3 * wall / steps
        # one question alone against a kept state: the weight-streaming (GEMV) regime
        q_wall, q_gpu, q_roof = question_alone(eng, cfg, state, branches[0], groups[0], steps, warmup)
        if args.calib_mb:
            calibration_copy(eng.ctx, args.calib_mb)
        roof = _forward_fraction(cfg, 1024 + 256, [1024] + [32] * 8, gpu_ms)
        log(f"shared: prefill 1024 + 8 x 32 questions {gpu_ms:.3f} ms (GPU); one question alone {q_gpu:.3f} ms "
            f"({q_roof['achieved']} {q_roof['unit']}, {100 * q_roof['frac']:.1f}% of peak)")
        out = _line("decisions/sec (config-5: prefill 1024-token state + 8 questions x 32 tokens) on 1 MI355X", 8 * steps / wall,
                    "decisions/s", steps, warmup, ms, "f16",
                    "configs[4]: d3lite-0.8b-q8 (20 layers), 1024-id state prefilled once, 8 questions of 32 ids on its kept K/V",
                    roof, {"gpu_ms_per_step": round(gpu_ms, 3), "question_alone_ms": round(1e3 * q_wall, 4),
                           "question_alone_gpu_ms": round(q_gpu, 4), "question_alone_roofline": q_roof})
        eng.destroy()
    elif args.workload in ("omni", "laya"):
        out = omni_ticket(args, steps, warmup, args.workload)
    elif args.workload == "d3lite":
        out = d3_lite_ticket(args, steps, warmup)
    elif args.workload == "eg2":
        out = eg2_ticket(args, steps, warmup)
    else:
        from decision_js_amd.encoder import EncoderEngine, cosine_logits
        cfg = synth.CONFIGS["eg2-encoder-q8"]
        mdir = os.path.join(args.model_dir, "eg2-encoder-q8")
        synth.generate(cfg, mdir, seed=0, threads=16)
        eng = EncoderEngine.load(mdir, {"graphs": not args.no_graphs})
        ids_rng = np.random.Generator(np.random.PCG64(1))
        V = cfg["vocab"]
        lens = [256] + [24] * 3 + [8] * 7
        tickets = [[[int(x) for x in ids_rng.integers(0, V, n)] for n in lens] for _ in range(warmup + steps)]

        def unit(texts):
            e = eng.embed(texts)["embeddings"]
            for q in range(3):
                cosine_logits(e[0], e[1 + q], e[4:])

        for t in tickets[:warmup]:
            unit(t)
        eng.ctx.timer_begin()
        t0 = time.perf_counter()
        for t in tickets[warmup:]:
            unit(t)
        wall = time.perf_counter() - t0
        gpu_ms = eng.ctx.timer_end() / steps
        ms = 1e3 * wall / steps
        T = sum(lens)
        roof = _forward_fraction(cfg, T, lens, gpu_ms, causal=False)
        log(f"encoder: ticket of 11 texts (T={T}) {ms:.3f} ms wall, {gpu_ms:.3f} ms GPU")
        out = _line("decisions/sec (config-1 encoder tickets: 11 texts, 3 questions x 7 options) on 1 MI355X", 3 * steps / wall,
                    "decisions/s", steps, warmup, ms, "f16",
                    "configs[0]: eg2-encoder-q8 (24 layers), 1 x 256 + 3 x 24 + 7 x 8 random ids embedded in one forward, cosine over 7 options",
                    roof, {"gpu_ms_per_step": round(gpu_ms, 4)})
        eng.destroy()
    print(json.dumps(out), flush=True)


def omni_tickets(cfg, n, seq_len=384, q_len=44, question_first=False):
    """n d1-omni tickets: a state of seq_len - q_len random ids (PCG64 seed 1) read by 3 questions (a noul, a
    3-way choice, a 5-level score) of q_len ids each, one sequence per question, markers 6 ids apart in the
    question. question_first: Laya's layout (laya-prompt.ts: the question's ids, then the state's)."""
    rng = np.random.Generator(np.random.PCG64(1))
    V, P = cfg["vocab"], seq_len - q_len
    out = []
    for _ in range(n):
        state = [int(x) for x in rng.integers(0, V, P)]
        tk = []
        for t, k in (("noul", 2), ("choice", 3), ("score", 5)):
            q = [int(x) for x in rng.integers(0, V, q_len)]
            at = 0 if question_first else P
            tk.append({"ids": q + state if question_first else state + q, "type": t, "markers": [at + 2 + 6 * j for j in range(k)]})
        out.append(tk)
    return out


MARKER_MODELS = {
    # kind: (config, engine module and class, description, the reference's published ms/ticket)
    "omni": ("d1-omni-q8", "omni", "OmniEngine", "LFM2-350M-shaped bidirectional trunk, 16 layers, 2-layer head",
             {"value": 34.0, "hardware": "Apple M5 Pro, Chrome WebGPU", "model": "d1-omni-600M q8 (real weights)",
              "source": "README.md:31"}),
    "laya": ("laya-q8", "laya", "LayaEngine", "ModernBERT-shaped encoder, 28 layers (every third global, the others "
             "+-64 tokens), 2-layer head", {"value": 39.0, "hardware": "Apple M5 Pro, Chrome WebGPU",
                                            "model": "Laya q8 (real weights, 447 MB)", "source": "README.md:34"}),
}


def omni_ticket(args, steps, warmup, kind="omni"):
    """d1-omni or Laya tickets (the form of the reference's published 34 / 39 ms per ticket on an Apple M5 Pro,
    README.md:31, 34): 3 questions over one 340-id state, each question its own 384-id sequence (the state read
    anew per question, omni-engine.ts:5; Laya's question first), packed in one forward (T = 1152): the trunk,
    decision head, marker scorer, then the temperature softmax on the host. A step is one ticket, inputs staged
    in HBM."""
    import importlib
    from decision_js_amd import synth
    from decision_js_amd.d1 import softmax
    from decision_js_amd.omni import temperature
    name, mod, cls, desc, published = MARKER_MODELS[kind]
    Engine = getattr(importlib.import_module(f"decision_js_amd.{mod}"), cls)
    cfg = synth.CONFIGS[name]
    mdir = os.path.join(args.model_dir, name)
    synth.generate(cfg, mdir, seed=0, threads=16)
    eng = Engine.load(mdir, {"graphs": not args.no_graphs})
    tickets = omni_tickets(cfg, warmup + steps, question_first=kind == "laya")
    staged = [eng.stage(t) for t in tickets]

    def unit(st):
        z = eng.run_staged(st)["logits"]
        return [softmax(np.asarray(l) / temperature(cfg, s["type"], len(l))) for s, l in zip(st["seqs"], z)]

    for st in staged[:warmup]:
        unit(st)
    eng.ctx.timer_begin()
    t0 = time.perf_counter()
    times = []
    for st in staged[warmup:]:
        a = time.perf_counter()
        unit(st)
        times.append(time.perf_counter() - a)
    wall = time.perf_counter() - t0
    gpu_ms = eng.ctx.timer_end() / steps
    ms = 1e3 * wall / steps
    lens = [len(s["ids"]) for s in tickets[0]]
    T = sum(lens)
    roof = _forward_fraction(cfg, T, lens, gpu_ms, causal=False, markers=10)
    eng.graphs = False
    eng.ctx.profile_reset()
    eng.ctx.profile(True)
    for st in staged[:3]:
        eng.run_staged(st)
    eng.ctx.profile(False)
    table = eng.ctx.profile_table()
    total = sum(v[0] for v in table.values())
    for k, (t_ms, cnt) in sorted(table.items(), key=lambda kv: -kv[1][0])[:10]:
        log(f"  {k:48s} {t_ms / 3:8.4f} ms/ticket  {100 * t_ms / total:5.1f}%  ({cnt // 3}/ticket, {1e3 * t_ms / cnt:7.2f} us each)")
    p50 = 1e3 * float(np.median(times))
    log(f"{kind}: ticket (T={T}) {ms:.3f} ms wall (p50 {p50:.3f}), {gpu_ms:.3f} ms GPU, {3 * steps / wall:.1f} decisions/s")
    for st in staged:
        eng.free_staged(st)
    eng.destroy()
    label = "d1-omni" if kind == "omni" else "Laya"
    return _line(f"decisions/sec ({label} tickets: 3 questions, one 384-id sequence each) on 1 MI355X", 3 * steps / wall,
                 "decisions/s", steps, warmup, ms, "f16", f"{name} ({desc}), 3 x 384 random ids in one forward, 10 markers",
                 roof, {"gpu_ms_per_step": round(gpu_ms, 4), "p50_ms_per_ticket": round(p50, 4),
                        "reference_published_ms_per_ticket": published})


def d3_lite_ticket(args, steps, warmup):
    """d3-lite tickets on its shipped layout (the reference publishes 95 ms per ticket, 58 ms with shareState, on
    an Apple M5 Pro, README.md:33, 44): 3 questions over one 340-id state, each question a 384-id sequence with 2 /
    3 / 5 codes read at its last token, packed in one forward (T = 1152; with shareState the state is read once:
    T = 472). A step is one ticket of each form, inputs packed and uploaded by the host (as the API does)."""
    from decision_js_amd import synth
    from decision_js_amd.d3 import D3Engine
    cfg = synth.CONFIGS["d3-lite-q8"]
    mdir = os.path.join(args.model_dir, "d3-lite-q8")
    synth.generate(cfg, mdir, seed=0, threads=16)
    eng = D3Engine.load(mdir, {"graphs": not args.no_graphs})
    rng = np.random.Generator(np.random.PCG64(1))
    V = cfg["vocab"]
    tickets = []
    for _ in range(warmup + steps):
        state = [int(x) for x in rng.integers(0, V, 340)]
        tickets.append([{"ids": state + [int(x) for x in rng.integers(0, V, 44)], "options": k} for k in (2, 3, 5)])
    res = {}
    for name, groups in (("plain", None), ("shared", [3])):
        for t in tickets[:warmup]:
            eng.logits_d3(t, groups)
        eng.ctx.timer_begin()
        t0 = time.perf_counter()
        for t in tickets[warmup:]:
            eng.logits_d3(t, groups)
        wall = time.perf_counter() - t0
        res[name] = (1e3 * wall / steps, eng.ctx.timer_end() / steps)
        log(f"d3-lite {name}: {res[name][0]:.3f} ms per ticket wall, {res[name][1]:.3f} ms GPU")
    eng.graphs = False
    eng.ctx.profile_reset()
    eng.ctx.profile(True)
    for t in tickets[:3]:
        eng.logits_d3(t)
    eng.ctx.profile(False)
    table = eng.ctx.profile_table()
    total = sum(v[0] for v in table.values())
    for k, (t_ms, cnt) in sorted(table.items(), key=lambda kv: -kv[1][0])[:10]:
        log(f"  {k:48s} {t_ms / 3:8.4f} ms/ticket  {100 * t_ms / total:5.1f}%  ({cnt // 3}/ticket, {1e3 * t_ms / cnt:7.2f} us each)")
    eng.destroy()
    ms, gpu = res["plain"]
    return _line("decisions/sec (d3-lite tickets: 3 questions, one 384-id sequence each) on 1 MI355X", 3e3 / ms,
                 "decisions/s", steps, warmup, ms, "f16",
                 "d3-lite-q8 (Qwen3.5-0.8B-shaped: 18 Gated DeltaNet + 6 gated attention layers), 3 x 384 random ids in one "
                 "forward, 2/3/5 codes", None,
                 {"gpu_ms_per_step": round(gpu, 4), "share_state_ms_per_ticket": round(res["shared"][0], 4),
                  "share_state_gpu_ms": round(res["shared"][1], 4),
                  "reference_published_ms_per_ticket": {"value": 95.0, "share_state": 58.0, "hardware": "Apple M5 Pro, Chrome WebGPU",
                                                        "model": "d3-lite q8 (real weights)", "source": "README.md:33, 44"}})


def eg2_ticket(args, steps, warmup):
    """EmbeddingGemma 2 tickets on its shipped layout (the reference publishes 6 ms per ticket on an Apple M5 Pro with
    the schema's embeddings cached and a ~70-token state per ticket, README.md:35): through the Decision API, 3
    questions (a 3-way choice, a noul, a 5-level score) whose question and option texts are embedded once (first
    ticket), then per ticket one new ~70-id state embedded and the learned head on the host."""
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    cfg = synth.CONFIGS["eg2-q8"]
    mdir = os.path.join(args.model_dir, "eg2-q8")
    synth.generate(cfg, mdir, seed=0, threads=16)
    d = Decision.load(mdir, {"graphs": not args.no_graphs})
    rng = np.random.Generator(np.random.PCG64(1))
    V = cfg["vocab"]
    ids = lambda n: [int(x) for x in rng.integers(0, V, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": ""}, "ids": ids(24),
                    "option_ids": [ids(8) for _ in range(3)]},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(20), "option_ids": [ids(4), ids(4)]},
          "urgency": {"type": "score", "instructions": "?", "criteria": ["1", "2", "3", "4", "5"], "ids": ids(24),
                      "option_ids": [ids(10) for _ in range(5)]}}
    states = [ids(70) for _ in range(warmup + steps)]
    for st in states[:warmup]:
        d.system_one(st, qs)
    d.engine.ctx.timer_begin()
    times = []
    t0 = time.perf_counter()
    for st in states[warmup:]:
        a = time.perf_counter()
        d.system_one(st, qs)
        times.append(time.perf_counter() - a)
    wall = time.perf_counter() - t0
    gpu = d.engine.ctx.timer_end() / steps
    d.destroy()
    ms = 1e3 * wall / steps
    p50 = 1e3 * float(np.median(times))
    log(f"eg2: {ms:.3f} ms per ticket (p50 {p50:.3f}), {gpu:.3f} ms GPU")
    return _line("decisions/sec (EmbeddingGemma 2 tickets: 3 questions, schema cached, a 70-id state) on 1 MI355X",
                 3e3 / ms, "decisions/s", steps, warmup, ms, "f16",
                 "eg2-q8 (24 layers at hidden 512, per-layer embeddings, sliding 256-dim / global 512-dim heads), "
                 "one 70-id state embedded per ticket, learned head on the host", None,
                 {"gpu_ms_per_step": round(gpu, 4), "p50_ms_per_ticket": round(p50, 4),
                  "reference_published_ms_per_ticket": {"value": 6.0, "hardware": "Apple M5 Pro, Chrome WebGPU",
                                                        "model": "EmbeddingGemma 2 q8 (real weights)", "source": "README.md:35"}})


def _linear_shapes(c):
    """(N, K) of one decoder layer's linears: qkv, o_proj, w13, w2."""
    H, I, h, kv, D = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"]
    return [((h + 2 * kv) * D, H), (H, h * D), (2 * I, H), (H, I)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="qwen3-0.6b-q8")
    ap.add_argument("--model-dir", default=os.environ.get("DJ_MODEL_DIR", "/tmp/dj_models"))
    ap.add_argument("--no-graphs", action="store_true", help="launch every kernel (no HIP graph replay)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--calib-mb", type=int, default=0, help="also run a plain device copy of this many MiB (counter calibration)")
    ap.add_argument("--workload", default="ticket", choices=["ticket", "batch", "shared", "encoder", "omni", "laya", "d3lite", "eg2"],
                    help="ticket: configs[1] (the metric; configs[2] with --config qwen2.5-3b-q4 --seq-len 512); "
                         "batch: configs[3]; shared: configs[4]; encoder: configs[0]")
    ap.add_argument("--seq-len", type=int, default=384, help="tokens per question of a ticket")
    ap.add_argument("--no-north-star", action="store_true", help="skip the configs[3] / configs[4] target measurements")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (the path shards by "
              f"independent tickets: each GPU runs its own engine on its own share of them)", file=sys.stderr)
        sys.exit(2)

    # the reference's CPU path is probed before anything touches the GPU (child processes only)
    probe = probe_reference_cpu_path() if args.workload == "ticket" and not args.no_cpu else None
    pkg = load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.engine import DecoderEngine
    if args.workload != "ticket":
        return run_workload(args)

    cfg = synth.CONFIGS[args.config]
    mdir = os.path.join(args.model_dir, args.config)
    t0 = time.time()
    synth.generate(cfg, mdir, seed=0, threads=16)
    log(f"model {args.config} ready in {time.time() - t0:.1f} s at {mdir}")
    eng = DecoderEngine.load(mdir, {"graphs": not args.no_graphs})
    log(f"device {eng.ctx.info()}; weights on device")

    n = args.warmup + args.steps
    tickets = make_tickets(n, cfg["vocab"], seq_len=args.seq_len)
    staged = [eng.stage(t) for t in tickets]
    T = sum(len(b) for tr in tickets[0] for b in tr["branches"])

    for i in range(args.warmup):
        eng.run_staged(staged[i])
    times = []
    eng.ctx.timer_begin()
    t_all = time.perf_counter()
    for i in range(args.warmup, n):
        t = time.perf_counter()
        eng.run_staged(staged[i])  # ends with the logits readback: the step is complete on return
        times.append(time.perf_counter() - t)
    wall = time.perf_counter() - t_all
    gpu_ms = eng.ctx.timer_end()
    ms_per_step = 1e3 * wall / args.steps
    p50 = float(np.median(times) * 1e3)
    value = 3 * args.steps / wall
    log(f"{args.steps} tickets: {ms_per_step:.3f} ms/ticket (p50 {p50:.3f}), {value:.1f} decisions/s; GPU-timed {gpu_ms / args.steps:.3f} ms/ticket")

    # profiled pass: every kernel launched alone, HIP events around each on the engine's stream
    eng.graphs = False
    eng.ctx.profile_reset()
    eng.ctx.profile(True)
    for i in range(args.profile_steps):
        eng.run_staged(staged[i % n])
    eng.ctx.profile(False)
    table = eng.ctx.profile_table()
    eng.graphs = not args.no_graphs
    total = sum(v[0] for v in table.values())
    for k, (ms, cnt) in sorted(table.items(), key=lambda kv: -kv[1][0])[:12]:
        log(f"  {k:48s} {ms / args.profile_steps:8.4f} ms/ticket  {100 * ms / total:5.1f}%  ({cnt // args.profile_steps}/ticket, {1e3 * ms / cnt:7.2f} us each)")
    name, shape, ev_ms = roofline_from_profile(table)
    roof = None
    if shape and name.startswith("matmul"):
        k_ms = isolated_gemm_ms(eng, name, shape)
        if k_ms:
            M, N, K = shape
            fl = 2.0 * M * N * K
            achieved = fl / (k_ms * 1e-3) / 1e12
            roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": None, "kernel": name,
                    "launch_ms": round(k_ms, 5), "launch_ms_events": round(ev_ms, 5), "flops_per_launch": fl}
            log(f"dominant kernel {name}: {1e3 * k_ms:.2f} us per launch alone (graph of 50), {1e3 * ev_ms:.2f} us "
                f"between per-op events; {achieved:.0f} TFLOP/s")
    flops, wbytes = model_flops_bytes(cfg, T, [args.seq_len] * 3)
    t_roof_ms = max(flops / (MFMA_F16_PEAK_TFLOPS * 1e12), wbytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    if args.calib_mb:
        calibration_copy(eng.ctx, args.calib_mb)
    # HBM bytes per launch of this kernel from the committed counter summary that names it (FETCH_SIZE and
    # WRITE_SIZE, each scaled by its reading for a copy of known size); not measured in this run
    if roof:
        import glob
        for f in sorted(glob.glob(os.path.join(ROOT, "profiles", "traffic_*.json"))):
            tr = json.load(open(f))
            if tr.get("kernel_key") == name:
                roof["traffic"] = tr.get("bytes_per_launch")
                roof["traffic_source"] = os.path.relpath(f, ROOT) + " (committed rocprofv3 counter summary, not this run)"

    # the north star's two targets, measured in this run on their own workloads
    north = None
    if not args.no_north_star and args.config == "qwen3-0.6b-q8":
        north = north_star(args, eng, cfg)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(mdir, tickets[0], args.cpu_budget)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "decisions/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "p50_ms_per_ticket": round(p50, 4),
        "gpu_ms_per_ticket": round(gpu_ms / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"{'configs[1]' if args.config == 'qwen3-0.6b-q8' and args.seq_len == 384 else 'configs[2]' if args.config == 'qwen2.5-3b-q4' else 'custom'}: "
                               f"{args.config} causal decoder, seeded N(0,0.02) weights; ticket = 3 questions x {args.seq_len} random-id "
                               f"tokens packed in one forward (T={3 * args.seq_len}), answer sets of 2/3/5 ids at each last token",
                   "tokens_per_ticket": T, "graphs": not args.no_graphs},
        "roofline": roof,
        "forward_roofline": {"t_roof_ms": round(t_roof_ms, 4), "frac_of_roofline": round(t_roof_ms / (gpu_ms / args.steps), 4),
                             "flops_per_ticket": flops, "weight_bytes": wbytes},
        "cpu_baseline": cpu,
        "north_star": north,
        "cpu_reference_probe": probe,
    }
    eng.destroy()
    print(json.dumps(out), flush=True)


def north_star(args, eng, cfg):
    """BASELINE.json's targets, each on its own configuration: (1) batched prefill GEMMs at >= 60% of dense f16
    MFMA peak on configs[3] (192 sequences, one varlen forward on this same model: every op timed on its own);
    (2) >= 70% of HBM bandwidth on a weight-bound single question of configs[4] (the ~0.8B q8 decoder, one
    32-token question against a kept 1024-token state; GPU time of replayed forwards)."""
    from decision_js_amd import synth
    from decision_js_amd.engine import DecoderEngine
    out = {}
    t0 = time.time()
    trees, lens = batch_trees(cfg)
    st = eng.stage(trees)
    T = sum(lens)
    eng.run_staged(st)  # warm (buffers grown, kernels loaded)
    out["batched_prefill_gemms"] = dict(batched_gemm_fraction(eng, cfg, st, T), workload="configs[3]: 192 x U[128,768] ids")
    eng.free_staged(st)
    log(f"north star 1: batched prefill GEMMs {out['batched_prefill_gemms']['gemm_tflops']} TFLOP/s "
        f"({100 * out['batched_prefill_gemms']['frac']:.1f}% of dense f16) in {time.time() - t0:.1f} s")
    t0 = time.time()
    qcfg = synth.CONFIGS["d3lite-0.8b-q8"]
    qdir = os.path.join(args.model_dir, "d3lite-0.8b-q8")
    synth.generate(qcfg, qdir, seed=0, threads=16)
    qeng = DecoderEngine.load(qdir, {"graphs": not args.no_graphs})
    try:
        ids_rng = np.random.Generator(np.random.PCG64(1))
        ans_rng = np.random.Generator(np.random.PCG64(3))
        V = qcfg["vocab"]
        state = [int(x) for x in ids_rng.integers(0, V, 1024)]
        branch = [int(x) for x in ids_rng.integers(0, V, 32)]
        group = [[int(a)] for a in ans_rng.choice(V, size=2, replace=False)]
        wall, gpu, roof = question_alone(qeng, qcfg, state, branch, group, steps=30, warmup=5)
    finally:
        qeng.destroy()
    out["question_alone"] = {"gpu_ms": round(gpu, 4), "wall_ms": round(1e3 * wall, 4), "weight_gbs": roof["achieved"],
                             "peak": HBM_PEAK_GBS, "frac": roof["frac"], "target": 0.70,
                             "workload": "configs[4]: d3lite-0.8b-q8, one 32-id question on a kept 1024-id state"}
    log(f"north star 2: question alone {gpu:.3f} ms, {roof['achieved']} GB/s ({100 * roof['frac']:.1f}% of HBM) "
        f"in {time.time() - t0:.1f} s")
    return out


if __name__ == "__main__":
    main()
