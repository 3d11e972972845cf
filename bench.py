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


def model_flops_bytes(c, T, seqs_len):
    """Appendix-B algorithmic work of one forward: 2 T sum(N K) over the linears plus 4 D h (allowed
    query-key pairs) per layer; bytes = quantized linear weights + gathered embedding rows."""
    H, I, h, kv, D, L = c["hidden"], c["intermediate"], c["heads"], c["kv_heads"], c["head_dim"], c["layers"]
    nk = (h + 2 * kv) * D * H + H * h * D + 2 * I * H + H * I
    pairs = sum(n * (n + 1) // 2 for n in seqs_len)
    flops = 2 * T * nk * L + 4 * D * h * pairs * L
    qbytes = 1.0625 if c.get("bits", 8) == 8 else 0.5625
    return flops, nk * L * qbytes + T * H * qbytes


def roofline_from_profile(table):
    """The dominant kernel by total GPU time in the profiled pass: (name, shape (M, N, K) or None, event ms)."""
    name, (ms, n) = max(table.items(), key=lambda kv: kv[1][0])
    m = re.search(r"\[(\d+)x(\d+)x(\d+)\]", name)
    return name, (tuple(map(int, m.groups())) if m else None), ms / n


def isolated_gemm_ms(eng, name, shape, reps=50, rounds=4):
    """That GEMM alone: the model's own weight of this shape, `reps` launches captured in one HIP graph and
    replayed `rounds` times between two HIP events on the engine's stream. Back-to-back launches in a graph
    leave no per-launch event overhead, so this is the kernel's own duration (what rocprofv3 reports)."""
    from decision_js_amd import _dj
    M, N, K = shape
    glu = name.startswith("matmul_glu")
    want = _dj.W_MFMA_GLU if glu else _dj.W_MFMA
    w = next((w for w in eng.w.values() if isinstance(w, _dj.Weight) and w.N == N and w.K == K
              and (w.layout & ~_dj.W_DIRECT) == want), None)
    if w is None:
        return None
    ctx = eng.ctx
    rng = np.random.default_rng(5)
    X = ctx.array((rng.standard_normal((M, K)) * 0.5).astype(np.float16))
    Y = ctx.alloc(M * (N // 2 if glu else N) * 2)
    key = 0x6A5EB0000 + (M * 131 + N * 7 + K) % 65521

    def run():
        rec = ctx.recorder(key)
        if not rec.replay:
            for _ in range(reps):
                rec.matmul_glu(X, w, Y, M) if glu else rec.matmul(X, w, Y, M)
        rec.finish()

    run()
    ctx.timer_begin()
    for _ in range(rounds):
        run()
    ms = ctx.timer_end() / (rounds * reps)
    X.free()
    Y.free()
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
            "sample": f"{done} ticket(s) of the same workload (3 x 384 tokens, all {model.c['layers']} layers) through "
                      f"oracle/ref.decoder_forward (numpy f32, CPU restatement of the reference path); {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="qwen3-0.6b-q8")
    ap.add_argument("--model-dir", default=os.environ.get("DJ_MODEL_DIR", "/tmp/dj_models"))
    ap.add_argument("--no-graphs", action="store_true", help="launch every kernel (no HIP graph replay)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--profile-steps", type=int, default=5)
    ap.add_argument("--calib-mb", type=int, default=0, help="also run a plain device copy of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (the path shards by "
              f"independent tickets: see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    pkg = load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.engine import DecoderEngine

    cfg = synth.CONFIGS[args.config]
    mdir = os.path.join(args.model_dir, args.config)
    t0 = time.time()
    synth.generate(cfg, mdir, seed=0, threads=16)
    log(f"model {args.config} ready in {time.time() - t0:.1f} s at {mdir}")
    eng = DecoderEngine.load(mdir, {"graphs": not args.no_graphs})
    log(f"device {eng.ctx.info()}; weights on device")

    n = args.warmup + args.steps
    tickets = make_tickets(n, cfg["vocab"])
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
    flops, wbytes = model_flops_bytes(cfg, T, [384, 384, 384])
    t_roof_ms = max(flops / (MFMA_F16_PEAK_TFLOPS * 1e12), wbytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    if args.calib_mb:
        src, dst = eng.ctx.alloc(args.calib_mb << 20), eng.ctx.alloc(args.calib_mb << 20)
        dst.copy_from(src)
        eng.ctx.timer_begin()
        dst.copy_from(src)
        log(f"calibration copy {args.calib_mb} MiB: {eng.ctx.timer_end():.3f} ms")
    # HBM bytes per launch of this kernel from the committed counter summary that names it (FETCH_SIZE and
    # WRITE_SIZE, each scaled by its reading for a copy of known size)
    if roof:
        import glob
        for f in sorted(glob.glob(os.path.join(ROOT, "profiles", "traffic_*.json"))):
            tr = json.load(open(f))
            if tr.get("kernel_key") == name:
                roof["traffic"] = tr.get("bytes_per_launch")
                roof["traffic_source"] = os.path.relpath(f, ROOT)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(mdir, tickets[0], args.cpu_budget)
        log(f"cpu baseline: {cpu}")

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "decisions/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "p50_ms_per_ticket": round(p50, 4),
        "gpu_ms_per_ticket": round(gpu_ms / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic",
        "config": {"workload": f"configs[1]: {args.config} causal decoder, seeded N(0,0.02) weights; ticket = 3 questions x 384 random-id "
                               "tokens packed in one forward (T=1152), answer sets of 2/3/5 ids at each last token",
                   "tokens_per_ticket": T, "graphs": not args.no_graphs},
        "roofline": roof,
        "forward_roofline": {"t_roof_ms": round(t_roof_ms, 4), "frac_of_roofline": round(t_roof_ms / (gpu_ms / args.steps), 4),
                             "flops_per_ticket": flops, "weight_bytes": wbytes},
        "cpu_baseline": cpu,
    }
    eng.destroy()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
