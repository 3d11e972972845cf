"""The Node host (decision.js_amd/node/: the Decision API in JavaScript over the N-API binding of the C ABI)
against the Python host and the oracle. CPU: the binding exports one function per entry point of
include/dj.h; forest packing, group-max readout, question answers and errors, and pass splitting equal the
Python host's; loading without a GPU fails with the library's error. GPU: systemOne / probabilities /
systemOneBatch / shareState through Node give the Python host's probabilities and bit-identical logits (the
same library, op sequence and packing)."""
import json
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

from _pkg import ROOT, load_pkg

NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "decision.js_amd", "lib", "dj_napi.node")
pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def node(req, timeout=120, env=None):
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "check.js")], input=json.dumps(req),
                       capture_output=True, text=True, timeout=timeout, env=dict(os.environ, **(env or {})))
    if r.returncode != 0:
        raise RuntimeError(f"node failed: {r.stderr}")
    return json.loads(r.stdout)


def camel(name):
    head, *rest = name.split("_")
    return head + "".join(p.capitalize() for p in rest)


def test_binding_exports_every_entry_point():
    if not os.path.exists(ADDON):
        pytest.skip("the Node binding is not built (no Node headers)")
    header = open(os.path.join(ROOT, "include", "dj.h")).read()
    fns = sorted(set(re.findall(r"^\w[\w\s\*]*?\b(dj_\w+)\(", header, re.M)))
    got = set(node({"cmd": "exports"}))
    missing = [f for f in fns if camel(f[3:]) not in got]
    assert not missing, f"entry points without a Node binding: {missing}"
    assert {"recFinishAsync", "W_MFMA", "W_DIRECT", "ABI_VERSION"} <= got


def _trees(rng, V=5000):
    out = []
    for trunk, branches in [(40, [5, 9, 1]), (0, [7]), (13, []), (1, [1, 1, 30]), (200, [24, 31, 17])]:
        groups = []
        for b in range(len(branches)):
            n = (2, 3, 5)[b % 3]
            ids = rng.choice(V, size=2 * n, replace=False)
            groups.append([[int(ids[2 * i])] if i % 2 else [int(ids[2 * i]), int(ids[2 * i + 1])] for i in range(n)])
        out.append({"trunk": [int(x) for x in rng.integers(0, V, trunk)],
                    "branches": [[int(x) for x in rng.integers(0, V, b)] for b in branches], "groups": groups})
    return out


def test_packing_and_readout_match_python_host():
    load_pkg()
    from decision_js_amd import engine
    rng = np.random.default_rng(0)
    trees = _trees(rng)
    js = node({"cmd": "pack", "trees": trees})
    py = engine.pack_forest(trees)
    assert js["T"] == py["T"] and js["L"] == py["L"] and js["nIds"] == py["n_ids"]
    for k_js, k_py in [("ids", "ids"), ("pos", "pos"), ("rng", "rng"), ("taps", "taps"), ("leaves", "leaves"), ("leafIds", "leaf_ids")]:
        assert np.array_equal(np.asarray(js[k_js]), np.asarray(py[k_py]).reshape(-1)), k_js
    out = rng.standard_normal(py["L"] * py["n_ids"]).astype(np.float32)
    got = node({"cmd": "groupmax", "out": [float(x) for x in out], "nIds": py["n_ids"], "trees": trees})
    assert got == engine.group_max(out, py["n_ids"], trees)


def test_questions_match_python_host():
    load_pkg()
    from decision_js_amd import questions as Q
    items = [
        ({"type": "noul", "instructions": "?"}, [0.7, 0.3]),
        ({"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": ""}}, [0.2, 0.5, 0.3]),
        ({"type": "score", "instructions": "?", "criteria": ["lo", "mid", "hi"]}, [0.1, 0.3, 0.6]),
        ({"type": "choice", "instructions": "?", "criteria": {"a": ""}}, [1.0]),
        ({"type": "score", "instructions": "?", "criteria": ["x"]}, [1.0]),
        ({"type": "maybe", "instructions": "?"}, [1.0]),
        ({"instructions": "?"}, [1.0]),
        ({"type": "noul", "instructions": "?", "criteria": ["yes", "no"]}, [0.5, 0.5]),
    ]
    js = node({"cmd": "answer", "items": items})
    for (q, p), j in zip(items, js):
        try:
            want = Q.answer(Q.check_question(q), p)
        except Q.QuestionError as e:
            assert j == {"error": str(e)}
            continue
        assert j == want


def test_encoder_packing_kinds_and_head_match_python_host():
    """Encoder packing equals the Python host's bit for bit; manifests route to the reference's kinds
    (d1.ts:63-64); the learned decision head (eg2-head.ts) gives the Python host's logits."""
    load_pkg()
    from decision_js_amd import encoder
    from decision_js_amd.eg2_head import Eg2Head
    seqs = [[5, 6, 7], [1], list(range(40)), [9, 9]]
    js = node({"cmd": "packenc", "seqs": seqs})
    py = encoder.pack_encoder(seqs)
    assert js["T"] == py["T"] and js["S"] == py["S"]
    for k in ("ids", "meta", "full", "ranges"):
        assert np.array_equal(np.asarray(js[k]), py[k].reshape(-1)), k
    configs = [{"model": "decoder"}, {"model": "d1-3b"}, {"model": "eg2-encoder"}, {"model": "eg2"}, {"model": "d3"},
               {"model": "d1-omni", "head_layers": 2}, {"head_layers": 2}, {"model": "laya", "head_layers": 2},
               {"model": "d1-3b", "head_layers": 2}]
    kinds = node({"cmd": "kinds", "configs": configs})
    assert kinds == ["d1-3b", "d1-3b", "eg2", "eg2", "d3", "d1-omni", "d1-omni", "laya", "d1-3b"]
    from decision_js_amd import d1
    assert [d1._kind(c) for c in configs] == kinds
    import test_eg2_head as H
    tensors = H._tensors(3)
    rng = np.random.default_rng(4)
    calls = []
    for qtype in ("choice", "noul", "score", "choice"):
        s, q = H._unit(rng), H._unit(rng)
        opts = [(f"o{len(calls)}{i}", H._unit(rng)) for i in range(3)]
        calls.append((qtype, ("s", s) if len(calls) != 2 else ("s2", s), (f"q{len(calls)}", q), opts))
    js = node({"cmd": "eg2head", "config": H.CFG, "tensors": {k: [float(x) for x in v.reshape(-1)] for k, v in tensors.items()},
               "calls": [[t, [s[0], s[1].tolist()], [q[0], q[1].tolist()], [[k, e.tolist()] for k, e in o]] for t, s, q, o in calls]})
    head = Eg2Head(H.CFG, tensors)
    for got, (t, s, q, o) in zip(js, calls):
        want = head.logits(t, s, q, o)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6), (got, want)


def test_shared_prefix_packing_matches_python_host():
    """packShared (Node) == engine.pack_shared (Python) bit for bit, with and without groups."""
    load_pkg()
    from decision_js_amd import engine
    import test_host
    rng = np.random.default_rng(33)
    for groups in ([2, 1, 3], [1, 1], [4]):
        seqs = test_host._d3_seqs(rng, groups)
        for g in (groups, None):
            js = node({"cmd": "packshared", "seqs": seqs, "groups": g})
            py = engine.pack_shared(seqs, g)
            assert js["T"] == py["T"] and js["P"] == py["P"]
            for k in ("ids", "pos", "rng", "pairs"):
                assert np.array_equal(np.asarray(js[k]), py[k].reshape(-1)), k


def test_pass_splitting_matches_python_host():
    load_pkg()
    from decision_js_amd.d1 import Decision
    d = Decision.__new__(Decision)
    for sizes, budget in [([50, 300, 10, 500, 20], 400), ([1000], 10), ([5] * 9, 12), ([], 100)]:
        d.tokens_per_pass = budget
        assert node({"cmd": "passes", "sizes": sizes, "budget": budget}) == [list(p) for p in d._passes(sizes)]


def test_load_without_gpu_throws_the_library_error(tmp_path):
    if not os.path.exists(ADDON):
        pytest.skip("the Node binding is not built (no Node headers)")
    load_pkg()
    from decision_js_amd import synth
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present: the no-device path is not reachable")
    except ImportError:
        pass
    mdir = synth.generate(synth.reduced("qwen3-0.6b-q8", layers=1, vocab=512), str(tmp_path / "m"), seed=0)
    got = node({"cmd": "load", "model": mdir})
    assert got["error"].startswith("decision.js: no HIP device")


@pytest.mark.gpu
def test_node_decision_matches_python_host(tmp_path):
    """The same model, state and questions through the Node host and the Python host: identical logits (bit for
    bit) and probabilities; a malformed question throws the reference's message without wedging the queue;
    a batch under a token budget reports progress; shareState answers agree."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    from decision_js_amd.engine import DecoderEngine
    mdir = synth.generate(synth.reduced("qwen3-0.6b-q8", layers=3, vocab=4096), str(tmp_path / "m"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(6)
    V = 4096
    ids = lambda n: [int(x) for x in rng.integers(0, V, n)]  # noqa: E731
    opt = lambda: [int(rng.integers(0, V))]  # noqa: E731
    qs = {
        "topic": {"type": "choice", "instructions": "?", "criteria": {"billing": "", "delivery": "", "bug": ""},
                  "ids": ids(30), "options": [opt(), opt(), opt() + opt()]},
        "churn": {"type": "noul", "instructions": "?", "ids": ids(20), "options": [opt() + opt(), opt()]},
        "urgency": {"type": "score", "instructions": "?", "criteria": ["1", "2", "3", "4", "5"], "ids": ids(25),
                    "options": [opt() for _ in range(5)]},
    }
    state = ids(200)
    batch = [[ids(n), qs] for n in (50, 300, 10)]
    trees = [{"trunk": state, "branches": [q["ids"] for q in qs.values()], "groups": [q["options"] for q in qs.values()]}]
    js = node({"cmd": "decide", "model": mdir, "state": state, "questions": qs, "batch": batch, "budget": 400,
               "shared": True, "trees": trees}, timeout=300)
    d = Decision.load(mdir)
    try:
        py_one = d.system_one(state, qs)
        py_probs = d.probabilities(state, list(qs.values()))
        d.tokens_per_pass = 400
        py_batch = d.system_one_batch([tuple(b) for b in batch])
    finally:
        d.destroy()
    eng = DecoderEngine.load(mdir)
    try:
        py_logits = eng.run(trees)["logits"]
    finally:
        eng.destroy()
    assert np.array_equal(np.asarray(js["logits"], dtype=np.float32), py_logits)
    for a, b in zip(js["probs"], py_probs):
        assert np.allclose(a, b, rtol=0, atol=1e-12)
    assert js["one"]["usage"] == py_one["usage"] == {"input_tokens": 275, "output_tokens": 0}
    assert js["one"]["answers"]["topic"]["choice"] == py_one["answers"]["topic"]["choice"]
    assert abs(js["one"]["answers"]["churn"]["noul"] - py_one["answers"]["churn"]["noul"]) < 1e-12
    assert js["again"] == js["one"] and js["afterError"] == js["one"]
    assert js["badError"] == "decision.js: a choice needs criteria {name: description} with at least two options"
    assert js["progress"][-1] == [3, 3] and len(js["progress"]) >= 2
    assert js["progressP"] == js["progress"]  # probabilitiesBatch(requests, {onProgress}) as well
    for a, b in zip(js["probsBatch"], py_batch):
        assert abs(a[1][0] - b["answers"]["churn"]["noul"]) < 1e-12
    for a, b in zip(js["batch"], py_batch):
        assert abs(a["answers"]["churn"]["noul"] - b["answers"]["churn"]["noul"]) < 1e-12
    for n in qs:
        key = "noul" if n == "churn" else "confidence"
        assert abs(js["shared"]["answers"][n][key] - js["one"]["answers"][n][key]) < 5e-4
    assert js["shared2"] == js["shared"]


def test_graph_keys_from_second_use_match_python_host():
    """Both hosts run a forward's first use of a key eagerly (key 0), capture on the second and replay after;
    distinct forwards never share a key; a shared state's graphs are dropped when the state is freed (and
    only they); with graphs off every key is 0."""
    load_pkg()
    from decision_js_amd.engine import GpuEngine
    seq = [[["run", 100, 3, 5], None], [["run", 100, 3, 5], None], [["run", 100, 3, 5], None], [["run", 60, 3, 5], None],
           [["shared", 32, 8, 5], 1], [["run", 60, 3, 5], None], [["shared", 32, 8, 5], 2], [["shared", 32, 8, 5], 1],
           [["shared", 32, 8, 5], 1]]

    class FakeCtx:
        def __init__(self):
            self.dropped = []

        def graph_drop(self, key):
            self.dropped.append(key)

    class FakeState:
        serial = 1

        def free(self):
            pass

    def py_keys(graphs):
        e = GpuEngine.__new__(GpuEngine)
        e.graphs, e._gen, e._keys, e._state_keys, e.ctx = graphs, 0, {}, {}, FakeCtx()
        keys = [e._key(*parts, state=st) for parts, st in seq]
        e.free_state(FakeState())
        after = e._key(*seq[7][0], state=1)  # the freed state's forward starts over: eager
        return keys, [int(k) for k in e.ctx.dropped], after

    for graphs in (True, False):
        js = node({"cmd": "graphkeys", "graphs": graphs, "seq": seq, "free": 1})
        py = py_keys(graphs)
        for keys, dropped, after in ([int(k) for k in js["keys"]], [int(k) for k in js["dropped"]], int(js["after"])), py:
            if not graphs:
                assert keys == [0] * len(seq) and dropped == [] and after == 0
                continue
            assert keys[0] == 0 and keys[1] == keys[2] != 0  # eager, capture, replay
            assert keys[3] == 0 and keys[5] not in (0, keys[1])  # another shape: eager, then its own graph
            assert keys[4] == 0 and keys[6] == 0  # a new state's questions: eager each time
            assert keys[7] == keys[8] != 0 and keys[7] not in (keys[1], keys[5])  # state 1's second use
            assert dropped == [keys[7]] and after == 0


@pytest.mark.gpu
def test_node_question_alone_matches_python_host(tmp_path):
    """One 24-token question on a prefilled 300-token state through each host's DecoderEngine: with the q/k
    norm folded into attention (the default for at most 64 rows) and without it, the Node host's scores equal
    the Python host's bit for bit, on eager runs, graph capture and replay alike."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.engine import DecoderEngine
    mdir = synth.generate(synth.reduced("qwen3-0.6b-q8", layers=3, vocab=4096), str(tmp_path / "m"), seed=2, norm_std=0.1)
    rng = np.random.default_rng(9)
    state = [int(x) for x in rng.integers(0, 4096, 300)]
    branches = [[int(x) for x in rng.integers(0, 4096, 24)]]
    groups = [[[int(a)] for a in rng.choice(4096, 4, replace=False)]]
    py = {}
    for on in (True, False):
        eng = DecoderEngine.load(mdir, {"qk_attention": on})
        try:
            st = eng.prefill(state)
            py[on] = eng.run_shared(st, branches, groups)
            st.free()
        finally:
            eng.destroy()
    assert py[True] == py[False]
    for on in (True, False):
        js = node({"cmd": "question", "model": mdir, "state": state, "branches": branches, "groups": groups,
                   "opts": {"qkAttention": on}}, timeout=300)
        assert js["qkAttention"] == on
        for run in js["runs"]:
            assert run == py[True]


@pytest.mark.gpu
def test_node_encoder_matches_python_host(tmp_path):
    """The EmbeddingGemma-shaped encoder through the Node host (D1 kind "eg2", runEg2 with the learned decision
    head) against the Python host: the same embeddings and probabilities, progress through BatchOptions, and
    cached texts skipped on the second call."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    cfg = synth.reduced("eg2-encoder-q8", layers=2, vocab=2048, learned_head={"width": 64})
    mdir = synth.generate(cfg, str(tmp_path / "enc"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(8)
    ids = lambda n: [int(x) for x in rng.integers(0, 2048, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": ""}, "ids": ids(24),
                    "option_ids": [ids(8), ids(8), ids(6)]},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(20), "option_ids": [ids(3), ids(2)]}}
    batch = [[ids(n), qs] for n in (60, 33)]
    texts = [ids(n) for n in (12, 1, 40)]
    js = node({"cmd": "encode", "model": mdir, "batch": batch, "texts": texts}, timeout=300)
    assert js["kind"] == "eg2" and js["tokensPerPass"] == 8192
    d = Decision.load(mdir)
    try:
        py = d.system_one_batch([tuple(b) for b in batch])
        emb = d.engine.embed(texts)["embeddings"]
    finally:
        d.destroy()
    assert np.allclose(np.asarray(js["embeddings"], dtype=np.float32), emb, rtol=0, atol=1e-6)
    for a, b in zip(js["batch"], py):
        assert a["answers"]["topic"]["choice"] == b["answers"]["topic"]["choice"]
        assert abs(a["answers"]["topic"]["confidence"] - b["answers"]["topic"]["confidence"]) < 1e-6
        assert abs(a["answers"]["churn"]["noul"] - b["answers"]["churn"]["noul"]) < 1e-6
        assert a["usage"] == b["usage"]
    assert js["progress"] and js["progress"][-1][0] == js["progress"][-1][1]
    assert js["again"][0]["usage"]["input_tokens"] == 0 and js["again"][0]["answers"] == js["batch"][0]["answers"]


@pytest.mark.gpu
def test_node_injected_fault_surfaces_and_next_call_succeeds(tmp_path):
    """DJ_FAULT_INJECT=matmul:1 in the Node process: the first forward rejects with the library's "decision.js:
    fault injected in matmul" error (the recording aborted), and the next calls give the Python host's clean
    probabilities."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    mdir = synth.generate(synth.reduced("qwen3-0.6b-q8", layers=2, vocab=4096), str(tmp_path / "m"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(12)
    ids = lambda n: [int(x) for x in rng.integers(0, 4096, n)]  # noqa: E731
    qs = {"churn": {"type": "noul", "instructions": "?", "ids": ids(20), "options": [[5], [6, 7]]},
          "topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": ""}, "ids": ids(9), "options": [[1], [2]]}}
    state = ids(150)
    js = node({"cmd": "fault", "model": mdir, "state": state, "questions": qs}, timeout=300, env={"DJ_FAULT_INJECT": "matmul:1"})
    assert js["error"].startswith("decision.js: fault injected in matmul")
    d = Decision.load(mdir)
    try:
        want = d.probabilities(state, list(qs.values()))
    finally:
        d.destroy()
    for got in (js["after"], js["again"]):
        for a, b in zip(got, want):
            assert np.allclose(a, b, rtol=0, atol=1e-12)


@pytest.mark.gpu
def test_node_d3_matches_python_host(tmp_path):
    """The d3 kind through Node (kindOf -> runD3 -> logitsD3 -> READOUT) against the Python host: identical code
    logits (the same packing, op sequence and library) with and without shareState."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    mdir = synth.generate(synth.reduced("d3-attn-0.8b-q8", layers=2, vocab=4096), str(tmp_path / "d3"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(14)
    ids = lambda n: [int(x) for x in rng.integers(0, 4096, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": "", "d": ""}, "ids": ids(16)},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(5)}}
    batch = [[ids(90), qs], [ids(33), qs]]
    js = node({"cmd": "d3", "model": mdir, "batch": batch}, timeout=300)
    assert js["kind"] == "d3"
    d = Decision.load(mdir)
    try:
        for share, key in ((False, "plain"), (True, "shared")):
            d.share_state = share
            py = d.probabilities_batch([(s, list(q.values())) for s, q in batch])
            for a, b in zip(js[key], py):
                for x, y in zip(a, b):
                    assert np.allclose(x, y, rtol=0, atol=1e-12)
    finally:
        d.destroy()


@pytest.mark.gpu
def test_node_lfm2_matches_python_host(tmp_path):
    """A model with LFM2 conv layers through the Node host (taps packed in packForest, dj_short_conv in the
    layer loop) gives the Python host's logits bit for bit."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.engine import DecoderEngine
    cfg = synth.reduced("lfm2-d1-3b-q4", layers=3, vocab=4096, layer_types=["conv", "full_attention", "conv"])
    mdir = synth.generate(cfg, str(tmp_path / "lfm2"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(16)
    trees = _trees(rng, V=4096)
    js = node({"cmd": "logits", "model": mdir, "trees": trees}, timeout=300)
    eng = DecoderEngine.load(mdir)
    try:
        py = eng.run(trees)["logits"]
    finally:
        eng.destroy()
    assert np.array_equal(np.asarray(js["logits"], dtype=np.float32), py)


def test_omni_packing_matches_python_host():
    """packOmni (Node) == omni.pack_omni (Python) bit for bit."""
    load_pkg()
    from decision_js_amd import omni
    seqs = [{"ids": [5, 6, 7, 8], "markers": [1, 3], "type": "choice"}, {"ids": [1], "markers": [0], "type": "noul"},
            {"ids": list(range(30)), "markers": [0, 10, 29], "type": "score"}]
    js = node({"cmd": "packomni", "seqs": seqs})
    py = omni.pack_omni(seqs)
    assert js["T"] == py["T"] and js["M"] == py["M"]
    for k in ("ids", "pos", "qtype", "taps", "rng", "markers"):
        assert np.array_equal(np.asarray(js[k]), py[k].reshape(-1)), k


def test_laya_packing_and_prompt_match_python_host():
    """packLaya (Node) == laya.pack_laya (Python) bit for bit, windows included; idPrompt.sequenceLaya gives
    IdPrompt.sequence_laya's sequences and the same refusals."""
    load_pkg()
    from decision_js_amd import laya
    from decision_js_amd.d1 import IdPrompt
    seqs = [{"ids": list(range(40)), "markers": [3, 9, 30], "type": "choice"}, {"ids": [1], "markers": [0], "type": "noul"},
            {"ids": list(range(13)), "markers": [0, 12], "type": "score"}]
    for w in (0, 2, 64):
        js = node({"cmd": "packlaya", "seqs": seqs, "window": w})
        py = laya.pack_laya(seqs, w)
        assert js["T"] == py["T"] and js["M"] == py["M"]
        for k in ("ids", "pos", "qtype", "rng", "win", "markers"):
            assert np.array_equal(np.asarray(js[k]), py[k].reshape(-1)), (w, k)
    q = {"type": "noul", "instructions": "?", "ids": [1, 2, 3, 4, 5], "markers": [1, 3]}
    calls = [[[9, 8, 7], q, 512], [{"ids": [9, 8, 7]}, q, 6], [[9], q, 3], [[9], dict(q, markers=[1, 5]), 512]]
    js = node({"cmd": "layaprompt", "calls": calls})
    p = IdPrompt()
    for (state, qq, L), got in zip(calls, js):
        try:
            want = p.sequence_laya(state, qq, L)
        except Exception as e:  # noqa: BLE001
            assert got == {"error": str(e)}
        else:
            assert got == want


@pytest.mark.gpu
def test_node_laya_matches_python_host(tmp_path):
    """The laya kind through Node (kindOf -> runOmni with sequenceLaya -> LayaEngine: ModernBERT encoder, head,
    scorer) against the Python host: identical marker logits (the same packing, op sequence and library) and the
    same answers."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    cfg = synth.reduced("laya-q8", layers=3, vocab=4096, window=8,
                        layer_types=["full_attention", "sliding_attention", "sliding_attention"])
    mdir = synth.generate(cfg, str(tmp_path / "laya"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(19)
    ids = lambda n: [int(x) for x in rng.integers(0, 4096, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": ""}, "ids": ids(16),
                    "markers": [2, 7, 12]},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(6), "markers": [1, 4]},
          "urgency": {"type": "score", "instructions": "?", "criteria": ["low", {"x": 2.5}], "ids": ids(9), "markers": [3, 6]}}
    batch = [[ids(70), qs], [ids(600), qs]]  # the second state runs past max_len
    seqs = [{"ids": ids(40), "markers": [3, 9, 30], "type": "choice"}, {"ids": ids(12), "markers": [0, 11], "type": "noul"}]
    js = node({"cmd": "omni", "model": mdir, "batch": batch, "seqs": seqs}, timeout=300)
    assert js["kind"] == "laya"
    d = Decision.load(mdir)
    try:
        assert d.kind == "laya"
        py = d.system_one_batch([(s, q) for s, q in batch])
        for a, b in zip(js["batch"], py):
            assert a["usage"] == b["usage"]
            assert abs(a["answers"]["churn"]["noul"] - b["answers"]["churn"]["noul"]) < 1e-12
            assert a["answers"]["topic"]["choice"] == b["answers"]["topic"]["choice"]
            assert abs(a["answers"]["urgency"]["confidence"] - b["answers"]["urgency"]["confidence"]) < 1e-12
        want = d.engine.logits(seqs)["logits"]
        for a, b in zip(js["logits"], want):
            assert np.array_equal(np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32))
    finally:
        d.destroy()


@pytest.mark.gpu
def test_node_omni_matches_python_host(tmp_path):
    """The d1-omni kind through Node (kindOf -> runOmni -> OmniEngine: trunk, head, scorer) against the Python
    host: identical marker logits (the same packing, op sequence and library) and the same answers."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    cfg = synth.reduced("d1-omni-q8", layers=3, vocab=4096, layer_types=["conv", "full_attention", "conv"])
    mdir = synth.generate(cfg, str(tmp_path / "omni"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(17)
    ids = lambda n: [int(x) for x in rng.integers(0, 4096, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": ""}, "ids": ids(16),
                    "markers": [2, 7, 12]},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(6), "markers": [1, 4]},
          "urgency": {"type": "score", "instructions": "?", "criteria": ["low", {"x": 2.5}], "ids": ids(9), "markers": [3, 6]}}
    batch = [[ids(70), qs], [ids(25), qs]]
    seqs = [{"ids": ids(40), "markers": [3, 9, 30], "type": "choice"}, {"ids": ids(12), "markers": [0, 11], "type": "noul"}]
    js = node({"cmd": "omni", "model": mdir, "batch": batch, "seqs": seqs}, timeout=300)
    assert js["kind"] == "d1-omni"
    d = Decision.load(mdir)
    try:
        assert d.kind == "d1-omni"
        py = d.system_one_batch([(s, q) for s, q in batch])
        for a, b in zip(js["batch"], py):
            assert a["usage"] == b["usage"]
            assert abs(a["answers"]["churn"]["noul"] - b["answers"]["churn"]["noul"]) < 1e-12
            assert a["answers"]["topic"]["choice"] == b["answers"]["topic"]["choice"]
            assert a["answers"]["urgency"]["legend"] == b["answers"]["urgency"]["legend"] == {"0": "low", "1": '{"x": 2.5}'}
        want = d.engine.logits(seqs)["logits"]
        for a, b in zip(js["logits"], want):
            assert np.array_equal(np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32))
    finally:
        d.destroy()


def test_gdn_spans_match_python_host():
    """gdnSpans (Node) == d3.gdn_spans (Python) bit for bit, with and without groups."""
    load_pkg()
    from decision_js_amd import d3
    rng = np.random.default_rng(6)
    state = [int(x) for x in rng.integers(0, 9, 12)]
    seqs = [{"ids": state + [int(x) for x in rng.integers(0, 9, n)], "options": 2} for n in (3, 1, 7, 2)]
    for groups in (None, [3, 1], [4], [1, 1, 2]):
        js = node({"cmd": "gdnspans", "seqs": seqs, "groups": groups})
        assert np.array_equal(np.asarray(js, dtype=np.uint32), d3.gdn_spans(seqs, groups).reshape(-1)), groups


@pytest.mark.gpu
def test_node_d3_lite_matches_python_host(tmp_path):
    """The shipped d3-lite layout through Node (kindOf -> runD3 -> D3Engine: DeltaNet and gated attention layers,
    READOUT) against the Python host: identical code probabilities with and without shareState."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    cfg = synth.reduced("d3-lite-q8", layers=4, vocab=4096,
                        layer_types=["linear_attention", "linear_attention", "linear_attention", "full_attention"])
    mdir = synth.generate(cfg, str(tmp_path / "d3lite"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(18)
    ids = lambda n: [int(x) for x in rng.integers(0, 4096, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": "", "c": "", "d": ""}, "ids": ids(16)},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(5)}}
    batch = [[ids(90), qs], [ids(33), qs]]
    js = node({"cmd": "d3", "model": mdir, "batch": batch}, timeout=300)
    assert js["kind"] == "d3"
    d = Decision.load(mdir)
    try:
        assert type(d.engine).__name__ == "D3Engine"
        for share, key in ((False, "plain"), (True, "shared")):
            d.share_state = share
            py = d.probabilities_batch([(s, list(q.values())) for s, q in batch])
            for a, b in zip(js[key], py):
                for x, y in zip(a, b):
                    assert np.allclose(x, y, rtol=0, atol=1e-12)
    finally:
        d.destroy()


@pytest.mark.gpu
def test_node_eg2_shipped_matches_python_host(tmp_path):
    """The shipped EmbeddingGemma 2 through Node (kindOf -> runEg2 -> Eg2Engine, the learned head) against the
    Python host: the same answers and embeddings."""
    load_pkg()
    from decision_js_amd import synth
    from decision_js_amd.d1 import Decision
    cfg = synth.reduced("eg2-q8", layers=3, vocab=4096, window=16,
                        layer_types=["sliding_attention", "full_attention", "sliding_attention"])
    mdir = synth.generate(cfg, str(tmp_path / "eg2ship"), seed=0, norm_std=0.1)
    rng = np.random.default_rng(19)
    ids = lambda n: [int(x) for x in rng.integers(0, 4096, n)]  # noqa: E731
    qs = {"topic": {"type": "choice", "instructions": "?", "criteria": {"a": "", "b": ""}, "ids": ids(24),
                    "option_ids": [ids(8), ids(6)]},
          "churn": {"type": "noul", "instructions": "?", "ids": ids(20), "option_ids": [ids(3), ids(2)]}}
    batch = [[ids(100), qs], [ids(37), qs]]
    texts = [ids(30), ids(1), ids(64)]
    js = node({"cmd": "encode", "model": mdir, "batch": batch, "texts": texts}, timeout=300)
    assert js["kind"] == "eg2"
    d = Decision.load(mdir)
    try:
        py = d.system_one_batch(batch)
        for a, b in zip(js["batch"], py):
            assert a["usage"] == b["usage"]
            assert abs(a["answers"]["churn"]["noul"] - b["answers"]["churn"]["noul"]) < 1e-6
            assert abs(a["answers"]["topic"]["confidence"] - b["answers"]["topic"]["confidence"]) < 1e-6
        emb = d.engine.embed(texts)["embeddings"]
        assert np.allclose(np.asarray(js["embeddings"], dtype=np.float32), emb, rtol=0, atol=1e-6)
    finally:
        d.destroy()
