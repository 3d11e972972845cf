"""Host-side logic on the CPU: the Decision API's queue, passes, softmax and typed answers (with a stand-in
engine: no GPU), question validation, packing, the weights format, and the synthetic generator."""
import os

import numpy as np
import pytest

from oracle import ref


class FakeDecoder:
    """Scores every option by its token id (so answers are predictable) and records the passes."""

    def __init__(self, fail_once=False):
        self.passes, self.fail_once = [], fail_once

    def run(self, trees):
        if self.fail_once:
            self.fail_once = False
            raise RuntimeError("decision.js: injected failure")
        self.passes.append(sum(len(t["trunk"]) + sum(len(b) for b in t["branches"]) for t in trees))
        return {"scores": [[[float(max(g)) / 10 for g in groups] for groups in t["groups"]] for t in trees]}

    def destroy(self):
        pass


def _qs():
    return {
        "topic": {"type": "choice", "instructions": "?", "criteria": {"a": None, "b": None, "c": None}, "ids": [1, 2],
                  "options": [[5], [30, 7], [20]]},
        "churn": {"type": "noul", "instructions": "?", "ids": [3], "options": [[10], [1, 2]]},
        "urgency": {"type": "score", "instructions": "?", "criteria": ["low", "mid", "high"], "ids": [4, 4, 4],
                    "options": [[1], [2], [3]]},
    }


def test_system_one_answers(pkg):
    from decision_js_amd import d1
    D = d1.Decision("d1-3b", FakeDecoder(), d1.IdPrompt(), 4096)
    r = D.system_one([9, 9, 9, 9], _qs())
    a = r["answers"]
    assert a["topic"]["choice"] == "b" and abs(sum(a["topic"]["probabilities"].values()) - 1) < 1e-12
    want = ref.softmax([0.5, 3.0, 2.0])
    assert abs(a["topic"]["confidence"] - want[1]) < 1e-12
    assert abs(a["churn"]["noul"] - ref.softmax([1.0, 0.2])[0]) < 1e-12  # [yes, no] as given (run3B: no reversal)
    p = ref.softmax([0.1, 0.2, 0.3])
    assert abs(a["urgency"]["score"] - (p[1] + 2 * p[2])) < 1e-12 and a["urgency"]["legend"] == {"0": "low", "1": "mid", "2": "high"}
    assert r["usage"] == {"input_tokens": 4 + 2 + 1 + 3, "output_tokens": 0}


def test_passes_follow_the_token_budget(pkg):
    """Whole requests per pass up to tokensPerPass; a pass always takes at least one (d1.ts:217-219)."""
    from decision_js_amd import d1
    eng = FakeDecoder()
    D = d1.Decision("d1-3b", eng, d1.IdPrompt(), 20)
    reqs = [([1] * n, _qs()) for n in (5, 4, 30, 1, 1)]  # each request adds 6 question tokens
    seen = []
    out = D.system_one_batch(reqs, {"on_progress": lambda a, b: seen.append((a, b))})  # BatchOptions (d1.ts:33-35)
    assert eng.passes == [11, 10, 36, 14] and seen == [(1, 5), (2, 5), (3, 5), (5, 5)]
    assert [o["usage"]["input_tokens"] for o in out] == [11, 10, 36, 7, 7]
    as_lists = [(s, list(q.values())) for s, q in reqs]
    assert D.probabilities_batch(as_lists)[2] == D.probabilities(*as_lists[2])


def test_a_failed_call_does_not_wedge_the_queue(pkg):
    from decision_js_amd import d1
    D = d1.Decision("d1-3b", FakeDecoder(fail_once=True), d1.IdPrompt(), 4096)
    with pytest.raises(RuntimeError, match="decision.js: injected failure"):
        D.system_one([1], _qs())
    assert D.system_one([1], _qs())["answers"]["topic"]["choice"] == "b"


@pytest.mark.parametrize("q,msg", [
    ({"type": "choice", "instructions": "x", "criteria": {"a": 1}}, "at least two options"),
    ({"type": "score", "instructions": "x", "criteria": ["a"]}, "2 to 10"),
    ({"type": "score", "instructions": "x", "criteria": list(range(11))}, "2 to 10"),
    ({"type": "noul", "instructions": "x", "criteria": [1]}, "noul criteria are optional"),
    ({"type": "maybe", "instructions": "x"}, "must be noul, choice or score"),
    ({"type": "noul"}, "is an object with"),
])
def test_check_question(pkg, q, msg):
    from decision_js_amd import d1, questions
    with pytest.raises(questions.QuestionError, match=msg):
        questions.check_question(q)
    D = d1.Decision("d1-3b", FakeDecoder(), d1.IdPrompt(), 4096)
    with pytest.raises(questions.QuestionError):
        D.system_one([1], {"q": q})


def test_option_group_count_must_match(pkg):
    from decision_js_amd import d1, questions
    q = dict(_qs()["urgency"], options=[[1], [2]])
    D = d1.Decision("d1-3b", FakeDecoder(), d1.IdPrompt(), 4096)
    with pytest.raises(questions.QuestionError, match="option groups"):
        D.system_one([1], {"u": q})


def test_engine_packing_and_helpers(pkg):
    from decision_js_amd import engine
    rng = np.random.default_rng(1)
    trees = [{"trunk": list(rng.integers(0, 50, 12)), "branches": [list(rng.integers(0, 50, n)) for n in (3, 1, 7)],
              "groups": [[[1, 2], [3]], [[4]], [[5], [6, 7, 8]]]}, {"trunk": [], "branches": [[1, 2]], "groups": [[[9]]]}]
    pk = engine.pack_forest(trees)
    ids, pos, meta, leaves, leaf_ids, n_ids = ref.pack_forest(trees)
    assert np.array_equal(pk["ids"], ids) and np.array_equal(pk["meta"], meta) and np.array_equal(pk["leaves"], leaves)
    assert np.array_equal(pk["leaf_ids"], leaf_ids) and pk["n_ids"] == n_ids == 4
    assert np.array_equal(ref.ranges_mask(pk["rng"], pk["T"]), ref.forest_mask(meta))
    assert np.array_equal(pk["taps"], ref.forest_taps(trees))  # the short conv's taps, bit for bit
    assert engine.common_prefix([[1, 2, 3], [1, 2, 4], [1, 2]]) == 1
    assert engine.common_prefix([[1, 2, 3, 4], [1, 2, 3, 5]]) == 3 and engine.common_prefix([[1, 2]]) == 0
    out = np.random.default_rng(5).standard_normal(4 * 4).astype(np.float32)
    per_tree = engine.group_max(out, 4, trees)
    assert [len(t) for t in per_tree] == [3, 1]
    assert [s for t in per_tree for s in t] == ref.group_max(out, 4, [g for t in trees for g in t["groups"]])
    # known answer: leaf 2 (tree 0, question 2) has groups [5] and [6, 7, 8] over out[8:12]
    assert per_tree[0][2] == [float(out[8]), float(out[9:12].max())]


def test_encoder_packing_matches_oracle_bit_exact(pkg):
    """encoder.pack_encoder (the engine's host packing) == the oracle's restatement of eg2-engine.ts:74-86,
    bit for bit: ids, meta, full and windowed key ranges, per-text ranges; empty-free ragged texts, one-token
    texts, windows wider than a text."""
    from decision_js_amd import encoder
    rng = np.random.default_rng(6)
    for window in (None, 0, 3, 50):
        seqs = [[int(x) for x in rng.integers(0, 1000, n)] for n in (1, 17, 2, 64, 5)]
        got = encoder.pack_encoder(seqs, window)
        ids, meta, full, slide, ranges = ref.pack_encoder(seqs, window)
        assert got["T"] == len(ids) and got["S"] == len(seqs)
        assert got["ids"].dtype == ids.dtype and np.array_equal(got["ids"], ids)
        assert got["meta"].dtype == meta.dtype and np.array_equal(got["meta"], meta)
        assert np.array_equal(got["full"], full) and np.array_equal(got["ranges"], ranges)
        if window is None:
            assert got["slide"] is None and slide is None
        else:
            assert np.array_equal(got["slide"], slide)


def test_format_roundtrip(pkg, tmp_path):
    from decision_js_amd import fmt
    rng = np.random.default_rng(2)
    b = fmt.Blob(str(tmp_path), {"model": "decoder", "x": 1}, 8)
    w8 = rng.standard_normal((64, 96)).astype(np.float32) * 0.02
    w4 = rng.standard_normal((32, 64)).astype(np.float32) * 0.02
    b.quant("a", w8)
    b.quant("b", w4, bits=4)
    b.f16("n", np.ones(7))
    b.f32("h", np.arange(5))
    b.close()
    m = fmt.load_manifest(str(tmp_path))
    t = m["tensors"]
    assert all(v["offset"] % 256 == 0 for v in t.values()) and all(v.get("scales", 0) % 256 == 0 for v in t.values())
    assert t["a"] == {"dtype": "q8", "shape": [64, 96], "offset": t["a"]["offset"], "bytes": 64 * 96, "scales": t["a"]["scales"],
                      "scales_bytes": 64 * 3 * 2}
    assert m["format"] == "d1.js/1" and m["bytes"] == os.path.getsize(tmp_path / "weights.bin")
    tf = fmt.TensorFile(str(tmp_path))
    c, s = tf.tensor(t["a"])
    c2, s2, _ = fmt.quantize8(w8)
    assert np.array_equal(c, c2) and np.array_equal(s, s2)
    c, s = tf.tensor(t["b"])
    assert c.shape == (32, 32) and np.array_equal(c, fmt.quantize4(w4)[0])
    assert np.array_equal(tf.tensor(t["h"]), np.arange(5, dtype=np.float32))
    with pytest.raises(ValueError, match="range read returned"):
        tf.range(m["bytes"] - 4, 16)


def test_synthetic_generator(pkg, tmp_path):
    from decision_js_amd import fmt, synth
    cfg = synth.reduced("qwen3-0.6b-q8", layers=2, vocab=512)
    p = synth.generate(cfg, str(tmp_path / "m"), norm_std=0.1)
    m = fmt.load_manifest(p)
    assert m["tensors"]["layers.1.qkv"]["shape"] == [(16 + 16) * 128, 1024]
    assert m["tensors"]["layers.0.w13"]["shape"] == [6144, 1024] and m["tensors"]["embed"]["shape"] == [512, 1024]
    mt = os.path.getmtime(os.path.join(p, "weights.bin"))
    assert synth.generate(cfg, p, norm_std=0.1) == p and os.path.getmtime(os.path.join(p, "weights.bin")) == mt  # cached
    a = synth.normal("x", (4,), seed=0)
    assert np.array_equal(a, synth.normal("x", (4,), seed=0)) and not np.array_equal(a, synth.normal("y", (4,), seed=0))


def _d3_seqs(rng, groups):
    """Requests whose questions share a state prefix (sometimes all of a question, sometimes nothing)."""
    seqs = []
    for n in groups:
        state = [int(x) for x in rng.integers(0, 50, rng.integers(0, 12))]
        for _ in range(n):
            q = [int(x) for x in rng.integers(0, 50, rng.integers(1, 6))]
            seqs.append({"ids": state + q, "options": int(rng.integers(1, 5))})
    return seqs


def test_shared_prefix_packing_matches_oracle_bit_exact(pkg):
    """engine.pack_shared (the product path of D3Engine.logits's packing, d3-engine.ts:67-93) equals the oracle's
    restatement bit for bit: ids, key ranges, (row, code) pairs, and positions = the oracle's meta positions;
    ragged groups, one-question groups, identical questions (the prefix stops one token short), no groups."""
    from decision_js_amd import engine
    rng = np.random.default_rng(31)
    cases = [[1, 3, 2], [4], [1, 1, 1], [2, 2]]
    for groups in cases:
        seqs = _d3_seqs(rng, groups)
        if groups == [2, 2]:
            seqs[1]["ids"] = list(seqs[0]["ids"])  # two identical questions: each keeps its last token
        for g in (groups, None):
            got = engine.pack_shared(seqs, g)
            ids, meta, r, pairs = ref.pack_shared(seqs, g)
            assert np.array_equal(got["ids"], ids) and np.array_equal(got["rng"], r)
            assert np.array_equal(got["pos"], meta[:, 3]) and np.array_equal(got["pairs"], pairs)
            assert got["T"] == len(ids) and got["P"] == len(pairs)
    with pytest.raises(ValueError, match="groups cover"):
        engine.pack_shared(_d3_seqs(rng, [2]), [3])


class FakeD3:
    """logits_d3 stand-in: code k of a sequence scores k * (its length) / 10; records the groups it was given."""

    def __init__(self, temperature=2.0):
        self.calls, self.m = [], {"config": {"temperature": temperature}}

    def logits_d3(self, seqs, groups=None):
        self.calls.append((len(seqs), groups))
        return [[k * len(s["ids"]) / 10 for k in range(s["options"])] for s in seqs]

    def destroy(self):
        pass


def test_run_d3_temperature_noul_and_groups(pkg):
    """runD3 (d1.ts:150-169): one sequence per question (state ids then question ids) with its option count,
    softmax at the model's temperature, a noul reversed to [yes, no]; share_state passes each request's question
    count as its group; passes follow the token budget."""
    from decision_js_amd import d1
    eng = FakeD3()
    D = d1.Decision("d3", eng, d1.IdPrompt(), 4096)
    qs = _qs()
    r = D.system_one([9] * 5, qs)
    n = {"topic": 5 + 2, "churn": 5 + 1, "urgency": 5 + 3}
    want_topic = ref.softmax([k * n["topic"] / 10 / 2.0 for k in range(3)])
    assert abs(r["answers"]["topic"]["confidence"] - max(want_topic)) < 1e-12
    churn = ref.softmax([0.0, n["churn"] / 10 / 2.0])
    assert abs(r["answers"]["churn"]["noul"] - churn[1]) < 1e-12  # [false, true] reversed
    assert eng.calls == [(3, None)]
    D.share_state = True
    D.probabilities_batch([([1, 2], list(qs.values())), ([3], list(qs.values())[:2])])
    assert eng.calls[-1] == (5, [3, 2])


def _omni_seqs(rng, n):
    types = ["choice", "noul", "score"]
    out = []
    for k in range(n):
        L = int(rng.integers(1, 12))
        out.append({"ids": [int(x) for x in rng.integers(0, 50, L)], "type": types[k % 3],
                    "markers": sorted(int(x) for x in rng.choice(L, min(L, int(rng.integers(1, 4))), replace=False))})
    return out


def test_omni_packing_matches_oracle_bit_exact(pkg):
    """omni.pack_omni (the product path of D1OmniEngine.logits's packing, omni-engine.ts:62-75) equals the
    oracle's restatement bit for bit: ids, positions, question types, centred taps that never cross a sequence
    (one-token sequences read only themselves), key ranges, marker rows; a marker past its sequence is refused."""
    from decision_js_amd import omni
    rng = np.random.default_rng(8)
    for n in (1, 2, 5, 9):
        seqs = _omni_seqs(rng, n)
        got, want = omni.pack_omni(seqs), ref.pack_omni(seqs)
        for k in ("ids", "pos", "qtype", "taps", "rng", "markers"):
            assert got[k].dtype == want[k].dtype and np.array_equal(got[k], want[k]), k
        assert got["T"] == want["T"] and got["M"] == len(want["markers"])
    one = omni.pack_omni([{"ids": [7], "markers": [0], "type": "noul"}])
    assert one["taps"].tolist() == [[-1, 0, -1, 0]] and one["qtype"].tolist() == [2]
    with pytest.raises(ValueError, match="marker outside"):
        omni.pack_omni([{"ids": [1, 2], "markers": [2], "type": "choice"}])


def test_laya_packing_windows_bit_exact(pkg):
    """laya.pack_laya (laya-engine.ts:57-66) is pack_omni plus each token's window; the windows equal the oracle's
    per-token restatement bit for bit, and (the oracle pinned by the mask they stand for) a token sees key j
    exactly when j is in its sequence and |t - j| <= window."""
    from decision_js_amd import laya
    rng = np.random.default_rng(9)
    for n, w in ((1, 0), (3, 1), (7, 2), (9, 64)):
        seqs = _omni_seqs(rng, n)
        got, want = laya.pack_laya(seqs, w), ref.pack_omni(seqs)
        for k in ("ids", "pos", "qtype", "rng", "markers"):
            assert np.array_equal(got[k], want[k]), k
        win = ref.laya_windows(want["rng"], w)
        assert got["win"].dtype == win.dtype and np.array_equal(got["win"], win)
        T = want["T"]
        t = np.arange(T)
        same = (want["rng"][:, None, 0] == want["rng"][None, :, 0])
        assert np.array_equal(ref.ranges_mask(win, T), same & (np.abs(t[:, None] - t[None, :]) <= w))


def test_laya_id_prompt_layout(pkg):
    """IdPrompt.sequence_laya (laya-prompt.ts:27-56 on ids): the question's ids first and the state's after, cut
    to max_len; markers index the question's ids unshifted; a marker past max_len is refused with the reference's
    message, one outside the question's ids as for d1-omni."""
    from decision_js_amd import questions as Q
    from decision_js_amd.d1 import IdPrompt
    p = IdPrompt()
    q = {"type": "noul", "instructions": "?", "ids": [1, 2, 3, 4, 5], "markers": [1, 3]}
    assert p.sequence_laya([9, 8, 7], q, 512) == {"ids": [1, 2, 3, 4, 5, 9, 8, 7], "markers": [1, 3], "type": "noul"}
    assert p.sequence_laya({"ids": [9, 8, 7]}, q, 6)["ids"] == [1, 2, 3, 4, 5, 9]
    assert p.sequence_laya([9], q, 4)["ids"] == [1, 2, 3, 4]
    with pytest.raises(Q.QuestionError, match="only 1 of the 2 option markers fit in 3 tokens"):
        p.sequence_laya([9], q, 3)
    with pytest.raises(Q.QuestionError, match="outside the question"):
        p.sequence_laya([9], dict(q, markers=[1, 5]), 512)
    with pytest.raises(Q.QuestionError, match="3 markers for a noul"):
        p.sequence_laya([9], dict(q, markers=[0, 1, 2]), 512)


def test_omni_temperature_keys(pkg):
    """temperature() of omni-engine.ts:22-26: the type:bucket key, else the type, else 1."""
    from decision_js_amd import omni
    c = {"temperatures": {"choice": 1.1, "choice:2": 1.05, "choice:3-5": 1.15, "score:6-10": 0.8, "noul": 1.2}}
    assert omni.temperature(c, "choice", 2) == 1.05 and omni.temperature(c, "choice", 5) == 1.15
    assert omni.temperature(c, "choice", 6) == 1.1 and omni.temperature(c, "score", 10) == 0.8
    assert omni.temperature(c, "score", 11) == 1.0 and omni.temperature(c, "noul", 2) == 1.2
    for k in (2, 3, 5, 6, 10, 11):
        assert omni.temperature(c, "choice", k) == ref.omni_temperature(c["temperatures"], "choice", k)


class FakeOmni:
    """OmniEngine.logits stand-in: marker j of a sequence scores j * (its length) / 10; records each pass."""

    def __init__(self, temps):
        self.calls, self.m = [], {"config": {"temperatures": temps}}

    def logits(self, seqs):
        self.calls.append([len(s["ids"]) for s in seqs])
        return {"logits": [[j * len(s["ids"]) / 10 for j in range(len(s["markers"]))] for s in seqs]}

    def destroy(self):
        pass


def test_run_omni_sequences_temperatures_and_noul(pkg):
    """runEncoder (d1.ts:121-147) for d1-omni: one sequence per question (state ids then question ids, markers
    shifted past the state), the temperature of the question's type and option-count bucket, a noul reversed
    from [false, true]; score legends rendered as omni's criterion (the text, else json.dumps); whole requests
    per pass up to the token budget; markers that do not match the options are refused."""
    from decision_js_amd import d1
    temps = {"choice:3-5": 2.0, "noul": 0.5, "score": 4.0}
    eng = FakeOmni(temps)
    D = d1.Decision("d1-omni", eng, d1.IdPrompt(), 30)
    qs = _qs()
    qs["topic"]["markers"] = [0, 1, 1]
    qs["churn"]["markers"] = [0, 0]
    qs["urgency"]["markers"] = [0, 1, 2]
    qs["urgency"]["criteria"] = ["low", {"x": 1.5}, 3]
    r = D.system_one([9] * 5, qs)
    n = {"topic": 7, "churn": 6, "urgency": 8}
    assert eng.calls == [[7, 6, 8]]
    assert abs(r["answers"]["topic"]["confidence"] - max(ref.softmax([j * 7 / 10 / 2.0 for j in range(3)]))) < 1e-12
    churn = ref.softmax([0.0, n["churn"] / 10 / 0.5])
    assert abs(r["answers"]["churn"]["noul"] - churn[1]) < 1e-12  # [false, true] reversed to [yes, no]
    assert r["answers"]["urgency"]["legend"] == {"0": "low", "1": '{"x": 1.5}', "2": "3"}
    assert r["usage"]["input_tokens"] == 21
    D.probabilities_batch([([1] * 10, list(qs.values())), ([2] * 3, list(qs.values()))])
    assert eng.calls[1:] == [[12, 11, 13], [5, 4, 6]]  # 36 tokens, then 15: one request per pass at 30
    bad = dict(qs["topic"], markers=[0, 1])
    with pytest.raises(d1.Q.QuestionError, match="2 markers for a choice with 3 options"):
        D.probabilities([1], [bad])


class FakeEncoder:
    """EncoderEngine stand-in for runEg2: the embedding of a text is its one-hot on its first id's axis."""

    def __init__(self):
        self.m, self.host = {"config": {"temperatures": {"noul": 1.0}}}, {}

    def embed(self, texts):
        e = np.zeros((len(texts), 8), np.float32)
        for k, t in enumerate(texts):
            e[k, t[0] % 8] = 1.0
        return {"embeddings": e}


def test_run_eg2_reverses_noul(pkg):
    """runEg2 (d1.ts:196-198): a noul's option texts are listed [no, yes] and its probabilities reversed to
    [yes, no]: with "yes" the option nearest to state + question, P(yes) is the larger."""
    from decision_js_amd import d1
    D = d1.Decision("eg2", FakeEncoder(), d1.IdPrompt(), 4096)
    q = {"type": "noul", "instructions": "?", "ids": [1], "option_ids": [[5], [1]]}  # no: axis 5, yes: axis 1
    p = D.probabilities([1], [q])[0]
    assert p[0] > p[1]
    r = D.system_one([1], {"q": q})
    assert r["answers"]["q"]["noul"] == p[0]
