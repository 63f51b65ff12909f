"""Laya decide layer (src/models/laya/decision.rs) on the CPU: lg_laya_decide_encode /
lg_laya_decide_scores against the token-level restatement in oracle/pydecide.py.

The restatement itself is pinned by hand-written layouts (the [cls] head [sep] ([mask] option)
[sep] state [sep] order, the 48-token option cut, the per-option cut when the options crowd the
head budget, the state room), by temperatures recovered from the probabilities (log p1/p0 =
(z1 - z0)/T), by the closed forms of uniform and one-hot outputs (confidence 0 and 1, ties to the
lower index, expected score) and by the act probability 1/(1 + e^(a1 - a0)).  The reference's own
goldens need the real checkpoint and tokenizer, which are absent.
"""
import math

import numpy as np
import pytest

import pydecide as pd

V = 1024
CLS, SEP, MASK = V - 3, V - 2, V - 1


@pytest.fixture(scope="module")
def tiny(lh, po):
    img = lh.SynthImage("laya-tiny", seed=7)
    return lh.Gguf.from_bytes(img), po.Gguf(img.array())


def q(kind, ins, opts):
    return {"type": kind, "instruction": ins, "options": [{"name": n, "desc": d} for n, d in opts]}


def test_spec_reads_the_synthetic_metadata(tiny):
    _, g = tiny
    s = pd.laya_spec(g)
    assert (s["max"], s["head_max"], s["cls"], s["sep"], s["mask"]) == (512, 192, CLS, SEP, MASK)
    assert s["temperature"] == [1.25, 0.9, 1.1] and s["buckets"] == {"choice:2": 1.05, "choice:3-5": 1.2}


def test_hand_written_layout(tiny, lh):
    h, g = tiny
    req = {"state": [100, 101, 102, 103, 104],
           "questions": [q("choice", [5, 6, 7], [([10], None), ([11, 12], [13])])]}
    want = [CLS, 5, 6, 7, SEP, MASK, 10, MASK, 11, 12, 13, SEP, 100, 101, 102, 103, 104, SEP]
    ids, mk = pd.laya_encode(pd.laya_spec(g), req, 0)
    assert ids == want and mk == [5, 7]
    got, gmk = lh.laya_decide_encode(h, req, 0)
    assert got.tolist() == want and gmk.tolist() == [5, 7]


def test_option_and_head_cuts(tiny, lh):
    h, g = tiny
    s = pd.laya_spec(g)
    # one long option: name + desc cut to 48 tokens after the mask
    req = {"state": [], "questions": [q("noul", list(range(300)), [(list(range(40)), list(range(40, 70))), ([1], None)])]}
    ids, mk = pd.laya_encode(s, req, 0)
    assert mk[1] - mk[0] == 49 and ids[mk[0] + 1:mk[1]] == list(range(48))
    # head keeps head_max - sum(options) = 192 - 51 tokens
    assert mk[0] == 1 + (192 - 51) + 1 and ids[1:mk[0] - 1] == list(range(141))
    assert np.array_equal(lh.laya_decide_encode(h, req, 0)[0], ids)
    # 16 options of 49 tokens crowd the head budget: each cut to (192 - 16) // 16 = 11, head to 16
    req = {"state": list(range(2000)), "questions": [q("choice", list(range(50)), [(list(range(60)), None)] * 16)]}
    ids, mk = pd.laya_encode(s, req, 0)
    assert np.diff(mk).tolist() == [11] * 15 and mk[0] == 1 + 16 + 1
    # the state fills the rest: exactly max_len tokens ending in [sep], its first tokens kept
    st = mk[-1] + 11 + 1
    assert len(ids) == 512 and ids[-1] == SEP and ids[st:st + 3] == [0, 1, 2] and ids[st - 1] == SEP
    got, gmk = lh.laya_decide_encode(h, req, 0)
    assert np.array_equal(got, ids) and np.array_equal(gmk, mk)


@pytest.mark.parametrize("seed", range(12))
def test_encode_matches_restatement(tiny, lh, seed):
    h, g = tiny
    rng = np.random.default_rng(seed)
    req = random_request(rng)
    s = pd.laya_spec(g)
    for i in range(len(req["questions"])):
        ids, mk = pd.laya_encode(s, req, i)
        got, gmk = lh.laya_decide_encode(h, req, i)
        assert got.tolist() == ids and gmk.tolist() == mk


def random_request(rng, nq=None):
    kinds = ("choice", "score", "noul")
    qs = []
    for _ in range(nq or int(rng.integers(1, 5))):
        kind = kinds[int(rng.integers(0, 3))]
        k = 2 if kind == "noul" else int(rng.integers(2 if kind == "score" else 1, 17))
        opts = [(rng.integers(0, 1000, int(rng.integers(0, 70))).tolist(),
                 rng.integers(0, 1000, int(rng.integers(0, 20))).tolist() if rng.random() < 0.5 else None)
                for _ in range(k)]
        qs.append(q(kind, rng.integers(0, 1000, int(rng.integers(0, 250))).tolist(), opts))
    return {"state": rng.integers(0, 1000, int(rng.integers(0, 700))).tolist(), "questions": qs}


@pytest.mark.parametrize("seed", range(12))
def test_scores_match_restatement(tiny, lh, seed):
    h, g = tiny
    rng = np.random.default_rng(100 + seed)
    req = random_request(rng)
    ks = [len(x["options"]) for x in req["questions"]]
    logits = (rng.standard_normal(sum(ks)) * 3).astype(np.float32)
    act = (rng.standard_normal((len(ks), 2)) * 2).astype(np.float32)
    got = lh.laya_decide_scores(h, req, logits, act)
    s = pd.laya_spec(g)
    outs, at = [], 0
    for i, k in enumerate(ks):
        outs.append((logits[at:at + k], act[i]))
        at += k
    want = pd.laya_aggregate(s, req, outs, sum(len(pd.laya_encode(s, req, i)[0]) for i in range(len(ks))))
    assert got["usage"]["input_tokens"] == want["input_tokens"]
    for a, b in zip(got["answers"], want["answers"]):
        assert np.array_equal(a["probabilities"], b["probabilities"])
        assert a["choice"] == b["choice"] and a["act_probability"] == np.float32(b["act_probability"])
        assert a["confidence"] == np.float32(b["confidence"])
        if "score" in b:
            assert a["score"] == np.float32(b["score"])


@pytest.mark.parametrize("kind,k,T", [("choice", 2, 1.05), ("choice", 3, 1.2), ("choice", 5, 1.2), ("choice", 6, 1.25),
                                      ("score", 2, 0.9), ("score", 11, 0.9), ("noul", 2, 1.1)])
def test_temperature_recovered_from_probabilities(tiny, lh, kind, k, T):
    h, g = tiny
    req = {"state": [1], "questions": [q(kind, [2], [([3], None)] * k)]}
    z = np.zeros(k, np.float32)
    z[1] = 2.0
    for got in (lh.laya_decide_scores(h, req, z, np.zeros((1, 2), np.float32))["answers"][0],
                pd.laya_aggregate(pd.laya_spec(g), req, [(z, np.zeros(2, np.float32))], 0)["answers"][0]):
        p = np.asarray(got["probabilities"], np.float64)
        assert 2.0 / math.log(p[1] / p[0]) == pytest.approx(T, rel=1e-5)


def test_closed_forms(tiny, lh):
    h, g = tiny
    req = {"state": [], "questions": [q("choice", [1], [([2], None)] * 4), q("score", [1], [([2], None)] * 3),
                                      q("noul", [1], [([2], None)] * 2), q("choice", [1], [([2], None)])]}
    logits = np.array([0.5, 0.5, 0.5, 0.5, -60, 60, -60, 0.3, 0.3, 7.0], np.float32)
    act = np.array([[1.0, 1.0], [0.0, math.log(3.0)], [2.0, -1.0], [0, 0]], np.float32)
    s = pd.laya_spec(g)
    for res in (lh.laya_decide_scores(h, req, logits, act)["answers"],
                pd.laya_aggregate(s, req, [(logits[0:4], act[0]), (logits[4:7], act[1]), (logits[7:9], act[2]),
                                           (logits[9:], act[3])], 0)["answers"]):
        a, b, c, d = res
        assert a["choice"] == 0 and a["confidence"] == pytest.approx(0.0, abs=1e-6)  # ties: lower index
        assert np.allclose(a["probabilities"], 0.25, atol=1e-7) and a["act_probability"] == pytest.approx(0.5)
        assert b["score"] == pytest.approx(1.0, abs=1e-6) and b["confidence"] == pytest.approx(1.0, abs=1e-6)
        assert b["act_probability"] == pytest.approx(0.25, abs=1e-7)
        assert c["confidence"] == pytest.approx(0.5) and c["noul"] == pytest.approx(0.5)
        assert c["act_probability"] == pytest.approx(1 / (1 + math.exp(-3.0)), rel=1e-6)
        assert d["confidence"] == 1.0 and d["choice"] == 0 and d["probabilities"][0] == 1.0


@pytest.mark.parametrize("req,msg", [
    ({"questions": []}, "questions must contain 1..256 named questions"),
    ({"questions": [q("choice", [1], [([2], None)])] * 257}, "questions must contain 1..256 named questions"),
    ({"questions": [q("choice", [1], [])]}, "choice requires a criteria object"),
    ({"questions": [q("score", [1], [([2], None)])]}, "score requires at least two ordered criteria"),
    ({"questions": [q("noul", [1], [([2], None)] * 3)]}, "noul has exactly two options"),
    ({"questions": [q("choice", [1], [([2], None)] * 17)]}, "requires 1..16 options"),
])
def test_validation_messages(tiny, lh, req, msg):
    h, _ = tiny
    with pytest.raises(lh.LayaError, match=msg):
        lh.laya_decide_encode(h, req, 0)


def test_planted_mistakes_are_caught(tiny, lh, monkeypatch):
    """A wrong head budget or an off-by-one state room in the restatement fails the comparison."""
    h, g = tiny
    req = {"state": list(range(900)), "questions": [q("choice", list(range(200)), [(list(range(30)), None)] * 3)]}
    good = pd.laya_encode(pd.laya_spec(g), req, 0)
    for key, val in (("head_max", 191), ("max", 511)):
        s = pd.laya_spec(g)
        s[key] = val
        assert pd.laya_encode(s, req, 0) != good
    assert lh.laya_decide_encode(h, req, 0)[0].tolist() == good[0]
