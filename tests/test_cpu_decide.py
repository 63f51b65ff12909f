"""Request-level decide on the host: pass count, option orders, token layout and aggregation.

Reference: src/models/openthai/decision.rs (questions :20-107, orders :125-139, permutations
:140-162, encode :169-233, scoring :268-279, answers :297-336).  The library's host code
(lg_decide_encode / lg_decide_scores, the same code lg_decide runs around the GPU batch) is
checked against the oracle's independent restatement (oracle/pydecide.py) and against values
worked out by hand from the reference's formulas.
"""
import numpy as np
import pytest

import pydecide as pd


@pytest.fixture(scope="module")
def model(lh, po):
    img = lh.SynthImage("tiny-q8", seed=3)
    return lh.Gguf.from_bytes(img), po.Gguf(img.array()), img


def _req(rng, V, nq=3, state_len=40, perms=None, oi=None, descs=True):
    qs = []
    for i in range(nq):
        kind = ["choice", "score", "noul"][i % 3]
        k = {"choice": int(rng.integers(1, 7)), "score": int(rng.integers(2, 11)), "noul": 2}[kind]
        opts = []
        for j in range(k):
            name = rng.integers(0, V - 300, int(rng.integers(1 if kind == "choice" else 0, 4))).tolist()
            desc = rng.integers(0, V - 300, int(rng.integers(0, 3))).tolist() if descs else []
            opts.append({"name": name, "desc": desc})
        qs.append({"type": kind, "instruction": rng.integers(0, V - 300, int(rng.integers(0, 6))).tolist(),
                   "options": opts})
    return {"state": rng.integers(0, V - 300, state_len).tolist(), "questions": qs, "permutations": perms,
            "order_invariant": oi}


def test_orders_known_values():
    # offsets = j*k/n rounded half to even, j < n = min(n, k): worked by hand from decision.rs:125-139
    assert pd.orders(4, 2) == [[0, 1, 2, 3], [2, 3, 0, 1]]
    assert [o[0] for o in pd.orders(5, 2)] == [0, 2]      # 5/2 = 2.5 -> 2 (even)
    assert [o[0] for o in pd.orders(3, 2)] == [0, 2]      # 3/2 = 1.5 -> 2 (even)
    assert [o[0] for o in pd.orders(7, 3)] == [0, 2, 5]   # 7/3 -> 2, 14/3 -> 5
    assert [o[0] for o in pd.orders(2, 8)] == [0, 1]      # n clamps to k
    assert [o[0] for o in pd.orders(6, 4)] == [0, 2, 3, 4]  # 1.5 -> 2, 3, 4.5 -> 4
    assert pd.orders(1, 5) == [[0]]


def test_pass_count_rule():
    def req(ks, perms=None, oi=None):
        return {"questions": [{"type": "choice", "options": [{}] * k} for k in ks] + [{"type": "noul",
                "options": [{}, {}]}], "permutations": perms, "order_invariant": oi}
    assert pd.passes(req([4])) == 1
    assert pd.passes(req([11])) == 8
    assert pd.passes(req([4], oi=True)) == 4
    assert pd.passes(req([20], oi=False)) == 1
    assert pd.passes(req([3, 9], perms=5)) == 5
    assert pd.passes(req([3], perms=32)) == 3
    assert pd.passes({"questions": [{"type": "score", "options": [{}] * 5}], "permutations": 4}) == 1


@pytest.mark.parametrize("seed", range(12))
def test_encode_matches_oracle(model, lh, seed):
    g, og, _ = model
    rng = np.random.default_rng(seed)
    V = int(og.num("laya.decoder.vocab_size"))
    req = _req(rng, V, nq=int(rng.integers(1, 6)), state_len=int(rng.integers(0, 700)),
               perms=[None, 1, 3, 8, 32][seed % 5], oi=[None, True, False][seed % 3], descs=seed % 2 == 0)
    s = pd.spec(og)
    n = pd.passes(req)
    for p in range(n):
        ids, pos, order, trunc, npass = lh.decide_encode(g, req, p)
        wids, wpos, word, wtrunc = pd.encode(s, req, n, p)
        assert npass == n
        assert np.array_equal(ids, wids), f"pass {p}"
        assert np.array_equal(pos, wpos)
        assert order == word
        assert trunc == wtrunc
        assert all(ids[q] == s["answer"] for q in pos)


def test_state_truncation_keeps_first_token_and_tail(model, lh):
    g, og, _ = model
    s = pd.spec(og)
    ctx = s["max_tokens"]
    state = np.arange(5, 5 + 3 * ctx).astype(np.int32) % 200
    req = {"state": state.tolist(), "questions": [{"type": "noul", "instruction": [1, 2],
                                                  "options": [{"name": [3]}, {"name": [4]}]}]}
    ids, pos, _, trunc, _ = lh.decide_encode(g, req, 0)
    block = 2 + 2 + 1 + 2 * 3 + 2  # question, kind, instruction, newline, 2 x (slot, name, newline), answer, newline
    assert trunc and len(ids) == min(s["max_state"], ctx - block) + block
    assert ids[0] == s["state"]
    budget = len(ids) - block
    full = [s["state"]] + state.tolist() + [s["newline"]]
    assert ids[1:budget].tolist() == full[len(full) - (budget - 1):]
    assert pos[0] == len(ids) - 2


def test_encode_errors_follow_reference(model, lh):
    g, _, _ = model
    ok = {"type": "noul", "options": [{"name": [1]}, {"name": [2]}]}
    cases = [
        ({"questions": []}, "questions must contain 1..256 named questions"),
        ({"questions": [ok] * 257}, "questions must contain 1..256 named questions"),
        ({"questions": [{"type": "choice", "options": [{"name": [1]}] * 256}]}, "choice requires 1..255 options"),
        ({"questions": [{"type": "choice", "options": []}]}, "choice requires 1..255 options"),
        ({"questions": [{"type": "choice", "options": [{"name": []}]}]}, "option name is empty"),
        ({"questions": [{"type": "score", "options": [{}]}]}, "score requires 2..10 levels"),
        ({"questions": [{"type": "score", "options": [{}] * 11}]}, "score requires 2..10 levels"),
        ({"questions": [{"type": "noul", "options": [{"name": [1]}] * 3}]}, "noul has exactly two options"),
        ({"questions": [ok], "permutations": 33}, "permutations must be 1..32"),
        ({"questions": [ok], "state": [1 << 20]}, "outside the vocabulary"),
        ({"questions": [{"type": "choice", "options": [{"name": [1], "desc": [-3]}]}]}, "outside the vocabulary"),
        ({"questions": [{"type": "noul", "instruction": [7] * 600, "options": [{"name": [1]}, {"name": [2]}]}]},
         "question tokens exceed the context budget"),
    ]
    for req, msg in cases:
        with pytest.raises(lh.LayaError) as ei:
            lh.decide_encode(g, req, 0)
        assert msg in str(ei.value), (req, str(ei.value))
    with pytest.raises(lh.LayaError, match="invalid question type"):
        lh.decide_encode(g, {"questions": [{"type": "rank", "options": []}]}, 0)


@pytest.mark.parametrize("seed", range(8))
def test_scores_match_oracle_bit_exact(model, lh, seed):
    g, og, _ = model
    rng = np.random.default_rng(100 + seed)
    V = int(og.num("laya.decoder.vocab_size"))
    req = _req(rng, V, nq=int(rng.integers(1, 7)), state_len=30, perms=[None, 2, 5, 8][seed % 4])
    s = pd.spec(og)
    n = pd.passes(req)
    logits = (rng.normal(size=(n, len(req["questions"]), 256)) * 3).astype(np.float32)
    got = lh.decide_scores(g, req, logits)
    encs = [pd.encode(s, req, n, p) for p in range(n)]
    want = pd.aggregate(s, req, n, encs, logits)
    assert got["usage"]["permutations"] == n and got["usage"]["input_tokens"] == want["input_tokens"]
    for a, b in zip(got["answers"], want["answers"]):
        assert np.array_equal(a["probabilities"], b["probabilities"])
        assert a["confidence"] == b["confidence"] and a["choice"] == b["choice"]
        for key in ("abstain", "score", "noul"):
            assert (key in a) == (key in b) and a.get(key) == b.get(key)


def test_scores_closed_forms(model, lh):
    g, og, _ = model
    q = {"type": "choice", "options": [{"name": [1]}, {"name": [2]}, {"name": [3]}, {"name": [4]}]}
    # equal option logits, abstain logit ln(4): softmax over 5 gives 1/8 each option, 1/2 abstain
    sl = np.zeros((4, 1, 256), np.float32)
    sl[:, 0, 255] = np.log(4.0)
    out = lh.decide_scores(g, {"questions": [q], "permutations": 4}, sl)["answers"][0]
    assert np.allclose(out["probabilities"], 0.25, atol=1e-6)
    assert abs(out["abstain"] - 0.5) < 1e-6 and abs(out["confidence"]) < 1e-6 and out["choice"] == 0
    # one dominant slot in every pass: the option shown at slot 0 of each pass gets the mass
    sl = np.full((4, 1, 256), -50.0, np.float32)
    sl[:, 0, 0] = 50.0
    out = lh.decide_scores(g, {"questions": [q], "permutations": 4}, sl)["answers"][0]
    assert np.allclose(out["probabilities"], 0.25, atol=1e-6)  # rotations put each option at slot 0 once
    sl = np.full((1, 1, 256), -50.0, np.float32)
    sl[0, 0, 2] = 50.0
    out = lh.decide_scores(g, {"questions": [q]}, sl)["answers"][0]
    assert out["choice"] == 2 and out["confidence"] > 0.9999 and out["abstain"] < 1e-20
    # score: expected level sum_j j p_j
    sq = {"type": "score", "options": [{}, {}, {}]}
    sl = np.zeros((1, 1, 256), np.float32)
    sl[0, 0, :3] = np.log([1.0, 2.0, 5.0])
    out = lh.decide_scores(g, {"questions": [sq]}, sl)["answers"][0]
    assert abs(out["score"] - (0 * 0.125 + 1 * 0.25 + 2 * 0.625)) < 1e-6
