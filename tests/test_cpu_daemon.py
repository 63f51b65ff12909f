"""JSON-lines daemon protocol (src/main.rs:139-151): one JSON line out per non-empty line in, an
{"error": ...} line for a bad request and the loop goes on; answer shapes of
src/models/openthai/decision.rs:297-389.  The engine here computes its slot logits from a seeded
generator and scores them with the library's own host aggregation (lg_decide_scores), so the
whole daemon path except the GPU forward runs."""
import io
import json
import os
import sys

import numpy as np
import pytest

import pydecide as pd

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "laya-goish_amd"))
import daemon  # noqa: E402


class HostScoredEngine:
    def __init__(self, lh, gguf, seed=0):
        self.lh, self.g, self.rng = lh, gguf, np.random.default_rng(seed)

    def decide(self, treq):
        n = pd.passes(treq)
        logits = self.rng.normal(size=(n, len(treq["questions"]), 256)).astype(np.float32)
        return self.lh.decide_scores(self.g, treq, logits)

    def decide_batch(self, treqs):
        return [self.decide(t) for t in treqs]

    def layers(self):
        return 2

    def close(self):
        pass


@pytest.fixture(scope="module")
def gguf(lh):
    return lh.Gguf.from_bytes(lh.SynthImage("tiny-q8", seed=3))


REQ = {"id": "r1", "state": [5, 6, 7, 8],
       "questions": {"topic": {"type": "choice", "instructions": [9, 10],
                               "criteria": {"billing": {"name": [11], "desc": [12, 13]}, "refund": {"name": [14]},
                                            "other": {"name": [22, 23], "desc": None}}},
                     "urgency": {"type": "score", "instructions": [15], "criteria": [[16], [17], [18, 19]]},
                     "human": {"type": "noul", "instructions": [20], "criteria": {"true": [21]}}},
       "permutations": 3}


def run(lines, eng):
    out = io.StringIO()
    daemon.serve(eng, "laya-decoder test", io.StringIO("".join(l + "\n" for l in lines)), out)
    return [json.loads(l) for l in out.getvalue().splitlines()]


def test_daemon_answers_and_recovers(lh, gguf):
    eng = HostScoredEngine(lh, gguf)
    noname = {"questions": {"q": {"type": "choice", "criteria": {"a": [3]}}}}  # a choice option needs name ids
    outs = run([json.dumps(REQ), "", "{not json", json.dumps({"questions": {}}),
                json.dumps({"questions": {"q": {"type": "rank"}}}), json.dumps(noname), json.dumps(REQ)], eng)
    assert len(outs) == 6
    assert all("error" in o for o in outs[1:5])
    assert "questions must contain 1..256 named questions" in outs[2]["error"]
    assert "invalid question type" in outs[3]["error"]
    assert "option name is empty" in outs[4]["error"]
    for o in (outs[0], outs[5]):
        assert o["id"] == "r1" and o["model"] == "laya-decoder test"
        topic, urg, human = o["answers"]["topic"], o["answers"]["urgency"], o["answers"]["human"]
        assert set(topic["probabilities"]) == {"billing", "refund", "other"}
        assert abs(sum(topic["probabilities"].values()) - 1) < 1e-5
        assert topic["choice"] == max(topic["probabilities"], key=topic["probabilities"].get)
        assert 0 <= topic["abstain"] <= 1 and 0 <= topic["confidence"] <= 1
        assert set(urg["probabilities"]) == {"0", "1", "2"} and urg["legend"] == {"0": [16], "1": [17], "2": [18, 19]}
        assert abs(urg["score"] - sum(int(k) * v for k, v in urg["probabilities"].items())) < 1e-5
        assert set(human) == {"type", "noul"} and 0 <= human["noul"] <= 1
        assert o["usage"]["permutations"] == 3 and o["usage"]["output_tokens"] == 0


# token fields that are not lists of int32-range integers: each gets its error line (with the id)
BAD_TOKENS = [
    dict(REQ, id="big", state=[5, 2 ** 40]),
    dict(REQ, id="dict", questions={"q": {"type": "choice", "criteria": {"a": {"name": {"a": 1}}}}}),
    dict(REQ, id="float", questions={"q": {"type": "noul", "instructions": [1.5]}}),
    dict(REQ, id="str", state="hello"),
    dict(REQ, id="bool", questions={"q": {"type": "score", "criteria": [[True], [2]]}}),
]


def test_daemon_rejects_bad_token_fields_and_goes_on(lh, gguf):
    eng = HostScoredEngine(lh, gguf)
    outs = run([json.dumps(r) for r in BAD_TOKENS] + [json.dumps(REQ)], eng)
    assert len(outs) == len(BAD_TOKENS) + 1
    for r, o in zip(BAD_TOKENS, outs):
        assert "error" in o and o["id"] == r["id"], o
        assert "token id" in o["error"] or "list of token ids" in o["error"], o
    assert outs[-1]["id"] == "r1" and "answers" in outs[-1]


def test_daemon_survives_unexpected_engine_errors(lh, gguf):
    """An exception the request checks do not anticipate still becomes that request's error line."""
    class Flaky(HostScoredEngine):
        def decide(self, treq):
            if treq["state"] == [666]:
                raise OverflowError("engine blew up")
            return super().decide(treq)
    outs = run([json.dumps(dict(REQ, id="x", state=[666])), json.dumps(REQ)], Flaky(lh, gguf))
    assert outs[0] == {"error": "OverflowError: engine blew up", "id": "x"}
    assert outs[1]["id"] == "r1" and "answers" in outs[1]


def test_daemon_request_validation():
    bad = [({"questions": {"q": {"type": "choice", "criteria": [1]}}}, "choice requires 1..255 options"),
           ({"questions": {"q": {"type": "score", "criteria": {"a": 1}}}}, "score requires 2..10 levels"),
           ({"questions": {"q": {"type": "noul", "criteria": {"maybe": None}}}}, "noul criteria keys must be false/true"),
           ({"questions": {"q": {"type": "noul"}}, "permutations": 0}, "permutations must be 1..32"),
           ({"questions": {"q": {"type": "noul"}}, "order_invariant": "yes"}, "order_invariant must be boolean"),
           ({"questions": {"q": {"type": "noul"}}, "state": "text"}, "state must be a list of token ids")]
    for req, msg in bad:
        with pytest.raises(daemon.RequestError, match=msg):
            daemon.to_tokens_request(req)


def test_daemon_states_batch(lh, gguf):
    """A /v1/decide/batch body (src/server.rs:235-283): one result per state, limits checked first."""
    eng = HostScoredEngine(lh, gguf, seed=1)
    body = {k: v for k, v in REQ.items() if k != "state"}
    body["states"] = [[5, 6], [7, 8, 9], []]
    outs = run([json.dumps(body), json.dumps(dict(body, states=[])),
                json.dumps(dict(body, states=[[1]] * 86))], eng)
    assert len(outs) == 3 and outs[0]["id"] == "r1" and len(outs[0]["results"]) == 3
    for r in outs[0]["results"]:
        assert set(r["answers"]) == {"topic", "urgency", "human"} and r["usage"]["permutations"] == 3
    assert "states must be an array of 1..256 states" in outs[1]["error"]
    assert "At most 256 total questions per request" in outs[2]["error"]


def _two_models(lh, tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    lh.synth_file("tiny-q8", 3, a)
    lh.synth_file("tiny-f16", 3, b)
    return a, b


def test_registry_preflight_and_selection(lh, tmp_path):
    a, b = _two_models(lh, tmp_path)
    opened = []

    def opener(g):
        opened.append(g)
        return HostScoredEngine(lh, g)
    with pytest.raises(daemon.RegistryError, match="duplicate model name or alias"):
        daemon.Registry([a, a], None, opener)
    with pytest.raises(daemon.RegistryError, match="unknown default model nope"):
        daemon.Registry([a, b], "nope", opener)
    assert not opened  # nothing was loaded for a rejected registry
    reg = daemon.Registry([a, b], "laya-decoder synthetic tiny-f16", opener)
    assert reg.model_names == ["laya-decoder synthetic tiny-q8", "laya-decoder synthetic tiny-f16"]
    assert reg.select({}) == 1 and reg.select({"model": "laya-decoder synthetic tiny-q8"}) == 0
    with pytest.raises(daemon.RequestError, match="unknown model x; see /v1/models"):
        reg.select({"model": "x"})
    with pytest.raises(daemon.RequestError, match="model must be a string"):
        reg.select({"model": 3})


def test_serve_registry_routes_per_model(lh, tmp_path):
    """Per-model queues: each model answers its own requests in order; every line gets one answer."""
    a, b = _two_models(lh, tmp_path)
    reg = daemon.Registry([a, b], None, lambda g: HostScoredEngine(lh, g))
    lines = []
    for i in range(6):
        r = dict(REQ, id=i)
        if i % 2:
            r["model"] = "laya-decoder synthetic tiny-f16"
        lines.append(json.dumps(r))
    lines.append(json.dumps(dict(REQ, id=99, model="missing")))
    out = io.StringIO()
    daemon.serve_registry(reg, io.StringIO("".join(l + "\n" for l in lines)), out)
    outs = [json.loads(l) for l in out.getvalue().splitlines()]
    assert len(outs) == 7
    answered = [o for o in outs if "answers" in o]
    assert sorted(o["id"] for o in answered) == list(range(6))
    for m in ("laya-decoder synthetic tiny-q8", "laya-decoder synthetic tiny-f16"):
        ids = [o["id"] for o in answered if o["model"] == m]
        assert ids == sorted(ids)  # in order within one model
    assert any("unknown model missing" in o.get("error", "") for o in outs)


def test_serve_registry_bad_lines_keep_the_worker_alive(lh, tmp_path):
    """A bad token field in a request for one model answers with an error line; the model's worker
    goes on answering the requests queued after it."""
    a, b = _two_models(lh, tmp_path)
    reg = daemon.Registry([a, b], None, lambda g: HostScoredEngine(lh, g))
    lines = [json.dumps(r) for r in BAD_TOKENS] + [json.dumps(dict(REQ, id=i)) for i in range(3)] + ["[1, 2]"]
    out = io.StringIO()
    daemon.serve_registry(reg, io.StringIO("".join(l + "\n" for l in lines)), out)
    outs = [json.loads(l) for l in out.getvalue().splitlines()]
    assert len(outs) == len(lines)
    errs = {o.get("id"): o for o in outs if "error" in o}
    assert set(r["id"] for r in BAD_TOKENS) <= set(errs)
    assert sorted(o["id"] for o in outs if "answers" in o) == [0, 1, 2]


class LayaScoredEngine:
    """Laya encoder stand-in: seeded option and act logits scored by lg_laya_decide_scores."""

    def __init__(self, lh, gguf, seed=0):
        self.lh, self.g, self.rng = lh, gguf, np.random.default_rng(seed)

    def decide(self, treq):
        ks = [len(q["options"]) for q in treq["questions"]]
        logits = self.rng.normal(size=sum(ks)).astype(np.float32)
        act = self.rng.normal(size=(len(ks), 2)).astype(np.float32)
        return self.lh.laya_decide_scores(self.g, treq, logits, act)

    def decide_batch(self, treqs):
        return [self.decide(t) for t in treqs]

    def layers(self):
        return 4

    def close(self):
        pass


def test_daemon_laya_answer_shape(lh):
    """A Laya encoder's answers carry confidence, probabilities and action.act_probability for every
    kind, noul probabilities keyed false/true (src/models/laya/decision.rs:213-289)."""
    eng = LayaScoredEngine(lh, lh.Gguf.from_bytes(lh.SynthImage("laya-tiny", seed=7)))
    req = {k: v for k, v in REQ.items() if k != "permutations"}
    o, = run([json.dumps(req)], eng)
    topic, urg, human = o["answers"]["topic"], o["answers"]["urgency"], o["answers"]["human"]
    for a in (topic, urg, human):
        assert 0 <= a["action"]["act_probability"] <= 1 and 0 <= a["confidence"] <= 1
        assert abs(sum(a["probabilities"].values()) - 1) < 1e-5 and "abstain" not in a
    assert topic["choice"] == max(topic["probabilities"], key=topic["probabilities"].get)
    assert set(urg["probabilities"]) == {"0", "1", "2"} and urg["legend"] == {"0": [16], "1": [17], "2": [18, 19]}
    assert set(human["probabilities"]) == {"false", "true"} and human["noul"] == human["probabilities"]["true"]
    assert human["confidence"] == pytest.approx(max(human["noul"], 1 - human["noul"]), abs=1e-6)
    # src/models/laya/decision.rs:293-303: usage has no option-order passes or state truncation
    assert set(o["usage"]) == {"input_tokens", "output_tokens", "latency_ms"}


def test_daemon_laya_empty_score_label_stays_empty(lh):
    """A score level without a description keeps its empty label in the legend
    (src/models/laya/decision.rs:247-257); the level index is OpenThai's fallback, not Laya's."""
    eng = LayaScoredEngine(lh, lh.Gguf.from_bytes(lh.SynthImage("laya-tiny", seed=7)))
    req = {"id": 1, "state": [5, 6], "questions": {"u": {"type": "score", "instructions": [15],
                                                          "criteria": [[16], None, [18]]}}}
    o, = run([json.dumps(req)], eng)
    assert o["answers"]["u"]["legend"] == {"0": [16], "1": [], "2": [18]}


def test_registry_laya_answers_name_laya_model_name(lh, tmp_path):
    """Laya answers report laya.model_name (src/models/laya/decision.rs:293); requests still select the
    model by its registry name."""
    path = str(tmp_path / "laya.gguf")
    lh.synth_file("laya-tiny", 7, path)
    reg = daemon.Registry([path], None, lambda g: LayaScoredEngine(lh, g))
    assert reg.model_names == ["laya"] and reg.answer_names == ["laya"]
    assert reg.select({"model": "jev-latest"}) == 0 and reg.select({"model": "english"}) == 0
    out = io.StringIO()
    req = {k: v for k, v in REQ.items() if k != "permutations"}
    daemon.serve(reg.engines[0], reg.answer_names[0], io.StringIO(json.dumps(req) + "\n"), out)
    assert json.loads(out.getvalue())["model"] == "laya"
