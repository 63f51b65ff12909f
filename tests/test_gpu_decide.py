"""Request-level decide on the GPU (lg_decide) against the CPU oracle.

Reference: Backend::decide / decide (src/models/mod.rs:16-22, src/models/openthai/decision.rs:
243-390): every option-order pass is encoded, run through the model and scored over the 256
slot rows at each answer position, then averaged.  The GPU runs all passes as one batch; the
oracle (oracle/pydecide.py) runs them one forward at a time on the CPU.  Bars: option
probabilities within 1e-3 absolute and the same choice unless the oracle's top two are within
that margin (a near tie).
"""
import numpy as np
import pytest

import pydecide as pd

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=[("tiny-q8", 0), ("tiny-f16", 0), ("plumbing-f16", 0), ("tiny-f16", 1),
                                        ("tiny-f16", 2)],
                ids=lambda p: f"{p[0]}-{('exact', 'fast', 'kv16')[p[1]]}")
def setup(request, lh, po):
    preset, prec = request.param
    img = lh.SynthImage(preset, seed=11, n_layers=2 if preset == "plumbing-f16" else 0)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=16384, precision=prec)
    og = po.Gguf(img.array())
    om = po.Model(og, threads=8)
    yield preset, eng, om, og
    eng.close()


def _request(rng, V, perms):
    def toks(lo, hi):
        return rng.integers(0, V - 300, int(rng.integers(lo, hi))).tolist()
    return {
        "state": toks(60, 200),
        "questions": [
            {"type": "choice", "instruction": toks(3, 9),
             "options": [{"name": toks(1, 3), "desc": toks(0, 4)} for _ in range(5)]},
            {"type": "score", "instruction": toks(2, 6), "options": [{"name": [], "desc": toks(1, 3)} for _ in range(4)]},
            {"type": "noul", "instruction": toks(2, 6), "options": [{"name": toks(1, 2)}, {"name": toks(1, 2)}]},
        ],
        "permutations": perms,
    }


@pytest.mark.parametrize("perms", [1, 5])
def test_decide_matches_oracle(setup, lh, perms):
    preset, eng, om, og = setup
    rng = np.random.default_rng(perms)
    req = _request(rng, om.V, perms)
    print(f"{preset}: decide with {perms} passes", flush=True)
    got = eng.decide(req)
    want, _ = pd.decide(om, og, req)
    assert got["usage"]["permutations"] == want["permutations"] == perms
    assert got["usage"]["input_tokens"] == want["input_tokens"]
    assert got["usage"]["truncated_state"] == want["truncated_state"]
    for a, b in zip(got["answers"], want["answers"]):
        assert a["type"] == b["type"]
        err = float(np.abs(a["probabilities"] - b["probabilities"]).max())
        assert err <= 1e-3, f"{a['type']}: probability error {err:.3e}"
        assert abs(a["confidence"] - b["confidence"]) <= 2e-3
        top = np.sort(b["probabilities"])[::-1]
        if len(top) < 2 or top[0] - top[1] > 1e-3:
            assert a["choice"] == b["choice"]
        if "abstain" in b:
            assert abs(a["abstain"] - b["abstain"]) <= 1e-3
        if "score" in b:
            assert abs(a["score"] - b["score"]) <= 1e-2


def test_decide_equals_per_pass_forward_and_host_scores(setup, lh):
    """The batched passes give the same slot logits as one forward per pass (bit-exact), and the
    host aggregation over them gives the same answers."""
    preset, eng, om, og = setup
    rng = np.random.default_rng(7)
    req = _request(rng, om.V, 3)
    got = eng.decide(req)
    s = pd.spec(og)
    logits = []
    for p in range(3):
        ids, pos, _, _, _ = lh.decide_encode(eng.gguf, req, p)
        sq = eng.seq_create()
        logits.append(eng.forward(sq, ids, pos, s["slot"]))
        eng.seq_free(sq)
    again = lh.decide_scores(eng.gguf, req, np.stack(logits))
    for a, b in zip(got["answers"], again["answers"]):
        assert np.array_equal(a["probabilities"], b["probabilities"])
        assert a["choice"] == b["choice"] and a["confidence"] == b["confidence"]


def test_decide_repeat_and_no_leak(setup):
    """Repeat determinism and no state left behind (validation/smoke.py:25-28,
    validation/openthai_edges.py): the same request twice, with another request between."""
    preset, eng, om, og = setup
    req = _request(np.random.default_rng(3), om.V, 2)
    other = _request(np.random.default_rng(4), om.V, 4)
    a = eng.decide(req)
    eng.decide(other)
    b = eng.decide(req)
    for x, y in zip(a["answers"], b["answers"]):
        assert np.array_equal(x["probabilities"], y["probabilities"])


def test_decide_cancel(setup, lh):
    preset, eng, om, og = setup
    req = _request(np.random.default_rng(5), om.V, 2)
    with pytest.raises(lh.LayaError) as ei:
        eng.decide(req, cancel=lambda _: 1)
    assert ei.value.kind == "CANCELED"
    assert eng.decide(req)["usage"]["permutations"] == 2  # the engine stays usable


def test_daemon_process_matches_engine(lh, tmp_path):
    """The JSON-lines daemon as its own process (src/main.rs:139-151) over a model file: answers
    equal an in-process lg_decide of the same request, and a bad line gets an error line."""
    import json
    import os
    import subprocess
    import sys

    path = str(tmp_path / "tiny-q8.gguf")
    lh.synth_file("tiny-q8", 11, path)
    req = {"id": 9, "state": list(range(20, 90)),
           "questions": {"pick": {"type": "choice", "instructions": [1, 2, 3],
                                  "criteria": {f"o{i}": {"name": [30 + i], "desc": [40 + i]} for i in range(4)}},
                         "flag": {"type": "noul", "instructions": [4], "criteria": {"false": [5], "true": [6]}}},
           "permutations": 4}
    script = os.path.join(os.path.dirname(lh.__file__), "daemon.py")
    print("daemon: starting child process", flush=True)
    proc = subprocess.run([sys.executable, script, path, "--kv-tokens", "8192"], input=json.dumps(req) + "\nnot json\n",
                          capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [json.loads(l) for l in proc.stdout.splitlines()]
    assert len(lines) == 2 and "error" in lines[1] and lines[0]["id"] == 9
    sys.path.insert(0, os.path.dirname(script))
    import daemon
    treq, labels = daemon.to_tokens_request(req)
    eng = lh.Engine(lh.Gguf.open(path), kv_tokens=8192)
    want = eng.decide(treq)
    eng.close()
    got = lines[0]["answers"]
    for (qid, kind, names, _), a in zip(labels, want["answers"]):
        if kind == "noul":
            assert got[qid]["noul"] == float(a["probabilities"][1])
        else:
            assert [got[qid]["probabilities"][n] for n in names] == [float(x) for x in a["probabilities"]]
            assert got[qid]["choice"] == names[a["choice"]]


def test_decide_batch_equals_single_requests(setup, lh):
    """lg_decide_batch (the states of /v1/decide/batch, src/server.rs:235-319) gives every request
    the same bits as lg_decide on it alone, and rejects a batch before running any of it."""
    preset, eng, om, og = setup
    reqs = [_request(np.random.default_rng(30 + i), om.V, i % 3 + 1) for i in range(4)]
    got = eng.decide_batch(reqs)
    for r, g in zip(reqs, got):
        want = eng.decide(r)
        assert g["usage"] == want["usage"]
        for a, b in zip(g["answers"], want["answers"]):
            assert np.array_equal(a["probabilities"], b["probabilities"]) and a["choice"] == b["choice"]
    bad = dict(reqs[0], permutations=40)
    with pytest.raises(lh.LayaError, match="permutations must be 1..32"):
        eng.decide_batch([reqs[1], bad])
    with pytest.raises(lh.LayaError, match="At most 256 total questions"):
        eng.decide_batch([reqs[0]] * 86)
    with pytest.raises(lh.LayaError, match="1..256 states"):
        eng.decide_batch([])
