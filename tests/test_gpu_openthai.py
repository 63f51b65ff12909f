"""OpenThai-SystemOne on the GPU (gated DeltaNet + gated full attention + slot head) against the
CPU oracle (oracle/openthai.c, itself pinned in test_cpu_openthai.py).

Reference: Model::forward (src/models/openthai/model.rs:192-241) -> slot logits; decide
(src/models/openthai/decision.rs:243-390).  Bars: slot logits within 2e-3 absolute
(validation/openthai_check.py:31) in the EXACT mode, option probabilities within 1e-3.
"""
import numpy as np
import pytest

import pydecide as pd

pytestmark = pytest.mark.gpu

TOL = {0: 2e-3, 1: 5e-2}  # EXACT, FAST


@pytest.fixture(scope="module", params=[0, 1], ids=["exact", "fast"])
def tiny(request, lh, po):
    img = lh.SynthImage("openthai-tiny", seed=21)
    eng = lh.Engine(lh.Gguf.from_bytes(img), precision=request.param)
    og = po.Gguf(img.array())
    yield request.param, eng, po.OpenThai(og, threads=8), og
    eng.close()


def test_info(tiny, lh):
    _, eng, _, _ = tiny
    i = eng.info
    assert i["arch"] == lh.ARCH_OPENTHAI and i["linear_heads"] == 2 and i["full_layers"] == 1
    assert (i["layers"], i["d_model"], i["heads"], i["kv_heads"], i["head_dim"], i["vocab"]) == (4, 256, 8, 2, 256, 1024)


@pytest.mark.parametrize("n", [1, 3, 16, 17, 33, 100, 300])
def test_forward_matches_oracle(tiny, n):
    prec, eng, om, _ = tiny
    ids = np.random.default_rng(n).integers(0, 960, n)
    pos = sorted({0, n // 3, n - 1})
    print(f"openthai-tiny prec {prec}: forward n={n}", flush=True)
    s = eng.seq_create()
    got = eng.forward(s, ids, pos)
    eng.seq_free(s)
    want = om.forward(ids, pos)
    err = float(np.abs(got - want).max())
    assert got.shape == (len(pos), 256) and err <= TOL[prec], f"slot logits differ by {err:.3e}"


def test_batch_equals_single_and_repeats(tiny):
    """Ragged batch of fresh sequences: each row equals its own single-sequence forward, bit for
    bit, and a repeat gives the same bits (validation/smoke.py:25-28)."""
    prec, eng, om, _ = tiny
    rng = np.random.default_rng(5)
    reqs = [(rng.integers(0, 960, n), [n - 1, n // 2]) for n in (40, 7, 129, 64, 1)]
    seqs = [eng.seq_create() for _ in reqs]
    b = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)])
    slots = list(range(256))
    logits, _, _ = b.run(slots)
    b.free()
    row = 0
    for s, (ids, pos) in zip(seqs, reqs):
        eng.seq_free(s)
        s2 = eng.seq_create()
        single = eng.forward(s2, ids, pos)
        eng.seq_free(s2)
        assert np.array_equal(logits[row:row + len(pos)], single)
        row += len(pos)


def test_slot_subset_and_errors(tiny, lh):
    prec, eng, om, _ = tiny
    ids = np.arange(10, 60)
    s = eng.seq_create()
    part = eng.forward(s, ids, [49], [3, 255, 0])
    full_s = eng.seq_create()
    full = eng.forward(full_s, ids, [49])
    assert np.array_equal(part[0], full[0, [3, 255, 0]])
    # a second forward on a used sequence: the recurrent state is local to one forward
    with pytest.raises(lh.LayaError) as ei:
        eng.forward(s, ids, [0])
    assert ei.value.kind == "INVALID" and "empty sequence" in str(ei.value)
    with pytest.raises(lh.LayaError) as ei:
        eng.decode(full_s, 5, 2)
    assert ei.value.kind == "UNSUPPORTED"
    with pytest.raises(lh.LayaError) as ei:
        eng.seq_fork(full_s, 10)
    assert ei.value.kind == "UNSUPPORTED"
    s3 = eng.seq_create()
    with pytest.raises(lh.LayaError) as ei:
        eng.forward(s3, ids, [0], [256])
    assert ei.value.kind == "INVALID" and "256 slots" in str(ei.value)
    with pytest.raises(lh.LayaError):
        eng.forward(s3, [1, 2, 1024], [0])
    for q in (s, full_s, s3):
        eng.seq_free(q)


def _request(rng, perms):
    def toks(lo, hi):
        return rng.integers(0, 600, int(rng.integers(lo, hi))).tolist()
    return {"state": toks(80, 300),
            "questions": [
                {"type": "choice", "instruction": toks(3, 8), "options": [{"name": toks(1, 3), "desc": toks(0, 4)} for _ in range(6)]},
                {"type": "score", "instruction": toks(2, 5), "options": [{"name": [], "desc": toks(1, 3)} for _ in range(5)]},
                {"type": "noul", "instruction": toks(2, 5), "options": [{"name": toks(1, 2)}, {"name": toks(1, 2)}]}],
            "permutations": perms}


@pytest.mark.parametrize("perms", [1, 4])
def test_decide_matches_oracle(tiny, perms):
    prec, eng, om, og = tiny
    req = _request(np.random.default_rng(perms + 10), perms)
    print(f"openthai-tiny prec {prec}: decide, {perms} passes", flush=True)
    got = eng.decide(req)
    want, _ = pd.decide(om, og, req)
    assert got["usage"]["permutations"] == want["permutations"] == perms
    assert got["usage"]["input_tokens"] == want["input_tokens"]
    bar = 1e-3 if prec == 0 else 2e-2
    for a, b in zip(got["answers"], want["answers"]):
        err = float(np.abs(a["probabilities"] - b["probabilities"]).max())
        assert err <= bar, f"{a['type']}: probability error {err:.3e}"
        top = np.sort(b["probabilities"])[::-1]
        if top[0] - top[1] > bar:
            assert a["choice"] == b["choice"]


@pytest.mark.parametrize("n", [160, 1437])
def test_full_width_layers_match_oracle(lh, po, n):
    """The first four layers of the 0.8B shape (d 1024, 16 linear heads, 8/2 x 256 attention,
    vocab 248339): three DeltaNet layers and one full-attention layer; 160 tokens, and the
    reference's 1437-token request length (45 scan chunks of 32 tokens, the last one partial)."""
    img = lh.SynthImage("openthai-0.8b", seed=3, n_layers=4)
    eng = lh.Engine(lh.Gguf.from_bytes(img))
    om = po.OpenThai(po.Gguf(img.array()), threads=8)
    ids = np.random.default_rng(n).integers(0, 247000, n)
    pos = [0, 77, n // 2, n - 1]
    print(f"openthai-0.8b (4 layers): forward n={n}", flush=True)
    s = eng.seq_create()
    got = eng.forward(s, ids, pos)
    eng.close()
    want = om.forward(ids, pos)
    err = float(np.abs(got - want).max())
    print(f"openthai-0.8b (4 layers) n={n}: slot logits max abs error {err:.3e}", flush=True)
    assert err <= 2e-3, f"slot logits differ by {err:.3e}"


def test_decide_batch_equals_single_requests(tiny):
    prec, eng, om, og = tiny
    reqs = [_request(np.random.default_rng(50 + i), [1, 2, 4][i % 3]) for i in range(5)]
    got = eng.decide_batch(reqs)
    for r, g in zip(reqs, got):
        want = eng.decide(r)
        assert g["usage"] == want["usage"]
        for a, b in zip(g["answers"], want["answers"]):
            assert np.array_equal(a["probabilities"], b["probabilities"]) and a["choice"] == b["choice"]


def test_daemon_serves_two_models(lh, tmp_path):
    """The daemon with an OpenThai model and a laya-decoder model loaded side by side, one engine
    (one stream) each: requests routed by "model", answers equal in-process lg_decide, and a
    "states" body answered per state."""
    import json
    import os
    import subprocess
    import sys

    ot, dec = str(tmp_path / "ot.gguf"), str(tmp_path / "dec.gguf")
    lh.synth_file("openthai-tiny", 21, ot)
    lh.synth_file("tiny-q8", 11, dec)
    q = {"pick": {"type": "choice", "instructions": [1, 2, 3],
                  "criteria": {f"o{i}": {"name": [30 + i], "desc": [40 + i]} for i in range(4)}},
         "flag": {"type": "noul", "instructions": [4], "criteria": {"false": [5], "true": [6]}}}
    lines = [{"id": 1, "state": list(range(20, 90)), "questions": q, "permutations": 2},
             {"id": 2, "model": "laya-decoder synthetic tiny-q8", "state": list(range(20, 60)), "questions": q},
             {"id": 3, "states": [list(range(5, 40)), list(range(50, 70))], "questions": q}]
    script = os.path.join(os.path.dirname(lh.__file__), "daemon.py")
    print("daemon: two models", flush=True)
    proc = subprocess.run([sys.executable, script, ot, "--model", dec, "--kv-tokens", "8192"],
                          input="".join(json.dumps(l) + "\n" for l in lines), capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stderr[-2000:]
    outs = {o["id"]: o for o in map(json.loads, proc.stdout.splitlines())}
    assert set(outs) == {1, 2, 3} and outs[2]["model"] == "laya-decoder synthetic tiny-q8"
    sys.path.insert(0, os.path.dirname(script))
    import daemon
    for path, ids in ((ot, [1, 3]), (dec, [2])):
        eng = lh.Engine(lh.Gguf.open(path), kv_tokens=8192)
        for i in ids:
            body = lines[i - 1]
            if "states" in body:
                treqs, labels = daemon.states_requests(body)
                wants = eng.decide_batch(treqs)
                gots = outs[i]["results"]
            else:
                treq, labels = daemon.to_tokens_request(body)
                wants, gots = [eng.decide(treq)], [outs[i]]
            for got, want in zip(gots, wants):
                for (qid, kind, names, _), a in zip(labels, want["answers"]):
                    if kind == "noul":
                        assert got["answers"][qid]["noul"] == float(a["probabilities"][1])
                    else:
                        assert [got["answers"][qid]["probabilities"][n] for n in names] == [float(x) for x in a["probabilities"]]
        eng.close()


def test_kv16_mode_is_the_exact_mode(lh):
    """The OpenThai family keeps no KV cache, so an engine created in the kv16 mode computes exactly as
    the exact mode does: the same slot logits, bit for bit."""
    img = lh.SynthImage("openthai-tiny", seed=21)
    ids = np.random.default_rng(5).integers(0, 960, 90)
    out = []
    for prec in (lh.PREC_EXACT, lh.PREC_KV16):
        eng = lh.Engine(lh.Gguf.from_bytes(img), precision=prec)
        out.append(eng.forward(eng.seq_create(), ids, [0, 44, 89]))
        eng.close()
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
