"""Laya encoder on the GPU against the CPU oracle (oracle/laya.c, pinned in test_cpu_laya.py).

Reference: Model::forward (src/models/laya/model.rs:303-416) -> option logits at the marker
positions and the act logits.  Bars: 2e-3 absolute in EXACT mode (the reference's own F16
check allows 0.03 on logits, validation/check.py:41-54), 3e-2 in FAST.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL = {0: 2e-3, 1: 3e-2}


@pytest.fixture(scope="module", params=[0, 1], ids=["exact", "fast"])
def tiny(request, lh, po):
    img = lh.SynthImage("laya-tiny", seed=13)
    eng = lh.Engine(lh.Gguf.from_bytes(img), precision=request.param)
    yield request.param, eng, po.Laya(po.Gguf(img.array()), threads=8)
    eng.close()


def test_info(tiny, lh):
    _, eng, _ = tiny
    i = eng.info
    assert i["arch"] == lh.ARCH_LAYA and (i["layers"], i["d_model"], i["head_dim"], i["vocab"], i["context"]) == (4, 128, 64, 1024, 512)


@pytest.mark.parametrize("n,markers,qtype", [(1, [0], 0), (9, [1, 4], 2), (33, [0, 5, 31, 32], 1), (130, [5, 9, 60, 127], 0),
                                             (512, list(range(3, 19)), 2)])
def test_forward_matches_oracle(tiny, n, markers, qtype):
    prec, eng, om = tiny
    ids = np.random.default_rng(n).integers(0, 1000, n)
    print(f"laya-tiny prec {prec}: forward n={n}", flush=True)
    (got_l, got_a), = eng.laya_forward([(ids, markers, qtype)])
    want_l, want_a = om.forward(ids, markers, qtype)
    assert np.abs(got_l - want_l).max() <= TOL[prec] and np.abs(got_a - want_a).max() <= TOL[prec]


def test_batch_equals_single(tiny):
    prec, eng, om = tiny
    rng = np.random.default_rng(3)
    inputs = [(rng.integers(0, 1000, n), sorted(rng.choice(n, min(n, k), replace=False).tolist()), q)
              for n, k, q in ((70, 4, 0), (200, 16, 1), (5, 2, 2), (300, 3, 0))]
    batch = eng.laya_forward(inputs)
    for inp, (bl, ba) in zip(inputs, batch):
        (sl, sa), = eng.laya_forward([inp])
        assert np.array_equal(bl, sl) and np.array_equal(ba, sa)


def test_errors_follow_reference(tiny, lh):
    _, eng, _ = tiny
    for inp, msg in (([1, 2], [2], 0), "invalid inference input shape"), (([1] * 513, [0], 0), "invalid inference input shape"), \
                    (([1, 2], [0], 3), "invalid inference input shape"), (([1, 2], list(range(2)) * 9, 0), "invalid inference input shape"), \
                    (([1, 5000], [0], 0), "token ID out of range"):
        with pytest.raises(lh.LayaError, match=msg):
            eng.laya_forward([inp])
    s = eng.seq_create()
    with pytest.raises(lh.LayaError) as ei:
        eng.forward(s, [1, 2, 3], [0])
    assert ei.value.kind == "UNSUPPORTED"
    eng.seq_free(s)


def test_full_width_matches_oracle(lh, po):
    """The ModernBERT-base shape (22 layers, d 768, 12 x 64 heads, GeGLU 1152, vocab 50368) on a
    full 512-token input with 16 markers."""
    img = lh.SynthImage("laya-english", seed=5)
    eng = lh.Engine(lh.Gguf.from_bytes(img))
    om = po.Laya(po.Gguf(img.array()), threads=8)
    ids = np.random.default_rng(1).integers(0, 50000, 512)
    markers = list(range(20, 36))
    print("laya-english: forward n=512", flush=True)
    (gl, ga), = eng.laya_forward([(ids, markers, 1)])
    eng.close()
    wl, wa = om.forward(ids, markers, 1)
    assert np.abs(gl - wl).max() <= 2e-3 and np.abs(ga - wa).max() <= 2e-3


def test_full_width_large_batch_equals_single(lh, po):
    """The ModernBERT-base shape with 64 inputs of 512 tokens: 32,768 rows put every trunk GEMM on the
    256 x 256 tiles (GeGLU epilogue included), while an input alone takes the small tiles; the batch rows
    equal the single runs bit for bit, and the oracle within 2e-3."""
    img = lh.SynthImage("laya-english", seed=6)
    eng = lh.Engine(lh.Gguf.from_bytes(img))
    rng = np.random.default_rng(31)
    inputs = [(rng.integers(0, 50000, 512), sorted(rng.choice(512, 4, replace=False).tolist()), i % 3) for i in range(64)]
    print("laya-english: 64 x 512 batch", flush=True)
    batch = eng.laya_forward(inputs)
    for i in (0, 41):
        (sl, sa), = eng.laya_forward([inputs[i]])
        assert np.array_equal(batch[i][0], sl) and np.array_equal(batch[i][1], sa), f"input {i}"
    eng.close()
    om = po.Laya(po.Gguf(img.array()), threads=8)
    wl, wa = om.forward(*inputs[41])
    assert np.abs(batch[41][0] - wl).max() <= 2e-3 and np.abs(batch[41][1] - wa).max() <= 2e-3


def _request(rng, nq):
    kinds = ("choice", "score", "noul")
    qs = []
    for i in range(nq):
        kind = kinds[i % 3]
        k = 2 if kind == "noul" else int(rng.integers(2, 17))
        qs.append({"type": kind, "instruction": rng.integers(0, 1000, int(rng.integers(1, 200))).tolist(),
                   "options": [{"name": rng.integers(0, 1000, int(rng.integers(1, 40))).tolist(),
                                "desc": rng.integers(0, 1000, 5).tolist() if j % 2 else None} for j in range(k)]})
    return {"state": rng.integers(0, 1000, int(rng.integers(0, 600))).tolist(), "questions": qs}


@pytest.mark.parametrize("seed", [0, 1])
def test_decide_matches_oracle(tiny, po, seed):
    """lg_decide on a Laya encoder (src/models/laya/decision.rs:168-318) against the token-level
    restatement over the CPU oracle's forward."""
    import pydecide as pd
    prec, eng, om = tiny
    req = _request(np.random.default_rng(seed), 4)
    print(f"laya-tiny prec {prec}: decide seed {seed}", flush=True)
    got = eng.decide(req)
    want, _ = pd.laya_decide(om, om.g, req)
    assert got["usage"]["input_tokens"] == want["input_tokens"]
    for a, b in zip(got["answers"], want["answers"]):
        assert np.abs(a["probabilities"] - b["probabilities"]).max() <= TOL[prec]
        assert abs(a["act_probability"] - b["act_probability"]) <= TOL[prec]
        p = np.sort(b["probabilities"])
        if len(p) < 2 or p[-1] - p[-2] > 4 * TOL[prec]:
            assert a["choice"] == b["choice"]
        if "score" in b:
            assert abs(a["score"] - b["score"]) <= TOL[prec] * len(p) ** 2


def test_decide_is_forward_then_scores(tiny, lh):
    """lg_decide equals lg_laya_decide_encode -> lg_laya_forward -> lg_laya_decide_scores bit for bit."""
    prec, eng, om = tiny
    req = _request(np.random.default_rng(7), 5)
    h = lh.Gguf.from_bytes(lh.SynthImage("laya-tiny", seed=13))
    encs = [lh.laya_decide_encode(h, req, i) for i in range(5)]
    outs = eng.laya_forward([(ids, mk, ("choice", "score", "noul").index(q["type"]))
                             for (ids, mk), q in zip(encs, req["questions"])])
    want = lh.laya_decide_scores(h, req, np.concatenate([o[0] for o in outs]), np.stack([o[1] for o in outs]))
    got = eng.decide(req)
    assert got["usage"]["input_tokens"] == sum(len(e[0]) for e in encs)
    for a, b in zip(got["answers"], want["answers"]):
        assert np.array_equal(a["probabilities"], b["probabilities"])
        assert {k: v for k, v in a.items() if k != "probabilities"} == {k: v for k, v in b.items() if k != "probabilities"}


def test_decide_batch_and_budget_split(tiny, lh):
    """lg_decide_batch (every question of every state in GPU batches) and an engine whose batch
    budget splits the questions give the results of lg_decide on each request alone."""
    prec, eng, om = tiny
    rng = np.random.default_rng(11)
    reqs = [_request(rng, n) for n in (3, 1, 6)]
    single = [eng.decide(r) for r in reqs]
    batch = eng.decide_batch(reqs)
    small = lh.Engine(lh.Gguf.from_bytes(lh.SynthImage("laya-tiny", seed=13)), precision=prec, max_batch_tokens=600)
    try:
        split = [small.decide(r) for r in reqs]
    finally:
        small.close()
    for s, b, t in zip(single, batch, split):
        for x, y, z in zip(s["answers"], b["answers"], t["answers"]):
            assert np.array_equal(x["probabilities"], y["probabilities"])
            assert np.array_equal(x["probabilities"], z["probabilities"])
            assert x["act_probability"] == y["act_probability"] == z["act_probability"]


def test_large_batch_equals_single(tiny):
    """64 inputs of 512 tokens (the GEMMs then take 128 x 128 tiles, the attention 12,288
    workgroups) give the results of each input alone bit for bit, and match the oracle."""
    prec, eng, om = tiny
    rng = np.random.default_rng(21)
    inputs = [(rng.integers(0, 1000, 512), sorted(rng.choice(512, 4, replace=False).tolist()), i % 3) for i in range(64)]
    print(f"laya-tiny prec {prec}: 64 x 512 batch", flush=True)
    batch = eng.laya_forward(inputs)
    for i in (0, 17, 63):
        (sl, sa), = eng.laya_forward([inputs[i]])
        assert np.array_equal(batch[i][0], sl) and np.array_equal(batch[i][1], sa)
        wl, wa = om.forward(*inputs[i])
        assert np.abs(sl - wl).max() <= TOL[prec] and np.abs(sa - wa).max() <= TOL[prec]


@pytest.mark.parametrize("layers", [1, 4])
def test_exact_attention_precision(lh, po, layers):
    """The exact mode's split-operand MFMAs (three f16 products per pair, ~22 significant bits) in
    the Laya attention and GEMMs: option and act logits within 5e-6 of the largest |logit| at one
    layer (layer 0 is a global-attention layer) and at full depth (measured 1.7e-7 to 2.8e-7).  One
    f16-only operand anywhere costs ~1e-3, two hundred times this bar."""
    img = lh.SynthImage("laya-tiny", seed=17, n_layers=layers)
    eng = lh.Engine(lh.Gguf.from_bytes(img))
    om = po.Laya(po.Gguf(img.array()), threads=8)
    worst = 0.0
    for n, markers, qtype in ((200, [3, 50, 120, 199], 1), (512, list(range(40, 56)), 0)):
        ids = np.random.default_rng(n + layers).integers(0, 1000, n)
        (gl, ga), = eng.laya_forward([(ids, markers, qtype)])
        wl, wa = om.forward(ids, markers, qtype)
        scale = max(np.abs(wl).max(), np.abs(wa).max())
        err = max(np.abs(gl - wl).max(), np.abs(ga - wa).max()) / scale
        print(f"laya-tiny L{layers} n={n}: relative logit error {err:.2e}", flush=True)
        worst = max(worst, err)
    eng.close()
    assert worst <= 5e-6


def test_activations_beyond_f16_range_are_reported(lh, po):
    """The exact mode splits activations into f16 hi/lo planes, which hold |x| <= 65504.  A q
    projection row of 60000s in layer 0 drives q past that range for every token: the forward then
    fails with the reference's "non-finite model output" (src/models/laya/model.rs:412-414) instead
    of returning values, while the f32 reference would still produce finite logits."""
    img = lh.SynthImage("laya-tiny", seed=13)
    arr = img.array().copy()
    og = po.Gguf(arr)
    kind, dims, _ = og.tensor("qkv.0.weight")
    assert kind == 1  # F16
    off, d = og.offset("qkv.0.weight"), dims[0]
    arr[off:off + 2 * d] = np.frombuffer(np.full(d, 0x7B53, np.uint16).tobytes(), np.uint8)  # 60000.0
    eng = lh.Engine(lh.Gguf.from_bytes(arr))
    ids = np.random.default_rng(5).integers(0, 1000, 64)
    with pytest.raises(lh.LayaError, match="non-finite model output"):
        eng.laya_forward([(ids, [3, 9], 0)])
    want_l, want_a = po.Laya(po.Gguf(arr), threads=8).forward(ids, [3, 9], 0)
    assert np.isfinite(want_l).all() and np.isfinite(want_a).all()
    eng.close()


def test_kv16_mode_is_the_exact_mode(lh):
    """The Laya encoder keeps no KV cache, so an engine created in the kv16 mode computes exactly as the
    exact mode does: the same option and act logits, bit for bit."""
    img = lh.SynthImage("laya-tiny", seed=13)
    ids = np.random.default_rng(6).integers(0, 1000, 130)
    out = []
    for prec in (lh.PREC_EXACT, lh.PREC_KV16):
        eng = lh.Engine(lh.Gguf.from_bytes(img), precision=prec)
        out.append(eng.laya_forward([(ids, [5, 9, 60, 127], 0)])[0])
        eng.close()
    for a, b in zip(out[0], out[1]):
        assert np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))
