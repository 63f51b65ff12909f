"""Pinning the oracle's decoder forward pass on the CPU.

1. Against the float64 brute force of tests/np_model.py on tiny synthetic models (all three
   weight families: F16, Q8_0, Q4_K/Q6_K; GQA and MHA; with and without QKV bias), and
   against the committed golden logits in tests/golden/.
2. Each planted mistake in the brute force (gate/up swapped, wrong kv-head map, missing
   1/sqrt(hd), wrong RoPE pairing, missing final norm, missing eps, no causal mask) moves the
   logits far outside the tolerance, so the comparison would catch it.
3. Invariants the reference's behaviour fixes: causality, KV-cache continuation == one shot,
   fork == unshared, thread-count and repeat bit-exactness, GQA == MHA with duplicated heads.
"""
import os

import numpy as np
import pytest

import gguf_writer as gw
from np_model import MISTAKES, F64Model

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "forward_tiny.npz")
TOL = 2e-5  # relative to the largest |logit|; the f32 oracle sits at ~1e-6 of the f64 brute force


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(1e-30, np.abs(b).max()))


@pytest.fixture(scope="module", params=["tiny-f16", "tiny-q8", "tiny-q4k"])
def model(request, lh, po):
    img = lh.SynthImage(request.param, seed=5)
    g = po.Gguf(img.array().copy())
    return request.param, g, po.Model(g, threads=4), F64Model(g)


def _ids(n, V, seed):
    return np.random.default_rng(seed).integers(0, V, n).astype(np.int32)


def test_oracle_vs_f64_bruteforce(model):
    name, g, om, ref = model
    ids = _ids(40, om.V, 1)
    pos = [39, 20, 0, 7]
    got = om.forward(ids, pos)
    want = ref.logits(ids, pos)
    err = _rel(got, want)
    print(f"{name}: oracle vs f64 rel {err:.2e}")
    assert err < TOL


@pytest.mark.parametrize("mistake", MISTAKES)
def test_planted_mistakes_are_caught(model, mistake):
    name, g, om, _ = model
    if mistake == "kv_head_mod" and om.hq == om.hkv:
        pytest.skip("with one query head per kv head every kv-head map is the identity")
    ids = _ids(40, om.V, 1)
    pos = [39, 20, 7]
    err = _rel(om.forward(ids, pos), F64Model(g, mistake).logits(ids, pos))
    assert err > 5 * TOL, f"{mistake} changes logits by only {err:.2e}"


def test_golden_logits(lh, po):
    """Committed float64 logits (tests/golden/make_golden.py) for the tiny models."""
    gold = np.load(GOLDEN, allow_pickle=False)
    for preset in ("tiny-f16", "tiny-q8", "tiny-q4k"):
        img = lh.SynthImage(preset, seed=int(gold["seed"]))
        digest = np.frombuffer(__import__("hashlib").sha256(img.bytes()).digest(), np.uint8)
        assert np.array_equal(digest, gold[f"{preset}/sha256"]), \
            f"the {preset} generator changed: regenerate tests/golden with make_golden.py"
        om = po.Model(po.Gguf(img.array().copy()), threads=4)
        got = om.forward(gold[f"{preset}/ids"], gold[f"{preset}/pos"])
        assert _rel(got, gold[f"{preset}/logits"]) < TOL


def test_causality_bit_exact(model):
    name, g, om, _ = model
    ids = _ids(50, om.V, 2)
    pos = list(range(0, 30))
    a = om.forward(ids, pos)
    ids2 = ids.copy()
    ids2[30:] = _ids(20, om.V, 3)
    assert np.array_equal(a, om.forward(ids2, pos))
    ids3 = ids.copy()
    ids3[29] = (ids3[29] + 1) % om.V
    assert not np.array_equal(a[29], om.forward(ids3, pos)[29])


def test_cache_continuation_and_fork(model):
    name, g, om, _ = model
    ids = _ids(70, om.V, 4)
    c1 = om.cache(128)
    one = om.head(om.prefill(c1, ids, [69, 50]))
    c2 = om.cache(128)
    om.prefill(c2, ids[:33], [])
    om.prefill(c2, ids[33:50], [])
    two = om.head(om.prefill(c2, ids[50:], [19, 0]))
    assert np.array_equal(one, two)
    # fork at 40: shared prefix + own suffix == the whole sequence from scratch
    c3 = c1.fork(40)
    suffix = _ids(10, om.V, 5)
    got = om.head(om.prefill(c3, suffix, [9]))
    c4 = om.cache(128)
    want = om.head(om.prefill(c4, np.concatenate([ids[:40], suffix]), [49]))
    assert np.array_equal(got, want)


def test_threads_and_repeat_bit_exact(model):
    name, g, om, _ = model
    ids = _ids(37, om.V, 6)
    outs = []
    for t in (1, 3, 8, 1):
        om.set_threads(t)
        outs.append(om.forward(ids, [36, 5]))
    om.set_threads(4)
    for o in outs[1:]:
        assert np.array_equal(outs[0], o)


def _meta(g, hkv):
    keys = ["block_count", "embedding_length", "head_count", "head_count_kv", "key_length",
            "feed_forward_length", "vocab_size", "context_length"]
    meta = [("general.architecture", gw.STR, "ggmlc"), ("laya.model_name", gw.STR, "laya-decoder")]
    for k in keys:
        v = hkv if k == "head_count_kv" else int(g.num(f"laya.decoder.{k}"))
        meta.append((f"laya.decoder.{k}", gw.U32, v))
    for k in ("layer_norm_rms_epsilon", "rope_freq_base"):
        meta.append((f"laya.decoder.{k}", gw.F32, float(g.num(f"laya.decoder.{k}"))))
    return meta


def test_gqa_equals_mha_with_duplicated_heads(lh, po):
    """tiny-f16 has 4 query heads over 2 kv heads.  Rewriting it with 4 kv heads, kv head h a
    copy of kv head h // 2, must give bit-identical logits: head h reads kv head h // (hq/hkv)."""
    img = lh.SynthImage("tiny-f16", seed=5)
    g = po.Gguf(img.array().copy())
    L, hq, hkv, hd = (int(g.num(f"laya.decoder.{k}")) for k in ("block_count", "head_count", "head_count_kv",
                                                                 "key_length"))
    assert hkv * 2 == hq
    names = ["tok_emb.weight", "final_norm.weight", "output.weight", "cos_full", "sin_full"]
    tensors = []
    for n in names:
        kind, dims, raw = g.tensor(n)
        tensors.append((n, dims, kind, raw))
    for l in range(L):
        for n in (f"attn_norm.{l}.weight", f"ffn_norm.{l}.weight", f"wo.{l}.weight", f"mlp_wi.{l}.weight",
                  f"mlp_wo.{l}.weight"):
            kind, dims, raw = g.tensor(n)
            tensors.append((n, dims, kind, raw))
        kind, dims, raw = g.tensor(f"qkv.{l}.weight")
        assert kind == 1  # F16 rows can be copied as bytes
        d = dims[0]
        w = np.frombuffer(raw, np.uint16).reshape(-1, d)
        q, k, v = w[:hq * hd], w[hq * hd:(hq + hkv) * hd], w[(hq + hkv) * hd:]
        dup = lambda a: np.concatenate([a[(h // 2) * hd:(h // 2 + 1) * hd] for h in range(hq)])
        w2 = np.concatenate([q, dup(k), dup(v)])
        tensors.append((f"qkv.{l}.weight", [d, w2.shape[0]], 1, w2.tobytes()))
        try:
            kind, dims, raw = g.tensor(f"qkv.{l}.bias")
            b = np.frombuffer(raw, np.float32)
            b2 = np.concatenate([b[:hq * hd], dup(b[hq * hd:(hq + hkv) * hd].reshape(-1, 1)).reshape(-1),
                                 dup(b[(hq + hkv) * hd:].reshape(-1, 1)).reshape(-1)])
            tensors.append((f"qkv.{l}.bias", [b2.size], 0, b2.astype(np.float32).tobytes()))
        except KeyError:
            pass
    mha = po.Gguf(gw.build(_meta(g, hq), tensors))
    ids = _ids(45, int(g.num("laya.decoder.vocab_size")), 7)
    a = po.Model(g, threads=2).forward(ids, [44, 3, 20])
    b = po.Model(mha, threads=2).forward(ids, [44, 3, 20])
    assert np.array_equal(a, b)


def test_streamed_layers_bit_exact(model):
    """The layer-streamed oracle (each layer's weights decoded only while it runs, over 1 or 7 decode
    workers) gives the eager oracle's bits: one-shot forwards, cache continuation and a fork."""
    name, g, om, _ = model
    ids = _ids(70, om.V, 9)
    pos = [69, 31, 0]
    want = om.forward(ids, pos)
    for t in (1, 7):
        sm = type(om)(g, threads=t, streamed=True)
        got = sm.forward(ids, pos)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{name}: streamed ({t}) != eager"
        c = sm.cache(100)
        sm.prefill(c, ids[:40], [])
        k = c.fork(40)
        h = sm.head(sm.prefill(k, ids[40:], [29, 0]))
        ce = om.cache(100)
        om.prefill(ce, ids[:40], [])
        he = om.head(om.prefill(ce.fork(40), ids[40:], [29, 0]))
        assert np.array_equal(h.view(np.uint32), he.view(np.uint32)), f"{name}: streamed fork != eager"
