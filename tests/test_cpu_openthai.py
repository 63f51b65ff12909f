"""OpenThai-SystemOne oracle (oracle/openthai.c) pinned on the CPU.

Reference: src/models/openthai/model.rs (rms :84-94, forward :192-241, Full::run :244-299,
Delta::run :302-362).  The reference's own goldens (validation/openthai.reference.json) need the
real checkpoint, which is absent, so the oracle is pinned by:
  * an independent float64 restatement in matrix form (tests/np_openthai.py) on the synthetic
    tiny model, with planted mistakes that the comparison must catch;
  * closed forms of the pieces: the delta rule's write property (beta = 1 stores v under key k),
    a fully decayed state, a frozen empty state, a one-hot causal conv, RoPE identity at position
    0 and its relative-position property, a one-key softmax;
  * invariants of the whole forward: causality, thread-count and repeat bit-exactness.
"""
import numpy as np
import pytest

import np_openthai as nt


@pytest.fixture(scope="module")
def tiny(lh, po):
    img = lh.SynthImage("openthai-tiny", seed=5)
    g = po.Gguf(img.array())
    return img, g, po.OpenThai(g, threads=4)


def test_synthetic_image_follows_the_converter(tiny, po):
    img, g, m = tiny
    assert g.str("general.architecture") == "openthai_systemone"
    cfg = po.openthai_config(g)
    assert cfg["full"] == [0, 0, 0, 1] and (cfg["hq"], cfg["hkv"], cfg["nh"]) == (8, 2, 2)
    kind, dims, _ = g.tensor("model.layers.0.linear_attn.conv1d.weight")
    assert kind == 1 and dims == [4, 1, 3 * 2 * 128]   # F16, torch [C, 1, 4] reversed
    kind, dims, _ = g.tensor("model.layers.3.self_attn.q_proj.weight")
    assert kind == 1 and dims == [256, 2 * 8 * 256]
    for name, n in (("model.layers.0.linear_attn.A_log", 2), ("slot_head.bias", 256), ("log_temperature", 3)):
        kind, dims, _ = g.tensor(name)
        assert kind == 0 and dims == [n]


@pytest.mark.parametrize("n", [1, 5, 64, 150])
def test_forward_matches_f64_restatement(tiny, n):
    _, g, m = tiny
    ids = np.random.default_rng(n).integers(0, 700, n)
    pos = sorted({n - 1, n // 2, 0})
    got = m.forward(ids, pos)
    want = nt.F64OpenThai(g).forward(ids, pos)
    err = np.abs(got - want).max()
    assert err <= 2e-5 * max(1.0, np.abs(want).max()), err


@pytest.mark.parametrize("mistake", nt.MISTAKES)
def test_planted_mistakes_are_caught(tiny, mistake):
    _, g, m = tiny
    ids = np.random.default_rng(1).integers(0, 700, 48)
    pos = [47, 20]
    got = m.forward(ids, pos)
    bad = nt.F64OpenThai(g, mistake).forward(ids, pos)
    assert np.abs(got - bad).max() > 1e-3, mistake


def _qkv(rng, s, nh):
    return rng.normal(size=(s, 3 * nh * 128)).astype(np.float32)


def test_delta_rule_write_property(po):
    """beta = 1 and q = k at the last step: S^T k_hat = v exactly (k_hat . k_hat = 1), so the
    output is v / sqrt(128) whatever the earlier state."""
    rng = np.random.default_rng(2)
    s, nh = 9, 2
    qkv = _qkv(rng, s, nh)
    lw = nh * 128
    qkv[-1, :lw] = qkv[-1, lw:2 * lw]            # q = k at the last token
    a = rng.normal(size=(s, nh)).astype(np.float32)
    b = rng.normal(size=(s, nh)).astype(np.float32)
    b[-1] = 40.0                                   # sigmoid(40) == 1 in f32
    alog = np.array([0.5, 1.5], np.float32)
    dt = np.array([0.1, -0.2], np.float32)
    out = po.ot_gated_delta(qkv, a, b, alog, dt)
    v = qkv[-1, 2 * lw:]
    np.testing.assert_allclose(out[-1], v / np.sqrt(128.0), rtol=2e-4, atol=2e-5)


def test_delta_rule_full_decay_and_frozen_state(po):
    rng = np.random.default_rng(3)
    s, nh = 7, 2
    lw = nh * 128
    qkv = _qkv(rng, s, nh)
    a = rng.normal(size=(s, nh)).astype(np.float32)
    b = rng.normal(size=(s, nh)).astype(np.float32)
    # exp(-exp(20) * softplus(.)) == 0: each step sees an empty state, o = (k.q) beta v
    out = po.ot_gated_delta(qkv, a, b, np.full(nh, 20.0, np.float32), np.zeros(nh, np.float32))
    for t in range(s):
        for h in range(nh):
            q = qkv[t, h * 128:(h + 1) * 128].astype(np.float64)
            k = qkv[t, lw + h * 128:lw + (h + 1) * 128].astype(np.float64)
            v = qkv[t, 2 * lw + h * 128:2 * lw + (h + 1) * 128].astype(np.float64)
            kq = (k / np.sqrt(k @ k + 1e-6)) @ (q / np.sqrt(q @ q + 1e-6) / np.sqrt(128.0))
            beta = 1.0 / (1.0 + np.exp(-float(b[t, h])))
            np.testing.assert_allclose(out[t, h * 128:(h + 1) * 128], kq * beta * v, rtol=1e-4, atol=1e-6)
    # beta == 0 everywhere (sigmoid(-200) underflows to 0): nothing is ever written
    out = po.ot_gated_delta(qkv, a, np.full((s, nh), -200.0, np.float32), np.zeros(nh, np.float32),
                            np.zeros(nh, np.float32))
    assert not out.any()


def test_conv_one_hot_is_causal_kernel(po):
    rng = np.random.default_rng(4)
    s, ch = 12, 6
    conv = rng.normal(size=(ch, 4)).astype(np.float32)
    raw = np.zeros((s, ch), np.float32)
    raw[5, 2] = 1.0
    out = po.ot_conv_silu(raw, conv)
    silu = lambda x: x / (1.0 + np.exp(-x))
    want = np.zeros((s, ch))
    for i in range(5, 9):
        want[i, 2] = silu(conv[2, 3 - (i - 5)])
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=0)


def test_rope_identity_at_zero_and_relative_positions(po):
    rng = np.random.default_rng(6)
    x = rng.normal(size=(1, 256)).astype(np.float32)
    assert np.array_equal(po.ot_rope(x), x)            # position 0 rotates by 0
    s = 40
    u = np.tile(rng.normal(size=256).astype(np.float32), (s, 1))
    w = np.tile(rng.normal(size=256).astype(np.float32), (s, 1))
    ru, rw = po.ot_rope(u).astype(np.float64), po.ot_rope(w).astype(np.float64)
    assert np.array_equal(ru[:, 64:], u[:, 64:])       # only the first 64 dims rotate
    # <R(i) u, R(j) w> depends only on i - j; norms are preserved
    np.testing.assert_allclose(ru[7] @ rw[3], ru[30] @ rw[26], rtol=2e-5)
    np.testing.assert_allclose(np.linalg.norm(ru, axis=1), np.linalg.norm(u.astype(np.float64), axis=1), rtol=1e-6)


def test_attention_first_row_and_causality(po):
    rng = np.random.default_rng(8)
    s, hq, hkv = 10, 8, 2
    q = rng.normal(size=(s, hq * 256)).astype(np.float32)
    k = rng.normal(size=(s, hkv * 256)).astype(np.float32)
    v = rng.normal(size=(s, hkv * 256)).astype(np.float32)
    out = po.ot_attention(q, k, v)
    for h in range(hq):  # one visible key: p = 1, head h reads kv head h // 4
        assert np.array_equal(out[0, h * 256:(h + 1) * 256], v[0, (h // 4) * 256:(h // 4 + 1) * 256])
    k2, v2 = k.copy(), v.copy()
    k2[6:] += 1.0
    v2[6:] -= 2.0
    assert np.array_equal(po.ot_attention(q, k2, v2)[:6], out[:6])


def test_forward_causal_and_thread_exact(tiny, po):
    img, g, m = tiny
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 700, 80)
    pos = [10, 40, 79]
    a = m.forward(ids, pos)
    ids2 = ids.copy()
    ids2[41:] = rng.integers(0, 700, 39)
    b = m.forward(ids2, pos)
    assert np.array_equal(a[:2], b[:2]) and not np.array_equal(a[2], b[2])
    m1 = po.OpenThai(g, threads=1)
    assert np.array_equal(m1.forward(ids, pos), a)
    assert np.array_equal(m.forward(ids, pos), a)


def test_forward_rejects_invalid_sequences(tiny):
    _, _, m = tiny
    for ids, pos in (([], []), ([1, 2, 1024], [0]), ([1, 2, 3], [3]), ([1, -1], [0])):
        with pytest.raises(ValueError, match="invalid OpenThai token sequence"):
            m.forward(ids, pos)


# ---- request-level decide on an OpenThai model (host side: lg_decide_encode / lg_decide_scores)

def _req(rng, V, nq, perms=None, state_len=50):
    kinds = ["choice", "score", "noul"]
    qs = []
    for i in range(nq):
        kind = kinds[i % 3]
        k = {"choice": int(rng.integers(2, 9)), "score": int(rng.integers(2, 11)), "noul": 2}[kind]
        opts = [{"name": rng.integers(0, 600, int(rng.integers(1, 3))).tolist(),
                 "desc": rng.integers(0, 600, int(rng.integers(0, 3))).tolist()} for _ in range(k)]
        qs.append({"type": kind, "instruction": rng.integers(0, 600, int(rng.integers(0, 6))).tolist(), "options": opts})
    return {"state": rng.integers(0, 600, state_len).tolist(), "questions": qs, "permutations": perms}


def test_decide_control_tokens_come_from_the_tokenizer(tiny, lh):
    import pydecide as pd
    img, g, _ = tiny
    s = pd.spec(g)
    # where the synthetic writer put them (the openthai-tiny preset)
    assert (s["question"], s["state"], s["kind"], s["answer"]) == (960, 961, [962, 963, 964], 970)
    assert s["slot"][:3] == [700, 701, 702] and s["slot"][254] == 954 and (s["newline"], s["colon"]) == (198, 25)
    assert s["head_rows"] == list(range(256)) and (s["max_tokens"], s["max_state"]) == (1024, 512)
    req = {"state": [5, 6], "questions": [{"type": "noul", "instruction": [7], "options": [{"name": [8]}, {"name": [9]}]}]}
    ids, pos, _, _, _ = lh.decide_encode(lh.Gguf.from_bytes(img), req, 0)
    assert ids.tolist() == [961, 5, 6, 198, 960, 964, 7, 198, 700, 8, 198, 701, 9, 198, 970, 198]
    assert pos.tolist() == [14]


@pytest.mark.parametrize("seed", range(6))
def test_decide_encode_and_scores_match_oracle(tiny, lh, seed):
    import pydecide as pd
    img, g, _ = tiny
    lg = lh.Gguf.from_bytes(img)
    rng = np.random.default_rng(40 + seed)
    req = _req(rng, 1024, int(rng.integers(1, 5)), perms=[None, 3, 8][seed % 3], state_len=int(rng.integers(0, 900)))
    s = pd.spec(g)
    n = pd.passes(req)
    encs = []
    for p in range(n):
        ids, pos, order, trunc, npass = lh.decide_encode(lg, req, p)
        want = pd.encode(s, req, n, p)
        assert npass == n and np.array_equal(ids, want[0]) and np.array_equal(pos, want[1])
        assert order == want[2] and trunc == want[3]
        encs.append(want)
    logits = (rng.normal(size=(n, len(req["questions"]), 256)) * 2).astype(np.float32)
    got = lh.decide_scores(lg, req, logits)
    want = pd.aggregate(s, req, n, encs, logits)
    for a, b in zip(got["answers"], want["answers"]):
        assert np.array_equal(a["probabilities"], b["probabilities"])
        assert a["confidence"] == b["confidence"] and a["choice"] == b["choice"]
