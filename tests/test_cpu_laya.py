"""Laya encoder oracle (oracle/laya.c) pinned on the CPU.

Reference: src/models/laya/model.rs:60-416 and src/tensor.rs:103-192.  The reference's own
goldens (validation/refund.reference.json, numeric.reference.json) need the real checkpoints,
which are absent, so the oracle is pinned by:
  * an independent float64 restatement with its own graph walk (tests/np_laya.py) on the
    synthetic laya-tiny model, with planted mistakes that the comparison must catch;
  * closed forms of the pieces: LayerNorm output moments, the tanh-GELU formula, the local
    window and the bidirectional mask, RoPE identity at position 0;
  * invariants of the forward: window locality of a local layer, thread-count and repeat
    bit-exactness.
"""
import numpy as np
import pytest

import np_laya as nl


@pytest.fixture(scope="module")
def tiny(lh, po):
    img = lh.SynthImage("laya-tiny", seed=7)
    g = po.Gguf(img.array())
    return img, g, po.Laya(g, threads=4)


def test_synthetic_image_follows_the_reference_loader(tiny, po):
    img, g, m = tiny
    assert g.str("general.architecture") == "ggmlc" and "laya" in g.str("laya.checkpoint")
    assert g.num("laya.max_opts") == 16 and (m.L, m.d, m.hd, m.V) == (4, 128, 64, 1024)
    assert m.full == [True, False, False, True]


@pytest.mark.parametrize("n,markers,qtype", [(1, [0], 0), (9, [1, 4], 2), (130, [5, 9, 60, 127], 1), (512, list(range(3, 19)), 0)])
def test_forward_matches_f64_restatement(tiny, n, markers, qtype):
    _, g, m = tiny
    ids = np.random.default_rng(n).integers(0, 1000, n)
    got = m.forward(ids, markers, qtype)
    want = nl.F64Laya(g).forward(ids, markers, qtype)
    for a, b in zip(got, want):
        assert np.abs(a - b).max() <= 2e-6 * max(1.0, np.abs(b).max()), np.abs(a - b).max()


@pytest.mark.parametrize("mistake", nl.MISTAKES)
def test_planted_mistakes_are_caught(tiny, mistake):
    _, g, m = tiny
    ids = np.random.default_rng(2).integers(0, 1000, 200)
    markers = [7] if mistake == "entropy_k" else [3, 10, 50, 120]
    got = m.forward(ids, markers, 1)
    with np.errstate(all="ignore"):
        bad = nl.F64Laya(g, mistake).forward(ids, markers, 1)
    diff = max(float(np.nan_to_num(np.abs(a - b), nan=1.0).max()) for a, b in zip(got, bad))
    assert diff > 2e-5, mistake


def test_layer_norm_and_gelu_closed_forms(po):
    rng = np.random.default_rng(0)
    x = (rng.normal(size=(5, 96)) * 3 + 1).astype(np.float32)
    y = po.layer_norm(x, eps=1e-5).astype(np.float64)
    assert np.abs(y.mean(1)).max() < 1e-6 and np.abs(y.var(1) - 1).max() < 1e-4
    w, b = rng.normal(size=96).astype(np.float32), rng.normal(size=96).astype(np.float32)
    np.testing.assert_allclose(po.layer_norm(x, w, b, 1e-5), y * w + b, rtol=1e-5, atol=1e-5)
    assert po.gelu(0.0) == 0.0 and abs(po.gelu(10.0) - 10.0) < 1e-6 and abs(po.gelu(-10.0)) < 1e-6
    for v in (-2.5, -0.3, 0.7, 1.9):  # tanh form, not the erf form
        want = 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))
        assert abs(po.gelu(v) - want) < 2e-7


def test_attention_window_and_bidirectional(po):
    rng = np.random.default_rng(3)
    s, d, hd = 200, 128, 64
    qkv = rng.normal(size=(s, 3 * d)).astype(np.float32)
    out = po.laya_attention(qkv, hd, window=64)
    q2 = qkv.copy()
    q2[150:, d:] += 1.0       # keys/values of tokens >= 150
    out2 = po.laya_attention(q2, hd, window=64)
    assert np.array_equal(out[:85], out2[:85])       # |i - j| > 64 for every i < 86
    assert not np.array_equal(out[86:150], out2[86:150])  # later tokens are visible (bidirectional)
    full = po.laya_attention(qkv, hd)
    assert not np.array_equal(full[:85], po.laya_attention(q2, hd)[:85])
    # RoPE at position 0 is the identity (cos 1, sin 0)
    c, sn = np.ones((s, hd), np.float32), np.zeros((s, hd), np.float32)
    assert np.array_equal(po.laya_attention(qkv, hd, c, sn, 64), out)


def test_forward_repeat_and_threads(tiny, po):
    img, g, m = tiny
    ids = np.random.default_rng(4).integers(0, 1000, 300)
    a = m.forward(ids, [1, 2, 3], 0)
    m1 = po.Laya(g, threads=1)
    b = m1.forward(ids, [1, 2, 3], 0)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    assert all(np.array_equal(x, y) for x, y in zip(a, m.forward(ids, [1, 2, 3], 0)))


def test_forward_rejects_invalid_input(tiny):
    _, _, m = tiny
    with pytest.raises(ValueError, match="invalid inference input shape"):
        m.forward([1, 2], [2], 0)
    with pytest.raises(ValueError, match="invalid inference input shape"):
        m.forward([1] * 513, [0], 0)
    with pytest.raises(ValueError, match="invalid inference input shape"):
        m.forward([1, 2], [0], 3)
    with pytest.raises(ValueError, match="token ID out of range"):
        m.forward([1, 5000], [0], 0)
