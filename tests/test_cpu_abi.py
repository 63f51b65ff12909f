"""The C-ABI library on a host without a GPU: it loads, exports every function include/lg.h
declares, and its host-only entry points (formats, GGUF, synthetic models, option scoring)
work.  Nothing here launches a kernel.
"""
import ctypes
import hashlib
import os

import numpy as np
import pytest

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14


def test_exports_every_header_function(lh):
    L = lh.lib()
    declared = lh.header_functions()
    assert len(declared) >= 30
    missing = [n for n in declared if not hasattr(L, n)]
    assert not missing, f"declared in lg.h but not exported: {missing}"
    # the Python binding types every declared function (and nothing undeclared)
    raw = ctypes.CDLL(lh.LIB_PATH)
    for n in declared:
        assert getattr(L, n).argtypes is not None or n in ("lg_last_error", "lg_version"), n
        assert hasattr(raw, n)
    assert lh.lib().lg_version().decode().startswith("laya-mi355x ")


def test_error_reporting_contract(lh):
    L = lh.lib()
    z = np.zeros(4, np.float32)
    rc = L.lg_option_scores(z.ctypes.data_as(ctypes.c_void_p), 0, 1.0, None, None)
    assert rc == 1 and b"k must be" in L.lg_last_error()
    rc = L.lg_option_scores(z.ctypes.data_as(ctypes.c_void_p), 4, 0.0, None, None)
    assert rc == 1 and b"temperature" in L.lg_last_error()
    rc = L.lg_option_scores(None, 4, 1.0, None, None)
    assert rc == 1 and L.lg_last_error() == b"logits must not be null"
    # a successful call clears the message
    assert L.lg_option_scores(z.ctypes.data_as(ctypes.c_void_p), 4, 1.0, None, None) == 0
    assert L.lg_last_error() == b""
    with pytest.raises(lh.LayaError) as e:
        lh.option_confidence([0.5, 0.5], mode=7)
    assert e.value.kind == "INVALID"


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks behaviour on a host without a GPU")
def test_engine_without_gpu_fails_loudly(lh):
    img = lh.SynthImage("tiny-f16", seed=1)
    g = lh.Gguf.from_bytes(img)
    with pytest.raises(lh.LayaError) as e:
        lh.Engine(g)
    assert e.value.kind == "DEVICE"


PRESETS = {
    # preset: (L, d, hq, hkv, hd, f, V, eps, theta, matrix kinds)
    "plumbing-f16": (6, 512, 8, 8, 64, 1408, 32000, 1e-5, 1e4, {F16}),
    "q8-2048": (24, 2048, 16, 16, 128, 5632, 32000, 1e-5, 1e4, {Q8_0}),
    "q4km-7b": (28, 3584, 28, 4, 128, 18944, 152064, 1e-6, 1e6, {Q4_K, Q6_K}),
    "f16-7b": (28, 3584, 28, 4, 128, 18944, 152064, 1e-6, 1e6, {F16}),
}


@pytest.mark.parametrize("preset", list(PRESETS))
def test_synthetic_presets(lh, po, preset):
    """Shapes of the workload models; one layer generated (the others are the same shape)."""
    L, d, hq, hkv, hd, f, V, eps, theta, kinds = PRESETS[preset]
    img = lh.SynthImage(preset, seed=3, n_layers=1)
    g = lh.Gguf.from_bytes(img)
    got = [g.num(f"laya.decoder.{k}") for k in ("embedding_length", "head_count", "head_count_kv", "key_length",
                                                "feed_forward_length", "vocab_size")]
    assert got == [d, hq, hkv, hd, f, V] and g.num("laya.decoder.block_count") == 1
    assert np.float32(g.num("laya.decoder.layer_norm_rms_epsilon")) == np.float32(eps)
    assert g.num("laya.decoder.rope_freq_base") == theta
    assert g.str("general.architecture") == "ggmlc" and g.str("laya.model_name") == "laya-decoder"
    mats = [n for n in g.names() if n.endswith(".weight") and "norm" not in n and n != "tok_emb.weight"]
    assert {g.tensor(n)[0] for n in mats if n != "output.weight"} == kinds
    # the oracle's reader agrees on every tensor
    o = po.Gguf(img.array())
    for n in g.names():
        k1, d1, r1 = g.tensor(n)
        k2, d2, r2 = o.tensor(n)
        assert (k1, d1) == (k2, d2) and len(r1) == len(r2)
    # RoPE tables: cos/sin of pos * theta^(-2j/hd), the same angle for j and j + hd/2
    kind, dims, raw = g.tensor("cos_full")
    cos = np.frombuffer(raw, np.float32).reshape(dims[1], dims[0])
    sin = np.frombuffer(g.tensor("sin_full")[2], np.float32).reshape(dims[1], dims[0])
    assert dims[0] == hd
    pos = np.array([0, 1, 7, 100, dims[1] - 1])[:, None]
    j = np.arange(hd // 2)[None, :]
    ang = pos * theta ** (-2.0 * j / hd)
    for tab, fn in ((cos, np.cos), (sin, np.sin)):
        assert np.abs(tab[pos[:, 0], :hd // 2] - fn(ang)).max() < 2e-6 * max(1, pos.max() / 1000)
        assert np.array_equal(tab[:, :hd // 2], tab[:, hd // 2:])
    assert (cos[0] == 1).all() and (sin[0] == 0).all()
    g.close()


def test_synthetic_determinism(lh):
    a = lh.SynthImage("tiny-q4k", seed=9).bytes()
    b = lh.SynthImage("tiny-q4k", seed=9).bytes()
    c = lh.SynthImage("tiny-q4k", seed=10).bytes()
    assert a == b and a != c and len(a) == len(c)
    # layer count override: the embeddings and the first layer do not depend on how many follow
    g1 = lh.Gguf.from_bytes(lh.SynthImage("tiny-q8", seed=2, n_layers=1))
    g3 = lh.Gguf.from_bytes(lh.SynthImage("tiny-q8", seed=2, n_layers=3))
    assert g3.num("laya.decoder.block_count") == 3
    for n in g1.names():
        if n == "tok_emb.weight" or ".0." in n:
            assert g1.tensor(n) == g3.tensor(n), n
    with pytest.raises(lh.LayaError, match="preset"):
        lh.SynthImage("no-such-preset")


def test_synthetic_value_distributions(lh):
    """Value rules of the workload models: Q8_0 codes in [-127, 127] with scales
    f16(|N(0, 0.002)|); F16 plumbing weights ~N(0, 0.02); norms 1.0."""
    g = lh.Gguf.from_bytes(lh.SynthImage("q8-2048", seed=4, n_layers=1))
    kind, dims, raw = g.tensor("qkv.0.weight")
    blocks = np.frombuffer(raw, np.uint8).reshape(-1, 34)[:20000]
    codes = blocks[:, 2:].view(np.int8)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    assert codes.min() == -127 and codes.max() == 127
    # U{-127..127}: mean 0, std sqrt(127*128/3) = 73.7; bounds at ~5 standard errors of 640k draws
    assert abs(codes.astype(np.float64).mean()) < 0.5 and abs(codes.std() - np.sqrt(127 * 128 / 3)) < 0.5
    assert (d >= 0).all() and abs(d.mean() - 0.002 * np.sqrt(2 / np.pi)) < 5e-5
    g = lh.Gguf.from_bytes(lh.SynthImage("plumbing-f16", seed=4, n_layers=1))
    w = np.frombuffer(g.tensor("wo.0.weight")[2], np.float16).astype(np.float64)
    assert abs(w.std() - 0.02) < 5e-4 and abs(w.mean()) < 5e-4
    norm = np.frombuffer(g.tensor("attn_norm.0.weight")[2], np.float32)
    assert (norm == 1).all()


def test_synth_file_roundtrip(lh, tmp_path):
    p = str(tmp_path / "tiny.gguf")
    lh.synth_file("tiny-f16", 4, p)
    img = lh.SynthImage("tiny-f16", seed=4)
    assert hashlib.sha256(open(p, "rb").read()).digest() == hashlib.sha256(img.bytes()).digest()
    g = lh.Gguf.open(p)
    assert g.num("laya.decoder.head_count") == 4
    g.close()
