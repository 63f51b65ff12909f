"""Error paths of the decoder engine on the GPU: every failure is a status and a message, nothing
aborts, and the engine stays usable (the reference's Result<_, String> contract,
src/models/mod.rs:13-23).

  KV pages exhausted by a batch: LG_ERR_OOM before anything runs, no page consumed;
  a KV pool no device can hold: engine creation fails with LG_ERR_OOM;
  non-finite output (src/models/laya/model.rs:412-414): an error, the sequence keeps its length.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _ids(n, V, seed):
    return np.random.default_rng(seed).integers(0, V, n).astype(np.int32)


def test_kv_exhaustion_is_oom_and_leaves_the_pool_intact(lh):
    img = lh.SynthImage("tiny-q8", seed=2)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=4 * 64)  # 4 pages
    V = eng.info["vocab"]
    print("kv exhaustion: 3 requests of 100 tokens need 6 of 4 pages", flush=True)
    seqs = [eng.seq_create() for _ in range(3)]
    with pytest.raises(lh.LayaError) as e:
        eng.batch([(s, _ids(100, V, i), [99]) for i, s in enumerate(seqs)])
    assert e.value.kind == "OOM" and "KV cache exhausted" in str(e.value)
    assert all(eng.seq_len(s) == 0 for s in seqs)
    # every page is still free: two requests of 128 tokens take all four
    out = eng.batch([(seqs[0], _ids(128, V, 7), [127]), (seqs[1], _ids(128, V, 8), [127])]).run([1, 2])
    assert np.isfinite(out[0]).all()
    # the pool is now full: one more token anywhere is OOM, for prefill and for decode alike
    with pytest.raises(lh.LayaError) as e:
        eng.forward(seqs[2], _ids(1, V, 9), [0], [1])
    assert e.value.kind == "OOM"
    with pytest.raises(lh.LayaError) as e:
        eng.decode(seqs[0], 3, 1)
    assert e.value.kind == "OOM" and eng.seq_len(seqs[0]) == 128
    # freeing a sequence gives its pages back
    eng.seq_free(seqs[1])
    assert eng.decode(seqs[0], 3, 4).shape == (4,)
    eng.close()


def test_kv_pool_beyond_any_device_fails_cleanly(lh):
    img = lh.SynthImage("tiny-q8", seed=2)
    g = lh.Gguf.from_bytes(img)
    for tokens in (1 << 40, 1 << 62):
        with pytest.raises(lh.LayaError) as e:
            lh.Engine(g, kv_tokens=tokens)
        assert e.value.kind == "OOM" and "KV pages" in str(e.value)
    eng = lh.Engine(g, kv_tokens=1024)  # the device is still usable
    assert np.isfinite(eng.forward(eng.seq_create(), [1, 2, 3], [2], [4, 5])).all()
    eng.close()


def test_non_finite_output_is_an_error(lh, po):
    """Head rows 7 and 8 get a +Inf / -Inf weight in column 0, so their logits are infinite: any call
    that returns them, and any greedy step (whose maximum is then +Inf), fails with
    "non-finite model output"; the sequence keeps its length and other rows still work."""
    img = lh.SynthImage("tiny-f16", seed=4)
    arr = img.array().copy()
    og = po.Gguf(arr)
    kind, dims, _ = og.tensor("output.weight")
    assert kind == 1  # F16
    off, d = og.offset("output.weight"), dims[0]
    arr[off + 2 * 7 * d:off + 2 * 7 * d + 2] = np.frombuffer(np.uint16(0x7C00).tobytes(), np.uint8)
    arr[off + 2 * 8 * d:off + 2 * 8 * d + 2] = np.frombuffer(np.uint16(0xFC00).tobytes(), np.uint8)
    eng = lh.Engine(lh.Gguf.from_bytes(arr), kv_tokens=2048)
    V = eng.info["vocab"]
    ids = _ids(40, V, 3)
    s = eng.seq_create()
    print("non-finite: option rows 7, 8", flush=True)
    with pytest.raises(lh.LayaError, match="non-finite model output"):
        eng.forward(s, ids, [39], [5, 7])
    assert eng.seq_len(s) == 0
    with pytest.raises(lh.LayaError, match="non-finite model output"):
        eng.forward(s, ids, [39])  # full vocabulary
    assert eng.seq_len(s) == 0
    ok = eng.forward(s, ids, [39], [5, 6])
    assert np.isfinite(ok).all() and eng.seq_len(s) == 40
    with pytest.raises(lh.LayaError, match="non-finite model output"):
        eng.decode(s, 1, 3)
    assert eng.seq_len(s) == 40
    eng.close()
