"""lg_decode_noalloc (the allocation-free decode) against lg_decode through the C ABI.

Both run the same kernels on the same sequence state, so tokens and every step's full-vocabulary
logits must be bit-identical.  Two calls in a row, the second with a shorter context and fewer
steps, so a stale scratch from the first call would show.  On a fresh engine the allocation-free
decode grows none of the engine's device workspaces (lg_engine_workspace_bytes), while lg_decode
then grows its decode workspace.  (The 16 MiB scratch is not reachable with the shipped model
shapes: decode refuses contexts beyond 65,536 tokens, and the 7B shape would need it at ~70k.)
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("preset,layers", [("tiny-q8", 0), ("q8-2048", 2)])
def test_decode_noalloc_equals_decode(lh, preset, layers):
    img = lh.SynthImage(preset, seed=21, n_layers=layers)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=4096)
    V = eng.info["vocab"]
    rng = np.random.default_rng(4)
    for ctx, steps in ((300, 12), (70, 5)):  # the second call is smaller
        print(f"{preset}: decode_noalloc after {ctx} tokens, {steps} steps", flush=True)
        ids = rng.integers(0, V, ctx).astype(np.int32)
        base = eng.seq_create()
        eng.forward(base, ids, [], [0])
        a, b = eng.seq_fork(base, ctx), eng.seq_fork(base, ctx)
        want_t, want_l = eng.decode(a, int(ids[-1]), steps, want_logits=True)
        got_t, got_l = eng.decode(b, int(ids[-1]), steps, want_logits=True, noalloc=True)
        assert np.array_equal(got_t, want_t)
        assert np.array_equal(got_l.view(np.uint32), want_l.view(np.uint32))
        assert eng.seq_len(b) == ctx + steps
        # without logits as well (tokens only)
        c = eng.seq_fork(base, ctx)
        assert np.array_equal(eng.decode(c, int(ids[-1]), steps, noalloc=True), want_t)
        for s in (a, b, c, base):
            eng.seq_free(s)
    eng.close()


def test_decode_noalloc_allocates_nothing(lh):
    img = lh.SynthImage("tiny-q8", seed=22)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=2048)
    V = eng.info["vocab"]
    ids = np.random.default_rng(5).integers(0, V, 200).astype(np.int32)
    s = eng.seq_create()
    eng.forward(s, ids, [], [0])
    before = eng.workspace_bytes()
    print(f"fresh engine: {before} workspace bytes before the first decode", flush=True)
    a, b = eng.seq_fork(s, 200), eng.seq_fork(s, 200)
    got = eng.decode(a, int(ids[-1]), 6, noalloc=True)
    assert eng.workspace_bytes() == before, "lg_decode_noalloc grew a device workspace"
    want = eng.decode(b, int(ids[-1]), 6)
    assert eng.workspace_bytes() > before, "lg_decode's workspace is not visible to the query"
    assert np.array_equal(got, want)
    eng.close()


def test_decode_noalloc_errors_leave_the_sequence(lh):
    img = lh.SynthImage("tiny-q8", seed=21)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=1024)
    s = eng.seq_create()
    eng.forward(s, np.arange(10, dtype=np.int32), [], [0])
    with pytest.raises(lh.LayaError, match="outside the vocabulary"):
        eng.decode(s, eng.info["vocab"], 3, noalloc=True)
    with pytest.raises(lh.LayaError, match="exceeds the context length"):
        eng.decode(s, 1, eng.info["context"], noalloc=True)
    assert eng.seq_len(s) == 10
    assert eng.decode(s, 1, 2, noalloc=True).shape == (2,)
    eng.close()
