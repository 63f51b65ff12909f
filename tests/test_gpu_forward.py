"""GPU forward-pass parity through the C ABI against the CPU oracle.

Reference path: Model::forward (src/models/openthai/model.rs:192-241) with the decoder
assembled from the reference primitives, option scoring (src/models/openthai/decision.rs:
268-279), argmax first-max-wins (:330-335).  Invariants the reference's own tests hold
(validation/smoke.py:25-28 repeat determinism, openthai_edges.py no state leakage) are
checked as bit-exact properties of the GPU path.
"""
import numpy as np
import pytest

from parity import (PREC_NAMES, assert_argmax_equal, assert_bits_equal, assert_logits_close, assert_probs_close,
                    logit_bar, logit_error, tie_window)

pytestmark = pytest.mark.gpu

OPTIONS = [3, 17, 42, 99]


@pytest.fixture(scope="module", params=[("tiny-f16", 0), ("tiny-q8", 0), ("tiny-q4k", 0), ("tiny-f16-128", 0),
                                        ("tiny-f16", 1), ("tiny-f16-128", 1),
                                        ("tiny-f16", 2), ("tiny-q4k", 2), ("tiny-f16-128", 2)],
                ids=lambda p: f"{p[0]}-{PREC_NAMES[p[1]]}")
def pair(request, lh, po):
    preset, prec = request.param
    img = lh.SynthImage(preset, seed=5)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=8192, precision=prec)
    om = po.Model(po.Gguf(img.array()), threads=8)
    yield preset, eng, om
    eng.close()


def _ids(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.int32)


def test_forward_options_and_probs(pair, lh, po):
    preset, eng, om = pair
    ids = _ids(150, om.V, 1)
    pos = [149, 100, 63, 64, 0]
    print(f"{preset}: forward 150 tokens", flush=True)
    s = eng.seq_create()
    b = eng.batch([(s, ids, pos)])
    logits, probs, logprobs = b.run(OPTIONS, temperature=1.0)
    want = om.forward(ids, pos, OPTIONS)
    prec = eng.info["precision"]
    assert_logits_close(logits, want, rel=logit_bar(prec))
    assert_argmax_equal(logits, want, rel=tie_window(prec))
    for r in range(len(pos)):
        p_ref, lp_ref, _ = po.option_scores(want[r])
        assert_probs_close(probs[r], p_ref)
        assert np.abs(logprobs[r] - lp_ref).max() < 2e-2 * max(1.0, np.abs(lp_ref).max())
    eng.seq_free(s)


def test_forward_full_vocab(pair):
    preset, eng, om = pair
    ids = _ids(77, om.V, 2)
    s = eng.seq_create()
    got = eng.forward(s, ids, [76, 30])
    want = om.forward(ids, [76, 30])
    prec = eng.info["precision"]
    assert_logits_close(got, want, rel=logit_bar(prec))
    assert_argmax_equal(got, want, rel=tie_window(prec))
    eng.seq_free(s)


def test_repeat_is_bit_identical(pair):
    preset, eng, om = pair
    ids = _ids(90, om.V, 3)
    outs = []
    for _ in range(3):
        s = eng.seq_create()
        outs.append(eng.forward(s, ids, [89, 5], OPTIONS))
        eng.seq_free(s)
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_batch_equals_single(pair):
    """Batch composition must not change any request's result (bit-exact)."""
    preset, eng, om = pair
    reqs = [(_ids(n, om.V, 10 + n), [n - 1, n // 2]) for n in (33, 100, 64, 7)]
    singles = []
    for ids, pos in reqs:
        s = eng.seq_create()
        singles.append(eng.forward(s, ids, pos, OPTIONS))
        eng.seq_free(s)
    seqs = [eng.seq_create() for _ in reqs]
    b = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)])
    logits, _, _ = b.run(OPTIONS)
    assert np.array_equal(np.concatenate(singles), logits)
    for s in seqs:
        eng.seq_free(s)


def test_continuation_equals_one_shot(pair):
    """Prefill in two calls over the KV cache == one call (bit-exact per row)."""
    preset, eng, om = pair
    ids = _ids(130, om.V, 4)
    s1 = eng.seq_create()
    one = eng.forward(s1, ids, [129], OPTIONS)
    s2 = eng.seq_create()
    eng.forward(s2, ids[:70], [], OPTIONS)
    two = eng.forward(s2, ids[70:], [59], OPTIONS)
    assert eng.seq_len(s2) == 130
    assert np.array_equal(one, two)
    eng.seq_free(s1)
    eng.seq_free(s2)


def test_fork_shared_prefix(pair):
    """Forked sequences (shared whole pages, copied partial page) == unshared one-shot."""
    preset, eng, om = pair
    prefix = _ids(150, om.V, 6)
    a = eng.seq_create()
    eng.forward(a, prefix, [], OPTIONS)
    for cut, seed in ((128, 7), (150, 8), (97, 9)):
        suffix = _ids(40, om.V, seed)
        b = eng.seq_fork(a, cut)
        got = eng.forward(b, suffix, [39, 0], OPTIONS)
        s = eng.seq_create()
        ref = eng.forward(s, np.concatenate([prefix[:cut], suffix]), [cut + 39, cut], OPTIONS)
        assert np.array_equal(got, ref), f"fork at {cut} differs"
        want = om.forward(np.concatenate([prefix[:cut], suffix]), [cut + 39, cut], OPTIONS)
        assert_logits_close(got, want)
        eng.seq_free(b)
        eng.seq_free(s)
    eng.seq_free(a)


def test_decode_teacher_forced(pair, po):
    """Greedy decode over the paged cache; every step's argmax and logits vs the oracle fed
    the same tokens (teacher-forced, so one near-tie cannot desynchronise later steps)."""
    preset, eng, om = pair
    ids = _ids(70, om.V, 12)
    s = eng.seq_create()
    eng.forward(s, ids[:-1], [], OPTIONS)
    toks, logits = eng.decode(s, int(ids[-1]), 12, want_logits=True)
    c = om.cache(200)
    om.prefill(c, ids[:-1], [])
    feed = [int(ids[-1])] + [int(t) for t in toks[:-1]]
    ties = 0
    for i, t in enumerate(feed):
        want = om.head(om.prefill(c, [t], [0]))
        err = assert_logits_close(logits[i], want)
        # near-ties: top-2 gap under 50x the observed error (at least 1e-4 of the top logit)
        ties += assert_argmax_equal(logits[i][None], want, rel=max(1e-4, 50 * err))
        assert int(toks[i]) == int(np.argmax(logits[i]))
    print(f"{preset}: decode near-ties {ties}")
    eng.seq_free(s)


def test_decode_graph_equals_stream_decode(pair):
    """lg_decode_graph (every step's kernels captured into one HIP graph) gives the same tokens as
    lg_decode and leaves the sequence as long, with the same cache contents."""
    preset, eng, om = pair
    ids = _ids(40, om.V, 13)
    s = eng.seq_create()
    eng.forward(s, ids[:-1], [], OPTIONS)
    a, b = eng.seq_fork(s, len(ids) - 1), eng.seq_fork(s, len(ids) - 1)
    want = eng.decode(a, int(ids[-1]), 9)
    for _ in range(2):                       # twice: the second capture starts from a longer sequence
        got, cap_ms, run_ms = eng.decode_graph(b, int(ids[-1]) if _ == 0 else int(want[-1]), 9)
        if _ == 0:
            np.testing.assert_array_equal(got, want)
            assert eng.seq_len(b) == eng.seq_len(a)
            ka, kb = eng.seq_kv_read(a, 0, 0, eng.seq_len(a)), eng.seq_kv_read(b, 0, 0, eng.seq_len(b))
            for x, y in zip(ka, kb):
                np.testing.assert_array_equal(x, y)
        assert cap_ms > 0 and run_ms > 0
    more = eng.decode(a, int(want[-1]), 9)
    np.testing.assert_array_equal(got, more)
    for q in (a, b, s):
        eng.seq_free(q)


def test_decode_after_canceled_forward(pair, lh):
    """A canceled forward keeps the pages it reserved, so the sequence's page table outgrows its
    tokens; decode then lays its attention partials out by the whole table and gives the tokens of
    an untouched sequence (stream and no-allocation entry points)."""
    preset, eng, om = pair
    ids = _ids(20, om.V, 17)
    a, b = eng.seq_create(), eng.seq_create()
    eng.forward(a, ids, [], OPTIONS)
    eng.forward(b, ids, [], OPTIONS)
    n = min(300, om.ctx - 40)
    with pytest.raises(lh.LayaError) as e:
        eng.forward(b, _ids(n, om.V, 18), [n - 1], OPTIONS, cancel=lambda _: 1)
    assert e.value.kind == "CANCELED" and eng.seq_len(b) == 20
    want = eng.decode(a, 5, 6)
    np.testing.assert_array_equal(eng.decode(b, 5, 6), want)
    np.testing.assert_array_equal(eng.decode(b, int(want[-1]), 3, noalloc=True), eng.decode(a, int(want[-1]), 3))
    for q in (a, b):
        eng.seq_free(q)


@pytest.mark.parametrize("zeroed", [0, 100])
def test_decode_argmax_ties_keep_the_first_index(lh, po, zeroed):
    """The decode's full-vocab argmax keeps the first maximum (src/models/openthai/decision.rs:330-335).
    Every head row set to row 1 makes all logits tie bit for bit, so each step emits token 0; with rows
    0..99 zeroed as well, the first tied maximum is 0 or 100 by the sign of the shared logit."""
    img = lh.SynthImage("tiny-f16", seed=3)  # keeps the image's memory alive while it is copied
    arr = img.array().copy()
    og = po.Gguf(arr)
    kind, (cols, rows), _ = og.tensor("output.weight")
    assert kind == 1  # F16
    off = og.offset("output.weight")
    head = arr[off:off + rows * cols * 2].reshape(rows, cols * 2)
    head[:] = head[1]
    head[:zeroed] = 0
    eng = lh.Engine(lh.Gguf.from_bytes(arr), kv_tokens=1024)
    s = eng.seq_create()
    eng.forward(s, [3, 4, 5], [], OPTIONS)
    toks, logits = eng.decode(s, 6, 5, want_logits=True)
    for i in range(5):
        assert int(toks[i]) == int(np.argmax(logits[i]))
        if zeroed == 0:
            assert int(toks[i]) == 0 and (logits[i] == logits[i][0]).all()
        else:
            assert int(toks[i]) == (100 if logits[i][100] > 0 else 0)
    eng.seq_free(s)
    eng.close()


def test_errors_are_reported(pair, lh):
    preset, eng, om = pair
    s = eng.seq_create()
    with pytest.raises(lh.LayaError) as e:
        eng.forward(s, [om.V], [0], OPTIONS)
    assert e.value.kind == "INVALID" and "vocabulary" in str(e.value)
    with pytest.raises(lh.LayaError):
        eng.forward(s, [1, 2, 3], [3], OPTIONS)
    with pytest.raises(lh.LayaError):
        eng.forward(s, np.ones(om.ctx + 1, np.int32), [0], OPTIONS)
    with pytest.raises(lh.LayaError) as e:
        eng.forward(s, [1, 2], [1], OPTIONS, cancel=lambda _: 1)
    assert e.value.kind == "CANCELED"
    with pytest.raises(lh.LayaError) as e:  # an empty request is refused, not run
        eng.forward(s, np.zeros(0, np.int32), [], OPTIONS)
    assert e.value.kind == "INVALID" and "empty" in str(e.value)
    assert eng.seq_len(s) == 0
    # the engine stays usable after errors
    out = eng.forward(eng.seq_create(), [1, 2, 3], [2], OPTIONS)
    assert np.isfinite(out).all()
    eng.seq_free(s)


@pytest.mark.parametrize("prec", [0, 1, 2], ids=["exact", "fast", "kv16"])
def test_golden_logits(lh, prec):
    """The committed float64 brute-force logits (tests/golden/forward_tiny.npz)."""
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "forward_tiny.npz"), allow_pickle=False)
    for preset in ("tiny-f16", "tiny-q8", "tiny-q4k"):
        img = lh.SynthImage(preset, seed=int(gold["seed"]))
        eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=1024, precision=prec)
        got = eng.forward(eng.seq_create(), gold[f"{preset}/ids"], gold[f"{preset}/pos"])
        err = assert_logits_close(got, gold[f"{preset}/logits"], rel=logit_bar(prec))
        assert_argmax_equal(got, gold[f"{preset}/logits"], rel=tie_window(prec))
        print(f"{preset} prec {prec}: golden rel {err:.2e}")
        eng.close()


@pytest.mark.parametrize("prec", [0, 1, 2], ids=["exact", "fast", "kv16"])
def test_plumbing_model_decision(lh, po, prec):
    """The CPU-runnable plumbing model: 128-token prompt + one yes/no question block."""
    img = lh.SynthImage("plumbing-f16", seed=1)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=4096, precision=prec)
    om = po.Model(po.Gguf(img.array()), threads=8)
    rng = np.random.default_rng(99)
    ids = np.concatenate([rng.integers(0, 32000, 128), rng.integers(0, 32000, 16)]).astype(np.int32)
    yes_no = [1939, 4874]
    s = eng.seq_create()
    logits, probs, _ = eng.batch([(s, ids, [143])]).run(yes_no)
    want = om.forward(ids, [143], yes_no)
    p_ref, _, _ = po.option_scores(want[0])
    assert_logits_close(logits, want, rel=logit_bar(prec))
    assert_probs_close(probs[0], p_ref)
    assert int(np.argmax(probs[0])) == int(np.argmax(p_ref))
    print(f"plumbing: logit err {logit_error(logits, want):.2e} probs {probs[0]} ref {p_ref}")
    eng.close()


@pytest.mark.parametrize("layers,tokens", [(4, 400)])
def test_q8_2048_full_width(lh, po, layers, tokens):
    """The Q8_0 d2048 decoder at full width (reduced depth so the oracle finishes in seconds):
    f32-faithful prefill against the oracle, 12 answer positions, 4 options each."""
    img = lh.SynthImage("q8-2048", seed=3, n_layers=layers)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=4096)
    om = po.Model(po.Gguf(img.array()), threads=16)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, 32000, tokens).astype(np.int32)
    pos = np.sort(rng.choice(tokens, 12, replace=False)).astype(np.int32)
    opts = rng.choice(32000, 4, replace=False).astype(np.int32)
    s = eng.seq_create()
    logits, probs, _ = eng.batch([(s, ids, pos)]).run(opts)
    want = om.forward(ids, pos, opts)
    p_ref = np.stack([po.option_scores(w)[0] for w in want])
    # this model amplifies f32 rounding layer over layer: at 4 layers two correct f32 orders already
    # sit up to 2.1e-4 apart (the oracle against a float64 forward), so the exact mode's bar here is
    # 5e-4 -- still a quarter of what one f16-only operand costs at a single layer (~2e-3)
    err = assert_logits_close(logits, want, rel=5e-4)
    perr = assert_probs_close(probs, p_ref)
    assert_argmax_equal(logits, want, rel=1e-3)
    print(f"q8-2048 L{layers} T{tokens}: logit rel {err:.2e} prob {perr:.2e}")
    eng.close()


def test_q8_large_batch_tiles_equal_single_requests(lh, po):
    """Exact Q8_0 prefill GEMMs take 256 x 256 tiles over the weights' prefill copy once a launch has
    at least one tile per CU, and 128 x 128 tiles below that.  Both must give the same bits: a batch of
    16 x 512 tokens (every projection on the large tiles) equals each request run alone (small tiles),
    and a request of the batch matches the oracle at the exact mode's bar."""
    img = lh.SynthImage("q8-2048", seed=11, n_layers=2)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=16 * 576, max_batch_tokens=16 * 512)
    rng = np.random.default_rng(7)
    reqs = [(rng.integers(0, 32000, 512).astype(np.int32), [7, 100, 511]) for _ in range(16)]
    opts = [5, 77, 901, 31999]
    seqs = [eng.seq_create() for _ in reqs]
    logits, _, _ = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)]).run(opts)
    for s in seqs:
        eng.seq_free(s)
    for r in (0, 9, 15):
        s = eng.seq_create()
        single = eng.forward(s, reqs[r][0], reqs[r][1], opts)
        eng.seq_free(s)
        assert_bits_equal(single, logits[3 * r:3 * r + 3])
    om = po.Model(po.Gguf(img.array()), threads=16)
    want = om.forward(reqs[9][0], reqs[9][1], opts)
    err = assert_logits_close(logits[27:30], want, rel=logit_bar(0))
    print(f"q8-2048 L2 16 x 512: bit-identical to single requests; logit rel {err:.2e} vs oracle")
    eng.close()


@pytest.mark.parametrize("prec", [0, 2], ids=["exact", "kv16"])
def test_q8_fused_qkv_epilogue_ragged_continuations(lh, po, prec):
    """A batch big enough for the 256 x 256 q|k|v GEMM stores q, k and v from its own epilogue
    (RoPE, q planes, K page rows, V page columns); requests alone keep the f32 q|k|v rows and the
    RoPE kernel.  Ragged requests continue sequences that already hold 0..130 tokens, so rows meet
    positions that are not multiples of 4 and quads of rows that straddle a sequence or a page: the
    V columns' four-slot stores and their one-slot fallback both run.  Batch == alone, bit for bit,
    at positions in every request, and one request matches the oracle.  Both cache formats (hi/lo
    planes, f16)."""
    img = lh.SynthImage("q8-2048", seed=29, n_layers=2)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=2 * 4608, max_batch_tokens=4096, precision=prec)
    rng = np.random.default_rng(31)
    # tokens each sequence holds before the batch: request 0's rows and positions agree mod 4 (the
    # four-slot V stores), every other request's do not
    heads = [36, 0, 61, 5, 0, 130, 2]
    lens = [701, 1290, 333, 999, 517, 65, 7]  # 3912 batch rows: 16 row tiles x 24 column tiles
    opts = [5, 77, 901, 31999]
    ctx = [rng.integers(0, 32000, h + n).astype(np.int32) for h, n in zip(heads, lens)]
    pos = [sorted({0, 1, 2, 3, n // 2, n - 2, n - 1} & set(range(n))) for n in lens]
    seqs = []
    for h, ids in zip(heads, ctx):
        s = eng.seq_create()
        if h:
            eng.forward(s, ids[:h], [], opts)
        seqs.append(s)
    print(f"q8-2048 L2: ragged batch of {sum(lens)} rows after heads {heads}", flush=True)
    logits, _, _ = eng.batch([(s, ids[h:], p) for s, h, ids, p in zip(seqs, heads, ctx, pos)]).run(opts)
    row = 0
    for r, (h, ids, p) in enumerate(zip(heads, ctx, pos)):
        s = eng.seq_create()
        if h:
            eng.forward(s, ids[:h], [], opts)
        single = eng.forward(s, ids[h:], p, opts)
        eng.seq_free(s)
        assert_bits_equal(single, logits[row:row + len(p)])
        row += len(p)
    om = po.Model(po.Gguf(img.array()), threads=16)
    want = om.forward(ctx[5], [heads[5] + q for q in pos[5]], opts)
    first = sum(len(p) for p in pos[:5])
    err = assert_logits_close(logits[first:first + len(pos[5])], want, rel=logit_bar(prec))
    print(f"q8-2048 ragged continuations ({PREC_NAMES[prec]}): bit-identical to single requests; logit rel "
          f"{err:.2e} vs oracle")
    for s in seqs:
        eng.seq_free(s)
    eng.close()


def test_kv16_cache_holds_the_exact_values_rounded(lh):
    """The kv16 mode's cache holds each k and v the exact mode holds (as hi + lo planes) rounded to the
    nearest f16, from every writer: the fused q|k|v epilogue (a 16 x 512 batch), the RoPE kernel (a
    request alone) and the decode step.  Layer 0 only: from layer 1 on the two modes' inputs differ by
    the cache rounding itself."""
    img = lh.SynthImage("q8-2048", seed=41, n_layers=2)
    rng = np.random.default_rng(43)
    reqs = [rng.integers(0, 32000, 512).astype(np.int32) for _ in range(16)]
    alone = rng.integers(0, 32000, 200).astype(np.int32)
    got = {}
    for prec in (0, 2):
        eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=16 * 576 + 1024, max_batch_tokens=16 * 512,
                        precision=prec)
        assert eng.info["kv_elem_bytes"] == (4 if prec == 0 else 2)
        seqs = [eng.seq_create() for _ in reqs]
        eng.batch([(s, ids, [511]) for s, ids in zip(seqs, reqs)]).run([1, 2])
        one = eng.seq_create()
        eng.forward(one, alone, [], [1, 2])
        toks = eng.decode(one, 7, 3)
        got[prec] = ([eng.seq_kv_read(s, 0, 0, 512) for s in (seqs[0], seqs[9], seqs[15])],
                     eng.seq_kv_read(one, 0, 0, 203), toks)
        eng.close()
    (bx, ox, tx), (bh, oh, th) = got[0], got[2]
    n_one = 201 + int(np.argmin(tx[:2] == th[:2])) if not np.array_equal(tx[:2], th[:2]) else 203
    pairs = [(x, h) for bxr, bhr in zip(bx, bh) for x, h in zip(bxr, bhr)]
    pairs += [(x[:n_one], h[:n_one]) for x, h in zip(ox, oh)]
    # the kv16 value is the exact mode's hi plane, f16(k); f16(hi + lo) equals it except where lo is
    # exactly half an f16 step of hi (a tie the sum rounds to even, while hi was rounded from k itself)
    worst, mism, total = 0.0, 0, 0
    for x, h in pairs:
        r16 = x.astype(np.float16)
        ulp = np.spacing(np.abs(h.astype(np.float16))).astype(np.float64)
        dist = np.abs(h.astype(np.float64) - x.astype(np.float64)) / ulp
        worst = max(worst, float(dist.max()))
        off = r16.astype(np.float32) != h
        x64 = x.astype(np.float64)
        assert (np.abs(x64 - h)[off] == np.abs(x64 - r16.astype(np.float64))[off]).all(), \
            "a kv16 value that is neither the exact value rounded nor the other side of a tie"
        mism += int(off.sum())
        total += h.size
    print(f"kv16 cache vs exact cache: worst distance {worst:.4f} f16 steps, {mism} of {total} values at an "
          f"exact half-step tie of the hi + lo sum", flush=True)
    assert worst <= 0.5


def test_decode_at_the_combine_limit(lh):
    """Decode at the longest context the decode attention combines (1024 pages of 64 = 65,536 tokens): the
    step at position 65,535 gives the logits the prefill path gives at that position (within 1e-4 of the
    largest |logit|: the two paths sum in different orders; both are checked against the oracle at smaller
    sizes), and a step that would open a 1025th page is refused before any page is reserved."""
    img = lh.SynthImage("tiny-long", seed=7)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=2 * 65536 + 512, max_batch_tokens=65536)
    ids = np.random.default_rng(19).integers(0, eng.info["vocab"], 65536).astype(np.int32)
    a, b = eng.seq_create(), eng.seq_create()
    print("tiny-long: 65,535-token prefill, one decode step at position 65,535", flush=True)
    eng.forward(a, ids[:-1], [], OPTIONS)
    toks, logits = eng.decode(a, int(ids[-1]), 1, want_logits=True)
    want = eng.forward(b, ids, [65535])
    err = assert_logits_close(logits, want, rel=1e-4)
    assert_argmax_equal(logits, want, rel=1e-4)
    print(f"decode at 1024 pages against prefill: logits rel {err:.2e}", flush=True)
    assert eng.seq_len(a) == 65536
    with pytest.raises(lh.LayaError) as e:
        eng.decode(a, int(toks[0]), 1)
    assert e.value.kind == "INVALID" and "65536" in str(e.value)
    assert eng.seq_len(a) == 65536
    # the refused step reserved nothing: the pool's last 8 pages (2056 - 2 x 1024) still take 500 tokens
    assert eng.info["kv_pages"] == 2056
    c = eng.seq_create()
    eng.forward(c, ids[:500], [], OPTIONS)
    for q in (a, b, c):
        eng.seq_free(q)
    eng.close()

