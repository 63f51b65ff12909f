"""Full-depth GPU parity on the headline workloads, against the oracle at the same depth.

  Q8_0 batched prefill decide (24 layers, d2048, 16 x 128 heads, FFN 5632, vocab 32000): the
  benchmark's own batch of 64 requests x 560 tokens runs on the GPU; eight of its requests (3
  answer positions x 4 option tokens each) are recomputed by the oracle through all 24 layers,
  the first and last also by a float64 and a numpy f32 forward.
  Q8_0 batch-1 greedy decode (same model): the benchmark's 2048-token context, then 64 greedy
  steps; the oracle is fed the same tokens (teacher forcing) through its KV-cached decode and
  every step's full-vocabulary logits and argmax are compared.

  Q4_K/Q6_K 7B-shape prefill (28 layers, d3584, GQA 28/4, FFN 18944, vocab 152064, QKV bias): the
  benchmark's own batch of 32 x 1024 tokens on the GPU, three of its requests again alone (bit for
  bit), and one request through all 28 layers of the layer-streamed oracle (full-vocabulary logits).
  F16 7B-shape shared prefix (28 layers): a 1024-token prefix computed once and forked into two
  requests of 256 own tokens with 8 answer positions each, against the oracle's forked cache, and
  against the same request computed unshared (bit for bit).

Every workload runs in the exact mode (hi/lo KV planes) and in the kv16 mode (the same projections
over an f16 KV cache); the 7B workloads also in the fast mode, which misses a bar (strict xfail).
The oracle's answers are computed once per module and shared by the modes.

Bars: logits within 2e-2 of the largest |logit| per row, option probabilities within
1e-3 absolute, argmax equal.  For the decode's argmax, a step whose oracle top-2 gap is below twice
the oracle's own distance to a float64 forward of the same steps is a near-tie, and is decided
against the float64 argmax instead.  The measured errors are printed.

Reference path: Model::forward (src/models/openthai/model.rs:192-241), option scoring
(src/models/openthai/decision.rs:268-279), greedy argmax with the first maximum winning
(decision.rs:330-335).
"""
import time

import numpy as np
import pytest

from parity import LOGIT_REL, PREC_NAMES, PROB_ABS, logit_error

pytestmark = pytest.mark.gpu

SEED = 20261201  # the benchmark's model and workload seed
THREADS = 16


@pytest.fixture(scope="module")
def q8_full(lh, po):
    img = lh.SynthImage("q8-2048", seed=SEED)
    t0 = time.perf_counter()
    po.set_blocked(True)
    om = po.Model(po.Gguf(img.array()), threads=THREADS)
    print(f"\noracle q8-2048 L24 loaded in {time.perf_counter() - t0:.1f}s", flush=True)
    yield img, om, {}
    po.set_blocked(False)
    del om


def out_of_bar(mode, measured):
    """A mode with an f16 KV cache (kv16: the exact projections over it; fast: f16 operands as well) misses
    a parity bar at full depth of these synthetic models; a strict expected failure, so a mode that
    came within the bars would be noticed."""
    return pytest.mark.xfail(strict=True, reason=f"{mode} mode outside the parity bars at full depth ({measured}); "
                                                 "the exact mode is the measured one")


def _memo(memo, key, fn):
    """fn() once per key: the oracle's answers shared by the precision modes."""
    if key not in memo:
        memo[key] = fn()
    return memo[key]


def _near_tie_report(gpu, ref, window):
    """(argmax mismatches outside near-ties, [(row, gap)] near-ties) with an absolute window."""
    bad, ties = [], []
    for i, (g, r) in enumerate(zip(np.atleast_2d(gpu), np.atleast_2d(ref))):
        order = np.argsort(-r, kind="stable")
        gap = float(r[order[0]] - r[order[1]])
        if gap < window:
            ties.append((i, gap))
        elif int(np.argmax(g)) != int(order[0]):
            bad.append((i, gap, int(np.argmax(g)), int(order[0])))
    return bad, ties


@pytest.mark.parametrize("prec", [0, pytest.param(2, marks=out_of_bar(
    "kv16", "measured: logits 8.1e-2 of the largest, option probabilities 8.7e-2"))], ids=["exact", "kv16"])
def test_q8_prefill_decide_24_layers(lh, po, q8_full, tmp_path, prec):
    import bench
    import np_model

    img, om, memo = q8_full
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=64 * 640, max_batch_tokens=40000, precision=prec)
    reqs, option_ids = bench.prefill_workload(eng.info["vocab"])
    seqs = [eng.seq_create() for _ in reqs]
    print(f"GPU ({PREC_NAMES[prec]}): {len(reqs)} x {len(reqs[0][0])} tokens, 24 layers", flush=True)
    logits, probs, _ = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)]).run(option_ids)
    eng.close()
    npos = len(reqs[0][1])
    og = po.Gguf(img.array())

    def P(L):
        return np.stack([po.option_scores(np.float32(r))[0] for r in L])

    # eight requests across the batch against the oracle; the first and last also against float64
    # and a numpy f32 forward with its own operation order (the noise floor of two correct f32 orders)
    worst_l, worst_p = 0.0, 0.0
    for r in (9, 18, 27, 36, 45, 54):
        ids, pos = reqs[r]
        want = _memo(memo, ("c2", r), lambda: om.forward(ids, pos, option_ids))
        got_l = logits[r * npos:(r + 1) * npos]
        got_p = probs[r * npos:(r + 1) * npos]
        el, ep = logit_error(got_l, want), float(np.abs(got_p - P(want)).max())
        worst_l, worst_p = max(worst_l, el), max(worst_p, ep)
        print(f"request {r} gpu-oracle   : logits rel {el:.3e}, probs abs {ep:.3e}", flush=True)
        assert np.isfinite(got_l).all() and np.isfinite(got_p).all()
        assert el <= LOGIT_REL
        assert (np.argmax(got_l, axis=1) == np.argmax(want, axis=1)).all()
        assert ep <= PROB_ABS
    print(f"requests 9-54: worst logits rel {worst_l:.3e}, worst probs abs {worst_p:.3e}", flush=True)
    for r in (0, len(reqs) - 1):
        ids, pos = reqs[r]
        t0 = time.perf_counter()
        want = _memo(memo, ("c2", r), lambda: om.forward(ids, pos, option_ids))
        exact = _memo(memo, ("c2-f64", r), lambda: np_model.F64Model(og).logits(ids, pos, option_ids))
        other = _memo(memo, ("c2-npf32", r),
                      lambda: np_model.F64Model(og, dtype=np.float32).logits(ids, pos, option_ids))
        print(f"oracle, f64 and numpy-f32 forwards of request {r}: {time.perf_counter() - t0:.1f}s", flush=True)
        got_l = logits[r * npos:(r + 1) * npos]
        got_p = probs[r * npos:(r + 1) * npos]
        p_ref, p_ex, p_ot = P(want), P(exact), P(other)
        np.save(tmp_path / f"c2_{PREC_NAMES[prec]}_req{r}.npy", np.stack([got_l.astype(np.float64), want, exact, other]))
        for what, a, b, pa, pb in (("gpu-oracle", got_l, want, got_p, p_ref), ("gpu-f64", got_l, exact, got_p, p_ex),
                                   ("oracle-f64", want, exact, p_ref, p_ex), ("npf32-f64", other, exact, p_ot, p_ex),
                                   ("oracle-npf32", want, other, p_ref, p_ot)):
            print(f"request {r} {what:13s}: logits rel {logit_error(a, b):.3e}, probs abs "
                  f"{float(np.abs(pa - pb).max()):.3e}", flush=True)
        assert np.isfinite(got_l).all() and np.isfinite(got_p).all()
        assert logit_error(got_l, want) <= LOGIT_REL
        assert (np.argmax(got_l, axis=1) == np.argmax(want, axis=1)).all()
        assert float(np.abs(got_p - p_ref).max()) <= PROB_ABS


@pytest.mark.parametrize("prec", [0, pytest.param(2, marks=out_of_bar(
    "kv16", "measured: decode logits up to 9.2e-2 of the largest, and the greedy argmax differs from the oracle "
            "at 5 of 64 steps outside the near-tie window (top-2 gaps 0.10 to 0.83)"))], ids=["exact", "kv16"])
def test_q8_decode_24_layers_64_steps(lh, po, q8_full, prec):
    import bench
    import np_model

    img, om, memo = q8_full
    V = 32000
    rng = np.random.default_rng(SEED + 1)  # the benchmark's decode context
    ids = rng.integers(0, V, bench.DECODE_CTX).astype(np.int32)
    steps = bench.DECODE_STEPS
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=bench.DECODE_CTX + steps + 64, precision=prec)
    s = eng.seq_create()
    eng.forward(s, ids, [], [0])
    print(f"GPU ({PREC_NAMES[prec]}): {bench.DECODE_CTX}-token context, {steps} greedy steps, 24 layers", flush=True)
    toks, logits = eng.decode(s, int(ids[-1]), steps, want_logits=True)
    eng.close()
    # greedy: every emitted token is the first maximum of its step's logits
    assert np.isfinite(logits).all()
    assert (toks == np.argmax(logits, axis=1)).all()

    feed = [int(ids[-1])] + [int(t) for t in toks[:-1]]

    def oracle_steps():
        t0 = time.perf_counter()
        c = om.cache(bench.DECODE_CTX + steps + 8)
        om.prefill(c, ids, [])
        out = np.empty_like(logits)
        for i, t in enumerate(feed):
            out[i] = om.head(om.prefill(c, [t], [0]))[0]
        print(f"oracle prefill {bench.DECODE_CTX} and {steps} decode steps: {time.perf_counter() - t0:.1f}s", flush=True)
        return out

    want = _memo(memo, ("c3", tuple(feed)), oracle_steps)

    per_step = [logit_error(logits[i], want[i]) for i in range(steps)]
    abs_err = float(np.abs(logits - want).max())
    print(f"decode logits: worst rel {max(per_step):.3e} (step {int(np.argmax(per_step))}), worst abs "
          f"{abs_err:.3e}, median rel {float(np.median(per_step)):.3e}", flush=True)

    # The near-tie window comes from the oracle alone: the same 64 steps in float64 (one forward over the
    # context and the fed tokens), and twice the oracle's largest distance to them, the room two correct
    # f32 orders have on either side of the exact value.  A step outside the window must give the
    # oracle's argmax; a step inside it must give the float64 argmax.
    t0 = time.perf_counter()
    seq = np.concatenate([ids, np.asarray(feed, np.int32)])
    exact = _memo(memo, ("c3-f64", tuple(feed)), lambda: np_model.F64Model(po.Gguf(img.array())).logits(
        seq, np.arange(bench.DECODE_CTX, bench.DECODE_CTX + steps)))
    print(f"float64 forward over {len(seq)} tokens: {time.perf_counter() - t0:.1f}s", flush=True)
    oracle_spread = float(np.abs(want - exact).max())
    gpu_f64 = float(np.abs(logits - exact).max())
    window = 2.0 * oracle_spread
    print(f"largest |oracle - f64| {oracle_spread:.3e}, |gpu - f64| {gpu_f64:.3e}; near-tie window {window:.3e}",
          flush=True)
    bad, ties = _near_tie_report(logits, want, window)
    flips = []
    for i, gap in ties:
        g, o, x = int(np.argmax(logits[i])), int(np.argmax(want[i])), int(np.argmax(exact[i]))
        top = np.sort(exact[i])
        print(f"  near-tie at step {i}: oracle gap {gap:.3e}, f64 gap {top[-1] - top[-2]:.3e}; argmax gpu {g}, "
              f"oracle {o}, f64 {x}", flush=True)
        if g != x:
            flips.append((i, g, x))
    gaps = [float(np.sort(w)[-1] - np.sort(w)[-2]) for w in want]
    print(f"argmax: {steps - len(ties)} steps asserted against the oracle, {len(ties)} near-ties decided in "
          f"float64, GPU != f64 at {flips}; smallest oracle gap {min(gaps):.3e}", flush=True)
    print(f"argmax mismatches outside near-ties (step, gap, gpu, oracle): {bad}", flush=True)
    assert max(per_step) <= LOGIT_REL
    assert not bad, f"argmax mismatches outside near-ties (step, gap, gpu, oracle): {bad}"
    assert not flips, f"near-tie steps where the GPU's argmax is not the float64 one (step, gpu, f64): {flips}"


def _argmax_ok(gpu, ref, window):
    """Row-wise argmax equal wherever the reference's top-2 gap is at least `window`; returns the
    smallest gap seen."""
    gaps = []
    for g, r in zip(np.atleast_2d(gpu), np.atleast_2d(ref)):
        top = np.sort(r)
        gaps.append(float(top[-1] - top[-2]))
        if gaps[-1] >= window:
            assert int(np.argmax(g)) == int(np.argmax(r)), f"argmax {int(np.argmax(g))} != {int(np.argmax(r))}"
    return min(gaps)


@pytest.fixture(scope="module")
def q4k_full(lh, po):
    """The C4 model and workload, and the layer-streamed oracle's answer for request 0 (full vocabulary at
    its scored position)."""
    import bench

    img = lh.SynthImage("q4km-7b", seed=SEED)
    reqs, opts = bench.q4k_workload()
    t0 = time.perf_counter()
    po.set_blocked(True)
    om = po.Model(po.Gguf(img.array()), threads=THREADS, streamed=True)
    ids, pos = reqs[0]
    full = om.forward(ids, pos)
    po.set_blocked(False)
    print(f"\noracle q4km-7b L28, request 0 ({len(ids)} tokens): {time.perf_counter() - t0:.1f}s", flush=True)
    del om
    yield img, reqs, opts, full




@pytest.mark.parametrize("prec", [0, pytest.param(2, marks=out_of_bar(
    "kv16", "measured: logits 4.1e-2 of the largest, option probabilities 1.6e-2")), pytest.param(1, marks=out_of_bar(
    "fast", "measured: logits 7.3e-2 of the largest, option probabilities 5.7e-2"))], ids=["exact", "kv16", "fast"])
def test_q4km_7b_prefill_28_layers(lh, po, q4k_full, prec):
    img, reqs, opts, want_full = q4k_full
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=len(reqs) * 1024 + 2048, max_batch_tokens=32768,
                    precision=prec)
    seqs = [eng.seq_create() for _ in reqs]
    print(f"GPU ({PREC_NAMES[prec]}): {len(reqs)} x {len(reqs[0][0])} tokens, 28 layers", flush=True)
    logits, probs, _ = eng.batch([(s, ids, pos) for s, (ids, pos) in zip(seqs, reqs)]).run(opts)
    for s in seqs:
        eng.seq_free(s)
    assert np.isfinite(logits).all() and np.isfinite(probs).all()
    for r in (0, 13, 31):  # the wide 256 x 256 launches of the batch == a request alone
        s = eng.seq_create()
        single = eng.forward(s, reqs[r][0], reqs[r][1], opts)
        eng.seq_free(s)
        assert np.array_equal(single.view(np.uint32), logits[r:r + 1].view(np.uint32)), f"request {r}: batch != alone"
    s = eng.seq_create()
    full = eng.forward(s, reqs[0][0], reqs[0][1])  # full vocabulary (the head GEMV)
    eng.close()
    want_opts = want_full[:, opts]
    p_ref = np.stack([po.option_scores(w)[0] for w in want_opts])
    err_full, err_opt = logit_error(full, want_full), logit_error(logits[:1], want_opts)
    perr = float(np.abs(probs[:1] - p_ref).max())
    gap = _argmax_ok(full, want_full, 0.0)
    print(f"q4km-7b L28 {PREC_NAMES[prec]}: full-vocab logits rel {err_full:.3e}, option logits rel "
          f"{err_opt:.3e}, option probs abs {perr:.3e}, argmax {int(np.argmax(full))} (oracle "
          f"{int(np.argmax(want_full))}, oracle top-2 gap {gap:.3e})", flush=True)
    assert err_full <= LOGIT_REL and err_opt <= LOGIT_REL
    assert perr <= PROB_ABS
    assert int(np.argmax(full)) == int(np.argmax(want_full))


C5_SMALL_PREFIX, C5_SMALL_OWN, C5_SMALL_REQS = 1024, 256, 2


@pytest.fixture(scope="module")
def f16_full(lh, po):
    """The C5 model, a shortened C5 workload (the bench's own prefix and suffixes cut to 1024 + 2 x 256
    tokens, 8 answer positions per suffix) and the layer-streamed oracle's answers: the prefix prefilled
    once, its cache forked per request."""
    import bench

    img = lh.SynthImage("f16-7b", seed=SEED)
    prefix, own, _, opts = bench.c5_workload()
    prefix = prefix[:C5_SMALL_PREFIX]
    own = [o[:C5_SMALL_OWN] for o in own[:C5_SMALL_REQS]]
    pos = np.arange(C5_SMALL_OWN // 8 - 1, C5_SMALL_OWN, C5_SMALL_OWN // 8).astype(np.int32)
    t0 = time.perf_counter()
    po.set_blocked(True)
    om = po.Model(po.Gguf(img.array()), threads=THREADS, streamed=True)
    c = om.cache(C5_SMALL_PREFIX + C5_SMALL_OWN + 8)
    om.prefill(c, prefix, [])
    want, full = [], None
    for r, ids in enumerate(own):
        hid = om.prefill(c.fork(C5_SMALL_PREFIX), ids, pos)
        want.append(om.head(hid, opts))
        if r == 0:
            full = om.head(hid[-1:])
    po.set_blocked(False)
    print(f"\noracle f16-7b L28, {C5_SMALL_PREFIX}-token prefix + {C5_SMALL_REQS} x {C5_SMALL_OWN}: "
          f"{time.perf_counter() - t0:.1f}s", flush=True)
    del om
    yield img, prefix, own, pos, opts, np.concatenate(want), full


@pytest.mark.parametrize("prec", [0, pytest.param(2, marks=out_of_bar(
    "kv16", "measured: logits 3.9e-3 of the largest, within 2e-2, but option probabilities 1.3e-3 against 1e-3")),
    pytest.param(1, marks=out_of_bar(
        "fast", "measured: logits 9.8e-3 of the largest, within 2e-2, but option probabilities 2.8e-3 against 1e-3"))],
    ids=["exact", "kv16", "fast"])
def test_f16_7b_shared_prefix_28_layers(lh, po, f16_full, prec):
    img, prefix, own, pos, opts, want, want_full = f16_full
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=8192, max_batch_tokens=8192, precision=prec)
    print(f"GPU ({PREC_NAMES[prec]}): {len(prefix)}-token prefix forked into {len(own)} x "
          f"{len(own[0])}, 28 layers", flush=True)
    base = eng.seq_create()
    eng.forward(base, prefix, [], opts)
    kids = [eng.seq_fork(base, len(prefix)) for _ in own]
    logits, probs, _ = eng.batch([(k, ids, pos) for k, ids in zip(kids, own)]).run(opts)
    k0 = eng.seq_fork(base, len(prefix))
    full = eng.forward(k0, own[0], pos[-1:])
    fresh = eng.seq_create()
    unshared = eng.forward(fresh, np.concatenate([prefix, own[0]]), len(prefix) + pos, opts)
    eng.close()
    assert np.isfinite(logits).all() and np.isfinite(probs).all()
    assert np.array_equal(unshared.view(np.uint32), logits[:len(pos)].view(np.uint32)), "fork != unshared"
    p_ref = np.stack([po.option_scores(w)[0] for w in want])
    err, err_full = logit_error(logits, want), logit_error(full, want_full)
    perr = float(np.abs(probs - p_ref).max())
    gap = _argmax_ok(logits, want, 0.0)
    print(f"f16-7b L28 {PREC_NAMES[prec]}: option logits rel {err:.3e}, probs abs {perr:.3e}, "
          f"full-vocab logits rel {err_full:.3e}, argmax {int(np.argmax(full))} (oracle {int(np.argmax(want_full))}); "
          f"smallest option top-2 gap {gap:.3e}", flush=True)
    assert err <= LOGIT_REL and err_full <= LOGIT_REL
    assert perr <= PROB_ABS
    assert int(np.argmax(full)) == int(np.argmax(want_full))
