"""Pinning the CPU oracle: the reference's own known-answer tests, closed forms, independent
numpy restatements (tests/np_ref.py) and brute force.  CPU only.

Reference KATs used here:
  src/tensor.rs:196-214   Matrix::apply, 11x17 weights, 9x17 input, bias 0.25, 1/2/4 threads
  src/tensor.rs:215-217   half(0x3c00) = 1, half(1) = 2^-24
  src/models/laya/decision.rs:331-333   confidence([.5,.5]) = 0, confidence([1,0]) >= 0.9999
"""
import numpy as np
import pytest

import np_ref

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
KINDS = [F32, F16, Q4_0, Q8_0, Q4_K, Q6_K]


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_same_floats(got, want):
    """Bit-identical, except that any NaN matches any NaN (payloads are not part of the
    reference's contract once arithmetic has produced them)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"NaN positions differ at {np.flatnonzero(gn != wn)[:8]}"
    bad = np.flatnonzero((bits(got) != bits(want)) & ~gn)
    assert bad.size == 0, f"{bad.size} values differ, first at {bad[:8]}: {got[bad[:4]]} vs {want[bad[:4]]}"


# ------------------------------------------------------------------ half / layout

def test_half_kat(po, lh):
    for half in (po.half, lh.half):
        assert abs(half(0x3C00) - 1.0) <= 1e-8
        assert half(0x0001) == 1.0 / 16777216.0


def test_half_exhaustive_vs_numpy(po, lh):
    codes = np.arange(65536, dtype=np.uint16)
    want = np_ref.half(codes)
    got = po.decode(F16, codes.tobytes())
    # IEEE conversion is exact, NaN payloads included (src/gguf.rs:241-242)
    assert np.array_equal(bits(got), bits(want))
    # lg_half returns a C float, which ctypes widens to a Python float: that widening quiets
    # signalling NaNs, so NaN codes are compared as NaN, everything else bit for bit
    got_lh = np.array([lh.half(int(c)) for c in codes], np.float32)
    nan = np.isnan(want)
    assert np.isnan(got_lh[nan]).all()
    assert np.array_equal(bits(got_lh[~nan]), bits(want[~nan]))


def test_layout_table(po, lh):
    want = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
    for k, v in want.items():
        assert po.layout(k) == v == lh.layout(k)
    for k in (3, 6, 7, 9, 10, 11, 13, 15, 16, 30):
        with pytest.raises(ValueError):
            po.layout(k)
        with pytest.raises(lh.LayaError, match=f"unsupported GGML tensor type {k}; supported "
                                               "F32/F16/Q4_0/Q8_0/Q4_K/Q6_K"):
            lh.layout(k)


# ------------------------------------------------------------------ dequantisation

def _random_blocks(kind, nblocks, rng):
    _, size = np_ref.LAYOUT[kind]
    raw = rng.integers(0, 256, nblocks * size, dtype=np.uint8)
    if kind in (Q8_0, Q4_0, Q4_K, Q6_K):
        # keep scales finite and moderate so values are ordinary numbers; special scales are KATs
        r = raw.reshape(nblocks, size)
        scale_off = {Q8_0: [0], Q4_0: [0], Q4_K: [0, 2], Q6_K: [208]}[kind]
        for o in scale_off:
            h = rng.normal(0, 1e-2, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
            r[:, o:o + 2] = h
    if kind == F32:
        raw = rng.normal(0, 1, nblocks).astype(np.float32).view(np.uint8)
    return raw


@pytest.mark.parametrize("kind", KINDS, ids=lambda k: {0: "F32", 1: "F16", 2: "Q4_0", 8: "Q8_0", 12: "Q4_K",
                                                        14: "Q6_K"}[k])
def test_decode_matches_numpy_restatement(po, kind):
    rng = np.random.default_rng(100 + kind)
    raw = _random_blocks(kind, 64 if kind in (Q4_K, Q6_K) else 512, rng)
    assert_same_floats(po.decode(kind, raw.tobytes()), np_ref.decode(kind, raw))


@pytest.mark.parametrize("kind", [Q8_0, Q4_0, Q4_K, Q6_K], ids=["Q8_0", "Q4_0", "Q4_K", "Q6_K"])
def test_decode_random_bytes_any_scale(po, kind):
    """Fully random bytes: scales include subnormals, Inf and NaN."""
    rng = np.random.default_rng(7 + kind)
    _, size = np_ref.LAYOUT[kind]
    raw = rng.integers(0, 256, 40 * size, dtype=np.uint8)
    assert_same_floats(po.decode(kind, raw.tobytes()), np_ref.decode(kind, raw))


def _h(x):
    return np.array([x], np.float16).view(np.uint16)[0]


def test_q8_0_kat(po):
    codes = np.arange(-128, 128, dtype=np.int64).reshape(8, 32)
    f = np.float32

    def block(dbits, c):
        return np.array([dbits], "<u2").tobytes() + c.astype(np.int8).tobytes()

    # d = 1: values are the codes; d = 2^-24 (smallest subnormal): codes * 2^-24, exact
    raw = b"".join(block(0x3C00, c) for c in codes)
    assert np.array_equal(po.decode(Q8_0, raw), codes.reshape(-1).astype(f))
    raw = b"".join(block(0x0001, c) for c in codes)
    assert np.array_equal(po.decode(Q8_0, raw), (codes.reshape(-1) * 2.0 ** -24).astype(f))
    # d = -0: -0 * positive = -0, -0 * negative = +0, -0 * 0 = -0
    got = po.decode(Q8_0, block(0x8000, codes[4]))
    want = np.where(codes[4] < 0, f(0.0), f(-0.0)).astype(f)
    assert np.array_equal(bits(got), bits(want))
    # d = +Inf: sign of the code, and Inf * 0 = NaN
    got = po.decode(Q8_0, block(0x7C00, codes[4]))
    assert np.isnan(got[codes[4] == 0]).all()
    nz = codes[4] != 0
    assert np.array_equal(got[nz], np.where(codes[4][nz] > 0, np.inf, -np.inf).astype(f))
    # d = NaN: every output is NaN
    assert np.isnan(po.decode(Q8_0, block(0x7E00, codes[0]))).all()


def test_q4_0_kat(po):
    nib = np.arange(32) % 16
    q = (nib[:16] | (nib[16:][::-1] << 4)).astype(np.uint8)
    raw = np.array([0x3C00], "<u2").tobytes() + q.tobytes()
    got = po.decode(Q4_0, raw)
    want = np.concatenate([(q & 15).astype(np.float32) - 8, (q >> 4).astype(np.float32) - 8])
    assert np.array_equal(got, want)


def _pack_q4k_scales(s, m):
    """Inverse of the 6-bit scale/min unpack of src/gguf.rs:287-296."""
    sc = np.zeros(12, np.uint8)
    for j in range(4):
        sc[j] = (s[j] & 63) | ((s[j + 4] >> 4) << 6)
        sc[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        sc[j + 8] = (s[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return sc


def test_q4_k_kat_both_unpack_branches(po):
    # scales/mins chosen so sub-blocks 0-3 (direct 6 bits) and 4-7 (split nibble + 2 high bits)
    # each use values with the high bits set
    s = np.array([1, 63, 32, 17, 63, 48, 5, 33])
    m = np.array([0, 62, 31, 16, 60, 47, 63, 40])
    rng = np.random.default_rng(3)
    nibbles = rng.integers(0, 16, 256)
    qs = np.zeros(128, np.uint8)
    for g in range(4):
        qs[g * 32:(g + 1) * 32] = nibbles[g * 64:g * 64 + 32] | (nibbles[g * 64 + 32:g * 64 + 64] << 4)
    for d, dm in ((1.0, 1.0), (0.5, 0.25), (2.0 ** -24, 2.0 ** -14)):
        raw = np.array([_h(d), _h(dm)], "<u2").tobytes() + _pack_q4k_scales(s, m).tobytes() + qs.tobytes()
        got = po.decode(Q4_K, raw)
        sub = np.arange(256) // 32
        want = ((np.float32(d) * s[sub].astype(np.float32)) * nibbles.astype(np.float32)
                - np.float32(dm) * m[sub].astype(np.float32))
        assert np.array_equal(bits(got), bits(want.astype(np.float32)))


def _pack_q6k(codes):
    """Inverse of the ql/qh bit layout of src/gguf.rs:315-324: codes[256] in 0..63."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for n in range(2):
        for l in range(32):
            q = [codes[n * 128 + j * 32 + l] for j in range(4)]
            lo = n * 64 + l
            ql[lo] = (q[0] & 15) | ((q[2] & 15) << 4)
            ql[lo + 32] = (q[1] & 15) | ((q[3] & 15) << 4)
            qh[n * 32 + l] = (q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6)
    return ql, qh


def test_q6_k_kat_every_bit_slice(po):
    rng = np.random.default_rng(11)
    codes = rng.integers(0, 64, 256)
    codes[:4] = [0, 63, 32, 31]
    sc = np.array([-128, -1, 0, 1, 127, 64, -64, 3, 2, -2, 100, -100, 7, -7, 50, 9], np.int8)
    ql, qh = _pack_q6k(codes)
    for d in (1.0, 2.0 ** -24, 0.125):
        raw = ql.tobytes() + qh.tobytes() + sc.tobytes() + np.array([_h(d)], "<u2").tobytes()
        got = po.decode(Q6_K, raw)
        si = (np.arange(256) // 128) * 8 + (np.arange(256) % 32) // 16 + 2 * ((np.arange(256) % 128) // 32)
        want = (np.float32(d) * sc[si].astype(np.float32)) * (codes.astype(np.float32) - 32)
        assert np.array_equal(bits(got), bits(want.astype(np.float32)))


# ------------------------------------------------------------------ Matrix::apply

def _kat_inputs():
    w = ((np.arange(187, dtype=np.float32) - 83.0) / 71.0).astype(np.float32).reshape(11, 17)
    x = ((np.arange(153, dtype=np.float32) - 71.0) / 43.0).astype(np.float32).reshape(9, 17)
    return w, x, np.full(11, 0.25, np.float32)


def test_apply_reference_kat(po):
    """src/tensor.rs:196-214 verbatim: |apply - (dot + 0.25)| <= 1e-4 at 1, 2 and 4 threads."""
    w, x, b = _kat_inputs()
    for threads in (1, 2, 4):
        y = po.apply(w, x, b, threads)
        for r in range(9):
            for c in range(11):
                want = po.dot(x[r], w[c]) + np.float32(0.25)
                assert abs(y[r, c] - want) <= 1e-4


def test_apply_operation_order(po):
    """Bit-exact against the numpy restatement of the 8-lane FMA order (tail, bias included),
    across thread counts and both the AVX2 and scalar code paths of the oracle."""
    w, x, b = _kat_inputs()
    want = np_ref.kernel(w, x, b)
    outs = []
    for scalar in (False, True):
        po.set_scalar_apply(scalar)
        try:
            for threads in (1, 2, 4, 8):
                outs.append(po.apply(w, x, b, threads))
        finally:
            po.set_scalar_apply(False)
    for y in outs:
        assert np.array_equal(bits(y), bits(want))
    # an 8-lane change (plain sequential dot) would not be bit-exact on these inputs
    seq = np.array([[np.float32(sum(np.float32(a) * np.float32(c) for a, c in zip(xr, wr))) for wr in w]
                    for xr in x], np.float32) + np.float32(0.25)
    assert not np.array_equal(bits(seq), bits(want))


@pytest.mark.parametrize("m,rows,K", [(1, 3, 5), (5, 7, 8), (4, 9, 16), (13, 6, 37), (3, 33, 64)])
def test_apply_shapes(po, m, rows, K):
    rng = np.random.default_rng(m * 100 + K)
    w = rng.normal(0, 1, (rows, K)).astype(np.float32)
    x = rng.normal(0, 1, (m, K)).astype(np.float32)
    b = rng.normal(0, 1, rows).astype(np.float32)
    assert np.array_equal(bits(po.apply(w, x, b, 3)), bits(np_ref.kernel(w, x, b)))
    assert np.array_equal(bits(po.apply(w, x, None, 2)), bits(np_ref.kernel(w, x, None)))
    ref64 = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.abs(po.apply(w, x, b) - ref64).max() <= 1e-5 * max(1.0, np.abs(ref64).max()) * np.sqrt(K)


@pytest.mark.parametrize("m,rows,K", [(1, 3, 5), (1, 1100, 37), (2, 2048, 64), (5, 7, 8), (7, 130, 2048),
                                      (13, 601, 99), (64, 96, 5632)])
def test_apply_blocked_mode_same_bits(po, m, rows, K):
    """The cache-blocked loop nest (column blocks, two columns per pass, column split for few rows)
    gives the bits of the numpy restatement of the reference order, tails and bias included."""
    rng = np.random.default_rng(m * 7 + rows + K)
    w = rng.normal(0, 1, (rows, K)).astype(np.float32)
    x = rng.normal(0, 1, (m, K)).astype(np.float32)
    b = rng.normal(0, 1, rows).astype(np.float32)
    want = np_ref.kernel(w, x, b)
    po.set_blocked(True)
    try:
        for threads in (1, 3, 8):
            assert np.array_equal(bits(po.apply(w, x, b, threads)), bits(want))
    finally:
        po.set_blocked(False)


def test_forward_blocked_mode_same_bits(lh, po):
    """A whole forward (GQA attention over a cache, continuation by one token) in the blocked mode
    equals the reference loop order bit for bit."""
    img = lh.SynthImage("tiny-q4k", seed=3)
    om = po.Model(po.Gguf(img.array()), threads=4)
    ids = np.random.default_rng(4).integers(0, om.V, 70).astype(np.int32)
    outs = []
    for blocked in (False, True):
        po.set_blocked(blocked)
        try:
            c = om.cache(128)
            h1 = om.prefill(c, ids[:-1], [68, 3, 40])
            h2 = om.prefill(c, ids[-1:], [0])
            outs.append((om.head(h1), om.head(h2)))
        finally:
            po.set_blocked(False)
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(bits(a), bits(b))


# ------------------------------------------------------------------ elementwise rules

def test_dot_is_sequential(po):
    rng = np.random.default_rng(5)
    a, b = rng.normal(0, 1, (2, 101)).astype(np.float32)
    s = np.float32(0.0)
    for u, v in zip(a, b):
        s = np.float32(s + np.float32(u * v))
    assert bits(po.dot(a, b)) == bits(s)


def test_softmax(po):
    rng = np.random.default_rng(6)
    x = rng.normal(0, 3, 50).astype(np.float32)
    p = po.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.abs(p - e / e.sum()).max() < 1e-6
    assert abs(float(p.astype(np.float64).sum()) - 1) < 1e-5
    assert np.array_equal(po.softmax(x + np.float32(0.0)), p)
    # masked (-inf) entries get exactly zero
    xm = x.copy()
    xm[::3] = -np.inf
    pm = po.softmax(xm)
    assert (pm[::3] == 0).all() and abs(float(pm.sum()) - 1) < 1e-5


def test_rms_and_silu(po):
    rng = np.random.default_rng(8)
    x = rng.normal(0, 2, (3, 64)).astype(np.float32)
    w = rng.normal(1, 0.1, 64).astype(np.float32)
    for eps, off in ((1e-5, 0.0), (1e-6, 1.0)):
        y = po.rms(x, w, off, eps)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * (off + w)
        assert np.abs(y - want).max() < 1e-5
    for v in (-20.0, -1.5, 0.0, 0.3, 4.0, 30.0):
        assert abs(po.silu(v) - v / (1 + np.exp(-v))) <= 1e-6 * max(1, abs(v))


# ------------------------------------------------------------------ option scoring

def test_option_scores_closed_form(po, lh):
    rng = np.random.default_rng(9)
    for k in (2, 4, 7):
        z = rng.normal(0, 4, k).astype(np.float32)
        for T in (1.0, 0.7, 2.5):
            p, lp, ab = po.option_scores(z, T)
            zz = z.astype(np.float64) / T
            ref = np.exp(zz - zz.max())
            ref /= ref.sum()
            assert np.abs(p - ref).max() < 1e-6 and abs(p.sum() - 1) < 1e-6 and ab == 0
            assert np.abs(lp - np.log(ref)).max() < 1e-5
            p2, lp2 = lh.option_scores(z, T)
            assert np.abs(p2 - p).max() < 1e-6 and np.abs(lp2 - lp).max() < 1e-5
    # abstain slot: softmax over k + 1, the k option probabilities renormalised
    z = np.array([1.0, 2.0, 0.5], np.float32)
    p, _, ab = po.option_scores(z, 1.0, abstain=3.0)
    full = np.exp(np.array([1.0, 2.0, 0.5, 3.0]) - 3.0)
    full /= full.sum()
    assert np.abs(p - full[:3] / full[:3].sum()).max() < 1e-6 and abs(ab - full[3]) < 1e-6


def test_argmax_first_max_wins(po):
    assert po.argmax(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert po.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert po.argmax(np.array([0.0, np.nan, 1.0], np.float32)) == 2


def test_confidence_kat(po, lh):
    """src/models/laya/decision.rs:331-333, for both entropy precisions and both libraries."""
    for f64 in (False, True):
        assert abs(po.confidence([0.5, 0.5], f64)) <= 1e-6
        assert po.confidence([1.0, 0.0], f64) >= 0.9999
        assert po.confidence([1.0], f64) == 1.0
        mode = lh.CONF_F64 if f64 else lh.CONF_F32
        assert abs(lh.option_confidence([0.5, 0.5], mode)) <= 1e-6
        assert lh.option_confidence([1.0, 0.0], mode) >= 0.9999
        assert lh.option_confidence([0.3], mode) == 1.0


def test_confidence_closed_form(po, lh):
    rng = np.random.default_rng(12)
    for k in (2, 3, 4, 8):
        for _ in range(20):
            p = rng.dirichlet(np.ones(k)).astype(np.float32)
            q = np.maximum(p.astype(np.float64), 1e-12)
            want = float(np.clip(1 + (q * np.log(q)).sum() / np.log(k), 0, 1))
            for f64, mode in ((False, lh.CONF_F32), (True, lh.CONF_F64)):
                c = po.confidence(p, f64)
                assert abs(c - want) < 1e-5
                assert np.float32(lh.option_confidence(p, mode)) == np.float32(c)
    # an all-zero vector floors every entry at 1e-12: entropy ~ k*1e-12*27.6 -> confidence 1
    assert po.confidence([0.0, 0.0, 0.0]) == lh.option_confidence([0.0, 0.0, 0.0]) == 1.0


@pytest.mark.parametrize("hq,hkv,hd,pos0,n", [(4, 2, 16, 7, 5), (28, 4, 128, 60, 9), (8, 8, 64, 0, 33)])
def test_attention_against_float64(po, hq, hkv, hd, pos0, n):
    """or_attention (src/models/openthai/model.rs:276-294): causal, head h reads kv head h // (hq/hkv),
    scores / sqrt(hd); float64 textbook within f32 rounding; a kv-head map of h % hkv would not match;
    the blocked mode gives the same bits."""
    rng = np.random.default_rng(hq + hd + n)
    q = rng.standard_normal((n, hq * hd)).astype(np.float32)
    k = rng.standard_normal((pos0 + n, hkv * hd)).astype(np.float32)
    v = rng.standard_normal((pos0 + n, hkv * hd)).astype(np.float32)
    got = po.attention(q, k, v, pos0, hq, hkv, threads=3)

    def ref(kv_head):
        out = np.zeros((n, hq * hd))
        for i in range(n):
            for h in range(hq):
                kh = kv_head(h)
                s = k[:pos0 + i + 1, kh * hd:(kh + 1) * hd].astype(np.float64) @ q[i, h * hd:(h + 1) * hd] / np.sqrt(hd)
                p = np.exp(s - s.max())
                out[i, h * hd:(h + 1) * hd] = (p / p.sum()) @ v[:pos0 + i + 1, kh * hd:(kh + 1) * hd]
        return out
    assert np.abs(got - ref(lambda h: h // (hq // hkv))).max() < 1e-5
    if hkv != hq and hkv > 1:
        assert np.abs(got - ref(lambda h: h % hkv)).max() > 1e-2
    po.set_blocked(True)
    try:
        assert np.array_equal(bits(po.attention(q, k, v, pos0, hq, hkv, threads=2)), bits(got))
    finally:
        po.set_blocked(False)
