"""GPU parity of the kernels through the C ABI: bit-exact dequant, GEMV/GEMM vs Matrix::apply.

Reference: src/gguf.rs:250-336 (decode), src/tensor.rs:10-102 (Matrix::apply), restated by
the CPU oracle.  Bars: see tests/parity.py.
"""
import numpy as np
import pytest

from parity import assert_argmax_equal, assert_bits_equal, assert_logits_close

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20261201)


def _blocks(kind, n, lh):
    block, size = lh.layout(kind)
    raw = RNG.integers(0, 256, size=n * size, dtype=np.uint8)
    return raw


def _edge_q8():
    out = []
    for d in (0x3C00, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E01, 0x8000, 0x0000):
        codes = np.arange(-128, 128, 8, dtype=np.int8)  # 32 codes incl. -128 and 120
        out.append(np.frombuffer(np.uint16(d).tobytes() + codes.tobytes(), dtype=np.uint8))
    return np.concatenate(out)


@pytest.mark.parametrize("kind", [0, 1, 2, 8, 12, 14])
def test_dequant_bit_exact(lh, po, kind):
    print(f"dequant kind={kind}", flush=True)
    raw = _blocks(kind, 4096 if kind not in (12, 14) else 512, lh)
    if kind == 8:
        raw = np.concatenate([raw, _edge_q8()])
    got = lh.dequant(kind, raw)
    want = po.decode(kind, raw)
    assert_bits_equal(got, want)


def test_dequant_f16_exhaustive(lh, po):
    codes = np.arange(65536, dtype=np.uint16)
    got = lh.dequant(1, codes.view(np.uint8))
    assert_bits_equal(got, po.decode(1, codes.view(np.uint8)))


@pytest.fixture(scope="module", params=[("tiny-f16", 0), ("tiny-q8", 0), ("tiny-q4k", 0), ("tiny-f16", 1),
                                        ("tiny-q8", 1)],
                ids=lambda p: f"{p[0]}-{'exact' if p[1] == 0 else 'fast'}")
def model(request, lh, po):
    preset, prec = request.param
    img = lh.SynthImage(preset, seed=11)
    g = lh.Gguf.from_bytes(img)
    eng = lh.Engine(g, kv_tokens=4096, precision=prec)
    og = po.Gguf(img.array())
    yield f"{preset}-{'exact' if prec == 0 else 'fast'}", img, eng, og
    eng.close()


def _matrices(og):
    names = []
    for base in ("qkv.0.weight", "q.0.weight", "k.0.weight", "v.0.weight", "wo.0.weight", "mlp_wi.0.weight",
                 "mlp_wo.1.weight", "output.weight"):
        try:
            og.tensor(base)
            names.append(base)
        except KeyError:
            pass
    return names


@pytest.mark.parametrize("m", [1, 5, 64, 130, 300])
def test_matmul_vs_apply(model, po, m):
    preset, img, eng, og = model
    for name in _matrices(og):
        kind, dims, raw = og.tensor(name)
        cols, rows = dims
        w = po.decode(kind, raw).reshape(rows, cols)
        x = RNG.standard_normal((m, cols)).astype(np.float32)
        bias = RNG.standard_normal(rows).astype(np.float32) if m % 2 else None
        print(f"{preset} {name} m={m}", flush=True)
        got = eng.matmul(name, x, bias)
        want = po.apply(w, x, bias, threads=4)
        # m == 1 runs the f32 GEMV in both modes.  m > 1 runs the MFMA GEMM: in the exact mode on
        # hi/lo f16 planes of x with the weights applied exactly (about 2^-22 per product, so
        # 1e-5 of the largest output; a GEMM that dropped the lo plane errs by ~1e-3), in the
        # fast mode on f16 x and f16-rounded weights (within 1e-2, and measurably above 1e-5:
        # the exact-mode bar tells the two apart).
        if m == 1 or preset.endswith("exact"):
            assert_logits_close(got, want, rel=1e-5)
        else:
            err = assert_logits_close(got, want, rel=1e-2)
            assert err > 1e-5, f"fast-mode error {err:.2e} is inside the exact-mode bar"


def test_probe_read_launch_floor(lh):
    """lg_probe_read (the launch-floor probe): a plain read chain gives a positive time per launch that
    grows with the bytes read, and bad arguments are refused without launching."""
    small = lh.probe_read(16, 50)
    big = lh.probe_read(64 << 20, 50)
    print(f"probe: 16 B {small:.2f} us, 64 MiB {big:.2f} us per launch", flush=True)
    assert 0.0 < small < big
    with pytest.raises(lh.LayaError):
        lh.probe_read(8, 10)
    with pytest.raises(lh.LayaError):
        lh.probe_read(1024, 0)


def _uncentred_q4k(nblocks, rng):
    """Q4_K blocks drawn as the letter of the config reads (d and dmin f16(|N(0, 1e-3)|) drawn
    independently, every 6-bit scale and min any value, nibbles uniform): the block minimum does not
    cancel the nibble mean, so the two terms of the two-pass form, A (x . q) and B sum(x), are large
    against their difference."""
    out = np.empty((nblocks, 144), np.uint8)
    out[:, 0:2] = np.abs(rng.normal(0, 1e-3, nblocks)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = np.abs(rng.normal(0, 1e-3, nblocks)).astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 4:] = rng.integers(0, 256, (nblocks, 140), dtype=np.uint8)
    return out


@pytest.mark.parametrize("mean", [0.0, 2.0], ids=["x-zero-mean", "x-mean-2"])
def test_q4k_two_pass_on_uncentred_blocks(lh, po, mean):
    """The exact Q4_K GEMM (two passes over the codes plus the depth-K/32 correction) and the Q4_K GEMV
    (A sum(x q) - B sum(x) per half sub-block) against Matrix::apply on Q4_K matrices whose blocks are not
    zero-centred, with activations of zero and of large mean (the correction's chunk sums then dominate):
    the GEMV (1 row), the 128 x 128 tiles (130 and 300 rows) and the 256 x 256 kernel (16,384 rows), each
    within the exact mode's 1e-5 of the largest output."""
    rng = np.random.default_rng(31)
    img = lh.SynthImage("tiny-q4k", seed=12)
    buf = img.array().copy()
    og0 = po.Gguf(buf)
    names = [n for n in _matrices(og0) if og0.tensor(n)[0] == 12]
    assert names, "the preset holds Q4_K matrices"
    for n in names:
        _, _, raw = og0.tensor(n)
        off = og0.offset(n)
        buf[off:off + len(raw)] = _uncentred_q4k(len(raw) // 144, rng).ravel()
    og = po.Gguf(buf)
    eng = lh.Engine(lh.Gguf.from_bytes(buf), kv_tokens=1024, max_batch_tokens=16384)
    for n in names:
        kind, dims, raw = og.tensor(n)
        cols, rows = dims
        w = po.decode(kind, raw).reshape(rows, cols)
        for m in (1, 130, 300, 16384):
            x = (mean + rng.standard_normal((m, cols))).astype(np.float32)
            print(f"{n} ({rows} x {cols}) m={m} x mean {mean}", flush=True)
            got = eng.matmul(n, x)
            want = po.apply(w, x, None, threads=16)
            err = assert_logits_close(got, want, rel=1e-5)
            print(f"  max err / max |out| {err:.2e}", flush=True)
    eng.close()


def test_q4k_gemv_wide_rows(lh, po):
    """The Q4_K GEMV at rows wider than its register prologue: K = 5120 (four words a lane, x loaded
    ahead of the weights) and K = 9472 (down: x staged after the first words' loads, three chunk groups),
    with and without a bias, against Matrix::apply at 1e-5 of the largest output, on the F32 epilogue of
    lg_matmul; the fused epilogues run in the decode test of the same model."""
    rng = np.random.default_rng(37)
    img = lh.SynthImage("wide-q4k", seed=5)
    og = po.Gguf(img.array())
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=1024)
    for name in ("q.0.weight", "wo.0.weight", "mlp_wi.0.weight", "mlp_wo.0.weight"):
        kind, dims, raw = og.tensor(name)
        assert kind == 12
        cols, rows = dims
        w = po.decode(kind, raw).reshape(rows, cols)
        for mean, bias in ((0.0, None), (1.5, rng.standard_normal(rows).astype(np.float32))):
            x = (mean + rng.standard_normal((1, cols))).astype(np.float32)
            got = eng.matmul(name, x, bias)
            want = po.apply(w, x, bias, threads=16)
            err = assert_logits_close(got, want, rel=1e-5)
            print(f"{name} ({rows} x {cols}) x mean {mean}: max err / max |out| {err:.2e}", flush=True)
    eng.close()


def test_q4k_gemv_decode_wide_model(lh, po):
    """Greedy decode on the one-layer wide Q4_K model (every layer matrix Q4_K: the q|k|v GEMV with bias,
    o with the residual add, gate|up with SwiGLU at K = 5120, down at K = 9472), teacher-forced against the
    oracle's KV-cached decode: logits within 1e-4 of the largest, argmax equal."""
    img = lh.SynthImage("wide-q4k", seed=5)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=1024)
    om = po.Model(po.Gguf(img.array()), threads=16)
    ids = np.random.default_rng(41).integers(0, 1000, 60).astype(np.int32)
    s = eng.seq_create()
    eng.forward(s, ids[:-1], [], [1, 2])
    toks, logits = eng.decode(s, int(ids[-1]), 6, want_logits=True)
    eng.close()
    c = om.cache(100)
    om.prefill(c, ids[:-1], [])
    feed = [int(ids[-1])] + [int(t) for t in toks[:-1]]
    for i, t in enumerate(feed):
        want = om.head(om.prefill(c, [t], [0]))
        err = assert_logits_close(logits[i], want, rel=1e-4)
        assert_argmax_equal(logits[i][None], want, rel=1e-4)
        print(f"step {i}: logits rel {err:.2e}", flush=True)



@pytest.mark.parametrize("preset", ["plumbing-f16", "tiny-f16", "tiny-q8", "tiny-q4k"])
def test_exact_gemm_tilings_agree(lh, preset):
    """The exact GEMM takes small tiles over two LDS stages for short launches (32 x 32; 32 x 128 for Q4_K)
    and 64 x 64, 64 x 128 or 128 x 128 tiles for longer ones: every tiling runs the same per-element MFMA
    sequence, so the first rows of a 2048-row product equal the same rows computed alone at any row
    count, bit for bit (with and without a bias).  F16, Q8_0 (block scales per 32-deep chunk) and the
    K-quants' three-pass form over dequantised hi/lo planes."""
    img = lh.SynthImage(preset, seed=13)
    eng = lh.Engine(lh.Gguf.from_bytes(img), kv_tokens=1024)
    rng = np.random.default_rng(17)
    names = []
    for name in ("qkv.0.weight", "q.0.weight", "v.0.weight", "wo.0.weight", "mlp_wi.0.weight", "mlp_wo.0.weight"):
        try:
            eng.gguf.tensor(name)
            names.append(name)
        except (KeyError, lh.LayaError):
            pass
    assert len(names) >= 4, names
    for name in names:
        _, dims, _ = eng.gguf.tensor(name)
        cols, rows = dims[0], int(np.prod(dims[1:]))
        x = rng.standard_normal((2048, cols)).astype(np.float32)
        bias = rng.standard_normal(rows).astype(np.float32)
        big, big_b = eng.matmul(name, x), eng.matmul(name, x, bias)
        for M in (2, 17, 33, 100, 256, 700):
            print(f"{preset} {name} ({rows} x {cols}) M={M}", flush=True)
            assert_bits_equal(eng.matmul(name, x[:M]), big[:M])
            assert_bits_equal(eng.matmul(name, x[:M], bias), big_b[:M])
    eng.close()


def test_exact_gemm_deep_k_tilings_agree(lh):
    """Narrow outputs over a deep K (OpenThai 0.8B shape: out_proj 1024 x 2048, down_proj 1024 x 3584): a
    few hundred rows take 32 x 64 tiles over two LDS stages, fewer take 32 x 32, 2048 rows 64 x 128; the
    rows agree bit for bit."""
    img = lh.SynthImage("openthai-0.8b", seed=5, n_layers=1)
    eng = lh.Engine(lh.Gguf.from_bytes(img))
    rng = np.random.default_rng(23)
    for name in ("model.layers.0.linear_attn.out_proj.weight", "model.layers.0.mlp.down_proj.weight"):
        _, dims, _ = eng.gguf.tensor(name)
        cols, rows = dims[0], int(np.prod(dims[1:]))
        assert cols >= 2048 and rows == 1024, (name, dims)
        x = rng.standard_normal((2048, cols)).astype(np.float32)
        big = eng.matmul(name, x)
        for M in (100, 300, 480, 700):
            print(f"openthai-0.8b {name} ({rows} x {cols}) M={M}", flush=True)
            assert_bits_equal(eng.matmul(name, x[:M]), big[:M])
    eng.close()
