"""GGUF v3 parsing: the engine's reader (C ABI, host only) and the oracle's must accept what
src/gguf.rs:95-179 accepts and reject the rest with the reference's messages.

Every malformed case below is built from a valid file by one targeted change, so each message
is reached by exactly the check it names.
"""
import struct

import numpy as np
import pytest

import gguf_writer as gw

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14


def _valid_meta():
    return [("general.architecture", gw.STR, "ggmlc"), ("laya.decoder.block_count", gw.U32, 2)]


def _valid_tensors():
    return [("a.weight", [32, 2], Q8_0, bytes(range(68))),
            ("b.weight", [4], F32, gw.f32_bytes([1, 2, 3, 4]))]


def _open_both(lh, po, data):
    """(engine message or None, oracle message or None)."""
    try:
        g = lh.Gguf.from_bytes(data)
        g.close()
        m1 = None
    except lh.LayaError as e:
        assert e.kind == "FORMAT", e.kind
        m1 = str(e)
    try:
        po.Gguf(data)
        m2 = None
    except ValueError as e:
        m2 = str(e)
    return m1, m2


def test_valid_file_roundtrip(lh, po):
    meta = _valid_meta() + [
        ("k.u8", gw.U8, 250), ("k.i8", gw.I8, -5), ("k.u16", gw.U16, 65535), ("k.i16", gw.I16, -32768),
        ("k.u32", gw.U32, 4000000000), ("k.i32", gw.I32, -7), ("k.f32", gw.F32, 0.25),
        ("k.bool", gw.BOOL, 1), ("k.u64", gw.U64, 2 ** 40), ("k.i64", gw.I64, -(2 ** 40)),
        ("k.f64", gw.F64, 1e-6), ("k.arr", gw.ARR, (gw.STR, ["x", "yz"])),
        ("k.nested", gw.ARR, (gw.ARR, [(gw.U8, [1, 2]), (gw.U8, [])])),
        ("k.utf8", gw.STR, "ไทย \U0001f600")]
    data = gw.build(meta, _valid_tensors())
    g = lh.Gguf.from_bytes(data)
    o = po.Gguf(data)
    assert sorted(g.names()) == ["a.weight", "b.weight"] and o.ntensors() == 2
    want = {"k.u8": 250, "k.i8": -5, "k.u16": 65535, "k.i16": -32768, "k.u32": 4e9, "k.i32": -7,
            "k.f32": 0.25, "k.u64": 2.0 ** 40, "k.i64": -(2.0 ** 40), "k.f64": 1e-6}
    for k, v in want.items():
        assert g.num(k) == v and o.num(k) == v, k
    # J::num() of a bool, string or array is 0 (src/json.rs), present or not is separate
    assert g.num("k.bool") == 0 and o.num("k.bool") == 0
    assert g.num("missing", -1) == -1 and o.num("missing", -1.0) == -1
    assert g.str("general.architecture") == "ggmlc" == o.str("general.architecture")
    assert g.str("k.utf8") == "ไทย \U0001f600"
    for name, dims, kind, raw in _valid_tensors():
        k1, d1, r1 = g.tensor(name)
        k2, d2, r2 = o.tensor(name)
        assert (k1, d1, r1) == (kind, dims, raw) == (k2, d2, r2)
    with pytest.raises(lh.LayaError, match="missing tensor nope"):
        g.tensor("nope")
    g.close()


def test_file_open_errors(lh, tmp_path):
    data = gw.build(_valid_meta(), _valid_tensors())
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    g = lh.Gguf.open(str(p))  # mmap path (src/io.rs:65-88)
    assert g.tensor("b.weight")[2] == gw.f32_bytes([1, 2, 3, 4])
    g.close()
    with pytest.raises(lh.LayaError, match=r"open .*nonexistent.gguf: errno 2"):
        lh.Gguf.open(str(tmp_path / "nonexistent.gguf"))
    (tmp_path / "empty.gguf").write_bytes(b"")
    with pytest.raises(lh.LayaError, match="empty/unreadable model"):
        lh.Gguf.open(str(tmp_path / "empty.gguf"))


def _mk(meta=None, tensors=None, align=32):
    return gw.build(_valid_meta() if meta is None else meta, _valid_tensors() if tensors is None else tensors,
                    align)


def _raw_header_then(nt, nk, body):
    return gw.header(nt, nk) + body


CASES = {
    "not a GGUF file": lambda: b"GGUX" + _mk()[4:],
    "expected GGUF version 3": lambda: _mk()[:4] + struct.pack("<I", 2) + _mk()[8:],
    "truncated GGUF": lambda: _mk()[:30],
    "GGUF table too large": lambda: gw.header(100001, 0),
    "GGUF table too large ": lambda: gw.header(0, 100001),
    "duplicate GGUF metadata key": lambda: _mk(meta=_valid_meta() + [("general.architecture", gw.STR, "x")]),
    "GGUF string too large": lambda: _raw_header_then(0, 1, struct.pack("<Q", 32 * 1024 * 1024 + 1)),
    "invalid GGUF UTF-8": lambda: _raw_header_then(0, 1, gw.gstr(b"\xff\xfe")),
    "invalid GGUF UTF-8 ": lambda: _raw_header_then(0, 1, gw.gstr(b"\xed\xa0\x80")),  # surrogate
    "invalid GGUF UTF-8  ": lambda: _raw_header_then(0, 1, gw.gstr(b"\xc0\xaf")),  # overlong
    "unsupported GGUF metadata type 13": lambda: _raw_header_then(0, 1, gw.gstr("k") + struct.pack("<I", 13)),
    "GGUF array too large": lambda: _raw_header_then(0, 1, gw.gstr("k") + struct.pack("<IIQ", 9, 0, 1000001)),
    "GGUF metadata nesting too deep": lambda: _raw_header_then(
        0, 1, gw.gstr("k") + struct.pack("<I", 9) + struct.pack("<IQ", 9, 1) * 5 + struct.pack("<IQ", 0, 0)),
    "invalid tensor rank": lambda: _mk(tensors=[("t", [], F32, b"")]),
    "invalid tensor rank ": lambda: _mk(tensors=[("t", [1, 1, 1, 1, 1], F32, b"\0" * 4)]),
    "empty tensor": lambda: _mk(tensors=[("t", [4, 0], F32, b"")]),
    "tensor size overflow": lambda: _mk(tensors=[("t", [2 ** 33, 2 ** 33], F32, b"")]),
    "unsupported GGML tensor type 7; supported F32/F16/Q4_0/Q8_0/Q4_K/Q6_K":
        lambda: _mk(tensors=[("t", [32], 7, b"\0" * 34)]),
    "invalid quantized row alignment": lambda: _mk(tensors=[("t", [31, 2], Q8_0, b"\0" * 68)]),
    "tensor byte size overflow": lambda: _mk(tensors=[("t", [2 ** 62], F32, b"")]),
    "duplicate tensor": lambda: _mk(tensors=[("t", [1], F32, b"\0" * 4), ("t", [1], F32, b"\0" * 4)]),
    "invalid GGUF alignment": lambda: _mk(meta=_valid_meta() + [("general.alignment", gw.U32, 48)]),
    "invalid GGUF alignment ": lambda: _mk(meta=_valid_meta() + [("general.alignment", gw.U32, 8192)]),
    "invalid GGUF alignment  ": lambda: _mk(meta=_valid_meta() + [("general.alignment", gw.I32, -32)]),
    "invalid GGUF alignment   ": lambda: _mk(meta=_valid_meta() + [("general.alignment", gw.STR, "32")]),
    "invalid GGUF alignment    ": lambda: _mk(meta=_valid_meta() + [("general.alignment", gw.BOOL, 1)]),
    "invalid GGUF alignment     ": lambda: _mk(meta=_valid_meta() + [("general.alignment", gw.F64, float("nan"))]),
    "unaligned GGUF tensor": lambda: _unaligned(),
    "truncated tensor data": lambda: _mk()[:-1],
}


def _unaligned():
    body = gw.kv("general.architecture", gw.STR, "ggmlc") + gw.tensor_info("t", [4], F32, 4)
    data = gw.header(1, 1) + body
    return data + b"\0" * ((-len(data)) % 32) + b"\0" * 64


@pytest.mark.parametrize("msg", list(CASES), ids=lambda m: m.strip().replace(" ", "_")[:40] + str(len(m)))
def test_malformed_rejected_with_reference_message(lh, po, msg):
    m1, m2 = _open_both(lh, po, CASES[msg]())
    assert m1 == msg.strip(), f"engine: {m1!r}"
    assert m2 == msg.strip(), f"oracle: {m2!r}"


def test_alignment_variants_accepted(lh, po):
    for a in (1, 8, 64, 4096):
        data = _mk(meta=_valid_meta() + [("general.alignment", gw.U32, a)], align=a)
        assert _open_both(lh, po, data) == (None, None)
    # a float alignment truncates like `as usize` (64.9 -> 64)
    data = _mk(meta=_valid_meta() + [("general.alignment", gw.F32, 64.9)], align=64)
    assert _open_both(lh, po, data) == (None, None)


def test_bounds_checked_in_name_order(lh, po):
    """With two bad tensors the reference reports the one first in name order."""
    body = gw.kv("general.architecture", gw.STR, "ggmlc")
    body += gw.tensor_info("z", [4], F32, 4) + gw.tensor_info("a", [1 << 20], F32, 0)
    data = gw.header(2, 1) + body
    data += b"\0" * ((-len(data)) % 32) + b"\0" * 64
    m1, m2 = _open_both(lh, po, data)
    assert m1 == m2 == "truncated tensor data"


def test_truncation_at_every_byte(lh, po):
    """Every strict prefix of a valid file fails in both readers with the same message."""
    data = _mk()
    for n in range(len(data)):
        m1, m2 = _open_both(lh, po, data[:n])
        assert m1 is not None and m1 == m2, (n, m1, m2)


def test_random_mutations_read_alike(lh, po):
    """4000 seeded mutations of a valid file (one to three byte overwrites, bit flips, deletions or
    insertions each): the engine's reader and the oracle's accept the same files and reject the rest
    with the same message, and neither crashes on any of them."""
    import random
    base = _mk()
    rng = random.Random(20261202)
    accepted, seen = 0, set()
    for i in range(4000):
        d = bytearray(base)
        for _ in range(rng.randint(1, 3)):
            op, p = rng.random(), rng.randrange(len(d))
            if op < 0.5:
                d[p] = rng.randrange(256)
            elif op < 0.8:
                d[p] ^= 1 << rng.randrange(8)
            elif op < 0.9:
                del d[p]
            else:
                d.insert(p, rng.randrange(256))
        m1, m2 = _open_both(lh, po, bytes(d))
        assert m1 == m2, (i, m1, m2)
        accepted += m1 is None
        seen.add(m1)
    # the mutations reach acceptance and at least eight distinct rejections
    assert 0 < accepted < 4000 and len(seen) >= 9, (accepted, sorted(map(str, seen)))
