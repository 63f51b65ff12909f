"""Independent numpy restatements used to pin the oracle (test infrastructure).

Written from the closed forms of the reference, not from the oracle's C:
  half      src/gguf.rs:226-246   (checked against numpy's own float16 -> float32)
  decode    src/gguf.rs:250-336   (elementwise float32, no fused multiply-add)
  kernel    src/tensor.rs:59-102  (8 FMA lanes, sequential lane sum, separate tail mul/add, bias)
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
LAYOUT = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def half(u16: np.ndarray) -> np.ndarray:
    return np.asarray(u16, dtype="<u2").view("<f2").astype(np.float32)


def decode(kind: int, raw: bytes | np.ndarray) -> np.ndarray:
    with np.errstate(invalid="ignore", over="ignore"):  # Inf/NaN scales are legal inputs
        return _decode(kind, raw)


def _decode(kind: int, raw: bytes | np.ndarray) -> np.ndarray:
    b = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.astype(np.uint8)
    block, size = LAYOUT[kind]
    nb = b.size // size
    c = b[: nb * size].reshape(nb, size)
    f = np.float32
    if kind == F32:
        return c.copy().view("<f4").reshape(-1)
    if kind == F16:
        return half(c.copy().view("<u2").reshape(-1))
    if kind == Q8_0:
        d = half(c[:, :2].copy().view("<u2"))  # [nb,1]
        q = c[:, 2:].view(np.int8).astype(f)
        return (d * q).reshape(-1)
    if kind == Q4_0:
        d = half(c[:, :2].copy().view("<u2"))
        lo = (c[:, 2:] & 15).astype(f) - f(8)
        hi = (c[:, 2:] >> 4).astype(f) - f(8)
        return np.concatenate([d * lo, d * hi], axis=1).reshape(-1)
    if kind == Q4_K:
        d = half(c[:, 0:2].copy().view("<u2"))[:, 0]
        dm = half(c[:, 2:4].copy().view("<u2"))[:, 0]
        sc = c[:, 4:16].astype(np.int32)
        qs = c[:, 16:]
        s = np.empty((nb, 8), np.int32)
        m = np.empty((nb, 8), np.int32)
        for j in range(8):
            if j < 4:
                s[:, j], m[:, j] = sc[:, j] & 63, sc[:, j + 4] & 63
            else:
                s[:, j] = (sc[:, j + 4] & 15) | ((sc[:, j - 4] >> 6) << 4)
                m[:, j] = (sc[:, j + 4] >> 4) | ((sc[:, j] >> 6) << 4)
        out = np.empty((nb, 256), f)
        for g in range(4):
            q = qs[:, g * 32:(g + 1) * 32]
            for half_i, nib in ((0, q & 15), (1, q >> 4)):
                j = 2 * g + half_i
                ds = d * s[:, j].astype(f)          # d * s
                mm = dm * m[:, j].astype(f)         # dm * m
                out[:, g * 64 + half_i * 32: g * 64 + half_i * 32 + 32] = \
                    ds[:, None] * nib.astype(f) - mm[:, None]
        return out.reshape(-1)
    if kind == Q6_K:
        ql, qh, sc = c[:, :128], c[:, 128:192], c[:, 192:208].view(np.int8).astype(f)
        d = half(c[:, 208:210].copy().view("<u2"))[:, 0]
        out = np.empty((nb, 256), f)
        for n in range(2):
            for l in range(32):
                lo, hi, si = n * 64 + l, qh[:, n * 32 + l], n * 8 + l // 16
                q = [(ql[:, lo] & 15) | ((hi & 3) << 4), (ql[:, lo + 32] & 15) | (((hi >> 2) & 3) << 4),
                     (ql[:, lo] >> 4) | (((hi >> 4) & 3) << 4), (ql[:, lo + 32] >> 4) | (((hi >> 6) & 3) << 4)]
                for j in range(4):
                    out[:, n * 128 + j * 32 + l] = (d * sc[:, si + 2 * j]) * (q[j].astype(f) - f(32))
        return out.reshape(-1)
    raise ValueError(kind)


def fma32(a, b, c):
    """f32 fused multiply-add via float64: a*b is exact in f64 (48-bit product), and the f64
    sum is rounded once more to f32.  This double rounding differs from a true FMA only when the
    f64 sum lands exactly on an f32 rounding midpoint (about 2^-29 of random cases); the tests
    use fixed inputs, so a bit-exact match shows no such case occurs in them."""
    return (np.float64(a) * np.float64(b) + np.float64(c)).astype(np.float32)


def kernel(w: np.ndarray, x: np.ndarray, bias=None) -> np.ndarray:
    """out[r][c] per src/tensor.rs:75-97, vectorised over (r, c)."""
    w = np.asarray(w, np.float32)
    x = np.asarray(x, np.float32)
    rows, K = w.shape
    m = x.shape[0]
    body = K // 8 * 8
    acc = np.zeros((8, m, rows), np.float32)
    for j in range(0, body, 8):
        for l in range(8):
            acc[l] = fma32(x[:, j + l][:, None], w[:, j + l][None, :], acc[l])
    v = np.full((m, rows), -0.0, np.float32)
    for l in range(8):
        v = v + acc[l]
    for j in range(body, K):
        v = v + x[:, j][:, None] * w[:, j][None, :]
    if bias is not None:
        v = v + np.asarray(bias, np.float32)[None, :]
    return v
