"""Writes tests/golden/forward_tiny.npz: float64 brute-force logits (tests/np_model.py) of the
tiny synthetic laya-decoder models, with the SHA-256 of each generated GGUF image so a change
in the generator is detected rather than silently re-baselined.

Run from the repository root after building: python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.dirname(HERE), os.path.join(ROOT, "laya-goish_amd"), os.path.join(ROOT, "oracle")]

import laya_hip as lh  # noqa: E402
import pyoracle as po  # noqa: E402
from np_model import F64Model  # noqa: E402

SEED = 5


def main():
    out = {"seed": np.int64(SEED)}
    for i, preset in enumerate(("tiny-f16", "tiny-q8", "tiny-q4k")):
        img = lh.SynthImage(preset, seed=SEED)
        g = po.Gguf(img.array().copy())
        V = int(g.num("laya.decoder.vocab_size"))
        rng = np.random.default_rng(1000 + i)
        ids = rng.integers(0, V, 48).astype(np.int32)
        pos = np.array([47, 31, 16, 0], np.int32)
        out[f"{preset}/sha256"] = np.frombuffer(hashlib.sha256(img.bytes()).digest(), np.uint8)
        out[f"{preset}/ids"] = ids
        out[f"{preset}/pos"] = pos
        # stored as f32: the rounding (6e-8 relative) is far below the test tolerance
        out[f"{preset}/logits"] = F64Model(g).logits(ids, pos).astype(np.float32)
    path = os.path.join(HERE, "forward_tiny.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
