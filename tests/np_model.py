"""Float64 brute-force restatement of the laya-decoder forward pass (test infrastructure).

Independent of the oracle's C: weights are dequantised by np_ref.decode and every op is the
textbook definition in float64:
  rms      y = x / sqrt(mean(x^2) + eps) * w           src/models/openthai/model.rs:84-94 (offset 0)
  rope     rotate-half pairs (j, j + hd/2) from the cos_full/sin_full tables, src/tensor.rs:158-172
  attn     causal, head h reads kv head h // (hq/hkv), scores / sqrt(hd),
           src/models/openthai/model.rs:276-294
  mlp      silu(x Wg^T) * (x Wu^T) then Wd, gate rows first in mlp_wi,
           src/models/openthai/model.rs:71-76,225-230
  head     final rms, then the output rows, src/models/openthai/model.rs:232-240

`mistake` plants one plausible error, so tests can show that the comparison would catch it.
"""
from __future__ import annotations

import numpy as np

import np_ref

MISTAKES = ("swap_gate_up", "kv_head_mod", "no_sqrt_scale", "rope_adjacent_pairs", "no_final_norm",
            "rms_no_eps", "noncausal")


class F64Model:
    def __init__(self, gguf, mistake: str | None = None, dtype=np.float64):
        """gguf: any reader with .tensor(name) -> (kind, dims, raw) and .num(key).  dtype float32
        runs the same textbook forward in f32 with numpy's (BLAS) summation orders: another
        correct f32 ordering, used to measure how far two f32 implementations drift apart."""
        self.mistake = mistake
        self.dtype = np.dtype(dtype)
        num = gguf.num
        self.L = int(num("laya.decoder.block_count"))
        self.d = int(num("laya.decoder.embedding_length"))
        self.hq = int(num("laya.decoder.head_count"))
        self.hkv = int(num("laya.decoder.head_count_kv"))
        self.hd = int(num("laya.decoder.key_length"))
        self.f = int(num("laya.decoder.feed_forward_length"))
        self.V = int(num("laya.decoder.vocab_size"))
        self.eps = float(np.float32(num("laya.decoder.layer_norm_rms_epsilon")))
        self.g = gguf

    def _t(self, name):
        kind, dims, raw = self.g.tensor(name)
        a = np_ref.decode(kind, raw).astype(self.dtype)
        return a.reshape(list(reversed(dims))) if len(dims) > 1 else a

    def _has(self, name):
        try:
            self.g.tensor(name)
            return True
        except Exception:
            return False

    def _rms(self, x, w):
        ms = (x * x).mean(axis=-1, keepdims=True)
        eps = 0.0 if self.mistake == "rms_no_eps" else self.eps
        return x / np.sqrt(ms + eps) * w

    def _rope(self, a, pos, heads, cos, sin):
        hd, half = self.hd, self.hd // 2
        a = a.reshape(len(pos), heads, hd).copy()
        c, s = cos[pos][:, None, :], sin[pos][:, None, :]
        if self.mistake == "rope_adjacent_pairs":
            u, v = a[..., 0::2].copy(), a[..., 1::2].copy()
            a[..., 0::2] = u * c[..., :half] - v * s[..., :half]
            a[..., 1::2] = v * c[..., half:] + u * s[..., half:]
        else:
            u, v = a[..., :half].copy(), a[..., half:].copy()
            a[..., :half] = u * c[..., :half] - v * s[..., :half]
            a[..., half:] = v * c[..., half:] + u * s[..., half:]
        return a.reshape(len(pos), heads * hd)

    def hidden(self, ids):
        """Final hidden states [n][d] (before the final norm) of one sequence."""
        ids = np.asarray(ids)
        n, d, hq, hkv, hd, f = len(ids), self.d, self.hq, self.hkv, self.hd, self.f
        emb = self._t("tok_emb.weight")
        cos, sin = self._t("cos_full"), self._t("sin_full")
        x = emb[ids].copy()
        pos = np.arange(n)
        grp = hq // hkv
        for l in range(self.L):
            h = self._rms(x, self._t(f"attn_norm.{l}.weight"))
            if self._has(f"qkv.{l}.weight"):
                w = self._t(f"qkv.{l}.weight")
                b = self._t(f"qkv.{l}.bias") if self._has(f"qkv.{l}.bias") else None
            else:
                w = np.concatenate([self._t(f"{p}.{l}.weight") for p in "qkv"])
                b = (np.concatenate([self._t(f"{p}.{l}.bias") for p in "qkv"])
                     if self._has(f"q.{l}.bias") else None)
            qkv = h @ w.T + (0 if b is None else b)
            q = self._rope(qkv[:, :hq * hd], pos, hq, cos, sin)
            k = self._rope(qkv[:, hq * hd:(hq + hkv) * hd], pos, hkv, cos, sin)
            v = qkv[:, (hq + hkv) * hd:]
            att = np.zeros((n, hq * hd), self.dtype)
            scale = self.dtype.type(1.0 if self.mistake == "no_sqrt_scale" else np.sqrt(hd))
            for hh in range(hq):
                kh = hh % hkv if self.mistake == "kv_head_mod" else hh // grp
                qh = q[:, hh * hd:(hh + 1) * hd]
                kk = k[:, kh * hd:(kh + 1) * hd]
                vv = v[:, kh * hd:(kh + 1) * hd]
                s = qh @ kk.T / scale
                if self.mistake != "noncausal":
                    s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
                s = np.exp(s - s.max(axis=1, keepdims=True))
                s /= s.sum(axis=1, keepdims=True)
                att[:, hh * hd:(hh + 1) * hd] = s @ vv
            x = x + att @ self._t(f"wo.{l}.weight").T
            h = self._rms(x, self._t(f"ffn_norm.{l}.weight"))
            if self._has(f"mlp_wi.{l}.weight"):
                wi = self._t(f"mlp_wi.{l}.weight")
                wg, wu = wi[:f], wi[f:]
            else:
                wg, wu = self._t(f"gate.{l}.weight"), self._t(f"up.{l}.weight")
            if self.mistake == "swap_gate_up":
                wg, wu = wu, wg
            g, u = h @ wg.T, h @ wu.T
            x = x + (g / (1 + np.exp(-g)) * u) @ self._t(f"mlp_wo.{l}.weight").T
        return x

    def logits(self, ids, positions, vocab_ids=None):
        x = self.hidden(ids)[np.asarray(positions)]
        if self.mistake != "no_final_norm":
            x = self._rms(x, self._t("final_norm.weight"))
        head = self._t("output.weight")
        if vocab_ids is not None:
            head = head[np.asarray(vocab_ids)]
        return x @ head.T
