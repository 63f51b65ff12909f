"""Float64 brute-force restatement of the OpenThai-SystemOne text tower (test infrastructure).

Independent of the oracle's C: weights are dequantised by np_ref.decode, every op is the
published definition in float64 and written in matrix form (not the reference's loops):
  rms       y = x / sqrt(mean(x^2) + 1e-6) * (offset + w)        model.rs:84-94
  full      q|gate per head, per-head q/k rms (offset 1), partial RoPE on the first 64 of
            256 dims (pairs j, j+32, angle = pos * 1e7^(-2j/64)), causal GQA softmax(q k^T/16) v,
            out * sigmoid(gate), o_proj                           model.rs:244-299
  delta     causal depthwise conv (kernel 4, zero history) + silu; per head the gated delta
            rule S <- a S;  S <- S + k (beta (v - S^T k))^T;  o = S^T q  with k, q
            L2-normalised (q also / sqrt(128)), a = exp(-exp(A_log) softplus(a_t + dt_bias)),
            beta = sigmoid(b_t); rms(o) (offset 0) * silu(z); out_proj    model.rs:302-362
  layer     x += mixer(rms(x)); x += down(silu(gate(h)) * up(h)) with h = rms(x)  model.rs:214-231
  head      rms(x[positions]) (offset 1) . slot_head^T + bias     model.rs:232-240

`mistake` plants one plausible error, so tests can show that the comparison would catch it.
"""
from __future__ import annotations

import json

import numpy as np

import np_ref

MISTAKES = ("norm_offset_zero", "conv_taps_reversed", "output_before_update", "no_beta", "rope_adjacent_pairs",
            "full_rotary", "gate_after_proj_swap", "kv_head_mod", "decay_after_update", "no_q_scale")


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _silu(x):
    return x * _sigmoid(x)


def _softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


class F64OpenThai:
    def __init__(self, gguf, mistake: str | None = None):
        """gguf: any reader with .tensor(name) -> (kind, dims, raw) and .str(key)."""
        self.g, self.mistake = gguf, mistake
        cfg = json.loads(gguf.str("openthai.config"))
        c = cfg["text_config"]
        self.d, self.f, self.L = int(c["hidden_size"]), int(c["intermediate_size"]), int(c["num_hidden_layers"])
        self.hq, self.hkv = int(c["num_attention_heads"]), int(c["num_key_value_heads"])
        self.nh = int(c["linear_num_value_heads"])
        self.types = c["layer_types"][: self.L]

    def _t(self, name):
        kind, dims, raw = self.g.tensor(name)
        a = np_ref.decode(kind, raw).astype(np.float64)
        return a.reshape(list(reversed(dims))) if len(dims) > 1 else a

    def _rms(self, x, w, offset):
        if self.mistake == "norm_offset_zero":
            offset = 0.0
        return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + 1e-6) * (offset + w)

    def _rope(self, a):  # a [s, heads, 256]
        s = a.shape[0]
        rot = 128 if self.mistake == "full_rotary" else 32
        j = np.arange(rot)
        ang = np.arange(s)[:, None] * 1e7 ** (-2.0 * j / (2 * rot))
        c, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        a = a.copy()
        if self.mistake == "rope_adjacent_pairs":
            x1, x2 = a[..., 0:2 * rot:2].copy(), a[..., 1:2 * rot:2].copy()
            a[..., 0:2 * rot:2], a[..., 1:2 * rot:2] = x1 * c - x2 * sn, x2 * c + x1 * sn
            return a
        x1, x2 = a[..., :rot].copy(), a[..., rot:2 * rot].copy()
        a[..., :rot], a[..., rot:2 * rot] = x1 * c - x2 * sn, x2 * c + x1 * sn
        return a

    def _full(self, p, x):
        s, hq, hkv = x.shape[0], self.hq, self.hkv
        qg = (x @ self._t(p + "self_attn.q_proj.weight").T).reshape(s, hq, 2, 256)
        q, gate = qg[:, :, 0], qg[:, :, 1]
        if self.mistake == "gate_after_proj_swap":
            q, gate = gate, q
        k = (x @ self._t(p + "self_attn.k_proj.weight").T).reshape(s, hkv, 256)
        v = (x @ self._t(p + "self_attn.v_proj.weight").T).reshape(s, hkv, 256)
        q = self._rope(self._rms(q, self._t(p + "self_attn.q_norm.weight"), 1.0))
        k = self._rope(self._rms(k, self._t(p + "self_attn.k_norm.weight"), 1.0))
        grp = hq // hkv
        kv = np.arange(hq) % hkv if self.mistake == "kv_head_mod" else np.arange(hq) // grp
        sc = np.einsum("ihd,jhd->hij", q, k[:, kv]) / 16.0
        sc = np.where(np.tril(np.ones((s, s), bool))[None], sc, -np.inf)
        pr = np.exp(sc - sc.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        out = np.einsum("hij,jhd->ihd", pr, v[:, kv]) * _sigmoid(gate)
        return out.reshape(s, hq * 256) @ self._t(p + "self_attn.o_proj.weight").T

    def _delta(self, p, x):
        s, nh = x.shape[0], self.nh
        lw = nh * 128
        raw = x @ self._t(p + "linear_attn.in_proj_qkv.weight").T
        z = x @ self._t(p + "linear_attn.in_proj_z.weight").T
        a = x @ self._t(p + "linear_attn.in_proj_a.weight").T
        b = x @ self._t(p + "linear_attn.in_proj_b.weight").T
        w = self._t(p + "linear_attn.conv1d.weight").reshape(3 * lw, 4)
        if self.mistake == "conv_taps_reversed":
            w = w[:, ::-1]
        pad = np.concatenate([np.zeros((3, 3 * lw)), raw])
        conv = sum(pad[t:t + s] * w[:, t] for t in range(4))
        qkv = _silu(conv)
        q, k, v = qkv[:, :lw].reshape(s, nh, 128), qkv[:, lw:2 * lw].reshape(s, nh, 128), qkv[:, 2 * lw:].reshape(s, nh, 128)
        q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6)
        if self.mistake != "no_q_scale":
            q = q / np.sqrt(128.0)
        k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
        alpha = np.exp(-np.exp(self._t(p + "linear_attn.A_log")) * _softplus(a + self._t(p + "linear_attn.dt_bias")))
        beta = np.ones_like(b) if self.mistake == "no_beta" else _sigmoid(b)
        out = np.zeros((s, nh, 128))
        for h in range(nh):
            S = np.zeros((128, 128))
            for t in range(s):
                if self.mistake == "output_before_update":
                    out[t, h] = (alpha[t, h] * S).T @ q[t, h]
                if self.mistake != "decay_after_update":
                    S = alpha[t, h] * S
                S = S + np.outer(k[t, h], beta[t, h] * (v[t, h] - S.T @ k[t, h]))
                if self.mistake == "decay_after_update":
                    S = alpha[t, h] * S
                if self.mistake != "output_before_update":
                    out[t, h] = S.T @ q[t, h]
        o = self._rms(out, self._t(p + "linear_attn.norm.weight"), 0.0).reshape(s, lw) * _silu(z)
        return o @ self._t(p + "linear_attn.out_proj.weight").T

    def forward(self, ids, positions) -> np.ndarray:
        ids = np.asarray(ids)
        emb = self._t("model.embed_tokens.weight")
        x = emb[ids]
        for l in range(self.L):
            p = f"model.layers.{l}."
            h = self._rms(x, self._t(p + "input_layernorm.weight"), 1.0)
            x = x + (self._full(p, h) if self.types[l] == "full_attention" else self._delta(p, h))
            h = self._rms(x, self._t(p + "post_attention_layernorm.weight"), 1.0)
            act = _silu(h @ self._t(p + "mlp.gate_proj.weight").T) * (h @ self._t(p + "mlp.up_proj.weight").T)
            x = x + act @ self._t(p + "mlp.down_proj.weight").T
        h = self._rms(x[np.asarray(positions)], self._t("model.norm.weight"), 1.0)
        return h @ self._t("slot_head.weight").T + self._t("slot_head.bias")
