"""Float64 restatement of the Laya encoder (test infrastructure).

Independent of the oracle's C and of its graph walk: the graph is indexed once (every linear's
bias inputs, every named layer norm), weights are dequantised by np_ref.decode, and every op is
the textbook form in float64 (src/models/laya/model.rs:301-416, src/tensor.rs:103-192):
  layernorm  (x - mean) / sqrt(var + eps) * w + b
  gelu       tanh approximation 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
  attention  bidirectional; local layers see keys |i - j| <= 64; RoPE (j, j + hd/2) from the
             cos/sin tables (full tables on global layers, slide tables on local ones); scores
             q.k / sqrt(hd)
  trunk      h += wo(attn(qkv(ln1 h))); h += down(gelu(gate) * up) of wi(ln2 h); no ln1 on layer 0
  head       ln_final, + type_emb[qtype], 2 full layers with a ReLU MLP
  scorer     logits = fc2(gelu(fc1(ln(h[markers])))); act = act2(gelu(act1([h[0], top1,
             top1 - top2, entropy / ln max(k, 2), max(k, 2) / 255])))

`mistake` plants one plausible error, so tests can show that the comparison would catch it.
"""
from __future__ import annotations

import json

import numpy as np

import np_ref

MISTAKES = ("causal", "window_63", "rope_full_everywhere", "rms_not_layernorm", "gelu_erf", "head_gelu",
            "type_emb_before_norm", "drop_bias_add", "no_embnorm", "entropy_k")


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def _gelu_erf(x):
    from math import erf
    return 0.5 * x * (1.0 + np.vectorize(erf)(x / np.sqrt(2.0)))


class F64Laya:
    def __init__(self, gguf, mistake: str | None = None):
        self.g, self.mistake = gguf, mistake
        graph = json.loads(gguf.str("ggmlc.graph_spec"))
        name = {int(k): v["name"] for k, v in graph["tensors"].items()}
        out_of = {}      # linear output id -> weight name
        self.bias = {}   # weight name -> bias tensor names
        self.added = set()  # biases that come from separate add nodes
        self.norms = {}  # layer-norm node name -> (weight, bias, eps)
        self.attn_full = []
        full_mask = None
        for n in graph["nodes"]:
            ins = n["inputs"]
            if n["opcode"] == 29:
                w = name[ins[0]]
                self.bias[w] = [name[ins[2]]] if len(ins) > 2 else []
                out_of[n["outputs"][0]] = w
            elif n["opcode"] == 200 and ins[0] in out_of:
                self.bias[out_of[ins[0]]].append(name[ins[1]])
                self.added.add(name[ins[1]])
            elif n["opcode"] == 201:
                self.norms[n["name"]] = (name[ins[1]] if len(ins) > 1 else None, name[ins[2]] if len(ins) > 2 else None,
                                         float(np.float32(n["attributes"]["eps"])))
            elif n["opcode"] == 74:
                full_mask = ins[-1] if full_mask is None else full_mask
                self.attn_full.append(ins[-1] == full_mask)
        self.L = sum(1 for t in range(64) if self._has(f"qkv.{t}.weight"))
        self.hd = gguf.tensor("cos_full")[1][0]

    def _has(self, n):
        try:
            self.g.tensor(n)
            return True
        except KeyError:
            return False

    def _t(self, n):
        kind, dims, raw = self.g.tensor(n)
        a = np_ref.decode(kind, raw).astype(np.float64)
        return a.reshape(list(reversed(dims))) if len(dims) > 1 else a

    def _lin(self, key, x):
        w = self._t(key + ".weight")
        if w.ndim == 1:
            w = w[None, :]
        y = x @ w.T
        biases = self.bias[key + ".weight"]
        if self.mistake == "drop_bias_add":
            biases = [b for b in biases if b not in self.added]
        for b in biases:
            y = y + self._t(b)
        return y

    def _ln(self, i, x):
        key = "layer_norm" if i == 0 else f"layer_norm_{i}"
        w, b, eps = self.norms[key]
        if self.mistake == "rms_not_layernorm":
            y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
        else:
            mu = x.mean(-1, keepdims=True)
            y = (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + eps)
        if w is not None:
            y = y * self._t(w)
        if b is not None:
            y = y + self._t(b)
        return y

    def _attn(self, qkv, tables, window):
        s, d3 = qkv.shape
        d, hd = d3 // 3, self.hd
        h = d // hd
        q, k, v = (qkv[:, i * d:(i + 1) * d].reshape(s, h, hd) for i in range(3))
        if tables is not None:
            c, sn = (self._t(t)[:s][:, None, :] for t in tables)
            half = hd // 2

            def rot(a):
                u, w = a[..., :half], a[..., half:]
                return np.concatenate([u * c[..., :half] - w * sn[..., :half], w * c[..., half:] + u * sn[..., half:]], -1)
            q, k = rot(q), rot(k)
        sc = np.einsum("ihd,jhd->hij", q, k) / np.sqrt(hd)
        i, j = np.arange(s)[:, None], np.arange(s)[None, :]
        allowed = np.ones((s, s), bool)
        if window is not None:
            allowed &= np.abs(i - j) <= window
        if self.mistake == "causal":
            allowed &= j <= i
        sc = np.where(allowed[None], sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        return np.einsum("hij,jhd->ihd", p, v).reshape(s, d)

    def forward(self, ids, markers, qtype):
        L = self.L
        gelu = _gelu_erf if self.mistake == "gelu_erf" else _gelu
        h = self._t("tok_emb.weight")[np.asarray(ids)]
        if self.mistake != "no_embnorm":
            h = self._ln(0, h)
        for l in range(L):
            full = self.attn_full[l]
            x = self._ln(2 * l, h) if l else h
            if self.mistake == "rope_full_everywhere":
                tables = ("cos_full", "sin_full")
            else:
                tables = ("cos_full", "sin_full") if full else ("cos_slide", "sin_slide")
            window = None if full else (63 if self.mistake == "window_63" else 64)
            h = h + self._lin(f"wo.{l}", self._attn(self._lin(f"qkv.{l}", x), tables, window))
            up = self._lin(f"mlp_wi.{l}", self._ln(2 * l + 1, h))
            f = up.shape[1] // 2
            h = h + self._lin(f"mlp_wo.{l}", gelu(up[:, :f]) * up[:, f:])
        temb = self._t("type_emb.weight")[qtype]
        if self.mistake == "type_emb_before_norm":
            h = self._ln(2 * L, h + temb)
        else:
            h = self._ln(2 * L, h) + temb
        for i in range(2):
            x = self._ln(2 * L + 1 + 2 * i, h)
            h = h + self._lin(f"head_wo.{i}", self._attn(self._lin(f"head_qkv.{i}", x), None, None))
            fc = self._lin(f"head_fc1.{i}", self._ln(2 * L + 2 + 2 * i, h))
            fc = gelu(fc) if self.mistake == "head_gelu" else np.maximum(fc, 0.0)
            h = h + self._lin(f"head_fc2.{i}", fc)
        g = self._ln(2 * L + 5, h[np.asarray(markers)])
        logits = self._lin("scorer_fc2", gelu(self._lin("scorer_fc1", g)))[:, 0]
        p = np.exp(logits - logits.max())
        p /= p.sum()
        top1 = p.max()
        top2 = (p * (top1 - p) / ((top1 - p) + 1e-6)).max()
        k = len(markers) if self.mistake == "entropy_k" else max(len(markers), 2)
        ent = -(p * np.log(np.maximum(p, 1e-9))).sum() / np.log(k)
        pooled = np.concatenate([h[0], [top1, top1 - top2, ent, max(len(markers), 2) / 255.0]])
        act = self._lin("act_fc2", gelu(self._lin("act_fc1", pooled[None, :])))[0]
        return logits, act
