"""Token-level restatement of the reference decision layer -- TEST INFRASTRUCTURE ONLY.

Only tests load this module, and only to check the results of lg_decide / lg_decide_encode /
lg_decide_scores.  It restates src/models/openthai/decision.rs over token ids:
  passes        decision.rs:140-162
  orders        decision.rs:125-139 (written as round-half-to-even of j*k/n, an independent form)
  encode        decision.rs:169-233 (question blocks, state budget keeping its first token)
  aggregate     decision.rs:268-279 (slot softmax with abstain, pass average) and :297-336
                (normalisation, entropy confidence, first-max choice, expected score)
Arithmetic is f32 in the reference's order; softmax and the confidence go through the C oracle
(tensor::softmax, src/tensor.rs:132-140, over glibc expf/logf).
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np

import pyoracle as po

KINDS = {"choice": 0, "score": 1, "noul": 2}


_SIZES = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def gguf_strings(buf, key: str) -> list:
    """The string array stored under `key` in a GGUF v3 image (src/gguf.rs:48-79 value kinds),
    read independently of both GGUF readers under test."""
    import struct
    b = bytes(buf)
    off = 24
    n_kv = struct.unpack_from("<Q", b, 16)[0]

    def rstr(o):
        n = struct.unpack_from("<Q", b, o)[0]
        return b[o + 8:o + 8 + n].decode("utf-8"), o + 8 + n

    def skip(t, o):
        if t in _SIZES:
            return o + _SIZES[t]
        if t == 8:
            return rstr(o)[1]
        et, cnt = struct.unpack_from("<IQ", b, o)
        o += 12
        for _ in range(cnt):
            o = skip(et, o)
        return o

    for _ in range(n_kv):
        k, off = rstr(off)
        t = struct.unpack_from("<I", b, off)[0]
        off += 4
        if k == key and t == 9:
            et, cnt = struct.unpack_from("<IQ", b, off)
            off += 12
            out = []
            for _ in range(cnt):
                v, off = rstr(off)
                out.append(v)
            return out if et == 8 else []
        off = skip(t, off)
    return []


def _expf(v: float) -> float:
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype, libm.expf.argtypes = ctypes.c_float, [ctypes.c_float]
    return float(np.float32(libm.expf(v)))


def _temperatures(gguf: po.Gguf, temps: list) -> list:
    """expf(log_temperature) when the model has the tensor (src/models/openthai/model.rs:175-178)."""
    try:
        kind, dims, raw = gguf.tensor("log_temperature")
    except KeyError:
        return temps
    return [_expf(float(v)) for v in np.frombuffer(raw, "<f4")]


def _openthai_spec(gguf: po.Gguf) -> dict:
    """OpenThai: the tokenizer's special tokens (decision.rs:185-224), the config's answer id,
    openthai.context_length / state_length; the 256 slot-head rows are scored."""
    cfg = po.openthai_config(gguf)
    index = {}
    for i, t in enumerate(gguf_strings(gguf.buf, "tokenizer.ggml.tokens")):
        index.setdefault(t, i)
    slot = [index[f"<|ts_opt_{i}|>"] for i in range(255)]
    return {
        "V": cfg["V"], "slot": slot + [slot[254]], "head_rows": list(range(256)),
        "state": index["<|ts_state|>"], "question": index["<|ts_q|>"],
        "kind": [index["<|ts_choice|>"], index["<|ts_score|>"], index["<|ts_noul|>"]],
        "answer": cfg["answer"], "newline": index["\u010a"], "colon": index[":"],
        "temperature": _temperatures(gguf, [1.0, 1.0, 1.0]),
        "max_tokens": cfg["max_tokens"], "max_state": cfg["max_state"],
    }


def spec(gguf: po.Gguf) -> dict:
    """Control tokens and budgets: laya.decide.* metadata, else the layout at the top of the
    vocabulary (slot s = V-256+s, state V-257, question V-258, kinds V-259..V-261, answer V-262,
    newline V-263, colon V-264).  OpenThai models: _openthai_spec."""
    if gguf.str("general.architecture") == "openthai_systemone":
        return _openthai_spec(gguf)
    V = int(gguf.num("laya.decoder.vocab_size"))
    ctx = int(gguf.num("laya.decoder.context_length"))
    base = int(gguf.num("laya.decide.slot_base", V - 256))
    temps = [float(np.float32(gguf.num(f"laya.decide.temperature_{k}", 1.0))) for k in ("choice", "score", "noul")]
    temps = _temperatures(gguf, temps)
    return {
        "V": V,
        "slot": [base + i for i in range(256)],
        "head_rows": [base + i for i in range(256)],
        "state": int(gguf.num("laya.decide.state_id", V - 257)),
        "question": int(gguf.num("laya.decide.question_id", V - 258)),
        "kind": [int(gguf.num("laya.decide.choice_id", V - 259)), int(gguf.num("laya.decide.score_id", V - 260)),
                 int(gguf.num("laya.decide.noul_id", V - 261))],
        "answer": int(gguf.num("laya.decide.answer_id", V - 262)),
        "newline": int(gguf.num("laya.decide.newline_id", V - 263)),
        "colon": int(gguf.num("laya.decide.colon_id", V - 264)),
        "temperature": temps,
        "max_tokens": int(gguf.num("laya.decide.context_length", ctx)),
        "max_state": int(gguf.num("laya.decide.state_length", min(2048, ctx))),
    }


def passes(req: dict) -> int:
    ks = [len(q["options"]) for q in req["questions"] if q["type"] == "choice"]
    k = max(ks) if ks else 1
    if req.get("permutations"):
        n = int(req["permutations"])
    elif req.get("order_invariant") is False:
        n = 1
    elif req.get("order_invariant") is True:
        n = 8
    else:
        n = 8 if k >= 11 else 1
    return max(min(n, k), 1)


def orders(k: int, n: int) -> list[list[int]]:
    n = max(min(n, k), 1)
    offsets = sorted({round(Fraction(j * k, n)) % k for j in range(n)})  # Python rounds half to even
    return [[(i + off) % k for i in range(k)] for off in offsets]


def encode(s: dict, req: dict, n: int, pass_: int):
    blocks, order = [], []
    for q in req["questions"]:
        k = len(q["options"])
        if q["type"] == "choice":
            allo = orders(k, n)
            ord_ = allo[pass_ % len(allo)]
        else:
            ord_ = list(range(k))
        b = [s["question"], s["kind"][KINDS[q["type"]]]] + list(q.get("instruction") or []) + [s["newline"]]
        for slot, i in enumerate(ord_):
            o = q["options"][i]
            b += [s["slot"][slot]] + list(o.get("name") or [])
            if o.get("desc"):
                b += [s["colon"]] + list(o["desc"])
            b += [s["newline"]]
        b += [s["answer"], s["newline"]]
        blocks.append(b)
        order.append(ord_)
    total = sum(len(b) for b in blocks)
    if total >= s["max_tokens"]:
        raise ValueError("question tokens exceed the context budget")
    ids = [s["state"]] + list(req.get("state") or []) + [s["newline"]]
    budget = min(s["max_state"], s["max_tokens"] - total)
    truncated = len(ids) > budget
    if truncated:
        ids = ids[:1] + ids[len(ids) - (budget - 1):] if budget > 1 else ids[:1]
    positions = []
    for b in blocks:
        p = max(i for i, t in enumerate(b) if t == s["answer"])
        positions.append(len(ids) + p)
        ids += b
    return np.array(ids, np.int32), np.array(positions, np.int32), order, truncated


def aggregate(s: dict, req: dict, n: int, encs, slot_logits) -> dict:
    f = np.float32
    qs = req["questions"]
    sl = np.asarray(slot_logits, np.float32).reshape(n, len(qs), 256)
    probs = [[f(0)] * len(q["options"]) for q in qs]
    abstain = [f(0)] * len(qs)
    for p in range(n):
        for i, q in enumerate(qs):
            k = len(q["options"])
            T = f(s["temperature"][KINDS[q["type"]]])
            v = [sl[p, i, j] / T for j in range(k)] + [sl[p, i, 255] / T]
            pr = po.softmax(np.array(v, np.float32))
            tot = f(0)
            for j in range(k):
                tot = f(tot + pr[j])
            tot = max(tot, f(1e-12))
            for slot in range(k):
                idx = encs[p][2][i][slot]
                probs[i][idx] = f(probs[i][idx] + f(f(pr[slot] / tot) / f(n)))
            abstain[i] = f(abstain[i] + f(pr[k] / f(n)))
    out = []
    for i, q in enumerate(qs):
        pv = probs[i]
        tot = f(0)
        for x in pv:
            tot = f(tot + x)
        tot = max(tot, f(1e-12))
        pv = np.array([f(x / tot) for x in pv], np.float32)
        conf = f(po.confidence(pv))
        best = 0
        for j in range(1, len(pv)):
            if pv[j] > pv[best]:
                best = j
        score = f(0)
        for j, x in enumerate(pv):
            score = f(score + f(f(j) * x))
        a = {"type": q["type"], "probabilities": pv, "confidence": float(conf), "choice": best}
        if q["type"] == "choice":
            a["abstain"] = float(abstain[i])
        if q["type"] == "score":
            a["score"] = float(score)
        if q["type"] == "noul":
            a["noul"] = float(pv[1])
        out.append(a)
    return {"answers": out, "input_tokens": len(encs[0][0]), "permutations": n,
            "truncated_state": any(e[3] for e in encs)}


def decide(model: po.Model, gguf: po.Gguf, req: dict) -> dict:
    """The whole decision on the CPU oracle: every pass's forward, then the aggregation."""
    s = spec(gguf)
    n = passes(req)
    encs = [encode(s, req, n, p) for p in range(n)]
    if isinstance(model, po.OpenThai):  # slot head: all 256 rows
        logits = np.stack([model.forward(e[0], e[1]) for e in encs])
    else:
        logits = np.stack([model.forward(e[0], e[1], s["head_rows"]) for e in encs])
    return aggregate(s, req, n, encs, logits), logits


# ---- Laya encoder decide (src/models/laya/decision.rs), token level ----

LAYA_KINDS = ("choice", "score", "noul")


def _laya_json(gguf: po.Gguf, key: str):
    """json::parse of a metadata string; unparsable (or repeated keys) counts as absent
    (decision.rs:181-182, src/json.rs:157-166)."""
    import json

    def pairs(kv):
        keys = [k for k, _ in kv]
        if len(keys) != len(set(keys)):
            raise ValueError("duplicate JSON key")
        return dict(kv)

    try:
        return json.loads(gguf.str(key), object_pairs_hook=pairs)
    except (ValueError, KeyError, TypeError):
        return None


def laya_spec(gguf: po.Gguf) -> dict:
    """laya.max_len / head_max_len, the [mask]/[sep]/[cls] ids (decision.rs:104-113) and the two
    temperature tables (decision.rs:180-182)."""
    return {
        "max": int(gguf.num("laya.max_len", 512)), "head_max": int(gguf.num("laya.head_max_len", 192)),
        "mask": int(gguf.num("laya.mask_token_id", 50284)), "sep": int(gguf.num("laya.sep_token_id", 50282)),
        "cls": int(gguf.num("laya.cls_token_id", 50281)),
        "temperature": _laya_json(gguf, "laya.temperature"), "buckets": _laya_json(gguf, "laya.temperature_by_options"),
    }


def laya_encode(s: dict, req: dict, qi: int):
    """decision.rs:100-154 over token ids: -> (ids, markers)."""
    q = req["questions"][qi]
    if s["head_max"] < 32 or s["head_max"] >= s["max"]:
        raise ValueError("invalid sequence budgets")
    head = list(q.get("instruction") or [])
    opts = []
    for o in q["options"]:
        tok = (list(o.get("name") or []) + list(o.get("desc") or []))[:48]
        opts.append([s["mask"]] + tok)
    total = sum(map(len, opts))
    if s["head_max"] - total < 16:
        per = max((s["head_max"] - 16) // len(opts), 4)
        opts = [o[:per] for o in opts]
        total = sum(map(len, opts))
    head = head[:max(s["head_max"] - total, 0, 8)]
    ids, markers = [s["cls"], *head, s["sep"]], []
    for o in opts:
        markers.append(len(ids))
        ids += o
    ids.append(s["sep"])
    room = max(s["max"] - (len(ids) + 1), 0)
    ids = (ids + list(req.get("state") or [])[:room] + [s["sep"]])[:s["max"]]
    if any(m >= len(ids) for m in markers):
        raise ValueError("option markers exceed context")
    return ids, markers


def laya_temperature(s: dict, kind: str, k: int) -> np.float32:
    """The options bucket, else the kind's entry, else 1; at least 1e-3 (decision.rs:190-212)."""
    bucket = f"{kind}:{'2' if k <= 2 else '3-5' if k <= 5 else '6-10' if k <= 10 else '11+'}"
    num = lambda v: float(v) if isinstance(v, (int, float)) and not isinstance(v, bool) else 0.0  # noqa: E731
    b = s["buckets"]
    if isinstance(b, dict) and b.get(bucket) is not None:
        t = np.float32(num(b[bucket]))
    elif isinstance(s["temperature"], list) and LAYA_KINDS.index(kind) < len(s["temperature"]):
        t = np.float32(num(s["temperature"][LAYA_KINDS.index(kind)]))
    else:
        t = np.float32(1.0)
    return max(t, np.float32(1e-3))


def laya_aggregate(s: dict, req: dict, outs, tokens: int) -> dict:
    """decision.rs:185-298: softmax(z / T), act probability, choice, expected score, confidence."""
    f = np.float32
    answers = []
    for q, (z, act) in zip(req["questions"], outs):
        kind, k = q["type"], len(z)
        T = laya_temperature(s, kind, k)
        p = po.softmax(np.array([f(v) / T for v in z], np.float32))
        ap = float(po.softmax(np.asarray(act, np.float32))[0])
        best = max(range(k), key=lambda i: (p[i], -i))
        a = {"type": kind, "probabilities": p, "choice": best, "act_probability": ap}
        if kind == "noul":
            a["confidence"] = float(max(p[1], f(f(1) - p[1])))
            a["noul"] = float(p[1])
        else:
            a["confidence"] = float(po.confidence(p, f64=True))
        if kind == "score":
            a["score"] = float(sum(i * float(v) for i, v in enumerate(p)))
        answers.append(a)
    return {"answers": answers, "input_tokens": tokens}


def laya_decide(model: po.Laya, gguf: po.Gguf, req: dict):
    """The whole Laya decision on the CPU oracle: one forward per question, then the aggregation."""
    s = laya_spec(gguf)
    encs = [laya_encode(s, req, i) for i in range(len(req["questions"]))]
    outs = [model.forward(ids, mk, LAYA_KINDS.index(q["type"])) for (ids, mk), q in zip(encs, req["questions"])]
    return laya_aggregate(s, req, outs, sum(len(e[0]) for e in encs)), outs
