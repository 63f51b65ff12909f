#!/usr/bin/env python3
"""JSON-lines decide daemon over the GPU engine (the counterpart of `laya daemon`,
src/main.rs:139-151): one engine is loaded once, then every non-empty stdin line is a request
and gets exactly one JSON line on stdout -- the answer, or {"error": message} after which the
loop goes on.

The tokenizer is not on this path, so requests carry token ids where the reference carries text
(src/models/openthai/decision.rs:20-107 for the shape):

  {"id": any, "state": [ids],
   "questions": {
     "<name>": {"type": "choice", "instructions": [ids],
                "criteria": {"<option>": {"name": [ids], "desc": [ids] | null}, ...}},
     "<name>": {"type": "score", "instructions": [ids],
                "criteria": [{"name": [ids], "desc": [ids]}, ...]},        # levels 0..k-1
     "<name>": {"type": "noul", "instructions": [ids],
                "criteria": {"false": {...} | null, "true": {...} | null}}},
   "permutations": 1..32, "order_invariant": bool}

A criterion may also be a bare list of description ids.  Answers follow decision.rs:297-389:
choice -> probabilities by option, confidence, choice, abstain; score -> probabilities by level,
confidence, score, legend (level -> description ids); noul -> noul (P(yes)); plus usage and the
echoed id.

  python3 laya-goish_amd/daemon.py MODEL.gguf [--device N] [--precision exact|fast]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import laya_hip as lh  # noqa: E402


class RequestError(Exception):
    pass


def _option(v, what):
    if v is None:
        return {"name": [], "desc": []}
    if isinstance(v, list):
        return {"name": [], "desc": v}
    if isinstance(v, dict):
        return {"name": v.get("name") or [], "desc": v.get("desc") or []}
    raise RequestError(f"{what}: criteria entries must be token lists, objects or null")


def to_tokens_request(req) -> tuple[dict, list]:
    """Body -> the token-level request of laya_hip.Engine.decide, plus per-question labels."""
    if not isinstance(req, dict):
        raise RequestError("request must be a JSON object")
    qs = req.get("questions")
    if not isinstance(qs, dict) or not 1 <= len(qs) <= 256:
        raise RequestError("questions must contain 1..256 named questions")
    state = req.get("state", [])
    if not isinstance(state, list):
        raise RequestError("state must be a list of token ids")
    out, labels = [], []
    for qid, q in qs.items():
        if not isinstance(q, dict):
            raise RequestError(f"{qid}: question must be an object")
        kind = q.get("type")
        crit = q.get("criteria")
        if kind == "choice":
            if not isinstance(crit, dict):
                raise RequestError(f"{qid}: choice requires 1..255 options")
            names = list(crit.keys())
            opts = [_option(crit[n], qid) for n in names]
        elif kind == "score":
            if not isinstance(crit, list):
                raise RequestError(f"{qid}: score requires 2..10 levels")
            names = [str(i) for i in range(len(crit))]
            opts = [_option(c, qid) for c in crit]
        elif kind == "noul":
            crit = crit or {}
            if not isinstance(crit, dict) or any(k not in ("false", "true") for k in crit):
                raise RequestError(f"{qid}: noul criteria keys must be false/true")
            names = ["no", "yes"]
            opts = [_option(crit.get("false"), qid), _option(crit.get("true"), qid)]
        else:
            raise RequestError(f"{qid}: invalid question type")
        ins = q.get("instructions", [])
        if not isinstance(ins, list):
            raise RequestError(f"{qid}: instructions must be a list of token ids")
        out.append({"type": kind, "instruction": ins, "options": opts})
        labels.append((qid, kind, names, opts))
    perms = req.get("permutations")
    if perms is not None and (not isinstance(perms, int) or isinstance(perms, bool) or not 1 <= perms <= 32):
        raise RequestError("permutations must be 1..32")
    oi = req.get("order_invariant")
    if oi is not None and not isinstance(oi, bool):
        raise RequestError("order_invariant must be boolean")
    return {"state": state, "questions": out, "permutations": perms, "order_invariant": oi}, labels


def answer_json(model_name, req, labels, res, t0) -> dict:
    answers = {}
    for (qid, kind, names, opts), a in zip(labels, res["answers"]):
        p = [float(x) for x in a["probabilities"]]
        if kind == "noul":
            answers[qid] = {"type": kind, "noul": p[1]}
            continue
        ans = {"type": kind, "probabilities": dict(zip(names, p)), "confidence": a["confidence"]}
        if kind == "choice":
            ans["choice"] = names[a["choice"]]
            ans["abstain"] = a["abstain"]
        else:
            ans["score"] = a["score"]
            ans["legend"] = {str(j): o["desc"] if o["desc"] else str(j) for j, o in enumerate(opts)}
        answers[qid] = ans
    usage = dict(res["usage"])
    usage["latency_ms"] = int((time.perf_counter() - t0) * 1000)
    out = {"model": model_name, "answers": answers, "usage": usage}
    if req.get("id") is not None:
        out["id"] = req["id"]
    return out


def serve(engine, model_name, fin, fout) -> None:
    for line in fin:
        if not line.strip():
            continue
        t0 = time.perf_counter()
        try:
            req = json.loads(line)
            treq, labels = to_tokens_request(req)
            res = engine.decide(treq)
            out = answer_json(model_name, req, labels, res, t0)
        except (ValueError, RequestError, lh.LayaError) as e:
            out = {"error": str(e)}
        fout.write(json.dumps(out) + "\n")
        fout.flush()


def main() -> int:
    ap = argparse.ArgumentParser(description="JSON-lines decide daemon (token-level requests)")
    ap.add_argument("model", help="laya-decoder GGUF file")
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--precision", choices=["exact", "fast"], default="exact")
    ap.add_argument("--kv-tokens", type=int, default=65536)
    args = ap.parse_args()
    g = lh.Gguf.open(args.model)
    eng = lh.Engine(g, device=args.device, kv_tokens=args.kv_tokens,
                    precision=lh.PREC_EXACT if args.precision == "exact" else lh.PREC_FAST)
    name = g.str("general.name", "laya-decoder") or "laya-decoder"
    print(f"loaded {args.model} ({eng.layers()} layers, device {args.device})", file=sys.stderr, flush=True)
    serve(eng, name, sys.stdin, sys.stdout)
    eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
