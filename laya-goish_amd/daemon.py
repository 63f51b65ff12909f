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
echoed id.  A Laya encoder's answers follow laya/decision.rs:213-289 instead: every kind carries
confidence, probabilities and action.act_probability (no abstain).

A body with "states": [state, ...] instead of "state" is a /v1/decide/batch request
(src/server.rs:235-258): one result per state, every pass of every state run as GPU batches.

  python3 laya-goish_amd/daemon.py MODEL.gguf [--model MODEL2.gguf ...] [--default-model NAME]
                                   [--device N] [--precision exact|kv16|fast]
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


def _ids(v, what):
    """A token-id list: JSON integers in [0, 2^31) (the C ABI's int32 ids; the engine checks
    them against the vocabulary)."""
    if v is None:
        return []
    if not isinstance(v, list):
        raise RequestError(f"{what} must be a list of token ids")
    for t in v:
        if isinstance(t, bool) or not isinstance(t, int) or not 0 <= t < 2 ** 31:
            raise RequestError(f"{what}: token id {json.dumps(t)} is not an integer in [0, 2^31)")
    return v


def _option(v, what):
    if v is None:
        return {"name": [], "desc": []}
    if isinstance(v, list):
        return {"name": [], "desc": _ids(v, f"{what}: criterion")}
    if isinstance(v, dict):
        return {"name": _ids(v.get("name"), f"{what}: criterion name"),
                "desc": _ids(v.get("desc"), f"{what}: criterion desc")}
    raise RequestError(f"{what}: criteria entries must be token lists, objects or null")


def to_tokens_request(req) -> tuple[dict, list]:
    """Body -> the token-level request of laya_hip.Engine.decide, plus per-question labels."""
    if not isinstance(req, dict):
        raise RequestError("request must be a JSON object")
    qs = req.get("questions")
    if not isinstance(qs, dict) or not 1 <= len(qs) <= 256:
        raise RequestError("questions must contain 1..256 named questions")
    state = _ids(req.get("state", []), "state")
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
        ins = _ids(q.get("instructions", []), f"{qid}: instructions")
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
        if "act_probability" in a:  # Laya encoder answers (src/models/laya/decision.rs:213-289)
            ans = {"type": kind}
            if kind == "choice":
                ans["choice"] = names[a["choice"]]
            elif kind == "score":
                ans["score"] = a["score"]
                ans["legend"] = {str(j): o["desc"] for j, o in enumerate(opts)}  # an empty label stays empty
            else:
                ans["noul"] = p[1]
            ans["confidence"] = a["confidence"]
            keys = [str(j) for j in range(len(p))] if kind == "score" else ["false", "true"] if kind == "noul" else names
            ans["probabilities"] = dict(zip(keys, p))
            ans["action"] = {"act_probability": a["act_probability"]}
            answers[qid] = ans
            continue
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


def states_requests(req) -> tuple[list, list]:
    """A /v1/decide/batch body (src/server.rs:235-258): one request per state, all sharing the
    questions and options of the body."""
    states = req.get("states")
    if not isinstance(states, list) or not 1 <= len(states) <= 256:
        raise RequestError("states must be an array of 1..256 states")
    out, labels = [], None
    for st in states:
        one = {k: req.get(k) for k in ("questions", "permutations", "order_invariant")}
        one["state"] = st
        t, labels = to_tokens_request(one)
        out.append(t)
    if sum(len(t["questions"]) for t in out) > 256:
        raise RequestError("At most 256 total questions per request")
    return out, labels


def handle(engine, model_name, req, t0) -> dict:
    """One parsed body -> its answer (a single request, or a "states" batch run as GPU batches)."""
    if not isinstance(req, dict):
        raise RequestError("request body must be a JSON object")
    if "states" in req:
        treqs, labels = states_requests(req)
        res = engine.decide_batch(treqs)
        out = {"model": model_name, "results": [answer_json(model_name, {}, labels, r, t0) for r in res]}
        if req.get("id") is not None:
            out["id"] = req["id"]
        return out
    treq, labels = to_tokens_request(req)
    return answer_json(model_name, req, labels, engine.decide(treq), t0)


class RegistryError(Exception):
    pass


class Registry:
    """Loaded models by name (src/registry.rs:10-74): every file is opened and every name checked
    before any weights load; one engine (one HIP stream) per model; requests pick a model with
    "model" or get the default."""

    def __init__(self, paths, default=None, open_engine=None):
        # the library's preflight: every file opened and described, names and aliases unique, the
        # default known -- before any weights load
        try:
            self.default = lh.registry_preflight(list(paths), default)
        except lh.LayaError as e:
            raise RegistryError(str(e)) from None
        self.names, ggufs, self.model_names = {}, [], []
        for i, path in enumerate(paths):
            g = lh.Gguf.open(path)
            d = lh.describe(g)
            for n in [d["name"]] + d["aliases"]:
                self.names[n] = i
            self.model_names.append(d["name"])
            ggufs.append(g)
        # answers name the model as the reference's engine does (a Laya encoder: laya.model_name,
        # src/models/laya/decision.rs:293)
        self.answer_names = list(self.model_names)
        self.engines = [open_engine(g) for g in ggufs]

    def select(self, req) -> int:
        if not isinstance(req, dict):
            raise RequestError("request body must be a JSON object")
        m = req.get("model")
        if m is None:
            return self.default
        if not isinstance(m, str):
            raise RequestError("model must be a string naming a loaded model")
        if m not in self.names:
            raise RequestError(f"unknown model {m}; see /v1/models")
        return self.names[m]

    def close(self):
        for e in self.engines:
            e.close()


def error_json(e, req) -> dict:
    """{"error": message} for a request that failed, with its "id" echoed when it has one."""
    out = {"error": str(e) if isinstance(e, (ValueError, RequestError, lh.LayaError))
           else f"{type(e).__name__}: {e}"}
    if isinstance(req, dict) and req.get("id") is not None:
        out["id"] = req["id"]
    return out


def serve(engine, model_name, fin, fout) -> None:
    """One model, requests answered in order.  Any failure of one request becomes its error line
    and the loop goes on."""
    for line in fin:
        if not line.strip():
            continue
        t0 = time.perf_counter()
        req = None
        try:
            req = json.loads(line)
            out = handle(engine, model_name, req, t0)
        except Exception as e:  # noqa: BLE001 -- one JSON line per request, whatever went wrong
            out = error_json(e, req)
        fout.write(json.dumps(out) + "\n")
        fout.flush()


def serve_registry(reg: Registry, fin, fout) -> None:
    """Several models: one worker thread and FIFO queue per model (in place of the reference's
    global busy flag, src/server.rs:283-297), so models run concurrently on their own streams
    while each model answers its requests in arrival order.  Lines for different models may be
    answered out of input order; "id" is echoed to match them."""
    import queue
    import threading

    lock = threading.Lock()

    def write(obj):
        with lock:
            fout.write(json.dumps(obj) + "\n")
            fout.flush()

    queues = [queue.Queue() for _ in reg.engines]

    def worker(i):
        while True:
            item = queues[i].get()
            if item is None:
                return
            req, t0 = item
            try:
                out = handle(reg.engines[i], reg.answer_names[i], req, t0)
            except Exception as e:  # noqa: BLE001 -- the worker outlives any one request
                out = error_json(e, req)
            write(out)

    threads = [threading.Thread(target=worker, args=(i,), daemon=True) for i in range(len(queues))]
    for t in threads:
        t.start()
    for line in fin:
        if not line.strip():
            continue
        t0 = time.perf_counter()
        req = None
        try:
            req = json.loads(line)
            queues[reg.select(req)].put((req, t0))
        except Exception as e:  # noqa: BLE001
            write(error_json(e, req))
    for q in queues:
        q.put(None)
    for t in threads:
        t.join()


def main() -> int:
    ap = argparse.ArgumentParser(description="JSON-lines decide daemon (token-level requests)")
    ap.add_argument("model", help="model GGUF file (laya-decoder or OpenThai-SystemOne)")
    ap.add_argument("--model", dest="more", action="append", default=[], metavar="GGUF",
                    help="another model to serve (requests select one with \"model\": NAME)")
    ap.add_argument("--default-model", default=None, metavar="NAME")
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--precision", choices=["exact", "kv16", "fast"], default="exact")
    ap.add_argument("--kv-tokens", type=int, default=65536)
    args = ap.parse_args()
    prec = {"exact": lh.PREC_EXACT, "kv16": lh.PREC_KV16, "fast": lh.PREC_FAST}[args.precision]
    opener = lambda g: lh.Engine(g, device=args.device, kv_tokens=args.kv_tokens, precision=prec)  # noqa: E731
    try:
        reg = Registry([args.model] + args.more, args.default_model, opener)
    except (RegistryError, lh.LayaError) as e:
        print(f"error: {e}", file=sys.stderr, flush=True)
        return 1
    for name, e in zip(reg.model_names, reg.engines):
        print(f"loaded {name} ({e.layers()} layers, device {args.device})", file=sys.stderr, flush=True)
    if len(reg.engines) == 1:
        serve(reg.engines[0], reg.answer_names[0], sys.stdin, sys.stdout)
    else:
        serve_registry(reg, sys.stdin, sys.stdout)
    reg.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
