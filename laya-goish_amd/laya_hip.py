"""ctypes binding of liblaya_hip.so (the C ABI declared in include/lg.h).

Host-side mirror of the reference's model surfaces for the decoder forward path:
``Gguf`` (src/gguf.rs: open/data/get/num), ``Engine`` (src/engine.rs: new/layers,
src/models/openthai/model.rs: forward(ids, positions)), ``Engine.matmul``
(src/tensor.rs: Matrix::apply) and option scoring (src/models/openthai/decision.rs:268-279).
Errors surface as ``LayaError`` carrying the library's message, as the reference's
``Result<_, String>`` does.  The library must be built (``make -C laya-goish_amd``); there
is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblaya_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "lg.h")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 8, 12, 14
PREC_EXACT, PREC_FAST, PREC_KV16 = 0, 1, 2
ARCH_LAYA_DECODER, ARCH_OPENTHAI, ARCH_LAYA = 0, 1, 2
KIND_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}
ERR = {1: "INVALID", 2: "FORMAT", 3: "DEVICE", 4: "OOM", 5: "CANCELED", 6: "UNSUPPORTED"}


class LayaError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code
        self.kind = ERR.get(code, str(code))


class EngineOpts(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int), ("kv_pages", ctypes.c_int),
                ("kv_tokens", ctypes.c_int64), ("max_batch_tokens", ctypes.c_int64),
                ("precision", ctypes.c_int)]


class ModelInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("layers", "d_model", "heads", "kv_heads", "head_dim", "ffn", "vocab", "context")] + \
               [("kind_attn", ctypes.c_uint32), ("kind_ffn", ctypes.c_uint32), ("kind_head", ctypes.c_uint32),
                ("weight_bytes", ctypes.c_int64), ("kv_bytes", ctypes.c_int64),
                ("kv_pages", ctypes.c_int), ("kv_page_tokens", ctypes.c_int),
                ("precision", ctypes.c_int), ("kv_elem_bytes", ctypes.c_int),
                ("arch", ctypes.c_int), ("linear_heads", ctypes.c_int), ("full_layers", ctypes.c_int),
                ("load_seconds", ctypes.c_double)]

    def asdict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


class Request(ctypes.Structure):
    _fields_ = [("seq", ctypes.c_int), ("ids", ctypes.POINTER(ctypes.c_int32)), ("n", ctypes.c_int),
                ("positions", ctypes.POINTER(ctypes.c_int32)), ("npos", ctypes.c_int)]


Q_KINDS = {"choice": 0, "score": 1, "noul": 2}
_I32P = ctypes.POINTER(ctypes.c_int32)


class Question(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("instruction", _I32P), ("n_instruction", ctypes.c_int32),
                ("n_options", ctypes.c_int32), ("names", ctypes.POINTER(_I32P)), ("name_len", _I32P),
                ("descs", ctypes.POINTER(_I32P)), ("desc_len", _I32P)]


class DecideRequest(ctypes.Structure):
    _fields_ = [("state", _I32P), ("n_state", ctypes.c_int32), ("questions", ctypes.POINTER(Question)),
                ("n_questions", ctypes.c_int32), ("permutations", ctypes.c_int32),
                ("order_invariant", ctypes.c_int32)]


class DecideResult(ctypes.Structure):
    _fields_ = [("probs", ctypes.POINTER(ctypes.c_float)), ("abstain", ctypes.POINTER(ctypes.c_float)),
                ("confidence", ctypes.POINTER(ctypes.c_float)), ("score", ctypes.POINTER(ctypes.c_float)),
                ("choice", _I32P), ("input_tokens", ctypes.c_int32), ("permutations", ctypes.c_int32),
                ("truncated", ctypes.c_int32)]


class LayaInput(ctypes.Structure):
    _fields_ = [("ids", _I32P), ("n", ctypes.c_int32), ("markers", _I32P), ("k", ctypes.c_int32),
                ("qtype", ctypes.c_int32)]


class DecideArgs:
    """ctypes form of a token-level decide request:
    {"state": [ids], "questions": [{"type": "choice"|"score"|"noul", "instruction": [ids],
      "options": [{"name": [ids], "desc": [ids] | None}, ...]}, ...],
     "permutations": int | None, "order_invariant": bool | None}
    (the token-level counterpart of the /v1/decide body, src/models/openthai/decision.rs:20-107).
    Keeps every array alive for the duration of the call."""

    def __init__(self, req: dict):
        self.keep = []
        qs = req.get("questions") or []
        self.kinds = []
        self.nopts = []
        qarr = (Question * max(1, len(qs)))()
        for i, q in enumerate(qs):
            if q.get("type") not in Q_KINDS:
                raise LayaError(1, f"question {i}: invalid question type")
            opts = q.get("options") or []
            ins = self._arr(q.get("instruction") or [])
            names = [self._arr(o.get("name") or []) for o in opts]
            descs = [self._arr(o.get("desc") or []) for o in opts]
            name_ptrs = (_I32P * max(1, len(opts)))(*[ctypes.cast(a.ctypes.data, _I32P) for a in names])
            desc_ptrs = (_I32P * max(1, len(opts)))(*[ctypes.cast(a.ctypes.data, _I32P) for a in descs])
            name_len = self._arr([len(a) for a in names])
            desc_len = self._arr([len(a) for a in descs])
            self.keep += [name_ptrs, desc_ptrs]
            qarr[i] = Question(Q_KINDS[q["type"]], ctypes.cast(ins.ctypes.data, _I32P), len(ins), len(opts),
                               name_ptrs, ctypes.cast(name_len.ctypes.data, _I32P), desc_ptrs,
                               ctypes.cast(desc_len.ctypes.data, _I32P))
            self.kinds.append(q["type"])
            self.nopts.append(len(opts))
        self.keep.append(qarr)
        state = self._arr(req.get("state") or [])
        oi = req.get("order_invariant")
        self.req = DecideRequest(ctypes.cast(state.ctypes.data, _I32P), len(state), qarr, len(qs),
                                 int(req.get("permutations") or 0), -1 if oi is None else int(bool(oi)))

    def _arr(self, v):
        if not isinstance(v, (list, tuple, np.ndarray)):
            raise LayaError(1, "token ids must be a list of integers")
        if not isinstance(v, np.ndarray):
            for t in v:  # int32 ids; the library checks them against the vocabulary
                if isinstance(t, bool) or not isinstance(t, (int, np.integer)) or not -2 ** 31 <= int(t) < 2 ** 31:
                    raise LayaError(1, f"token id {t!r} is not a 32-bit integer")
        a = np.ascontiguousarray(np.asarray(v, dtype=np.int32).reshape(-1))
        if a.size == 0:
            a = np.zeros(1, np.int32)[:0]
        self.keep.append(a)
        return a

    def result(self):
        nq = len(self.nopts)
        self.out = {"probs": np.zeros(max(1, sum(self.nopts)), np.float32), "abstain": np.zeros(max(1, nq), np.float32),
                    "confidence": np.zeros(max(1, nq), np.float32), "score": np.zeros(max(1, nq), np.float32),
                    "choice": np.zeros(max(1, nq), np.int32)}
        o = self.out
        fp = lambda a: ctypes.cast(a.ctypes.data, ctypes.POINTER(ctypes.c_float))  # noqa: E731
        self.res = DecideResult(fp(o["probs"]), fp(o["abstain"]), fp(o["confidence"]), fp(o["score"]),
                                ctypes.cast(o["choice"].ctypes.data, _I32P), 0, 0, 0)
        return self.res

    def answers(self, laya: bool = False):
        """Per-question answers; for a Laya encoder the abstain entry carries the act probability
        (src/models/laya/decision.rs:286-289)."""
        o, out, at = self.out, [], 0
        for i, (kind, k) in enumerate(zip(self.kinds, self.nopts)):
            p = o["probs"][at:at + k].copy()
            at += k
            a = {"type": kind, "probabilities": p, "confidence": float(o["confidence"][i]),
                 "choice": int(o["choice"][i])}
            if laya:
                a["act_probability"] = float(o["abstain"][i])
            elif kind == "choice":
                a["abstain"] = float(o["abstain"][i])
            if kind == "score":
                a["score"] = float(o["score"][i])
            if kind == "noul":
                a["noul"] = float(p[1])
            out.append(a)
        r = self.res
        if laya:  # src/models/laya/decision.rs:293-303: no option-order passes, no state budget
            return {"answers": out, "usage": {"input_tokens": int(r.input_tokens), "output_tokens": 0}}
        return {"answers": out, "usage": {"input_tokens": int(r.input_tokens), "output_tokens": 0,
                                          "permutations": int(r.permutations),
                                          "truncated_state": bool(r.truncated)}}


def decide_encode(gguf: "Gguf", req: dict, pass_: int = 0):
    """Token layout of one pass: (ids, answer positions, option order per question, truncated,
    passes).  Host only."""
    a = DecideArgs(req)
    n, trunc, passes = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(lib().lg_decide_encode(gguf.h, ctypes.byref(a.req), pass_, None, 0, ctypes.byref(n), None, None,
                                 ctypes.byref(trunc), ctypes.byref(passes)))
    ids = np.zeros(n.value, np.int32)
    pos = np.zeros(max(1, len(a.nopts)), np.int32)
    order = np.full((max(1, len(a.nopts)), 255), -1, np.int32)
    check(lib().lg_decide_encode(gguf.h, ctypes.byref(a.req), pass_, _ptr(ids), n.value, ctypes.byref(n),
                                 _ptr(pos), _ptr(order), ctypes.byref(trunc), ctypes.byref(passes)))
    orders = [order[i, :k].tolist() for i, k in enumerate(a.nopts)]
    return ids, pos[:len(a.nopts)], orders, bool(trunc.value), passes.value


def decide_scores(gguf: "Gguf", req: dict, slot_logits) -> dict:
    """Aggregation of decide over caller-held slot logits [passes][questions][256]."""
    a = DecideArgs(req)
    sl = _c(slot_logits, np.float32)
    res = a.result()
    check(lib().lg_decide_scores(gguf.h, ctypes.byref(a.req), _ptr(sl), ctypes.byref(res)))
    return a.answers()


def laya_decide_encode(gguf: "Gguf", req: dict, question: int = 0):
    """Laya token layout of one question: (ids, option marker positions).  Host only."""
    a = DecideArgs(req)
    n = ctypes.c_int()
    check(lib().lg_laya_decide_encode(gguf.h, ctypes.byref(a.req), question, None, 0, ctypes.byref(n), None))
    ids = np.zeros(n.value, np.int32)
    k = a.nopts[question] if 0 <= question < len(a.nopts) else 0
    mk = np.zeros(max(1, k), np.int32)
    check(lib().lg_laya_decide_encode(gguf.h, ctypes.byref(a.req), question, _ptr(ids), n.value, ctypes.byref(n),
                                      _ptr(mk)))
    return ids, mk[:k]


def laya_decide_scores(gguf: "Gguf", req: dict, logits, act) -> dict:
    """Laya aggregation over caller-held option logits (concatenated) and act logits [questions][2]."""
    a = DecideArgs(req)
    lg_, ac = _c(logits, np.float32), _c(act, np.float32)
    res = a.result()
    check(lib().lg_laya_decide_scores(gguf.h, ctypes.byref(a.req), _ptr(lg_), _ptr(ac), ctypes.byref(res)))
    return a.answers(laya=True)


CANCEL_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)

_lib = None


def lib() -> ctypes.CDLL:
    """Load the built library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C laya-goish_amd`")
        L = ctypes.CDLL(LIB_PATH)
        P, I, U32, U64, I64, F = (ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64,
                                  ctypes.c_int64, ctypes.c_float)
        sig = {
            "lg_last_error": (ctypes.c_char_p, []),
            "lg_version": (ctypes.c_char_p, []),
            "lg_layout": (I, [U32, ctypes.POINTER(U64), ctypes.POINTER(U64)]),
            "lg_half": (F, [ctypes.c_uint16]),
            "lg_gguf_open": (I, [ctypes.c_char_p, ctypes.POINTER(P)]),
            "lg_gguf_open_memory": (I, [P, U64, ctypes.POINTER(P)]),
            "lg_gguf_close": (None, [P]),
            "lg_gguf_tensor_count": (I, [P]),
            "lg_gguf_tensor_name": (ctypes.c_char_p, [P, I]),
            "lg_gguf_tensor": (I, [P, ctypes.c_char_p, ctypes.POINTER(U32), ctypes.POINTER(U64),
                                   ctypes.POINTER(I), ctypes.POINTER(P), ctypes.POINTER(U64)]),
            "lg_gguf_meta_num": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(I)]),
            "lg_gguf_meta_str": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(I)]),
            "lg_dequant": (I, [U32, P, U64, P]),
            "lg_synth_gguf": (I, [ctypes.c_char_p, U64, I, ctypes.POINTER(P), ctypes.POINTER(U64)]),
            "lg_synth_gguf_file": (I, [ctypes.c_char_p, U64, I, ctypes.c_char_p]),
            "lg_synth_free": (None, [P]),
            "lg_engine_create": (I, [P, ctypes.POINTER(EngineOpts), ctypes.POINTER(P)]),
            "lg_engine_destroy": (None, [P]),
            "lg_engine_info": (I, [P, ctypes.POINTER(ModelInfo)]),
            "lg_engine_sync": (I, [P]),
            "lg_probe_read": (I, [ctypes.c_uint64, I, ctypes.POINTER(ctypes.c_double)]),
            "lg_engine_workspace_bytes": (I, [P, ctypes.POINTER(ctypes.c_int64)]),
            "lg_matmul": (I, [P, ctypes.c_char_p, P, I, P, P]),
            "lg_seq_create": (I, [P, ctypes.POINTER(I)]),
            "lg_seq_fork": (I, [P, I, I, ctypes.POINTER(I)]),
            "lg_seq_free": (I, [P, I]),
            "lg_seq_len": (I, [P, I, ctypes.POINTER(I)]),
            "lg_seq_kv_read": (I, [P, I, I, I, I, P, P]),
            "lg_forward": (I, [P, I, P, I, P, I, P, I, P, CANCEL_FN, P]),
            "lg_batch_create": (I, [P, ctypes.POINTER(Request), I, ctypes.POINTER(P)]),
            "lg_batch_free": (None, [P, P]),
            "lg_batch_run": (I, [P, P, P, I, F, P, P, P, CANCEL_FN, P]),
            "lg_batch_rewind": (I, [P, P]),
            "lg_decode": (I, [P, I, ctypes.c_int32, I, P, P]),
            "lg_decode_noalloc": (I, [P, I, ctypes.c_int32, I, P, P]),
            "lg_decode_graph": (I, [P, I, ctypes.c_int32, I, P, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double)]),
            "lg_option_scores": (I, [P, I, F, P, P]),
            "lg_decide": (I, [P, ctypes.POINTER(DecideRequest), ctypes.POINTER(DecideResult), CANCEL_FN, P]),
            "lg_laya_forward": (I, [P, ctypes.POINTER(LayaInput), I, P, P, CANCEL_FN, P]),
            "lg_decide_batch": (I, [P, ctypes.POINTER(DecideRequest), I, ctypes.POINTER(DecideResult), CANCEL_FN, P]),
            "lg_decide_encode": (I, [P, ctypes.POINTER(DecideRequest), I, P, I, ctypes.POINTER(I), P, P,
                                     ctypes.POINTER(I), ctypes.POINTER(I)]),
            "lg_decide_scores": (I, [P, ctypes.POINTER(DecideRequest), P, ctypes.POINTER(DecideResult)]),
            "lg_laya_decide_encode": (I, [P, ctypes.POINTER(DecideRequest), I, P, I, ctypes.POINTER(I), P]),
            "lg_laya_decide_scores": (I, [P, ctypes.POINTER(DecideRequest), P, P, ctypes.POINTER(DecideResult)]),
            "lg_option_confidence": (I, [P, I, I, ctypes.POINTER(F)]),
            "lg_profile_enable": (I, [P, I]),
            "lg_profile_read": (I, [P, ctypes.c_char_p, ctypes.POINTER(I64), ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
            "lg_profile_reset": (I, [P]),
            "lg_model_describe": (I, [P, P]),
            "lg_registry_preflight": (I, [P, I, ctypes.c_char_p, ctypes.POINTER(I)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_functions() -> list[str]:
    """Names of every function declared in include/lg.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lg_[a-z0-9_]+)\s*\(", text)) - {"lg_cancel_fn"})


def check(rc: int) -> None:
    if rc != 0:
        raise LayaError(rc, lib().lg_last_error().decode())


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


def layout(kind: int) -> tuple[int, int]:
    b, s = ctypes.c_uint64(), ctypes.c_uint64()
    check(lib().lg_layout(kind, ctypes.byref(b), ctypes.byref(s)))
    return b.value, s.value


def half(bits: int) -> float:
    return lib().lg_half(bits)


def probe_read(nbytes: int, launches: int = 200) -> float:
    """lg_probe_read: microseconds per dependent launch of a plain read kernel over nbytes."""
    us = ctypes.c_double()
    check(lib().lg_probe_read(nbytes, launches, ctypes.byref(us)))
    return us.value


def dequant(kind: int, raw: bytes | np.ndarray) -> np.ndarray:
    """gguf::decode on the GPU (through the engine's repacked weight layout)."""
    buf = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else _c(raw, np.uint8)
    block, size = layout(kind)
    out = np.empty(buf.size // size * block, dtype=np.float32)
    check(lib().lg_dequant(kind, _ptr(buf), buf.size, _ptr(out)))
    return out


def option_scores(logits, temperature: float = 1.0):
    z = _c(logits, np.float32)
    p = np.empty_like(z)
    lp = np.empty_like(z)
    check(lib().lg_option_scores(_ptr(z), z.size, temperature, _ptr(p), _ptr(lp)))
    return p, lp


CONF_F32, CONF_F64 = 0, 1


def option_confidence(probs, mode: int = CONF_F32) -> float:
    """1 - H(p)/ln k (decision confidence); mode CONF_F32 or CONF_F64."""
    p = _c(probs, np.float32)
    out = ctypes.c_float()
    check(lib().lg_option_confidence(_ptr(p), p.size, mode, ctypes.byref(out)))
    return out.value


class SynthImage:
    """A seeded synthetic laya-decoder GGUF image held in library-allocated memory."""

    def __init__(self, preset: str, seed: int = 0, n_layers: int = 0):
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        check(lib().lg_synth_gguf(preset.encode(), seed, n_layers, ctypes.byref(p), ctypes.byref(n)))
        self.ptr, self.len = p, n.value
        self.preset, self.seed = preset, seed

    def bytes(self) -> bytes:
        return ctypes.string_at(self.ptr, self.len)

    def array(self) -> np.ndarray:
        return np.ctypeslib.as_array(ctypes.cast(self.ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(self.len,))

    def __del__(self):
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.lg_synth_free(self.ptr)
            self.ptr = None


def synth_file(preset: str, seed: int, path: str, n_layers: int = 0) -> None:
    check(lib().lg_synth_gguf_file(preset.encode(), seed, n_layers, path.encode()))


class ModelDesc(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("family", ctypes.c_char * 64), ("architecture", ctypes.c_char * 64),
                ("aliases", (ctypes.c_char * 64) * 4), ("n_aliases", ctypes.c_int), ("release_date", ctypes.c_char * 16)]


def describe(g: "Gguf") -> dict:
    """models::describe (src/models/mod.rs:32-64): name, family, architecture, aliases, release date."""
    d = ModelDesc()
    check(lib().lg_model_describe(g.h, ctypes.byref(d)))
    return {"name": d.name.decode(), "family": d.family.decode(), "architecture": d.architecture.decode(),
            "aliases": [d.aliases[i].value.decode() for i in range(d.n_aliases)],
            "release_date": d.release_date.decode()}


def registry_preflight(paths, default=None) -> int:
    """Registry::load's preflight (src/registry.rs:16-39) before any weights load; the default's index."""
    arr = (ctypes.c_char_p * max(1, len(paths)))(*[p.encode() for p in paths])
    idx = ctypes.c_int()
    check(lib().lg_registry_preflight(arr, len(paths), None if default is None else default.encode(),
                                      ctypes.byref(idx)))
    return idx.value


class Gguf:
    """GGUF v3 reader (mirrors src/gguf.rs Gguf::open / data / get / num)."""

    def __init__(self, handle, keep=None):
        self.h = handle
        self._keep = keep

    @classmethod
    def open(cls, path: str) -> "Gguf":
        h = ctypes.c_void_p()
        check(lib().lg_gguf_open(path.encode(), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_bytes(cls, data) -> "Gguf":
        if isinstance(data, SynthImage):
            h = ctypes.c_void_p()
            check(lib().lg_gguf_open_memory(data.ptr, data.len, ctypes.byref(h)))
            return cls(h, data)
        buf = np.frombuffer(bytes(data), dtype=np.uint8).copy()
        h = ctypes.c_void_p()
        check(lib().lg_gguf_open_memory(_ptr(buf), buf.size, ctypes.byref(h)))
        return cls(h, buf)

    def names(self) -> list[str]:
        L = lib()
        return [L.lg_gguf_tensor_name(self.h, i).decode() for i in range(L.lg_gguf_tensor_count(self.h))]

    def tensor(self, name: str):
        kind, nd, data, n = ctypes.c_uint32(), ctypes.c_int(), ctypes.c_void_p(), ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 4)()
        check(lib().lg_gguf_tensor(self.h, name.encode(), ctypes.byref(kind), dims, ctypes.byref(nd),
                                   ctypes.byref(data), ctypes.byref(n)))
        raw = ctypes.string_at(data, n.value)
        return kind.value, [dims[i] for i in range(nd.value)], raw

    def num(self, key: str, default=None):
        v, found = ctypes.c_double(), ctypes.c_int()
        check(lib().lg_gguf_meta_num(self.h, key.encode(), ctypes.byref(v), ctypes.byref(found)))
        return v.value if found.value else default

    def str(self, key: str, default=None):
        v, found = ctypes.c_char_p(), ctypes.c_int()
        check(lib().lg_gguf_meta_str(self.h, key.encode(), ctypes.byref(v), ctypes.byref(found)))
        return v.value.decode() if found.value else default

    def close(self):
        if self.h:
            lib().lg_gguf_close(self.h)
            self.h = None

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.lg_gguf_close(self.h)
            self.h = None


class Batch:
    def __init__(self, engine: "Engine", handle, requests, total_positions: int):
        self.engine, self.h, self._keep, self.R = engine, handle, requests, total_positions

    def run(self, option_ids, temperature: float = 1.0, cancel=None):
        """Head rows `option_ids` at every answer position: (logits, probs, logprobs); option
        scores only for k <= 32 (else None)."""
        k = len(option_ids)
        ids = _c(option_ids, np.int32)
        out = [np.empty((self.R, k), dtype=np.float32) if i == 0 or k <= 32 else None for i in range(3)]
        cb = CANCEL_FN(cancel) if cancel else CANCEL_FN(0)
        check(lib().lg_batch_run(self.engine.h, self.h, _ptr(ids), k, temperature,
                                 *(_ptr(o) for o in out), cb, None))
        return tuple(out)

    def rewind(self):
        check(lib().lg_batch_rewind(self.engine.h, self.h))

    def free(self):
        if self.h:
            lib().lg_batch_free(self.engine.h, self.h)
            self.h = None

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None and self.engine.h:
            _lib.lg_batch_free(self.engine.h, self.h)
            self.h = None


class Engine:
    """One model on one GPU (mirrors src/engine.rs Engine::new / layers / decide)."""

    def __init__(self, gguf: Gguf, device: int = 0, kv_tokens: int = 65536, max_batch_tokens: int = 65536,
                 kv_pages: int = 0, precision: int = PREC_EXACT):
        self.gguf = gguf
        opts = EngineOpts(device, kv_pages, kv_tokens, max_batch_tokens, precision)
        h = ctypes.c_void_p()
        check(lib().lg_engine_create(gguf.h, ctypes.byref(opts), ctypes.byref(h)))
        self.h = h
        info = ModelInfo()
        check(lib().lg_engine_info(self.h, ctypes.byref(info)))
        self.info = info.asdict()

    def layers(self) -> int:
        return self.info["layers"]

    def close(self):
        if self.h:
            lib().lg_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.lg_engine_destroy(self.h)
            self.h = None

    def sync(self):
        check(lib().lg_engine_sync(self.h))

    def workspace_bytes(self) -> int:
        """Device bytes held by the engine's grow-only workspaces (lg_engine_workspace_bytes)."""
        n = ctypes.c_int64()
        check(lib().lg_engine_workspace_bytes(self.h, ctypes.byref(n)))
        return n.value

    def matmul(self, tensor: str, x, bias=None) -> np.ndarray:
        x = _c(x, np.float32)
        if x.ndim == 1:
            x = x[None, :]
        b = None if bias is None else _c(bias, np.float32)
        kind, dims, _ = self.gguf.tensor(tensor)
        rows = int(np.prod(dims[1:]))
        y = np.empty((x.shape[0], rows), dtype=np.float32)
        check(lib().lg_matmul(self.h, tensor.encode(), _ptr(x), x.shape[0], _ptr(b), _ptr(y)))
        return y

    def seq_create(self) -> int:
        s = ctypes.c_int()
        check(lib().lg_seq_create(self.h, ctypes.byref(s)))
        return s.value

    def seq_fork(self, parent: int, ntokens: int) -> int:
        s = ctypes.c_int()
        check(lib().lg_seq_fork(self.h, parent, ntokens, ctypes.byref(s)))
        return s.value

    def seq_free(self, seq: int) -> None:
        check(lib().lg_seq_free(self.h, seq))

    def seq_len(self, seq: int) -> int:
        n = ctypes.c_int()
        check(lib().lg_seq_len(self.h, seq, ctypes.byref(n)))
        return n.value

    def seq_kv_read(self, seq: int, layer: int, pos0: int, n: int):
        """(K, V) cached rows of positions [pos0, pos0 + n) of one layer, f32 [n][kv_heads * head_dim]."""
        w = self.info["kv_heads"] * self.info["head_dim"]
        k = np.empty((n, w), np.float32)
        v = np.empty((n, w), np.float32)
        check(lib().lg_seq_kv_read(self.h, seq, layer, pos0, n, _ptr(k), _ptr(v)))
        return k, v

    def forward(self, seq: int, ids, positions, vocab_ids=None, cancel=None) -> np.ndarray:
        """Model::forward(ids, positions): logits at `positions` for `vocab_ids` (None = all)."""
        ids = _c(ids, np.int32)
        pos = _c(positions, np.int32)
        vid = None if vocab_ids is None else _c(vocab_ids, np.int32)
        full = 256 if self.info["arch"] == ARCH_OPENTHAI else self.info["vocab"]  # slot head or LM head rows
        nv = full if vid is None else vid.size
        out = np.empty((pos.size, nv), dtype=np.float32)
        cb = CANCEL_FN(cancel) if cancel else CANCEL_FN(0)
        check(lib().lg_forward(self.h, seq, _ptr(ids), ids.size, _ptr(pos), pos.size, _ptr(vid),
                               0 if vid is None else vid.size, _ptr(out), cb, None))
        return out

    def batch(self, requests) -> Batch:
        """requests: list of (seq, ids, positions)."""
        keep, arr = [], (Request * len(requests))()
        total = 0
        for i, (seq, ids, pos) in enumerate(requests):
            ids = _c(ids, np.int32)
            pos = _c(pos, np.int32)
            keep += [ids, pos]
            arr[i] = Request(seq, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ids.size,
                             pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), pos.size)
            total += pos.size
        h = ctypes.c_void_p()
        check(lib().lg_batch_create(self.h, arr, len(requests), ctypes.byref(h)))
        return Batch(self, h, (arr, keep), total)

    def decide(self, req: dict, cancel=None) -> dict:
        """Request-level decide over token ids (Backend::decide, src/models/openthai/decision.rs:243-390):
        every option-order pass prefilled as one GPU batch, slot scoring and aggregation."""
        a = DecideArgs(req)
        res = a.result()
        cb = CANCEL_FN(cancel) if cancel else CANCEL_FN(0)
        check(lib().lg_decide(self.h, ctypes.byref(a.req), ctypes.byref(res), cb, None))
        return a.answers(laya=self.info["arch"] == ARCH_LAYA)

    def decide_batch(self, reqs: list, cancel=None) -> list:
        """Several requests at once (the states of /v1/decide/batch, src/server.rs:235-319): all
        validated and encoded first, every pass of every request run as GPU batches, one answer
        per request."""
        args = [DecideArgs(r) for r in reqs]
        arr = (DecideRequest * max(1, len(args)))(*[a.req for a in args])
        outs = (DecideResult * max(1, len(args)))(*[a.result() for a in args])
        cb = CANCEL_FN(cancel) if cancel else CANCEL_FN(0)
        check(lib().lg_decide_batch(self.h, arr, len(args), outs, cb, None))
        res = []
        for a, o in zip(args, outs):
            a.res = o
            res.append(a.answers(laya=self.info["arch"] == ARCH_LAYA))
        return res

    def laya_forward(self, inputs, cancel=None):
        """Laya Model::forward (src/models/laya/model.rs:303-416) for [(ids, markers, qtype), ...] as
        one GPU batch -> [(option logits [k], act logits [2]), ...]."""
        keep, arr = [], (LayaInput * max(1, len(inputs)))()
        ks = []
        for i, (ids, markers, qtype) in enumerate(inputs):
            ids, mk = _c(ids, np.int32), _c(markers, np.int32)
            keep += [ids, mk]
            arr[i] = LayaInput(ctypes.cast(ids.ctypes.data, _I32P), ids.size, ctypes.cast(mk.ctypes.data, _I32P), mk.size,
                               int(qtype))
            ks.append(mk.size)
        logits = np.empty(max(1, sum(ks)), np.float32)
        act = np.empty((max(1, len(inputs)), 2), np.float32)
        cb = CANCEL_FN(cancel) if cancel else CANCEL_FN(0)
        check(lib().lg_laya_forward(self.h, arr, len(inputs), _ptr(logits), _ptr(act), cb, None))
        out, at = [], 0
        for i, k in enumerate(ks):
            out.append((logits[at:at + k].copy(), act[i].copy()))
            at += k
        return out

    def decode(self, seq: int, first: int, steps: int, want_logits: bool = False, noalloc: bool = False):
        """Greedy decode (lg_decode); noalloc=True runs lg_decode_noalloc (workspace in the per-GPU
        scratch, no device allocation)."""
        toks = np.empty(steps, dtype=np.int32)
        lg = np.empty((steps, self.info["vocab"]), dtype=np.float32) if want_logits else None
        fn = lib().lg_decode_noalloc if noalloc else lib().lg_decode
        check(fn(self.h, seq, first, steps, _ptr(toks), _ptr(lg)))
        return (toks, lg) if want_logits else toks

    def decode_graph(self, seq: int, first: int, steps: int):
        """lg_decode_graph: the step loop captured into one HIP graph and launched once.
        (tokens, capture + instantiation ms, graph launch ms)."""
        toks = np.empty(steps, dtype=np.int32)
        cap, run = ctypes.c_double(), ctypes.c_double()
        check(lib().lg_decode_graph(self.h, seq, first, steps, _ptr(toks), ctypes.byref(cap), ctypes.byref(run)))
        return toks, cap.value, run.value

    def profile(self, on: bool = True) -> None:
        check(lib().lg_profile_enable(self.h, 1 if on else 0))

    def profile_reset(self) -> None:
        check(lib().lg_profile_reset(self.h))

    def profile_read(self, cls: str) -> dict:
        n, ms, b, f = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        check(lib().lg_profile_read(self.h, cls.encode(), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(b),
                                    ctypes.byref(f)))
        return {"launches": n.value, "ms": ms.value, "bytes": b.value, "flops": f.value}
