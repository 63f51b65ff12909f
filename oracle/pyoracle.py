"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests, the smoke check and the bench's CPU-baseline leg load this module, and only to
check (or time beside) the GPU path's results.  See oracle.h for the reference file:line each function restates.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        P, I, U32, U64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
        sig = {
            "or_layout": (I, [U32, ctypes.POINTER(U64), ctypes.POINTER(U64)]),
            "or_half": (F, [ctypes.c_uint16]),
            "or_decode": (I, [U32, P, U64, P]),
            "or_gguf_open": (P, [P, U64, ctypes.c_char_p, I]),
            "or_gguf_close": (None, [P]),
            "or_gguf_ntensors": (I, [P]),
            "or_gguf_tensor": (I, [P, ctypes.c_char_p, ctypes.POINTER(U32), ctypes.POINTER(U64),
                                   ctypes.POINTER(I), ctypes.POINTER(P), ctypes.POINTER(U64)]),
            "or_gguf_num": (ctypes.c_double, [P, ctypes.c_char_p, ctypes.c_double]),
            "or_gguf_str": (ctypes.c_char_p, [P, ctypes.c_char_p]),
            "or_apply": (None, [P, I, I, P, I, P, I, P]),
            "or_set_scalar_apply": (None, [I]),
            "or_set_blocked": (None, [I]),
            "or_dot": (F, [P, P, I]),
            "or_softmax": (None, [P, I, P]),
            "or_rms": (None, [P, I, I, P, F, F, P]),
            "or_silu": (F, [F]),
            "or_model_load": (P, [P, I, ctypes.c_char_p, I]),
            "or_model_load_streamed": (P, [P, I, ctypes.c_char_p, I]),
            "or_model_free": (None, [P]),
            "or_model_dims": (None, [P, P]),
            "or_model_set_threads": (None, [P, I]),
            "or_cache_new": (P, [P, I]),
            "or_cache_fork": (P, [P, I]),
            "or_cache_free": (None, [P]),
            "or_cache_len": (I, [P]),
            "or_cache_read": (I, [P, I, I, I, P, P]),
            "or_attention": (I, [P, P, P, I, I, I, I, I, I, P]),
            "or_prefill": (I, [P, P, P, I, P, I, P]),
            "or_head": (I, [P, P, I, P, I, P]),
            "or_argmax": (I, [P, I]),
            "or_option_scores": (None, [P, I, F, I, F, P, P, P]),
            "or_confidence": (F, [P, I, I]),
            "or_openthai_load": (P, [P, P, P, I, ctypes.c_char_p, I]),
            "or_openthai_free": (None, [P]),
            "or_openthai_dims": (None, [P, P]),
            "or_openthai_set_threads": (None, [P, I]),
            "or_openthai_forward": (I, [P, P, I, P, I, P]),
            "or_ot_conv_silu": (None, [P, I, I, P, P]),
            "or_ot_gated_delta": (None, [P, P, P, P, P, I, I, I, P]),
            "or_ot_rope": (None, [P, I, I]),
            "or_ot_attention": (None, [P, P, P, I, I, I, I, P]),
            "or_layer_norm": (None, [P, I, I, P, P, F, P]),
            "or_gelu": (F, [F]),
            "or_laya_attention": (None, [P, I, I, I, P, P, I, P]),
            "or_laya_forward": (I, [P, P, I, P, I, I, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(np.asarray(a, dtype=dt))


def layout(kind):
    b, s = ctypes.c_uint64(), ctypes.c_uint64()
    if lib().or_layout(kind, ctypes.byref(b), ctypes.byref(s)):
        raise ValueError(f"unsupported kind {kind}")
    return b.value, s.value


def half(bits: int) -> float:
    return lib().or_half(bits)


def decode(kind: int, raw) -> np.ndarray:
    buf = _c(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw, np.uint8)
    block, size = layout(kind)
    out = np.empty(buf.size // size * block, dtype=np.float32)
    if lib().or_decode(kind, _p(buf), buf.size, _p(out)):
        raise ValueError("decode failed")
    return out


def apply(w, x, bias=None, threads=1) -> np.ndarray:
    w = _c(w, np.float32)
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    rows, cols = w.shape
    m = x.shape[0]
    assert x.shape[1] == cols
    b = None if bias is None else _c(bias, np.float32)
    out = np.empty((m, rows), dtype=np.float32)
    lib().or_apply(_p(w), rows, cols, _p(x), m, _p(b), threads, _p(out))
    return out


def set_scalar_apply(on: bool) -> None:
    lib().or_set_scalar_apply(1 if on else 0)


def set_blocked(on: bool) -> None:
    """Cache-blocked apply and eight-wide attention: the same bits as the reference loop order,
    several times faster on long inputs (the full-depth parity tests use it)."""
    lib().or_set_blocked(1 if on else 0)


def dot(a, b) -> float:
    a, b = _c(a, np.float32), _c(b, np.float32)
    return lib().or_dot(_p(a), _p(b), a.size)


def softmax(x) -> np.ndarray:
    x = _c(x, np.float32)
    p = np.empty_like(x)
    lib().or_softmax(_p(x), x.size, _p(p))
    return p


def rms(x, w, offset=0.0, eps=1e-5) -> np.ndarray:
    x, w = _c(x, np.float32), _c(w, np.float32)
    rows = x.size // w.size
    y = np.empty_like(x)
    lib().or_rms(_p(x), rows, w.size, _p(w), offset, eps, _p(y))
    return y


def silu(v: float) -> float:
    return lib().or_silu(v)


def option_scores(logits, temperature=1.0, abstain=None):
    z = _c(logits, np.float32)
    p, lp, ab = np.empty_like(z), np.empty_like(z), ctypes.c_float()
    lib().or_option_scores(_p(z), z.size, 0.0 if abstain is None else abstain, 0 if abstain is None else 1,
                           temperature, _p(p), _p(lp), ctypes.byref(ab))
    return p, lp, ab.value


def confidence(p, f64=False) -> float:
    p = _c(p, np.float32)
    return lib().or_confidence(_p(p), p.size, 1 if f64 else 0)


class Gguf:
    def __init__(self, data):
        self.buf = _c(np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data,
                      np.uint8)
        err = ctypes.create_string_buffer(256)
        self.h = lib().or_gguf_open(_p(self.buf), self.buf.size, err, 256)
        if not self.h:
            raise ValueError(err.value.decode())

    def tensor(self, name):
        kind, nd, data, n = ctypes.c_uint32(), ctypes.c_int(), ctypes.c_void_p(), ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 4)()
        if lib().or_gguf_tensor(self.h, name.encode(), ctypes.byref(kind), dims, ctypes.byref(nd),
                                ctypes.byref(data), ctypes.byref(n)):
            raise KeyError(name)
        return kind.value, [dims[i] for i in range(nd.value)], ctypes.string_at(data, n.value)

    def offset(self, name) -> int:
        """Byte offset of a tensor's data inside the buffer (to patch bytes in tests)."""
        kind, nd, data, n = ctypes.c_uint32(), ctypes.c_int(), ctypes.c_void_p(), ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 4)()
        if lib().or_gguf_tensor(self.h, name.encode(), ctypes.byref(kind), dims, ctypes.byref(nd),
                                ctypes.byref(data), ctypes.byref(n)):
            raise KeyError(name)
        return data.value - self.buf.ctypes.data

    def num(self, key, default=0.0):
        return lib().or_gguf_num(self.h, key.encode(), default)

    def str(self, key):
        return lib().or_gguf_str(self.h, key.encode()).decode()

    def ntensors(self):
        return lib().or_gguf_ntensors(self.h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_gguf_close(self.h)
            self.h = None


class Model:
    """The assembled decoder on the CPU: prefill with an f32 K/V cache, head, argmax."""

    def __init__(self, gguf: Gguf, threads: int = 4, streamed: bool = False):
        """streamed=True decodes each layer's weights only while it runs (or_model_load_streamed):
        one layer of F32 weights resident instead of the whole model, the same results."""
        self.g = gguf
        err = ctypes.create_string_buffer(256)
        load = lib().or_model_load_streamed if streamed else lib().or_model_load
        self.h = load(gguf.h, threads, err, 256)
        if not self.h:
            raise ValueError(err.value.decode())
        dims = np.zeros(8, dtype=np.int32)
        lib().or_model_dims(self.h, _p(dims))
        (self.L, self.d, self.hq, self.hkv, self.hd, self.f, self.V, self.ctx) = (int(v) for v in dims)

    def set_threads(self, n: int) -> None:
        lib().or_model_set_threads(self.h, n)

    def cache(self, capacity: int | None = None) -> "Cache":
        return Cache(self, capacity or self.ctx)

    def prefill(self, cache: "Cache", ids, gather) -> np.ndarray:
        ids = _c(ids, np.int32)
        gather = _c(gather, np.int32)
        out = np.empty((gather.size, self.d), dtype=np.float32)
        if lib().or_prefill(self.h, cache.h, _p(ids), ids.size, _p(gather), gather.size, _p(out)):
            raise ValueError("oracle prefill rejected its input")
        return out

    def head(self, hidden, vocab_ids=None) -> np.ndarray:
        hidden = _c(hidden, np.float32).reshape(-1, self.d)
        vid = None if vocab_ids is None else _c(vocab_ids, np.int32)
        nv = self.V if vid is None else vid.size
        out = np.empty((hidden.shape[0], nv), dtype=np.float32)
        if lib().or_head(self.h, _p(hidden), hidden.shape[0], _p(vid), nv, _p(out)):
            raise ValueError("oracle head rejected its input")
        return out

    def forward(self, ids, positions, vocab_ids=None) -> np.ndarray:
        """Full recompute over `ids` (Model::forward): logits at `positions`."""
        c = self.cache(len(ids))
        return self.head(self.prefill(c, ids, positions), vocab_ids)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_model_free(self.h)
            self.h = None


class Cache:
    def __init__(self, model: Model, capacity: int, handle=None):
        self.model = model
        self.h = handle or lib().or_cache_new(model.h, capacity)

    def fork(self, ntokens: int) -> "Cache":
        return Cache(self.model, 0, lib().or_cache_fork(self.h, ntokens))

    def __len__(self):
        return lib().or_cache_len(self.h)

    def read(self, layer: int, pos0: int, n: int):
        """(K, V) rows of positions [pos0, pos0 + n) of one layer, f32 [n][hkv*hd]."""
        w = self.model.hkv * self.model.hd
        k = np.empty((n, w), np.float32)
        v = np.empty((n, w), np.float32)
        if lib().or_cache_read(self.h, layer, pos0, n, _p(k), _p(v)):
            raise ValueError("cache read outside the cached positions")
        return k, v

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_cache_free(self.h)
            self.h = None


def attention(q, k, v, pos0, hq, hkv, threads=1) -> np.ndarray:
    """Causal GQA attention (src/models/openthai/model.rs:276-294) of query rows q [n][hq*hd] at
    positions pos0.. over rotated keys/values k, v [pos0+n][hkv*hd]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    n, hd = q.shape[0], q.shape[1] // hq
    assert k.shape == v.shape == (pos0 + n, hkv * hd)
    out = np.empty_like(q)
    if lib().or_attention(_p(q), _p(k), _p(v), n, pos0, hq, hkv, hd, threads, _p(out)):
        raise ValueError("attention: bad shape")
    return out


def argmax(v) -> int:
    v = _c(v, np.float32)
    return lib().or_argmax(_p(v), v.size)


# ---- OpenThai-SystemOne (openthai.c) ----

def openthai_config(gguf: Gguf) -> dict:
    """Dimensions and layer kinds from the openthai.config JSON (src/models/openthai/model.rs:97-126)."""
    import json
    cfg = json.loads(gguf.str("openthai.config"))
    c = cfg["text_config"]
    full = [1 if t == "full_attention" else 0 for t in c["layer_types"][: int(c["num_hidden_layers"])]]
    return {"d": int(c["hidden_size"]), "f": int(c["intermediate_size"]), "L": int(c["num_hidden_layers"]),
            "hq": int(c["num_attention_heads"]), "hkv": int(c["num_key_value_heads"]),
            "nh": int(c["linear_num_value_heads"]), "V": int(c["vocab_size"]), "full": full,
            "answer": int(cfg["answer_token_id"]),
            "max_tokens": int(gguf.num("openthai.context_length", 4096)),
            "max_state": int(gguf.num("openthai.state_length", 2048))}


class OpenThai:
    """The OpenThai text tower on the CPU: Model::forward -> slot logits [npos][256]."""

    def __init__(self, gguf: Gguf, threads: int = 4):
        self.g = gguf
        self.cfg = openthai_config(gguf)
        c = self.cfg
        dims = np.array([c["d"], c["f"], c["L"], c["hq"], c["hkv"], c["nh"], c["V"]], dtype=np.int32)
        self._full = np.array(c["full"], dtype=np.int32)
        err = ctypes.create_string_buffer(256)
        self.h = lib().or_openthai_load(gguf.h, _p(dims), _p(self._full), threads, err, 256)
        if not self.h:
            raise ValueError(err.value.decode())
        self.d, self.V, self.L = c["d"], c["V"], c["L"]

    def set_threads(self, n: int) -> None:
        lib().or_openthai_set_threads(self.h, n)

    def forward(self, ids, positions) -> np.ndarray:
        ids, pos = _c(ids, np.int32), _c(positions, np.int32)
        out = np.empty((pos.size, 256), dtype=np.float32)
        if lib().or_openthai_forward(self.h, _p(ids), ids.size, _p(pos), pos.size, _p(out)):
            raise ValueError("invalid OpenThai token sequence")
        return out

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.or_openthai_free(self.h)
            self.h = None


def ot_conv_silu(raw, conv) -> np.ndarray:
    raw, conv = _c(raw, np.float32), _c(conv, np.float32)
    s, ch = raw.shape
    out = np.empty_like(raw)
    lib().or_ot_conv_silu(_p(raw), s, ch, _p(conv), _p(out))
    return out


def ot_gated_delta(qkv, a, b, alog, dt, threads=1) -> np.ndarray:
    qkv, a, b = _c(qkv, np.float32), _c(a, np.float32), _c(b, np.float32)
    alog, dt = _c(alog, np.float32), _c(dt, np.float32)
    s, nh = a.shape
    out = np.empty((s, nh * 128), dtype=np.float32)
    lib().or_ot_gated_delta(_p(qkv), _p(a), _p(b), _p(alog), _p(dt), s, nh, threads, _p(out))
    return out


def ot_rope(buf) -> np.ndarray:
    buf = _c(buf, np.float32).copy()
    s, heads = buf.shape[0], buf.shape[1] // 256
    lib().or_ot_rope(_p(buf), s, heads)
    return buf


def ot_attention(q, k, v, threads=1) -> np.ndarray:
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    s, hq, hkv = q.shape[0], q.shape[1] // 256, k.shape[1] // 256
    out = np.empty_like(q)
    lib().or_ot_attention(_p(q), _p(k), _p(v), s, hq, hkv, threads, _p(out))
    return out


# ---- Laya encoder (laya.c) ----

class _Ln(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("b", ctypes.c_void_p), ("eps", ctypes.c_float)]


class _Lin(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("b", ctypes.c_void_p), ("rows", ctypes.c_int), ("cols", ctypes.c_int)]


class _LayaLayer(ctypes.Structure):
    _fields_ = [("n1", _Ln), ("n2", _Ln), ("qkv", _Lin), ("wo", _Lin), ("wi", _Lin), ("down", _Lin),
                ("has_n1", ctypes.c_int), ("full", ctypes.c_int)]


class _Laya(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int), ("d", ctypes.c_int), ("hd", ctypes.c_int), ("vocab", ctypes.c_int),
                ("max_len", ctypes.c_int), ("threads", ctypes.c_int), ("emb", ctypes.c_void_p),
                ("embnorm", _Ln), ("finalnorm", _Ln), ("scorenorm", _Ln),
                ("trunk", ctypes.POINTER(_LayaLayer)), ("head", ctypes.POINTER(_LayaLayer)),
                ("type_emb", ctypes.c_void_p), ("score1", _Lin), ("score2", _Lin), ("act1", _Lin), ("act2", _Lin),
                ("cos_full", ctypes.c_void_p), ("sin_full", ctypes.c_void_p), ("cos_slide", ctypes.c_void_p),
                ("sin_slide", ctypes.c_void_p)]


class Laya:
    """The Laya encoder on the CPU (src/models/laya/model.rs): the layers are resolved from the
    GGUF's ggmlc.graph_spec here, as model.rs:60-291 does, and the forward runs in laya.c."""

    def __init__(self, gguf: Gguf, threads: int = 4):
        import json
        self.g, self.keep = gguf, []
        graph = json.loads(gguf.str("ggmlc.graph_spec"))
        self.graph = graph
        names = {int(k): v["name"] for k, v in graph["tensors"].items()}
        nodes = graph["nodes"]
        have = lambda n: self._has(n)  # noqa: E731
        L = 0
        while have(f"qkv.{L}.weight"):
            L += 1
        H = 0
        while have(f"head_qkv.{H}.weight"):
            H += 1
        if L == 0 or L > 64 or H != 2:
            raise ValueError("unsupported Laya encoder/head layout")
        kind, dims, _ = gguf.tensor("tok_emb.weight")
        d, vocab = dims[0], dims[1]
        hd = gguf.tensor("cos_full")[1][0]
        attns = [n for n in nodes if n["opcode"] == 74]
        if len(attns) != L + H:
            raise ValueError("unexpected attention graph")
        fullmask = attns[0]["inputs"][-1]

        def floats(name):
            k, dm, raw = gguf.tensor(name)
            a = decode(k, raw)
            self.keep.append(a)
            return a

        def ptr(a):
            return None if a is None else a.ctypes.data

        def linear(key):
            weight = key + ".weight"
            k, dm, raw = gguf.tensor(weight)
            cols, rows = dm[0], (dm[1] if len(dm) > 1 else 1)
            node = next((n for n in nodes if n["opcode"] == 29 and n["inputs"] and names[n["inputs"][0]] == weight), None)
            if node is None:
                raise ValueError(f"graph lacks linear {key}")
            biases = [names[node["inputs"][2]]] if len(node["inputs"]) > 2 else []
            for n in nodes:
                if n["opcode"] == 200 and n["inputs"][0] == node["outputs"][0]:
                    biases.append(names[n["inputs"][1]])
            b = None
            if biases:
                b = np.zeros(rows, np.float32)
                for bn in biases:
                    b = (b + floats(bn)).astype(np.float32)
                self.keep.append(b)
            w = floats(weight)
            return _Lin(ptr(w), ptr(b), rows, cols), (rows, cols)

        def norm(i):
            key = "layer_norm" if i == 0 else f"layer_norm_{i}"
            node = next((n for n in nodes if n.get("name") == key and n["opcode"] == 201), None)
            if node is None:
                raise ValueError(f"missing {key}")
            ins = node["inputs"]
            w = floats(names[ins[1]]) if len(ins) > 1 else None
            b = floats(names[ins[2]]) if len(ins) > 2 else None
            eps = float(np.float32(node["attributes"]["eps"]))
            if not 0 < eps < 0.1:
                raise ValueError("invalid layer norm epsilon")
            return _Ln(ptr(w), ptr(b), eps)

        trunk = (_LayaLayer * L)()
        for i in range(L):
            qkv, _ = linear(f"qkv.{i}")
            wo, _ = linear(f"wo.{i}")
            wi, _ = linear(f"mlp_wi.{i}")
            down, _ = linear(f"mlp_wo.{i}")
            trunk[i] = _LayaLayer(norm(2 * i) if i else _Ln(None, None, 1e-5), norm(2 * i + 1), qkv, wo, wi, down,
                                  1 if i else 0, 1 if attns[i]["inputs"][-1] == fullmask else 0)
        head = (_LayaLayer * 2)()
        for i in range(2):
            qkv, _ = linear(f"head_qkv.{i}")
            wo, _ = linear(f"head_wo.{i}")
            wi, _ = linear(f"head_fc1.{i}")
            down, _ = linear(f"head_fc2.{i}")
            head[i] = _LayaLayer(norm(2 * L + 1 + 2 * i), norm(2 * L + 2 + 2 * i), qkv, wo, wi, down, 1, 1)
        self.keep += [trunk, head]
        emb = floats("tok_emb.weight")
        m = _Laya(L, d, hd, vocab, int(gguf.num("laya.max_len", 512)), threads, ptr(emb), norm(0), norm(2 * L),
                  norm(2 * L + 1 + 2 * H), trunk, head, ptr(floats("type_emb.weight")), linear("scorer_fc1")[0],
                  linear("scorer_fc2")[0], linear("act_fc1")[0], linear("act_fc2")[0], ptr(floats("cos_full")),
                  ptr(floats("sin_full")), ptr(floats("cos_slide")), ptr(floats("sin_slide")))
        self.m = m
        self.L, self.d, self.hd, self.V = L, d, hd, vocab
        self.full = [bool(trunk[i].full) for i in range(L)]

    def _has(self, name):
        try:
            self.g.tensor(name)
            return True
        except KeyError:
            return False

    def set_threads(self, n: int) -> None:
        self.m.threads = n

    def forward(self, ids, markers, qtype):
        """Model::forward(ids, markers, qtype) -> (option logits [k], act logits [2])."""
        ids, mk = _c(ids, np.int32), _c(markers, np.int32)
        logits, act = np.empty(mk.size, np.float32), np.empty(2, np.float32)
        rc = lib().or_laya_forward(ctypes.byref(self.m), _p(ids), ids.size, _p(mk), mk.size, int(qtype), _p(logits),
                                   _p(act))
        if rc == -1:
            raise ValueError("invalid inference input shape")
        if rc == -2:
            raise ValueError("token ID out of range")
        if rc == -3:
            raise ValueError("non-finite model output")
        return logits, act


def layer_norm(x, w=None, b=None, eps=1e-5):
    x = _c(x, np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    lib().or_layer_norm(_p(x), x.size // d, d, _p(None if w is None else _c(w, np.float32)),
                        _p(None if b is None else _c(b, np.float32)), eps, _p(y))
    return y


def gelu(v: float) -> float:
    return lib().or_gelu(v)


def laya_attention(qkv, hd, cos=None, sin=None, window=-1):
    qkv = _c(qkv, np.float32)
    s, d = qkv.shape[0], qkv.shape[1] // 3
    out = np.empty((s, d), np.float32)
    cs = None if cos is None else _c(cos, np.float32)
    sn = None if sin is None else _c(sin, np.float32)
    lib().or_laya_attention(_p(qkv), s, d, hd, _p(cs), _p(sn), window, _p(out))
    return out
