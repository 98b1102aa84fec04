"""ctypes front end of the CPU oracle (oracle/ref_cpu.cpp -> oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this module, and only as the checker (or, in bench.py, as the timed CPU
baseline of the reference's path). The product never routes through it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

P, I64, I32, F32 = C.c_void_p, C.c_int64, C.c_int32, C.c_float


class Proj(C.Structure):
    _fields_ = [("kind", I32), ("pad", I32), ("rows", I64), ("cols", I64), ("q", P), ("scales", P), ("f", P)]


class Config(C.Structure):
    _fields_ = [("hidden", I64), ("layers", I64), ("heads", I64), ("kv_heads", I64), ("inter", I64),
                ("vocab", I64), ("eps", F32), ("theta", F32), ("window", I64)]


class Layer(C.Structure):
    _fields_ = [("attn_norm", P), ("wq", Proj), ("wk", Proj), ("wv", Proj), ("wo", Proj), ("ffn_norm", P),
                ("w1", Proj), ("w2", Proj), ("w3", Proj)]


class Entry(C.Structure):
    _fields_ = [("pos", I64), ("start", I64), ("table_off", I64), ("table_len", I64)]


_SIGS_SAMPLING = {
    "orc_rng_new": (C.c_uint64, [C.c_uint64]),
    "orc_rng_next_u64": (C.c_uint64, [C.POINTER(C.c_uint64)]),
    "orc_rng_next_f32": (F32, [C.POINTER(C.c_uint64)]),
    "orc_sample": (I64, [P, I64, F32, F32, I64, C.POINTER(C.c_uint64)]),
}
_SIGS = {
    "orc_set_threads": (None, [C.c_int]),
    "orc_threads": (C.c_int, []),
    "orc_force_portable": (None, [C.c_int]),
    "orc_have_avx2": (C.c_int, []),
    "orc_quantize_rows_i8": (None, [P, I64, I64, P, P]),
    "orc_dot_i8": (F32, [P, P, I64]),
    "orc_dot": (F32, [P, P, I64]),
    "orc_matvec_i8": (None, [P, P, P, P, I64, I64]),
    "orc_matmat_i8": (None, [P, P, P, P, I64, I64, I64]),
    "orc_matvec_f32": (None, [P, P, P, I64, I64]),
    "orc_rope_table": (None, [I64, I64, F32, P, P]),
    "orc_softmax": (None, [P, I64]),
    "orc_rms_norm": (None, [P, P, I64, F32]),
    "orc_argmax": (I64, [P, I64]),
    "orc_paged_attention": (None, [P, P, P, I64, I64, I64, I64, I64, I64, P, P, I64, I64]),
    "orc_model_create": (P, [C.POINTER(Config), P, P, C.POINTER(Proj)]),
    "orc_model_set_layer": (None, [P, I64, C.POINTER(Layer)]),
    "orc_model_destroy": (None, [P]),
    "orc_decode_batch": (None, [P, P, P, P, P, P, I64, P, I64, I64, P]),
    "orc_prefill": (None, [P, P, I64, I64, P, I64, P, I64, I64, I64, P]),
}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in {**_SIGS, **_SIGS_SAMPLING}.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def set_threads(n: int):
    lib().orc_set_threads(int(n))


def threads() -> int:
    return int(lib().orc_threads())


def quantize_rows_i8(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quantize_rows_i8(_p(w), rows, cols, _p(q), _p(s))
    return q, s


def dot_i8(w, x) -> float:
    w = np.ascontiguousarray(w, np.int8)
    x = np.ascontiguousarray(x, np.float32)
    return float(lib().orc_dot_i8(_p(w), _p(x), w.size))


def dot(a, b) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return float(lib().orc_dot(_p(a), _p(b), a.size))


def matvec_i8(q, s, x):
    rows, cols = q.shape
    out = np.empty(rows, np.float32)
    lib().orc_matvec_i8(_p(out), _p(np.ascontiguousarray(x, np.float32)), _p(q), _p(s), rows, cols)
    return out


def matmat_i8(q, s, x_br):
    rows, cols = q.shape
    x_br = np.ascontiguousarray(x_br, np.float32)
    batch = x_br.shape[0]
    out = np.empty((rows, batch), np.float32)
    lib().orc_matmat_i8(_p(out), _p(x_br), _p(q), _p(s), batch, rows, cols)
    return out


def matvec_f32(w, x):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.empty(rows, np.float32)
    lib().orc_matvec_f32(_p(out), _p(np.ascontiguousarray(x, np.float32)), _p(w), rows, cols)
    return out


def rope_table(pos: int, hd: int, theta: float):
    c = np.empty(hd // 2, np.float32)
    s = np.empty(hd // 2, np.float32)
    lib().orc_rope_table(pos, hd, theta, _p(c), _p(s))
    return c, s


def softmax(x):
    x = np.array(x, np.float32)
    lib().orc_softmax(_p(x), x.size)
    return x


def rms_norm(x, w, eps):
    x = np.array(x, np.float32)
    lib().orc_rms_norm(_p(x), _p(np.ascontiguousarray(w, np.float32)), x.size, eps)
    return x


def argmax(x) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().orc_argmax(_p(x), x.size))


def flatten_tables(tables):
    off, ln, flat = [], [], []
    for t in tables:
        off.append(len(flat))
        ln.append(len(t))
        flat.extend(t)
    return (np.asarray(off, np.int64), np.asarray(ln, np.int64),
            np.ascontiguousarray(np.asarray(flat if flat else [0], np.int32)))


def paged_attention(q, kv, layout, heads, entries, tables, layer):
    """q: [n][heads*hd]; layout = (layers, blocks, block_size, kv_heads, hd); entries = [(pos,start)]."""
    nl, nb, bs, hkv, hd = layout
    n = len(entries)
    off, ln, flat = flatten_tables(tables)
    ent = (Entry * max(n, 1))()
    for i, (pos, start) in enumerate(entries):
        ent[i] = Entry(pos, start, off[i], ln[i])
    q = np.ascontiguousarray(q, np.float32)
    out = np.zeros((n, heads * hd), np.float32)
    kv = np.ascontiguousarray(kv, np.float32)
    lib().orc_paged_attention(_p(out), _p(q), _p(kv), nl, nb, bs, hkv, hd, heads, C.addressof(ent), _p(flat), n,
                              layer)
    return out


class OracleModel:
    """The reference's forward pass (run_layers_batch et al.) over host arrays. `weights` has
    the layout produced by pia.synth_weights / the fixture loader."""

    def __init__(self, cfg, weights: dict):
        self.cfg = cfg
        self._keep = []
        c = Config(cfg.hidden, cfg.layers, cfg.heads, cfg.kv_heads, cfg.inter, cfg.vocab, cfg.rms_eps, cfg.rope_theta,
                   -1 if cfg.attention_window is None else cfg.attention_window)
        self._cfg = c
        emb = self._k(np.ascontiguousarray(weights["embed"], np.uint16))
        fn = self._k(np.ascontiguousarray(weights["final_norm"], np.float32))
        lm = self._proj(weights["lm_head"])
        self.h = lib().orc_model_create(C.byref(c), _p(emb), _p(fn), C.byref(lm))
        for i, lw in enumerate(weights["layers"]):
            L = Layer(_p(self._k(np.ascontiguousarray(lw["attn_norm"], np.float32))), self._proj(lw["wq"]),
                      self._proj(lw["wk"]), self._proj(lw["wv"]), self._proj(lw["wo"]),
                      _p(self._k(np.ascontiguousarray(lw["ffn_norm"], np.float32))), self._proj(lw["w1"]),
                      self._proj(lw["w2"]), self._proj(lw["w3"]))
            lib().orc_model_set_layer(self.h, i, C.byref(L))

    def _k(self, a):
        self._keep.append(a)
        return a

    def _proj(self, p) -> Proj:
        if isinstance(p, tuple):
            q = self._k(np.ascontiguousarray(p[0], np.int8))
            s = self._k(np.ascontiguousarray(p[1], np.float32))
            return Proj(1, 0, q.shape[0], q.shape[1], _p(q), _p(s), None)
        w = self._k(np.ascontiguousarray(p, np.float32))
        return Proj(0, 0, w.shape[0], w.shape[1], None, None, _p(w))

    def __del__(self):
        try:
            if self.h:
                lib().orc_model_destroy(self.h)
                self.h = None
        except Exception:
            pass

    def decode(self, tokens, positions, tables, kv, num_blocks, block_size):
        b = len(tokens)
        tok = np.ascontiguousarray(np.asarray(tokens, np.uint32))
        pos = np.ascontiguousarray(np.asarray(positions, np.int64))
        off, ln, flat = flatten_tables(tables)
        logits = np.empty((b, self.cfg.vocab), np.float32)
        lib().orc_decode_batch(self.h, _p(tok), _p(pos), _p(off), _p(ln), _p(flat), b, _p(kv), num_blocks, block_size,
                               _p(logits))
        return logits

    def prefill(self, tokens, start_pos, table, kv, num_blocks, block_size, chunk=32):
        tok = np.ascontiguousarray(np.asarray(tokens, np.uint32))
        t = np.ascontiguousarray(np.asarray(table if len(table) else [0], np.int32))
        logits = np.empty(self.cfg.vocab, np.float32)
        lib().orc_prefill(self.h, _p(tok), tok.size, start_pos, _p(t), len(table), _p(kv), num_blocks, block_size,
                          chunk, _p(logits))
        return logits


def kv_floats(cfg, num_blocks: int, block_size: int) -> int:
    return cfg.layers * num_blocks * block_size * cfg.kv_heads * 2 * cfg.head_dim


class Rng:
    """Rng (src/sampling.rs:15-41) over the oracle's restatement."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(lib().orc_rng_new(seed))

    def next_u64(self) -> int:
        return int(lib().orc_rng_next_u64(C.byref(self.state)))

    def next_f32(self) -> float:
        return float(lib().orc_rng_next_f32(C.byref(self.state)))


class Sampler:
    """Sampler (src/sampling.rs:43-138) over the oracle's restatement."""

    def __init__(self, temperature: float, top_p: float, top_k: int, seed: int):
        self.temperature, self.top_p, self.top_k = temperature, top_p, top_k
        self.rng = Rng(seed)

    def sample(self, logits) -> int:
        x = np.ascontiguousarray(np.asarray(logits, np.float32))
        return int(lib().orc_sample(_p(x), x.size, self.temperature, self.top_p, self.top_k, C.byref(self.rng.state)))

