"""ctypes binding of libpaged_infer_amd.so (the C ABI declared in include/paged_infer_amd.h).

This is the reference-side binding a Python caller uses; it mirrors the reference's seams:
  - kernel tier:  quantize_rows_i8 / matvec_i8 / matmat_i8 (src/math.rs), Projection::
                  apply_batched (src/model.rs:247-259), PagedAttention::run (src/attention.rs),
                  the per-step KV write (src/model.rs:1093-1107), KvLayout::copy_block
                  (src/memory/layout.rs)
  - memory tier:  KvCacheManager / BlockTable / block_hash (src/memory/*.rs)
  - model tier:   LlamaWeights::decode_batch_into / prefill_batched (src/model.rs:1184-1255)
It never falls back to anything: when the library is missing or no gfx950 device is present,
the calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
import re
import weakref
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIB_PATH = HERE / "libpaged_infer_amd.so"
HEADER = ROOT / "include" / "paged_infer_amd.h"

PIA_OK = 0
PIA_ERR_INVALID, PIA_ERR_HIP, PIA_ERR_OOM, PIA_ERR_NO_DEVICE = 1, 2, 3, 4
SLOTS = {"wq": 0, "wk": 1, "wv": 2, "wo": 3, "w1": 4, "w2": 5, "w3": 6, "lm_head": 7}
NORM_ATTN, NORM_FFN, NORM_FINAL = 0, 1, 2


class PiaError(RuntimeError):
    pass


class KvLayout(C.Structure):
    _fields_ = [("num_layers", C.c_int64), ("num_blocks", C.c_int64), ("block_size", C.c_int64),
                ("num_kv_heads", C.c_int64), ("head_dim", C.c_int64)]


class AttnEntry(C.Structure):
    _fields_ = [("pos", C.c_int32), ("start", C.c_int32), ("table_off", C.c_int32), ("table_len", C.c_int32)]


class Admission(C.Structure):
    _fields_ = [("cached_tokens", C.c_int64), ("reused_blocks", C.c_int64), ("allocated_blocks", C.c_int64)]


class KvmStats(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("inserts", C.c_uint64), ("evictions", C.c_uint64),
                ("tokens_saved", C.c_uint64), ("cow_copies", C.c_uint64), ("available_blocks", C.c_int64),
                ("total_blocks", C.c_int64), ("active_sequences", C.c_int64), ("cached_entries", C.c_int64)]


class Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32), ("reserved", C.c_int32)]


SAMPLING_DTYPE = np.dtype([("temperature", "<f4"), ("top_p", "<f4"), ("top_k", "<i4"), ("reserved", "<i4")])


def sampling_array(params) -> np.ndarray:
    """[(temperature, top_p, top_k), ...] as a pia_sampling array."""
    a = np.zeros(len(params), SAMPLING_DTYPE)
    for i, (t, p, k) in enumerate(params):
        a[i] = (t, p, k, 0)
    return a


def rng_new(seed: int) -> int:
    """Rng::new (src/sampling.rs:20-25): the xorshift64* state for a seed."""
    return int(lib().pia_rng_new(seed))


class SpecGroup(C.Structure):
    _fields_ = [("pos", C.c_int64), ("n_tokens", C.c_int64), ("tokens_off", C.c_int64), ("table_off", C.c_int64),
                ("table_len", C.c_int64)]


class ModelConfig(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("layers", C.c_int64), ("heads", C.c_int64), ("kv_heads", C.c_int64),
                ("inter", C.c_int64), ("vocab", C.c_int64), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("attention_window", C.c_int64)]


P = C.c_void_p
I64, I32, U64, F32 = C.c_int64, C.c_int32, C.c_uint64, C.c_float

_SIGS = {
    "pia_last_error": (C.c_char_p, []),
    "pia_version": (C.c_char_p, []),
    "pia_context_create": (I32, [C.c_int, C.POINTER(P)]),
    "pia_context_destroy": (I32, [P]),
    "pia_context_synchronize": (I32, [P]),
    "pia_context_stream": (P, [P]),
    "pia_malloc": (I32, [P, C.c_size_t, C.POINTER(P)]),
    "pia_free": (I32, [P, P]),
    "pia_memcpy_h2d": (I32, [P, P, P, C.c_size_t]),
    "pia_memcpy_d2h": (I32, [P, P, P, C.c_size_t]),
    "pia_quantize_rows_i8": (I32, [P, I64, I64, P, P]),
    "pia_quantize_rows_i8_dev": (I32, [P, P, I64, I64, P, P, P]),
    "pia_matvec_i8": (I32, [P, P, P, P, P, I64, I64]),
    "pia_matvec_i8_dev": (I32, [P, P, P, P, P, I64, I64, P]),
    "pia_matmat_i8": (I32, [P, P, P, P, P, I64, I64, I64]),
    "pia_matmat_i8_dev": (I32, [P, P, P, P, P, I64, I64, I64, P]),
    "pia_qlinear_apply_dev": (I32, [P, P, P, P, P, I64, I64, I64, P]),
    "pia_qlinear_apply_noalloc_dev": (I32, [P, P, P, P, P, I64, I64, I64, P]),
    "pia_qlinear_apply": (I32, [P, P, P, P, P, I64, I64, I64]),
    "pia_paged_attention_dev": (I32, [P, P, P, P, C.POINTER(KvLayout), I64, P, P, I64, I64, P]),
    "pia_kv_write_dev": (I32, [P, P, C.POINTER(KvLayout), P, P, P, P, I64, I64, P]),
    "pia_kv_copy_block_dev": (I32, [P, P, C.POINTER(KvLayout), I64, I64, P]),
    "pia_argmax_dev": (I32, [P, P, P, I64, I64, P]),
    "pia_block_hash": (U64, [U64, P, I64]),
    "pia_kvm_create": (I32, [I64, I64, I32, C.POINTER(P)]),
    "pia_kvm_destroy": (I32, [P]),
    "pia_kvm_admit": (I32, [P, I64, P, I64, U64, C.POINTER(I32), C.POINTER(P), C.POINTER(Admission)]),
    "pia_kvm_publish": (I32, [P, P, C.POINTER(I64)]),
    "pia_kvm_append_block": (I32, [P, I64, P, U64, C.POINTER(I32)]),
    "pia_kvm_fork": (I32, [P, P, I64, U64, C.POINTER(P)]),
    "pia_kvm_ensure_writable": (I32, [P, I64, P, I64, P, P, C.POINTER(KvLayout), C.POINTER(I32)]),
    "pia_kvm_touch": (I32, [P, I64, U64]),
    "pia_kvm_release": (I32, [P, I64]),
    "pia_kvm_clear": (I32, [P]),
    "pia_kvm_stats_get": (I32, [P, C.POINTER(KvmStats)]),
    "pia_kvm_ref_count": (I32, [P, I64, C.POINTER(I64)]),
    "pia_table_create": (I32, [C.POINTER(P)]),
    "pia_table_destroy": (I32, [P]),
    "pia_table_len": (I64, [P]),
    "pia_table_blocks": (I32, [P, P]),
    "pia_table_append": (I32, [P, I64]),
    "pia_table_slot": (I32, [P, I64, C.POINTER(U64), C.POINTER(I32), C.POINTER(I32)]),
    "pia_model_create": (I32, [P, C.POINTER(ModelConfig), C.POINTER(P)]),
    "pia_model_destroy": (I32, [P]),
    "pia_model_set_embedding": (I32, [P, P]),
    "pia_model_set_norm": (I32, [P, I64, I32, P]),
    "pia_model_set_proj_i8": (I32, [P, I64, I32, P, P]),
    "pia_model_set_proj_f32": (I32, [P, I64, I32, P]),
    "pia_model_weight_bytes": (I64, [P]),
    "pia_model_get_config": (I32, [P, C.POINTER(ModelConfig)]),
    "pia_rng_new": (U64, [U64]),
    "pia_sample_dev": (I32, [P, P, P, I64, I64, I64, P, P, I32, P]),
    "pia_model_sample": (I32, [P, P, P, I64, I32, P]),
    "pia_prompt_lookup_draft": (I32, [P, I64, I64, I64, I64, P, C.POINTER(I64)]),
    "pia_verify_greedy": (I32, [P, I64, P, I64, C.POINTER(I64), C.POINTER(C.c_uint32)]),
    "pia_model_verify_groups": (I32, [P, P, I64, P, P, I64, P, P, P, C.POINTER(I64)]),
    "pia_hf_config_read": (I32, [C.c_char_p, C.POINTER(ModelConfig)]),
    "pia_model_load_safetensors": (I32, [P, C.c_char_p, I32, I32]),
    "pia_model_kv_alloc": (I32, [P, I64, I64]),
    "pia_model_kv": (I32, [P, C.POINTER(P), C.POINTER(KvLayout)]),
    "pia_model_decode": (I32, [P, P, P, P, P, P, I64, P, P]),
    "pia_model_prefill": (I32, [P, P, I64, I64, P, I64, P, P]),
    "pia_model_profile": (I32, [P, I32]),
    "pia_model_set_decode_path": (I32, [P, I32]),
    "pia_model_decode_path_used": (I32, [P]),
    "pia_model_last_upload": (I32, [P, P, P, P]),
    "pia_model_last_shared": (I32, [P, P, P]),
    "pia_model_profile_get": (I32, [P, P, P, P, I32]),
    "pia_model_bench_class": (I32, [P, I32, I64, I32, C.POINTER(C.c_double), C.POINTER(I64)]),
    "pia_bench_projection": (I32, [P, I64, I64, I64, I32, I32, C.POINTER(C.c_double), C.POINTER(I64)]),
    "pia_synth_normal": (I32, [U64, U64, F32, P, I64]),
    "pia_f32_to_bf16": (I32, [P, P, I64]),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function the C ABI header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(pia_[a-z0-9_]+)\s*\(", text)))


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise PiaError(f"{LIB_PATH} is not built; run `make -C paged-infer_amd` (or __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int):
    if status != PIA_OK:
        raise PiaError(f"status {status}: {lib().pia_last_error().decode()}")


def ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the C ABI must be C-contiguous"
    return a.ctypes.data


# ------------------------------------------------------------------------------------------
# Host-only helpers (no device needed).
# ------------------------------------------------------------------------------------------
def quantize_rows_i8(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    check(lib().pia_quantize_rows_i8(ptr(w), rows, cols, ptr(q), ptr(s)))
    return q, s


def prompt_lookup_draft(context, k: int, min_ngram: int = 2, max_ngram: int = 8) -> list[int]:
    """PromptLookupDrafter::draft (src/speculative.rs:71-101); the engine's drafter is (2, 8)."""
    c = np.ascontiguousarray(np.asarray(context, np.uint32))
    out = np.zeros(max(k, 1), np.uint32)
    n = I64()
    check(lib().pia_prompt_lookup_draft(ptr(c) if c.size else None, c.size, k, min_ngram, max_ngram, ptr(out),
                                        C.byref(n)))
    return [int(t) for t in out[:n.value]]


def verify_greedy(drafts, model_argmax) -> tuple[list[int], int]:
    """verify_greedy (src/speculative.rs:204-223): (accepted drafts, corrected token)."""
    d = np.ascontiguousarray(np.asarray(drafts, np.uint32))
    m = np.ascontiguousarray(np.asarray(model_argmax, np.uint32))
    a, corr = I64(), C.c_uint32()
    check(lib().pia_verify_greedy(ptr(d) if d.size else None, d.size, ptr(m) if m.size else None, m.size,
                                  C.byref(a), C.byref(corr)))
    return [int(t) for t in d[:a.value]], int(corr.value)


def synth_normal(seed: int, stream: int, n: int, std: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().pia_synth_normal(seed, stream, std, ptr(out), n))
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    check(lib().pia_f32_to_bf16(ptr(x), ptr(out), x.size))
    return out


def block_hash(parent: int, tokens) -> int:
    t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
    return int(lib().pia_block_hash(parent, ptr(t) if t.size else None, t.size))


# ------------------------------------------------------------------------------------------
# Context and device buffers.
# ------------------------------------------------------------------------------------------
class Context:
    def __init__(self, device: int = 0):
        h = P()
        check(lib().pia_context_create(device, C.byref(h)))
        self.h = h
        self._children = weakref.WeakSet()  # models / buffers that must go before the context

    def close(self):
        if self.h:
            for child in list(self._children):
                child.close()
            lib().pia_context_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self):
        check(lib().pia_context_synchronize(self.h))

    def to_device(self, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = DeviceArray(self, a.shape, a.dtype)
        check(lib().pia_memcpy_h2d(self.h, d.ptr, ptr(a), a.nbytes))
        return d

    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)


class DeviceArray:
    def __init__(self, ctx: Context, shape, dtype):
        self.ctx, self.shape, self.dtype = ctx, tuple(shape), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        h = P()
        check(lib().pia_malloc(ctx.h, max(self.nbytes, 1), C.byref(h)))
        self.ptr = h
        ctx._children.add(self)

    def close(self):
        self.free()

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().pia_memcpy_d2h(self.ctx.h, ptr(out), self.ptr, self.nbytes))
        return out

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(lib().pia_memcpy_h2d(self.ctx.h, self.ptr, ptr(a), a.nbytes))

    def free(self):
        if self.ptr and self.ctx.h:
            lib().pia_free(self.ctx.h, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


SAMPLE_REFERENCE, SAMPLE_EXACT_SUMS = 0, 1


def sample_rows(ctx: Context, logits: np.ndarray, params, rng_state: np.ndarray, draws: int = 1,
                mode: int = SAMPLE_REFERENCE):
    """pia_sample_dev over host logits [n][vocab]: `draws` consecutive samples per row (the
    generator state advancing on the device between them). Returns (tokens [draws][n], final
    rng states)."""
    logits = np.ascontiguousarray(logits, np.float32)
    n, vocab = logits.shape
    dl, dp = ctx.to_device(logits), ctx.to_device(sampling_array(params))
    dr = ctx.to_device(np.ascontiguousarray(rng_state, np.uint64))
    do = ctx.empty((n,), np.int32)
    outs = []
    for _ in range(draws):
        check(lib().pia_sample_dev(ctx.h, do.ptr, dl.ptr, vocab, n, vocab, dp.ptr, dr.ptr, mode, None))
        outs.append(do.numpy())
    states = dr.numpy()
    for d in (dl, dp, dr, do):
        d.free()
    return np.stack(outs), states


BENCH_NORM, BENCH_SWIGLU, BENCH_ADD, BENCH_MFMA = 1, 2, 4, 8


def bench_projection(ctx: "Context", rows: int, cols: int, batch: int = 1, reps: int = 20, flags: int = 0):
    """(microseconds per launch, algorithmic bytes per launch) of one int8 projection shape."""
    us, by = C.c_double(), I64()
    check(lib().pia_bench_projection(ctx.h, rows, cols, batch, reps, flags, C.byref(us), C.byref(by)))
    return us.value, by.value


# ------------------------------------------------------------------------------------------
# Memory tier.
# ------------------------------------------------------------------------------------------
class Table:
    def __init__(self, h=None):
        if h is None:
            h = P()
            check(lib().pia_table_create(C.byref(h)))
        self.h = h

    def __len__(self):
        return int(lib().pia_table_len(self.h))

    def blocks(self) -> list[int]:
        n = len(self)
        out = np.empty(max(n, 1), np.int32)
        check(lib().pia_table_blocks(self.h, ptr(out)))
        return [int(v) for v in out[:n]]

    def append(self, block: int):
        check(lib().pia_table_append(self.h, block))

    def slot(self, i: int):
        h, has, cached = U64(), I32(), I32()
        check(lib().pia_table_slot(self.h, i, C.byref(h), C.byref(has), C.byref(cached)))
        return (int(h.value) if has.value else None), bool(cached.value)

    def __del__(self):
        try:
            if self.h:
                lib().pia_table_destroy(self.h)
                self.h = None
        except Exception:
            pass


class KvCacheManager:
    def __init__(self, total_blocks: int, block_size: int, prefix_cache: bool = True):
        h = P()
        check(lib().pia_kvm_create(total_blocks, block_size, int(prefix_cache), C.byref(h)))
        self.h = h
        self.block_size = block_size

    def __del__(self):
        try:
            if self.h:
                lib().pia_kvm_destroy(self.h)
                self.h = None
        except Exception:
            pass

    def admit(self, seq_id: int, tokens, tick: int):
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        ok, th, info = I32(), P(), Admission()
        check(lib().pia_kvm_admit(self.h, seq_id, ptr(t) if t.size else None, t.size, tick, C.byref(ok), C.byref(th),
                                  C.byref(info)))
        if not ok.value:
            return None
        return Table(th), (info.cached_tokens, info.reused_blocks, info.allocated_blocks)

    def publish(self, table: Table) -> int:
        n = I64()
        check(lib().pia_kvm_publish(self.h, table.h, C.byref(n)))
        return n.value

    def append_block(self, seq_id: int, table: Table, tick: int) -> bool:
        ok = I32()
        check(lib().pia_kvm_append_block(self.h, seq_id, table.h, tick, C.byref(ok)))
        return bool(ok.value)

    def fork(self, parent: Table, child_seq: int, tick: int) -> Table:
        th = P()
        check(lib().pia_kvm_fork(self.h, parent.h, child_seq, tick, C.byref(th)))
        return Table(th)

    def ensure_writable(self, seq_id: int, table: Table, pos: int, ctx: Context | None = None, kv=None,
                        layout: KvLayout | None = None) -> bool:
        copied = I32()
        check(lib().pia_kvm_ensure_writable(self.h, seq_id, table.h, pos, ctx.h if ctx else None, kv,
                                            C.byref(layout) if layout is not None else None, C.byref(copied)))
        return bool(copied.value)

    def touch(self, seq_id: int, tick: int):
        check(lib().pia_kvm_touch(self.h, seq_id, tick))

    def release(self, seq_id: int):
        check(lib().pia_kvm_release(self.h, seq_id))

    def clear(self):
        check(lib().pia_kvm_clear(self.h))

    def stats(self) -> dict:
        s = KvmStats()
        check(lib().pia_kvm_stats_get(self.h, C.byref(s)))
        return {f: getattr(s, f) for f, _ in KvmStats._fields_}

    def ref_count(self, block: int) -> int:
        v = I64()
        check(lib().pia_kvm_ref_count(self.h, block, C.byref(v)))
        return v.value


# ------------------------------------------------------------------------------------------
# Model tier.
# ------------------------------------------------------------------------------------------
@dataclass
class LlamaConfig:
    """LlamaConfig (src/model.rs:15-35)."""
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    inter: int
    vocab: int
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    attention_window: int | None = None

    @property
    def head_dim(self):
        return self.hidden // self.heads

    @classmethod
    def from_hf_config(cls, path) -> "LlamaConfig":
        """LlamaConfig::from_hf_config (src/model.rs:57-95): absent fields keep the TinyLlama
        defaults; raises PiaError for a missing or malformed file."""
        c = ModelConfig()
        check(lib().pia_hf_config_read(str(path).encode(), C.byref(c)))
        return cls._from_c(c)

    @classmethod
    def beside_checkpoint(cls, model_path) -> "LlamaConfig":
        """LlamaConfig::beside_checkpoint (src/model.rs:97-102): config.json next to the
        checkpoint, else the defaults."""
        try:
            return cls.from_hf_config(Path(model_path).with_name("config.json"))
        except PiaError:
            return cls(hidden=2048, layers=22, heads=32, kv_heads=4, inter=5632, vocab=32000)

    @classmethod
    def _from_c(cls, c: ModelConfig) -> "LlamaConfig":
        return cls(hidden=c.hidden, layers=c.layers, heads=c.heads, kv_heads=c.kv_heads, inter=c.inter,
                   vocab=c.vocab, rms_eps=c.rms_eps, rope_theta=c.rope_theta,
                   attention_window=None if c.attention_window < 0 else c.attention_window)

    def c(self) -> ModelConfig:
        return ModelConfig(self.hidden, self.layers, self.heads, self.kv_heads, self.inter, self.vocab, self.rms_eps,
                           self.rope_theta, -1 if self.attention_window is None else self.attention_window)


class Model:
    """Device-resident weights + KV cache. `weights` is the dict built by synth_weights() or a
    checkpoint loader: embed (uint16 bf16 bits [V][H]), final_norm, lm_head, and per layer
    attn_norm, ffn_norm and wq/wk/wv/wo/w1/w2/w3, each projection either a (q int8, scales f32)
    pair (Projection::Int8) or an f32 matrix (Projection::F32)."""

    def __init__(self, ctx: Context, cfg: LlamaConfig, weights: dict | None):
        self.ctx, self.cfg = ctx, cfg
        h = P()
        cc = cfg.c()
        check(lib().pia_model_create(ctx.h, C.byref(cc), C.byref(h)))
        self.h = h
        ctx._children.add(self)
        self.kv_ptr = None
        self.layout = None
        if weights is None:
            return
        L = lib()
        check(L.pia_model_set_embedding(h, ptr(np.ascontiguousarray(weights["embed"], np.uint16))))
        check(L.pia_model_set_norm(h, 0, NORM_FINAL, ptr(np.ascontiguousarray(weights["final_norm"], np.float32))))
        self._set_proj(-1, "lm_head", weights["lm_head"])
        for i, lw in enumerate(weights["layers"]):
            check(L.pia_model_set_norm(h, i, NORM_ATTN, ptr(np.ascontiguousarray(lw["attn_norm"], np.float32))))
            check(L.pia_model_set_norm(h, i, NORM_FFN, ptr(np.ascontiguousarray(lw["ffn_norm"], np.float32))))
            for name in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"):
                self._set_proj(i, name, lw[name])

    @classmethod
    def from_safetensors(cls, ctx: Context, path, cfg: LlamaConfig | None = None, quantization: str = "int8",
                         lm_head_int8: bool = False) -> "Model":
        """ModelLoader::load_weights (src/model.rs:388-447) straight into device memory: a bf16
        HF Llama checkpoint, projections widened ("f32") or quantized on the device ("int8");
        the LM head stays f32 unless lm_head_int8. cfg defaults to the config.json beside
        the checkpoint (LlamaConfig.beside_checkpoint)."""
        if quantization not in ("f32", "int8"):
            raise ValueError("quantization must be 'f32' or 'int8'")
        cfg = cfg or LlamaConfig.beside_checkpoint(path)
        m = cls(ctx, cfg, None)
        check(lib().pia_model_load_safetensors(m.h, str(path).encode(), 1 if quantization == "int8" else 0,
                                               1 if lm_head_int8 else 0))
        return m

    def _set_proj(self, layer, name, p):
        if isinstance(p, tuple):
            q, s = p
            check(lib().pia_model_set_proj_i8(self.h, layer, SLOTS[name], ptr(np.ascontiguousarray(q, np.int8)),
                                              ptr(np.ascontiguousarray(s, np.float32))))
        else:
            check(lib().pia_model_set_proj_f32(self.h, layer, SLOTS[name], ptr(np.ascontiguousarray(p, np.float32))))

    def close(self):
        if self.h:
            lib().pia_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_bytes(self) -> int:
        return int(lib().pia_model_weight_bytes(self.h))

    def kv_alloc(self, num_blocks: int, block_size: int):
        check(lib().pia_model_kv_alloc(self.h, num_blocks, block_size))
        kp, lay = P(), KvLayout()
        check(lib().pia_model_kv(self.h, C.byref(kp), C.byref(lay)))
        self.kv_ptr, self.layout = kp, lay

    def kv_numel(self) -> int:
        L = self.layout
        return L.num_layers * L.num_blocks * L.block_size * L.num_kv_heads * 2 * L.head_dim

    def kv_download(self) -> np.ndarray:
        out = np.empty(self.kv_numel(), np.float32)
        check(lib().pia_memcpy_d2h(self.ctx.h, ptr(out), self.kv_ptr, out.nbytes))
        return out

    def kv_upload(self, kv: np.ndarray):
        kv = np.ascontiguousarray(kv, np.float32)
        assert kv.size == self.kv_numel()
        check(lib().pia_memcpy_h2d(self.ctx.h, self.kv_ptr, ptr(kv), kv.nbytes))

    def decode(self, tokens, positions, tables: list[list[int]], want_logits: bool = True):
        """decode_batch_into: returns (logits [B][V] or None, argmax [B])."""
        b = len(tokens)
        tok = np.ascontiguousarray(np.asarray(tokens, np.uint32))
        pos = np.ascontiguousarray(np.asarray(positions, np.int64))
        off = np.zeros(b, np.int64)
        ln = np.zeros(b, np.int64)
        flat = []
        for i, t in enumerate(tables):
            off[i] = len(flat)
            ln[i] = len(t)
            flat.extend(t)
        flat = np.ascontiguousarray(np.asarray(flat if flat else [0], np.int32))
        logits = np.empty((b, self.cfg.vocab), np.float32) if want_logits else None
        am = np.empty(b, np.int32)
        check(lib().pia_model_decode(self.h, ptr(tok), ptr(pos), ptr(off), ptr(ln), ptr(flat), b, ptr(logits),
                                     ptr(am)))
        return logits, am

    def prefill(self, tokens, start_pos: int, table: list[int], want_logits: bool = True):
        tok = np.ascontiguousarray(np.asarray(tokens, np.uint32))
        t = np.ascontiguousarray(np.asarray(table if len(table) else [0], np.int32))
        logits = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        am = np.empty(1, np.int32)
        check(lib().pia_model_prefill(self.h, ptr(tok), tok.size, start_pos, ptr(t), len(table), ptr(logits),
                                      ptr(am)))
        return logits, int(am[0])

    def sample(self, params, rng_state: np.ndarray, mode: int = 0) -> list[int]:
        """Sampler::sample (src/sampling.rs:74-138) on the device for the first len(params) rows
        of the last decode's (or prefill's) logits; rng_state (uint64 [n]) advances in place."""
        a = sampling_array(params)
        assert rng_state.dtype == np.uint64 and rng_state.flags["C_CONTIGUOUS"] and rng_state.size == len(params)
        out = np.empty(len(params), np.int32)
        check(lib().pia_model_sample(self.h, ptr(a), ptr(rng_state), len(params), mode, ptr(out)))
        return [int(t) for t in out]

    def verify_groups(self, groups, capacity: int = 0):
        """Engine::run_groups + verification (src/engine.rs:702-783). `groups` is a list of
        (pos, tokens, table): the held token at pos followed by its drafts, on the sequence's
        block table. Returns (per-group predictions, per-group accepted count, per-group
        corrected token, passes)."""
        gs = (SpecGroup * max(1, len(groups)))()
        toks, flat_tables = [], []
        for g, (pos, tokens, table) in enumerate(groups):
            gs[g] = SpecGroup(pos, len(tokens), len(toks), len(flat_tables), len(table))
            toks += list(tokens)
            flat_tables += list(table)
        t = np.ascontiguousarray(np.asarray(toks or [0], np.uint32))
        tb = np.ascontiguousarray(np.asarray(flat_tables or [0], np.int32))
        pred = np.zeros(max(1, len(toks)), np.uint32)
        acc = np.zeros(max(1, len(groups)), np.int64)
        corr = np.zeros(max(1, len(groups)), np.uint32)
        passes = I64()
        check(lib().pia_model_verify_groups(self.h, C.cast(gs, P), len(groups), ptr(t), ptr(tb), capacity, ptr(pred),
                                            ptr(acc), ptr(corr), C.byref(passes)))
        out, off = [], 0
        for _, tokens, _ in groups:
            out.append([int(x) for x in pred[off:off + len(tokens)]])
            off += len(tokens)
        return out, [int(a) for a in acc[:len(groups)]], [int(c) for c in corr[:len(groups)]], passes.value

    def bench_class(self, cls: str, batch: int, reps: int = 5):
        """(us per launch, algorithmic bytes per launch) of one projection class at `batch`."""
        us, by = C.c_double(), I64()
        check(lib().pia_model_bench_class(self.h, self.PROFILE_CLASSES.index(cls), batch, reps, C.byref(us),
                                          C.byref(by)))
        return us.value, by.value

    def profile(self, on: bool):
        check(lib().pia_model_profile(self.h, int(on)))

    PROFILE_CLASSES = ("qkv", "o", "gate_up", "down", "lm_head", "attention", "other", "step")

    def set_decode_path(self, path: int):
        """0: per-kernel launches (default); 1: persistent batch-1 decode step when supported."""
        check(lib().pia_model_set_decode_path(self.h, path))

    def decode_path_used(self) -> int:
        """Path of the last decode: 0 per-kernel launches, 1 persistent step."""
        return int(lib().pia_model_decode_path_used(self.h))

    def last_upload(self):
        """(host-to-device bytes, table slots patched, whole image re-sent) of the last decode."""
        b, pch, full = I64(), I64(), I32()
        check(lib().pia_model_last_upload(self.h, C.byref(b), C.byref(pch), C.byref(full)))
        return b.value, pch.value, bool(full.value)

    def last_shared(self):
        """(virtual entries, splits) of the last decode's shared-prefix attention (0: not used)."""
        v, sp = I64(), I64()
        check(lib().pia_model_last_shared(self.h, C.byref(v), C.byref(sp)))
        return v.value, sp.value

    def profile_get(self):
        """(ms, algorithmic bytes, launches) per class of the last profiled call."""
        n = len(self.PROFILE_CLASSES)
        ms = np.zeros(n, np.float64)
        by = np.zeros(n, np.int64)
        calls = np.zeros(n, np.int64)
        check(lib().pia_model_profile_get(self.h, ptr(ms), ptr(by), ptr(calls), n))
        return ms, by, calls


# ------------------------------------------------------------------------------------------
# Synthetic weights (the configs' "random-init N(0, 0.02), then per-row int8").
# ------------------------------------------------------------------------------------------
def synth_weights(cfg: LlamaConfig, seed: int, quantize: bool = True, lm_head_int8: bool = True,
                  std: float = 0.02) -> dict:
    """Seeded synthetic Llama weights. Projections: N(0, std) f32, then quantize_rows_i8 when
    `quantize` (Projection::Int8). Embeddings: N(0, std) rounded to bf16. Norm weights: 1.0."""
    hd = cfg.head_dim
    kvd = cfg.kv_heads * hd
    shapes = {"wq": (cfg.hidden, cfg.hidden), "wk": (kvd, cfg.hidden), "wv": (kvd, cfg.hidden),
              "wo": (cfg.hidden, cfg.hidden), "w1": (cfg.inter, cfg.hidden), "w2": (cfg.hidden, cfg.inter),
              "w3": (cfg.inter, cfg.hidden)}

    def proj(stream, shape, q):
        w = synth_normal(seed, stream, shape[0] * shape[1], std).reshape(shape)
        return quantize_rows_i8(w) if q else w

    out = {"embed": f32_to_bf16(synth_normal(seed, 1, cfg.vocab * cfg.hidden, std).reshape(cfg.vocab, cfg.hidden)),
           "final_norm": np.ones(cfg.hidden, np.float32),
           "lm_head": proj(2, (cfg.vocab, cfg.hidden), quantize and lm_head_int8),
           "layers": []}
    for i in range(cfg.layers):
        lw = {"attn_norm": np.ones(cfg.hidden, np.float32), "ffn_norm": np.ones(cfg.hidden, np.float32)}
        for j, (name, shp) in enumerate(shapes.items()):
            lw[name] = proj(16 + 16 * i + j, shp, quantize)
        out["layers"].append(lw)
    return out


def projection_bytes(weights: dict) -> int:
    """LlamaWeights::weight_bytes (src/model.rs:590-608) of a weights dict."""
    def pb(p):
        if isinstance(p, tuple):
            return p[0].size + 4 * p[1].size
        return 4 * p.size
    t = pb(weights["lm_head"])
    for lw in weights["layers"]:
        t += sum(pb(lw[n]) for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3"))
    return t


# Shapes of the benchmark configurations (BASELINE.json "configs").
TINY_C1 = LlamaConfig(hidden=128, layers=2, heads=4, kv_heads=2, inter=344, vocab=512)
TINYLLAMA = LlamaConfig(hidden=2048, layers=22, heads=32, kv_heads=4, inter=5632, vocab=32000)
LLAMA3_8B = LlamaConfig(hidden=4096, layers=32, heads=32, kv_heads=8, inter=14336, vocab=128256,
                        rope_theta=500000.0)
