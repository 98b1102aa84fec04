"""Loader for the reference's committed golden fixture (tests/fixtures/ of Rohanr14/Paged-Infer,
copied here as data): tiny_llama.safetensors (bf16 HF Llama checkpoint), tiny_llama_golden.bin
(40 x vocab f32 LE logits from an independent NumPy transcription of HF modeling_llama) and
tiny_llama_meta.txt (config + token ids). Mirrors tests/golden_parity_tests.rs:33-84 of the
reference: same file parsing, same config (NeoX RoPE, no window, f32 projections).
The safetensors container is parsed directly (8-byte LE header length, JSON header, raw data);
nothing in it is executable."""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BLOCK_SIZE = 16


def read_safetensors(path: Path) -> dict:
    raw = path.read_bytes()
    (hlen,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        assert info["dtype"] == "BF16", f"{name}: {info['dtype']}"
        a, b = info["data_offsets"]
        out[name] = np.frombuffer(raw[base + a:base + b], dtype="<u2").reshape(info["shape"]).copy()
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def load():
    meta = {}
    for line in (HERE / "tiny_llama_meta.txt").read_text().splitlines():
        if "=" in line:
            k, v = line.split("=", 1)
            meta[k.strip()] = v.strip()
    cfg = dict(hidden=int(meta["hidden_size"]), layers=int(meta["num_hidden_layers"]),
               heads=int(meta["num_attention_heads"]), kv_heads=int(meta["num_key_value_heads"]),
               inter=int(meta["intermediate_size"]), vocab=int(meta["vocab_size"]),
               rms_eps=float(meta["rms_norm_eps"]), rope_theta=float(meta["rope_theta"]))
    tokens = [int(t) for t in meta["tokens"].split(",")]
    assert len(tokens) == int(meta["seq_len"])
    golden = np.fromfile(HERE / "tiny_llama_golden.bin", dtype="<f4").reshape(len(tokens), cfg["vocab"])
    t = read_safetensors(HERE / "tiny_llama.safetensors")
    f = lambda n: bf16_to_f32(t[n])
    lm = t.get("lm_head.weight", t["model.embed_tokens.weight"])
    weights = {"embed": t["model.embed_tokens.weight"], "final_norm": f("model.norm.weight"),
               "lm_head": bf16_to_f32(lm), "layers": []}
    for i in range(cfg["layers"]):
        p = f"model.layers.{i}"
        weights["layers"].append({
            "attn_norm": f(f"{p}.input_layernorm.weight"), "ffn_norm": f(f"{p}.post_attention_layernorm.weight"),
            "wq": f(f"{p}.self_attn.q_proj.weight"), "wk": f(f"{p}.self_attn.k_proj.weight"),
            "wv": f(f"{p}.self_attn.v_proj.weight"), "wo": f(f"{p}.self_attn.o_proj.weight"),
            "w1": f(f"{p}.mlp.gate_proj.weight"), "w2": f(f"{p}.mlp.down_proj.weight"),
            "w3": f(f"{p}.mlp.up_proj.weight")})
    return cfg, tokens, golden, weights


def compare(actual: np.ndarray, expected: np.ndarray):
    """tests/golden_parity_tests.rs:96-117: max |delta| and the number of rows whose argmax
    (last maximal index, f32 total order) moved."""
    actual = np.atleast_2d(actual)
    expected = np.atleast_2d(expected)
    max_abs = float(np.max(np.abs(actual - expected)))

    def pick(row):
        return len(row) - 1 - int(np.argmax(row[::-1]))

    mism = sum(pick(a) != pick(e) for a, e in zip(actual, expected))
    return max_abs, mism


def write_safetensors(path: Path, tensors: dict, dtypes: dict | None = None, metadata: dict | None = None):
    """Write a safetensors file: 8-byte LE header length, JSON header, raw little-endian data.
    `tensors` maps names to uint16 bf16-bit arrays (dtype "BF16") unless `dtypes` names another
    safetensors dtype for the entry (the array's bytes are written as they are)."""
    dtypes = dtypes or {}
    header = {"__metadata__": metadata or {"format": "pt"}}
    blobs, off = [], 0
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(arr)
        raw = arr.tobytes()
        header[name] = {"dtype": dtypes.get(name, "BF16"), "shape": list(arr.shape),
                        "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hj = json.dumps(header).encode()
    hj += b" " * (-len(hj) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)
