"""Checkpoint loading: LlamaConfig::from_hf_config (src/model.rs:57-95) and
ModelLoader::load_weights (src/model.rs:388-447) through the C ABI
(pia_hf_config_read, pia_model_load_safetensors).

CPU tests pin the config reader against the reference fixture's config.json (whose values
tiny_llama_meta.txt repeats) and the reference's default / type rules. GPU tests pin the
loader: a checkpoint loaded by the library (bf16 widened or quantized on the device) must give
logits bit-identical to the same weights widened and quantized on the host
(pia_quantize_rows_i8, itself pinned against quantize_rows_i8's closed form) and uploaded
slot by slot, and the reference's golden fixture must meet its own bar (max|delta| < 5e-4,
0 argmax mismatches, tests/golden_parity_tests.rs) when loaded from its safetensors file."""
import json

import numpy as np
import pytest

import pia
from golden import fixture

TINY_DEFAULT = dict(hidden=2048, layers=22, heads=32, kv_heads=4, inter=5632, vocab=32000)


def _write_cfg(tmp_path, obj, raw=None):
    p = tmp_path / "config.json"
    p.write_text(raw if raw is not None else json.dumps(obj))
    return p


def test_hf_config_matches_fixture_meta():
    cfg = pia.LlamaConfig.from_hf_config(fixture.HERE / "config.json")
    meta, *_ = fixture.load()
    assert cfg.hidden == meta["hidden"] and cfg.layers == meta["layers"]
    assert cfg.heads == meta["heads"] and cfg.kv_heads == meta["kv_heads"]
    assert cfg.inter == meta["inter"] and cfg.vocab == meta["vocab"]
    assert cfg.rms_eps == np.float32(meta["rms_eps"]) and cfg.rope_theta == meta["rope_theta"]
    assert cfg.attention_window is None


def test_hf_config_defaults_and_types(tmp_path):
    # Absent fields keep the defaults; num_key_value_heads follows num_attention_heads.
    cfg = pia.LlamaConfig.from_hf_config(_write_cfg(tmp_path, {"num_attention_heads": 8, "hidden_size": 512}))
    assert (cfg.hidden, cfg.heads, cfg.kv_heads) == (512, 8, 8)
    assert (cfg.layers, cfg.inter, cfg.vocab) == (22, 5632, 32000)
    assert cfg.rms_eps == np.float32(1e-5) and cfg.rope_theta == 10000.0
    # serde_json's as_u64 rejects 2048.0, negatives and strings: the default stays.
    cfg = pia.LlamaConfig.from_hf_config(
        _write_cfg(tmp_path, {"hidden_size": 1024.0, "num_hidden_layers": -3, "vocab_size": "7",
                              "rope_theta": 500000, "rms_norm_eps": 1e-6, "nested": {"hidden_size": 1},
                              "list": [1, 2, {"a": "é\\n"}], "flag": True, "none": None}))
    assert (cfg.hidden, cfg.layers, cfg.vocab) == (2048, 22, 32000)
    assert cfg.rope_theta == 500000.0 and cfg.rms_eps == np.float32(1e-6)
    # Empty object: the TinyLlama defaults, except num_key_value_heads, which follows the
    # (default) num_attention_heads as in the reference; only LlamaConfig::default() has 4.
    cfg = pia.LlamaConfig.from_hf_config(_write_cfg(tmp_path, {}))
    assert {k: getattr(cfg, k) for k in TINY_DEFAULT} == dict(TINY_DEFAULT, kv_heads=32)


def test_hf_config_errors(tmp_path):
    with pytest.raises(pia.PiaError, match="cannot open"):
        pia.LlamaConfig.from_hf_config(tmp_path / "absent.json")
    with pytest.raises(pia.PiaError, match="parsing"):
        pia.LlamaConfig.from_hf_config(_write_cfg(tmp_path, None, raw='{"hidden_size": 96,'))
    # beside_checkpoint falls back to the defaults (src/model.rs:97-102).
    cfg = pia.LlamaConfig.beside_checkpoint(tmp_path / "sub" / "model.safetensors")
    assert {k: getattr(cfg, k) for k in TINY_DEFAULT} == TINY_DEFAULT
    cfg = pia.LlamaConfig.beside_checkpoint(fixture.HERE / "tiny_llama.safetensors")
    assert cfg.hidden == 96


# ------------------------------------------------------------------------------------------
# GPU: the loader itself.
# ------------------------------------------------------------------------------------------
def _checkpoint_tensors(cfg: pia.LlamaConfig, seed: int, tied: bool = False) -> dict:
    """HF-named bf16 tensors of a seeded synthetic model (norm weights random, not 1.0, so
    they are checked too)."""
    w = pia.synth_weights(cfg, seed, quantize=False)
    rng = np.random.default_rng(seed)
    bf = lambda a: pia.f32_to_bf16(np.asarray(a, np.float32))
    t = {"model.embed_tokens.weight": w["embed"],
         "model.norm.weight": bf(1.0 + 0.1 * rng.standard_normal(cfg.hidden))}
    if not tied:
        t["lm_head.weight"] = bf(w["lm_head"])
    names = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
             "w1": "mlp.gate_proj", "w2": "mlp.down_proj", "w3": "mlp.up_proj"}
    for i, lw in enumerate(w["layers"]):
        p = f"model.layers.{i}"
        t[f"{p}.input_layernorm.weight"] = bf(1.0 + 0.1 * rng.standard_normal(cfg.hidden))
        t[f"{p}.post_attention_layernorm.weight"] = bf(1.0 + 0.1 * rng.standard_normal(cfg.hidden))
        for k, n in names.items():
            t[f"{p}.{n}.weight"] = bf(lw[k])
    return t


def _host_weights(cfg: pia.LlamaConfig, t: dict, quant: bool, lm_head_int8: bool) -> dict:
    """The same checkpoint widened and (optionally) quantized on the host, in Model's dict form."""
    wide = lambda n: fixture.bf16_to_f32(t[n])
    proj = lambda n, q: pia.quantize_rows_i8(wide(n)) if q else wide(n)
    lm = "lm_head.weight" if "lm_head.weight" in t else "model.embed_tokens.weight"
    out = {"embed": t["model.embed_tokens.weight"], "final_norm": wide("model.norm.weight"),
           "lm_head": proj(lm, lm_head_int8), "layers": []}
    names = {"wq": "self_attn.q_proj", "wk": "self_attn.k_proj", "wv": "self_attn.v_proj", "wo": "self_attn.o_proj",
             "w1": "mlp.gate_proj", "w2": "mlp.down_proj", "w3": "mlp.up_proj"}
    for i in range(cfg.layers):
        p = f"model.layers.{i}"
        lw = {"attn_norm": wide(f"{p}.input_layernorm.weight"),
              "ffn_norm": wide(f"{p}.post_attention_layernorm.weight")}
        for k, n in names.items():
            lw[k] = proj(f"{p}.{n}.weight", quant)
        out["layers"].append(lw)
    return out


def _run(model: pia.Model, prompt, steps: int, block_size: int = 16):
    """Prefill + greedy decode; returns (prefill logits, decode logits rows, tokens)."""
    n = len(prompt) + steps
    table = list(range((n + block_size - 1) // block_size))
    model.kv_alloc(len(table) + 1, block_size)
    lg, am = model.prefill(prompt, 0, table)
    rows, toks = [], [int(am)]
    for s in range(steps - 1):
        l2, a2 = model.decode([toks[-1]], [len(prompt) + s], [table])
        rows.append(l2[0])
        toks.append(int(a2[0]))
    return lg, np.stack(rows), toks


CFG_SMALL = pia.LlamaConfig(hidden=128, layers=2, heads=4, kv_heads=2, inter=344, vocab=512)
# Llama-3-style GQA with rows that are not multiples of the int8 row padding.
CFG_ODD = pia.LlamaConfig(hidden=320, layers=2, heads=8, kv_heads=2, inter=904, vocab=1000, rope_theta=500000.0)


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [CFG_SMALL, CFG_ODD], ids=["c1", "odd"])
@pytest.mark.parametrize("quant,lm_head_int8", [("int8", False), ("int8", True), ("f32", False)])
def test_loader_matches_host_upload(ctx, tmp_path, cfg, quant, lm_head_int8):
    t = _checkpoint_tensors(cfg, seed=7)
    path = tmp_path / "model.safetensors"
    fixture.write_safetensors(path, t)
    loaded = pia.Model.from_safetensors(ctx, path, cfg, quantization=quant, lm_head_int8=lm_head_int8)
    host = pia.Model(ctx, cfg, _host_weights(cfg, t, quant == "int8", lm_head_int8))
    assert loaded.weight_bytes() == host.weight_bytes()
    prompt = [int(x) for x in np.random.default_rng(3).integers(0, cfg.vocab, 37)]
    a = _run(loaded, prompt, 12)
    b = _run(host, prompt, 12)
    loaded.close(), host.close()
    print(f"loader {cfg.hidden}/{quant}/lm_head_int8={lm_head_int8}: tokens {a[2]}")
    assert a[2] == b[2]
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


@pytest.mark.gpu
def test_loader_tied_embeddings(ctx, tmp_path):
    cfg = CFG_SMALL
    t = _checkpoint_tensors(cfg, seed=11, tied=True)
    path = tmp_path / "model.safetensors"
    fixture.write_safetensors(path, t)
    loaded = pia.Model.from_safetensors(ctx, path, cfg, quantization="int8")
    host = pia.Model(ctx, cfg, _host_weights(cfg, t, True, False))
    prompt = list(range(5, 30))
    a, b = _run(loaded, prompt, 6), _run(host, prompt, 6)
    loaded.close(), host.close()
    assert a[2] == b[2]
    np.testing.assert_array_equal(a[1], b[1])


@pytest.mark.gpu
def test_loader_golden_fixture(ctx):
    """The reference's fixture from its safetensors file (config from the config.json beside
    it, f32 projections as in tests/golden_parity_tests.rs) against the golden logits."""
    _, tokens, golden, _ = fixture.load()
    gm = pia.Model.from_safetensors(ctx, fixture.HERE / "tiny_llama.safetensors", quantization="f32")
    gm.kv_alloc(8, fixture.BLOCK_SIZE)
    rows = [gm.decode([t], [p], [[0, 1, 2]])[0][0] for p, t in enumerate(tokens)]
    max_abs, mism = fixture.compare(np.stack(rows), golden)
    print(f"golden fixture via the loader: max|delta|={max_abs:.3g} mismatches={mism}")
    assert mism == 0 and max_abs < 5e-4
    # int8 load (device quantizer) equals the host-quantized upload bit for bit.
    cfg = gm.cfg
    gm.close()
    raw = fixture.read_safetensors(fixture.HERE / "tiny_llama.safetensors")
    loaded = pia.Model.from_safetensors(ctx, fixture.HERE / "tiny_llama.safetensors", quantization="int8")
    host = pia.Model(ctx, cfg, _host_weights(cfg, raw, True, False))
    a, b = _run(loaded, tokens[:20], 10), _run(host, tokens[:20], 10)
    loaded.close(), host.close()
    assert a[2] == b[2]
    np.testing.assert_array_equal(a[1], b[1])


@pytest.mark.gpu
def test_loader_errors(ctx, tmp_path):
    cfg = CFG_SMALL
    t = _checkpoint_tensors(cfg, seed=5)
    path = tmp_path / "m.safetensors"

    def load(tensors, dtypes=None, c=cfg):
        fixture.write_safetensors(path, tensors, dtypes)
        m = pia.Model(ctx, c, None)
        try:
            check = pia.lib().pia_model_load_safetensors(m.h, str(path).encode(), 1, 0)
            return check, pia.lib().pia_last_error().decode()
        finally:
            m.close()

    missing = dict(t)
    del missing["model.layers.1.mlp.up_proj.weight"]
    st, msg = load(missing)
    assert st == pia.PIA_ERR_INVALID and "missing tensor: model.layers.1.mlp.up_proj.weight" in msg
    st, msg = load(t, {"model.layers.0.self_attn.k_proj.weight": "F16"})
    assert st == pia.PIA_ERR_INVALID and "k_proj.weight: dtype F16" in msg
    wrong = pia.LlamaConfig(hidden=128, layers=2, heads=4, kv_heads=4, inter=344, vocab=512)
    st, msg = load(t, c=wrong)
    assert st == pia.PIA_ERR_INVALID and "k_proj.weight: shape [64, 128]" in msg
    # Truncated payload: data_offsets run past the end of the file.
    fixture.write_safetensors(path, t)
    raw = path.read_bytes()
    path.write_bytes(raw[:-100])
    m = pia.Model(ctx, cfg, None)
    with pytest.raises(pia.PiaError, match="out of range"):
        pia.check(pia.lib().pia_model_load_safetensors(m.h, str(path).encode(), 1, 0))
    # Header length larger than the file.
    path.write_bytes((10 ** 9).to_bytes(8, "little") + b"{}")
    with pytest.raises(pia.PiaError, match="header length"):
        pia.check(pia.lib().pia_model_load_safetensors(m.h, str(path).encode(), 1, 0))
    with pytest.raises(pia.PiaError, match="cannot open"):
        pia.check(pia.lib().pia_model_load_safetensors(m.h, str(tmp_path / "nope").encode(), 1, 0))
    m.close()
