"""Pins the CPU oracle's f32 forward against the reference's committed golden logits
(tests/golden_parity_tests.rs of the reference: max|delta| < 5e-4 and 0 argmax mismatches for
incremental decode and for prefill; < 1e-5 between split and whole prefill). The golden
logits come from an independent NumPy transcription of HF modeling_llama, so this checks the
oracle's embedding, RMSNorm, NeoX RoPE, GQA attention across three KV blocks, SwiGLU and LM
head -- not a retyped formula."""
import numpy as np
import pytest

from golden import fixture
from oracle import oracle as orc
import pia

BS = fixture.BLOCK_SIZE


@pytest.fixture(scope="module")
def fx():
    cfg, tokens, golden, weights = fixture.load()
    return pia.LlamaConfig(**cfg), tokens, golden, weights


def _kv(cfg, blocks=8):
    return np.zeros(orc.kv_floats(cfg, blocks, BS), np.float32)


def test_incremental_decode_matches_golden(fx):
    cfg, tokens, golden, weights = fx
    m = orc.OracleModel(cfg, weights)
    kv = _kv(cfg)
    table = list(range((len(tokens) + BS - 1) // BS))  # FIFO allocator hands out 0, 1, 2
    assert len(table) >= 3
    rows = [m.decode([t], [p], [table], kv, 8, BS)[0] for p, t in enumerate(tokens)]
    max_abs, mism = fixture.compare(np.stack(rows), golden)
    assert mism == 0
    assert max_abs < 5e-4, max_abs


def test_prefill_matches_golden(fx):
    cfg, tokens, golden, weights = fx
    m = orc.OracleModel(cfg, weights)
    kv = _kv(cfg)
    logits = m.prefill(tokens, 0, [0, 1, 2], kv, 8, BS)
    max_abs, mism = fixture.compare(logits, golden[-1])
    assert mism == 0
    assert max_abs < 5e-4, max_abs


def test_split_prefill_matches_whole(fx):
    cfg, tokens, golden, weights = fx
    m = orc.OracleModel(cfg, weights)
    whole = m.prefill(tokens, 0, [0, 1, 2], _kv(cfg), 8, BS)
    kv = _kv(cfg)
    m.prefill(tokens[:16], 0, [0, 1, 2], kv, 8, BS)
    split = m.prefill(tokens[16:], 16, [0, 1, 2], kv, 8, BS)
    assert np.max(np.abs(split - whole)) < 1e-5


@pytest.mark.parametrize("chunk", [1, 7, 32, 64])
def test_prefill_chunking_is_bit_identical(fx, chunk):
    # "Scheduling never changes arithmetic" (tests/batched_decode_tests.rs of the reference).
    cfg, tokens, golden, weights = fx
    m = orc.OracleModel(cfg, weights)
    ref = m.prefill(tokens, 0, [0, 1, 2], _kv(cfg), 8, BS, chunk=32)
    got = m.prefill(tokens, 0, [0, 1, 2], _kv(cfg), 8, BS, chunk=chunk)
    assert np.array_equal(ref, got)


def test_neox_not_interchangeable_with_interleaved(fx):
    # The fixture discriminates the rotary convention (gen_golden_fixture.py:238-241 of the
    # reference): a rotation that pairs (2i, 2i+1) instead of (j, j+hd/2) must miss the golden.
    cfg, tokens, golden, weights = fx
    hd = cfg.head_dim
    perm = np.concatenate([np.arange(0, hd, 2), np.arange(1, hd, 2)])
    w2 = {**weights, "layers": []}
    for lw in weights["layers"]:
        d = dict(lw)
        for name, nh in (("wq", cfg.heads), ("wk", cfg.kv_heads)):
            w = lw[name].reshape(nh, hd, -1)
            d[name] = np.ascontiguousarray(w[:, perm, :].reshape(nh * hd, -1))
        w2["layers"].append(d)
    # Permuting q/k rows so NeoX acts as "interleaved" must change the logits materially.
    m = orc.OracleModel(cfg, w2)
    logits = m.prefill(tokens, 0, [0, 1, 2], _kv(cfg), 8, BS)
    max_abs, _ = fixture.compare(logits, golden[-1])
    assert max_abs > 1e-3
