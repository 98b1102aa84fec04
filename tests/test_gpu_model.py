"""End-to-end parity of the GPU forward pass (C ABI model tier) with the CPU oracle and with
the reference's golden fixture.

Bar: greedy token sequences bit-exact vs the CPU reference path
on the same seeded inputs; logits within max|delta| <= 2e-3 relative to the logit scale
(max |logit| of the reference row); block tables and copy-on-write counts bit-exact. The
golden fixture (f32 projections) uses the reference's own bar: max|delta| < 5e-4 and 0
argmax mismatches over 40 positions (tests/golden_parity_tests.rs)."""
import numpy as np
import pytest

import pia
from golden import fixture
from oracle import memory as om
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
LOGIT_TOL = 2e-3


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / max(1e-30, np.max(np.abs(b))))


def greedy_session(ctx, cfg, weights, prompt, steps, block_size=16, path=0, expect_path=None):
    """Prefill `prompt`, then `steps` greedy decode steps at batch 1, independently on the GPU
    and on the oracle (each side feeds back its own argmax). `path` selects the GPU decode path
    (0: per-kernel launches, 1: persistent single-launch step where supported); every decode
    must have run on `expect_path` when given."""
    n_tok = len(prompt) + steps
    nb = (n_tok + block_size - 1) // block_size
    table = list(range(nb))  # a fresh FIFO pool hands out 0..nb-1
    gm = pia.Model(ctx, cfg, weights)
    gm.set_decode_path(path)
    gm.kv_alloc(nb + 1, block_size)
    om_ = orc.OracleModel(cfg, weights)
    kv = np.zeros(orc.kv_floats(cfg, nb + 1, block_size), np.float32)
    lg, tg = gm.prefill(prompt, 0, table)
    lc = om_.prefill(prompt, 0, table, kv, nb + 1, block_size)
    tc = orc.argmax(lc)
    rels = [_rel(lg, lc)]
    gtoks, ctoks = [tg], [tc]
    for i in range(steps - 1):
        pos = len(prompt) + i
        lg, am = gm.decode([gtoks[-1]], [pos], [table])
        if expect_path is not None:
            assert gm.decode_path_used() == expect_path
        lc = om_.decode([ctoks[-1]], [pos], [table], kv, nb + 1, block_size)
        if gtoks == ctoks:
            rels.append(_rel(lg[0], lc[0]))
        gtoks.append(int(am[0]))
        ctoks.append(orc.argmax(lc[0]))
    gm.close()
    return gtoks, ctoks, max(rels)


def test_golden_fixture_f32_on_gpu(ctx):
    cfg, tokens, golden, weights = fixture.load()
    cfg = pia.LlamaConfig(**cfg)
    gm = pia.Model(ctx, cfg, weights)
    gm.kv_alloc(8, fixture.BLOCK_SIZE)
    table = [0, 1, 2]
    rows = [gm.decode([t], [p], [table])[0][0] for p, t in enumerate(tokens)]
    max_abs, mism = fixture.compare(np.stack(rows), golden)
    print(f"golden incremental decode on GPU: max|delta|={max_abs:.3g} mismatches={mism}")
    assert mism == 0 and max_abs < 5e-4
    gm.kv_alloc(8, fixture.BLOCK_SIZE)
    lg, _ = gm.prefill(tokens, 0, table)
    max_abs, mism = fixture.compare(lg, golden[-1])
    assert mism == 0 and max_abs < 5e-4
    gm.kv_alloc(8, fixture.BLOCK_SIZE)
    gm.prefill(tokens[:16], 0, table)
    split, _ = gm.prefill(tokens[16:], 16, table)
    assert np.max(np.abs(split - lg)) < 1e-5


@pytest.mark.parametrize("path", [0, 1], ids=["per_kernel", "persistent"])
def test_config1_tiny_int8_greedy_parity(ctx, path):
    """dim 128, 2 layers, 4/2 heads, FFN 344, vocab 512, block 16, 48-token
    prompt, 40 greedy steps, int8 projections incl. lm_head; on both decode paths."""
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=1)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 48).tolist()
    g, c, rel = greedy_session(ctx, cfg, w, prompt, 40, path=path, expect_path=path)
    print(f"config1 path {path}: rel max|dlogit|={rel:.3g} tokens={g[:10]}...")
    assert g == c
    assert rel <= LOGIT_TOL


def test_config1_f32_lm_head_variant(ctx):
    # The reference keeps lm_head f32 by default (src/model.rs:441-444).
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=2, lm_head_int8=False)
    prompt = np.random.default_rng(2).integers(0, cfg.vocab, 48).tolist()
    # An f32 LM head keeps batch-1 decode on the per-kernel path even when the persistent
    # step is requested.
    g, c, rel = greedy_session(ctx, cfg, w, prompt, 40, path=1, expect_path=0)
    assert g == c and rel <= LOGIT_TOL


@pytest.mark.parametrize("path", [0, 1], ids=["per_kernel", "persistent"])
def test_sliding_window_model(ctx, path):
    cfg = pia.LlamaConfig(hidden=128, layers=2, heads=4, kv_heads=2, inter=344, vocab=512, attention_window=20)
    w = pia.synth_weights(cfg, seed=3)
    prompt = np.random.default_rng(3).integers(0, cfg.vocab, 37).tolist()
    g, c, rel = greedy_session(ctx, cfg, w, prompt, 12, path=path, expect_path=path)
    assert g == c and rel <= LOGIT_TOL


def test_persistent_step_unmapped_tail(ctx):
    """Batch-1 decode whose block table stops short of the position: the unmapped logical
    block scores -inf and this step's K/V write is skipped (src/attention.rs:233-240,
    src/model.rs:868-878), on the persistent step and on the oracle."""
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=5)
    prompt = np.random.default_rng(5).integers(0, cfg.vocab, 40).tolist()
    gm = pia.Model(ctx, cfg, w)
    gm.set_decode_path(1)
    gm.kv_alloc(4, 16)
    om_ = orc.OracleModel(cfg, w)
    kv = np.zeros(orc.kv_floats(cfg, 4, 16), np.float32)
    gm.prefill(prompt, 0, [0, 1, 2])
    om_.prefill(prompt, 0, [0, 1, 2], kv, 4, 16)
    tok = 7
    for pos in range(40, 46):
        lg, am = gm.decode([tok], [pos], [[0, 1]])
        assert gm.decode_path_used() == 1
        lc = om_.decode([tok], [pos], [[0, 1]], kv, 4, 16)
        assert _rel(lg[0], lc[0]) <= LOGIT_TOL
        assert int(am[0]) == orc.argmax(lc[0])
        tok = int(am[0])


def test_prefill_tiled_gemm_ragged_shapes(ctx):
    """Prefill of 300 tokens (four whole 64-entry chunks for the LDS-tiled matrix-core GEMM plus
    a 44-entry remainder) at config-1 shapes, whose projections are not whole 128-row tiles
    (gate/up 688 rows, q/k/v 256, o/down 128) and whose K is not whole 64-byte stages
    (down: 344 columns). Logits of the last position and the K/V written by the prefill are
    checked through the following greedy decode steps."""
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=7)
    prompt = np.random.default_rng(7).integers(0, cfg.vocab, 300).tolist()
    g, c, rel = greedy_session(ctx, cfg, w, prompt, 8)
    print(f"tiled prefill: rel max|dlogit|={rel:.3g}")
    assert g == c and rel <= LOGIT_TOL


PREFILL_ATTN = [  # hidden, heads, kv_heads, window, prompt tokens, resume split
    (512, 8, 1, None, 203, 0),    # head_dim 64, 8 heads per kv head, ragged last tile
    (512, 8, 2, None, 187, 37),   # second prefill starts at position 37 (tile window not chunk-aligned)
    (256, 4, 4, 45, 130, 0),      # one head per kv head, sliding window of 45
    (512, 4, 2, None, 100, 0),    # head_dim 128
    (1024, 8, 4, 70, 160, 64),    # head_dim 128, window, resumed prefill
    (1024, 16, 1, None, 150, 0),  # head_dim 64, 16 heads per kv head (four positions per tile)
]


@pytest.mark.parametrize("case", [0, 2, 4])
def test_prefill_tiled_attention_paired(ctx, case, monkeypatch):
    """The causal tile pairing (a workgroup takes tiles t and n - 1 - t) runs by default only on
    grids large enough to fill the chip when halved; here it is forced on small
    prefills: an even tile count, an odd one (the middle tile alone) and a resumed prefill."""
    monkeypatch.setenv("PIA_PREFILL_PAIR", "1")
    test_prefill_tiled_attention(ctx, case)


@pytest.mark.parametrize("case", range(len(PREFILL_ATTN)))
def test_prefill_tiled_attention(ctx, case):
    """Prefills of 64 or more positions run the query-tiled attention kernel (64 query-head
    rows per workgroup: 64/G positions x the G heads of a kv head, causal tiles paired; K/V
    staged in LDS by 64-token chunks, 32 at head_dim 128). Logits of the last position and the K/V written by the prefill (through
    the greedy decode steps that follow) are compared with the oracle."""
    hidden, heads, kvh, window, n, split = PREFILL_ATTN[case]
    print(f"[prefill-attn] hidden={hidden} heads={heads} kv={kvh} window={window} n={n} split={split}", flush=True)
    cfg = pia.LlamaConfig(hidden=hidden, layers=2, heads=heads, kv_heads=kvh, inter=344, vocab=512,
                          attention_window=window)
    w = pia.synth_weights(cfg, seed=20 + case)
    prompt = np.random.default_rng(20 + case).integers(0, cfg.vocab, n).tolist()
    if split == 0:
        g, c, rel = greedy_session(ctx, cfg, w, prompt, 6)
        assert g == c and rel <= LOGIT_TOL, (g, c, rel)
        return
    bs = 16
    nb = (n + 8 + bs - 1) // bs
    table = list(range(nb))
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(nb + 1, bs)
    om_ = orc.OracleModel(cfg, w)
    kv = np.zeros(orc.kv_floats(cfg, nb + 1, bs), np.float32)
    gm.prefill(prompt[:split], 0, table)
    om_.prefill(prompt[:split], 0, table, kv, nb + 1, bs)
    lg, tg = gm.prefill(prompt[split:], split, table)
    lc = om_.prefill(prompt[split:], split, table, kv, nb + 1, bs)
    assert tg == orc.argmax(lc) and _rel(lg, lc) <= LOGIT_TOL
    for i in range(4):
        lg, am = gm.decode([tg], [n + i], [table])
        lc = om_.decode([tg], [n + i], [table], kv, nb + 1, bs)
        assert int(am[0]) == orc.argmax(lc[0]) and _rel(lg[0], lc[0]) <= LOGIT_TOL
        tg = int(am[0])
    gm.close()


def test_persistent_step_llama3_shape(ctx):
    """The persistent step at Llama-3-8B layer shapes (hidden 4096, 32/8 heads, head_dim 128,
    FFN 14336, rotary theta 500000), two layers and a 16k vocabulary to keep the oracle fast:
    300-token prompt (several token splits per kv head), 12 greedy steps."""
    cfg = pia.LlamaConfig(hidden=4096, layers=2, heads=32, kv_heads=8, inter=14336, vocab=16384,
                          rope_theta=500000.0)
    print("[llama3-shape] building weights", flush=True)
    w = pia.synth_weights(cfg, seed=11)
    prompt = np.random.default_rng(11).integers(0, cfg.vocab, 300).tolist()
    g, c, rel = greedy_session(ctx, cfg, w, prompt, 12, path=1, expect_path=1)
    print(f"llama3-shape: rel max|dlogit|={rel:.3g}")
    assert g == c and rel <= LOGIT_TOL


@pytest.mark.slow
def test_config2_tinyllama_b1_greedy_parity(ctx):
    """TinyLlama-1.1B shape, int8 (incl. lm_head), 512-token random prompt,
    256 greedy decode steps at batch 1; greedy tokens bit-exact vs the CPU reference path."""
    cfg = pia.TINYLLAMA
    print("[config2] building weights", flush=True)
    w = pia.synth_weights(cfg, seed=2024)
    prompt = np.random.default_rng(2024).integers(0, cfg.vocab, 512).tolist()
    print("[config2] running GPU + oracle sessions", flush=True)
    g, c, rel = greedy_session(ctx, cfg, w, prompt, 256, expect_path=0)
    assert g == c
    # The same session on the persistent single-launch step.
    g, c, rel1 = greedy_session(ctx, cfg, w, prompt, 256, path=1, expect_path=1)
    rel = max(rel, rel1)
    print(f"config2: rel max|dlogit|={rel:.3g} first tokens {g[:8]}")
    assert g == c
    assert rel <= LOGIT_TOL


def test_config3_shape_batched_paged_decode(ctx):
    """BASELINE config 3 shape: TinyLlama, batch 32, contexts U[128, 2048] from the seed, KV
    blocks of 16 assigned by a random permutation of the pool; the KV history is synthetic
    (seeded) and identical on both sides; 3 greedy steps."""
    cfg = pia.TINYLLAMA
    rng = np.random.default_rng(33)
    B, steps, bs = 32, 3, 16
    ctxs = rng.integers(128, 2049, B)
    need = [(int(c) + steps + bs - 1) // bs for c in ctxs]
    nb = sum(need)
    perm = rng.permutation(nb).tolist()
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n])
        k += n
    print(f"[config3] {nb} blocks, building weights", flush=True)
    w = pia.synth_weights(cfg, seed=33)
    kv = (rng.standard_normal(orc.kv_floats(cfg, nb, bs), dtype=np.float32) * 0.5)
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(nb, bs)
    gm.kv_upload(kv)
    om_ = orc.OracleModel(cfg, w)
    toks_g = rng.integers(0, cfg.vocab, B).tolist()
    toks_c = list(toks_g)
    for s in range(steps):
        pos = [int(c) + s for c in ctxs]
        lg, am = gm.decode(toks_g, pos, tables)
        lc = om_.decode(toks_c, pos, tables, kv, nb, bs)
        rel = max(_rel(lg[b], lc[b]) for b in range(B))
        toks_g = am.tolist()
        toks_c = [orc.argmax(r) for r in lc]
        print(f"[config3] step {s} rel={rel:.3g}", flush=True)
        assert toks_g == toks_c
        assert rel <= LOGIT_TOL
    # The decode writes landed in the same slots: every other slot is untouched (bit-exact) and
    # the written K/V rows agree up to projection rounding.
    got = gm.kv_download().reshape(cfg.layers, nb * bs, -1)
    ref = kv.reshape(cfg.layers, nb * bs, -1)
    written = np.zeros(nb * bs, bool)
    for b in range(B):
        for s in range(steps):
            p = int(ctxs[b]) + s
            written[tables[b][p // bs] * bs + p % bs] = True
    assert np.array_equal(got[:, ~written], ref[:, ~written])
    scale = np.max(np.abs(ref[:, written]))
    assert np.max(np.abs(got[:, written] - ref[:, written])) <= 1e-4 * scale
    gm.close()


def test_prefix_sharing_and_cow_workload(ctx):
    """Config-5 workload in miniature (config-1 shapes): shared prefixes mapped through the
    prefix cache, forks whose first write copies the shared tail block, batched greedy decode.
    Block tables, COW counts and tokens bit-exact between (product manager + GPU model) and
    (oracle manager + oracle model)."""
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=5)
    bs, total = 16, 64
    rng = np.random.default_rng(5)
    prefixes = [rng.integers(0, cfg.vocab, 40).tolist() for _ in range(2)]
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(total, bs)
    kvp, lay = gm.kv_ptr, gm.layout
    om_ = orc.OracleModel(cfg, w)
    kv = np.zeros(orc.kv_floats(cfg, total, bs), np.float32)
    olay = om.KvLayout(cfg.layers, total, bs, cfg.kv_heads, cfg.head_dim)
    mg, mo = pia.KvCacheManager(total, bs), om.KvCacheManager(total, bs)
    seqs = []  # (seq_id, gpu_table, oracle_table, next_pos, gpu_tok, cpu_tok)
    sid, tick = 0, 0
    for pfx in prefixes:
        for rep in range(2):  # second admission of the same prompt hits the prefix cache
            tick += 1
            tg, info = mg.admit(sid, pfx, tick)
            ao = mo.admit(sid, pfx, tick)
            assert tg.blocks() == ao.table.blocks() and info[0] == ao.cached_tokens
            resume = min(info[0], len(pfx) - 1)
            lg, _ = gm.prefill(pfx[resume:], resume, tg.blocks())
            lc = om_.prefill(pfx[resume:], resume, ao.table.blocks(), kv, total, bs)
            assert _rel(lg, lc) <= LOGIT_TOL
            assert mg.publish(tg) == mo.publish_prompt_blocks(ao.table)
            seqs.append([sid, tg, ao.table, len(pfx), orc.argmax(lg), orc.argmax(lc)])
            sid += 1
            # Fork one child off each admitted sequence: it shares the partial tail block.
            tick += 1
            cg = mg.fork(tg, sid, tick)
            co = mo.fork(ao.table, sid, tick)
            seqs.append([sid, cg, co, len(pfx), seqs[-1][4], seqs[-1][5]])
            sid += 1
    for step in range(6):
        tick += 1
        for s in seqs:
            seq_id, tg, to, pos = s[0], s[1], s[2], s[3]
            while len(tg) * bs <= pos:
                assert mg.append_block(seq_id, tg, tick) == mo.append_block(seq_id, to, tick)
            cg = mg.ensure_writable(seq_id, tg, pos, ctx, kvp, lay)
            co = mo.ensure_writable(seq_id, to, pos, lambda a, b: olay.copy_block(kv, a, b))
            assert cg == co and tg.blocks() == to.blocks()
        lg, am = gm.decode([s[4] for s in seqs], [s[3] for s in seqs], [s[1].blocks() for s in seqs])
        lc = om_.decode([s[5] for s in seqs], [s[3] for s in seqs], [s[2].blocks() for s in seqs], kv, total, bs)
        for b, s in enumerate(seqs):
            assert int(am[b]) == orc.argmax(lc[b])
            assert _rel(lg[b], lc[b]) <= LOGIT_TOL
            s[4], s[5], s[3] = int(am[b]), orc.argmax(lc[b]), s[3] + 1
    assert mg.stats()["cow_copies"] == mo.cow_copies > 0
    assert mg.stats()["hits"] == mo.cache.hits
    got = gm.kv_download()
    assert np.max(np.abs(got - kv)) <= 1e-4 * np.max(np.abs(kv))
    gm.close()


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 7, 8, 13, 64, 65, 130])
def test_batched_decode_sizes(ctx, batch):
    """Decode batches on both sides of the streaming-GEMV / matrix-core switch and of the
    64-entry column tiles, ragged contexts, config-1 shapes (K = 344 exercises the padded
    k-steps)."""
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=10 + batch)
    rng = np.random.default_rng(batch)
    bs = 16
    ctxs = rng.integers(1, 90, batch)
    need = [(int(c) + 2 + bs - 1) // bs for c in ctxs]
    nb = sum(need)
    perm = rng.permutation(nb).tolist()
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n])
        k += n
    kv = rng.standard_normal(orc.kv_floats(cfg, nb, bs), dtype=np.float32)
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(nb, bs)
    gm.kv_upload(kv)
    om_ = orc.OracleModel(cfg, w)
    toks = rng.integers(0, cfg.vocab, batch).tolist()
    pos = [int(c) for c in ctxs]
    lg, am = gm.decode(toks, pos, tables)
    lc = om_.decode(toks, pos, tables, kv, nb, bs)
    rel = max(_rel(lg[b], lc[b]) for b in range(batch))
    print(f"[batch {batch}] rel={rel:.3g}")
    assert rel <= LOGIT_TOL
    assert am.tolist() == [orc.argmax(r) for r in lc]
    gm.close()


@pytest.mark.parametrize("batch", [5, 12])
def test_tinyllama_small_batch_decode(ctx, batch):
    """TinyLlama shapes at small batches (the LDS-staged projection kernel; the down projection's
    5632 columns split the batch into groups of 4): logits and greedy tokens vs the oracle."""
    cfg = pia.TINYLLAMA
    rng = np.random.default_rng(500 + batch)
    bs = 16
    ctxs = rng.integers(20, 300, batch)
    need = [(int(c) + 2 + bs - 1) // bs for c in ctxs]
    nb = sum(need)
    perm = rng.permutation(nb).tolist()
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n])
        k += n
    w = pia.synth_weights(cfg, seed=77)
    kv = (rng.standard_normal(orc.kv_floats(cfg, nb, bs), dtype=np.float32) * 0.5)
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(nb, bs)
    gm.kv_upload(kv)
    om_ = orc.OracleModel(cfg, w)
    toks = rng.integers(0, cfg.vocab, batch).tolist()
    pos = [int(c) for c in ctxs]
    lg, am = gm.decode(toks, pos, tables)
    lc = om_.decode(toks, pos, tables, kv, nb, bs)
    rel = max(_rel(lg[b], lc[b]) for b in range(batch))
    print(f"[tinyllama batch {batch}] rel={rel:.3g}", flush=True)
    assert rel <= LOGIT_TOL
    assert am.tolist() == [orc.argmax(r) for r in lc]
    gm.close()



def test_outlier_channels_batched_decode(ctx):
    """Decode at batch 8 (int8 matrix-core projections on digit-split activations) of a model
    whose RMSNorm weights carry 100x and 1000x channels, so every normalized activation row has
    outliers: logits and greedy tokens vs the oracle."""
    cfg = pia.LlamaConfig(hidden=512, layers=2, heads=8, kv_heads=2, inter=1024, vocab=2048)
    w = pia.synth_weights(cfg, seed=91)
    rng = np.random.default_rng(91)
    for lw in w["layers"]:
        for name in ("attn_norm", "ffn_norm"):
            ch = rng.choice(cfg.hidden, 5, replace=False)
            lw[name][ch[:3]] = 100.0
            lw[name][ch[3:]] = 1000.0
    batch, bs = 8, 16
    ctxs = rng.integers(20, 120, batch)
    need = [(int(c) + 4 + bs - 1) // bs for c in ctxs]
    nb = sum(need)
    perm = rng.permutation(nb).tolist()
    tables, k = [], 0
    for n in need:
        tables.append(perm[k:k + n])
        k += n
    kv = (rng.standard_normal(orc.kv_floats(cfg, nb, bs), dtype=np.float32) * 0.5)
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(nb, bs)
    gm.kv_upload(kv)
    om_ = orc.OracleModel(cfg, w)
    toks_g = rng.integers(0, cfg.vocab, batch).tolist()
    toks_c = list(toks_g)
    for s in range(3):
        pos = [int(c) + s for c in ctxs]
        lg, am = gm.decode(toks_g, pos, tables)
        lc = om_.decode(toks_c, pos, tables, kv, nb, bs)
        rel = max(_rel(lg[b], lc[b]) for b in range(batch))
        print(f"[outlier model] step {s} rel={rel:.3g}", flush=True)
        assert rel <= LOGIT_TOL
        toks_g, toks_c = am.tolist(), [orc.argmax(r) for r in lc]
        assert toks_g == toks_c
    gm.close()


def test_device_resident_tables_patch_only_changed_slots(ctx):
    """Block tables stay on the device between decode steps: after the first step (whole image),
    a step sends only the slots that append_block or a copy-on-write remap changed
    (src/memory/block_table.rs:86-93, src/engine.rs:614-693), and its host-to-device bytes are
    exactly tokens + entries + 8 bytes per changed slot. Tokens, logits and the KV cache the steps
    write (through the device tables) match the oracle, which reads the host tables."""
    cfg = pia.TINY_C1
    w = pia.synth_weights(cfg, seed=12)
    bs, total = 16, 64
    rng = np.random.default_rng(12)
    gm = pia.Model(ctx, cfg, w)
    gm.kv_alloc(total, bs)
    om_ = orc.OracleModel(cfg, w)
    kv = np.zeros(orc.kv_floats(cfg, total, bs), np.float32)
    olay = om.KvLayout(cfg.layers, total, bs, cfg.kv_heads, cfg.head_dim)
    mg, mo = pia.KvCacheManager(total, bs, prefix_cache=False), om.KvCacheManager(total, bs, prefix_cache=False)
    seqs, tick = [], 0
    for sid in range(4):
        prompt = rng.integers(0, cfg.vocab, 13 + 7 * sid).tolist()
        tick += 1
        tg, _ = mg.admit(sid, prompt, tick)
        ao = mo.admit(sid, prompt, tick)
        lg, _ = gm.prefill(prompt, 0, tg.blocks())
        lc = om_.prefill(prompt, 0, ao.table.blocks(), kv, total, bs)
        seqs.append([sid, tg, ao.table, len(prompt), orc.argmax(lg), orc.argmax(lc)])
    tick += 1
    seqs.append([4, mg.fork(seqs[0][1], 4, tick), mo.fork(seqs[0][2], 4, tick)] + seqs[0][3:])
    prev = None
    n = len(seqs)
    for step in range(24):
        tick += 1
        for s in seqs:
            sid, tg, to, pos = s[0], s[1], s[2], s[3]
            while len(tg) * bs <= pos:
                assert mg.append_block(sid, tg, tick) == mo.append_block(sid, to, tick)
            assert mg.ensure_writable(sid, tg, pos, ctx, gm.kv_ptr, gm.layout) == \
                mo.ensure_writable(sid, to, pos, lambda a, b: olay.copy_block(kv, a, b))
            assert tg.blocks() == to.blocks()
        tables = [s[1].blocks() for s in seqs]
        lg, am = gm.decode([s[4] for s in seqs], [s[3] for s in seqs], tables)
        lc = om_.decode([s[5] for s in seqs], [s[3] for s in seqs], [s[2].blocks() for s in seqs], kv, total, bs)
        up_bytes, patches, full = gm.last_upload()
        if prev is None:
            assert full
        else:
            changed = sum(1 for t, p in zip(tables, prev) for i in range(len(t)) if i >= len(p) or t[i] != p[i])
            assert not full and patches == changed, (step, patches, changed)
            assert up_bytes == n * 4 + n * 16 + 8 * changed
        prev = [list(t) for t in tables]
        for b, s in enumerate(seqs):
            assert int(am[b]) == orc.argmax(lc[b])
            assert _rel(lg[b], lc[b]) <= LOGIT_TOL
            s[4], s[5], s[3] = int(am[b]), orc.argmax(lc[b]), s[3] + 1
    assert mg.stats()["cow_copies"] == mo.cow_copies == 1
    got = gm.kv_download()
    assert np.max(np.abs(got - kv)) <= 1e-4 * np.max(np.abs(kv))
    gm.close()
