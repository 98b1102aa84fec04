"""Pins the CPU oracle's kernels with known answers, closed forms, invariants and independent
NumPy references (not retyped formulas):
- quantize_rows_i8 (src/math.rs:456-469): hand-computed rows in exact binary fractions;
- dot_i8 / dot (src/simd.rs): the exact f64 sum bounds the f32 result; i8::MIN widening;
  AVX2 and portable paths bit-identical; the batched kernel bit-identical to the single one
  (tests/simd_tests.rs:240-272 of the reference); int8 within 2% of f32 (tests/math_tests.rs);
- PagedAttention::run: the reference's own naive per-head reference design
  (tests/attention_tests.rs:84-131), reduced further to textbook softmax attention on the
  gathered dense K/V in f64; unmapped blocks, empty and sliding windows, shared tables;
- softmax all -inf -> zeros; argmax last-index ties and total order.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def test_quantize_known_answer():
    # Exact binary fractions: max = 127/128 -> scale = 1/128 exactly; halves round away from 0.
    row = np.array([127, 63.5, -63.5, 0.5, -0.5, 1.5, 0.0, -0.0, -127], np.float32) / 128
    q, s = orc.quantize_rows_i8(row[None, :])
    assert s[0] == np.float32(1 / 128)
    assert q[0].tolist() == [127, 64, -64, 1, -1, 2, 0, 0, -127]


def test_quantize_zero_row_scale_is_one():
    q, s = orc.quantize_rows_i8(np.zeros((2, 5), np.float32))
    assert s.tolist() == [1.0, 1.0] and not q.any()


def test_quantize_roundtrip_and_range():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, (64, 333)).astype(np.float32)
    q, s = orc.quantize_rows_i8(w)
    assert q.min() >= -127 and q.max() <= 127
    assert np.all(np.abs(q).max(axis=1) == 127)
    err = np.abs(q.astype(np.float64) * s[:, None] - w)
    assert np.all(err <= s[:, None] * 0.5 * (1 + 1e-6))  # round-to-nearest bound


def test_dot_i8_sign_extension():
    w = np.array([-128, 127, -1, 0, 1, -128, 127, -1, 5], np.int8)
    assert orc.dot_i8(w, np.ones(9, np.float32)) == float(w.astype(np.int64).sum())


@pytest.mark.parametrize("n", [0, 1, 7, 8, 31, 32, 33, 64, 129, 2048, 5632])
def test_dot_i8_error_bound_and_paths(n):
    rng = np.random.default_rng(n)
    w = rng.integers(-127, 128, n).astype(np.int8)
    x = rng.normal(0, 1, n).astype(np.float32)
    exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    got = orc.dot_i8(w, x)
    bound = n * 2 ** -23 * float(np.sum(np.abs(w.astype(np.float64) * x))) + 1e-30
    assert abs(got - exact) <= bound
    orc.lib().orc_force_portable(1)
    try:
        port = orc.dot_i8(w, x)
        portf = orc.dot(x, x)
    finally:
        orc.lib().orc_force_portable(0)
    assert port == got  # the lane emulation reproduces the AVX2 rounding exactly
    assert portf == orc.dot(x, x)


def test_batched_matmat_bit_identical_to_matvec():
    rng = np.random.default_rng(7)
    for rows, cols, batch in [(3, 7, 1), (17, 33, 3), (64, 129, 5), (40, 2048, 9)]:
        q = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
        s = rng.uniform(0.001, 0.01, rows).astype(np.float32)
        x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
        mm = orc.matmat_i8(q, s, x)
        for b in range(batch):
            assert np.array_equal(mm[:, b], orc.matvec_i8(q, s, x[b]))


def test_int8_matvec_tracks_f32():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (48, 96)).astype(np.float32)
    x = rng.normal(0, 1, 96).astype(np.float32)
    q, s = orc.quantize_rows_i8(w)
    f = orc.matvec_f32(w, x)
    i8 = orc.matvec_i8(q, s, x)
    dq = (q.astype(np.float64) * s[:, None].astype(np.float64)) @ x.astype(np.float64)
    assert np.allclose(i8, dq, rtol=1e-5, atol=1e-6)
    assert np.all(np.abs(f - i8) <= 0.02 * np.abs(f) + 3e-3)


def test_softmax_all_masked_is_zero():
    assert orc.softmax([-np.inf] * 5).tolist() == [0.0] * 5
    p = orc.softmax([1.0, 2.0, -np.inf])
    assert p[2] == 0.0 and abs(p.sum() - 1) < 1e-6


def test_argmax_ties_and_total_order():
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 2
    assert orc.argmax([0.0, -0.0]) == 0  # +0 > -0 under total_cmp
    assert orc.argmax([-0.0, 0.0]) == 1
    assert orc.argmax([-1.0, -2.0]) == 0


def test_rope_table_close_to_f64():
    c, s = orc.rope_table(777, 64, 10000.0)
    j = np.arange(32)
    ang = 777 * (1.0 / 10000.0 ** (2 * j / 64))
    assert np.allclose(c, np.cos(ang), atol=2e-4) and np.allclose(s, np.sin(ang), atol=2e-4)


def _attention_dense_f64(q, kv, layout, heads, entries, tables, layer):
    """Textbook softmax attention on K/V gathered through the block table (f64)."""
    nl, nb, bs, hkv, hd = layout
    kvr = kv.reshape(nl, nb, bs, hkv, 2, hd).astype(np.float64)
    g = heads // hkv
    out = np.zeros((len(entries), heads * hd))
    for e, ((pos, start), tab) in enumerate(zip(entries, tables)):
        ts = list(range(start, pos + 1))
        mapped = [t for t in ts if t // bs < len(tab)]
        if not mapped:
            continue
        for h in range(heads):
            K = np.stack([kvr[layer, tab[t // bs], t % bs, h // g, 0] for t in mapped])
            V = np.stack([kvr[layer, tab[t // bs], t % bs, h // g, 1] for t in mapped])
            sc = K @ q[e, h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
            p = np.exp(sc - sc.max())
            out[e, h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


def _case(rng, heads, hkv, hd, bs, nblocks, layers=2):
    layout = (layers, nblocks, bs, hkv, hd)
    kv = rng.uniform(-1.3, 1.6, layers * nblocks * bs * hkv * 2 * hd).astype(np.float32)
    return layout, kv


@pytest.mark.parametrize("heads,hkv,hd", [(8, 2, 4), (4, 2, 32), (32, 4, 64), (8, 8, 16)])
def test_attention_matches_dense_reference(heads, hkv, hd):
    rng = np.random.default_rng(heads * 100 + hd)
    bs = 8
    layout, kv = _case(rng, heads, hkv, hd, bs, 20)
    perm = rng.permutation(20).tolist()  # scattered physical blocks
    tables = [perm[0:5], perm[5:11], perm[11:14]]
    entries = [(33, 0), (40, 0), (20, 0)]
    q = rng.normal(0, 1, (3, heads * hd)).astype(np.float32)
    got = orc.paged_attention(q, kv, layout, heads, entries, tables, 1)
    ref = _attention_dense_f64(q, kv, layout, heads, entries, tables, 1)
    assert np.allclose(got, ref, atol=2e-5, rtol=1e-4)


def test_attention_unmapped_masked_and_empty_window():
    rng = np.random.default_rng(5)
    heads, hkv, hd, bs = 8, 2, 4, 8
    layout, kv = _case(rng, heads, hkv, hd, bs, 10)
    q = rng.normal(0, 1, (3, heads * hd)).astype(np.float32)
    # Entry 0 maps 2 of 6 blocks: positions past them must be masked, which equals attending
    # to the mapped span only (tests/attention_tests.rs:227-253 of the reference).
    masked = orc.paged_attention(q[:1], kv, layout, heads, [(40, 0)], [[3, 7]], 0)
    trunc = orc.paged_attention(q[:1], kv, layout, heads, [(15, 0)], [[3, 7]], 0)
    assert np.array_equal(masked, trunc)
    # Empty window (start > pos) and a fully unmapped window attend to nothing -> zeros.
    z = orc.paged_attention(q[:2], kv, layout, heads, [(4, 5), (9, 0)], [[1], []], 0)
    assert not z.any()


def test_attention_sliding_window_and_shared_table():
    rng = np.random.default_rng(9)
    heads, hkv, hd, bs = 8, 4, 4, 16
    layout, kv = _case(rng, heads, hkv, hd, bs, 6)
    tab = [5, 2, 4, 0]
    for pos in [0, 1, 15, 16, 17, 31, 47]:
        for w in [1, 2, 3]:
            q = rng.normal(0, 1, (1, heads * hd)).astype(np.float32)
            start = max(0, pos + 1 - w)
            got = orc.paged_attention(q, kv, layout, heads, [(pos, start)], [tab], 1)
            ref = _attention_dense_f64(q, kv, layout, heads, [(pos, start)], [tab], 1)
            assert np.allclose(got, ref, atol=2e-5, rtol=1e-4)
    # Entries sharing one table stay independent (prefill / speculative batches).
    q = rng.normal(0, 1, (3, heads * hd)).astype(np.float32)
    ents = [(7, 0), (19, 0), (33, 0)]
    both = orc.paged_attention(q, kv, layout, heads, ents, [tab] * 3, 0)
    for i, e in enumerate(ents):
        assert np.array_equal(both[i], orc.paged_attention(q[i:i + 1], kv, layout, heads, [e], [tab], 0)[0])
