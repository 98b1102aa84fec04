"""GPU kernel parity through the C ABI against the CPU oracle on the same seeded inputs.
Integer / index work (quantizer, block copy, argmax, block mapping) must be bit-exact; the
f32 projections and attention may differ from the reference's summation order only by
rounding, bounded here relative to sum(|w*x|) (projections) or 1e-5 (attention)."""
import numpy as np
import pytest

import pia
from oracle import memory as om
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _proj_case(rng, rows, cols, batch):
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    q, s = pia.quantize_rows_i8(w)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    return q, s, x


def _proj_bound(q, s, x):
    # |f32 dot in any order - exact| <= cols * 2^-24 * sum|q x| (x2 for the scale rounding).
    mag = np.abs(x.astype(np.float64)) @ np.abs(q.astype(np.float64)).T * s.astype(np.float64)[None, :]
    return 2.0 * q.shape[1] * 2.0 ** -24 * mag + 1e-30


SHAPES = [(1, 1, 1), (3, 7, 2), (17, 33, 3), (344, 128, 1), (128, 344, 5), (64, 129, 8), (2560, 2048, 1),
          (2048, 5632, 1), (11264, 2048, 2), (1000, 2048, 13), (333, 4096, 32), (32000, 2048, 1),
          # small batches on the LDS-staged kernel, including row groups split by LDS capacity
          (11264, 2048, 5), (2048, 5632, 6), (4096, 14336, 3), (50, 64, 16), (64, 48, 9), (2560, 2048, 8),
          # prefill tiles: 128 x 192 with a ragged tail; 256 x 384 over pairs of 64-entry chunks, the
          # odd last chunk on a 128 x 192 tile and a ragged tail (the [row][batch] output takes the
          # strided epilogue stores, the [batch][row] one the vector stores)
          (2560, 384, 300), (16384, 256, 1027)]


@pytest.mark.parametrize("rows,cols,batch", SHAPES)
def test_int8_projection_matches_oracle(ctx, rows, cols, batch):
    print(f"[gemv] rows={rows} cols={cols} batch={batch}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + batch)
    q, s, x = _proj_case(rng, rows, cols, batch)
    ref = orc.matmat_i8(q, s, x)  # [row][batch]
    dq, ds, dx = ctx.to_device(q), ctx.to_device(s), ctx.to_device(x)
    out_rb = ctx.empty((rows, batch), np.float32)
    pia.check(pia.lib().pia_matmat_i8_dev(ctx.h, out_rb.ptr, dx.ptr, dq.ptr, ds.ptr, batch, rows, cols, None))
    out_br = ctx.empty((batch, rows), np.float32)
    pia.check(pia.lib().pia_qlinear_apply_dev(ctx.h, out_br.ptr, dx.ptr, dq.ptr, ds.ptr, batch, rows, cols, None))
    ctx.sync()
    bound = _proj_bound(q, s, x).T  # [row][batch]
    got_rb = out_rb.numpy()
    assert np.all(np.abs(got_rb - ref) <= bound)
    assert np.array_equal(out_br.numpy(), got_rb.T)
    # Host-pointer forms run the same kernels: identical bits.
    host_rb = np.empty((rows, batch), np.float32)
    pia.check(pia.lib().pia_matmat_i8(ctx.h, pia.ptr(host_rb), pia.ptr(x), pia.ptr(q), pia.ptr(s), batch, rows, cols))
    assert np.array_equal(host_rb, got_rb)
    host_br = np.empty((batch, rows), np.float32)
    pia.check(pia.lib().pia_qlinear_apply(ctx.h, pia.ptr(host_br), pia.ptr(x), pia.ptr(q), pia.ptr(s), batch, rows,
                                          cols))
    assert np.array_equal(host_br, got_rb.T)
    if batch == 1:
        out = np.empty(rows, np.float32)
        pia.check(pia.lib().pia_matvec_i8(ctx.h, pia.ptr(out), pia.ptr(x[0]), pia.ptr(q), pia.ptr(s), rows, cols))
        assert np.array_equal(out, got_rb[:, 0])


def test_device_quantizer_bit_exact(ctx):
    rng = np.random.default_rng(5)
    for w in [rng.normal(0, 0.02, (300, 2048)), np.zeros((2, 33)), rng.integers(-500, 500, (7, 100)) / 8.0]:
        w = w.astype(np.float32)
        q_ref, s_ref = orc.quantize_rows_i8(w)
        dw = ctx.to_device(w)
        dq, ds = ctx.empty(w.shape, np.int8), ctx.empty((w.shape[0],), np.float32)
        pia.check(pia.lib().pia_quantize_rows_i8_dev(ctx.h, dw.ptr, w.shape[0], w.shape[1], dq.ptr, ds.ptr, None))
        ctx.sync()
        assert np.array_equal(dq.numpy(), q_ref)
        assert np.array_equal(ds.numpy().view(np.uint32), s_ref.view(np.uint32))


def _attn_entries(entries, tables):
    off, ln, flat = orc.flatten_tables(tables)
    arr = np.zeros((len(entries), 4), np.int32)
    for i, (pos, start) in enumerate(entries):
        arr[i] = (pos, start, off[i], ln[i])
    return arr, flat


ATTN = [  # heads, kv_heads, head_dim, block_size, windows
    (8, 2, 4, 8, [(33, 0), (40, 0), (20, 0)]),
    (4, 2, 24, 16, [(39, 0), (5, 0)]),
    (32, 4, 64, 16, [(700, 0), (129, 0), (255, 0), (256, 0), (1500, 0)]),
    (32, 8, 128, 16, [(1300, 0), (17, 0)]),
    (16, 16, 32, 4, [(63, 0), (10, 3), (5, 6)]),
]


@pytest.mark.parametrize("case", range(len(ATTN)))
def test_paged_attention_matches_oracle(ctx, case):
    heads, hkv, hd, bs, entries = ATTN[case]
    print(f"[attention] heads={heads} kv={hkv} hd={hd} bs={bs} entries={entries}", flush=True)
    rng = np.random.default_rng(case)
    layers = 2
    need = [(pos + bs) // bs for pos, _ in entries]
    nblocks = sum(need) + 3
    layout = (layers, nblocks, bs, hkv, hd)
    kv = rng.uniform(-1.3, 1.6, layers * nblocks * bs * hkv * 2 * hd).astype(np.float32)
    perm = rng.permutation(nblocks).tolist()
    tables, k = [], 0
    for i, n in enumerate(need):
        mapped = n if i != 1 else max(1, n // 2)  # entry 1 leaves its tail unmapped
        tables.append(perm[k:k + mapped])
        k += n
    q = rng.normal(0, 1, (len(entries), heads * hd)).astype(np.float32)
    ref = orc.paged_attention(q, kv, layout, heads, entries, tables, 1)
    ent, flat = _attn_entries(entries, tables)
    dq, dkv, de, dt = ctx.to_device(q), ctx.to_device(kv), ctx.to_device(ent), ctx.to_device(flat)
    out = ctx.empty(q.shape, np.float32)
    L = pia.KvLayout(*layout)
    pia.check(pia.lib().pia_paged_attention_dev(ctx.h, out.ptr, dq.ptr, dkv.ptr, L, heads, de.ptr, dt.ptr,
                                                len(entries), 1, None))
    got = out.numpy()
    assert np.allclose(got, ref, atol=1e-5, rtol=1e-5), np.max(np.abs(got - ref))


def test_kv_write_matches_oracle(ctx):
    # The standalone KV scatter (model.rs:1093-1107): mapped positions land where the layout
    # says, unmapped ones (entry 2) write nothing, other layers are untouched.
    layout = (3, 9, 4, 2, 8)
    rng = np.random.default_rng(11)
    L, oL = pia.KvLayout(*layout), om.KvLayout(*layout)
    kv = rng.normal(size=oL.total_floats()).astype(np.float32)
    tables = [[7, 2, 5], [0], [3]]
    entries = [(9, 0), (3, 0), (4, 0)]  # entry 2: logical block 1 is past its table
    n, hkv, hd = len(entries), layout[3], layout[4]
    k = rng.normal(size=(n, hkv, hd)).astype(np.float32)
    v = rng.normal(size=(n, hkv, hd)).astype(np.float32)
    ref = kv.copy()
    for i, (pos, _) in enumerate(entries):
        t = om.BlockTable()
        for b in tables[i]:
            t.append_block(b)
        oL.write_token(ref, 1, t, pos, k[i], v[i])
    ent, flat = _attn_entries(entries, tables)
    dkv, dk, dv, de, dt = ctx.to_device(kv), ctx.to_device(k), ctx.to_device(v), ctx.to_device(ent), ctx.to_device(flat)
    print("[kv_write] layout", layout, flush=True)
    pia.check(pia.lib().pia_kv_write_dev(ctx.h, dkv.ptr, L, dk.ptr, dv.ptr, de.ptr, dt.ptr, n, 1, None))
    ctx.sync()
    assert np.array_equal(dkv.numpy(), ref)
    # Out-of-range block ids and layers are rejected on the host before any launch.
    bad = ctx.to_device(np.array([7, 2, 99, 0, 3], np.int32))
    assert pia.lib().pia_kv_write_dev(ctx.h, dkv.ptr, L, dk.ptr, dv.ptr, de.ptr, bad.ptr, n, 1, None) != 0
    assert pia.lib().pia_kv_write_dev(ctx.h, dkv.ptr, L, dk.ptr, dv.ptr, de.ptr, dt.ptr, n, 3, None) != 0
    out = ctx.empty((n, 4 * hd), np.float32)
    q = ctx.to_device(rng.normal(size=(n, 4 * hd)).astype(np.float32))
    assert pia.lib().pia_paged_attention_dev(ctx.h, out.ptr, q.ptr, dkv.ptr, L, 4, de.ptr, bad.ptr, n, 1, None) != 0
    ctx.sync()
    assert np.array_equal(dkv.numpy(), ref)


def test_copy_block_and_device_cow(ctx):
    layout = (3, 4, 2, 2, 4)
    L = pia.KvLayout(*layout)
    kv = np.arange(np.prod(layout) * 2, dtype=np.float32)
    for src, dst in [(1, 3), (3, 1)]:
        dkv = ctx.to_device(kv)
        pia.check(pia.lib().pia_kv_copy_block_dev(ctx.h, dkv.ptr, L, src, dst, None))
        ref = kv.copy()
        om.KvLayout(*layout).copy_block(ref, src, dst)
        assert np.array_equal(dkv.numpy(), ref)
    # ensure_writable moves block data on the device (kv_cache_manager.rs:289-327).
    m = pia.KvCacheManager(4, 2)
    t, _ = m.admit(1, [1, 2, 3], 1)
    c = m.fork(t, 2, 2)
    dkv = ctx.to_device(kv)
    assert m.ensure_writable(2, c, 3, ctx, dkv.ptr, L)
    ctx.sync()
    ref = kv.copy()
    om.KvLayout(*layout).copy_block(ref, t.blocks()[1], c.blocks()[1])
    assert np.array_equal(dkv.numpy(), ref)


def test_argmax_ties_total_order(ctx):
    rows = np.array([[1, 3, 3, 2], [0.0, -0.0, -1, -2], [-0.0, 0.0, -1, -2], [-5, -4, -4, -7]], np.float32)
    big = np.random.default_rng(0).normal(0, 1, (3, 32000)).astype(np.float32)
    big[1, [5, 31999]] = 100.0
    for logits in (rows, big):
        d = ctx.to_device(logits)
        out = ctx.empty((logits.shape[0],), np.int32)
        pia.check(pia.lib().pia_argmax_dev(ctx.h, out.ptr, d.ptr, logits.shape[0], logits.shape[1], None))
        ctx.sync()
        assert out.numpy().tolist() == [orc.argmax(r) for r in logits]


def _outlier_case(rng, rows, cols, batch):
    """Activations N(0,1) with channels scaled by 100 and 1000 (the outlier channels of real
    Llama activations), weight rows N(0, 0.02) quantized, and the first 16 rows built to
    expose a fixed-point image tied to the row maximum: zero weights on the outlier channels,
    maximal (+-127) weights everywhere else."""
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    big100 = rng.choice(cols, 3, replace=False)
    big1000 = rng.choice(np.setdiff1d(np.arange(cols), big100), 2, replace=False)
    x[:, big100] *= 100.0
    x[:, big1000] *= 1000.0
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    q, s = pia.quantize_rows_i8(w)
    q[:16] = np.where(rng.random((16, cols)) < 0.5, -127, 127).astype(np.int8)
    q[:16, big100] = 0
    q[:16, big1000] = 0
    s[:16] = np.float32(0.02 / 127)
    return q, s, x


def _digit_bound(q, s, x):
    """Error bound of the matrix-core projection: each activation row b is rounded to the
    fixed-point grid 2^(e_b - 22), max|x_b| < 2^e_b (|error| <= 2^(e_b - 23) per element); the
    integer dot is exact; the int64 -> f32 conversion and the scale multiply round twice."""
    m = np.max(np.abs(x.astype(np.float64)), axis=1)
    e = np.frexp(m)[1].astype(np.float64)  # m = f * 2^e, f in [0.5, 1)
    grid = np.ldexp(1.0, (e - 23).astype(np.int64))  # half a grid step, per batch row
    qa = np.abs(q.astype(np.float64))
    exact = (x.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)[None, :]
    bound = (grid[:, None] * (qa.sum(axis=1)[None, :] * s.astype(np.float64)[None, :])) * (1 + 2.0 ** -20)
    return exact, bound + 2.0 ** -22 * np.abs(exact) + 1e-30


@pytest.mark.parametrize("rows,cols,batch", [(512, 2048, 8), (4096, 4096, 32), (256, 14336, 64)])
def test_digit_split_outlier_activations(ctx, rows, cols, batch):
    """The int8 matrix-core projection (three 8-bit digits of a 23-bit fixed-point image of each
    activation row) on rows with 100x and 1000x outlier channels: within its stated bound of the
    exact (f64) projection, and within that bound plus the oracle's f32 bound of the
    oracle (src/simd.rs:228-262 accumulation order)."""
    print(f"[digits-outlier] rows={rows} cols={cols} batch={batch}", flush=True)
    rng = np.random.default_rng(rows + cols + batch)
    q, s, x = _outlier_case(rng, rows, cols, batch)
    dq, ds, dx = ctx.to_device(q), ctx.to_device(s), ctx.to_device(x)
    out = ctx.empty((batch, rows), np.float32)
    pia.check(pia.lib().pia_qlinear_apply_dev(ctx.h, out.ptr, dx.ptr, dq.ptr, ds.ptr, batch, rows, cols, None))
    ctx.sync()
    got = out.numpy().astype(np.float64)
    exact, bound = _digit_bound(q, s, x)
    err = np.abs(got - exact)
    assert np.all(err <= bound), float(np.max(err / bound))
    ref = orc.matmat_i8(q, s, x).T.astype(np.float64)  # [batch][row]
    ref_bound = _proj_bound(q, s, x)
    assert np.all(np.abs(got - ref) <= bound + ref_bound)
    # How the two errors compare on the rows built against the fixed-point image, relative to
    # the scale of those outputs: far inside the logit tolerance (2e-3) the model is held to.
    scale = float(np.max(np.abs(exact[:, :16])))
    rel = float(np.max(err[:, :16])) / scale
    rel_ref = float(np.max(np.abs(ref - exact)[:, :16])) / scale
    print(f"[digits-outlier] max rel error: matrix cores {rel:.3g}, oracle f32 {rel_ref:.3g}", flush=True)
    assert rel < 1e-3
