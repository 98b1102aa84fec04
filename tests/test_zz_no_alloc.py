"""The allocation-free projection entry point (pia_qlinear_apply_noalloc_dev) gives exactly the
bits of pia_qlinear_apply_dev (same kernels; the scratch is the fixed per-device array instead
of the context's workspace) on two calls in a row, the second smaller; the GEMV path (batch < 5)
and the argument limits are covered too."""
import numpy as np
import pytest

import pia

pytestmark = pytest.mark.gpu


def _case(rng, rows, cols, batch):
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    q, s = pia.quantize_rows_i8(w)
    x = rng.normal(0, 1, (batch, cols)).astype(np.float32)
    return q, s, x


def _run(ctx, fn, q, s, x):
    batch, cols = x.shape
    rows = q.shape[0]
    dq, ds, dx = ctx.to_device(q), ctx.to_device(s), ctx.to_device(x)
    out = ctx.empty((batch, rows), np.float32)
    pia.check(fn(ctx.h, out.ptr, dx.ptr, dq.ptr, ds.ptr, batch, rows, cols, None))
    ctx.sync()
    return out.numpy()


def test_noalloc_projection_matches_allocating_entry_point(ctx):
    rng = np.random.default_rng(77)
    L = pia.lib()
    # Large first (split-K on the matrix cores, every digit group), then smaller: the second call
    # reuses the scratch the first left behind. Then the streaming-GEMV path and a ragged shape.
    for rows, cols, batch in [(4096, 14336, 64), (1000, 2048, 13), (2560, 2048, 3), (333, 4096, 32)]:
        print(f"[noalloc] rows={rows} cols={cols} batch={batch}", flush=True)
        q, s, x = _case(rng, rows, cols, batch)
        want = _run(ctx, L.pia_qlinear_apply_dev, q, s, x)
        got = _run(ctx, L.pia_qlinear_apply_noalloc_dev, q, s, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_projection_rejects_sizes_beyond_its_scratch(ctx):
    L = pia.lib()
    rng = np.random.default_rng(5)
    for rows, cols, batch in [(64, 64, 65), (64, 16448, 8)]:
        q, s, x = _case(rng, rows, cols, batch)
        with pytest.raises(pia.PiaError, match="at most 64 batch rows"):
            _run(ctx, L.pia_qlinear_apply_noalloc_dev, q, s, x)
