"""mbk_node_hist_split_noalloc (every scratch buffer in the library's fixed
device array) against mbk_node_hist_split (scratch owned by the context) on
the same inputs: histograms and split records bit for bit, on calls in a row
whose inputs shrink, so a result left over from the previous call cannot
pass; inputs past the array's limits fail with an error."""
import ctypes

import numpy as np
import pytest

import macboost_amd as mb
from macboost_amd import _core

pytestmark = pytest.mark.gpu

RESULT_BYTES = 72       # sizeof(mbk_split_result)


def _inputs(rng, rows, cols, nb, tile_w, n):
    bins = rng.integers(0, nb, size=(cols, rows)).astype(np.uint8)
    bins[3 % cols, rng.random(rows) < 0.3] = nb - 1               # missing values
    is_cat = np.zeros(cols, np.uint8)
    if cols > 4:
        bins[4] = rng.integers(0, 5, size=rows)                    # categorical
        is_cat[4] = 1
    mono = np.zeros(cols, np.int8)
    if cols > 8:
        mono[7], mono[8] = 1, -1
    qg = rng.integers(-32767, 32768, size=rows)
    qh = rng.integers(0, 128, size=rows)
    ghq = (((qg & 0xFFFF).astype(np.uint32) << 16) | qh.astype(np.uint32)).astype(np.uint32)
    idx = np.sort(rng.choice(rows, n, replace=False)).astype(np.uint32)
    T = (cols + tile_w - 1) // tile_w
    tiled = np.zeros((rows, T, tile_w), np.uint8)
    for f in range(cols):
        tiled[:, f // tile_w, f % tile_w] = bins[f]
    ent = np.stack([idx, ghq[idx]], axis=1).astype(np.uint32)
    mgh = np.array([3.5, 0.25], np.float32).view(np.uint32)
    return tiled, ent, mgh, is_cat, mono


def _call(ctx, name, dev, rows, cols, nb, tile_w, n):
    dt, de, dm, dc, dmo = dev
    # outputs start as garbage: nothing may survive from an earlier call
    dh = ctx.upload(np.full(nb * cols * 2, -1, np.int64))
    dr = ctx.upload(np.full(cols * RESULT_BYTES, 0xAB, np.uint8))
    err = ctypes.c_char_p()
    rc = getattr(_core.lib(), name)(ctx.ptr, dt, rows, cols, nb, tile_w, de, n, dm, dc, dmo,
                                    1.0, 1.0, 10.0, dh, dr, ctypes.byref(err))
    if rc != 0:
        raise mb.MacBoostError(_core._take_error(err))
    ctx.sync()
    return ctx.download(dh, (nb, cols, 2), np.int64), ctx.download(dr, (cols, RESULT_BYTES),
                                                                   np.uint8)


def test_noalloc_equals_the_allocating_entry_point():
    ctx = mb.Context(0)
    rng = np.random.default_rng(2024)
    cases = [(400_000, 100, 256, 64, 350_000),   # many items
             (60_000, 100, 256, 64, 7_001),      # smaller: the array keeps the last call's bytes
             (100_000, 100, 256, 32, 90_000),    # 32-wide tiles, the last tile folded in
             (9_000, 13, 64, 16, 5_000),         # another tile width and bin count
             (2_000, 5, 17, 8, 0)]               # an empty node
    for rows, cols, nb, tile_w, n in cases:
        tiled, ent, mgh, is_cat, mono = _inputs(rng, rows, cols, nb, tile_w, n)
        dev = (ctx.upload(tiled), ctx.upload(ent), ctx.upload(mgh), ctx.upload(is_cat),
               ctx.upload(mono))
        h0, r0 = _call(ctx, "mbk_node_hist_split_noalloc", dev, rows, cols, nb, tile_w, n)
        h1, r1 = _call(ctx, "mbk_node_hist_split", dev, rows, cols, nb, tile_w, n)
        assert np.array_equal(h0, h1), (rows, cols, nb, tile_w, n)
        assert np.array_equal(r0, r1), (rows, cols, nb, tile_w, n)
        assert int(h0[:, 0, 1].sum()) == int((ent[:, 1] & 0x7F).astype(np.int64).sum())
    ctx.close()


def test_noalloc_rejects_inputs_past_its_limits():
    ctx = mb.Context(0)
    rng = np.random.default_rng(7)
    tiled, ent, mgh, is_cat, mono = _inputs(rng, 1000, 5, 64, 8, 100)
    dev = (ctx.upload(tiled), ctx.upload(ent), ctx.upload(mgh), ctx.upload(is_cat),
           ctx.upload(mono))
    with pytest.raises(mb.MacBoostError, match="1..4096 features"):
        _call(ctx, "mbk_node_hist_split_noalloc", dev, 1000, 5000, 64, 8, 100)
    # the next call in range still works
    h0, r0 = _call(ctx, "mbk_node_hist_split_noalloc", dev, 1000, 5, 64, 8, 100)
    h1, r1 = _call(ctx, "mbk_node_hist_split", dev, 1000, 5, 64, 8, 100)
    assert np.array_equal(h0, h1) and np.array_equal(r0, r1)
    ctx.close()
