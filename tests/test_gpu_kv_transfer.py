"""KV windows in flight between HBM and host memory (zr_transfer): the
eviction / restore copies of the KV-pressure path on streams of their own.

Against the synchronous export / import (zrh_export_kv / zrh_import_kv,
forward_pass.rs:1169-1242), bit for bit:
* an async export's host copy, also when the session's pages are handed to
  another session and overwritten before the copy is waited for;
* an import straight from a still-running export's device buffer;
* an import from an upload;
* the segmented retention window.
"""
import numpy as np
import pytest

from mesh_amd import DeviceContext, KVCacheSnapshot, ModelGeometry

pytestmark = pytest.mark.gpu


def _ctx(kv_dtype):
    geo = ModelGeometry(hidden=2048, num_heads=32, num_kv_heads=4, num_layers=3, vocab=64, ffn=64)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=64, max_seqs=8, max_pages_per_seq=64)
    ctx.create_kv_pool(64)
    return ctx, geo


def _snap(rng, geo, rows, next_position, kv_dtype):
    k = rng.standard_normal((geo.num_layers, rows, geo.kv_cols), dtype=np.float32)
    v = rng.standard_normal((geo.num_layers, rows, geo.kv_cols), dtype=np.float32)
    if kv_dtype == "bf16":  # values the pool holds exactly
        k = (k.view(np.uint32) & 0xFFFF0000).view(np.float32)
        v = (v.view(np.uint32) & 0xFFFF0000).view(np.float32)
    return KVCacheSnapshot(next_position, rows, k, v)


def _same(a, b):
    assert a.cached_tokens == b.cached_tokens and a.next_position == b.next_position
    np.testing.assert_array_equal(a.keys, b.keys)
    np.testing.assert_array_equal(a.values, b.values)


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_async_export_survives_page_reuse_and_restores_from_its_device_buffer(kv_dtype):
    ctx, geo = _ctx(kv_dtype)
    rng = np.random.default_rng(11)
    a = ctx.new_backend(4096)
    a.import_kv_cache(_snap(rng, geo, 300, 1000, kv_dtype))
    want = a.export_kv_cache(200)                      # the synchronous export of the window
    snap, t = a.export_kv_cache_async(200)             # newest 200 rows, copy in flight
    assert snap.cached_tokens == 200 and snap.next_position == 1000
    a.close()                                          # pages back to the pool at once
    # another session takes those pages and overwrites them before the copy is waited for
    c = ctx.new_backend(4096)
    other = _snap(rng, geo, 300, 400, kv_dtype)
    c.import_kv_cache(other)
    # restore from the export's device buffer while its host copy may still run
    b = ctx.new_backend(4096)
    b.import_kv_cache_transfer(snap, t)
    t.wait()
    _same(snap, want)
    _same(b.export_kv_cache(), want)
    _same(c.export_kv_cache(), other)
    t.close()
    ctx.close()


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_upload_then_import_equals_synchronous_import(kv_dtype):
    ctx, geo = _ctx(kv_dtype)
    rng = np.random.default_rng(12)
    src = ctx.new_backend(4096)
    src.import_kv_cache(_snap(rng, geo, 77, 5077, kv_dtype))
    snap, t = src.export_kv_cache_async()              # pinned host copy of all 77 rows
    t.wait()
    t.close()
    want = src.export_kv_cache()
    _same(snap, want)
    for _ in range(2):                                 # the second upload reuses a finished buffer
        up = ctx.upload_kv_async(snap)
        d = ctx.new_backend(4096)
        d.import_kv_cache_transfer(snap, up)
        _same(d.export_kv_cache(), want)
        assert d.sequence_position() == 5077
        up.close()
        d.close()
    # a transfer holds one window: another row count is refused, the session unchanged
    e = ctx.new_backend(4096)
    up = ctx.upload_kv_async(snap)
    short = KVCacheSnapshot(5076, 76, snap.keys[:, :76].copy(), snap.values[:, :76].copy())
    with pytest.raises(RuntimeError, match="KV transfer holds 77 rows, not 76"):
        e.import_kv_cache_transfer(short, up)
    assert e.cache_seq_len() == 0
    up.close()
    ctx.close()


def test_kept_transfer_buffers_stay_bounded():
    """Finished transfers keep their device buffers for reuse: at most the 8
    largest, and a window that fits none of them frees the smaller ones."""
    ctx, geo = _ctx("f32")
    rng = np.random.default_rng(13)
    lib = ctx.lib
    per_row = 2 * geo.num_layers * geo.kv_cols * 4  # K and V bytes of one row
    for rows in range(10, 130, 8):  # 15 windows, each larger than every buffer before it
        up = ctx.upload_kv_async(_snap(rng, geo, rows, rows, "f32"))
        up.wait()
        up.close()
        cached = lib.zr_transfer_cached_bytes(ctx.h)
        # the window's own buffer (plus its page-table room) is all that is kept
        assert rows * per_row <= cached <= rows * per_row + 4 * 64, (rows, cached)
    ups = [ctx.upload_kv_async(_snap(rng, geo, r, r, "f32")) for r in (5, 6, 7, 8, 9, 10, 11, 12, 13, 14)]
    for up in ups:
        up.wait()
        up.close()
    cached = lib.zr_transfer_cached_bytes(ctx.h)
    assert cached <= 8 * (122 * per_row + 4 * 64), cached  # 8 buffers at most, the largest 122 rows
    ctx.close()


@pytest.mark.parametrize("first_row", [0, 37])
def test_scatter_transfer_takes_a_whole_session_table(first_row):
    """zr_kv_scatter_transfer with the session's full block table (spare pages
    included) writes the same rows zr_kv_scatter does."""
    import ctypes as C

    ctx, geo = _ctx("f32")
    rng = np.random.default_rng(14)
    lib = ctx.lib
    rows = 50
    s = ctx.new_backend(4096)
    s.kv_reserve(first_row + rows + 200)  # pages well past the window
    table = s.block_table()
    pages = np.ascontiguousarray([gp for _, _, _, gp in table], np.int32)
    assert pages.size > (rows + 15) // 16 + 2
    snap = _snap(rng, geo, rows, rows, "f32")
    up = ctx.upload_kv_async(snap)
    i32p = C.POINTER(C.c_int)
    ctx.check(lib.zr_kv_scatter_transfer(ctx.h, up.h, pages.ctypes.data_as(i32p), int(pages.size), int(table[0][1]),
                                         first_row, rows))
    k = np.zeros((geo.num_layers, rows, geo.kv_cols), np.float32)
    v = np.zeros_like(k)
    f32p = C.POINTER(C.c_float)
    ctx.check(lib.zr_kv_gather(ctx.h, pages.ctypes.data_as(i32p), int(pages.size), int(table[0][1]), first_row, rows,
                               k.ctypes.data_as(f32p), v.ctypes.data_as(f32p)))
    np.testing.assert_array_equal(k, snap.keys)
    np.testing.assert_array_equal(v, snap.values)
    up.close()
    s.close()
    ctx.close()
