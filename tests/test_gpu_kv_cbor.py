"""KV snapshot wire bytes encoded on the device (zrh_export_kv_cbor) and read
back (zrh_import_kv_cbor), against the oracle's encoder (oracle/kv_cbor.c).

Bars: the device document equals the oracle's byte for byte for the rows the
f32 export (zrh_export_kv) returns; import of a document restores the rows,
positions and page tables bit-exactly; malformed or mismatched documents fail
with ZR_E_INVALID as KVCacheSnapshot::validate_with_cache (kv_cache.rs:121-141)
and KVCache::from_bytes (889-895) would.
"""
import numpy as np
import pytest

import oracle as O
from mesh_amd import DeviceContext, KVCacheBlob, KVCacheSnapshot, KVCacheWireSnapshot, KVSequenceState, ModelGeometry
from mesh_amd._lib import ZrError

pytestmark = pytest.mark.gpu

SPECIALS = np.array([0.0, -0.0, 1.5, 65504.0, 65520.0, 1e-7, 2.0 ** -24, 2.0 ** -25, 3e38, np.inf, -np.inf,
                     1.0 + 2.0 ** -11, 1e-40, -(2.0 ** -14), 6.1e-5, -65504.0], np.float32)


def _ctx(kv_dtype, layers=2, kv_heads=4, head_dim=64, pages=512):
    geo = ModelGeometry(hidden=head_dim * 8, num_heads=8, num_kv_heads=kv_heads, num_layers=layers, vocab=64,
                        ffn=64)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=64, max_seqs=16, max_pages_per_seq=600)
    ctx.create_kv_pool(pages)
    return ctx, geo


def _fill(ctx, geo, rows, next_position, seed, specials=True, max_seq=8192):
    rng = np.random.default_rng(seed)
    shape = (geo.num_layers, rows, geo.num_kv_heads * (geo.hidden // geo.num_heads))
    k = rng.standard_normal(shape).astype(np.float32)
    v = (rng.standard_normal(shape) * 3).astype(np.float32)
    if specials:
        k[0, 0, :len(SPECIALS)] = SPECIALS
        v[-1, -1, -len(SPECIALS):] = SPECIALS[::-1]
    b = ctx.new_backend(max_seq)
    b.import_kv_cache(KVCacheSnapshot(next_position, rows, k, v))
    return b


def _want(ctx, geo, b, max_cached_tokens=None, max_seq=8192):
    snap = b.export_kv_cache(max_cached_tokens)
    return O.kv_cbor_encode(snap.keys, snap.values, snap.first_cached_position(), geo.num_layers, geo.num_kv_heads,
                            geo.hidden // geo.num_heads, max_seq), snap


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("rows,window", [(1, None), (37, None), (300, None), (300, 21), (1000, 1)])
def test_device_document_equals_oracle_bytes(kv_dtype, rows, window):
    ctx, geo = _ctx(kv_dtype)
    b = _fill(ctx, geo, rows, rows + 5, seed=rows)
    want, ref = _want(ctx, geo, b, window)
    got = b.export_kv_snapshot(window)
    assert got.sequence == KVSequenceState(ref.next_position, ref.cached_tokens)
    assert got.blob.encoding == "FullSnapshotCbor"
    assert bytes(got.blob.data) == want
    ctx.close()


def test_size_query_and_short_capacity():
    ctx, geo = _ctx("f32")
    b = _fill(ctx, geo, 40, 40, seed=1)
    want, _ = _want(ctx, geo, b)
    size = O.C.c_size_t()
    ctx.check(ctx.lib.zrh_export_kv_cbor(b.h, -1, None, 0, O.C.byref(size), None, None))
    assert size.value == len(want)
    short = np.zeros(len(want) - 1, np.uint8)
    with pytest.raises(ZrError) as e:
        ctx.check(ctx.lib.zrh_export_kv_cbor(b.h, -1, short.ctypes.data, short.size, O.C.byref(size), None, None))
    assert e.value.status == -1 and size.value == len(want)
    ctx.close()


def test_empty_cache_has_no_snapshot():
    ctx, geo = _ctx("bf16")
    b = ctx.new_backend(4096)
    assert b.export_kv_snapshot() is None
    ctx.close()


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_round_trip_restores_rows_positions_and_pages(kv_dtype):
    ctx, geo = _ctx(kv_dtype, layers=3)
    b = _fill(ctx, geo, 211, 260, seed=9)
    snap = b.export_kv_snapshot(max_cached_tokens=150, pinned=True)
    ref = b.export_kv_cache(150)
    b2 = ctx.new_backend(8192)
    b2.import_kv_snapshot(snap)
    back = b2.export_kv_cache()
    assert (back.next_position, back.cached_tokens) == (260, 150)
    assert b2.sequence_position() == 260
    np.testing.assert_array_equal(back.keys.view(np.uint32), ref.keys.view(np.uint32))
    np.testing.assert_array_equal(back.values.view(np.uint32), ref.values.view(np.uint32))
    # the imported session re-encodes to the same document
    assert bytes(b2.export_kv_snapshot().blob.data) == bytes(snap.blob.data)
    # oracle-encoded documents import too (the CPU provider's bytes)
    doc = O.kv_cbor_encode(ref.keys, ref.values, 110, geo.num_layers, geo.num_kv_heads, geo.hidden // geo.num_heads,
                           4096)
    b3 = ctx.new_backend(8192)
    b3.import_kv_snapshot(KVCacheWireSnapshot(KVSequenceState(260, 150), KVCacheBlob("FullSnapshotCbor",
                                                                                      memoryview(doc))))
    np.testing.assert_array_equal(b3.export_kv_cache().keys.view(np.uint32), ref.keys.view(np.uint32))
    ctx.close()


def test_malformed_and_mismatched_documents_are_rejected():
    ctx, geo = _ctx("f32")
    b = _fill(ctx, geo, 30, 30, seed=4)
    snap = b.export_kv_snapshot()
    data = bytes(snap.blob.data)
    b2 = ctx.new_backend(8192)

    def imp(blob, nxt=30, cached=30):
        b2.import_kv_snapshot(KVCacheWireSnapshot(KVSequenceState(nxt, cached),
                                                  KVCacheBlob("FullSnapshotCbor", memoryview(blob))))

    cases = [(data[:-1], 30, 30, "truncated"), (data + b"\x00", 30, 30, "trailing"),
             (data, 30, 29, "cached token mismatch"), (data, 31, 30, "base position mismatch"),
             (data, 30, 31, "exceeds next_position"), (b"\xa0", 30, 30, "misses layers")]
    kw = O.kv_cbor_encode(np.zeros((3, 30, 256), np.float32), np.zeros((3, 30, 256), np.float32), 0, 3, 4, 64, 8192)
    cases.append((kw, 30, 30, "layers"))
    kc = O.kv_cbor_encode(np.zeros((2, 30, 128), np.float32), np.zeros((2, 30, 128), np.float32), 0, 2, 4, 64, 8192)
    cases.append((kc, 30, 30, "width"))
    for blob, nxt, cached, what in cases:
        with pytest.raises(ZrError) as e:
            imp(blob, nxt, cached)
        assert e.value.status == -1, what
        assert what in str(e.value), (what, str(e.value))
        assert b2.cache_seq_len() == 0  # a failed import leaves the session as it was
    imp(data)
    assert b2.cache_seq_len() == 30
    ctx.close()


def test_llama3_shape_2048_token_window_document():
    # 32 layers x 2048 rows x 1024 (8 kv heads x 128) -- one session's eviction
    # snapshot at the 256-session decode shape, bf16 pool
    geo = ModelGeometry(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=32, vocab=64, ffn=64)
    ctx = DeviceContext(geo, kv_dtype="bf16", max_tokens=64, max_seqs=8, max_pages_per_seq=600)
    ctx.create_kv_pool(300)
    rng = np.random.default_rng(0xC5)
    rows = 3000
    k = rng.standard_normal((32, rows, 1024), np.float32)
    v = rng.standard_normal((32, rows, 1024), np.float32)
    b = ctx.new_backend(8192)
    b.import_kv_cache(KVCacheSnapshot(rows, rows, k, v))
    del k, v
    snap = b.export_kv_snapshot(max_cached_tokens=2048, pinned=True)
    ref = b.export_kv_cache(2048)
    want = O.kv_cbor_encode(ref.keys, ref.values, rows - 2048, 32, 8, 128, 8192)
    got = np.frombuffer(snap.blob.data, np.uint8)
    assert got.size == len(want)
    assert np.array_equal(got, np.frombuffer(want, np.uint8))
    ctx.close()


def test_workspaces_survive_kv_staging_growth():
    """The KV gather staging grows on demand; growing it must leave the CBOR
    encoder's and the sampler's workspaces in place.  On one context: sample
    a batch and encode a document, grow the staging with a larger gather,
    then sample and encode again: the same tokens and the same bytes, equal
    to the oracle's document."""
    from mesh_amd.provider import sample_device

    ctx, geo = _ctx("bf16", layers=2, kv_heads=4, head_dim=64, pages=512)
    small = _fill(ctx, geo, 40, 45, seed=3, specials=False)
    big = _fill(ctx, geo, 1500, 1500, seed=4, specials=False)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    temps = np.array([0.7, 1.0, 0.0, 1.3, 0.5, 0.9], np.float32)
    tops = np.array([0.9, 1.0, 1.0, 0.5, 0.95, 0.8], np.float32)
    seeds = rng.integers(0, 2 ** 63, 6, dtype=np.uint64)
    want, _ = _want(ctx, geo, small)
    t1 = sample_device(ctx, x, temps, tops, seeds)
    d1 = bytes(small.export_kv_snapshot().blob.data)
    big.export_kv_cache()  # 1500 rows x 2 layers: a larger staging than the first export's
    t2 = sample_device(ctx, x, temps, tops, seeds)
    d2 = bytes(small.export_kv_snapshot().blob.data)
    assert t1 == t2
    assert d1 == want and d2 == want
    ctx.close()
