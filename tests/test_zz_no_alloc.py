"""zr_argmax_noalloc (the entry point that allocates nothing) against
zr_argmax, through the C-ABI: two calls in a row on the library's fixed
scratch, the second with a smaller input, then a call beyond the scratch's
limit (an error, not a launch)."""
import numpy as np
import pytest

from mesh_amd import DeviceBuffer, DeviceContext, ModelGeometry

pytestmark = pytest.mark.gpu


def _argmax(ctx, fn, d_x, rows, cols):
    d_o = DeviceBuffer(ctx, 4 * rows)
    ctx.check(fn(ctx.h, d_x.ptr, rows, cols, d_o.ptr))
    ctx.check(ctx.lib.zr_synchronize(ctx.h))
    out = d_o.download(np.uint32, rows)
    d_o.free()
    return out


def test_argmax_noalloc_matches_argmax_on_two_calls_then_rejects_oversize():
    geo = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=4, num_layers=1, vocab=64, ffn=256)
    ctx = DeviceContext(geo, kv_dtype="f32", max_tokens=16, max_seqs=4, max_pages_per_seq=4)
    rng = np.random.default_rng(0xA0)
    lib = ctx.lib
    # the larger call first: 256 rows x 128256 logits (8192 partials), with
    # ties at the same value in one row and an all -inf row
    big = rng.standard_normal((256, 128256), dtype=np.float32)
    big[3, [5, 70000, 127999]] = 99.0
    big[7] = -np.inf
    d_big = DeviceBuffer.from_numpy(ctx, big)
    got = _argmax(ctx, lib.zr_argmax_noalloc, d_big, 256, 128256)
    want = _argmax(ctx, lib.zr_argmax, d_big, 256, 128256)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got, np.argmax(big, 1))
    assert got[3] == 5 and got[7] == 0
    # a smaller call on the same scratch: its partials must not mix with the last call's
    small = rng.standard_normal((5, 1000), dtype=np.float32)
    d_small = DeviceBuffer.from_numpy(ctx, small)
    got = _argmax(ctx, lib.zr_argmax_noalloc, d_small, 5, 1000)
    np.testing.assert_array_equal(got, _argmax(ctx, lib.zr_argmax, d_small, 5, 1000))
    np.testing.assert_array_equal(got, np.argmax(small, 1))
    # 33 x 4096 columns x 1000 rows > 32768 partials: refused before any launch
    d_o = DeviceBuffer(ctx, 4 * 1000)
    rc = lib.zr_argmax_noalloc(ctx.h, d_big.ptr, 1000, 33 * 4096, d_o.ptr)
    assert rc == -1 and b"fixed scratch" in lib.zr_last_error(ctx.h)
    ctx.check(lib.zr_synchronize(ctx.h))
    ctx.close()
