"""Replay of a staged decode step as a HIP graph (zr_graph_capture_staged /
zr_graph_launch; the fused profile's ReplayPreferred capture strategy,
fast_path.rs:831-837).

The model is the bench's TinyLlama-1.1B-shape workload (22 layers, 32
sessions, contexts U[128, 2048]).  Running one staged step again writes the
same KV rows at the same slots, so every run of it -- eager or replayed --
must produce the same logits and tokens bit for bit.  Each replay is checked
against the eager result, with the program's own eager runs and
synchronisations between the replays."""
import ctypes as C

import numpy as np
import pytest

import bench

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny():
    b = bench.GpuDecodeBench("tinyllama_b32", 2)
    yield b
    b.close()


def _read(b, d_logits, d_out):
    ctx = b.ctx
    logits = np.empty((b.B, b.geo.vocab), np.float32)
    toks = np.empty(b.B, np.uint32)
    ctx.check(ctx.lib.zr_memcpy_d2h(ctx.h, logits.ctypes.data, d_logits, logits.nbytes))
    ctx.check(ctx.lib.zr_memcpy_d2h(ctx.h, toks.ctypes.data, d_out, toks.nbytes))
    return logits, toks


def _upload(b, ptr, arr):
    b.ctx.check(b.ctx.lib.zr_memcpy_h2d(b.ctx.h, ptr, arr.ctypes.data, arr.nbytes))


def _clobber(b, d_logits, d_out):
    _upload(b, d_logits, np.full(b.B * b.geo.vocab, np.nan, np.float32))
    _upload(b, d_out, np.full(b.B, 0xFFFFFFFF, np.uint32))


def test_replayed_step_equals_the_eager_step_every_time(tiny):
    b = tiny
    ctx, lib = b.ctx, b.ctx.lib
    d_logits, d_out, d_in2, d_out2 = b._dev(4 * b.B * b.geo.vocab), b._dev(4 * b.B), b._dev(4 * b.B), b._dev(4 * b.B)
    g = C.c_void_p()
    try:
        ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[0], b.tok[0], d_out, d_logits))
        ctx.check(lib.zr_synchronize(ctx.h))
        want_logits, want_toks = _read(b, d_logits, d_out)
        assert np.isfinite(want_logits).all()
        np.testing.assert_array_equal(want_toks, np.argmax(want_logits, 1))
        _upload(b, d_in2, want_toks)
        ctx.check(lib.zr_graph_capture_staged(ctx.h, b.staged[0], b.tok[0], d_out, d_logits, C.byref(g)))
        for rep in range(4):
            _clobber(b, d_logits, d_out)
            ctx.check(lib.zr_graph_launch(ctx.h, g))
            ctx.check(lib.zr_synchronize(ctx.h))
            got_logits, got_toks = _read(b, d_logits, d_out)
            np.testing.assert_array_equal(got_logits, want_logits, err_msg=f"replay {rep}")
            np.testing.assert_array_equal(got_toks, want_toks, err_msg=f"replay {rep}")
            # the program's own eager work between replays: the next staged step
            # (it appends the following rows, which the first step does not see)
            ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[1], d_in2, d_out2, None))
            ctx.check(lib.zr_synchronize(ctx.h))
        # two replays back to back
        _clobber(b, d_logits, d_out)
        ctx.check(lib.zr_graph_launch(ctx.h, g))
        ctx.check(lib.zr_graph_launch(ctx.h, g))
        ctx.check(lib.zr_synchronize(ctx.h))
        got_logits, got_toks = _read(b, d_logits, d_out)
        np.testing.assert_array_equal(got_logits, want_logits)
        np.testing.assert_array_equal(got_toks, want_toks)
        # and the eager step once more after them
        _clobber(b, d_logits, d_out)
        ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[0], b.tok[0], d_out, d_logits))
        ctx.check(lib.zr_synchronize(ctx.h))
        got_logits, got_toks = _read(b, d_logits, d_out)
        np.testing.assert_array_equal(got_logits, want_logits)
    finally:
        if g.value:
            lib.zr_graph_destroy(g)
        for p in (d_logits, d_out, d_in2, d_out2):
            lib.zr_device_free(ctx.h, p)


def test_replayed_step_reports_a_device_fed_id_out_of_range(tiny):
    b = tiny
    ctx, lib = b.ctx, b.ctx.lib
    ids = np.arange(b.B, dtype=np.uint32)
    ids[5] = b.geo.vocab + 7
    d_ids, d_out = b._dev(4 * b.B), b._dev(4 * b.B)
    g = C.c_void_p()
    try:
        _upload(b, d_ids, ids)
        ctx.check(lib.zr_graph_capture_staged(ctx.h, b.staged[0], d_ids, d_out, None, C.byref(g)))
        assert lib.zr_synchronize(ctx.h) == 0  # capturing runs nothing
        ctx.check(lib.zr_graph_launch(ctx.h, g))
        rc = lib.zr_synchronize(ctx.h)
        assert rc == -1, rc
        assert f"Token {b.geo.vocab + 7} out of vocabulary bounds {b.geo.vocab}".encode() in lib.zr_last_error(ctx.h)
        assert lib.zr_synchronize(ctx.h) == 0  # reported once
    finally:
        if g.value:
            lib.zr_graph_destroy(g)
        lib.zr_device_free(ctx.h, d_ids)
        lib.zr_device_free(ctx.h, d_out)


def test_capture_is_refused_while_timing_is_on(tiny):
    b = tiny
    ctx, lib = b.ctx, b.ctx.lib
    g = C.c_void_p()
    ctx.check(lib.zr_timing_begin(ctx.h, 1))
    rc = lib.zr_graph_capture_staged(ctx.h, b.staged[0], b.tok[0], b.tok[1], None, C.byref(g))
    ms, n = (C.c_double * 5)(), (C.c_int * 5)()
    ctx.check(lib.zr_timing_end(ctx.h, ms, n))
    assert rc == -1 and not g.value
    assert b"timing" in lib.zr_last_error(ctx.h)


def test_a_graph_is_refused_once_a_buffer_it_reads_was_reallocated(tiny):
    """The step reads the context's argmax workspace; zr_argmax over more rows
    than the context was sized for reallocates it.  A graph captured before
    is refused (it would replay with the freed address); one captured again
    runs and equals the eager step."""
    b = tiny
    ctx, lib = b.ctx, b.ctx.lib
    rows = 2 * b.B
    d_logits, d_out = b._dev(4 * b.B * b.geo.vocab), b._dev(4 * b.B)
    d_x, d_am = b._dev(4 * rows * b.geo.vocab), b._dev(4 * rows)
    g = C.c_void_p()
    try:
        _upload(b, d_x, np.zeros(rows * b.geo.vocab, np.float32))
        ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[0], b.tok[0], d_out, d_logits))
        ctx.check(lib.zr_synchronize(ctx.h))
        want_logits, want_toks = _read(b, d_logits, d_out)
        ctx.check(lib.zr_graph_capture_staged(ctx.h, b.staged[0], b.tok[0], d_out, d_logits, C.byref(g)))
        ctx.check(lib.zr_argmax(ctx.h, d_x, rows, b.geo.vocab, d_am))  # regrows the argmax workspace
        rc = lib.zr_graph_launch(ctx.h, g)
        assert rc == -1, rc
        assert b"capture it again" in lib.zr_last_error(ctx.h)
        lib.zr_graph_destroy(g)
        g = C.c_void_p()
        ctx.check(lib.zr_graph_capture_staged(ctx.h, b.staged[0], b.tok[0], d_out, d_logits, C.byref(g)))
        _clobber(b, d_logits, d_out)
        ctx.check(lib.zr_graph_launch(ctx.h, g))
        ctx.check(lib.zr_synchronize(ctx.h))
        got_logits, got_toks = _read(b, d_logits, d_out)
        np.testing.assert_array_equal(got_logits, want_logits)
        np.testing.assert_array_equal(got_toks, want_toks)
    finally:
        if g.value:
            lib.zr_graph_destroy(g)
        for p in (d_logits, d_out, d_x, d_am):
            lib.zr_device_free(ctx.h, p)


def test_a_graph_is_refused_once_its_staged_microbatch_was_destroyed(tiny):
    """A graph replays its staged blob: after zr_staged_destroy the launch is
    refused instead of replaying freed device addresses."""
    from tests.gpu_util import stage_mixed

    b = tiny
    ctx, lib = b.ctx, b.ctx.lib
    st = stage_mixed(ctx, b.backends, [1] * b.B)
    g = C.c_void_p()
    try:
        ctx.check(lib.zr_graph_capture_staged(ctx.h, st, b.tok[0], b.tok[1], None, C.byref(g)))
        lib.zr_staged_destroy(st)
        st = None
        rc = lib.zr_graph_launch(ctx.h, g)
        assert rc == -1, rc
        assert b"staged microbatch was destroyed" in lib.zr_last_error(ctx.h)
        assert lib.zr_synchronize(ctx.h) == 0  # nothing was enqueued
    finally:
        if g.value:
            lib.zr_graph_destroy(g)
        if st is not None:
            lib.zr_staged_destroy(st)
