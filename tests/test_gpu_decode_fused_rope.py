"""The decode step with RoPE + KV append inside the attention launch (the
forward pass's path for microbatches of one-row sequences) against the same
step with the separate RopeKvWrite kernel (ZR_ATTN_FUSE_ROPE=1 / 0 at staging
force either path).

Two identically built TinyLlama-1.1B-shape models (22 layers, 32 sessions,
contexts U[128, 2048], seeded weights and KV) run two decode steps each --
the second attends over the rows the first appended -- and must agree bit for
bit: logits, greedy tokens and the appended K / V rows of every layer."""
import ctypes as C

import numpy as np
import pytest

import bench

pytestmark = pytest.mark.gpu


def _two_steps(b):
    ctx, lib = b.ctx, b.ctx.lib
    d_logits = b._dev(4 * b.B * b.geo.vocab)
    out = []
    try:
        for i in range(2):
            ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[i], b.tok[i % 2], b.tok[(i + 1) % 2], d_logits))
            ctx.check(lib.zr_synchronize(ctx.h))
            logits = np.empty((b.B, b.geo.vocab), np.float32)
            toks = np.empty(b.B, np.uint32)
            ctx.check(lib.zr_memcpy_d2h(ctx.h, logits.ctypes.data, d_logits, logits.nbytes))
            ctx.check(lib.zr_memcpy_d2h(ctx.h, toks.ctypes.data, b.tok[(i + 1) % 2], toks.nbytes))
            out.append((logits, toks))
    finally:
        lib.zr_device_free(ctx.h, d_logits)
    return out


def test_decode_step_with_rope_inside_attention_equals_separate_rope_kernel(monkeypatch):
    monkeypatch.setenv("ZR_ATTN_FUSE_ROPE", "1")  # short splits would keep the RoPE kernel
    fused = bench.GpuDecodeBench("tinyllama_b32", 2)
    try:
        got = _two_steps(fused)
        monkeypatch.setenv("ZR_ATTN_FUSE_ROPE", "0")
        apart = bench.GpuDecodeBench("tinyllama_b32", 2)
        try:
            want = _two_steps(apart)
            for step, ((gl, gt), (wl, wt)) in enumerate(zip(got, want)):
                assert np.isfinite(wl).all()
                np.testing.assert_array_equal(gl, wl, err_msg=f"logits of step {step}")
                np.testing.assert_array_equal(gt, wt, err_msg=f"tokens of step {step}")
            # the two appended rows of the shortest sessions, every layer
            for s in np.argsort(fused.ctxlens)[:2]:
                a, b = fused.backends[s].export_kv_cache(), apart.backends[s].export_kv_cache()
                assert a.cached_tokens == b.cached_tokens == int(fused.ctxlens[s]) + 2
                np.testing.assert_array_equal(a.keys[:, -2:], b.keys[:, -2:])
                np.testing.assert_array_equal(a.values[:, -2:], b.values[:, -2:])
        finally:
            apart.close()
    finally:
        fused.close()
