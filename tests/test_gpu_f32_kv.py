"""Parity at the reference's own KV precision, at full width.

The reference keeps every K / V page in f32 (forward_pass.rs:255-262,
DeviceKVPage::new with DType::F32).  These tests run the device with an f32
page pool against the unmodified oracle (f32 KV, no rounding), unforced: the
oracle computes and stores its own appended rows, as the CPU provider does.

* C2: TinyLlama-1.1B shape, 22 layers, 32 sessions, contexts U[128, 2048]
  (seed 0xC2), two greedy decode steps.
* C4: tensor-parallel shard 0 of 2 of Llama-3-8B, 32 layers, 64 sessions,
  lognormal contexts: every layer's pre-all-reduce partials, the logits and
  the KV pages written.
* The benchmarked step: the 256-session Llama-3-8B decode step exactly as
  bench.py stages it, with an f32 pool (~105 GB), 16 sampled sessions.
* The 256-session attention launch of that step with an f32 pool:
  test_gpu_kernels.test_c5_shape_attention_256_sessions_matches_oracle
  (parametrised over the KV dtype).

Prior context rows are f32 values that bf16 cannot hold (a bf16 N(0, 1) pool
value plus 2^-9 of another), so the kernels' hi + lo split of f32 K / V is
exercised.  Bars: logits within 1e-2 absolute, greedy ids equal where the
oracle's top-2 margin exceeds 1e-3, partials within 1e-2, imported rows bit
exact, appended rows within 1e-4 of the row's largest element (a wrong row is
off by O(1)).
"""
import time

import numpy as np
import pytest

import bench
import oracle as O
from mesh_amd import BackendMicrobatchExecutor, DecodeMicrobatchRequest, KVCacheSnapshot
from tests.test_gpu_model import _oracle_import, check_logits, make
from tests.testmodels import NormalPool, geometry, random_weights

pytestmark = pytest.mark.gpu

APPEND_RTOL = 1e-4


def _progress(msg):
    print(f"[f32-kv] {time.strftime('%H:%M:%S')} {msg}", flush=True)


def _f32_rows(pool, shape):
    """N(0, 1)-like f32 values with bits below bf16's mantissa."""
    a = pool.take(shape)
    a += pool.take(shape) * np.float32(2.0 ** -9)
    return a


def _sessions_f32(ctx, pool, layers, kv_cols, ctxlens, max_seq):
    dev, ref = [], []
    for L in ctxlens:
        snap = KVCacheSnapshot(int(L), int(L), _f32_rows(pool, (layers, int(L), kv_cols)),
                               _f32_rows(pool, (layers, int(L), kv_cols)))
        b = ctx.new_backend(max_seq)
        b.import_kv_cache(snap)
        s = O.Session(layers, kv_cols, 16, max_seq, kv_round_bf16=False)
        _oracle_import(s, snap)
        dev.append(b)
        ref.append(s)
    return dev, ref


def _check_appended(snap, sess, layers, label, new=1):
    """Rows before the last `new` steps bit exact; each appended row within
    APPEND_RTOL of the row's largest element."""
    for layer in layers:
        k, v = sess.gather(layer)
        assert snap.keys.shape[1] == k.shape[0], label
        np.testing.assert_array_equal(snap.keys[layer, :-new], k[:-new])
        np.testing.assert_array_equal(snap.values[layer, :-new], v[:-new])
        for r in range(1, new + 1):
            for got, want in ((snap.keys[layer, -r], k[-r]), (snap.values[layer, -r], v[-r])):
                err = float(np.max(np.abs(got - want)))
                assert err <= APPEND_RTOL * float(np.abs(want).max()), (label, layer, r, err)


def test_c2_tinyllama_22_layers_f32_kv_unforced():
    cfg = dict(hidden=2048, num_heads=32, num_kv_heads=4, num_layers=22, vocab=32000, ffn=5632, rms_norm_eps=1e-5,
               rope_base=10000.0)
    geo = geometry(cfg)
    weights = random_weights(cfg, geo, seed=0xC2, std=0.02, pooled=True)
    rng = np.random.default_rng(0xC2)
    pool = NormalPool(rng)
    ctxlens = rng.integers(128, 2049, 32)
    pages = int(sum((L + 2 + 15) // 16 + 1 for L in ctxlens))
    ctx, om = make(cfg, geo, weights, "f32", True, max_tokens=32, max_seqs=32, pages=pages, pps=140)
    dev, ref = _sessions_f32(ctx, pool, 22, geo["kv_cols"], ctxlens, 4096)
    toks = rng.integers(0, cfg["vocab"], 32).tolist()
    for step in range(2):
        reqs = [DecodeMicrobatchRequest(str(i), t, b) for i, (t, b) in enumerate(zip(toks, dev))]
        outs = BackendMicrobatchExecutor.decode_step_batch(reqs, want_logits=True)
        got = np.stack([o.logits for o in outs])
        want = om.decode(ref, toks)
        err = check_logits(got, want, f"C2 f32 KV step {step}")
        print(f"C2 f32 KV step {step}: max |logit - oracle| = {err:.3g} (unforced)", flush=True)
        toks = np.argmax(want, 1).tolist()
    for i in (0, 13, 31):
        _check_appended(dev[i].export_kv_cache(), ref[i], (0, 21), f"C2 session {i}", new=2)
    ctx.close()


def test_c4_tp_shard_32_layers_f32_kv_partials_and_pages():
    cfg = dict(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=32, vocab=128256, ffn=14336, rms_norm_eps=1e-5,
               rope_base=500000.0)
    geo = geometry(cfg, shard_start=0, shard_end=2048, ffn_cols=O.partition_columns(14336, 0, 2))
    weights = random_weights(cfg, geo, seed=0xC4, std=0.02, pooled=True)
    rng = np.random.default_rng(0xC4)
    pool = NormalPool(rng)
    ctxlens = np.clip(np.round(rng.lognormal(np.log(1024), 1.0, 64)), 64, 8192).astype(int)
    pages = int(sum((L + 1 + 15) // 16 + 1 for L in ctxlens))
    ctx, om = make(cfg, geo, weights, "f32", True, max_tokens=64, max_seqs=64, pages=pages, pps=8192 // 16 + 2)
    kv = geo["kv_cols"]
    dev, ref = _sessions_f32(ctx, pool, 32, kv, ctxlens, 8192)
    toks = rng.integers(0, cfg["vocab"], 64).tolist()
    parts = np.zeros((32, 2, 64, 4096), np.float32)
    reqs = [DecodeMicrobatchRequest(str(i), t, b) for i, (t, b) in enumerate(zip(toks, dev))]
    outs = BackendMicrobatchExecutor.decode_step_batch(reqs, want_logits=True, partials=parts)
    want, want_parts = om.decode(ref, toks, want_partials=True)
    perr = float(np.max(np.abs(parts - want_parts)))
    assert perr <= 1e-2, perr
    got = np.stack([o.logits for o in outs])
    err = check_logits(got, want, "C4 shard f32 KV logits")
    print(f"C4 f32 KV: max |partial - oracle| = {perr:.3g}, max |logit - oracle| = {err:.3g} (unforced)", flush=True)
    for i in (0, 17, 63):
        _check_appended(dev[i].export_kv_cache(), ref[i], (0, 31), f"C4 session {i}")
    ctx.close()


WORKLOAD = "llama3_8b_b256"


def test_benchmarked_256_session_step_f32_kv_unforced():
    host = {}
    ctx, g = bench.device_model(WORKLOAD, True, host_weights=host, kv_dtype="f32")
    try:
        geo = bench.WORKLOADS[WORKLOAD]["geo"]
        cfg = dict(hidden=g.hidden, num_heads=g.num_heads, num_kv_heads=g.num_kv_heads, num_layers=g.num_layers,
                   vocab=g.vocab, ffn_cols=g.ffn_cols, rms_norm_eps=1e-5, rope_base=geo["rope_base"])
        om = O.Model(cfg, host)
        del host
        _progress("model resident; staging the 256-session step with an f32 pool")
        b = bench.GpuDecodeBench(WORKLOAD, 1, model=(ctx, g))
        try:
            lib, B, V = ctx.lib, b.B, g.vocab
            tokens = b.tokens(0)
            d_logits = b._dev(4 * B * V)
            ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[0], b.tok[0], b.tok[1], d_logits))
            ctx.check(lib.zr_synchronize(ctx.h))
            logits = np.empty((B, V), np.float32)
            ctx.check(lib.zr_memcpy_d2h(ctx.h, logits.ctypes.data, d_logits, logits.nbytes))
            lib.zr_device_free(ctx.h, d_logits)
            assert np.isfinite(logits).all()
            np.testing.assert_array_equal(b.tokens(1), np.argmax(logits, 1))
            _progress("step ran")
            ctxlens = b.ctxlens
            sample = sorted({int(np.argmax(ctxlens)), int(np.argmin(ctxlens))} |
                            {int(x) for x in np.random.default_rng(16).choice(B, 14, replace=False)})
            while len(sample) < 16:
                sample = sorted(set(sample) | {int(np.random.default_rng(len(sample)).integers(B))})
            snaps = [b.backends[i].export_kv_cache() for i in sample]
            sess = []
            for i, snap in zip(sample, snaps):
                assert snap.next_position == int(ctxlens[i]) + 1
                rows = snap.cached_tokens - 1  # the oracle appends the step's row itself
                s = O.Session(g.num_layers, g.kv_cols, 16, b.max_seq, kv_round_bf16=False)
                s.import_snapshot({"keys": np.ascontiguousarray(snap.keys[:, :rows]),
                                   "values": np.ascontiguousarray(snap.values[:, :rows]),
                                   "base_position": snap.first_cached_position(),
                                   "next_position": snap.next_position - 1, "cached_tokens": rows})
                sess.append(s)
            want = om.decode(sess, tokens[sample])
            err = check_logits(logits[sample], want, "256-session step, f32 KV")
            print(f"256-session step, f32 KV: max |logit - oracle| = {err:.3g} over {len(sample)} sessions "
                  f"(unforced; contexts {sorted(int(ctxlens[i]) for i in sample)})", flush=True)
            for j in (0, len(sample) - 1):
                _check_appended(snaps[j], sess[j], (0, 15, 31), f"session {sample[j]}")
        finally:
            b.close()
    finally:
        ctx.close()
