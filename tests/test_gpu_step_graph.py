"""The pipelined serving loop (zrh_decode_pipeline over zr_step_graph): one
graph per bucket, replayed every step with that step's metadata.

Every step of the pipeline must equal the synchronous batched step
(zrh_decode_step_batch, BackendMicrobatchExecutor::decode_step_batch,
backend.rs:110-151) on a copy of the same sessions bit for bit: the greedy ids
of every step, the positions, and every K / V row the steps appended.  The
sessions cross page boundaries and slide their windows (first-page offsets
change) during the run; one test forces the attention work list past the
bucket's capacity, so the pipeline sets up a new bucket mid-run.
"""
import ctypes as C

import numpy as np
import pytest

import bench
from mesh_amd import BackendMicrobatchExecutor, DecodeMicrobatchRequest, DecodePipeline, KVCacheSnapshot
from tests.test_gpu_model import SMALL, make
from tests.testmodels import geometry, random_weights

pytestmark = pytest.mark.gpu


def _twin_sessions(ctx, rng, lens, max_seqs, kv_cols, layers):
    """Two sets of sessions holding the same imported windows."""
    a, b = [], []
    for L, m in zip(lens, max_seqs):
        snap = KVCacheSnapshot(int(L), int(L), rng.standard_normal((layers, int(L), kv_cols), dtype=np.float32),
                               rng.standard_normal((layers, int(L), kv_cols), dtype=np.float32))
        for group in (a, b):
            s = ctx.new_backend(int(m))
            s.import_kv_cache(snap)
            group.append(s)
    return a, b


def _sync_steps(sessions, first, steps, want_logits=False):
    """Synchronous batched steps.  With want_logits every step runs eagerly
    (kernel by kernel); greedy-only steps replay zr_forward's step graph from
    the third call of the same sequence count."""
    toks, out = list(map(int, first)), []
    for _ in range(steps):
        reqs = [DecodeMicrobatchRequest(str(i), t, s) for i, (t, s) in enumerate(zip(toks, sessions))]
        toks = [o.sampled_token for o in BackendMicrobatchExecutor.decode_step_batch(reqs, want_logits=want_logits)]
        out.append(np.asarray(toks, np.uint32))
    return out


def _pipeline_steps(sessions, first, steps):
    pipe = DecodePipeline(sessions, first)
    try:
        out = []
        for _ in range(steps):
            prev = pipe.step()
            if prev is not None:
                out.append(prev)
        out.append(pipe.finish())
        return out, pipe.info()
    finally:
        pipe.close()


def _same_sessions(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        assert x.sequence_position() == y.sequence_position(), i
        assert x.cache_seq_len() == y.cache_seq_len(), i
        sx, sy = x.export_kv_cache(), y.export_kv_cache()
        assert sx.next_position == sy.next_position
        np.testing.assert_array_equal(sx.keys, sy.keys, err_msg=f"session {i} keys")
        np.testing.assert_array_equal(sx.values, sy.values, err_msg=f"session {i} values")


@pytest.mark.parametrize("kv_dtype", ["bf16", "f32"])
def test_pipeline_equals_the_synchronous_step_bit_for_bit(kv_dtype):
    cfg = SMALL
    geo = geometry(cfg)
    weights = random_weights(cfg, geo, seed=31, std=0.05)
    ctx, _ = make(cfg, geo, weights, kv_dtype, True, max_tokens=16, max_seqs=16, pages=1024, pps=64)
    rng = np.random.default_rng(0x5EED)
    # contexts across page boundaries; two sessions with short windows slide
    # during the run (their first page offset moves)
    lens = [1, 15, 16, 17, 40, 100, 250, 60]
    max_seqs = [4096, 4096, 4096, 4096, 48, 4096, 4096, 70]
    a, b = _twin_sessions(ctx, rng, lens, max_seqs, geo["kv_cols"], cfg["num_layers"])
    first = rng.integers(0, cfg["vocab"], len(lens))
    steps = 40
    want = _sync_steps(a, first, steps, want_logits=True)
    got, info = _pipeline_steps(b, first, steps)
    assert len(got) == steps
    for k in range(steps):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"step {k}")
    _same_sessions(a, b)
    assert info["steps"] == steps and info["launches"] == steps
    assert info["buckets"] == 1 and info["captures"] == 2  # one graph per (ids in, ids out) pair
    ctx.close()


def test_pipeline_takes_a_new_bucket_when_the_work_list_outgrows_it(monkeypatch):
    cfg = SMALL
    geo = geometry(cfg)
    weights = random_weights(cfg, geo, seed=32, std=0.05)
    ctx, _ = make(cfg, geo, weights, "bf16", True, max_tokens=16, max_seqs=16, pages=2048, pps=128)
    rng = np.random.default_rng(0xB0C)
    lens = [300, 700, 1100, 1500]
    a, b = _twin_sessions(ctx, rng, lens, [4096] * 4, geo["kv_cols"], cfg["num_layers"])
    first = rng.integers(0, cfg["vocab"], len(lens))
    # 64-page splits for 3 steps, then 1-page splits: ~230 attention items where
    # the bucket has room for ~70
    want, got = [], []
    monkeypatch.setenv("ZR_ATTN_PAGES_PER_SPLIT", "64")
    want += _sync_steps(a, first, 3, want_logits=True)
    pipe = DecodePipeline(b, first)
    try:
        for _ in range(3):
            prev = pipe.step()
            if prev is not None:
                got.append(prev)
        monkeypatch.setenv("ZR_ATTN_PAGES_PER_SPLIT", "1")
        want += _sync_steps(a, want[-1], 3, want_logits=True)
        for _ in range(3):
            got.append(pipe.step())
        got.append(pipe.finish())
        info = pipe.info()
    finally:
        pipe.close()
    for k in range(6):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"step {k}")
    _same_sessions(a, b)
    assert info["buckets"] == 2, info
    assert info["items_capacity"] >= 230, info
    ctx.close()


def test_pipeline_rejects_ids_outside_the_vocabulary_and_prefill_less_sessions():
    cfg = SMALL
    geo = geometry(cfg)
    weights = random_weights(cfg, geo, seed=33, std=0.05)
    ctx, _ = make(cfg, geo, weights, "bf16", True, max_tokens=16, max_seqs=16, pages=64, pps=16)
    rng = np.random.default_rng(3)
    a, _b = _twin_sessions(ctx, rng, [5, 9], [4096, 4096], geo["kv_cols"], cfg["num_layers"])
    from mesh_amd._lib import ZrError
    with pytest.raises(ZrError, match=f"Token {cfg['vocab']} out of vocabulary bounds {cfg['vocab']}"):
        DecodePipeline(a, [1, cfg["vocab"]])
    fresh = ctx.new_backend(4096)
    pipe = DecodePipeline([a[0], fresh], [1, 2])
    with pytest.raises(ZrError, match="Decode microbatch requested before prompt prefill"):
        pipe.step()
    pipe.close()
    assert fresh.sequence_position() == 0 and a[0].sequence_position() == 5  # nothing moved
    ctx.close()


def test_pipeline_equals_the_synchronous_step_at_the_tinyllama_b32_workload():
    """The bench's 32-session, 22-layer TinyLlama-shape step: 6 pipelined steps
    against the synchronous batched step on a copy of the sessions."""
    bb = bench.GpuDecodeBench("tinyllama_b32", 0, host_steps=1200)  # pool room for a copy of every session
    try:
        ctx = bb.ctx
        twins = []
        for s in bb.backends:
            t = ctx.new_backend(bb.max_seq)
            t.import_kv_cache(s.export_kv_cache())
            twins.append(t)
        first = np.random.default_rng(9).integers(0, bb.geo.vocab, bb.B)
        want = _sync_steps(bb.backends, first, 6, want_logits=True)
        got, info = _pipeline_steps(twins, first, 6)
        for k in range(6):
            np.testing.assert_array_equal(got[k], want[k], err_msg=f"step {k}")
        for i in (0, 7, 31):
            x, y = bb.backends[i].export_kv_cache(2), twins[i].export_kv_cache(2)
            np.testing.assert_array_equal(x.keys, y.keys)
            np.testing.assert_array_equal(x.values, y.values)
        assert info["buckets"] == 1
        for t in twins:
            t.close()
    finally:
        bb.close()


@pytest.mark.parametrize("kv_dtype", ["bf16", "f32"])
def test_synchronous_greedy_steps_replay_and_equal_the_eager_steps(kv_dtype):
    """zr_forward replays greedy-only decode steps from the context's step
    graph once a sequence count has run three calls in a row.  On twin
    sessions, greedy-only steps (two eager calls, then replays; a new count
    starts over and sets up a new bucket) equal steps that also fetch the
    logits (always eager) bit for bit: the ids of every step, the positions
    and every appended K / V row."""
    cfg = SMALL
    geo = geometry(cfg)
    weights = random_weights(cfg, geo, seed=37, std=0.05)
    ctx, _ = make(cfg, geo, weights, kv_dtype, True, max_tokens=16, max_seqs=16, pages=1024, pps=64)
    rng = np.random.default_rng(0xF0)
    lens = [3, 15, 16, 33, 40, 100, 180, 61]
    max_seqs = [4096, 4096, 4096, 4096, 48, 4096, 4096, 70]
    a, b = _twin_sessions(ctx, rng, lens, max_seqs, geo["kv_cols"], cfg["num_layers"])
    first = rng.integers(0, cfg["vocab"], len(lens))
    assert ctx.forward_replay_info()["launches"] == 0
    got = _sync_steps(b, first, 8)
    info = ctx.forward_replay_info()
    assert (info["launches"], info["sequences"], info["buckets"]) == (6, 8, 1), info
    want = _sync_steps(a, first, 8, want_logits=True)
    assert ctx.forward_replay_info()["launches"] == 6  # steps that fetch logits stay eager
    for k in range(8):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"step {k}")
    # five of the sessions: a new sequence count
    got = _sync_steps(b[:5], got[-1][:5], 8)
    info = ctx.forward_replay_info()
    assert (info["launches"], info["sequences"], info["buckets"]) == (12, 5, 2), info
    want = _sync_steps(a[:5], want[-1][:5], 8, want_logits=True)
    for k in range(8):
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"five sessions, step {k}")
    _same_sessions(a, b)
    ctx.close()
