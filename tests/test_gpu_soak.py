"""Decode under KV-cache pressure with session churn (the soak configuration,
scaled to a small model so that every step is checked against the oracle).

The page pool holds 85% of the sessions' KV; sessions join (Poisson) and
leave; the planner evicts through the segmented-window export and restores
through import (mesh_amd/kv_pressure.py).  The oracle mirrors every session:
prefill, the same retention on eviction, decode of the same tokens.  Checked
every step: logits within 1e-2, greedy tokens where the top-2 margin exceeds
1e-3, cache lengths and positions equal; and the pool's page accounting.
"""
import numpy as np
import pytest

import oracle as O
from mesh_amd import DeviceContext, ModelGeometry
from mesh_amd.kv_pressure import KvPressureSoak
from tests.gpu_util import margin_ok_rows
from tests.testmodels import geometry, oracle_cfg, random_weights

pytestmark = pytest.mark.gpu

CFG = dict(hidden=256, num_heads=4, num_kv_heads=2, num_layers=2, vocab=512, ffn=512, rms_norm_eps=1e-5,
           rope_base=10000.0)


def test_kv_pressure_soak_matches_oracle_through_evictions():
    g = geometry(CFG)
    geo = ModelGeometry(CFG["hidden"], CFG["num_heads"], CFG["num_kv_heads"], CFG["num_layers"], CFG["vocab"],
                        CFG["ffn"], CFG["rms_norm_eps"], CFG["rope_base"], g["shard_start"], g["shard_end"],
                        g["ffn_cols"])
    weights = random_weights(CFG, g, seed=21, std=0.05)
    rng0 = np.random.default_rng(0xC5)
    n0, retention, max_seq = 24, 24, 256

    def sample_len(rng):
        return int(np.clip(np.round(rng.lognormal(np.log(40), 0.8)), 4, 200))

    initial = [sample_len(rng0) for _ in range(n0)]
    pool_pages = int(0.85 * sum((L + 15) // 16 for L in initial))
    ctx = DeviceContext(geo, kv_dtype="bf16", max_tokens=64, max_seqs=64, max_pages_per_seq=max_seq // 16 + 2,
                        split_activations=True)
    ctx.upload_f32_model(weights)
    ctx.create_kv_pool(pool_pages)
    om = O.Model(oracle_cfg(CFG, g), weights)
    mirror = {}

    def admit(s, L, rng):
        toks = rng.integers(0, CFG["vocab"], L).tolist()
        got = s.backend.prefill(toks)
        os_ = O.Session(CFG["num_layers"], geo.kv_cols, 16, max_seq, kv_round_bf16=True)
        want = om.prefill(os_, toks)
        assert np.max(np.abs(got - want)) <= 1e-2
        mirror[s.sid] = os_
        return int(np.argmax(want))

    def on_evict(s):
        snap = mirror[s.sid].export(retention)
        fresh = O.Session(CFG["num_layers"], geo.kv_cols, 16, max_seq, kv_round_bf16=True)
        fresh.import_snapshot(snap)
        mirror[s.sid] = fresh
        assert s.snapshot.cached_tokens == snap["cached_tokens"]
        assert s.snapshot.next_position == snap["next_position"]
        np.testing.assert_allclose(s.snapshot.keys, snap["keys"], rtol=0, atol=2e-2)

    checked = {"rows": 0}

    def on_step(sessions, toks_out, logits):
        want = om.decode([mirror[s.sid] for s in sessions], [s.token for s in sessions])
        assert np.max(np.abs(logits - want)) <= 1e-2, np.max(np.abs(logits - want))
        ok = margin_ok_rows(want)
        np.testing.assert_array_equal(np.asarray(toks_out)[ok], np.argmax(want, 1)[ok])
        for s in sessions:
            o = mirror[s.sid]
            assert s.backend.cache_seq_len() == o.seq_len(), s.sid
            assert s.backend.sequence_position() == o.position, s.sid
        checked["rows"] += len(sessions)

    soak = KvPressureSoak(ctx, max_sessions=40, join_rate=1.0, leave_prob=1 / 16, retention=retention,
                          max_seq_len=max_seq, context_sampler=sample_len, admit=admit, seed=7,
                          on_step=on_step, on_evict=on_evict)
    for L in initial:
        soak.add_session(L)
    for _ in range(16):
        soak.step(want_logits=True)
        used = sum(s.backend.allocated_pages() for s in soak.active)
        assert used + ctx.free_pages == pool_pages
    st = soak.stats
    assert st.evictions > 0 and st.restores > 0 and checked["rows"] > 100, st
    ctx.close()
