"""Parity of the full-width Llama-3-8B configurations against the oracle.

The model is the benchmark's own: 32 layers, hidden 4096, 32 q / 8 kv heads,
head_dim 128, FFN 14336, vocab 128256, bf16 N(0, 0.02) weights generated on
the device (bench.device_model), whose bf16 bit patterns are downloaded for
the oracle's bf16-weight model (bit-identical to its f32 form).  KV pages
hold the benchmark's synthetic N(0, 1) bf16 values; a session checked against
the oracle has its cached rows exported (a bit-exact gather) and imported into
an oracle session, then both run the same decode step.  Decode rows are
independent, so a sample of sessions is checked against the oracle running
only those sessions.

* The benchmarked step: 256 sessions, lognormal contexts (median 1024,
  sigma 1, clip [64, 8192], seed 0xC5), one staged decode step exactly as
  bench.py times it; 16 sampled sessions checked.
* C5, KV pressure: the same model and contexts with the page pool at 85% of
  their pages, Poisson joins (4 per step), leaves (1/64), eviction through the
  2048-token segmented-window export and restore through import
  (mesh_amd.kv_pressure, the reference coordinator's order).  Every step
  checks a sample that includes every session restored since the last step
  (its restored window must equal the evicted snapshot bit for bit), and the
  pool's page accounting.

The row a step appends is rounded from f32 to bf16 by both the device and
the oracle, each from its own f32 value; where that value sits near a bf16
rounding tie the two can store neighbouring bf16 values (a 2^-8 relative
jump), and 32 layers amplify such flips to ~1e-2 in the logits.  So each
check first requires every element the device stored to be within one bf16
step of the oracle's own rounding of its f32 value, then runs the oracle
with the device's stored rows (Model.decode_forced) and compares the step's
logits.  The unforced oracle's distance is printed for the record.

Bars: appended K / V elements within one bf16 step, logits within 1e-2
absolute, greedy ids equal where the oracle's top-2 margin exceeds 1e-3.
"""
import math
import time

import numpy as np
import pytest
import xxhash

import bench
import oracle as O
from mesh_amd.kv_pressure import KvPressureSoak
from tests.test_gpu_model import check_logits

pytestmark = pytest.mark.gpu

WORKLOAD = "llama3_8b_b256"


def _progress(msg):
    print(f"[llama3-8b] {time.strftime('%H:%M:%S')} {msg}", flush=True)


@pytest.fixture(scope="module")
def llama3():
    host = {}
    ctx, g = bench.device_model(WORKLOAD, True, host_weights=host)
    geo = bench.WORKLOADS[WORKLOAD]["geo"]
    cfg = dict(hidden=g.hidden, num_heads=g.num_heads, num_kv_heads=g.num_kv_heads, num_layers=g.num_layers,
               vocab=g.vocab, ffn_cols=g.ffn_cols, rms_norm_eps=1e-5, rope_base=geo["rope_base"])
    om = O.Model(cfg, host)
    assert om.bf16
    _progress("model resident on the device and in the oracle")
    yield ctx, g, om
    ctx.close()


def _oracle_session(g, snap, max_seq):
    """An oracle session holding the exported rows minus the newest one (the
    row the checked step appended), at the position before that step."""
    rows = snap.cached_tokens - 1
    s = O.Session(g.num_layers, g.kv_cols, 16, max_seq, kv_round_bf16=True)
    if rows:
        s.import_snapshot({"keys": np.ascontiguousarray(snap.keys[:, :rows]),
                           "values": np.ascontiguousarray(snap.values[:, :rows]),
                           "base_position": snap.first_cached_position(), "next_position": snap.next_position - 1,
                           "cached_tokens": rows})
    else:
        s.position = snap.next_position - 1
    return s


def _forced_step(g, om, snaps, tokens, max_seq, label):
    """The oracle's step over the exported sessions with the device's appended
    rows forced.  Every element the device stored must be a bf16 rounding of
    a value within f32 noise of the oracle's own: |stored - own| <= 2^-8 |own|
    (half a bf16 step of the value) + 2 noise, with the noise at 1e-3 of the
    row's largest element (the step's own f32 drift from layer to layer stays
    far below it; a wrong row is off by O(1)).  Returns the forced logits, the
    unforced oracle's logits and the number of elements whose rounding
    differs from the oracle's."""
    force_k = np.stack([snap.keys[:, -1] for snap in snaps], axis=1)
    force_v = np.stack([snap.values[:, -1] for snap in snaps], axis=1)
    want, own_k, own_v = om.decode_forced([_oracle_session(g, s, max_seq) for s in snaps], tokens, force_k,
                                          force_v)
    flips = 0
    for stored, own in ((force_k, own_k), (force_v, own_v)):
        noise = 1e-3 * np.abs(own).max(axis=-1, keepdims=True)
        bound = 2.0 ** -8 * np.abs(own) + 2 * noise
        excess = np.abs(stored - own) - bound
        assert excess.max() <= 0, f"{label}: a stored K / V element is {excess.max():.3g} beyond a valid rounding"
        flips += int((stored != O.round_bf16(own)).sum())
    free = om.decode([_oracle_session(g, s, max_seq) for s in snaps], tokens)
    return want, free, flips


def test_benchmarked_256_session_step_matches_oracle_on_sampled_sessions(llama3):
    ctx, g, om = llama3
    lib = ctx.lib
    b = bench.GpuDecodeBench(WORKLOAD, 1, model=(ctx, g))
    try:
        B, V = b.B, g.vocab
        tokens = b.tokens(0)
        d_logits = b._dev(4 * B * V)
        ctx.check(lib.zr_forward_staged_async(ctx.h, b.staged[0], b.tok[0], b.tok[1], d_logits))
        ctx.check(lib.zr_synchronize(ctx.h))
        logits = np.empty((B, V), np.float32)
        ctx.check(lib.zr_memcpy_d2h(ctx.h, logits.ctypes.data, d_logits, logits.nbytes))
        lib.zr_device_free(ctx.h, d_logits)
        out_tokens = b.tokens(1)
        assert np.isfinite(logits).all()
        # the step's own greedy ids are the argmax of its logits (first index on ties)
        np.testing.assert_array_equal(out_tokens, np.argmax(logits, 1))
        _progress("benchmarked step ran")
        ctxlens = b.ctxlens
        sample = sorted({int(np.argmax(ctxlens)), int(np.argmin(ctxlens))} |
                        {int(x) for x in np.random.default_rng(16).choice(B, 14, replace=False)})
        while len(sample) < 16:
            sample = sorted(set(sample) | {int(np.random.default_rng(len(sample)).integers(B))})
        snaps = [b.backends[i].export_kv_cache() for i in sample]
        for i, snap in zip(sample, snaps):  # an 8192-row window drops its oldest row on the append
            assert snap.next_position == int(ctxlens[i]) + 1
            assert snap.cached_tokens == min(int(ctxlens[i]) + 1, b.max_seq)
        want, free, flipped = _forced_step(g, om, snaps, tokens[sample], b.max_seq, "benchmarked step")
        _progress(f"oracle decoded {len(sample)} sampled sessions (contexts {sorted(int(ctxlens[i]) for i in sample)})")
        err = check_logits(logits[sample], want, "benchmarked step")
        print(f"benchmarked step: max |logit - oracle| = {err:.3g} over {len(sample)} sessions; "
              f"{flipped} of {2 * want.shape[0] * g.num_layers * g.kv_cols} appended K / V elements round the other way; "
              f"unforced oracle distance {float(np.max(np.abs(logits[sample] - free))):.3g}", flush=True)
    finally:
        b.close()


def test_c5_kv_pressure_soak_full_llama3_width(llama3):
    ctx, g, om = llama3
    w = bench.WORKLOADS[WORKLOAD]
    soak_cfg = bench.SOAK
    ctxlens = w["contexts"]()
    need = int(sum((int(L) + 15) // 16 for L in ctxlens))
    pool = int(soak_cfg["pool_frac"] * need)
    ctx.create_kv_pool(pool)
    ctx.check(ctx.lib.zr_kv_pool_fill_normal(ctx.h, 4242, 1.0))
    max_seq = w["max_seq_len"]
    evicted = {}  # sid -> (hash of K, hash of V, cached rows, next position)
    checked = {"rows": 0, "restored": 0, "steps": 0}
    pick = np.random.default_rng(0x5C)

    def digest(a):
        return xxhash.xxh3_64(np.ascontiguousarray(a).view(np.uint8)).intdigest()

    def sample_len(rng):
        return int(np.clip(np.round(rng.lognormal(math.log(1024), 1.0)), 64, 8192))

    def admit(s, L, rng):
        s.backend.kv_reserve(L)  # the pages hold synthetic KV, standing in for a prefill
        return int(rng.integers(0, g.vocab))

    def on_evict(s):
        snap = s.snapshot
        assert snap is not None and 0 < snap.cached_tokens <= soak_cfg["retention"]
        evicted[s.sid] = (digest(snap.keys), digest(snap.values), snap.cached_tokens, snap.next_position)

    def on_step(sessions, toks_out, logits):
        restored = [i for i, s in enumerate(sessions) if s.sid in evicted]
        others = [i for i in range(len(sessions)) if sessions[i].sid not in evicted]
        extra = max(0, 6 - len(restored[:4]))
        idx = sorted(restored + [int(x) for x in pick.choice(others, min(extra, len(others)), replace=False)])
        snaps = [sessions[i].backend.export_kv_cache() for i in idx]
        for i, snap in zip(idx, snaps):
            sid = sessions[i].sid
            if sid in evicted:  # the restored window is the evicted snapshot, bit for bit
                hk, hv, rows, nxt = evicted.pop(sid)
                assert snap.cached_tokens == rows + 1 and snap.next_position == nxt + 1, sid
                assert digest(snap.keys[:, :rows]) == hk and digest(snap.values[:, :rows]) == hv, sid
                checked["restored"] += 1
        label = f"soak step {checked['steps']}"
        want, free, flipped = _forced_step(g, om, snaps, [sessions[i].token for i in idx], max_seq, label)
        err = check_logits(logits[idx], want, label)
        ok = np.sort(want, 1)
        ok = (ok[:, -1] - ok[:, -2]) > 1e-3
        np.testing.assert_array_equal(np.asarray(toks_out)[idx][ok], np.argmax(want, 1)[ok])
        checked["rows"] += len(idx)
        checked["steps"] += 1
        _progress(f"soak step {checked['steps']}: {len(sessions)} active, checked {len(idx)} "
                  f"({len(restored)} restored), max err {err:.3g}, {flipped} rounding flips, "
                  f"unforced {float(np.max(np.abs(logits[idx] - free))):.3g}")

    soak = KvPressureSoak(ctx, max_sessions=soak_cfg["max_sessions"], join_rate=soak_cfg["join_rate"],
                          leave_prob=soak_cfg["leave_prob"], retention=soak_cfg["retention"], max_seq_len=max_seq,
                          context_sampler=sample_len, admit=admit, seed=soak_cfg["seed"], on_step=on_step,
                          on_evict=on_evict)
    for L in ctxlens:
        soak.add_session(int(L))
    _progress(f"admitted {len(soak.active)} sessions, {len(soak.evicted)} evicted, pool {pool} pages")
    # restores need a window's pages plus a page per resident session free,
    # which the churn reaches after a few steps
    for _ in range(24):
        soak.step(want_logits=True)
        used = sum(s.backend.allocated_pages() for s in soak.active)
        assert used + ctx.free_pages == pool, (used, ctx.free_pages, pool)
        if soak.stats.restores > 0 and checked["restored"] > 0 and soak.stats.steps >= 6:
            break
    st = soak.stats
    print(f"C5 soak: {st.steps} steps, joins {st.joins}, leaves {st.leaves}, evictions {st.evictions}, "
          f"restores {st.restores}, rows checked {checked['rows']} ({checked['restored']} restored)", flush=True)
    assert st.evictions > 0 and st.restores > 0 and checked["restored"] > 0, st
    for s in list(soak.active):
        s.backend.close()
    assert ctx.free_pages == pool
