"""Bookkeeping of the KV-pressure soak's copies in flight (mesh_amd.kv_pressure
with async transfers), on the CPU with a fake context: sessions, page pool,
transfers that finish a number of decode steps after they start.

Checked every call: a pinned snapshot buffer is never handed to a new
eviction while a copy into or out of it runs; a restore uses the session's
own transfer (its export still running, or its upload) when there is one and
otherwise uploads; the oldest evicted windows are uploaded ahead, at most
`prefetch` at a time; the pool's page accounting stays exact; finish()
leaves no transfer open."""
import math
from dataclasses import dataclass

import numpy as np
import pytest

import mesh_amd.kv_pressure as KP
from mesh_amd import KVCacheSnapshot

LAYERS, KV_COLS, RETENTION = 2, 8, 64


@dataclass
class Geo:
    num_layers: int = LAYERS
    kv_cols: int = KV_COLS


class FakePinned:
    count = 0

    def __init__(self, ctx, nbytes):
        FakePinned.count += 1
        self.ctx, self.nbytes, self.ptr = ctx, nbytes, 1


class FakeTransfer:
    def __init__(self, ctx, kind, storage, rows):
        self.ctx, self.kind, self.storage, self.rows = ctx, kind, storage, rows
        self.ready_at = ctx.clock + ctx.lag
        self.closed = False
        ctx.transfers.append(self)

    def done(self):
        assert not self.closed
        return self.ctx.clock >= self.ready_at

    def wait(self):
        self.ready_at = min(self.ready_at, self.ctx.clock)

    def close(self):
        self.wait()
        self.closed = True

    def busy(self):  # a copy into / out of its pinned buffer is running
        return not self.closed and self.ctx.clock < self.ready_at


class FakeBackend:
    def __init__(self, ctx):
        self.ctx, self.rows, self.position, self.open = ctx, 0, 0, True

    def pages(self):
        return (self.rows + 15) // 16 + 1 if self.rows else 0

    def kv_reserve(self, n):
        self.rows, self.position = n, n
        assert self.ctx.used() <= self.ctx.total

    def live_kv_cache_bytes(self):
        return self.rows

    def _window(self, retention):
        return min(self.rows, retention)

    def export_kv_cache_async(self, retention, into=None):
        assert into is not None and not any(t.busy() and t.storage is into for t in self.ctx.transfers), \
            "pinned buffer handed out while a copy uses it"
        n = self._window(retention)
        snap = KVCacheSnapshot(self.position, n, None, None, into)
        return snap, FakeTransfer(self.ctx, "out", into, n)

    def export_kv_cache(self, retention, pinned=True, into=None):
        n = self._window(retention)
        return KVCacheSnapshot(self.position, n, None, None, into)

    def import_kv_cache_transfer(self, snap, t):
        assert not t.closed and t.rows == snap.cached_tokens
        self.ctx.imports.append(t.kind)
        self.rows, self.position = snap.cached_tokens, snap.next_position
        assert self.ctx.used() <= self.ctx.total

    def import_kv_cache(self, snap):
        assert not any(t.busy() and t.storage is snap.storage for t in self.ctx.transfers)
        self.ctx.imports.append("host")
        self.rows, self.position = snap.cached_tokens, snap.next_position

    def close(self):
        self.open = False


class FakeCtx:
    def __init__(self, total, lag):
        self.geo, self.total, self.lag, self.clock = Geo(), total, lag, 0
        self.backends, self.transfers, self.imports = [], [], []

    def used(self):
        return sum(b.pages() for b in self.backends if b.open)

    @property
    def free_pages(self):
        return self.total - self.used()

    def new_backend(self, max_seq_len):
        b = FakeBackend(self)
        self.backends.append(b)
        return b

    def upload_kv_async(self, snap):
        assert not any(t.busy() and t.storage is snap.storage and t.kind == "out" for t in self.transfers), \
            "upload of a window whose export is still running"
        return FakeTransfer(self, "in", snap.storage, snap.cached_tokens)


@dataclass
class Out:
    sampled_token: int
    logits: object = None


@pytest.mark.parametrize("lag,prefetch", [(1, 2), (2, 4), (3, 1)])
def test_soak_transfer_bookkeeping(monkeypatch, lag, prefetch):
    ctx = FakeCtx(total=110, lag=lag)

    def decode_step_batch(reqs, want_logits=False):
        assert all(r.backend.open for r in reqs)
        for r in reqs:
            r.backend.rows += 1
            r.backend.position += 1
        assert ctx.used() <= ctx.total
        ctx.clock += 1  # copies in flight progress while the step runs
        return [Out(0) for _ in reqs]

    monkeypatch.setattr(KP.BackendMicrobatchExecutor, "decode_step_batch", staticmethod(decode_step_batch))
    monkeypatch.setattr(KP, "PinnedBuffer", FakePinned)
    FakePinned.count = 0

    def admit(s, L, rng):
        s.backend.kv_reserve(L)
        return 0

    soak = KP.KvPressureSoak(ctx, max_sessions=24, join_rate=1.5, leave_prob=1 / 40, retention=RETENTION,
                             max_seq_len=4096,
                             context_sampler=lambda rng: int(np.clip(rng.lognormal(math.log(60), 0.8), 8, 400)),
                             admit=admit, seed=lag * 10 + prefetch, prefetch=prefetch)
    for L in (40, 90, 150, 220, 30, 60, 300, 75, 120, 45):
        soak.add_session(L)
    for _ in range(40):
        soak.step()
        # uploads ahead only for the oldest evicted windows, at most `prefetch`
        ups = [s for s in soak.evicted if s.transfer is not None and s.transfer.kind == "in"]
        assert len(ups) <= prefetch and all(s in soak.evicted[:prefetch] for s in ups)
        # windows past the upload-ahead range keep their device buffer only while their export runs
        for s in soak.evicted[prefetch:]:
            assert s.transfer is None or s.transfer.kind == "out"
        open_t = [t for t in ctx.transfers if not t.closed]
        assert len(open_t) <= prefetch + soak.stats.evictions  # bounded by what can be in flight
        assert ctx.used() + ctx.free_pages == ctx.total
    st = soak.stats
    assert st.evictions > 5 and st.restores > 5, st
    # restores came from device buffers (running exports, uploads ahead, uploads issued at restore)
    assert set(ctx.imports) <= {"out", "in"} and "in" in ctx.imports
    soak.finish()
    assert all(t.closed for t in ctx.transfers)
    assert all(s.transfer is None for s in soak.evicted)
    # buffers circulate: far fewer pinned allocations than evictions
    assert FakePinned.count < st.evictions
    # and none is lost: each is free or holds an evicted window (also after evicted sessions left)
    held = [s.snapshot.storage for s in soak.evicted if s.snapshot is not None and s.snapshot.storage is not None]
    assert len({id(b) for b in held} | {id(b) for b in soak.free_pinned}) == len(held) + len(soak.free_pinned)
    assert len(held) + len(soak.free_pinned) == FakePinned.count


def test_synchronous_copies_keep_the_reference_order(monkeypatch):
    ctx = FakeCtx(total=120, lag=2)
    monkeypatch.setattr(KP.BackendMicrobatchExecutor, "decode_step_batch",
                        staticmethod(lambda reqs, want_logits=False: [Out(0) for _ in reqs]))
    monkeypatch.setattr(KP, "PinnedBuffer", FakePinned)
    soak = KP.KvPressureSoak(ctx, max_sessions=16, join_rate=1.0, leave_prob=0.0, retention=RETENTION,
                             max_seq_len=4096, context_sampler=lambda rng: 100, seed=3,
                             admit=lambda s, L, rng: s.backend.kv_reserve(L) or 0, async_transfers=False)
    for _ in range(12):
        soak.add_session(100)
    for _ in range(10):
        soak.step()
    assert not ctx.transfers and soak.stats.evictions > 0
    assert set(ctx.imports) <= {"host"}
