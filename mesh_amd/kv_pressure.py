"""Decode under KV-cache pressure: session churn, eviction and restore.

The caller side of the provider for the soak configuration (a page pool
smaller than the sessions' total KV): sessions join (Poisson arrivals) and
leave (per-step probability), and when the pool cannot hold the next decode
step the planner evicts sessions the way the reference coordinator does and
restores them when pages free up.

* Eviction = checkpoint + removal (coordinator.rs:871-894): the session's KV
  is exported with the segmented retention window (export_kv_cache with
  max_cached_tokens, forward_pass.rs:2442-2448 -> 1169-1204; the newest
  `retention` rows) and its pages go back to the pool.
* Candidate order = select_eviction_candidate (coordinator.rs:937-990) for
  the default ThroughputFirst mode (api/types.rs:117-121) with every session
  active and recently used: fewest decode steps served first, then the
  larger KV footprint.
* Restore = import_kv_cache (forward_pass.rs:2450-2454 -> 1206-1242): clear,
  scatter the window into fresh pages, continue at the saved position.

The reference makes these copies synchronously.  Here (async_transfers, the
default) each moves over PCIe on a stream of its own while decode steps run
(KVTransfer): an eviction gathers the window into a device buffer and returns
its pages at once, the copy to pinned host memory follows on the
device-to-host stream; the oldest evicted windows are uploaded ahead of their
restore on the host-to-device stream, and a session restored before its
eviction copy finished is scattered straight from that device buffer.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional

import numpy as np

from .provider import (BackendMicrobatchExecutor, DecodeMicrobatchRequest, DeviceContext, KVCacheSnapshot,
                       PinnedBuffer)


@dataclass
class SoakSession:
    sid: int
    token: int
    backend: object = None              # RocmExecutionBackend while resident
    snapshot: Optional[KVCacheSnapshot] = None  # while evicted
    steps_served: int = 0
    transfer: object = None             # KVTransfer of the evicted window: its export or its upload


@dataclass
class SoakStats:
    steps: int = 0
    tokens: int = 0
    joins: int = 0
    leaves: int = 0
    evictions: int = 0
    restores: int = 0
    decode_s: float = 0.0
    evict_s: float = 0.0
    restore_s: float = 0.0
    admit_s: float = 0.0
    wall_s: float = 0.0
    active_hist: List[int] = field(default_factory=list)


class KvPressureSoak:
    """Runs decode steps over a churning session set on one DeviceContext.

    `admit(session, context_len, rng)` fills a new session's KV through
    session.backend (a prefill, or a page reservation standing in for one) and
    returns its first token.  `on_evict(session)` sees each eviction after the
    snapshot is taken; `on_step(sessions, tokens_out, logits)` sees every
    step before the sessions' tokens advance."""

    def __init__(self, ctx: DeviceContext, *, max_sessions: int, join_rate: float, leave_prob: float,
                 retention: int, max_seq_len: int, context_sampler: Callable[[np.random.Generator], int],
                 admit: Callable[[SoakSession, int, np.random.Generator], int], seed: int,
                 on_step: Optional[Callable[[List[SoakSession], List[int], np.ndarray], None]] = None,
                 on_evict: Optional[Callable[[SoakSession], None]] = None, async_transfers: bool = True,
                 prefetch: int = 2):
        self.ctx = ctx
        self.max_sessions = max_sessions
        self.join_rate = join_rate
        self.leave_prob = leave_prob
        self.retention = retention
        self.max_seq_len = max_seq_len
        self.context_sampler = context_sampler
        self.admit = admit
        self.on_step = on_step
        self.on_evict = on_evict
        self.rng = np.random.default_rng(seed)
        self.active: List[SoakSession] = []
        self.evicted: List[SoakSession] = []   # FIFO
        self.free_pinned: list = []             # snapshot buffers of restored sessions, reused
        self.async_transfers = async_transfers
        self.prefetch = prefetch                # evicted windows uploaded ahead of their restore
        self.retiring: list = []                # (KVTransfer, pinned buffer to reuse once it is done)
        self.next_sid = 0
        self.stats = SoakStats()

    # -- pinned snapshot buffers --------------------------------------------------------
    def _window_bytes(self) -> int:
        g = self.ctx.geo
        return 2 * 4 * g.num_layers * self.retention * g.kv_cols

    def _pinned(self):
        """A pinned buffer for one eviction window: a recycled one, else a new one of the
        full window's size (any window fits any buffer, so they keep circulating)."""
        if self.free_pinned:
            return self.free_pinned.pop()
        return PinnedBuffer(self.ctx, self._window_bytes())

    def reserve_pinned(self, n: int):
        """Pins n window buffers ahead (pinning 0.5 GB takes ~10 ms of host time)."""
        for _ in range(n):
            self.free_pinned.append(PinnedBuffer(self.ctx, self._window_bytes()))

    # -- pages --------------------------------------------------------------------------
    @staticmethod
    def pages_for(rows: int) -> int:
        return (rows + 15) // 16 + 1  # a partial first page after a window trim

    def _free(self) -> int:
        return self.ctx.free_pages

    def _evict_one(self, protect: Optional[SoakSession] = None) -> bool:
        cands = [s for s in self.active if s is not protect]
        if not cands:
            return False
        victim = min(cands, key=lambda s: (s.steps_served, -s.backend.live_kv_cache_bytes(), s.sid))
        t0 = time.perf_counter()
        buf = self._pinned()
        if self.async_transfers:
            victim.snapshot, victim.transfer = victim.backend.export_kv_cache_async(self.retention, into=buf)
        else:
            victim.snapshot = victim.backend.export_kv_cache(self.retention, pinned=True, into=buf)
        if buf is not None and (victim.snapshot is None or victim.snapshot.storage is not buf):
            self.free_pinned.append(buf)
        victim.backend.close()  # pages back to the pool
        victim.backend = None
        self.stats.evict_s += time.perf_counter() - t0
        if self.on_evict is not None:
            if victim.transfer is not None:
                victim.transfer.wait()  # the callback reads the snapshot
            self.on_evict(victim)
        self.active.remove(victim)
        self.evicted.append(victim)
        self.stats.evictions += 1
        return True

    def _make_room(self, pages: int, protect: Optional[SoakSession] = None) -> bool:
        while self._free() < pages:
            if not self._evict_one(protect):
                return False
        return True

    # -- churn --------------------------------------------------------------------------
    def add_session(self, context_len: int) -> Optional[SoakSession]:
        if not self._make_room(self.pages_for(min(context_len, self.max_seq_len))):
            return None
        t0 = time.perf_counter()
        s = SoakSession(self.next_sid, 0, self.ctx.new_backend(self.max_seq_len))
        self.next_sid += 1
        s.token = int(self.admit(s, context_len, self.rng))
        self.stats.admit_s += time.perf_counter() - t0
        self.active.append(s)
        return s

    def _leaves(self):
        for s in list(self.active):
            if self.rng.random() < self.leave_prob:
                s.backend.close()
                self.active.remove(s)
                self.stats.leaves += 1
        for s in list(self.evicted):
            if self.rng.random() < self.leave_prob:
                self.evicted.remove(s)
                if s.transfer is not None:
                    self._retire(s.transfer, s.snapshot.storage)
                    s.transfer = None
                elif s.snapshot is not None and s.snapshot.storage is not None:
                    self.free_pinned.append(s.snapshot.storage)  # no copy uses it any more
                self.stats.leaves += 1

    def _joins(self):
        n = int(self.rng.poisson(self.join_rate))
        for _ in range(n):
            if len(self.active) + len(self.evicted) >= self.max_sessions:
                break
            L = int(self.context_sampler(self.rng))
            if self.add_session(L) is not None:
                self.stats.joins += 1

    def _restores(self):
        # oldest evictions first, while the pool holds them and the next step
        while self.evicted:
            s = self.evicted[0]
            rows = s.snapshot.cached_tokens if s.snapshot is not None else 0
            if self._free() < self.pages_for(rows) + len(self.active) + 1:
                break
            t0 = time.perf_counter()
            b = self.ctx.new_backend(self.max_seq_len)
            if s.snapshot is not None and self.async_transfers:
                # from the window's device buffer: its own export still in flight, its upload
                # (issued a step ahead), or an upload issued now that the scatter waits for on the device
                t = s.transfer if s.transfer is not None else self.ctx.upload_kv_async(s.snapshot)
                b.import_kv_cache_transfer(s.snapshot, t)
                self._retire(t, s.snapshot.storage)
                s.transfer = None
            elif s.snapshot is not None:
                b.import_kv_cache(s.snapshot)
                if s.snapshot.storage is not None:
                    self.free_pinned.append(s.snapshot.storage)
            s.backend, s.snapshot = b, None
            self.stats.restore_s += time.perf_counter() - t0
            self.evicted.pop(0)
            self.active.append(s)
            self.stats.restores += 1

    # -- transfers ----------------------------------------------------------------------
    def _retire(self, t, pinned):
        self.retiring.append((t, pinned))

    def _reap(self, block: bool = False):
        """Closes finished transfers (their device buffers go back to the context) and
        recycles their pinned buffers; an evicted window whose export has landed in host
        memory gives up its device buffer."""
        keep = []
        for t, pinned in self.retiring:
            if block or t.done():
                t.close()
                if pinned is not None:
                    self.free_pinned.append(pinned)
            else:
                keep.append((t, pinned))
        self.retiring = keep
        for s in self.evicted[self.prefetch:]:
            if s.transfer is not None and (block or s.transfer.done()):
                s.transfer.close()
                s.transfer = None

    def _prefetch(self):
        """Uploads the oldest evicted windows (the next restores) while the coming step runs."""
        for s in self.evicted[:self.prefetch]:
            if s.transfer is None and s.snapshot is not None:
                s.transfer = self.ctx.upload_kv_async(s.snapshot)

    def finish(self):
        """Waits for every copy in flight and releases the device buffers."""
        self._reap(block=True)
        for s in self.evicted:
            if s.transfer is not None:
                s.transfer.close()
                s.transfer = None

    # -- one decode step ----------------------------------------------------------------
    def step(self, want_logits: bool = False):
        t_start = time.perf_counter()
        if self.async_transfers:
            self._reap()
        self._leaves()
        self._restores()  # evicted sessions resume before new ones are admitted
        self._joins()
        # every resident session may open a new page this step
        self._make_room(len(self.active))
        if self.async_transfers:
            self._prefetch()
        if not self.active:
            return None
        reqs = [DecodeMicrobatchRequest(str(s.sid), s.token, s.backend) for s in self.active]
        t0 = time.perf_counter()
        outs = BackendMicrobatchExecutor.decode_step_batch(reqs, want_logits=want_logits)
        self.stats.decode_s += time.perf_counter() - t0
        toks = [o.sampled_token for o in outs]
        logits = np.stack([o.logits for o in outs]) if want_logits else None
        if self.on_step is not None:
            self.on_step(list(self.active), toks, logits)
        for s, t in zip(self.active, toks):
            s.token = int(t)
            s.steps_served += 1
        self.stats.steps += 1
        self.stats.tokens += len(toks)
        self.stats.active_hist.append(len(self.active))
        self.stats.wall_s += time.perf_counter() - t_start
        return toks, logits
