"""Decode-step benchmark of the rocm provider on one MI355X.

Headline workload: one ragged decode step of a Llama-3-8B-shape model
(32 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, FFN 14336, vocab
128256, bf16 weights and bf16 paged KV) over 256 sessions whose contexts are
lognormal (median 1024, sigma 1, clipped to [64, 8192]), page 16.  The bs-32
TinyLlama-shape step (22 layers, contexts U[128, 2048]) is measured in the same
run and reported under "bs32".

Inputs are resident in HBM before the timed region: weights are random-init
bf16 N(0, 0.02) generated on the device and the KV pages of every session's
context are filled with N(0, 1) bf16 (standing in for prefill output).  The
timed region is the serving loop (zrh_decode_pipeline): every step does its
host page-table work, stages its metadata, copies it to the device, replays
the bucket's captured step graph (the fused profile's ReplayPreferred
strategy, one capture per bucket, before the timing) and copies its greedy ids
back, which the host reads while the next step runs; the ids are fed to the
next step on the device.  The attention kernel's duration (the roofline)
comes from HIP events recorded on the provider's stream around every
attention launch of as many pre-staged steps launched kernel by kernel
("eager"; events recorded by graph nodes do not time).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--skip-bs32] [--skip-soak]
       python bench.py --calibrate-copy   (a plain 1 GiB device copy, for scaling
                                           rocprofv3 FETCH_SIZE / WRITE_SIZE)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "paged_attention_llama3_8b_b256_traffic.md")
METRIC = "decode tokens/sec @1 MI355X (bs 32/256); paged-attn HBM GB/s as % of peak"


def contexts_lognormal(seed, n, median, sigma, lo, hi):
    rng = np.random.default_rng(seed)
    return np.clip(np.round(rng.lognormal(math.log(median), sigma, n)), lo, hi).astype(np.int64)


def contexts_uniform(seed, n, lo, hi):
    return np.random.default_rng(seed).integers(lo, hi + 1, n).astype(np.int64)


WORKLOADS = {
    "llama3_8b_b256": dict(
        geo=dict(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=32, vocab=128256, ffn=14336,
                 rope_base=500000.0),
        batch=256, max_seq_len=8192,
        contexts=lambda: contexts_lognormal(0xC5, 256, 1024, 1.0, 64, 8192),
        desc="Llama-3-8B-shape decode step, 256 sessions, lognormal contexts (median 1024, sigma 1, "
             "clip [64, 8192]), page 16, bf16 weights + bf16 KV, 32 layers, greedy"),
    "llama3_8b_tp2_b64": dict(
        geo=dict(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=32, vocab=128256, ffn=14336,
                 rope_base=500000.0, shard_start=0, shard_end=2048, ffn_cols=7168),
        batch=64, max_seq_len=8192,
        contexts=lambda: contexts_lognormal(0xC4, 64, 1024, 1.0, 64, 8192),
        desc="Llama-3-8B tensor-parallel shard 0 of 2 (q columns 0-2047 = 16 q / 4 kv heads, FFN columns "
             "0-7167), decode step, 64 sessions, lognormal contexts (median 1024, sigma 1, clip [64, 8192]), "
             "page 16, bf16 weights + bf16 KV, 32 layers, greedy; O and down give the pre-all-reduce partials "
             "(the all-reduce is the identity on one worker)"),
    "tinyllama_b32": dict(
        geo=dict(hidden=2048, num_heads=32, num_kv_heads=4, num_layers=22, vocab=32000, ffn=5632,
                 rope_base=10000.0),
        batch=32, max_seq_len=4096,
        contexts=lambda: contexts_uniform(0xC2, 32, 128, 2048),
        desc="TinyLlama-1.1B-shape decode step, 32 sessions, contexts U[128, 2048], page 16, "
             "bf16 weights + bf16 KV, 22 layers, greedy"),
}


def gemm_flops(geo, batch):
    """MFMA work of one decode step's projections (2 flops per multiply-add)."""
    H, Q, KV, F, V, L = geo.hidden, geo.q_cols, geo.kv_cols, geo.ffn_cols, geo.vocab, geo.num_layers
    return 2.0 * batch * (L * (H * (Q + 2 * KV) + Q * H + H * 2 * F + F * H) + H * V)


def measured_traffic():
    """HBM bytes per paged-attention launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (already scaled by the copy calibration)."""
    try:
        for line in open(TRAFFIC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def step_bytes(geo, batch, kv_rows_total, kv_bytes=2):
    """Algorithmic HBM bytes of one decode step: every weight once (bf16), the
    embedding rows, every cached K/V row of every layer once (`kv_bytes` per
    element: 2 bf16, 4 f32), the new K/V rows written, and the per-row
    activations in and out of each kernel."""
    H, Q, KV, F, V, L = geo.hidden, geo.q_cols, geo.kv_cols, geo.ffn_cols, geo.vocab, geo.num_layers
    weights = 2 * (L * (H * (Q + 2 * KV) + Q * H + H * 2 * F + F * H) + H * V) + 4 * (2 * L + 1) * H
    kv = L * kv_rows_total * KV * 2 * kv_bytes + L * batch * KV * 2 * kv_bytes
    act = 4 * batch * (L * (3 * H + 2 * (Q + 2 * KV) + 2 * Q + 2 * H + 3 * F + 2 * H) + V)
    return weights + 2 * batch * H + kv + act


def device_model(name, split=True, max_tokens=None, max_seqs=None, host_weights=None, kv_dtype="bf16"):
    """A DeviceContext holding the workload's model with random-init bf16
    N(0, 0.02) weights generated on the device (RMSNorm gains 1) and a KV
    pool of `kv_dtype` ("bf16", or "f32" as the reference stores it).  A dict
    passed as `host_weights` receives host copies of the generated weights as
    bf16 bit patterns in the reference [in, out] layout (embedding, lm_head,
    final_norm, layers), e.g. for a parity check of the same model."""
    from mesh_amd import DeviceContext, ModelGeometry, _lib

    w = WORKLOADS[name]
    g = ModelGeometry(**w["geo"])
    B = w["batch"]
    ctx = DeviceContext(g, kv_dtype=kv_dtype, max_tokens=max_tokens or B, max_seqs=max_seqs or B,
                        max_pages_per_seq=w["max_seq_len"] // 16 + 2, split_activations=split)
    lib = ctx.lib

    def dev(nbytes):
        p = C.c_void_p()
        ctx.check(lib.zr_device_alloc(ctx.h, int(nbytes), C.byref(p)))
        return p.value

    H, Q, KV, F, V = g.hidden, g.q_cols, g.kv_cols, g.ffn_cols, g.vocab
    shapes = dict(w_q=(H, Q), w_k=(H, KV), w_v=(H, KV), w_o=(Q, H), w_gate=(H, F), w_up=(H, F), w_down=(F, H))
    bufs = {k: dev(2 * a * b) for k, (a, b) in shapes.items()}
    ones = np.ones(H, np.float32)

    def download(ptr, shape):
        out = np.empty(shape, np.uint16)
        ctx.check(lib.zr_memcpy_d2h(ctx.h, out.ctypes.data, ptr, out.nbytes))
        return out

    if host_weights is not None:
        host_weights["layers"] = []
    for layer in range(g.num_layers):
        for i, (k, (a, b)) in enumerate(shapes.items()):
            ctx.check(lib.zr_fill_normal_bf16(ctx.h, bufs[k], a * b, 1000 * layer + i + 1, 0.02))
        if host_weights is not None:
            hw = {k: download(bufs[k], shp) for k, shp in shapes.items()}
            hw["attn_norm"], hw["mlp_norm"] = ones, ones
            host_weights["layers"].append(hw)
        lw = _lib.LayerWeights()
        for k in shapes:
            setattr(lw, k, C.cast(bufs[k], _lib.c_u16_p))
        lw.attn_norm = ones.ctypes.data_as(_lib.c_f32_p)
        lw.mlp_norm = ones.ctypes.data_as(_lib.c_f32_p)
        ctx.check(lib.zr_upload_layer(ctx.h, layer, C.byref(lw)))
    for b in bufs.values():
        lib.zr_device_free(ctx.h, b)
    emb, head = dev(2 * V * H), dev(2 * H * V)
    ctx.check(lib.zr_fill_normal_bf16(ctx.h, emb, V * H, 777, 0.02))
    ctx.check(lib.zr_fill_normal_bf16(ctx.h, head, H * V, 778, 0.02))
    ctx.check(lib.zr_upload_globals(ctx.h, C.cast(emb, _lib.c_u16_p), ones.ctypes.data_as(_lib.c_f32_p),
                                    C.cast(head, _lib.c_u16_p)))
    if host_weights is not None:
        host_weights["embedding"] = download(emb, (V, H))
        host_weights["lm_head"] = download(head, (H, V))
        host_weights["final_norm"] = ones
    lib.zr_device_free(ctx.h, emb)
    lib.zr_device_free(ctx.h, head)
    return ctx, g


class GpuDecodeBench:
    """One workload resident on the GPU with `steps_total` decode steps staged.
    `model` = (DeviceContext, ModelGeometry) reuses a model built by
    device_model (its KV pool is replaced; the caller keeps the context)."""

    def __init__(self, name, steps_total, split=True, model=None, host_steps=0, kv_dtype="bf16"):
        from mesh_amd import _lib

        self._lib = _lib
        w = WORKLOADS[name]
        self.name, self.w = name, w
        self.B = w["batch"]
        self.ctxlens = w["contexts"]()
        self.max_seq = w["max_seq_len"]
        self.owns_ctx = model is None
        self.ctx, self.geo = device_model(name, split, kv_dtype=kv_dtype) if model is None else model
        ctx, lib, g = self.ctx, self.ctx.lib, self.geo
        V = g.vocab
        # KV pool: every session's context plus the benchmarked steps (staged
        # ahead, and `host_steps` more run through the host entry point)
        grow = steps_total + host_steps
        pages = int(sum((min(int(L) + grow, self.max_seq) + 15) // 16 + 1 for L in self.ctxlens))
        ctx.create_kv_pool(pages)
        ctx.check(lib.zr_kv_pool_fill_normal(ctx.h, 4242, 1.0))
        self.backends = [ctx.new_backend(self.max_seq) for _ in range(self.B)]
        for b, L in zip(self.backends, self.ctxlens):
            b.kv_reserve(int(L))  # the pages hold the synthetic prefix KV
        # stage every step's metadata on the device ahead of the timed region
        arr = (C.c_void_p * self.B)(*[b.h for b in self.backends])
        ptrs = C.cast(arr, C.POINTER(C.c_void_p))
        q_len = np.ones(self.B, np.int32)
        self.staged, self.kv_rows = [], []
        for _ in range(steps_total):
            st = C.c_void_p()
            ctx.check(lib.zrh_stage_mixed(ptrs, self.B, q_len.ctypes.data_as(_lib.c_int_p), None, C.byref(st)))
            self.staged.append(st.value)
            self.kv_rows.append(sum(b.cache_seq_len() for b in self.backends))
        self.tok = [self._dev(4 * self.B), self._dev(4 * self.B)]
        first = np.random.default_rng(1).integers(0, V, self.B).astype(np.uint32)
        ctx.check(lib.zr_memcpy_h2d(ctx.h, self.tok[0], first.ctypes.data, first.nbytes))

    def _dev(self, nbytes):
        p = C.c_void_p()
        self.ctx.check(self.ctx.lib.zr_device_alloc(self.ctx.h, int(nbytes), C.byref(p)))
        return p.value

    def run(self, first, count, timed, mask=0xF):
        """Runs staged steps [first, first + count); with `timed`, HIP events are
        recorded around the launches of the kernel classes in `mask`."""
        ctx, lib = self.ctx, self.ctx.lib
        if timed:
            ctx.check(lib.zr_timing_begin(ctx.h, mask))
        ctx.check(lib.zr_synchronize(ctx.h))
        t0 = time.perf_counter()
        for i in range(first, first + count):
            ctx.check(lib.zr_forward_staged_async(ctx.h, self.staged[i], self.tok[i % 2], self.tok[(i + 1) % 2], None))
        ctx.check(lib.zr_synchronize(ctx.h))
        dt = time.perf_counter() - t0
        ms = (C.c_double * 5)()
        n = (C.c_int * 5)()
        if timed:
            ctx.check(lib.zr_timing_end(ctx.h, ms, n))
        return dt, list(ms), list(n)

    def run_host(self, count, tokens):
        """`count` decode steps through zrh_decode_step_batch, the boundary's
        host entry point (host page tables, zr_stage with its H2D copy, the
        packing kernel, the forward pass, the token D2H), each step fed the
        previous step's greedy tokens.  Returns (seconds, last tokens)."""
        ctx, lib = self.ctx, self.ctx.lib
        arr = (C.c_void_p * self.B)(*[b.h for b in self.backends])
        ptrs = C.cast(arr, C.POINTER(C.c_void_p))
        u32 = C.POINTER(C.c_uint32)
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.zeros(self.B, np.uint32)
        t0 = time.perf_counter()
        for _ in range(count):
            ctx.check(lib.zrh_decode_step_batch(ptrs, self.B, toks.ctypes.data_as(u32), out.ctypes.data_as(u32),
                                                None, None))
            toks, out = out, toks
        return time.perf_counter() - t0, toks

    def run_pipeline(self, warmup, count, tokens):
        """The serving loop (zrh_decode_pipeline through mesh_amd.DecodePipeline):
        every step does its host page-table work (window trim, page
        reservation), stages its metadata into pinned memory, copies it to the
        device on a copy stream, replays the bucket's captured step graph and
        copies its greedy ids back; the host reads each step's ids while the
        next step runs.  `warmup` steps (the bucket's captures among them),
        then `count` timed steps, synchronised on both sides.  Returns
        (seconds, last ids, pipeline info)."""
        from mesh_amd import DecodePipeline

        pipe = DecodePipeline(self.backends, tokens)
        try:
            for _ in range(warmup):
                pipe.step()
            if warmup:
                pipe.finish()  # (a pipeline that has run no step has nothing to finish)
            t0 = time.perf_counter()
            for _ in range(count):
                pipe.step()
            last = pipe.finish()
            dt = time.perf_counter() - t0
            return dt, last, pipe.info()
        finally:
            pipe.close()

    def tokens(self, i):
        out = np.zeros(self.B, np.uint32)
        self.ctx.check(self.ctx.lib.zr_memcpy_d2h(self.ctx.h, out.ctypes.data, self.tok[i % 2], out.nbytes))
        return out

    def close(self):
        for st in self.staged:
            self.ctx.lib.zr_staged_destroy(st)
        self.staged = []
        for p in self.tok:
            self.ctx.lib.zr_device_free(self.ctx.h, p)
        self.tok = []
        if self.owns_ctx:
            self.ctx.close()
        else:
            for b in self.backends:
                b.close()
        self.backends = []


BREAKDOWN_STEPS = 2


def measure(name, steps, warmup, kv_dtype="bf16"):
    """Pre-staged steps first: `warmup` untimed, `steps` launched kernel by
    kernel (zr_forward_staged_async) with HIP events around the attention
    launches only (the roofline figure), then BREAKDOWN_STEPS with events
    around every kernel class, for the per-class time split.  Then the timed
    region, the headline: `steps` decode steps of the same sessions through the
    pipelined serving loop (GpuDecodeBench.run_pipeline: host page tables,
    metadata staging and copy, the replayed step graph and the id copy-back of
    every step inside the timing), after `warmup` untimed ones.  Then as many
    steps through the synchronous host entry point (zrh_decode_step_batch),
    timed end to end."""
    bench = GpuDecodeBench(name, warmup + steps + BREAKDOWN_STEPS, host_steps=2 * (steps + warmup), kv_dtype=kv_dtype)
    g, B = bench.geo, bench.B
    kv_size = 2 if kv_dtype == "bf16" else 4
    bench.run(0, warmup, timed=False)
    dt_eager, ms_t, n_t = bench.run(warmup, steps, timed=True, mask=1)
    assert bench.tokens(warmup + steps).max() < g.vocab
    _, ms_b, n_b = bench.run(warmup + steps, BREAKDOWN_STEPS, timed=True, mask=0xF)
    cached = [b.cache_seq_len() for b in bench.backends]
    dt, last, pinfo = bench.run_pipeline(warmup, steps, bench.tokens(warmup + steps + BREAKDOWN_STEPS))
    assert last.max() < g.vocab
    ms_per_step = dt / steps * 1000.0
    # attention: algorithmic bytes per launch (K+V of every attended row in the
    # pool's dtype; Q in and the output out, f32), averaged over the eager
    # steps' launches
    # rows the pipeline's timed steps attend (every window capped at max_seq_len)
    timed_rows = [sum(min(c + warmup + k + 1, bench.max_seq) for c in cached) for k in range(steps)]
    eager_rows = bench.kv_rows[warmup:warmup + steps]
    kv_bytes = sum(eager_rows) * g.num_layers * g.kv_cols * 2 * kv_size
    qo_bytes = steps * g.num_layers * B * g.q_cols * 4 * 2
    attn_launches = n_t[0]
    attn_bytes_per_launch = (kv_bytes + qo_bytes) / max(attn_launches, 1)
    attn_ms_per_launch = ms_t[0] / max(attn_launches, 1)
    attn_gbs = attn_bytes_per_launch / (attn_ms_per_launch * 1e-3) / 1e9
    # the read ceiling of the same launch: a read-only copy of its page stream
    # (zr_kv_read_probe) over one eager step's work list, every layer, 3
    # launches each; its K/V bytes over its time against the kernel's
    ctx, lib = bench.ctx, bench.ctx.lib
    probe_ms = []
    for layer in range(g.num_layers):
        ms = C.c_double()
        ctx.check(lib.zr_kv_read_probe(ctx.h, bench.staged[warmup], layer, 3, C.byref(ms)))
        probe_ms.append(ms.value)
    probe_kv_bytes = bench.kv_rows[warmup] * g.kv_cols * 2 * kv_size
    probe_gbs = probe_kv_bytes / (np.mean(probe_ms) * 1e-3) / 1e9
    attn_kv_gbs = (kv_bytes / max(attn_launches, 1)) / (attn_ms_per_launch * 1e-3) / 1e9
    sb = np.mean([step_bytes(g, B, r, kv_size) for r in timed_rows])
    nb = BREAKDOWN_STEPS
    gemm_tflops = gemm_flops(g, B) * nb / (ms_b[1] * 1e-3) / 1e12 if ms_b[1] > 0 else 0.0
    roof_tps = B / (sb / (HBM_PEAK_GBS * 1e9))
    result = dict(
        workload=WORKLOADS[name]["desc"], batch=B, layers=g.num_layers,
        context_tokens=int(np.sum(bench.ctxlens)), context_max=int(np.max(bench.ctxlens)),
        tokens_per_s=B / (ms_per_step / 1e3), ms_per_step=ms_per_step,
        step_bytes=float(sb), step_roofline_tokens_per_s=roof_tps,
        step_roofline_frac=(B / (ms_per_step / 1e3)) / roof_tps,
        kernel_ms_per_step={"attention": ms_b[0] / nb, "gemm": ms_b[1] / nb, "norm_rope_kv": ms_b[2] / nb,
                            "other": ms_b[3] / nb},
        attention=dict(launches=attn_launches, bytes_per_launch=attn_bytes_per_launch,
                       avg_ms=attn_ms_per_launch, achieved_gbs=attn_gbs, frac=attn_gbs / HBM_PEAK_GBS,
                       read_ceiling=dict(entry="zr_kv_read_probe", gbs=probe_gbs, ms_per_launch=float(np.mean(probe_ms)),
                                         kv_bytes_per_launch=probe_kv_bytes, kernel_kv_gbs=attn_kv_gbs,
                                         frac=attn_kv_gbs / probe_gbs,
                                         note="K/V bytes per launch over the time of a read-only copy of the "
                                              "attention launch's page stream (same grid, work records and "
                                              "16-byte nontemporal page loads; no Q, softmax, MFMA or output)")),
        gemm=dict(launches=n_b[1] // nb, ms_per_step=ms_b[1] / nb, achieved_tflops=gemm_tflops,
                  frac=gemm_tflops / MFMA_BF16_PEAK_TFLOPS,
                  weight_gbs=(gemm_flops(g, B) / B) * nb / (ms_b[1] * 1e-3) / 1e9 if ms_b[1] > 0 else 0.0),
    )
    result["pipeline"] = dict(entry="zrh_decode_pipeline_step", steps=steps, captures=pinfo["captures"],
                              buckets=pinfo["buckets"], attention_items_capacity=pinfo["items_capacity"],
                              metadata_bytes_per_step=pinfo["metadata_bytes"],
                              includes="per step: host page tables and window trim, attention work list and "
                                       "metadata staged into pinned memory, its H2D copy on a copy stream, "
                                       "pack_kernel + rope_table_kernel and the forward pass replayed from the "
                                       "bucket's captured graph, greedy ids copied back and read by the host "
                                       "(one step behind)")
    result["eager"] = dict(entry="zr_forward_staged_async", steps=steps, ms_per_step=dt_eager / steps * 1e3,
                           tokens_per_s=B * steps / dt_eager,
                           includes="pre-staged steps launched kernel by kernel (metadata staged before the "
                                    "timing), HIP events around their attention launches")
    result["kv_append"] = measure_kv_append(bench, kv_size)
    # end to end through the boundary's synchronous host entry point
    # at least three warm-up calls: zr_forward replays a steady batch's greedy
    # steps from the third call on, so the graph capture stays out of the timing
    _, last = bench.run_host(max(warmup, 3), last)
    dt_host, last = bench.run_host(steps, last)
    assert last.max() < g.vocab
    result["host_path"] = dict(
        entry="zrh_decode_step_batch", steps=steps, ms_per_step=dt_host / steps * 1e3,
        tokens_per_s=B * steps / dt_host,
        includes="host page tables and window trim, metadata staged and copied up with the ids, pack_kernel + "
                 "rope_table_kernel and the forward pass (replayed from the context's step graph from the third "
                 "step of the same sequence count; the warm-up steps run eagerly and capture it), greedy token "
                 "D2H and the stream synchronisation, per step",
        replays=bench.ctx.forward_replay_info()["launches"])
    bench.close()
    return result


def measure_kv_append(bench, kv_size=2, reps=5):
    """RoPE + KV append (the RopeKvWrite stage; rope_kv_write_vec_kernel at 256 rows) alone:
    one launch over a decode step's rows (layer 0, the last staged step, after
    the timed region), HIP events of class 2.  (The 256-session forward pass
    runs this stage inside the attention launch; the separate kernel serves
    mixed microbatches and decode steps with short splits.)  Algorithmic bytes: the f32 QKV
    row read, the rotated f32 Q written, and the new K and V rows written into
    their bf16 pages."""
    ctx, lib, g = bench.ctx, bench.ctx.lib, bench.geo
    T = bench.B
    width = g.q_cols + 2 * g.kv_cols
    qkv = np.random.default_rng(3).standard_normal((T, width)).astype(np.float32)
    d_qkv, d_q = bench._dev(qkv.nbytes), bench._dev(4 * T * g.q_cols)
    ctx.check(lib.zr_memcpy_h2d(ctx.h, d_qkv, qkv.ctypes.data, qkv.nbytes))
    st = bench.staged[-1]
    ctx.check(lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv, d_q, 1))  # warm-up
    times = []
    for _ in range(reps):
        ctx.check(lib.zr_timing_begin(ctx.h, 1 << 2))
        ctx.check(lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv, d_q, 1))
        ms = (C.c_double * 5)()
        n = (C.c_int * 5)()
        ctx.check(lib.zr_timing_end(ctx.h, ms, n))
        times.append(ms[2])
    lib.zr_device_free(ctx.h, d_qkv)
    lib.zr_device_free(ctx.h, d_q)
    k_ms = float(np.median(times))
    alg = T * width * 4 + T * g.q_cols * 4 + T * 2 * g.kv_cols * kv_size
    return dict(kernel="rope_kv_write_vec_kernel" if T >= 128 else "rope_kv_write_kernel", rows=T, kernel_ms=k_ms, algorithmic_bytes=alg,
                achieved_gbs=alg / (k_ms * 1e6), frac=alg / (k_ms * 1e6) / HBM_PEAK_GBS,
                note="one launch is a few MB, so it is launch/latency-bound rather than HBM-bound")


# ------------------------------------------------------------- CPU baseline --
def _cpu_host():
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    model_name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model_name = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), model_name)
    except OSError:
        pass
    return dict(cores=threads, kind="port", cpu_model=model_name, affinity_cpus=len(os.sched_getaffinity(0)),
                nproc=os.cpu_count())


def _median_time(fn, reps, budget_s):
    """Runs fn up to `reps` times, stopping early once `budget_s` is spent
    (at least once); returns (median seconds, samples)."""
    ts, spent = [], 0.0
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        spent += ts[-1]
        if spent >= budget_s:
            break
    return float(np.median(ts)), ts


def _oracle_geometry(geo):
    H, nh, nkv = geo["hidden"], geo["num_heads"], geo["num_kv_heads"]
    d = H // nh
    s0, s1 = geo.get("shard_start", 0), geo.get("shard_end", H)
    Q = s1 - s0
    KV = (Q // ((nh // nkv) * d)) * d
    F = geo.get("ffn_cols", geo["ffn"])
    cfg = dict(hidden=H, num_heads=nh, num_kv_heads=nkv, vocab=geo["vocab"], ffn_cols=F, shard_start=s0,
               shard_end=s1, rms_norm_eps=1e-5, rope_base=geo["rope_base"])
    return cfg, Q, KV, F


def _oracle_model(O, geo, layers, rng):
    """The oracle's model of the workload's shape with `layers` layers; every
    layer references one set of f32 N(0, 0.02) matrices (the per-layer work is
    the same, the host memory that of one layer)."""
    cfg, Q, KV, F = _oracle_geometry(geo)
    H, V = geo["hidden"], geo["vocab"]
    block = rng.standard_normal(1 << 20, dtype=np.float32) * np.float32(0.02)

    def fill(shape):
        return np.resize(block, shape).astype(np.float32)

    lw = dict(w_q=fill((H, Q)), w_k=fill((H, KV)), w_v=fill((H, KV)), w_o=fill((Q, H)), w_gate=fill((H, F)),
              w_up=fill((H, F)), w_down=fill((F, H)), attn_norm=np.ones(H, np.float32), mlp_norm=np.ones(H, np.float32))
    return O.Model(dict(cfg, num_layers=layers), dict(embedding=fill((V, H)), final_norm=np.ones(H, np.float32),
                                                      lm_head=fill((H, V)), layers=[lw] * layers)), KV


def cpu_baseline(name, reps=3, budget_s=10.0, full_depth=False):
    """The oracle (C restatement of the CPU provider) on this host's cores: one
    decode microbatch of the workload's sessions and contexts (f32 weights and
    KV as the reference CPU provider).  full_depth: the whole model, median of
    `reps` runs.  Otherwise (the oracle's f32 KV of every layer would not fit
    in host memory at full depth) the same step with 1 and with 2 layers, each
    the median of `reps` runs, and step = T1 + (L - 1) (T2 - T1)."""
    import oracle as O

    w = WORKLOADS[name]
    geo = w["geo"]
    B, ctxlens, max_seq = w["batch"], w["contexts"](), w["max_seq_len"]
    rng = np.random.default_rng(0)
    L = geo["num_layers"]
    kv_rows = None

    def step_time(layers):
        nonlocal kv_rows
        m, KV = _oracle_model(O, geo, layers, rng)
        if kv_rows is None:
            kv_rows = np.resize(rng.standard_normal(1 << 20, dtype=np.float32), (int(ctxlens.max()), KV))
        sess = []
        for n in ctxlens:
            s = O.Session(layers, KV, 16, max_seq)
            s.append_all_layers(kv_rows[:n], kv_rows[:n])
            s.position = int(n)
            sess.append(s)
        toks = rng.integers(0, geo["vocab"], B).astype(np.uint32)
        # untimed: one session's step first (thread pool start, first touch of the weights)
        m.decode(sess[:1], toks[:1])
        # every run appends its row and advances the sessions: contexts grow by one row a run
        med, ts = _median_time(lambda: m.decode(sess, toks), reps, budget_s)
        del sess, m
        return med, ts

    out = _cpu_host()
    if full_depth:
        step_s, ts = step_time(L)
        sample = (f"oracle decode microbatch of the same {B} sessions and contexts through all {L} layers, median of "
                  f"{len(ts)} runs ({', '.join(f'{t:.2f}' for t in ts)} s) after an untimed one-session step")
    else:
        t1, ts1 = step_time(1)
        t2, ts2 = step_time(2)
        step_s = t1 + (L - 1) * max(t2 - t1, 1e-9)
        sample = (f"oracle decode microbatch of the same {B} sessions and contexts with 1 and 2 layers of the model, "
                  f"medians of {len(ts1)} / {len(ts2)} runs (T1 {t1:.2f} s, T2 {t2:.2f} s); step = T1 + {L - 1} x "
                  f"(T2 - T1) = {step_s:.2f} s, each after an untimed one-session step")
    out.update(value=B / step_s, unit="tokens/s", ms_per_step=step_s * 1e3,
               sample=sample + "; f32 weights / KV as the reference CPU provider")
    return out


def cpu_baseline_mixed(reps=3, budget_s=10.0):
    """The oracle on the mixed microbatch's work as the reference CPU provider
    does it (no ragged batching: each prefill chunk on its own, then the 60
    decode rows as one microbatch), from a bounded sample: one 512-row chunk
    (prefix 1000) and the 60 decode rows, each with 1 and with 2 layers
    (medians of `reps` runs); per layer = T2 - T1, and the microbatch =
    4 x (chunk T1 + 3 per-layer) + (decode T1 + 3 per-layer).  The chunks'
    prefixes (0 to 1531) change only their attention, ~5% of a chunk's
    per-layer work (the GEMMs of 512 rows are the rest)."""
    import oracle as O

    geo = MIXED_WORKLOAD["geo"]
    rng = np.random.default_rng(0xC3)
    dec = rng.integers(256, 4097, 60)
    V = geo["vocab"]
    chunk = rng.integers(0, V, 512).astype(np.uint32)
    dtoks = rng.integers(0, V, 60).astype(np.uint32)
    t = {}
    for layers in (1, 2):
        m, KV = _oracle_model(O, geo, layers, rng)
        rows = np.resize(rng.standard_normal(1 << 20, dtype=np.float32), (int(dec.max()), KV))
        warm = O.Session(layers, KV, 16, 8192)
        warm.append_all_layers(rows[:16], rows[:16])
        warm.position = 16
        m.decode([warm], dtoks[:1])  # untimed warm-up (thread pool start, first touch of the weights)
        tc, td = [], []
        for _ in range(reps):  # fresh sessions every run, built outside the timing
            s = O.Session(layers, KV, 16, 8192)
            s.append_all_layers(rows[:1000], rows[:1000])
            s.position = 1000
            de = []
            for n in dec:
                d = O.Session(layers, KV, 16, 8192)
                d.append_all_layers(rows[:n], rows[:n])
                d.position = int(n)
                de.append(d)
            t0 = time.perf_counter()
            m.prefill_chunk(s, chunk)
            t1 = time.perf_counter()
            m.decode(de, dtoks)
            t2 = time.perf_counter()
            tc.append(t1 - t0)
            td.append(t2 - t1)
            del s, de
            if sum(tc) + sum(td) >= budget_s:
                break
        t[layers] = (float(np.median(tc)), float(np.median(td)), len(tc))
        del m
    (c1, d1, n1), (c2, d2, n2) = t[1], t[2]
    total = 4 * (c1 + 3 * max(c2 - c1, 0.0)) + d1 + 3 * max(d2 - d1, 0.0)
    out = _cpu_host()
    out.update(value=2108 / total, unit="rows/s", ms_per_microbatch=total * 1e3,
               sample=f"oracle, bounded sample: one 512-row prefill chunk (prefix 1000) and the 60 decode rows, with "
                      f"1 and 2 layers, medians of {n1} / {n2} runs (chunk {c1:.2f} / {c2:.2f} s, decode {d1:.2f} / "
                      f"{d2:.2f} s); microbatch = 4 chunks x 4 layers + the decode rows x 4 layers = {total:.2f} s; "
                      f"f32 weights / KV as the reference CPU provider")
    return out


# pinned_windows: eviction buffers (2048-row windows, 0.54 GB each) pinned before the steps, about the
# number of sessions the 85% pool keeps evicted at a time
SOAK = dict(workload="llama3_8b_b256", pool_frac=0.85, join_rate=4.0, leave_prob=1 / 64, retention=2048,
            max_sessions=256, seed=0xC5, pinned_windows=40, prefetch=4)


def measure_soak(steps, warmup):
    """Decode steps of the Llama-3-8B-shape model under KV pressure: the page
    pool holds 85% of the 256 sessions' lognormal contexts; Poisson joins
    (4 per step), leaves (1/64 per session per step), eviction through the
    2048-token segmented-window export and restore through import
    (mesh_amd.kv_pressure).  A joining session's context pages are reserved
    and hold the pool's synthetic values (standing in for its prefill).
    value = decoded tokens / wall time of the steps, host path included, with
    the window copies overlapping the steps; `synchronous_copies` continues
    the same soak for as many steps with each copy made before the step."""
    from mesh_amd.kv_pressure import KvPressureSoak

    w = WORKLOADS[SOAK["workload"]]
    ctx, g = device_model(SOAK["workload"])
    ctxlens = w["contexts"]()
    need = int(sum((int(L) + 15) // 16 for L in ctxlens))
    pool = int(SOAK["pool_frac"] * need)
    ctx.create_kv_pool(pool)
    ctx.check(ctx.lib.zr_kv_pool_fill_normal(ctx.h, 4242, 1.0))

    def sample_len(rng):
        return int(np.clip(np.round(rng.lognormal(math.log(1024), 1.0)), 64, 8192))

    def admit(s, L, rng):
        s.backend.kv_reserve(L)
        return int(rng.integers(0, g.vocab))

    soak = KvPressureSoak(ctx, max_sessions=SOAK["max_sessions"], join_rate=SOAK["join_rate"],
                          leave_prob=SOAK["leave_prob"], retention=SOAK["retention"],
                          max_seq_len=w["max_seq_len"], context_sampler=sample_len, admit=admit, seed=SOAK["seed"],
                          prefetch=SOAK["prefetch"])
    soak.reserve_pinned(SOAK["pinned_windows"])
    for L in ctxlens:
        soak.add_session(int(L))
    for _ in range(warmup):
        soak.step()

    def timed():
        st0 = dict(vars(soak.stats))
        t0 = time.perf_counter()
        for _ in range(steps):
            soak.step()
        dt = time.perf_counter() - t0
        st = soak.stats
        d = lambda k: getattr(st, k) - st0[k]
        return dict(value=d("tokens") / dt, unit="tokens/s", steps=steps, mean_active=float(np.mean(st.active_hist[-steps:])),
                    joins=d("joins"), leaves=d("leaves"), evictions=d("evictions"), restores=d("restores"),
                    ms_per_step=dt / steps * 1e3, ms_per_step_decode=d("decode_s") / steps * 1e3,
                    ms_per_step_evict=d("evict_s") / steps * 1e3, ms_per_step_restore=d("restore_s") / steps * 1e3,
                    ms_per_step_admit=d("admit_s") / steps * 1e3)

    out = timed()
    out.update(pool_pages=pool, pool_frac_of_need=pool / need,
               transfers="each window's PCIe copy on a stream of its own while the steps run (evict: gather into a "
                         "device buffer, pages released at once, copy-out to pinned host memory; restore: the oldest "
                         "evicted windows uploaded a step ahead); the evict / restore times are the host time to "
                         "issue them",
               workload="Llama-3-8B-shape decode under KV pressure: pool 85% of 256 lognormal contexts, Poisson "
                        "joins 4/step, leave 1/64, evict/restore via 2048-token window export/import")
    # the same soak continued with the copies made synchronously, as the reference makes them
    soak.finish()
    soak.async_transfers = False
    out["synchronous_copies"] = timed()
    soak.finish()
    ctx.close()
    return out


def measure_kv_snapshot(reps=5):
    """KV snapshot wire bytes at the 256-session Llama-3-8B shape: one
    session's 2048-token eviction window (32 layers x 2048 rows x 1024 f32 per
    K and V) exported as KVCache::to_bytes (zrh_export_kv_cbor) into pinned
    host memory.  The encoder kernels are timed with HIP events (class 4);
    their algorithmic bytes are the f32 rows read once and the document
    written once.  The CPU leg is the oracle's encoder on the same rows."""
    from mesh_amd import DeviceContext, KVCacheSnapshot, ModelGeometry

    g = ModelGeometry(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=32, vocab=64, ffn=64)
    ctx = DeviceContext(g, kv_dtype="bf16", max_tokens=64, max_seqs=8, max_pages_per_seq=8192 // 16 + 2)
    rows, window = 3000, 2048
    ctx.create_kv_pool(rows // 16 + 8)
    rng = np.random.default_rng(0xC5)
    k = rng.standard_normal((32, rows, g.kv_cols), np.float32)
    v = rng.standard_normal((32, rows, g.kv_cols), np.float32)
    b = ctx.new_backend(8192)
    b.import_kv_cache(KVCacheSnapshot(rows, rows, k, v))
    del k, v
    lib = ctx.lib
    snap = b.export_kv_snapshot(window, pinned=True)  # warm-up (workspaces, staging)
    enc_ms, wall_ms = [], []
    for _ in range(reps):
        ctx.check(lib.zr_timing_begin(ctx.h, 1 << 4))
        t0 = time.perf_counter()
        snap = b.export_kv_snapshot(window, pinned=True)
        wall_ms.append((time.perf_counter() - t0) * 1e3)
        ms = (C.c_double * 5)()
        n = (C.c_int * 5)()
        ctx.check(lib.zr_timing_end(ctx.h, ms, n))
        enc_ms.append(ms[4])
    floats = 2 * 32 * window * g.kv_cols
    doc = snap.blob.size_bytes()
    alg = 4 * floats + doc
    enc = float(np.median(enc_ms))
    out = dict(workload="one session's 2048-token window, 32 layers x 1024 kv cols, bf16 pool -> f32 KVCache CBOR",
               floats=floats, document_bytes=doc, bytes_per_float=doc / floats,
               encode_ms=enc, export_ms=float(np.median(wall_ms)),
               roofline={"bound": "hbm", "kernel": "cbor_count_kernel + cbor_scan_groups_kernel + cbor_scan_top_kernel + cbor_write_kernel",
                         "achieved": alg / (enc * 1e6), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": alg / (enc * 1e6) / HBM_PEAK_GBS, "algorithmic_bytes": alg})
    # the gather and scatter kernels alone (kv_copy_kernel, HIP events of
    # timing class 3), device memory on both sides: the same window read from
    # the bf16 pages into f32 rows, and those rows written back (identical bytes)
    table = b.block_table()
    pages = np.ascontiguousarray([gp for _, _, _, gp in table], np.int32)
    fbytes = 32 * window * g.kv_cols * 4

    def dev(nbytes):
        ptr = C.c_void_p()
        ctx.check(lib.zr_device_alloc(ctx.h, int(nbytes), C.byref(ptr)))
        return ptr.value

    d_k, d_v = dev(fbytes), dev(fbytes)
    i32p = C.POINTER(C.c_int)
    targs = (ctx.h, pages.ctypes.data_as(i32p), int(pages.size), int(table[0][1]), rows - window, window)
    copy_ms = {}
    fk, fv = C.cast(d_k, C.POINTER(C.c_float)), C.cast(d_v, C.POINTER(C.c_float))
    for name, fn in (("gather", lib.zr_kv_gather), ("scatter", lib.zr_kv_scatter)):
        ctx.check(fn(*targs, fk, fv))
        ts = []
        for _ in range(reps):
            ctx.check(lib.zr_timing_begin(ctx.h, 1 << 3))
            ctx.check(fn(*targs, fk, fv))
            ms = (C.c_double * 5)()
            n = (C.c_int * 5)()
            ctx.check(lib.zr_timing_end(ctx.h, ms, n))
            ts.append(ms[3])
        copy_ms[name] = float(np.median(ts))
    lib.zr_device_free(ctx.h, d_k)
    lib.zr_device_free(ctx.h, d_v)
    cbytes = 2 * fbytes + 2 * 32 * window * g.kv_cols * 2  # f32 rows + bf16 pages, K and V
    out["kv_copy"] = {name: dict(kernel="kv_copy_kernel", ms=t, algorithmic_bytes=cbytes,
                                 achieved_gbs=cbytes / (t * 1e6), frac=cbytes / (t * 1e6) / HBM_PEAK_GBS)
                      for name, t in copy_ms.items()}
    ref = b.export_kv_cache(window)
    ctx.close()
    try:
        import oracle as O

        t0 = time.perf_counter()
        O.kv_cbor_encode(ref.keys, ref.values, rows - window, 32, 8, 128, 8192)
        cpu_s = time.perf_counter() - t0
        out["cpu_baseline"] = dict(value=doc / cpu_s / 1e6, unit="MB/s of document", cores=1, kind="port",
                                   sample="the same document (oracle/kv_cbor.c, one thread)")
    except Exception as e:  # the oracle is test infrastructure; its absence only drops this leg
        out["cpu_baseline"] = {"error": str(e)}
    return out


def measure_sampling(reps=5):
    """Device sampling of the decode batch's logits at the 256-session
    Llama-3-8B shape: 256 rows x 128256 f32 logits already in HBM, sampled by
    zr_sample as sample_tokens_device_with_seeds (runtime.rs:534-601) with
    per-row seeds, in the three modes the path has: greedy (T = 0), full
    distribution (T = 0.7, top_p = 1) and nucleus (T = 0.7, top_p = 0.9).
    sample_kernel is timed with HIP events (class 3); its algorithmic bytes
    are the logits read once and one token written per row.  The CPU leg is
    the oracle's f64 restatement on a bounded sample of rows."""
    from mesh_amd import DeviceBuffer, DeviceContext, ModelGeometry

    rows, vocab = 256, 128256
    g = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=2, num_layers=1, vocab=vocab, ffn=64)
    ctx = DeviceContext(g, kv_dtype="f32", max_tokens=8, max_seqs=8, max_pages_per_seq=8)
    rng = np.random.default_rng(0x5A)
    x = (rng.standard_normal((rows, vocab)) * 3).astype(np.float32)
    d_x = DeviceBuffer.from_numpy(ctx, x)
    d_out = DeviceBuffer(ctx, 4 * rows)
    seeds = rng.integers(0, 2 ** 63, rows, dtype=np.uint64)
    lib = ctx.lib
    f32p, u64p = C.POINTER(C.c_float), C.POINTER(C.c_uint64)
    alg = rows * vocab * 4 + rows * 4
    modes = {}
    for name, t, p in (("greedy", 0.0, 1.0), ("full", 0.7, 1.0), ("nucleus", 0.7, 0.9)):
        temps = np.full(rows, t, np.float32)
        tops = np.full(rows, p, np.float32)
        args = (ctx.h, d_x.ptr, rows, vocab, temps.ctypes.data_as(f32p), tops.ctypes.data_as(f32p),
                seeds.ctypes.data_as(u64p), d_out.ptr)
        ctx.check(lib.zr_sample(*args))  # warm-up
        times = []
        for _ in range(reps):
            ctx.check(lib.zr_timing_begin(ctx.h, 1 << 3))
            ctx.check(lib.zr_sample(*args))
            ms = (C.c_double * 5)()
            n = (C.c_int * 5)()
            ctx.check(lib.zr_timing_end(ctx.h, ms, n))
            times.append(ms[3])
        k_ms = float(np.median(times))
        modes[name] = dict(kernel_ms=k_ms, achieved=alg / (k_ms * 1e6), frac=alg / (k_ms * 1e6) / HBM_PEAK_GBS)
    d_x.free()
    d_out.free()
    ctx.close()
    nuc = modes["nucleus"]
    out = dict(workload="256 rows x 128256 f32 logits (one decode step of 256 sessions), per-row seeds",
               modes=modes,
               roofline={"bound": "hbm", "kernel": "sample_kernel (nucleus)", "achieved": nuc["achieved"],
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": nuc["frac"], "algorithmic_bytes": alg})
    try:
        import oracle as O

        sample = 8
        t0 = time.perf_counter()
        for r in range(sample):
            O.sample_token_device(x[r], 0.7, 0.9, int(seeds[r]))
        cpu_s = time.perf_counter() - t0
        out["cpu_baseline"] = dict(value=sample / cpu_s, unit="rows/s (nucleus)", cores=1, kind="port",
                                   sample=f"{sample} rows of the same logits (oracle, f64, one thread)")
    except Exception as e:  # the oracle is test infrastructure; its absence only drops this leg
        out["cpu_baseline"] = {"error": str(e)}
    return out


MIXED_WORKLOAD = dict(
    geo=dict(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=4, vocab=128256, ffn=14336, rope_base=500000.0),
    batch=64, max_seq_len=8192, contexts=None,
    desc="Mixed chunked-prefill + decode microbatch at the Llama-3-8B layer shape, 4 layers: 4 prefill chunks "
         "of 512 rows (prefixes 0, 512, 1000, 1531) + 60 decode sessions (contexts U[256, 4096]) packed into "
         "2108 varlen rows, page 16 from a seeded permutation of the pool, bf16 weights + bf16 KV")


def measure_mixed(reps=5):
    """The MFMA-bound configuration: one mixed microbatch of 2108 rows through
    4 Llama-3-8B-shape layers (QKV / O / gate-up / down GEMMs at M = 2108, LM
    head on the 64 last rows).  Every timed microbatch runs on its own set of
    64 sessions, so each has exactly this shape (the chunks' prefixes do not
    grow).  Reported: rows/s, the per-class kernel split (HIP events, a second
    pass over the same staged microbatches), and the GEMMs' algorithmic
    TFLOP/s against the 2.5 PFLOP/s dense bf16 peak (executed MFMA work is
    2x: hi + lo activations)."""
    from mesh_amd import _lib

    WORKLOADS["llama3_layers4_mixed"] = MIXED_WORKLOAD
    sets = reps + 1
    ctx, g = device_model("llama3_layers4_mixed", True, max_tokens=4 * 512 + 60, max_seqs=64)
    lib = ctx.lib
    rng = np.random.default_rng(0xC3)
    prefixes = [0, 512, 1000, 1531]
    dec = rng.integers(256, 4097, 60)
    per_set = int(sum((p + 512 + 15) // 16 + 1 for p in prefixes) + sum((int(L) + 1 + 15) // 16 + 1 for L in dec))
    n_pages = per_set * sets
    ctx.create_kv_pool(n_pages, rng.permutation(n_pages))
    ctx.check(lib.zr_kv_pool_fill_normal(ctx.h, 4242, 1.0))
    q_len = np.array([512] * 4 + [1] * 60, np.int32)
    rows = int(q_len.sum())
    staged, keep = [], []
    for _ in range(sets):
        bks = [ctx.new_backend(8192) for _ in range(64)]
        for b, L in zip(bks, prefixes + [int(x) for x in dec]):
            if L:
                b.kv_reserve(int(L))
        arr = (C.c_void_p * 64)(*[b.h for b in bks])
        st = C.c_void_p()
        ctx.check(lib.zrh_stage_mixed(C.cast(arr, C.POINTER(C.c_void_p)), 64, q_len.ctypes.data_as(_lib.c_int_p),
                                      None, C.byref(st)))
        staged.append(st.value)
        keep.append((bks, arr))

    def dev(nbytes):
        ptr = C.c_void_p()
        ctx.check(lib.zr_device_alloc(ctx.h, int(nbytes), C.byref(ptr)))
        return ptr.value

    tok, out = dev(4 * rows), dev(4 * 64)
    t = rng.integers(0, g.vocab, rows).astype(np.uint32)
    ctx.check(lib.zr_memcpy_h2d(ctx.h, tok, t.ctypes.data, t.nbytes))

    def run(idx, mask):
        if mask:
            ctx.check(lib.zr_timing_begin(ctx.h, mask))
        ctx.check(lib.zr_synchronize(ctx.h))
        t0 = time.perf_counter()
        for i in idx:
            ctx.check(lib.zr_forward_staged_async(ctx.h, staged[i], tok, out, None))
        ctx.check(lib.zr_synchronize(ctx.h))
        dt = time.perf_counter() - t0
        ms = (C.c_double * 5)()
        n = (C.c_int * 5)()
        if mask:
            ctx.check(lib.zr_timing_end(ctx.h, ms, n))
        return dt, list(ms)

    run([0], 0)
    dt, _ = run(range(1, sets), 0)
    _, ms = run(range(1, sets), 0xF)
    toks = np.zeros(64, np.uint32)
    ctx.check(lib.zr_memcpy_d2h(ctx.h, toks.ctypes.data, out, toks.nbytes))
    assert toks.max() < g.vocab
    for st in staged:
        lib.zr_staged_destroy(st)
    ctx.close()
    H, Q, KV, F, V, L = g.hidden, g.q_cols, g.kv_cols, g.ffn_cols, g.vocab, g.num_layers
    flops = 2.0 * rows * L * (H * (Q + 2 * KV) + Q * H + H * 2 * F + F * H) + 2.0 * 64 * H * V
    gemm_ms = ms[1] / reps
    tflops = flops / (gemm_ms * 1e-3) / 1e12
    return dict(workload=MIXED_WORKLOAD["desc"], rows=rows, value=rows * reps / dt, unit="rows/s",
                ms_per_microbatch=dt / reps * 1e3,
                kernel_ms_per_microbatch={"attention": ms[0] / reps, "gemm": gemm_ms,
                                          "norm_rope_kv": ms[2] / reps, "other": ms[3] / reps},
                gemm_mfma={"achieved": tflops, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": tflops / MFMA_BF16_PEAK_TFLOPS, "mfma_ops_per_flop": 2,
                           "executed_frac": 2 * tflops / MFMA_BF16_PEAK_TFLOPS, "flops_per_microbatch": flops})


def calibrate_copy():
    """One plain device-to-device copy of 1 GiB (torch), the reference point
    for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = 1 << 28
    a = torch.ones(n, device="cuda", dtype=torch.float32)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n * 4}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-bs32", action="store_true")
    ap.add_argument("--workload", default="llama3_8b_b256", choices=sorted(WORKLOADS))
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--skip-soak", action="store_true", help="skip the KV-pressure soak leg")
    ap.add_argument("--skip-kv-snapshot", action="store_true", help="skip the KV snapshot wire-format leg")
    ap.add_argument("--skip-sampling", action="store_true", help="skip the device sampling leg")
    ap.add_argument("--skip-mixed", action="store_true", help="skip the mixed prefill + decode microbatch leg")
    ap.add_argument("--skip-tp-shard", action="store_true", help="skip the tensor-parallel shard decode leg")
    ap.add_argument("--skip-f32-kv", action="store_true", help="skip the headline step with an f32 KV pool")
    ap.add_argument("--mixed-only", action="store_true",
                    help="run only the mixed prefill + decode microbatch leg (for profiling its kernels)")
    a = ap.parse_args()
    if a.calibrate_copy:
        calibrate_copy()
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this provider runs one worker's shard on one GPU; --gpus must be 1 "
                                   "(sharding across GPUs is described, not implemented)"}))
        sys.exit(2)
    from mesh_amd import probe_provider

    ok, err = probe_provider(0)
    if not ok:
        raise SystemExit(f"rocm provider unavailable: {err}")
    if a.mixed_only:
        print(json.dumps({"mixed_prefill": measure_mixed(max(1, a.steps))}))
        return
    main_r = measure(a.workload, a.steps, a.warmup)
    bs32 = None
    if not a.skip_bs32 and a.workload != "tinyllama_b32":
        r = measure("tinyllama_b32", a.steps, a.warmup)
        bs32 = dict(value=r["tokens_per_s"], unit="tokens/s", ms_per_step=r["ms_per_step"],
                    workload=r["workload"], step_roofline_frac=r["step_roofline_frac"],
                    attention_gbs=r["attention"]["achieved_gbs"],
                    attention_read_ceiling=r["attention"]["read_ceiling"], kernel_ms_per_step=r["kernel_ms_per_step"],
                    gemm_tflops=r["gemm"]["achieved_tflops"], gemm_weight_gbs=r["gemm"]["weight_gbs"],
                    host_path=r["host_path"], eager=r["eager"], pipeline=r["pipeline"])
    tp_shard = None
    if not a.skip_tp_shard and a.workload != "llama3_8b_tp2_b64":
        r = measure("llama3_8b_tp2_b64", max(4, a.steps // 2), 2)
        tp_shard = dict(value=r["tokens_per_s"], unit="tokens/s (one shard's step)", ms_per_step=r["ms_per_step"],
                        workload=r["workload"], step_roofline_frac=r["step_roofline_frac"],
                        attention_gbs=r["attention"]["achieved_gbs"],
                    attention_read_ceiling=r["attention"]["read_ceiling"], kernel_ms_per_step=r["kernel_ms_per_step"],
                        gemm_tflops=r["gemm"]["achieved_tflops"], gemm_weight_gbs=r["gemm"]["weight_gbs"],
                        host_path=r["host_path"])
    f32_kv = None
    if not a.skip_f32_kv and a.workload == "llama3_8b_b256":
        r = measure(a.workload, max(4, a.steps // 2), 2, kv_dtype="f32")
        att32 = r["attention"]
        f32_kv = dict(value=r["tokens_per_s"], unit="tokens/s", ms_per_step=r["ms_per_step"],
                      workload=r["workload"].replace("bf16 KV", "f32 KV (the reference's page dtype)"),
                      step_roofline_frac=r["step_roofline_frac"],
                      step_roofline_tokens_per_s=r["step_roofline_tokens_per_s"],
                      kernel_ms_per_step=r["kernel_ms_per_step"], host_path=r["host_path"], eager=r["eager"],
                      roofline={"bound": "hbm", "kernel": "paged_attention_kernel<float>",
                                "achieved": att32["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": att32["frac"], "bytes_per_launch": att32["bytes_per_launch"],
                                "avg_ms": att32["avg_ms"], "launches": att32["launches"], "sizeof_kv": 4,
                                "read_ceiling_gbs": att32["read_ceiling"]["gbs"],
                                "frac_of_read_ceiling": att32["read_ceiling"]["frac"]})
    soak = None if a.skip_soak else measure_soak(max(4, a.steps // 2), 2)
    kv_snapshot = None if a.skip_kv_snapshot else measure_kv_snapshot()
    sampling = None if a.skip_sampling else measure_sampling()
    mixed = None if a.skip_mixed else measure_mixed()
    cpu = None if a.skip_cpu else cpu_baseline(a.workload)
    if not a.skip_cpu and a.workload == "llama3_8b_b256":
        # the other configurations' CPU figures, beside their GPU legs
        if bs32 is not None:
            bs32["cpu_baseline"] = cpu_baseline("tinyllama_b32", full_depth=True)
        if tp_shard is not None:
            tp_shard["cpu_baseline"] = cpu_baseline("llama3_8b_tp2_b64")
        if mixed is not None:
            mixed["cpu_baseline"] = cpu_baseline_mixed()
    att = main_r["attention"]
    line = {
        "metric": METRIC, "value": main_r["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": main_r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: random-init bf16 N(0,0.02) weights, KV pages filled with N(0,1) bf16 as prefill "
                "output, greedy tokens fed back on the device",
        "config": {"workload": main_r["workload"], "sessions": main_r["batch"], "layers": main_r["layers"],
                   "context_tokens": main_r["context_tokens"], "context_max": main_r["context_max"],
                   "parallelism": "one worker shard (1 of 1) on one GPU",
                   "step_launch": "serving loop: each step staged (host page tables, metadata H2D) and "
                                  "replayed from the bucket's captured step graph, ids copied back "
                                  "(zrh_decode_pipeline_step); kernel-by-kernel launch of pre-staged steps "
                                  "under eager",
                   "gemm_a_operand": "bf16 hi + lo pair (activation = hi + lo to 2^-16), fp32 accumulation"},
        "roofline": {"bound": "hbm", "kernel": "paged_attention_kernel", "achieved": att["achieved_gbs"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": att["frac"], "traffic": measured_traffic(),
                     "bytes_per_launch": att["bytes_per_launch"], "avg_ms": att["avg_ms"],
                     "launches": att["launches"], "read_ceiling_gbs": att["read_ceiling"]["gbs"],
                     "frac_of_read_ceiling": att["read_ceiling"]["frac"]},
        "step_roofline": {"tokens_per_s": main_r["step_roofline_tokens_per_s"], "frac": main_r["step_roofline_frac"],
                          "bytes_per_step": main_r["step_bytes"]},
        "kernel_ms_per_step": main_r["kernel_ms_per_step"],
        "pipeline": main_r["pipeline"],
        "host_path": main_r["host_path"],
        "eager": main_r["eager"],
        "kv_append": main_r["kv_append"],
        "gemm_mfma": {"achieved": main_r["gemm"]["achieved_tflops"], "peak": MFMA_BF16_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": main_r["gemm"]["frac"], "mfma_ops_per_flop": 2,
                      "weight_stream_gbs": main_r["gemm"]["weight_gbs"]},
        "bs32": bs32,
        "tp_shard": tp_shard,
        "f32_kv": f32_kv,
        "soak": soak,
        "kv_snapshot": kv_snapshot,
        "sampling": sampling,
        "mixed_prefill": mixed,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
