"""Op-level parity of the HIP kernels against the oracle, through the C-ABI.

Tolerances (from the provider's contract): packing, page tables, KV appends
and gathers, greedy ids are bit-exact; attention outputs within 2e-3 relative
(per head: max|got - want| <= 2e-3 * max|want|); GEMM / norm within the stated
float bounds below.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as O
from mesh_amd import DeviceBuffer, DeviceContext, ModelGeometry, _lib
from tests.gpu_util import f32p, i32p, max_rel_err_rows, stage_mixed, u32p

pytestmark = pytest.mark.gpu

ATTN_RTOL = 2e-3


def tiny_llama_attn_ctx(kv_dtype, n_pages=512, order=None, layers=1):
    # TinyLlama-1.1B attention shape: 32 q heads, 4 kv heads, head_dim 64
    geo = ModelGeometry(hidden=2048, num_heads=32, num_kv_heads=4, num_layers=layers, vocab=64, ffn=64)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=256, max_seqs=64, max_pages_per_seq=128)
    ctx.create_kv_pool(n_pages, order)
    return ctx, geo


# --------------------------------------------------------------- packing --
def test_pack_matches_oracle_bit_exact():
    ctx, geo = tiny_llama_attn_ctx("f32", n_pages=10000)
    rng = np.random.default_rng(5)
    n = 37
    q_len = rng.integers(1, 4, n).astype(np.int32)
    kv_before = rng.integers(0, 300, n).astype(np.int32)
    first_off = rng.integers(0, 16, n).astype(np.int32)
    first_pos = (kv_before + rng.integers(0, 1000, n)).astype(np.int32)
    pages = (first_off + kv_before + q_len + 15) // 16
    stride = int(pages.max())
    bt = np.zeros((n, stride), np.int32)
    perm = rng.permutation(10000)
    used = 0
    for s in range(n):
        bt[s, :pages[s]] = perm[used:used + pages[s]]
        used += pages[s]
    total = int(q_len.sum())
    mb = _lib.Microbatch(n, i32p(q_len), i32p(kv_before), i32p(first_pos), i32p(first_off), i32p(bt), stride, None)
    cu_q = np.zeros(n + 1, np.int32)
    cu_k = np.zeros(n + 1, np.int32)
    pos = np.zeros(total, np.int32)
    slot = np.zeros(total, np.int32)
    seq = np.zeros(total, np.int32)
    ctx.check(ctx.lib.zr_pack(ctx.h, C.byref(mb), i32p(cu_q), i32p(cu_k), i32p(pos), i32p(slot), i32p(seq)))
    w = O.pack(q_len, kv_before, first_pos, first_off, bt)
    for got, want in zip((cu_q, cu_k, pos, slot, seq), w):
        np.testing.assert_array_equal(got, want)
    ctx.close()


def test_stage_rejects_pages_outside_pool():
    ctx, geo = tiny_llama_attn_ctx("f32", n_pages=8)
    one = np.ones(1, np.int32)
    zero = np.zeros(1, np.int32)
    bt = np.array([[9]], np.int32)
    mb = _lib.Microbatch(1, i32p(one), i32p(zero), i32p(zero), i32p(zero), i32p(bt), 1, None)
    st = C.c_void_p()
    rc = ctx.lib.zr_stage(ctx.h, C.byref(mb), C.byref(st))
    assert rc == -4 and b"outside pool" in ctx.lib.zr_last_error(ctx.h)
    ctx.close()


# ------------------------------------------------------------------ RoPE --
@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,D,base", [(32, 4, 64, 1e4), (32, 8, 128, 5e5)])
def test_rope_kv_write_rotates_q_and_k_at_large_positions(kv_dtype, heads, kv_heads, D, base):
    """RoPE + KV append (the RopeKvWrite stage) with the rotation on, against
    the oracle's apply_rope (tensor_ops.rs:509-560) and the fp64 closed form,
    at positions 0, 1, 517, 4095 and 8191.  Both sides form theta = f32(pos) *
    inv_freq[i] in f32 from the same host powf table (runtime.rs:282-301), so
    only the cos / sin rounding differs from the oracle: 2e-5 of the row's
    scale.  Against fp64 the f32 theta itself moves by up to pos * 2^-24 rad
    (the position-scaled bound).  The rotated K rows are read back from their
    pages, V rows must be copied bit for bit."""
    positions = [0, 1, 517, 4095, 8191]
    Q, KV = heads * D, kv_heads * D
    geo = ModelGeometry(hidden=Q, num_heads=heads, num_kv_heads=kv_heads, num_layers=1, vocab=64, ffn=64,
                        rope_base=base)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=16, max_seqs=8, max_pages_per_seq=8)
    ctx.create_kv_pool(64)
    rng = np.random.default_rng(D)
    backends = []
    for p in positions:
        b = ctx.new_backend(8192 + 16)
        if p:  # a short window ending at position p - 1: the new row lands at p
            rows = min(p, 5)
            k = rng.standard_normal((1, rows, KV), dtype=np.float32)
            from mesh_amd import KVCacheSnapshot

            b.import_kv_cache(KVCacheSnapshot(p, rows, k, k.copy()))
        backends.append(b)
    st = stage_mixed(ctx, backends, [1] * len(positions))
    qkv = rng.standard_normal((len(positions), Q + 2 * KV), dtype=np.float32)
    d_qkv = DeviceBuffer.from_numpy(ctx, qkv)
    d_q = DeviceBuffer(ctx, 4 * len(positions) * Q)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 1))
    q_dev = d_q.download(np.float32, (len(positions), Q))
    ctx.lib.zr_staged_destroy(st)
    pos = np.asarray(positions, np.uint32)
    want_q = O.apply_rope(qkv[:, :Q], pos, D, base)
    want_k = O.apply_rope(qkv[:, Q:Q + KV], pos, D, base)
    k_dev = np.stack([b.export_kv_cache().keys[0, -1] for b in backends])
    v_dev = np.stack([b.export_kv_cache().values[0, -1] for b in backends])
    np.testing.assert_array_equal(q_dev[0], qkv[0, :Q])  # position 0 is the identity
    for r in range(len(positions)):
        scale = float(np.abs(qkv[r]).max())
        assert np.max(np.abs(q_dev[r] - want_q[r])) <= 2e-5 * scale, (positions[r], "q")
        if kv_dtype == "f32":
            assert np.max(np.abs(k_dev[r] - want_k[r])) <= 2e-5 * scale, (positions[r], "k")
            np.testing.assert_array_equal(v_dev[r], qkv[r, Q + KV:])
        else:  # the pool rounds to bf16: within one bf16 step (2^-7 relative) of the oracle's rounded row
            wk = O.round_bf16(want_k[r])
            assert np.all(np.abs(k_dev[r] - wk) <= 2.0 ** -7 * np.abs(wk) + 2e-5 * scale), (positions[r], "k")
            np.testing.assert_array_equal(v_dev[r], O.round_bf16(qkv[r, Q + KV:]))
        # the fp64 closed form, rotate-half pairing per head
        half = D // 2
        inv = 1.0 / (np.float64(base) ** (np.arange(half) * 2.0 / D))
        th = positions[r] * inv
        for h in range(heads):
            a = qkv[r, h * D:h * D + half].astype(np.float64)
            bb = qkv[r, h * D + half:(h + 1) * D].astype(np.float64)
            ref = np.concatenate([a * np.cos(th) - bb * np.sin(th), a * np.sin(th) + bb * np.cos(th)])
            bound = (3e-6 + 4e-7 * positions[r] * 8) * scale
            assert np.max(np.abs(q_dev[r, h * D:(h + 1) * D] - ref)) <= bound, (positions[r], h)
    ctx.close()


@pytest.mark.parametrize("rope", [0, 1])
@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,D,base", [(32, 4, 64, 1e4), (32, 8, 128, 5e5)])
@pytest.mark.parametrize("pages_per_split", [2, 9])
def test_rope_attention_equals_rope_kv_write_then_attention_bit_exact(monkeypatch, rope, kv_dtype, heads, kv_heads,
                                                                      D, base, pages_per_split):
    """RoPE + KV append inside the decode attention launch (zr_rope_attention,
    the forward pass's path for one-row decode microbatches) against the two
    stages run apart (zr_rope_kv_write, then zr_attention) on identically
    prepared sessions: the attention outputs and every KV row, the appended
    one included, bit for bit.  Splits of 2 pages give most tiles several
    splits (the last one appends the row) and the 1-row context a single
    one; positions run to ~5600.  Splits of 9 pages give last splits of 2 to
    9 pages: those of more than 4 issue their first pages before the append
    (which cannot touch them), the others after it."""
    from mesh_amd import KVCacheSnapshot

    monkeypatch.setenv("ZR_ATTN_PAGES_PER_SPLIT", str(pages_per_split))
    Q, KV = heads * D, kv_heads * D
    geo = ModelGeometry(hidden=Q, num_heads=heads, num_kv_heads=kv_heads, num_layers=1, vocab=64, ffn=64,
                        rope_base=base)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=16, max_seqs=16, max_pages_per_seq=64)
    ctx.create_kv_pool(600)
    rng = np.random.default_rng(D + rope)
    ctxlens = [0, 1, 15, 16, 17, 200, 431, 599]
    sets = [[ctx.new_backend(8192) for _ in ctxlens] for _ in range(2)]
    for i, L in enumerate(ctxlens):
        if L:
            k = rng.standard_normal((1, L, KV), dtype=np.float32)
            v = rng.standard_normal((1, L, KV), dtype=np.float32)
            for bs in sets:
                bs[i].import_kv_cache(KVCacheSnapshot(5000 + L, L, k, v))
    qkv = rng.standard_normal((len(ctxlens), Q + 2 * KV), dtype=np.float32)
    d_qkv = DeviceBuffer.from_numpy(ctx, qkv)
    d_q = DeviceBuffer(ctx, 4 * len(ctxlens) * Q)
    d_a, d_b = DeviceBuffer(ctx, 4 * len(ctxlens) * Q), DeviceBuffer(ctx, 4 * len(ctxlens) * Q)
    st_a, st_b = stage_mixed(ctx, sets[0], [1] * len(ctxlens)), stage_mixed(ctx, sets[1], [1] * len(ctxlens))
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st_a, 0, d_qkv.ptr, d_q.ptr, rope))
    ctx.check(ctx.lib.zr_attention(ctx.h, st_a, 0, d_q.ptr, d_a.ptr))
    ctx.check(ctx.lib.zr_rope_attention(ctx.h, st_b, 0, d_qkv.ptr, d_b.ptr, rope))
    ctx.lib.zr_staged_destroy(st_a)
    ctx.lib.zr_staged_destroy(st_b)
    out_a, out_b = d_a.download(np.float32, (len(ctxlens), Q)), d_b.download(np.float32, (len(ctxlens), Q))
    assert np.isfinite(out_a).all()
    np.testing.assert_array_equal(out_b, out_a)
    for i, L in enumerate(ctxlens):
        ka, kb = sets[0][i].export_kv_cache(), sets[1][i].export_kv_cache()
        assert ka.cached_tokens == kb.cached_tokens == L + 1
        np.testing.assert_array_equal(kb.keys, ka.keys)
        np.testing.assert_array_equal(kb.values, ka.values)
    # a microbatch with a two-row sequence is not a decode microbatch
    st = stage_mixed(ctx, [ctx.new_backend(64), ctx.new_backend(64)], [1, 2])
    assert ctx.lib.zr_rope_attention(ctx.h, st, 0, d_qkv.ptr, d_b.ptr, rope) == -5
    assert b"one-row decode" in ctx.lib.zr_last_error(ctx.h)
    ctx.lib.zr_staged_destroy(st)
    ctx.close()


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,D,base", [(32, 4, 64, 1e4), (32, 8, 128, 5e5)])
def test_rope_kv_write_float4_path_matches_scalar_path_bit_exact(kv_dtype, heads, kv_heads, D, base):
    """From 128 rows the stage runs its float4 kernel, which must reproduce the
    scalar kernel bit for bit (same angles, same slab order).  The same 160 rows
    (4 sessions x 40, positions from 1000 k + 7) run as one launch and as two
    80-row launches on identically prepared sessions: q and the appended K / V
    rows must be equal, and q within the oracle's RoPE bound."""
    from mesh_amd import KVCacheSnapshot

    Q, KV = heads * D, kv_heads * D
    geo = ModelGeometry(hidden=Q, num_heads=heads, num_kv_heads=kv_heads, num_layers=1, vocab=64, ffn=64,
                        rope_base=base)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=256, max_seqs=8, max_pages_per_seq=64)
    ctx.create_kv_pool(256)
    rng = np.random.default_rng(D + 1)
    rows, prefix = 40, [1000 * k + 7 for k in range(4)]
    qkv = rng.standard_normal((4 * rows, Q + 2 * KV), dtype=np.float32)

    def prepared():
        out = []
        for p in prefix:  # a 3-row window ending at position p - 1: the new rows land at p ..
            b = ctx.new_backend(8192)
            k = rng.standard_normal((1, 3, KV), dtype=np.float32)
            b.import_kv_cache(KVCacheSnapshot(p, 3, k, k.copy()))
            out.append(b)
        return out

    def run(backends, qkv_rows):
        st = stage_mixed(ctx, backends, [rows] * len(backends))
        d_qkv = DeviceBuffer.from_numpy(ctx, qkv_rows)
        d_q = DeviceBuffer(ctx, 4 * qkv_rows.shape[0] * Q)
        ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 1))
        ctx.lib.zr_staged_destroy(st)
        return d_q.download(np.float32, (qkv_rows.shape[0], Q))

    one = prepared()
    q_vec = run(one, qkv)
    two = prepared()
    q_scalar = np.concatenate([run(two[:2], qkv[:2 * rows]), run(two[2:], qkv[2 * rows:])])
    np.testing.assert_array_equal(q_vec, q_scalar)
    for b1, b2 in zip(one, two):
        s1, s2 = b1.export_kv_cache(), b2.export_kv_cache()
        assert s1.next_position == s2.next_position and s1.cached_tokens == 3 + rows
        np.testing.assert_array_equal(s1.keys[:, -rows:], s2.keys[:, -rows:])
        np.testing.assert_array_equal(s1.values[:, -rows:], s2.values[:, -rows:])
    pos = np.concatenate([np.arange(p, p + rows) for p in prefix]).astype(np.uint32)
    want_q = O.apply_rope(qkv[:, :Q], pos, D, base)
    scale = np.abs(qkv).max(1, keepdims=True)
    assert np.all(np.abs(q_vec - want_q) <= 2e-5 * scale)
    ctx.close()


# ------------------------------------------------ C1: attention + append --
def c1_inputs(seed=0xC1):
    rng = np.random.default_rng(seed)
    B = 8
    ctxlens = rng.integers(16, 513, B)
    order = rng.permutation(512)
    Q = rng.standard_normal((B, 32 * 64), dtype=np.float32)
    K = [rng.standard_normal((L, 256), dtype=np.float32) for L in ctxlens]
    V = [rng.standard_normal((L, 256), dtype=np.float32) for L in ctxlens]
    return B, ctxlens, order, Q, K, V


def run_c1(kv_dtype):
    B, ctxlens, order, Q, K, V = c1_inputs()
    ctx, geo = tiny_llama_attn_ctx(kv_dtype, 512, order)
    backends = [ctx.new_backend() for _ in range(B)]
    # prefix rows (L - 1) scattered into the permuted pool
    for b, L, k, v in zip(backends, ctxlens, K, V):
        if L > 1:
            b.import_kv_cache(_snapshot(k[:-1], v[:-1]))
    st = stage_mixed(ctx, backends, [1] * B)
    qkv = np.concatenate([Q, np.stack([k[-1] for k in K]), np.stack([v[-1] for v in V])], 1)
    d_qkv = DeviceBuffer.from_numpy(ctx, qkv)
    d_q = DeviceBuffer(ctx, Q.nbytes)
    d_o = DeviceBuffer(ctx, Q.nbytes)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 0))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, Q.shape)
    ctx.lib.zr_staged_destroy(st)
    return ctx, backends, (B, ctxlens, order, Q, K, V), out


def _snapshot(k, v):
    from mesh_amd import KVCacheSnapshot

    return KVCacheSnapshot(next_position=k.shape[0], cached_tokens=k.shape[0], keys=k[None], values=v[None])


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_kv_read_probe_times_the_decode_page_stream(kv_dtype):
    """zr_kv_read_probe (a diagnostic with no reference counterpart) launches
    a read-only copy of the decode attention launch's page stream: it returns
    a positive mean time, refuses out-of-range arguments, and leaves the pool
    as it was."""
    B, ctxlens, order, Q, K, V = c1_inputs()
    ctx, geo = tiny_llama_attn_ctx(kv_dtype, 512, order)
    backends = [ctx.new_backend() for _ in range(B)]
    for b, L, k, v in zip(backends, ctxlens, K, V):
        if L > 1:
            b.import_kv_cache(_snapshot(k[:-1], v[:-1]))
    st = stage_mixed(ctx, backends, [1] * B)  # (staging reserves each session's decode row)
    before = [b.export_kv_cache() for b in backends]
    ms = C.c_double()
    ctx.check(ctx.lib.zr_kv_read_probe(ctx.h, st, 0, 5, C.byref(ms)))
    assert 0.0 < ms.value < 100.0
    assert ctx.lib.zr_kv_read_probe(ctx.h, st, 1, 5, C.byref(ms)) == _lib.ZR_E_INVALID  # one layer
    assert ctx.lib.zr_kv_read_probe(ctx.h, st, 0, 0, C.byref(ms)) == _lib.ZR_E_INVALID
    assert ctx.lib.zr_kv_read_probe(ctx.h, st, 0, 5, None) == _lib.ZR_E_INVALID
    ctx.lib.zr_staged_destroy(st)
    for b, snap in zip(backends, before):
        after = b.export_kv_cache()
        np.testing.assert_array_equal(after.keys, snap.keys)
        np.testing.assert_array_equal(after.values, snap.values)
    ctx.close()


def test_op_entries_refuse_a_microbatch_staged_by_another_context():
    """A staged microbatch indexes its own context's pool and workspaces: the
    op-level entries refuse one staged by another context (ZR_E_INVALID)
    before launching anything."""
    B, ctxlens, order, Q, K, V = c1_inputs()
    ctx_a, _ = tiny_llama_attn_ctx("bf16", 512, order)
    ctx_b, _ = tiny_llama_attn_ctx("bf16", 512, order)
    backends = [ctx_a.new_backend() for _ in range(2)]
    st = stage_mixed(ctx_a, backends, [1, 1])
    d_qkv = DeviceBuffer(ctx_b, 4 * 2 * 2560)
    d_out = DeviceBuffer(ctx_b, 4 * 2 * 2048)
    ms = C.c_double()
    lib = ctx_b.lib
    assert lib.zr_attention(ctx_b.h, st, 0, d_qkv.ptr, d_out.ptr) == _lib.ZR_E_INVALID
    assert lib.zr_rope_kv_write(ctx_b.h, st, 0, d_qkv.ptr, d_out.ptr, 1) == _lib.ZR_E_INVALID
    assert lib.zr_rope_attention(ctx_b.h, st, 0, d_qkv.ptr, d_out.ptr, 1) == _lib.ZR_E_INVALID
    assert lib.zr_kv_read_probe(ctx_b.h, st, 0, 1, C.byref(ms)) == _lib.ZR_E_INVALID
    ctx_a.lib.zr_staged_destroy(st)
    ctx_b.close()
    ctx_a.close()


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_c1_paged_gqa_decode_attention_and_append(kv_dtype):
    ctx, backends, (B, ctxlens, order, Q, K, V), out = run_c1(kv_dtype)
    bf = kv_dtype == "bf16"
    for s in range(B):
        o = O.Session(1, 256, 16, 4096, kv_round_bf16=bf)
        o.append_layer(0, K[s], V[s])
        ok, ov = o.gather(0)
        # the appended row and every page: bit-exact against the oracle's cache
        snap = backends[s].export_kv_cache()
        assert snap.cached_tokens == ctxlens[s]
        np.testing.assert_array_equal(snap.keys[0], ok)
        np.testing.assert_array_equal(snap.values[0], ov)
        # attention per q head (GQA: q head h reads kv head h // 8)
        want = np.zeros(32 * 64, np.float32)
        for h in range(32):
            kvh = h // 8
            want[h * 64:(h + 1) * 64] = O.causal_attention_with_prefix(
                Q[s, h * 64:(h + 1) * 64][None], ok[:, kvh * 64:(kvh + 1) * 64], ov[:, kvh * 64:(kvh + 1) * 64],
                1 / math.sqrt(64), ctxlens[s] - 1)[0]
        err = max_rel_err_rows(out[s], want, 64)
        assert err <= ATTN_RTOL, (s, err)
    # page tables: session-local ids are the reference's sequential ids; the
    # global pages are exactly the first pops of the seeded permutation (LIFO)
    used = []
    for b in backends:
        table = b.block_table()
        assert [p for p, _, _, _ in table] == list(range(len(table)))
        used += [g for _, _, _, g in table]
    assert sorted(used) == sorted(int(x) for x in order[::-1][:len(used)])
    ctx.close()


@pytest.mark.parametrize("pages_per_split", [1, 3])
def test_c1_decode_attention_merges_many_splits(monkeypatch, pages_per_split):
    """Decode tiles split every 1 or 3 pages (ZR_ATTN_PAGES_PER_SPLIT): up to
    32 splits per tile at 512 keys, so the merge runs both its one-round-trip
    form (at most 16 splits) and its general form (more), against the
    oracle's attention over the same pages."""
    monkeypatch.setenv("ZR_ATTN_PAGES_PER_SPLIT", str(pages_per_split))
    ctx, backends, (B, ctxlens, order, Q, K, V), out = run_c1("bf16")
    pages = (ctxlens + 15) // 16
    assert pages_per_split > 1 or (pages.max() > 16 and pages.min() <= 16)  # both merge forms
    for s in range(B):
        o = O.Session(1, 256, 16, 4096, kv_round_bf16=True)
        o.append_layer(0, K[s], V[s])
        ok, ov = o.gather(0)
        want = np.zeros(32 * 64, np.float32)
        for h in range(32):
            kvh = h // 8
            want[h * 64:(h + 1) * 64] = O.causal_attention_with_prefix(
                Q[s, h * 64:(h + 1) * 64][None], ok[:, kvh * 64:(kvh + 1) * 64], ov[:, kvh * 64:(kvh + 1) * 64],
                1 / math.sqrt(64), ctxlens[s] - 1)[0]
        err = max_rel_err_rows(out[s], want, 64)
        assert err <= ATTN_RTOL, (s, err)
    ctx.close()


def _attend(kv_dtype, prefixes, new_rows, q_len=None):
    """TinyLlama attention shape (32 q heads, 4 kv heads, D 64): session s
    imports prefixes[s] = (K, V) rows, stages q_len[s] rows (default 1) whose
    q / K / V come from new_rows[s] ([q_len, 2048 + 512]), appends them
    (rope off) and attends.  Returns the f32 output [rows, 2048]."""
    B = len(prefixes)
    q_len = [1] * B if q_len is None else q_len
    ctx, _ = tiny_llama_attn_ctx(kv_dtype, 512)
    backends = [ctx.new_backend() for _ in range(B)]
    for b, (k, v) in zip(backends, prefixes):
        if k.shape[0]:
            b.import_kv_cache(_snapshot(k, v))
    st = stage_mixed(ctx, backends, q_len)
    qkv = np.ascontiguousarray(np.concatenate(new_rows, 0), np.float32)
    d_qkv = DeviceBuffer.from_numpy(ctx, qkv)
    d_q = DeviceBuffer(ctx, 4 * qkv.shape[0] * 2048)
    d_o = DeviceBuffer(ctx, 4 * qkv.shape[0] * 2048)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 0))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, (qkv.shape[0], 2048))
    ctx.lib.zr_staged_destroy(st)
    ctx.close()
    return out


def _kv_as_stored(x, kv_dtype):
    return O.round_bf16(x) if kv_dtype == "bf16" else x


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_attention_single_key_returns_its_value(kv_dtype):
    """Closed form: a query that sees one key gets that key's value row
    (softmax weight 1).  Decode rows of sessions with no prefix, and with a
    bf16 pool also the first row of a 16-row prefill chunk (the prefill
    kernel: row 0 sees key 0 only).  bf16 pool: exact; f32 pool (V split into
    bf16 hi + lo inside the MFMA): within 1e-5."""
    rng = np.random.default_rng(0x51)
    B = 6
    rows = [rng.standard_normal((1, 2560), dtype=np.float32) for _ in range(B)]
    empty = (np.zeros((0, 256), np.float32), np.zeros((0, 256), np.float32))
    out = _attend(kv_dtype, [empty] * B, rows)
    for s in range(B):
        v = _kv_as_stored(rows[s][0, 2304:], kv_dtype)
        want = np.concatenate([v[(h // 8) * 64:(h // 8 + 1) * 64] for h in range(32)])
        if kv_dtype == "bf16":
            np.testing.assert_array_equal(out[s], want)
        else:
            np.testing.assert_allclose(out[s], want, rtol=1e-5, atol=1e-6)
    if kv_dtype == "bf16":
        chunk = rng.standard_normal((16, 2560), dtype=np.float32)
        out = _attend(kv_dtype, [empty], [chunk], q_len=[16])
        v = _kv_as_stored(chunk[0, 2304:], kv_dtype)
        want = np.concatenate([v[(h // 8) * 64:(h // 8 + 1) * 64] for h in range(32)])
        np.testing.assert_array_equal(out[0], want)


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_attention_identical_keys_average_the_values(kv_dtype):
    """Closed form: when every visible key is the same vector, every score is
    the same and the output is the plain mean of the visible values.  Windows
    of 1..400 keys (one page to several splits, a partial last page)."""
    rng = np.random.default_rng(0x52)
    lens = [1, 15, 16, 17, 129, 400]
    prefixes, rows, want = [], [], []
    for L in lens:
        k = rng.standard_normal(256, dtype=np.float32)
        V = rng.standard_normal((L, 256), dtype=np.float32)
        prefixes.append((np.tile(k, (L - 1, 1)), V[:-1]))
        row = np.concatenate([rng.standard_normal(2048, dtype=np.float32), k, V[-1]])[None]
        rows.append(row)
        m = _kv_as_stored(V, kv_dtype).astype(np.float64).mean(0)
        want.append(np.concatenate([m[(h // 8) * 64:(h // 8 + 1) * 64] for h in range(32)]))
    out = _attend(kv_dtype, prefixes, rows)
    for s, L in enumerate(lens):
        np.testing.assert_allclose(out[s], want[s], rtol=1e-5, atol=1e-5, err_msg=f"L={L}")


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_attention_dominant_key_selects_its_value(kv_dtype):
    """Closed form at saturation: one key scores ~100 (natural log units)
    above every other visible key, so its softmax weight is 1 to within
    e^-90 and the output is its value row.  The dominant key sits at the
    window's start, middle or end, across several splits."""
    rng = np.random.default_rng(0x53)
    L = 300
    prefixes, rows, want = [], [], []
    for pos in (0, 151, L - 1):
        q = rng.standard_normal(2048, dtype=np.float32)
        K = 0.1 * rng.standard_normal((L, 256), dtype=np.float32)
        V = rng.standard_normal((L, 256), dtype=np.float32)
        for kvh in range(4):  # key `pos` of kv head kvh: 100 sqrt(d) / |q_h|^2 q_h of its first q head
            qh = q[kvh * 8 * 64:(kvh * 8 + 1) * 64]
            K[pos, kvh * 64:(kvh + 1) * 64] = 100.0 * 8.0 * qh / float(qh @ qh)
        q = q.copy()
        for h in range(32):  # every q head of a kv head asks the same question
            q[h * 64:(h + 1) * 64] = q[(h // 8) * 8 * 64:((h // 8) * 8 + 1) * 64]
        prefixes.append((K[:-1], V[:-1]))
        rows.append(np.concatenate([q, K[-1], V[-1]])[None])
        v = _kv_as_stored(V[pos], kv_dtype)
        want.append(np.concatenate([v[(h // 8) * 64:(h // 8 + 1) * 64] for h in range(32)]))
    out = _attend(kv_dtype, prefixes, rows)
    assert np.isfinite(out).all()
    for s in range(3):
        np.testing.assert_allclose(out[s], want[s], rtol=1e-5, atol=1e-6)


def _f32_page_order(e):
    """f32 pools: each 512-element block (64 lanes x 8) holds lane l's
    elements 0-3 at 4 l and 4-7 at 256 + 4 l."""
    w = e & 511
    return (e & ~511) | ((w & 4) << 6) | ((w >> 3) << 2) | (w & 3)


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_c1_raw_page_row_holds_appended_kv_in_pool_layout(kv_dtype):
    """The appended row sits in its page at the documented offsets: K element
    (t, d) at ((d/8)·16 + t)·8 + d%8, V element at ((((d/32)·4 + t/4)·16 +
    d%16)·2 + (d/16)%2)·4 + t%4 of its kv head's tile, f32 pools with each
    512-element block in the half-major order of _f32_page_order."""
    ctx, backends, (B, ctxlens, order, Q, K, V), out = run_c1(kv_dtype)
    s = 3
    table = backends[s].block_table()
    last = table[-1]
    row = (last[1] + last[2] - 1)  # row of the newest token inside its page
    f32 = kv_dtype == "f32"
    page = np.zeros(2 * 256 * 16, np.float32 if f32 else np.uint16)
    pages = np.array([last[3]], np.int32)
    ctx.check(ctx.lib.zr_kv_read_pages(ctx.h, 0, i32p(pages), 1, page.ctypes.data))
    if not f32:  # bf16 bits -> f32
        page = (page.astype(np.uint32) << 16).view(np.float32)
    order_of = _f32_page_order if f32 else (lambda e: e)
    want_k = K[s][-1] if f32 else O.round_bf16(K[s][-1])
    want_v = V[s][-1] if f32 else O.round_bf16(V[s][-1])
    kblk, vblk = page[:4096].reshape(4, 16 * 64), page[4096:].reshape(4, 16 * 64)
    for h in range(4):
        for d in range(64):
            assert kblk[h][order_of(((d // 8) * 16 + row) * 8 + d % 8)] == want_k[h * 64 + d]
            v_off = ((((d // 32) * 4 + row // 4) * 16 + d % 16) * 2 + (d // 16) % 2) * 4 + row % 4
            assert vblk[h][order_of(v_off)] == want_v[h * 64 + d]
    ctx.close()


@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_chunked_prefill_attention_causal_with_prefix(kv_dtype):
    """Masked multi-query attention with a cached prefix (forward_pass.rs:2764-2836):
    chunk rows see keys [0, prefix + r]; a page-unaligned prefix is included."""
    ctx, geo = tiny_llama_attn_ctx(kv_dtype, 4096)
    rng = np.random.default_rng(11)
    prefixes, chunks = [0, 37, 512, 1000], [5, 40, 33, 16]
    backends = [ctx.new_backend() for _ in prefixes]
    Ks, Vs = [], []
    for b, p, c in zip(backends, prefixes, chunks):
        k = rng.standard_normal((p + c, 256), dtype=np.float32)
        v = rng.standard_normal((p + c, 256), dtype=np.float32)
        Ks.append(k)
        Vs.append(v)
        if p:
            b.import_kv_cache(_snapshot(k[:p], v[:p]))
    T = sum(chunks)
    Q = rng.standard_normal((T, 2048), dtype=np.float32)
    newk = np.concatenate([k[p:] for k, p in zip(Ks, prefixes)])
    newv = np.concatenate([v[p:] for v, p in zip(Vs, prefixes)])
    st = stage_mixed(ctx, backends, chunks)
    d_qkv = DeviceBuffer.from_numpy(ctx, np.concatenate([Q, newk, newv], 1))
    d_q = DeviceBuffer(ctx, Q.nbytes)
    d_o = DeviceBuffer(ctx, Q.nbytes)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 0))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, Q.shape)
    ctx.lib.zr_staged_destroy(st)
    row = 0
    for s, (p, c) in enumerate(zip(prefixes, chunks)):
        k, v = Ks[s], Vs[s]
        if kv_dtype == "bf16":
            k, v = O.round_bf16(k), O.round_bf16(v)
        for h in range(32):
            kvh = h // 8
            want = O.causal_attention_with_prefix(Q[row:row + c, h * 64:(h + 1) * 64], k[:, kvh * 64:(kvh + 1) * 64],
                                                  v[:, kvh * 64:(kvh + 1) * 64], 1 / math.sqrt(64), p)
            err = max_rel_err_rows(out[row:row + c, h * 64:(h + 1) * 64], want, 64)
            assert err <= ATTN_RTOL, (s, h, err)
        row += c
    ctx.close()


@pytest.mark.parametrize("key_halves", ["1", "2"])
def test_prefill_blocks_llama3_heads_trimmed_windows_and_decode_rows(monkeypatch, key_halves):
    """Chunked-prefill attention at Llama-3 heads (32 q / 8 kv, head_dim 128,
    bf16 pool): chunks of 512, 100, 33 and 32 rows (whole and partial 32-row
    query blocks) against prefixes of 0, 1531, 700 and 40 rows, where the
    700-row window was trimmed by retain_suffix so its first page starts at
    row 9; two decode rows (one also trimmed) share the microbatch.  Both
    workgroup forms: 4 waves over every key tile, and 8 waves as two halves
    over alternate tiles whose (m, l, O) meet in LDS (odd tile counts leave
    the second half's last step empty)."""
    monkeypatch.setenv("ZR_ATTN_PREFILL_KEY_HALVES", key_halves)
    geo = ModelGeometry(hidden=4096, num_heads=32, num_kv_heads=8, num_layers=1, vocab=64, ffn=64)
    ctx = DeviceContext(geo, kv_dtype="bf16", max_tokens=1024, max_seqs=8, max_pages_per_seq=160)
    ctx.create_kv_pool(1024)
    rng = np.random.default_rng(12)
    cases = [(0, 512, 0), (1531, 100, 0), (700, 33, 57), (40, 32, 0), (300, 1, 0), (77, 1, 25)]  # (window, chunk, trimmed)
    backends, Ks, Vs = [], [], []
    for p, c, trim in cases:
        b = ctx.new_backend(max_seq_len=4096)
        k = rng.standard_normal((trim + p + c, 1024), dtype=np.float32)
        v = rng.standard_normal((trim + p + c, 1024), dtype=np.float32)
        if trim + p:
            b.import_kv_cache(_snapshot(k[:trim + p], v[:trim + p]))
        if trim:
            b.retain_suffix(p)
            assert b.block_table()[0][1] == trim % 16
        backends.append(b)
        Ks.append(k)
        Vs.append(v)
    chunks = [c for _, c, _ in cases]
    T = sum(chunks)
    Q = rng.standard_normal((T, 4096), dtype=np.float32)
    newk = np.concatenate([k[t + p:] for k, (p, _, t) in zip(Ks, cases)])
    newv = np.concatenate([v[t + p:] for v, (p, _, t) in zip(Vs, cases)])
    st = stage_mixed(ctx, backends, chunks)
    d_qkv = DeviceBuffer.from_numpy(ctx, np.concatenate([Q, newk, newv], 1))
    d_q = DeviceBuffer(ctx, Q.nbytes)
    d_o = DeviceBuffer(ctx, Q.nbytes)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 0))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, Q.shape)
    ctx.lib.zr_staged_destroy(st)
    row = 0
    for s, (p, c, trim) in enumerate(cases):
        k, v = O.round_bf16(Ks[s][trim:]), O.round_bf16(Vs[s][trim:])
        for h in range(32):
            kvh = h // 4
            want = O.causal_attention_with_prefix(Q[row:row + c, h * 128:(h + 1) * 128],
                                                  k[:, kvh * 128:(kvh + 1) * 128], v[:, kvh * 128:(kvh + 1) * 128],
                                                  1 / math.sqrt(128), p)
            err = max_rel_err_rows(out[row:row + c, h * 128:(h + 1) * 128], want, 128)
            assert err <= ATTN_RTOL, (s, h, err)
        row += c
    ctx.close()


@pytest.mark.parametrize("key_halves,tiles_per_split", [("1", "2"), ("2", "2"), ("2", "3")])
@pytest.mark.parametrize("heads,kv_heads,D", [(8, 8, 64), (8, 4, 128), (32, 8, 128), (16, 2, 64), (16, 1, 64),
                                           (16, 1, 128)])
def test_prefill_blocks_gqa_groups_with_forced_splits(monkeypatch, heads, kv_heads, D, key_halves, tiles_per_split):
    """The prefill kernel at G = 1, 2, 4, 8 and 16 (blocks of 128, 64, 32, 16
    and 8 rows; merge groups of 16, 8, 4, 2 and 1 rows), with its key splits forced to
    2 or 3 tiles (ZR_ATTN_PREFILL_TILES_PER_SPLIT) so every block of these
    chunks goes through the partials and the merge, in both workgroup forms
    (ZR_ATTN_PREFILL_KEY_HALVES; with two halves, splits of one or three tiles
    leave the second half an empty step).  The page-unaligned prefix puts the
    causal edge inside waves: a split can start past some rows' last visible
    key while the wave's other rows see keys in it (those columns must keep a
    zero weight, not NaN)."""
    monkeypatch.setenv("ZR_ATTN_PREFILL_TILES_PER_SPLIT", tiles_per_split)
    monkeypatch.setenv("ZR_ATTN_PREFILL_KEY_HALVES", key_halves)
    G = heads // kv_heads
    prows = 128 // G
    q_cols, kv_cols = heads * D, kv_heads * D
    geo = ModelGeometry(hidden=q_cols, num_heads=heads, num_kv_heads=kv_heads, num_layers=1, vocab=64, ffn=64)
    ctx = DeviceContext(geo, kv_dtype="bf16", max_tokens=512, max_seqs=4, max_pages_per_seq=64)
    ctx.create_kv_pool(256)
    rng = np.random.default_rng(G)
    prefixes, chunks = [0, 203], [prows + 5, 2 * prows]
    backends, Ks, Vs = [ctx.new_backend() for _ in prefixes], [], []
    for b, p, c in zip(backends, prefixes, chunks):
        k = rng.standard_normal((p + c, kv_cols), dtype=np.float32)
        v = rng.standard_normal((p + c, kv_cols), dtype=np.float32)
        Ks.append(k)
        Vs.append(v)
        if p:
            b.import_kv_cache(_snapshot(k[:p], v[:p]))
    T = sum(chunks)
    Q = rng.standard_normal((T, q_cols), dtype=np.float32)
    newk = np.concatenate([k[p:] for k, p in zip(Ks, prefixes)])
    newv = np.concatenate([v[p:] for v, p in zip(Vs, prefixes)])
    st = stage_mixed(ctx, backends, chunks)
    d_qkv = DeviceBuffer.from_numpy(ctx, np.concatenate([Q, newk, newv], 1))
    d_q = DeviceBuffer(ctx, Q.nbytes)
    d_o = DeviceBuffer(ctx, Q.nbytes)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 0))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, Q.shape)
    ctx.lib.zr_staged_destroy(st)
    row = 0
    for s, (p, c) in enumerate(zip(prefixes, chunks)):
        k, v = O.round_bf16(Ks[s]), O.round_bf16(Vs[s])
        for h in range(heads):
            kvh = h // G
            want = O.causal_attention_with_prefix(Q[row:row + c, h * D:(h + 1) * D], k[:, kvh * D:(kvh + 1) * D],
                                                  v[:, kvh * D:(kvh + 1) * D], 1 / math.sqrt(D), p)
            err = max_rel_err_rows(out[row:row + c, h * D:(h + 1) * D], want, D)
            assert err <= ATTN_RTOL, (s, h, err)
        row += c
    ctx.close()


# ------------------------------------------------------- gather / scatter --
@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
def test_kv_gather_scatter_round_trip_with_partial_first_page(kv_dtype):
    ctx, geo = tiny_llama_attn_ctx(kv_dtype, 256, layers=3)
    rng = np.random.default_rng(2)
    b = ctx.new_backend(max_seq_len=4096)
    k = rng.standard_normal((3, 50, 256), dtype=np.float32)
    v = rng.standard_normal((3, 50, 256), dtype=np.float32)
    if kv_dtype == "bf16":
        k, v = O.round_bf16(k), O.round_bf16(v)
    from mesh_amd import KVCacheSnapshot

    b.import_kv_cache(KVCacheSnapshot(50, 50, k, v))
    b.retain_suffix(37)  # first span now starts at row 13
    assert b.block_table()[0][1] == 13
    full = b.export_kv_cache()
    np.testing.assert_array_equal(full.keys, k[:, 13:])
    np.testing.assert_array_equal(full.values, v[:, 13:])
    seg = b.export_kv_cache(max_cached_tokens=20)  # segmented retention window
    assert seg.cached_tokens == 20 and seg.next_position == 50 and seg.first_cached_position() == 30
    np.testing.assert_array_equal(seg.keys, k[:, 30:])
    # import into a fresh session on other pages: identical bytes back
    b2 = ctx.new_backend(max_seq_len=4096)
    b2.import_kv_cache(seg)
    back = b2.export_kv_cache()
    np.testing.assert_array_equal(back.keys, seg.keys)
    np.testing.assert_array_equal(back.values, seg.values)
    assert b2.sequence_position() == 50 and b2.base_position() == 30
    ctx.close()


# -------------------------------------------------------------- GEMM etc --
@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("m,k,n", [(1, 64, 100), (7, 256, 4112), (32, 2048, 2048), (100, 512, 1000),
                                   (256, 4096, 1024), (300, 128, 64), (128, 4104, 4112), (130, 520, 66000),
                                   # more 128 x 256 tiles than CUs: K split 3 and 4 ways to fill the last pass
                                   (2108, 4096, 4096), (2108, 14336, 4096),
                                   # the 256-row decode products (QKV, O, down) and a head over
                                   # 16-wave 256 x 256 tiles
                                   (256, 4096, 6144), (256, 4096, 4096), (256, 14336, 4096), (200, 4096, 66000),
                                   # the 32-session TinyLlama products: QKV (11 splits), down (16), an
                                   # unsplit vocabulary head
                                   (32, 2048, 2560), (32, 5632, 2048), (32, 2048, 32000),
                                   # 33-64 rows on 64-row tiles (a 4-deep ring, one pass of splits): the
                                   # 64-session shard's QKV, O and down products, and a ragged one
                                   (64, 4096, 3072), (64, 2048, 4096), (64, 7168, 4096), (40, 512, 1000)])
def test_gemm_matches_fp64(split, m, k, n):
    geo = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=4, num_layers=1, vocab=64, ffn=256)
    ctx = DeviceContext(geo, kv_dtype="f32", max_tokens=16, max_seqs=4, max_pages_per_seq=4, split_activations=split)
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    w = O.round_bf16(rng.standard_normal((k, n), dtype=np.float32) * 0.02)
    d_a = DeviceBuffer.from_numpy(ctx, a)
    d_c = DeviceBuffer(ctx, m * n * 4)
    from mesh_amd import bf16_bits

    wb = bf16_bits(w)
    ctx.check(ctx.lib.zr_gemm(ctx.h, d_a.ptr, wb.ctypes.data, d_c.ptr, m, n, k))
    got = d_c.download(np.float32, (m, n))
    ref = a.astype(np.float64) @ w.astype(np.float64)
    scale = np.sqrt(k) * 0.02  # typical |c| magnitude
    # hi+lo activations: ~2^-16 relative per product; bf16 activations: ~2^-8
    tol = 2e-5 * scale if split else 1.5e-2 * scale
    assert np.max(np.abs(got - ref)) <= tol, np.max(np.abs(got - ref)) / scale
    ctx.close()


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("m,k,f", [(40, 320, 512),       # <= 64 rows, K = 10 steps: split-K slabs, the reduce
                                   (40, 512, 512), (33, 256, 96),  # 33-64 rows: K over 4 waves, two row tiles
                                   (64, 4096, 7168),     # the tensor-parallel shard's gate / up at 64 sessions
                                   (32, 2048, 5632),     # the 32-session TinyLlama gate / up: K over 4 waves
                                   (1, 128, 64), (7, 256, 96),  # <= 32 rows, K over 4 waves of 1 / 2 steps
                                   (5, 96, 64),          # K = 3 steps: split-K slabs and the reduce
                                   (100, 256, 512),      # 65-128 rows: fused, 64 x 256 tiles
                                   (130, 200, 96),       # fused, 128 x 256 tiles, K padded to 224
                                   (256, 4096, 14336),   # the Llama-3-8B gate / up product of the decode step
                                   (2108, 1024, 2048)])  # prefill-sized: fused 128 x 512 tiles
def test_gemm_swiglu_matches_fp64(split, m, k, f):
    # h = silu(A @ Wg) * (A @ Wu) (tensor_ops.rs:268-278, forward_pass.rs:2286-2289)
    geo = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=4, num_layers=1, vocab=64, ffn=256)
    ctx = DeviceContext(geo, kv_dtype="f32", max_tokens=16, max_seqs=4, max_pages_per_seq=4, split_activations=split)
    rng = np.random.default_rng(m + k + f)
    a = rng.standard_normal((m, k), dtype=np.float32)
    wg = O.round_bf16(rng.standard_normal((k, f), dtype=np.float32) * 0.02)
    wu = O.round_bf16(rng.standard_normal((k, f), dtype=np.float32) * 0.02)
    from mesh_amd import bf16_bits

    d_a, d_h = DeviceBuffer.from_numpy(ctx, a), DeviceBuffer(ctx, m * f * 4)
    wgb, wub = bf16_bits(wg), bf16_bits(wu)  # held until the call returns
    ctx.check(ctx.lib.zr_gemm_swiglu(ctx.h, d_a.ptr, wgb.ctypes.data, wub.ctypes.data, d_h.ptr, m, f, k))
    got = d_h.download(np.float32, (m, f))
    a64 = a.astype(np.float64)
    g, u = a64 @ wg.astype(np.float64), a64 @ wu.astype(np.float64)
    ref = g / (1.0 + np.exp(-g)) * u
    scale = np.sqrt(k) * 0.02  # typical |g|, |u|
    # g and u carry the product's error (the bar of test_gemm_matches_fp64:
    # 2e-5 scale with hi+lo activations, 1.5e-2 scale with bf16 ones), which
    # silu(g) * u scales by |silu'(g)| <= 1.1 and |u|, |silu(g)| <= |g|; h
    # is stored as hi + lo (2^-16 relative) or bf16 (2^-8)
    eps, rel = (2e-5, 2.0 ** -15) if split else (1.5e-2, 2.0 ** -8)
    bound = eps * scale * (1.1 * np.abs(u) + np.abs(g) + scale) + rel * np.abs(ref)
    excess = np.abs(got - ref) - bound
    assert excess.max() <= 0, (excess.max(), np.abs(got - ref).max())
    ctx.close()


@pytest.mark.parametrize("rows,cols", [(37, 4096), (200, 4096), (3, 2050), (5, 8192), (130, 64)])
def test_rms_norm_matches_oracle(rows, cols):
    geo = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=4, num_layers=1, vocab=64, ffn=256)
    ctx = DeviceContext(geo, kv_dtype="f32", max_tokens=16, max_seqs=4, max_pages_per_seq=4)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((rows, cols), dtype=np.float32) * 3
    g = rng.standard_normal(cols, dtype=np.float32)
    d_x, d_g, d_y = DeviceBuffer.from_numpy(ctx, x), DeviceBuffer.from_numpy(ctx, g), DeviceBuffer(ctx, x.nbytes)
    ctx.check(ctx.lib.zr_rms_norm(ctx.h, d_x.ptr, d_g.ptr, d_y.ptr, rows, cols))
    np.testing.assert_allclose(d_y.download(np.float32, x.shape), O.rms_norm(x, g, 1e-5), rtol=2e-6, atol=2e-6)
    ctx.close()


def test_argmax_first_index_on_ties_and_large_vocab():
    geo = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=4, num_layers=1, vocab=64, ffn=256)
    ctx = DeviceContext(geo, kv_dtype="f32", max_tokens=16, max_seqs=4, max_pages_per_seq=4)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 128256), dtype=np.float32)
    x[0, :4] = [1.0, 5.0, 2.0, 3.0]  # tensor_ops.rs:633-639 -> 1
    x[0, 4:] = -10
    x[1, 70000] = x[1, 3] = x[1, 100000] = 99.0  # ties -> lowest index
    x[2] = -np.inf
    x[3, 128255] = 50.0
    d_x, d_o = DeviceBuffer.from_numpy(ctx, x), DeviceBuffer(ctx, 6 * 4)
    ctx.check(ctx.lib.zr_argmax(ctx.h, d_x.ptr, 6, 128256, d_o.ptr))
    got = d_o.download(np.uint32, 6)
    want = [O.sample_greedy(r) for r in x]
    assert got.tolist() == want
    assert got[:4].tolist() == [1, 3, 0, 128255]
    ctx.close()


# -------------------------------- the benchmarked launch: 256 sessions --
@pytest.mark.parametrize("kv_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rope", [0, 1])
def test_c5_shape_attention_256_sessions_matches_oracle(rope, kv_dtype):
    # The attention launch of the 256-session decode benchmark: Llama-3-8B
    # attention shape (32 q heads, 8 kv heads, head_dim 128), the benchmark's
    # lognormal contexts (seed 0xC5: median 1024, sigma 1, clipped to
    # [64, 8192]; sum ~395k keys) with the launch's own split sizing (~96
    # pages per split, so long sessions merge several splits).  All 32 heads
    # of a sample of sessions (the longest, the shortest and six more) are
    # checked against the oracle; every output must be finite.  The bf16 pool
    # is the benchmark's; the f32 pool is the reference's own KV precision
    # (forward_pass.rs:255-262), checked against unrounded K / V.
    ctxlens = np.clip(np.round(np.random.default_rng(0xC5).lognormal(math.log(1024), 1.0, 256)), 64,
                      8192).astype(np.int64)
    B, H, KVC, D = 256, 4096, 1024, 128
    geo = ModelGeometry(hidden=H, num_heads=32, num_kv_heads=8, num_layers=1, vocab=64, ffn=64, rope_base=500000.0)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=B, max_seqs=B, max_pages_per_seq=520)
    ctx.create_kv_pool(int(((ctxlens + 15) // 16).sum()) + B)
    rng = np.random.default_rng(0xA5)
    rows = 1 << 16
    big = rng.standard_normal((rows, KVC), dtype=np.float32)  # K / V rows: per-session windows of one array
    koff = [(s * 7919) % (rows - 8192) for s in range(B)]
    voff = [(s * 104729 + 12345) % (rows - 8192) for s in range(B)]
    backends = [ctx.new_backend(8320) for _ in range(B)]
    for s, b in enumerate(backends):
        L = int(ctxlens[s])
        b.import_kv_cache(_snapshot(big[koff[s]:koff[s] + L - 1], big[voff[s]:voff[s] + L - 1]))
    st = stage_mixed(ctx, backends, [1] * B)
    qkv = rng.standard_normal((B, H + 2 * KVC), dtype=np.float32)
    d_qkv = DeviceBuffer.from_numpy(ctx, qkv)
    d_q = DeviceBuffer(ctx, 4 * B * H)
    d_o = DeviceBuffer(ctx, 4 * B * H)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, rope))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, (B, H))
    ctx.lib.zr_staged_destroy(st)
    assert np.isfinite(out).all()
    if rope:  # the new row of session s sits at position L - 1 (rope base 500000)
        pos = (ctxlens - 1).astype(np.uint32)
        qkv = qkv.copy()
        qkv[:, :H] = O.apply_rope(qkv[:, :H], pos, D, 500000.0)
        qkv[:, H:H + KVC] = O.apply_rope(qkv[:, H:H + KVC], pos, D, 500000.0)
    sample = sorted({int(np.argmax(ctxlens)), int(np.argmin(ctxlens))} |
                    {int(x) for x in np.random.default_rng(7).choice(B, 6, replace=False)})
    for s in sample:
        L = int(ctxlens[s])
        k = np.concatenate([big[koff[s]:koff[s] + L - 1], qkv[s:s + 1, H:H + KVC]])
        v = np.concatenate([big[voff[s]:voff[s] + L - 1], qkv[s:s + 1, H + KVC:]])
        if kv_dtype == "bf16":
            k, v = O.round_bf16(k), O.round_bf16(v)
        want = np.zeros(H, np.float32)
        for h in range(32):
            kvh = h // 4
            want[h * D:(h + 1) * D] = O.causal_attention_with_prefix(
                qkv[s, h * D:(h + 1) * D][None], np.ascontiguousarray(k[:, kvh * D:(kvh + 1) * D]),
                np.ascontiguousarray(v[:, kvh * D:(kvh + 1) * D]), 1 / math.sqrt(D), L - 1)[0]
        err = max_rel_err_rows(out[s], want, D)
        assert err <= ATTN_RTOL, (s, L, err)
    ctx.close()


# -------------------------------------------------- plain layout (any head_dim) --
@pytest.mark.parametrize("kv_dtype", ["f32", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,D", [(8, 2, 96), (6, 2, 16), (12, 4, 64)])
def test_generic_attention_and_plain_pages(kv_dtype, heads, kv_heads, D):
    """Head dims 96 and 16, and 3 q heads per kv head at D = 64: pages in the
    plain layout, attention by the generic kernel.  Decode rows and causal
    chunks over imported prefixes (one trimmed to start mid-page) against the
    oracle within 2e-3; the pages round-trip bit for bit through export /
    import."""
    Q, KV = heads * D, kv_heads * D
    geo = ModelGeometry(hidden=Q, num_heads=heads, num_kv_heads=kv_heads, num_layers=1, vocab=64, ffn=64)
    ctx = DeviceContext(geo, kv_dtype=kv_dtype, max_tokens=256, max_seqs=8, max_pages_per_seq=64)
    ctx.create_kv_pool(256)
    rng = np.random.default_rng(D + heads)
    cases = [(0, 37, 0), (300, 1, 0), (57, 20, 9), (130, 1, 5)]  # (window, chunk, trimmed)
    backends, Ks, Vs = [], [], []
    for p, c, trim in cases:
        b = ctx.new_backend(max_seq_len=4096)
        k = rng.standard_normal((trim + p + c, KV), dtype=np.float32)
        v = rng.standard_normal((trim + p + c, KV), dtype=np.float32)
        if trim + p:
            b.import_kv_cache(_snapshot(k[:trim + p], v[:trim + p]))
        if trim:
            b.retain_suffix(p)
        backends.append(b)
        Ks.append(k)
        Vs.append(v)
    chunks = [c for _, c, _ in cases]
    T = sum(chunks)
    Qm = rng.standard_normal((T, Q), dtype=np.float32)
    newk = np.concatenate([k[t + p:] for k, (p, _, t) in zip(Ks, cases)])
    newv = np.concatenate([v[t + p:] for v, (p, _, t) in zip(Vs, cases)])
    st = stage_mixed(ctx, backends, chunks)
    d_qkv = DeviceBuffer.from_numpy(ctx, np.concatenate([Qm, newk, newv], 1))
    d_q, d_o = DeviceBuffer(ctx, Qm.nbytes), DeviceBuffer(ctx, Qm.nbytes)
    ctx.check(ctx.lib.zr_rope_kv_write(ctx.h, st, 0, d_qkv.ptr, d_q.ptr, 0))
    ctx.check(ctx.lib.zr_attention(ctx.h, st, 0, d_q.ptr, d_o.ptr))
    out = d_o.download(np.float32, Qm.shape)
    ctx.lib.zr_staged_destroy(st)
    G = heads // kv_heads
    row = 0
    for s, (p, c, trim) in enumerate(cases):
        k, v = Ks[s][trim:], Vs[s][trim:]
        if kv_dtype == "bf16":
            k, v = O.round_bf16(k), O.round_bf16(v)
        for h in range(heads):
            kvh = h // G
            want = O.causal_attention_with_prefix(Qm[row:row + c, h * D:(h + 1) * D],
                                                  np.ascontiguousarray(k[:, kvh * D:(kvh + 1) * D]),
                                                  np.ascontiguousarray(v[:, kvh * D:(kvh + 1) * D]),
                                                  1 / math.sqrt(D), p)
            err = max_rel_err_rows(out[row:row + c, h * D:(h + 1) * D], want, D)
            assert err <= ATTN_RTOL, (s, h, err)
        row += c
        snap = backends[s].export_kv_cache()
        np.testing.assert_array_equal(snap.keys[0], k)
        np.testing.assert_array_equal(snap.values[0], v)
        b2 = ctx.new_backend(max_seq_len=4096)
        b2.import_kv_cache(snap)
        back = b2.export_kv_cache()
        np.testing.assert_array_equal(back.keys, snap.keys)
        np.testing.assert_array_equal(back.values, snap.values)
        b2.close()
    ctx.close()
