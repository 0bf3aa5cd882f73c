"""Pins the oracle to the reference's own known-answer tests, closed forms and
invariants.  Each KAT cites the reference test it reproduces."""
import math

import numpy as np
import pytest

import oracle as O
from tests.testmodels import TEST_CONFIG, constant_weights, geometry, oracle_cfg, random_weights


# ------------------------------------------------------------ page tables --
def test_block_table_tracks_reused_page_ids_after_trim():
    # forward_pass.rs:3794-3822
    s = O.Session(1, 2, 16, 48)
    s.append_layer(0, np.ones((48, 2)), np.full((48, 2), 2.0))
    s.retain_suffix(30)
    s.append_layer(0, np.full((18, 2), 3.0), np.full((18, 2), 4.0))
    bt = s.block_table(0)
    assert len(bt) == 4
    assert [p for p, _, _ in bt] == [1, 2, 0, 3]


def test_reuses_released_pages_after_suffix_trim():
    # forward_pass.rs:3766-3792
    s = O.Session(1, 2, 16, 32)
    s.append_layer(0, np.ones((32, 2)), np.full((32, 2), 2.0))
    assert s.allocated_pages(0) == 2
    s.retain_suffix(16)
    s.append_layer(0, np.full((16, 2), 3.0), np.full((16, 2), 4.0))
    assert s.allocated_pages(0) == 2
    assert len(s.block_table(0)) == 2


def test_retain_suffix_keeps_partial_page_without_rebuild():
    # forward_pass.rs:3728-3764
    s = O.Session(1, 2, 16, 32)
    s.append_layer(0, np.arange(36, dtype=np.float32).reshape(18, 2),
                   np.arange(100, 136, dtype=np.float32).reshape(18, 2))
    s.retain_suffix(17)
    s.append_layer(0, np.array([[36.0, 37.0]]), np.array([[136.0, 137.0]]))
    k, v = s.gather(0)
    assert k.shape[0] == 18
    assert k.reshape(-1).tolist() == list(range(2, 38))
    assert v.reshape(-1).tolist() == list(range(102, 138))


def test_imports_paged_live_kv_layout_17_tokens():
    # forward_pass.rs:3458-3507: 17 tokens -> 2 spans, tail 1
    kv = 16
    s = O.Session(2, kv, 16, 4096)
    snap = {"keys": np.stack([np.full((17, kv), 0.25 + l, np.float32) for l in range(2)]),
            "values": np.stack([np.full((17, kv), 0.5 + l, np.float32) for l in range(2)]),
            "base_position": 0, "next_position": 17, "cached_tokens": 17}
    s.import_snapshot(snap)
    bt = s.block_table(0)
    assert len(bt) == 2
    assert bt[-1][2] % 16 == 1
    ex = s.export()
    assert ex["cached_tokens"] == 17 and ex["next_position"] == 17
    np.testing.assert_array_equal(ex["keys"], snap["keys"])


def test_snapshot_round_trip_and_segmented_window():
    # forward_pass.rs:3356-3456
    kv = 16
    s = O.Session(2, kv, 16, 4096)
    keys = np.stack([np.full((4, kv), 0.2 + l, np.float32) for l in range(2)])
    vals = np.stack([np.full((4, kv), 0.4 + l, np.float32) for l in range(2)])
    s.import_snapshot({"keys": keys, "values": vals, "base_position": 0, "next_position": 4,
                       "cached_tokens": 4})
    assert s.position == 4 and s.seq_len() == 4
    full = s.export()
    np.testing.assert_array_equal(full["keys"], keys)
    np.testing.assert_array_equal(full["values"], vals)
    seg = s.export(2)
    assert seg["next_position"] == 4 and seg["cached_tokens"] == 2 and seg["base_position"] == 2
    np.testing.assert_array_equal(seg["keys"], keys[:, 2:])


def test_clear_reseeds_free_list_highest_first():
    # forward_pass.rs:840-850: the free list becomes 0..n, so pops return n-1 first.
    s = O.Session(1, 2, 16, 4096)
    s.append_layer(0, np.ones((40, 2)), np.ones((40, 2)))
    assert [p for p, _, _ in s.block_table()] == [0, 1, 2]
    s.clear()
    s.append_layer(0, np.ones((20, 2)), np.ones((20, 2)))
    assert [p for p, _, _ in s.block_table()] == [2, 1]
    assert s.base_position == 0


@pytest.mark.parametrize("seed", range(6))
def test_random_append_trim_sequences_keep_window_invariants(seed):
    """Invariant: gather() equals the newest seq_len rows of everything appended
    since the last clear, base_position counts the dropped rows, and every
    block table satisfies the LiveKVBlockTable contract (kv_cache.rs:372-415)."""
    rng = np.random.default_rng(seed)
    max_seq = int(rng.integers(20, 90))
    s = O.Session(2, 3, 16, max_seq)
    stream = np.zeros((0, 3), np.float32)
    counter = 0.0
    for _ in range(60):
        op = rng.random()
        if op < 0.65:
            n = int(rng.integers(1, 40))
            rows = (counter + np.arange(n * 3, dtype=np.float32)).reshape(n, 3)
            counter += n * 3
            s.append_all_layers(rows, -rows)
            stream = np.concatenate([stream, rows])[-max_seq:] if n <= max_seq else rows[-max_seq:]
            if n > max_seq:
                stream = rows[-max_seq:]
        elif op < 0.9 and s.seq_len() > 0:
            keep = int(rng.integers(0, s.seq_len() + 1))
            s.retain_suffix(keep)
            stream = stream[len(stream) - keep:] if keep > 0 else stream[:0]
        else:
            s.clear()
            stream = stream[:0]
        assert s.seq_len() == len(stream)
        if len(stream):
            for layer in range(2):
                k, v = s.gather(layer)
                np.testing.assert_array_equal(k, stream)
                np.testing.assert_array_equal(v, -stream)
            bt = s.block_table(1)
            assert sum(c for _, _, c in bt) == len(stream)
            # interior spans are full pages starting at row 0; only the first
            # may start mid-page (after retain_suffix) and only the last may
            # be partially filled.
            for i, (_, st, ct) in enumerate(bt):
                assert 0 < ct and st + ct <= 16
                if i > 0:
                    assert st == 0
                if i < len(bt) - 1:
                    assert st + ct == 16


# ------------------------------------------------------------------ shard --
def test_attention_shard_layout_supports_gqa_aligned_uneven_shards():
    # forward_pass.rs:3325-3354
    first, idx = O.resolve_shard_layout(576, 9, 3, 0, 384)
    assert (first.q_cols, first.local_q_heads, first.kv_cols, first.local_kv_heads) == (384, 6, 128, 2)
    assert idx == [0, 0, 0, 1, 1, 1]
    second, idx2 = O.resolve_shard_layout(576, 9, 3, 384, 576)
    assert (second.q_cols, second.local_q_heads, second.kv_cols, second.local_kv_heads) == (192, 3, 64, 1)
    assert idx2 == [0, 0, 0]
    with pytest.raises(O.OracleError):
        O.resolve_shard_layout(576, 9, 3, 0, 300)


def test_partition_columns():
    # artifact_loader.rs:351-366 -- e.g. FFN 14336 over 2 workers = 7168 each
    assert O.partition_columns(14336, 0, 2) == 7168
    assert [O.partition_columns(10, p, 3) for p in range(3)] == [4, 3, 3]


# -------------------------------------------------------------------- ops --
def test_matmul_kat():
    # tensor_ops.rs:577-590
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    c = O.matmul(a, b)
    assert c[0, 0] == 22.0 and c[0, 1] == 28.0


def test_matmul_matches_fp64():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((7, 300), dtype=np.float32)
    b = rng.standard_normal((300, 1100), dtype=np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    np.testing.assert_allclose(O.matmul(a, b), ref, rtol=0, atol=1e-4 * np.abs(ref).max())


def test_sample_greedy_kat_and_ties():
    # tensor_ops.rs:633-639; ties keep the first index (strict >, 461-473)
    assert O.sample_greedy([1.0, 5.0, 2.0, 3.0]) == 1
    assert O.sample_greedy([0.0, 7.0, 7.0, 1.0]) == 1


def test_sample_threshold_matches_splitmix64_vector():
    # deterministic_sample_threshold (tensor_ops.rs:372-388) is one SplitMix64
    # step; its published first output from state 0 is 0xE220A8397B1DCDAF.
    assert O.sample_threshold(0) == np.float32(0xE220A8 / float(1 << 24))


def test_sample_token_full_distribution_tracks_cdf():
    logits = np.array([0.5, -0.2, 0.8, 1.1, 0.0, -1.4], np.float32)
    p = np.exp((logits / 1.35) - (logits / 1.35).max())
    p = p / p.sum()
    cdf = np.cumsum(p)
    for seed in range(50):
        r = O.sample_threshold(seed)
        expected = int(np.searchsorted(cdf, r, side="right"))
        tok = O.sample_token(logits, 1.35, 1.0, seed)
        if abs(cdf[min(expected, 5)] - r) > 1e-5 and (expected == 0 or abs(cdf[expected - 1] - r) > 1e-5):
            assert tok == expected


def test_rms_norm_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 96), dtype=np.float32)
    g = rng.standard_normal(96, dtype=np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5) * g
    np.testing.assert_allclose(O.rms_norm(x, g, 1e-5), ref, rtol=2e-6, atol=2e-6)


def test_rope_closed_form_identity_and_norm():
    rng = np.random.default_rng(3)
    d, heads = 64, 3
    x = rng.standard_normal((4, heads * d), dtype=np.float32)
    pos = np.array([0, 1, 517, 8191], np.uint32)
    out = O.apply_rope(x, pos, d, 500000.0)
    np.testing.assert_array_equal(out[0], x[0])  # position 0 is the identity
    half = d // 2
    inv = 1.0 / (500000.0 ** (np.arange(half) * 2.0 / d))
    for r in range(4):
        th = pos[r] * inv
        for h in range(heads):
            a = x[r, h * d:h * d + half].astype(np.float64)
            b = x[r, h * d + half:(h + 1) * d].astype(np.float64)
            ref = np.concatenate([a * np.cos(th) - b * np.sin(th), a * np.sin(th) + b * np.cos(th)])
            # theta = pos * inv_freq rounded in f32 shifts the angle by up to
            # pos * 2^-24 rad, hence the position-scaled tolerance.
            np.testing.assert_allclose(out[r, h * d:(h + 1) * d], ref, atol=3e-6 + 4e-7 * float(pos[r]) * 8)
            np.testing.assert_allclose(np.linalg.norm(out[r, h * d:(h + 1) * d]),
                                       np.linalg.norm(x[r, h * d:(h + 1) * d]), rtol=1e-5)


def test_silu_closed_form():
    x = np.linspace(-20, 20, 1001, dtype=np.float32)
    np.testing.assert_allclose(O.silu(x), x / (1 + np.exp(-x.astype(np.float64))), rtol=1e-6, atol=1e-7)


def _attn64(q, k, v, scale, prefix):
    out = np.zeros((q.shape[0], v.shape[1]))
    for r in range(q.shape[0]):
        n = prefix + r + 1
        s = (k[:n].astype(np.float64) @ q[r].astype(np.float64)) * scale
        p = np.exp(s - s.max())
        out[r] = (p / p.sum()) @ v[:n].astype(np.float64)
    return out


@pytest.mark.parametrize("prefix,rows,kv", [(0, 1, 1), (0, 5, 5), (37, 4, 41), (511, 1, 512)])
def test_attention_matches_fp64_bruteforce(prefix, rows, kv):
    rng = np.random.default_rng(prefix + rows)
    d = 64
    q = rng.standard_normal((rows, d), dtype=np.float32)
    k = rng.standard_normal((kv, d), dtype=np.float32)
    v = rng.standard_normal((kv, d), dtype=np.float32)
    out = O.causal_attention_with_prefix(q, k, v, 1 / math.sqrt(d), prefix)
    np.testing.assert_allclose(out, _attn64(q, k, v, 1 / math.sqrt(d), prefix), rtol=1e-5, atol=1e-5)


def test_attention_special_cases():
    rng = np.random.default_rng(9)
    d = 32
    q = rng.standard_normal((1, d), dtype=np.float32)
    v = rng.standard_normal((7, d), dtype=np.float32)
    # L = 1: the output is v0 exactly
    out1 = O.causal_attention_with_prefix(q, rng.standard_normal((1, d), dtype=np.float32), v[:1], 0.3, 0)
    np.testing.assert_array_equal(out1[0], v[0])
    # identical keys: uniform weights -> mean of V
    k = np.repeat(rng.standard_normal((1, d), dtype=np.float32), 7, 0)
    out = O.causal_attention_with_prefix(q, k, v, 0.3, 6)
    np.testing.assert_allclose(out[0], v.astype(np.float64).mean(0), rtol=1e-6, atol=1e-6)


def test_bf16_rounding_matches_known_patterns():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38, 1e-40], np.float32)
    bits = O.to_bf16_bits(x)
    # 1.00390625 = 1 + 2^-8 is a tie between 0x3F80 and 0x3F81 -> even 0x3F80
    assert bits.tolist()[:4] == [0x3F80, 0x3F80, 0x3F81, 0xC020]
    for xv, b in zip(x, bits):
        assert O.lib().or_f32_to_bf16(float(xv)) == b


# ------------------------------------------------------------------ packing --
def test_pack_staging_kats():
    # fast_path.rs:974-1056: tokens/positions/seq lens/page ids [9, 4, 1]
    bt = np.full((3, 8), -1, np.int32)
    bt[:, :3] = [9, 4, 1]
    bt[:, 3] = 5
    cu_q, cu_k, pos, slot, seq = O.pack([1, 1, 1], [7, 8, 9], [31, 32, 33], [0, 0, 0], bt)
    assert pos.tolist() == [31, 32, 33]
    assert (cu_k[1:] - cu_k[:-1] - 1).tolist() == [7, 8, 9]
    assert cu_q.tolist() == [0, 1, 2, 3]
    assert slot.tolist() == [9 * 16 + 7, 9 * 16 + 8, 9 * 16 + 9]
    # a partial first span (start_token 2, 46 cached): the new row is row 48
    # of the page sequence [9, 4, 1, 5] -> page 5, row 0
    _, _, pos2, slot2, _ = O.pack([1], [46], [48], [2], bt[:1])
    assert pos2.tolist() == [48] and slot2.tolist() == [5 * 16 + 0]
    # prefill positions 64..67 (fast_path.rs:1058-1080)
    _, _, pos3, _, seq3 = O.pack([4], [0], [64], [0], bt[:1])
    assert pos3.tolist() == [64, 65, 66, 67] and seq3.tolist() == [0] * 4


def test_pack_closed_form_random():
    rng = np.random.default_rng(5)
    n = 37
    q_len = rng.integers(1, 40, n)
    kv_before = rng.integers(0, 300, n)
    first_off = rng.integers(0, 16, n)
    first_pos = kv_before + rng.integers(0, 1000, n)
    pages = (first_off + kv_before + q_len + 15) // 16
    bt = np.full((n, int(pages.max())), -1, np.int32)
    perm = rng.permutation(10000)
    used = 0
    for s in range(n):
        bt[s, :pages[s]] = perm[used:used + pages[s]]
        used += pages[s]
    cu_q, cu_k, pos, slot, seq = O.pack(q_len, kv_before, first_pos, first_off, bt)
    assert cu_q.tolist() == [0] + np.cumsum(q_len).tolist()
    assert cu_k.tolist() == [0] + np.cumsum(kv_before + q_len).tolist()
    for s in range(n):
        for i in range(q_len[s]):
            t = cu_q[s] + i
            row = first_off[s] + kv_before[s] + i
            assert seq[t] == s and pos[t] == first_pos[s] + i
            assert slot[t] == bt[s, row // 16] * 16 + row % 16


# ------------------------------------------------------------ forward pass --
def _test_model(cfg=TEST_CONFIG, **kw):
    geo = geometry(cfg)
    return O.Model(oracle_cfg(cfg, geo), constant_weights(cfg, geo)), geo


def test_local_incremental_decode_matches_full_recompute():
    # forward_pass.rs:3270-3292 (exact equality)
    m, geo = _test_model()
    s = O.Session(2, geo["kv_cols"], 16, 4096)
    first = m.prefill(s, [1, 2, 3])
    tok = O.sample_greedy(first)
    dec = m.decode([s], [tok])[0]
    ref_s = O.Session(2, geo["kv_cols"], 16, 4096)
    ref = m.prefill(ref_s, [1, 2, 3, tok])
    np.testing.assert_array_equal(dec, ref)
    assert s.seq_len() == 4 and s.position == 4


def test_incremental_decode_matches_full_recompute_random_gqa():
    cfg = dict(TEST_CONFIG, num_kv_heads=2, num_layers=3)
    geo = geometry(cfg)
    m = O.Model(oracle_cfg(cfg, geo), random_weights(cfg, geo, 11, std=0.2))
    s = O.Session(3, geo["kv_cols"], 16, 4096)
    prompt = [5, 17, 42, 3, 99, 0, 7]
    logits = m.prefill(s, prompt)
    toks = list(prompt)
    for _ in range(20):
        t = O.sample_greedy(logits)
        toks.append(t)
        logits = m.decode([s], [t])[0]
    ref = m.prefill(O.Session(3, geo["kv_cols"], 16, 4096), toks)
    np.testing.assert_array_equal(logits, ref)


def test_local_incremental_decode_slides_live_kv_window():
    # forward_pass.rs:3294-3310
    m, geo = _test_model()
    s = O.Session(2, geo["kv_cols"], 16, 2)
    first = m.prefill(s, [1, 2, 3])
    m.decode([s], [O.sample_greedy(first)])
    assert s.position == 4 and s.seq_len() == 2 and s.base_position == 2 and s.next_position() == 4


def test_decode_microbatch_respects_sliding_device_kv_window():
    # forward_pass.rs:3824-3907
    m, geo = _test_model()
    a = O.Session(2, geo["kv_cols"], 16, 2)
    b = O.Session(2, geo["kv_cols"], 16, 2)
    m.prefill(a, [1, 2, 3])
    m.prefill(b, [1, 2, 3])
    assert a.position == 3 and a.seq_len() == 2 and a.next_position() == 3
    logits = m.decode([a, b], [7, 8])
    assert logits.shape == (2, TEST_CONFIG["vocab"])
    for s in (a, b):
        assert s.position == 4 and s.seq_len() == 2 and s.base_position == 2 and s.next_position() == 4


def test_decode_batch_rows_are_independent():
    """A microbatch row equals the same session decoded alone (rows never mix)."""
    cfg = dict(TEST_CONFIG, num_kv_heads=2)
    geo = geometry(cfg)
    m = O.Model(oracle_cfg(cfg, geo), random_weights(cfg, geo, 3, std=0.2))
    sess = [O.Session(2, geo["kv_cols"]) for _ in range(3)]
    solo = [O.Session(2, geo["kv_cols"]) for _ in range(3)]
    for i in range(3):
        m.prefill(sess[i], list(range(1, 4 + 5 * i)))
        m.prefill(solo[i], list(range(1, 4 + 5 * i)))
    batch = m.decode(sess, [9, 10, 11])
    for i in range(3):
        np.testing.assert_array_equal(batch[i], m.decode([solo[i]], [9 + i])[0])


def test_chunked_prefill_equals_single_prefill():
    cfg = dict(TEST_CONFIG, num_kv_heads=2)
    geo = geometry(cfg)
    m = O.Model(oracle_cfg(cfg, geo), random_weights(cfg, geo, 4, std=0.2))
    toks = [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9, 7, 9, 3, 2, 3, 8, 4]
    whole = m.prefill(O.Session(2, geo["kv_cols"]), toks)
    s = O.Session(2, geo["kv_cols"])
    m.prefill(s, toks[:7])
    m.prefill_chunk(s, toks[7:13])
    last = m.prefill_chunk(s, toks[13:])
    np.testing.assert_allclose(last, whole, rtol=0, atol=1e-5)
    assert s.position == len(toks)


def test_bf16_weight_model_is_bit_identical_to_f32_model():
    """The oracle's bf16-weight form (used for full-width models) computes the
    same f32 products as the f32 form of the same values: logits, partials and
    KV rows must be bit-identical, not merely close."""
    from tests.testmodels import geometry, oracle_cfg, random_weights

    cfg = dict(hidden=256, num_heads=4, num_kv_heads=2, num_layers=2, vocab=300, ffn=320, rms_norm_eps=1e-5,
               rope_base=10000.0)
    geo = geometry(cfg)
    w32 = random_weights(cfg, geo, seed=5, std=0.05)
    mats = ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")
    w16 = dict(embedding=O.to_bf16_bits(w32["embedding"]), final_norm=w32["final_norm"],
               lm_head=O.to_bf16_bits(w32["lm_head"]),
               layers=[dict({k: O.to_bf16_bits(lw[k]) for k in mats}, attn_norm=lw["attn_norm"],
                            mlp_norm=lw["mlp_norm"]) for lw in w32["layers"]])
    m32, m16 = O.Model(oracle_cfg(cfg, geo), w32), O.Model(oracle_cfg(cfg, geo), w16)
    assert m16.bf16 and not m32.bf16
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, cfg["vocab"], n).tolist() for n in (3, 17, 40)]
    s32 = [O.Session(2, geo["kv_cols"]) for _ in prompts]
    s16 = [O.Session(2, geo["kv_cols"]) for _ in prompts]
    for a, b, p in zip(s32, s16, prompts):
        np.testing.assert_array_equal(m32.prefill(a, p), m16.prefill(b, p))
    toks = [1, 2, 3]
    for _ in range(3):
        l32, p32 = m32.decode(s32, toks, want_partials=True)
        l16, p16 = m16.decode(s16, toks, want_partials=True)
        np.testing.assert_array_equal(l32, l16)
        np.testing.assert_array_equal(p32, p16)
        toks = np.argmax(l32, 1).tolist()
    for a, b in zip(s32, s16):
        for layer in range(2):
            for x, y in zip(a.gather(layer), b.gather(layer)):
                np.testing.assert_array_equal(x, y)
    # the matmul itself, against the f32 form and against fp64
    a = rng.standard_normal((19, 300), dtype=np.float32)
    w = O.round_bf16(rng.standard_normal((300, 517), dtype=np.float32))
    wb = O.to_bf16_bits(w)
    out = np.empty((19, 517), np.float32)
    L = O.lib()
    import ctypes as C
    rc = L.or_matmul_bf16w(a.ctypes.data_as(C.POINTER(C.c_float)), wb.ctypes.data_as(C.POINTER(C.c_uint16)),
                           out.ctypes.data_as(C.POINTER(C.c_float)), 19, 300, 517)
    assert rc == 0
    np.testing.assert_array_equal(out, O.matmul(a, w))
    np.testing.assert_allclose(out, a.astype(np.float64) @ w.astype(np.float64), rtol=0, atol=2e-4)


def test_forced_kv_decode_reproduces_the_step_and_returns_its_own_rows():
    """decode_forced appends given bf16 rows instead of its own: forced with
    the rows the oracle itself stores (its bf16-rounded K / V), the step is
    bit-identical to decode(), and the f32 rows it hands back round to exactly
    those rows; a forced row moved by one bf16 step changes that session's
    logits only."""
    from tests.testmodels import geometry, oracle_cfg, random_weights

    cfg = dict(hidden=256, num_heads=4, num_kv_heads=2, num_layers=2, vocab=300, ffn=320, rms_norm_eps=1e-5,
               rope_base=10000.0)
    geo = geometry(cfg)
    m = O.Model(oracle_cfg(cfg, geo), random_weights(cfg, geo, seed=6, std=0.05))
    rng = np.random.default_rng(4)
    prompts = [rng.integers(0, cfg["vocab"], n).tolist() for n in (5, 18, 33)]

    def sessions():
        out = []
        for p in prompts:
            s = O.Session(2, geo["kv_cols"], kv_round_bf16=True)
            m.prefill(s, p)
            out.append(s)
        return out

    toks = [3, 1, 4]
    a = sessions()
    want = m.decode(a, toks)
    rows = np.stack([np.stack([s.gather(l)[i][-1] for s in a]) for l in range(2) for i in range(2)])
    fk, fv = rows[0::2], rows[1::2]  # [layers, B, kv_cols]
    got, own_k, own_v = m.decode_forced(sessions(), toks, fk, fv)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(O.round_bf16(own_k), fk)
    np.testing.assert_array_equal(O.round_bf16(own_v), fv)
    assert not np.array_equal(own_k, fk)  # the own rows are the f32 values before rounding
    fk2 = fk.copy()
    bits = O.to_bf16_bits(fk2[1, 2, :7])
    fk2[1, 2, :7] = O.bf16_bits_to_f32((bits + 1).astype(np.uint16))  # one bf16 step away from zero
    got2, _, _ = m.decode_forced(sessions(), toks, fk2, fv)
    np.testing.assert_array_equal(got2[:2], want[:2])
    assert not np.array_equal(got2[2], want[2])
    with pytest.raises(ValueError):
        m.decode_forced(sessions(), toks, fk[:, :2], fv)
