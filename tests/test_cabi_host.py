"""CPU checks of the C-ABI library: every declared symbol is exported, errors
follow the reference's convention, and the host page tables (the part of the
provider that runs on the CPU) match the oracle bit for bit."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle as O
from mesh_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in ("zip_rocm.h", "zip_rocm_host.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(zrh?_[a-z0-9_]+)\s*\(", text))
    return names


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declared_functions()
    assert len(declared) > 40
    bound = {name for name, _, _ in _lib.SIGNATURES}
    assert declared == bound, (declared - bound, bound - declared)
    for name in declared:
        assert hasattr(lib, name), name


def _gpu_present():
    lib = _lib.load()
    info = _lib.DeviceInfo()
    return lib.zr_probe(0, C.byref(info)) == 0


def test_probe_reports_missing_device_or_gfx950():
    lib = _lib.load()
    info = _lib.DeviceInfo()
    rc = lib.zr_probe(0, C.byref(info))
    if rc == 0:
        assert info.arch.decode().startswith("gfx950")
    else:
        assert rc in (-6, -3)
        assert lib.zr_global_last_error()


def _desc(**kw):
    d = _lib.ModelDesc()
    vals = dict(hidden=576, num_heads=9, num_kv_heads=3, num_layers=1, vocab=100, ffn_cols=64,
                shard_start=0, shard_end=384, rms_norm_eps=1e-5, rope_base=1e4, page_tokens=16,
                kv_dtype=1, max_tokens=8, max_seqs=8, max_pages_per_seq=8, flags=0)
    vals.update(kw)
    for k, v in vals.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,msg", [
    (dict(shard_start=0, shard_end=300), "not aligned to grouped-query shard width 192"),
    (dict(num_kv_heads=2), "Unsupported grouped-query attention geometry"),
    (dict(shard_start=384, shard_end=384), "Invalid shard range"),
    (dict(page_tokens=32), "page_tokens must be 16"),
    # GEMM operands are addressed with 32-bit buffer offsets: refused up front
    (dict(vocab=2_000_000), "packed lm_head [576, 2000000] exceeds the GEMM's 2 GiB operand limit"),
    (dict(max_tokens=1_000_000), "max_tokens 1000000 x K 576 activations exceed the GEMM's 2 GiB operand limit"),
])
def test_context_rejects_bad_geometry_with_reference_messages(kw, msg):
    # resolve_attention_shard_layout (forward_pass.rs:1257-1315) error texts
    lib = _lib.load()
    h = C.c_void_p()
    rc = lib.zr_context_create(C.byref(_desc(**kw)), 0, C.byref(h))
    assert rc == -1 or rc == -5
    assert msg in lib.zr_global_last_error().decode()
    assert not h.value


# ----------------------------------------------------- host page tables --
class HostBackend:
    """zrh_backend on a bookkeeping-only pool (no device)."""

    def __init__(self, pool, max_seq_len):
        self.lib = _lib.load()
        p = C.c_void_p()
        _lib.check(self.lib.zrh_backend_create(pool, max_seq_len, C.byref(p)))
        self.h = p.value

    def reserve(self, rows):
        _lib.check(self.lib.zrh_kv_reserve(self.h, rows))

    def retain(self, keep):
        _lib.check(self.lib.zrh_retain_suffix(self.h, keep))

    def clear(self):
        self.lib.zrh_clear(self.h)

    def table(self):
        n = self.lib.zrh_block_table(self.h, None, None, None, None, 0)
        ids = np.zeros(max(n, 1), np.uint32)
        st = np.zeros(max(n, 1), np.int32)
        ct = np.zeros(max(n, 1), np.int32)
        gl = np.zeros(max(n, 1), np.int32)
        i32 = lambda a: a.ctypes.data_as(_lib.c_int_p)
        self.lib.zrh_block_table(self.h, ids.ctypes.data_as(_lib.c_u32_p), i32(st), i32(ct), i32(gl), n)
        return [(int(ids[i]), int(st[i]), int(ct[i])) for i in range(n)], gl[:n].tolist()

    @property
    def seq_len(self):
        return self.lib.zrh_cache_seq_len(self.h)

    @property
    def base(self):
        return self.lib.zrh_base_position(self.h)

    def pages(self):
        return self.lib.zrh_allocated_pages(self.h)

    def close(self):
        self.lib.zrh_backend_destroy(self.h)


def host_pool(n, order=None):
    lib = _lib.load()
    p = C.c_void_p()
    if order is None:
        _lib.check(lib.zrh_pool_create(None, None, n, C.byref(p)))
    else:
        o = np.ascontiguousarray(order, np.int32)
        _lib.check(lib.zrh_pool_create(None, o.ctypes.data_as(_lib.c_int_p), n, C.byref(p)))
    return p.value


def test_host_block_table_kat_reused_page_ids():
    # forward_pass.rs:3794-3822: [1, 2, 0, 3]
    pool = host_pool(16)
    b = HostBackend(pool, 48)
    b.reserve(48)
    b.retain(30)
    b.reserve(18)
    table, globals_ = b.table()
    assert [p for p, _, _ in table] == [1, 2, 0, 3]
    assert globals_ == [1, 2, 0, 3]  # pages popped 0,1,2,3 from an ascending pool
    b.close()
    assert _lib.load().zrh_pool_free_pages(pool) == 16
    _lib.load().zrh_pool_destroy(pool)


def test_host_pool_permutation_maps_local_to_global():
    order = np.random.default_rng(0).permutation(512)
    pool = host_pool(512, order)
    b = HostBackend(pool, 4096)
    b.reserve(100)
    table, globals_ = b.table()
    assert [p for p, _, _ in table] == list(range(7))
    assert globals_ == order[::-1][:7].tolist()  # LIFO pops from the end of the order
    b.close()
    _lib.load().zrh_pool_destroy(pool)


def test_host_pool_exhaustion_is_an_error_not_a_crash():
    pool = host_pool(2)
    b = HostBackend(pool, 4096)
    b.reserve(32)
    with pytest.raises(_lib.ZrError) as e:
        b.reserve(1)
    assert "KV pool exhausted" in str(e.value)
    assert b.seq_len == 32  # state rolled back
    b.close()
    _lib.load().zrh_pool_destroy(pool)


@pytest.mark.parametrize("seed", range(8))
def test_host_page_tables_match_oracle_on_random_sequences(seed):
    rng = np.random.default_rng(100 + seed)
    max_seq = int(rng.choice([24, 48, 100, 4096]))
    pool = host_pool(4096)
    b = HostBackend(pool, max_seq)
    o = O.Session(2, 2, 16, max_seq)
    for _ in range(80):
        r = rng.random()
        if r < 0.6:
            n = int(rng.integers(1, 50))
            b.reserve(n)
            z = np.zeros((n, 2), np.float32)
            o.append_all_layers(z, z)
        elif r < 0.9:
            keep = int(rng.integers(0, b.seq_len + 2))
            b.retain(keep)
            o.retain_suffix(keep)
        else:
            b.clear()
            o.clear()
        table, _ = b.table()
        assert table == o.block_table(0) == o.block_table(1)
        assert b.seq_len == o.seq_len() and b.base == o.base_position
        assert b.pages() == o.allocated_pages(0)
    b.close()
    _lib.load().zrh_pool_destroy(pool)


def test_stage_map_names_kernels_that_exist():
    """Every kernel FUSED_KERNEL_STAGES lists (the executor contract's stages,
    engine.rs:240-273) is a __global__ function of the HIP sources."""
    import glob
    import re

    from mesh_amd.provider import FUSED_KERNEL_STAGES

    src = "".join(open(f).read() for f in glob.glob(os.path.join(ROOT, "mesh_amd", "csrc", "*.hip")))
    defined = set(re.findall(r"__global__\s+(?:__launch_bounds__\([^)]*\)\s*)?void\s+(\w+)\s*\(", src))
    for stage, kernels in FUSED_KERNEL_STAGES.items():
        for k in kernels:
            assert k in defined, (stage, k)


# ------------------------------------------------- rollback of failed calls --
def test_failed_multi_page_reserve_returns_global_pages():
    # 48 rows need 3 pages, the pool has 2: the call fails after binding 2
    lib = _lib.load()
    pool = host_pool(2)
    b = HostBackend(pool, 4096)
    with pytest.raises(_lib.ZrError) as e:
        b.reserve(48)
    assert "KV pool exhausted" in str(e.value)
    assert b.seq_len == 0 and b.pages() == 0
    assert lib.zrh_pool_free_pages(pool) == 2
    b.close()
    assert lib.zrh_pool_free_pages(pool) == 2
    lib.zrh_pool_destroy(pool)


def test_failed_reserve_keeps_the_pool_lifo_order():
    order = np.random.default_rng(3).permutation(8)
    pool = host_pool(8, order)
    expect = order[::-1].tolist()  # LIFO pops from the end of the initial order
    b = HostBackend(pool, 4096)
    b.reserve(16 * 5)
    with pytest.raises(_lib.ZrError):
        b.reserve(16 * 4)  # 3 pages left
    _, g = b.table()
    assert g == expect[:5]
    b.reserve(16 * 3)
    _, g = b.table()
    assert g == expect  # the rolled-back pages come out again in order
    b.close()
    _lib.load().zrh_pool_destroy(pool)


def _decode_batch(backends, tokens):
    lib = _lib.load()
    arr = (C.c_void_p * len(backends))(*[b.h for b in backends])
    tok = np.ascontiguousarray(tokens, np.uint32)
    out = np.zeros(len(backends), np.uint32)
    return lib.zrh_decode_step_batch(arr, len(backends), tok.ctypes.data_as(_lib.c_u32_p),
                                     out.ctypes.data_as(_lib.c_u32_p), None, None)


def test_failed_multi_session_assemble_returns_global_pages():
    # three sessions on full pages each need a new page; the pool has one
    lib = _lib.load()
    pool = host_pool(4)
    bs = [HostBackend(pool, 4096) for _ in range(3)]
    for b in bs:
        b.reserve(16)
    before = [b.table() for b in bs]
    assert lib.zrh_pool_free_pages(pool) == 1
    rc = _decode_batch(bs, [1, 2, 3])
    assert rc == -2 and "KV pool exhausted" in lib.zr_global_last_error().decode()
    assert lib.zrh_pool_free_pages(pool) == 1
    assert [b.table() for b in bs] == before
    assert [b.seq_len for b in bs] == [16, 16, 16]
    for b in bs:
        b.close()
    assert lib.zrh_pool_free_pages(pool) == 4
    lib.zrh_pool_destroy(pool)


def test_microbatch_without_device_rolls_back_its_page_tables():
    # assembly succeeds (pages bound), the compute is refused: nothing sticks
    lib = _lib.load()
    pool = host_pool(8)
    bs = [HostBackend(pool, 4096) for _ in range(2)]
    for b in bs:
        b.reserve(16)
    free = lib.zrh_pool_free_pages(pool)
    before = [b.table() for b in bs]
    rc = _decode_batch(bs, [5, 6])
    assert rc == -1 and "bookkeeping-only" in lib.zr_global_last_error().decode()
    assert lib.zrh_pool_free_pages(pool) == free
    assert [b.table() for b in bs] == before
    assert [lib.zrh_sequence_position(b.h) for b in bs] == [16, 16]
    for b in bs:
        b.close()
    lib.zrh_pool_destroy(pool)


def test_failed_import_and_prefill_return_global_pages():
    lib = _lib.load()
    pool = host_pool(3)
    b = HostBackend(pool, 4096)
    b.reserve(20)
    before = b.table()
    k = np.zeros((1, 64, 2), np.float32)
    # 64 rows need 4 pages; the session holds 2 and the pool 1
    rc = lib.zrh_import_kv(b.h, k.ctypes.data_as(_lib.c_f32_p), k.ctypes.data_as(_lib.c_f32_p), 64, 0, 64)
    assert rc == -2
    assert lib.zrh_pool_free_pages(pool) == 1 and b.table() == before and b.seq_len == 20
    # a prefill that fits is assembled, then refused for lack of a device
    toks = np.arange(40, dtype=np.uint32)
    rc = lib.zrh_prefill(b.h, toks.ctypes.data_as(_lib.c_u32_p), 40, None, None)
    assert rc == -1
    assert lib.zrh_pool_free_pages(pool) == 1 and b.table() == before and b.seq_len == 20
    b.close()
    assert lib.zrh_pool_free_pages(pool) == 3
    lib.zrh_pool_destroy(pool)
