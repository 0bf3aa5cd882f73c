"""ctypes binding of the oracle (CPU restatement of the zip engine's hot path).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package ``mesh_amd``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int)
u32p = C.POINTER(C.c_uint32)


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.check_call(["make", "-s", "-B" if force else "-s", "-C", _HERE])
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.or_last_error.restype = C.c_char_p
        L.or_session_new.restype = C.c_void_p
        L.or_session_new.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
        L.or_session_free.argtypes = [C.c_void_p]
        for name in ("or_session_append_layer",):
            getattr(L, name).argtypes = [C.c_void_p, C.c_int, f32p, f32p, C.c_int]
        L.or_session_retain_suffix.argtypes = [C.c_void_p, C.c_int]
        L.or_session_clear.argtypes = [C.c_void_p]
        for name in ("or_session_seq_len", "or_session_allocated_pages"):
            getattr(L, name).argtypes = [C.c_void_p, C.c_int]
        for name in ("or_session_base_position", "or_session_position"):
            getattr(L, name).argtypes = [C.c_void_p]
        L.or_session_set_position.argtypes = [C.c_void_p, C.c_int]
        L.or_session_block_table.argtypes = [C.c_void_p, C.c_int, u32p, i32p, i32p, C.c_int]
        L.or_session_gather.argtypes = [C.c_void_p, C.c_int, f32p, f32p]
        L.or_session_export.argtypes = [C.c_void_p, C.c_int, f32p, f32p, i32p, i32p]
        L.or_session_import.argtypes = [C.c_void_p, f32p, f32p, C.c_int, C.c_int, C.c_int]
        L.or_model_new.restype = C.c_void_p
        L.or_model_free.argtypes = [C.c_void_p]
        L.or_model_set_globals.argtypes = [C.c_void_p, f32p, f32p, f32p]
        L.or_model_set_layer.argtypes = [C.c_void_p, C.c_int] + [f32p] * 9
        u16p = C.POINTER(C.c_uint16)
        L.or_model_set_globals_bf16.argtypes = [C.c_void_p, u16p, f32p, u16p]
        L.or_model_set_layer_bf16.argtypes = [C.c_void_p, C.c_int] + [u16p] * 7 + [f32p] * 2
        L.or_matmul_bf16w.argtypes = [f32p, u16p, f32p, C.c_int, C.c_int, C.c_int]
        L.or_decode_microbatch.argtypes = [C.c_void_p, C.POINTER(C.c_void_p), C.c_int, u32p, f32p, f32p]
        L.or_decode_microbatch_forced.argtypes = [C.c_void_p, C.POINTER(C.c_void_p), C.c_int, u32p, f32p, f32p,
                                                  f32p, f32p, f32p, f32p]
        L.or_prefill.argtypes = [C.c_void_p, C.c_void_p, u32p, C.c_int, f32p]
        L.or_prefill_chunk.argtypes = [C.c_void_p, C.c_void_p, u32p, C.c_int, f32p, f32p]
        L.or_matmul.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int]
        L.or_cbor_uint.argtypes = [C.c_int, C.c_uint64, C.c_void_p]
        L.or_cbor_float.argtypes = [C.c_float, C.c_void_p]
        L.or_kv_cbor_encode.restype = C.c_int64
        L.or_kv_cbor_encode.argtypes = [f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int64, C.c_int, C.c_int,
                                        C.c_int, C.c_int, C.c_void_p, C.c_int64]
        L.or_rms_norm.argtypes = [f32p, f32p, f32p, C.c_int, C.c_int, C.c_float]
        L.or_silu.argtypes = [f32p, f32p, C.c_int64]
        L.or_apply_rope.argtypes = [f32p, f32p, C.c_int, C.c_int, u32p, C.c_int, C.c_float]
        L.or_rope_inv_freq.argtypes = [C.c_int, C.c_float, f32p]
        L.or_sample_greedy.argtypes = [f32p, C.c_int]
        L.or_sample_greedy.restype = C.c_uint32
        L.or_sample_token.argtypes = [f32p, C.c_int, C.c_float, C.c_float, C.c_uint64]
        L.or_sample_token.restype = C.c_uint32
        L.or_sample_threshold.argtypes = [C.c_uint64]
        L.or_sample_token_device.restype = C.c_uint32
        L.or_sample_token_device.argtypes = [f32p, C.c_int, C.c_float, C.c_float, C.c_uint64,
                                             C.POINTER(C.c_double)]
        L.or_sample_threshold.restype = C.c_float
        L.or_causal_attention_with_prefix.argtypes = [f32p, f32p, f32p, f32p, C.c_int, C.c_int,
                                                      C.c_int, C.c_float, C.c_int]
        L.or_f32_to_bf16.argtypes = [C.c_float]
        L.or_f32_to_bf16.restype = C.c_uint16
        L.or_resolve_shard_layout.argtypes = [C.c_int] * 5 + [C.c_void_p, u32p]
        L.or_partition_columns.argtypes = [C.c_int, C.c_int, C.c_int]
        L.or_pack.argtypes = [C.c_int, i32p, i32p, i32p, i32p, i32p, C.c_int, C.c_int,
                              i32p, i32p, i32p, i32p, i32p]
        _lib = L
    return _lib


class OracleError(RuntimeError):
    pass


def _check(rc):
    if rc < 0:
        raise OracleError(lib().or_last_error().decode())
    return rc


def _f(a):
    return a.ctypes.data_as(f32p)


def _i(a):
    return a.ctypes.data_as(i32p)


def _u(a):
    return a.ctypes.data_as(u32p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------- ops --
def matmul(a, b):
    a, b = f32(a), f32(b)
    out = np.empty((a.shape[0], b.shape[1]), np.float32)
    _check(lib().or_matmul(_f(a), _f(b), _f(out), a.shape[0], a.shape[1], b.shape[1]))
    return out


def rms_norm(x, gamma, eps):
    x, gamma = f32(x), f32(gamma)
    out = np.empty_like(x)
    _check(lib().or_rms_norm(_f(x), _f(gamma), _f(out), x.shape[0], x.shape[1], eps))
    return out


def silu(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().or_silu(_f(x), _f(out), x.size)
    return out


def apply_rope(x, positions, head_dim, base):
    x = f32(x)
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    out = np.empty_like(x)
    _check(lib().or_apply_rope(_f(x), _f(out), x.shape[0], x.shape[1], _u(pos), head_dim, base))
    return out


def rope_inv_freq(head_dim, base):
    out = np.empty(head_dim // 2, np.float32)
    lib().or_rope_inv_freq(head_dim, base, _f(out))
    return out


def sample_greedy(logits):
    x = f32(logits)
    return int(lib().or_sample_greedy(_f(x), x.size))


def sample_token(logits, temperature, top_p, seed):
    x = f32(logits)
    return int(lib().or_sample_token(_f(x), x.size, temperature, top_p, seed))


def sample_token_device(logits, temperature, top_p, seed):
    """runtime.rs:534-601 device sampler for one row -> (token, margin)."""
    x = f32(logits)
    m = C.c_double()
    t = lib().or_sample_token_device(_f(x), x.size, float(temperature), float(top_p), int(seed), C.byref(m))
    return int(t), m.value


def sample_threshold(seed):
    return float(lib().or_sample_threshold(seed))


def causal_attention_with_prefix(q, k, v, scale, prefix_len):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty((q.shape[0], v.shape[1]), np.float32)
    _check(lib().or_causal_attention_with_prefix(_f(q), _f(k), _f(v), _f(out), q.shape[0],
                                                 k.shape[0], q.shape[1], scale, prefix_len))
    return out


def to_bf16_bits(x):
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h):
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x):
    return bf16_bits_to_f32(to_bf16_bits(x))


class ShardLayout(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("head_dim", "q_heads_per_kv_head", "q_cols", "q_head_start",
                                       "local_q_heads", "kv_cols", "kv_head_start", "local_kv_heads")]


def resolve_shard_layout(hidden, num_heads, num_kv_heads, shard_start, shard_end):
    lay = ShardLayout()
    idx = np.zeros(num_heads, np.uint32)
    _check(lib().or_resolve_shard_layout(hidden, num_heads, num_kv_heads, shard_start, shard_end,
                                         C.byref(lay), _u(idx)))
    return lay, idx[:lay.local_q_heads].tolist()


def cbor_uint(major, v):
    """RFC 8949 head of `major` with argument v (shortest form)."""
    buf = (C.c_uint8 * 9)()
    n = lib().or_cbor_uint(int(major), int(v), buf)
    return bytes(buf[:n])


def cbor_float(x):
    """ciborium's float item for an f32 (narrowest exact of half / single / double)."""
    buf = (C.c_uint8 * 9)()
    n = lib().or_cbor_float(float(np.float32(x)), buf)
    return bytes(buf[:n])


def kv_cbor_encode(k, v, base_position, cfg_num_layers, cfg_num_heads, cfg_head_dim, cfg_max_seq_len):
    """KVCache::to_bytes (kv_cache.rs:880-887) of an export_snapshot cache; k, v [layers, rows, cols] f32."""
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    L, rows, cols = k.shape
    args = (_f(k), _f(v), L, rows, cols, int(base_position), cfg_num_layers, cfg_num_heads, cfg_head_dim,
            cfg_max_seq_len)
    n = lib().or_kv_cbor_encode(*args, None, 0)
    if n < 0:
        raise ValueError("bad KV cache shape")
    out = np.zeros(n, np.uint8)
    m = lib().or_kv_cbor_encode(*args, out.ctypes.data_as(C.c_void_p), n)
    assert m == n
    return out.tobytes()


def partition_columns(total, position, workers):
    return int(lib().or_partition_columns(total, position, workers))


def pack(q_len, kv_before, first_pos, first_offset, block_tables, page_rows=16):
    q_len = np.ascontiguousarray(q_len, np.int32)
    kv_before = np.ascontiguousarray(kv_before, np.int32)
    first_pos = np.ascontiguousarray(first_pos, np.int32)
    first_offset = np.ascontiguousarray(first_offset, np.int32)
    bt = np.ascontiguousarray(block_tables, np.int32)
    n = q_len.size
    total = int(q_len.sum())
    cu_q = np.zeros(n + 1, np.int32)
    cu_k = np.zeros(n + 1, np.int32)
    pos = np.zeros(max(total, 1), np.int32)
    slot = np.zeros(max(total, 1), np.int32)
    seq = np.zeros(max(total, 1), np.int32)
    _check(lib().or_pack(n, _i(q_len), _i(kv_before), _i(first_pos), _i(first_offset), _i(bt),
                         bt.shape[1], page_rows, _i(cu_q), _i(cu_k), _i(pos), _i(slot), _i(seq)))
    return cu_q, cu_k, pos[:total], slot[:total], seq[:total]


# ---------------------------------------------------------------- session --
class Session:
    """One session's paged device KV cache (DeviceKVCache) + ForwardPass.position."""

    def __init__(self, num_layers, kv_cols, page_rows=16, max_seq_len=4096, kv_round_bf16=False):
        self.num_layers, self.kv_cols = num_layers, kv_cols
        self.h = lib().or_session_new(num_layers, kv_cols, page_rows, max_seq_len, int(kv_round_bf16))
        if not self.h:
            raise OracleError(lib().or_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_session_free(self.h)
            self.h = None

    def append_layer(self, layer, k, v):
        k, v = f32(k), f32(v)
        _check(lib().or_session_append_layer(self.h, layer, _f(k), _f(v), k.shape[0]))

    def append_all_layers(self, k, v):
        for layer in range(self.num_layers):
            self.append_layer(layer, k, v)

    def retain_suffix(self, keep):
        _check(lib().or_session_retain_suffix(self.h, keep))

    def clear(self):
        lib().or_session_clear(self.h)

    def seq_len(self, layer=0):
        return _check(lib().or_session_seq_len(self.h, layer))

    @property
    def base_position(self):
        return lib().or_session_base_position(self.h)

    @property
    def position(self):
        return lib().or_session_position(self.h)

    @position.setter
    def position(self, p):
        lib().or_session_set_position(self.h, p)

    def next_position(self):
        return self.base_position + self.seq_len()

    def allocated_pages(self, layer=0):
        return _check(lib().or_session_allocated_pages(self.h, layer))

    def block_table(self, layer=0):
        n = _check(lib().or_session_block_table(self.h, layer, None, None, None, 0))
        ids = np.zeros(max(n, 1), np.uint32)
        st = np.zeros(max(n, 1), np.int32)
        ct = np.zeros(max(n, 1), np.int32)
        _check(lib().or_session_block_table(self.h, layer, _u(ids), _i(st), _i(ct), n))
        return [(int(ids[i]), int(st[i]), int(ct[i])) for i in range(n)]

    def gather(self, layer=0):
        n = self.seq_len(layer)
        k = np.zeros((n, self.kv_cols), np.float32)
        v = np.zeros((n, self.kv_cols), np.float32)
        _check(lib().or_session_gather(self.h, layer, _f(k), _f(v)))
        return k, v

    def export(self, max_cached_tokens=None):
        n = self.seq_len()
        k = np.zeros((self.num_layers, max(n, 1), self.kv_cols), np.float32)
        v = np.zeros_like(k)
        base = C.c_int()
        nxt = C.c_int()
        rows = _check(lib().or_session_export(self.h, -1 if max_cached_tokens is None else max_cached_tokens,
                                              _f(k), _f(v), C.byref(base), C.byref(nxt)))
        if rows == 0:
            return None
        flat_k = k.reshape(-1)[: self.num_layers * rows * self.kv_cols].reshape(self.num_layers, rows, self.kv_cols)
        flat_v = v.reshape(-1)[: self.num_layers * rows * self.kv_cols].reshape(self.num_layers, rows, self.kv_cols)
        return {"keys": flat_k.copy(), "values": flat_v.copy(), "base_position": base.value,
                "next_position": nxt.value, "cached_tokens": rows}

    def import_snapshot(self, snap):
        k, v = f32(snap["keys"]), f32(snap["values"])
        _check(lib().or_session_import(self.h, _f(k), _f(v), int(snap["cached_tokens"]),
                                       int(snap["base_position"]), int(snap["next_position"])))


class ModelConfig(C.Structure):
    _fields_ = [("hidden", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
                ("num_layers", C.c_int), ("vocab", C.c_int), ("ffn_cols", C.c_int),
                ("shard_start", C.c_int), ("shard_end", C.c_int),
                ("rms_norm_eps", C.c_float), ("rope_base", C.c_float)]


class Model:
    """Weights are numpy arrays in the reference [in, out] layout (kept alive
    here): f32 values, or uint16 bf16 bit patterns for every matrix (the
    embedding, LM head and the seven layer matrices; norms stay f32), which
    gives bit-identical results in half the host memory."""

    def __init__(self, cfg: dict, weights: dict):
        c = ModelConfig(cfg["hidden"], cfg["num_heads"], cfg["num_kv_heads"], cfg["num_layers"],
                        cfg["vocab"], cfg["ffn_cols"], cfg.get("shard_start", 0),
                        cfg.get("shard_end", cfg["hidden"]), cfg.get("rms_norm_eps", 1e-5),
                        cfg.get("rope_base", 10000.0))
        self.cfg = cfg
        self.h = lib().or_model_new(C.byref(c))
        if not self.h:
            raise OracleError(lib().or_last_error().decode())
        self._keep = []

        def keep(a):
            a = f32(a)
            self._keep.append(a)
            return _f(a)

        def keep16(a):
            a = np.ascontiguousarray(a, np.uint16)
            self._keep.append(a)
            return a.ctypes.data_as(C.POINTER(C.c_uint16))

        mats = ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")
        self.bf16 = np.asarray(weights["embedding"]).dtype == np.uint16
        if self.bf16:
            _check(lib().or_model_set_globals_bf16(self.h, keep16(weights["embedding"]), keep(weights["final_norm"]),
                                                   keep16(weights["lm_head"])))
        else:
            _check(lib().or_model_set_globals(self.h, keep(weights["embedding"]), keep(weights["final_norm"]),
                                              keep(weights["lm_head"])))
        for l, lw in enumerate(weights["layers"]):
            if self.bf16:
                _check(lib().or_model_set_layer_bf16(self.h, l, *[keep16(lw[k]) for k in mats],
                                                     keep(lw["attn_norm"]), keep(lw["mlp_norm"])))
            else:
                _check(lib().or_model_set_layer(self.h, l, *[keep(lw[k]) for k in mats], keep(lw["attn_norm"]),
                                                keep(lw["mlp_norm"])))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None

    def decode(self, sessions, tokens, want_partials=False):
        B = len(sessions)
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros((B, self.cfg["vocab"]), np.float32)
        parts = (np.zeros((self.cfg["num_layers"], 2, B, self.cfg["hidden"]), np.float32)
                 if want_partials else None)
        arr = (C.c_void_p * B)(*[s.h for s in sessions])
        _check(lib().or_decode_microbatch(self.h, arr, B, _u(toks), _f(logits),
                                          _f(parts) if parts is not None else None))
        return (logits, parts) if want_partials else logits

    def decode_forced(self, sessions, tokens, force_k, force_v):
        """decode() with the appended K / V rows taken from force_k / force_v
        [num_layers, B, kv_cols] (rows another implementation stored as
        bf16).  Returns (logits, own_k, own_v): own_* are this oracle's own
        f32 rows of the step, before rounding, in the same shape."""
        B = len(sessions)
        toks = np.ascontiguousarray(tokens, np.uint32)
        fk, fv = f32(force_k), f32(force_v)
        L, KV = self.cfg["num_layers"], fk.shape[-1]
        if fk.shape != (L, B, KV) or fv.shape != (L, B, KV):
            raise ValueError(f"forced rows must be [{L}, {B}, kv_cols], got {fk.shape} / {fv.shape}")
        logits = np.zeros((B, self.cfg["vocab"]), np.float32)
        own_k, own_v = np.zeros_like(fk), np.zeros_like(fv)
        arr = (C.c_void_p * B)(*[s.h for s in sessions])
        _check(lib().or_decode_microbatch_forced(self.h, arr, B, _u(toks), _f(logits), None, _f(fk), _f(fv),
                                                 _f(own_k), _f(own_v)))
        return logits, own_k, own_v

    def prefill(self, session, tokens):
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros(self.cfg["vocab"], np.float32)
        _check(lib().or_prefill(self.h, session.h, _u(toks), toks.size, _f(logits)))
        return logits

    def prefill_chunk(self, session, tokens, want_partials=False):
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros(self.cfg["vocab"], np.float32)
        parts = (np.zeros((self.cfg["num_layers"], 2, toks.size, self.cfg["hidden"]), np.float32)
                 if want_partials else None)
        _check(lib().or_prefill_chunk(self.h, session.h, _u(toks), toks.size, _f(logits),
                                      _f(parts) if parts is not None else None))
        return (logits, parts) if want_partials else logits


# ------------------------------------------------------- fast-path planner --
# FastPathPlanner / DecodeWorkspaceLease restated in Python (the planner is
# host bookkeeping): agent/src/inference/fast_path.rs.
DECODE_BUCKET_BATCHES = (1, 2, 4, 8)                         # fast_path.rs:15
DECODE_BUCKET_KV_TOKENS = (2048, 8192, 16384, 32768, 65536)  # fast_path.rs:16
U32_MAX = 0xFFFFFFFF


PREFILL_BUCKET_TOKENS = (128, 512, 2048, 8192, 16384)        # fast_path.rs:17


def fnv1a64(data):
    """FNV-1a, 64-bit (Fowler, Noll, Vo; offset basis 0xcbf29ce484222325,
    prime 0x100000001b3): the hash the library's layout hash uses."""
    h = 0xcbf29ce484222325
    for b in data:
        h = ((h ^ b) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def fast_path_layout_hash(phase, batch_size_ceiling, token_ceiling, fields):
    """The layout hash of a bucket key (phase 0 decode / 1 prefill, provider
    rocm, profile rocm_fused, both ceilings) and its metadata fields, hashed
    in the order of FastPathPlanner::layout_hash (fast_path.rs:892-902).  The
    reference's hasher (Rust's DefaultHasher) is process-local; the library
    uses FNV-1a 64 over the same items (integers as 8 little-endian bytes,
    names as their bytes then 0xff), restated here."""
    out = bytearray()

    def u64(v):
        out.extend(int(v).to_bytes(8, "little"))

    def name(s):
        out.extend(s.encode())
        out.append(0xFF)

    u64(phase)
    name("rocm")
    name("rocm_fused")
    u64(batch_size_ceiling)
    u64(token_ceiling)
    for field, count, stride in fields:
        name(field)
        u64(4)
        u64(count)
        u64(stride)
    return fnv1a64(bytes(out))


def _fast_path_plan(phase, b, t, actual_batch, actual_tokens):
    """FastPathPlanner::build_plan (fast_path.rs:780-829) for the rocm_fused
    profile: metadata_fields (839-867), capture_strategy (831-837: the fused
    profile replays), the prefill strategy of plan_prefill (697)."""
    slots = -(-t // 16)
    fields = [(name, n, 4 * n) for name, n in (("slot_sequence_lengths", b), ("slot_positions", b),
                                               ("slot_block_tables", b * slots), ("slot_mapping", b))]
    label = f"decode-b{b}-kv{t}-rocm" if phase == 0 else f"prefill-t{t}-rocm"
    return dict(phase=phase, batch_size_ceiling=b, token_ceiling=t, page_slots=slots, fields=fields,
                bucket_label=label, actual_batch_size=actual_batch, actual_token_count=actual_tokens,
                capture_strategy="replay_preferred",
                prefill_strategy="single_sequence_buckets" if phase == 1 else "",
                workspace_bytes=sum(f[2] for f in fields) + 96 * t + 32 * 1024 * b,
                layout_hash=fast_path_layout_hash(phase, b, t, fields))


def fast_path_plan_decode(batch_size, total_kv_tokens, profile="RocmFused"):
    """FastPathPlanner::plan_decode (fast_path.rs:644-669): the first bucket of
    supported_decode_buckets (batch outer, kv tokens inner; 606-623) holding
    the batch, and the metadata layout of metadata_fields (839-867): field
    name -> (element count, stride bytes) with u32 elements."""
    for b in DECODE_BUCKET_BATCHES:
        for t in DECODE_BUCKET_KV_TOKENS:
            if batch_size <= b and total_kv_tokens <= t:
                return _fast_path_plan(0, b, t, batch_size, total_kv_tokens)
    raise OracleError(f"no stable Decode bucket supports batch_size={batch_size} token_count={total_kv_tokens} "
                      f"for {profile}")


def fast_path_plan_prefill(prompt_tokens, profile="RocmFused"):
    """FastPathPlanner::plan_prefill (fast_path.rs:680-702): the first bucket of
    supported_prefill_buckets (625-642: batch ceiling 1) holding the prompt."""
    for t in PREFILL_BUCKET_TOKENS:
        if prompt_tokens <= t:
            return _fast_path_plan(1, 1, t, 1, prompt_tokens)
    raise OracleError(f"no stable Prefill bucket supports batch_size=1 token_count={prompt_tokens} for {profile}")


def fast_path_stage_prefill_positions(plan, absolute_position_start, token_count):
    """PrefillWorkspaceLease::stage_positions (fast_path.rs:409-445) after
    PrefillWorkspaceBuffers::reset (207-210): the lease's positions buffer."""
    T = plan["token_ceiling"]
    if token_count > T:
        raise OracleError(f"fast-path capture invariant failed for prefill-t{T}-rocm: prefill token count "
                          f"{token_count} exceeds bucket ceiling {T}")
    out = np.zeros(T, np.uint32)
    for i in range(token_count):
        p = absolute_position_start + i
        if p > U32_MAX:
            raise OracleError("prefill absolute position exceeded u32 addressable range")
        out[i] = p
    return out


def fast_path_validate_decode_contexts(plan, contexts):
    """FastPathPlanner::validate_decode_contexts (fast_path.rs:704-778).
    contexts: dicts of FastPathBackendContext (provider, optimization_profile,
    model_id or None, logical_kv_tokens); the plan's bucket is rocm /
    rocm_fused."""
    label = plan["bucket_label"]

    def unsafe(detail):
        return OracleError(f"fast-path capture invariant failed for {label}: {detail}")

    if len(contexts) != plan["actual_batch_size"]:
        raise unsafe(f"planned batch size {plan['actual_batch_size']} but executor received {len(contexts)} requests")
    if not contexts:
        return

    def same_kind(c):
        return c["provider"] == "rocm" and c["optimization_profile"] == "rocm_fused"

    if not same_kind(contexts[0]):
        raise unsafe("primary backend context does not match planned provider/profile")
    primary = contexts[0].get("model_id")
    for c in contexts:
        if not same_kind(c):
            raise unsafe("mixed provider/profile contexts cannot reuse a single fast-path bucket")
        if c["logical_kv_tokens"] > plan["token_ceiling"]:
            raise unsafe(f"session KV footprint {c['logical_kv_tokens']} exceeds bucket token ceiling "
                         f"{plan['token_ceiling']}")
        if primary is not None and c.get("model_id") is not None and c["model_id"] != primary:
            raise unsafe("mixed model residencies cannot share one replay-valid bucket")
    observed = fast_path_layout_hash(plan["phase"], plan["batch_size_ceiling"], plan["token_ceiling"], plan["fields"])
    if observed != plan["layout_hash"]:
        raise OracleError(f"fast-path metadata drift for {label}: expected layout hash {plan['layout_hash']}, "
                          f"observed {observed}")


def fast_path_stage_decode(plan, tokens, slots):
    """DecodeWorkspaceLease::stage_with_slot_reader (fast_path.rs:263-338) after
    DecodeWorkspaceBuffers::reset (227-235).  slots: (position, sequence_len,
    page_ids) per slot, the DecodeSlotState of each session.  Returns the
    token / position buffers and the four metadata fields."""
    B, T, S = plan["batch_size_ceiling"], plan["token_ceiling"], plan["page_slots"]
    label = plan["bucket_label"]
    if len(tokens) > B:
        raise OracleError(f"fast-path capture invariant failed for {label}: runtime batch size {len(tokens)} "
                          f"exceeds bucket ceiling {B}")
    out = dict(token_ids=np.zeros(B, np.uint32), positions=np.zeros(B, np.uint32),
               slot_sequence_lengths=np.zeros(B, np.uint32), slot_positions=np.zeros(B, np.uint32),
               slot_block_tables=np.full(B * S, U32_MAX, np.uint32), slot_mapping=np.full(B, U32_MAX, np.uint32))
    out["token_ids"][:len(tokens)] = tokens
    for i, (position, seq_len, page_ids) in enumerate(slots[:len(tokens)]):
        if seq_len > T:
            raise OracleError(f"fast-path capture invariant failed for {label}: slot {i} sequence length {seq_len} "
                              f"exceeds bucket token ceiling {T}")
        if len(page_ids) > S:
            raise OracleError(f"fast-path capture invariant failed for {label}: slot {i} block table length "
                              f"{len(page_ids)} exceeds workspace capacity {S}")
        out["positions"][i] = position
        out["slot_sequence_lengths"][i] = seq_len
        out["slot_positions"][i] = position
        out["slot_mapping"][i] = i
        out["slot_block_tables"][i * S:i * S + len(page_ids)] = page_ids
    return out
