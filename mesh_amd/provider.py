"""The `rocm` execution provider, mirroring zip's provider interface.

Names, argument meaning and error behaviour follow the reference:
  ExecutionProviderKind           agent/src/provider/mod.rs:8-33 (+ "rocm")
  ExecutionBackend / ProviderExecutionBackend
                                  agent/src/inference/backend.rs:30-88, 400-662
  BackendMicrobatchExecutor.decode_step_batch
                                  agent/src/inference/backend.rs:107-151
  DecodeMicrobatchRequest / Output  backend.rs:90-105
  KVCacheSnapshot                 agent/src/inference/kv_cache.rs:102-187
Every compute call goes through libzip_rocm.so (HIP kernels on gfx950); a
missing library raises instead of falling back to the CPU.
"""
from __future__ import annotations

import ctypes as C
import time
import weakref
from dataclasses import dataclass, field
from enum import Enum
from typing import List, Optional, Sequence

import numpy as np

from . import _lib
from ._lib import ZrError, check


class ExecutionProviderKind(str, Enum):
    CPU = "cpu"
    METAL = "metal"
    CUDA = "cuda"
    ROCM = "rocm"

    @classmethod
    def from_str(cls, value: str) -> Optional["ExecutionProviderKind"]:
        try:
            return cls(value.strip().lower())
        except ValueError:
            return None


# FusedKernelStage (engine.rs:124-132) -> the kernels that implement it here.
FUSED_KERNEL_STAGES = {
    "norm_qkv": ["rms_norm_vec_kernel", "rms_norm_kernel", "gemm_kernel"],
    # one-row decode microbatches: RoPE + KV append run inside paged_attention_kernel
    "rope_kv_write": ["rope_table_kernel", "rope_kv_write_kernel", "rope_kv_write_vec_kernel", "paged_attention_kernel"],
    "paged_attention": ["paged_attention_kernel", "paged_prefill_attention_kernel", "attention_merge_kernel"],
    "residual_mlp": ["rms_norm_vec_kernel", "rms_norm_kernel", "gemm_kernel", "gemm_swiglu_ksplit_kernel",
                     "splitk_reduce_kernel"],
    "device_sampling": ["argmax_partial_kernel", "argmax_final_kernel", "sample_kernel"],
}


def executor_contract() -> dict:
    """LocalExecutorContract + BackendContractDescriptor of the rocm arm
    (engine.rs:171-273, provider/mod.rs:88-150) as the library reports it
    (zr_get_executor_contract); "stage_kernels" maps each fused stage to the
    kernels that implement it."""
    lib = _lib.load()
    c = _lib.ExecutorContract()
    check(lib.zr_get_executor_contract(C.byref(c)))
    out = {name: getattr(c, name) for name, _ in _lib.ExecutorContract._fields_
           if not name.startswith("n_") and name not in ("host_kernels", "fused_stages", "stage_kernels")}
    out = {k: (v.decode() if isinstance(v, bytes) else v) for k, v in out.items()}
    out["host_kernels"] = [c.host_kernels[i].decode() for i in range(c.n_host_kernels)]
    out["fused_stages"] = [c.fused_stages[i].decode() for i in range(c.n_fused_stages)]
    out["stage_kernels"] = {c.fused_stages[i].decode(): c.stage_kernels[i].decode().split(",")
                            for i in range(c.n_fused_stages)}
    return out


class FastPathPlanner:
    """FastPathPlanner (fast_path.rs:604-890) for the rocm_fused profile, the
    DecodeWorkspaceLease staging (263-338) and PrefillWorkspaceLease
    positions (409-445), through the C-ABI."""

    @staticmethod
    def plan_decode(batch_size: int, total_kv_tokens: int, max_sequence_len: int) -> "_lib.FastPathPlan":
        plan = _lib.FastPathPlan()
        check(_lib.load().zrh_fast_path_plan_decode(batch_size, total_kv_tokens, max_sequence_len, C.byref(plan)))
        return plan

    @staticmethod
    def plan_prefill(prompt_tokens: int) -> "_lib.FastPathPlan":
        """plan_prefill (680-702): SingleSequenceBuckets over 128 ... 16384 tokens."""
        plan = _lib.FastPathPlan()
        check(_lib.load().zrh_fast_path_plan_prefill(prompt_tokens, C.byref(plan)))
        return plan

    @staticmethod
    def stage_prefill_positions(plan, absolute_position_start: int, token_count: int) -> np.ndarray:
        """PrefillWorkspaceLease::stage_positions (409-445): the staged
        positions (token_count words of the lease's token_ceiling)."""
        out = np.zeros(max(plan.token_ceiling, 1), np.uint32)
        check(_lib.load().zrh_fast_path_stage_prefill_positions(C.byref(plan), absolute_position_start, token_count,
                                                                _ptr(out, C.c_uint32)))
        return out[:token_count]

    @staticmethod
    def validate_decode_contexts(plan, contexts: Sequence[dict]) -> None:
        """validate_decode_contexts (704-778) over FastPathBackendContext dicts
        (provider, optimization_profile, model_id, logical_kv_tokens)."""
        arr = (_lib.FastPathBackendContext * max(len(contexts), 1))()
        keep = []
        for i, c in enumerate(contexts):
            enc = [None if c.get(k) is None else str(c[k]).encode() for k in
                   ("provider", "optimization_profile", "model_id")]
            keep.append(enc)
            arr[i] = _lib.FastPathBackendContext(enc[0], enc[1], enc[2], int(c["logical_kv_tokens"]))
        check(_lib.load().zrh_fast_path_validate_decode_contexts(C.byref(plan), arr, len(contexts)))

    @staticmethod
    def stage_decode(plan, backends: Sequence["RocmExecutionBackend"], tokens: Sequence[int]) -> dict:
        lib = _lib.load()
        B = plan.batch_size_ceiling
        meta = np.zeros(plan.metadata_bytes // 4, np.uint32)
        token_ids = np.zeros(B, np.uint32)
        positions = np.zeros(B, np.uint32)
        toks = np.ascontiguousarray(tokens, np.uint32)
        arr = (C.c_void_p * max(len(backends), 1))(*[b.h for b in backends])
        ctx = getattr(getattr(backends[0], "ctx", None), "h", None) if backends else None
        check(lib.zrh_fast_path_stage_decode(C.byref(plan), C.cast(arr, C.POINTER(C.c_void_p)), len(backends),
                                             _ptr(toks, C.c_uint32), _ptr(meta, C.c_uint32),
                                             _ptr(token_ids, C.c_uint32), _ptr(positions, C.c_uint32)), ctx)
        names = ("slot_sequence_lengths", "slot_positions", "slot_block_tables", "slot_mapping")
        out = {"token_ids": token_ids, "positions": positions}
        for f, name in enumerate(names):
            o, n = plan.field_offset[f] // 4, plan.field_bytes[f] // 4
            out[name] = meta[o:o + n]
        return out


def probe_provider(device: int = 0):
    """runtime.rs:335-385: (available, error message)."""
    try:
        lib = _lib.load()
    except ImportError as exc:
        return False, str(exc)
    info = _lib.DeviceInfo()
    rc = lib.zr_probe(device, C.byref(info))
    if rc != 0:
        return False, lib.zr_global_last_error().decode()
    return True, None


def device_info(device: int = 0) -> dict:
    lib = _lib.load()
    info = _lib.DeviceInfo()
    check(lib.zr_probe(device, C.byref(info)))
    return {"device_count": info.device_count, "compute_units": info.compute_units,
            "clock_mhz": info.clock_mhz, "hbm_bytes": info.hbm_bytes, "arch": info.arch.decode()}


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(C.POINTER(ctype))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


class KVTransfer:
    """A session's KV window between HBM and host memory, its PCIe copy on a
    stream of its own (zr_transfer): from zrh_export_kv_async (to the host) or
    zr_kv_upload_async (from the host)."""

    def __init__(self, ctx: "DeviceContext", handle: int):
        self.ctx = ctx
        self.h = handle
        ctx._transfers.add(self)

    def done(self) -> bool:
        """The host copy has finished."""
        r = self.ctx.lib.zr_transfer_done(self.h)
        if r < 0:
            self.ctx.check(r)
        return r == 1

    def wait(self):
        self.ctx.check(self.ctx.lib.zr_transfer_wait(self.h))

    def close(self):
        """Waits for the copy and for the last kernel on the device buffer, which the context keeps for reuse."""
        if getattr(self, "h", None) and self.ctx.h:
            self.ctx.lib.zr_transfer_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class PinnedBuffer:
    """Pinned host memory of a context (zr_host_alloc), viewed as numpy."""

    def __init__(self, ctx: "DeviceContext", nbytes: int):
        self.ctx = ctx
        p = C.c_void_p()
        ctx.check(ctx.lib.zr_host_alloc(ctx.h, int(nbytes), C.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)
        ctx._pinned.add(self)

    def array(self, dtype, shape) -> np.ndarray:
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        assert n <= self.nbytes
        buf = (C.c_char * n).from_address(self.ptr)
        return np.frombuffer(buf, dtype=dtype).reshape(shape)

    def free(self):
        if getattr(self, "ptr", None) and self.ctx.h:
            self.ctx.lib.zr_host_free(self.ctx.h, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceBuffer:
    """Device memory owned by a context (zr_device_alloc)."""

    def __init__(self, ctx: "DeviceContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(ctx.lib.zr_device_alloc(ctx.h, self.nbytes, C.byref(p)), ctx.h)
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, ctx, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(ctx, arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(self.ctx.lib.zr_memcpy_h2d(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes), self.ctx.h)

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(self.ctx.lib.zr_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes), self.ctx.h)
        return out

    def free(self):
        if self.ptr:
            self.ctx.lib.zr_device_free(self.ctx.h, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class ModelGeometry:
    """ModelConfig (forward_pass.rs:156-174) plus this worker's shard range."""
    hidden: int
    num_heads: int
    num_kv_heads: int
    num_layers: int
    vocab: int
    ffn: int
    rms_norm_eps: float = 1e-5
    rope_base: float = 10000.0
    shard_start: int = 0
    shard_end: Optional[int] = None
    ffn_cols: Optional[int] = None

    def __post_init__(self):
        if self.shard_end is None:
            self.shard_end = self.hidden
        if self.ffn_cols is None:
            self.ffn_cols = self.ffn

    @property
    def head_dim(self):
        return self.hidden // self.num_heads

    @property
    def q_cols(self):
        return self.shard_end - self.shard_start

    @property
    def kv_cols(self):
        qpk = self.num_heads // self.num_kv_heads
        return (self.q_cols // (qpk * self.head_dim)) * self.head_dim


class DeviceContext:
    """SharedModelResidency + KV pool of one worker on one GPU (zr_context)."""

    def __init__(self, geo: ModelGeometry, *, kv_dtype: str = "bf16", max_tokens: int = 256,
                 max_seqs: int = 256, max_pages_per_seq: int = 512, split_activations: bool = False,
                 device: int = 0, model_id: Optional[str] = None):
        self.lib = _lib.load()
        self.geo = geo
        self.model_id = model_id  # SharedModelResidency's model id (FastPathBackendContext.model_id)
        d = _lib.ModelDesc()
        d.hidden, d.num_heads, d.num_kv_heads = geo.hidden, geo.num_heads, geo.num_kv_heads
        d.num_layers, d.vocab, d.ffn_cols = geo.num_layers, geo.vocab, geo.ffn_cols
        d.shard_start, d.shard_end = geo.shard_start, geo.shard_end
        d.rms_norm_eps, d.rope_base = geo.rms_norm_eps, geo.rope_base
        d.page_tokens = 16
        d.kv_dtype = _lib.ZR_DTYPE_BF16 if kv_dtype == "bf16" else _lib.ZR_DTYPE_F32
        d.max_tokens, d.max_seqs, d.max_pages_per_seq = max_tokens, max_seqs, max_pages_per_seq
        d.flags = _lib.ZR_FLAG_SPLIT_ACTIVATIONS if split_activations else 0
        self.desc = d
        self.kv_dtype = kv_dtype
        h = C.c_void_p()
        check(self.lib.zr_context_create(C.byref(d), device, C.byref(h)))
        self.h = h.value
        self.pool = None
        self._backends = weakref.WeakSet()
        self._pinned = weakref.WeakSet()
        self._transfers = weakref.WeakSet()

    def forward_replay_info(self) -> dict:
        """The step graph that zr_forward replays greedy decode steps from
        (zr_forward_replay_info; zeros before the first replay)."""
        st = _lib.StepGraphStats()
        self.check(self.lib.zr_forward_replay_info(self.h, C.byref(st)))
        return {name: getattr(st, name) for name, _ in _lib.StepGraphStats._fields_}

    def close(self):
        for b in list(getattr(self, "_backends", ())):
            b.close()
        for t in list(getattr(self, "_transfers", ())):  # before the pinned buffers they copy into
            t.close()
        for p in list(getattr(self, "_pinned", ())):
            p.free()
        if getattr(self, "pool", None) is not None:
            self.lib.zrh_pool_destroy(self.pool)
            self.pool = None
        if getattr(self, "h", None):
            self.lib.zr_context_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc):
        return check(rc, self.h)

    # -- weights (bf16 bits, reference [in, out] layout) -------------------------------
    def upload_layer(self, layer: int, w: dict):
        keep = {k: np.ascontiguousarray(v, np.float32 if k.endswith("norm") else np.uint16) for k, v in w.items()}
        lw = _lib.LayerWeights()
        for name in ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down"):
            setattr(lw, name, _ptr(keep[name], C.c_uint16))
        lw.attn_norm = _ptr(keep["attn_norm"], C.c_float)
        lw.mlp_norm = _ptr(keep["mlp_norm"], C.c_float)
        self.check(self.lib.zr_upload_layer(self.h, layer, C.byref(lw)))

    def upload_globals(self, embedding: np.ndarray, final_norm: np.ndarray, lm_head: np.ndarray):
        e = np.ascontiguousarray(embedding, np.uint16)
        f = np.ascontiguousarray(final_norm, np.float32)
        l = np.ascontiguousarray(lm_head, np.uint16)
        self.check(self.lib.zr_upload_globals(self.h, _ptr(e, C.c_uint16), _ptr(f, C.c_float), _ptr(l, C.c_uint16)))

    def upload_f32_model(self, weights: dict):
        """Upload a model given as f32 arrays holding bf16-exact values."""
        for l, lw in enumerate(weights["layers"]):
            w = {k: bf16_bits(lw[k]) for k in ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")}
            w["attn_norm"], w["mlp_norm"] = lw["attn_norm"], lw["mlp_norm"]
            self.upload_layer(l, w)
        self.upload_globals(bf16_bits(weights["embedding"]), weights["final_norm"], bf16_bits(weights["lm_head"]))

    # -- KV pool -----------------------------------------------------------------------
    def create_kv_pool(self, n_pages: int, initial_order: Optional[Sequence[int]] = None):
        self.check(self.lib.zr_kv_pool_create(self.h, n_pages))
        if self.pool is not None:
            self.lib.zrh_pool_destroy(self.pool)
        p = C.c_void_p()
        if initial_order is None:
            self.check(self.lib.zrh_pool_create(self.h, None, 0, C.byref(p)))
        else:
            order = np.ascontiguousarray(initial_order, np.int32)
            self.check(self.lib.zrh_pool_create(self.h, _ptr(order, C.c_int), order.size, C.byref(p)))
        self.pool = p.value

    @property
    def free_pages(self) -> int:
        return self.lib.zrh_pool_free_pages(self.pool)

    def kv_pool_bytes(self) -> int:
        return int(self.lib.zr_kv_pool_bytes(self.h))

    def kv_head_map(self) -> List[int]:
        n = C.c_int()
        out = np.zeros(max(self.geo.num_heads, 1), np.uint32)
        self.check(self.lib.zr_kv_head_map(self.h, _ptr(out, C.c_uint32), out.size, C.byref(n)))
        return out[: n.value].tolist()

    def upload_kv_async(self, snap: "KVCacheSnapshot") -> KVTransfer:
        """Starts copying a snapshot's rows into a device buffer (zr_kv_upload_async) for a
        later import_kv_cache_transfer; the arrays must stay untouched until the transfer is done."""
        k, v = snap.keys, snap.values
        assert k.dtype == np.float32 and v.dtype == np.float32 and k.flags.c_contiguous and v.flags.c_contiguous
        t = C.c_void_p()
        self.check(self.lib.zr_kv_upload_async(self.h, _ptr(k, C.c_float), _ptr(v, C.c_float), snap.cached_tokens,
                                               C.byref(t)))
        return KVTransfer(self, t.value)

    def new_backend(self, max_seq_len: int = 4096) -> "RocmExecutionBackend":
        b = RocmExecutionBackend(self, max_seq_len)
        self._backends.add(b)
        return b


@dataclass
class KVCacheSnapshot:
    """Sequence state + per-layer KV rows (KVCacheSnapshot, kv_cache.rs:102-187)."""
    next_position: int
    cached_tokens: int
    keys: np.ndarray    # [layers, cached_tokens, kv_cols] f32
    values: np.ndarray
    storage: object = field(default=None, repr=False, compare=False)  # pinned owner, if any

    def first_cached_position(self) -> int:
        return self.next_position - self.cached_tokens


@dataclass
class KVSequenceState:
    """KVSequenceState (kv_cache.rs:20-26)."""
    next_position: int
    cached_tokens: int

    def first_cached_position(self) -> int:
        return self.next_position - self.cached_tokens


@dataclass
class KVCacheBlob:
    """KVCacheBlob (kv_cache.rs:68-100): encoding + the serialized KVCache."""
    encoding: str  # "FullSnapshotCbor" (KVCacheEncoding, kv_cache.rs:12-17)
    data: memoryview = field(repr=False)
    storage: object = field(default=None, repr=False, compare=False)  # pinned owner, if any

    def size_bytes(self) -> int:
        return len(self.data)


@dataclass
class KVCacheWireSnapshot:
    """KVCacheSnapshot (kv_cache.rs:102-107) with its blob as wire bytes."""
    sequence: KVSequenceState
    blob: KVCacheBlob


class RocmExecutionBackend:
    """One session's ExecutionBackend on the rocm provider (zrh_backend)."""

    provider_kind = ExecutionProviderKind.ROCM
    optimization_profile = "rocm_fused"

    def __init__(self, ctx: DeviceContext, max_seq_len: int = 4096):
        self.ctx = ctx
        self.lib = ctx.lib
        p = C.c_void_p()
        ctx.check(self.lib.zrh_backend_create(ctx.pool, max_seq_len, C.byref(p)))
        self.h = p.value
        self.max_seq_len = max_seq_len

    def close(self):
        if getattr(self, "h", None) and self.ctx.pool is not None:
            self.lib.zrh_backend_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- ExecutionBackend ---------------------------------------------------------------
    def prefill(self, tokens: Sequence[int]) -> np.ndarray:
        toks = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros(self.ctx.geo.vocab, np.float32)
        greedy = C.c_uint32()
        self.ctx.check(self.lib.zrh_prefill(self.h, _ptr(toks, C.c_uint32), toks.size, _ptr(logits, C.c_float),
                                            C.byref(greedy)))
        self.last_greedy = int(greedy.value)
        return logits

    def decode_step(self, token: int) -> np.ndarray:
        logits = np.zeros(self.ctx.geo.vocab, np.float32)
        greedy = C.c_uint32()
        self.ctx.check(self.lib.zrh_decode_step(self.h, int(token), _ptr(logits, C.c_float), C.byref(greedy)))
        self.last_greedy = int(greedy.value)
        return logits

    def sample(self, logits: np.ndarray, temperature: float, top_p: float, seed: int) -> int:
        """ForwardPass::sample (forward_pass.rs:2046-2086): greedy when temperature <= 0
        or (temperature == 1 and top_p >= 1) -- the argmax computed on the GPU with the
        logits; otherwise sample_token_device (runtime.rs:622-632) on the GPU."""
        if temperature <= 0.0 or (temperature == 1.0 and top_p >= 1.0):
            return self.last_greedy
        return sample_device(self.ctx, np.asarray(logits, np.float32)[None], [temperature], [top_p], [seed])[0]

    def fast_path_context(self) -> dict:
        """FastPathBackendContext (fast_path.rs:102-108, backend.rs:748-755)."""
        c = _lib.FastPathContext()
        self.ctx.check(self.lib.zrh_get_fast_path_context(self.h, C.byref(c)))
        return {"provider": ExecutionProviderKind.ROCM.value, "optimization_profile": self.optimization_profile,
                "model_id": self.ctx.model_id, "logical_kv_tokens": c.logical_kv_tokens, "position": c.position,
                "cached_tokens": c.cached_tokens,
                "decode_token_ceiling": None if c.decode_token_ceiling < 0 else c.decode_token_ceiling}

    def cache_seq_len(self) -> int:
        return self.lib.zrh_cache_seq_len(self.h)

    def live_kv_cache_bytes(self) -> int:
        return int(self.lib.zrh_live_kv_cache_bytes(self.h))

    def logical_kv_tokens(self) -> int:
        return self.lib.zrh_logical_kv_tokens(self.h)

    def sequence_position(self) -> int:
        return self.lib.zrh_sequence_position(self.h)

    def base_position(self) -> int:
        return self.lib.zrh_base_position(self.h)

    def allocated_pages(self) -> int:
        return self.lib.zrh_allocated_pages(self.h)

    def export_kv_cache(self, max_cached_tokens: Optional[int] = None, pinned: bool = False,
                        into: Optional[PinnedBuffer] = None) -> Optional[KVCacheSnapshot]:
        """export_kv_cache (backend.rs:73): the newest `max_cached_tokens` rows
        (all when None) of every layer as f32.  With `pinned`, the snapshot's
        arrays live in pinned host memory (full-rate PCIe copies): in `into`
        when it is large enough, else in a new PinnedBuffer."""
        geo = self.ctx.geo
        n = self.cache_seq_len()
        if max_cached_tokens is not None:
            n = min(n, max(int(max_cached_tokens), 1))
        shape = (geo.num_layers, max(n, 1), geo.kv_cols)
        owner = None
        if pinned:
            need = 2 * 4 * int(np.prod(shape))
            owner = into if into is not None and into.ptr and into.nbytes >= need else PinnedBuffer(self.ctx, need)
            both = owner.array(np.float32, (2,) + shape)
            k, v = both[0], both[1]
        else:
            k = np.zeros(shape, np.float32)
            v = np.zeros_like(k)
        rows, base, nxt = C.c_int(), C.c_int(), C.c_int()
        self.ctx.check(self.lib.zrh_export_kv(self.h, -1 if max_cached_tokens is None else int(max_cached_tokens),
                                              _ptr(k, C.c_float), _ptr(v, C.c_float), C.byref(rows),
                                              C.byref(base), C.byref(nxt)))
        r = rows.value
        if r == 0:
            if owner is not None:
                owner.free()
            return None
        assert r == n
        if owner is not None:
            return KVCacheSnapshot(nxt.value, r, k, v, owner)
        return KVCacheSnapshot(nxt.value, r, k, v)

    def export_kv_cache_async(self, max_cached_tokens: Optional[int] = None,
                              into: Optional[PinnedBuffer] = None):
        """export_kv_cache with the copy to pinned host memory in flight
        (zrh_export_kv_async): returns (snapshot, transfer), (None, None) for
        an empty cache.  The session's pages may be released at once; the
        snapshot's arrays hold the rows after transfer.wait() (or done())."""
        geo = self.ctx.geo
        n = self.cache_seq_len()
        if max_cached_tokens is not None:
            n = min(n, max(int(max_cached_tokens), 1))
        shape = (geo.num_layers, max(n, 1), geo.kv_cols)
        need = 2 * 4 * int(np.prod(shape))
        owner = into if into is not None and into.ptr and into.nbytes >= need else PinnedBuffer(self.ctx, need)
        both = owner.array(np.float32, (2,) + shape)
        k, v = both[0], both[1]
        rows, base, nxt, t = C.c_int(), C.c_int(), C.c_int(), C.c_void_p()
        self.ctx.check(self.lib.zrh_export_kv_async(self.h, -1 if max_cached_tokens is None else int(max_cached_tokens),
                                                    _ptr(k, C.c_float), _ptr(v, C.c_float), C.byref(rows),
                                                    C.byref(base), C.byref(nxt), C.byref(t)))
        if rows.value == 0:
            if owner is not into:
                owner.free()
            return None, None
        assert rows.value == n and t.value
        return KVCacheSnapshot(nxt.value, rows.value, k, v, owner), KVTransfer(self.ctx, t.value)

    def import_kv_cache_transfer(self, snap: KVCacheSnapshot, transfer: KVTransfer):
        """import_kv_cache from a transfer's device buffer (zrh_import_kv_transfer): an upload of
        `snap`, or the in-flight export that produced it."""
        self.ctx.check(self.lib.zrh_import_kv_transfer(self.h, transfer.h, snap.cached_tokens,
                                                       snap.first_cached_position(), snap.next_position))

    def import_kv_cache(self, snap: KVCacheSnapshot):
        k = np.ascontiguousarray(snap.keys, np.float32)
        v = np.ascontiguousarray(snap.values, np.float32)
        self.ctx.check(self.lib.zrh_import_kv(self.h, _ptr(k, C.c_float), _ptr(v, C.c_float), snap.cached_tokens,
                                              snap.first_cached_position(), snap.next_position))

    def export_kv_snapshot(self, max_cached_tokens: Optional[int] = None,
                           pinned: bool = False) -> Optional[KVCacheWireSnapshot]:
        """export_kv_cache (backend.rs:73) as the reference's snapshot: sequence
        state + KVCache::to_bytes (kv_cache.rs:880-887) encoded on the device.
        With `pinned`, the bytes live in pinned host memory."""
        geo = self.ctx.geo
        n = self.cache_seq_len()
        if n == 0:
            return None
        if max_cached_tokens is not None:
            n = min(n, max(int(max_cached_tokens), 1))
        # f16 / f32 items: at most 5 B a float, plus the fixed map and key bytes
        bound = 5 * 2 * geo.num_layers * n * geo.kv_cols + 128 * (2 * geo.num_layers + 1) + 512
        mc = -1 if max_cached_tokens is None else int(max_cached_tokens)
        size, nxt, cached = C.c_size_t(), C.c_int(), C.c_int()
        for attempt in range(2):
            owner = PinnedBuffer(self.ctx, bound) if pinned else None
            buf = owner.array(np.uint8, (bound,)) if pinned else np.empty(bound, np.uint8)
            rc = self.lib.zrh_export_kv_cbor(self.h, mc, buf.ctypes.data, bound, C.byref(size), C.byref(nxt),
                                             C.byref(cached))
            if rc == _lib.ZR_E_INVALID and size.value > bound and attempt == 0:  # NaN items take 9 B
                bound = size.value
                if owner is not None:
                    owner.free()
                continue
            self.ctx.check(rc)
            break
        if cached.value == 0:
            return None
        data = memoryview(buf)[:size.value]
        return KVCacheWireSnapshot(KVSequenceState(nxt.value, cached.value),
                                   KVCacheBlob("FullSnapshotCbor", data, owner))

    def import_kv_snapshot(self, snap: KVCacheWireSnapshot):
        """import_kv_cache (backend.rs:74) from the reference's snapshot bytes."""
        if snap.blob.encoding != "FullSnapshotCbor":
            raise ValueError(f"unsupported KV snapshot encoding {snap.blob.encoding}")
        data = np.frombuffer(snap.blob.data, np.uint8)
        self.ctx.check(self.lib.zrh_import_kv_cbor(self.h, data.ctypes.data if data.size else None, data.size,
                                                   snap.sequence.next_position, snap.sequence.cached_tokens))

    def clear(self):
        self.lib.zrh_clear(self.h)

    def release_pages(self):
        self.ctx.check(self.lib.zrh_release_pages(self.h))

    # -- page-table introspection --------------------------------------------------------
    def block_table(self):
        n = self.lib.zrh_block_table(self.h, None, None, None, None, 0)
        if n < 0:
            self.ctx.check(n)
        ids = np.zeros(max(n, 1), np.uint32)
        st = np.zeros(max(n, 1), np.int32)
        ct = np.zeros(max(n, 1), np.int32)
        gl = np.zeros(max(n, 1), np.int32)
        self.ctx.check(min(0, self.lib.zrh_block_table(self.h, _ptr(ids, C.c_uint32), _ptr(st, C.c_int),
                                                       _ptr(ct, C.c_int), _ptr(gl, C.c_int), n)))
        return [(int(ids[i]), int(st[i]), int(ct[i]), int(gl[i])) for i in range(n)]

    def kv_reserve(self, rows: int):
        self.ctx.check(self.lib.zrh_kv_reserve(self.h, rows))

    def retain_suffix(self, keep: int):
        self.ctx.check(self.lib.zrh_retain_suffix(self.h, keep))


def sample_device(ctx: "DeviceContext", logits: np.ndarray, temperature, top_p, seeds) -> List[int]:
    """sample_tokens_device_with_seeds (runtime.rs:534-601) per row with its own
    temperature / top_p / seed, on the GPU (zr_sample)."""
    x = np.ascontiguousarray(logits, np.float32)
    rows, cols = x.shape
    temps = np.ascontiguousarray(temperature, np.float32)
    tops = np.ascontiguousarray(top_p, np.float32)
    sd = np.ascontiguousarray(seeds, np.uint64)
    d_x = DeviceBuffer.from_numpy(ctx, x)
    d_out = DeviceBuffer(ctx, 4 * rows)
    try:
        ctx.check(ctx.lib.zr_sample(ctx.h, d_x.ptr, rows, cols, _ptr(temps, C.c_float), _ptr(tops, C.c_float),
                                    _ptr(sd, C.c_uint64), d_out.ptr))
        out = d_out.download(np.uint32, (rows,))
    finally:
        d_x.free()
        d_out.free()
    return [int(t) for t in out]


@dataclass
class DecodeMicrobatchRequest:
    session_id: str
    token: int
    backend: RocmExecutionBackend
    job_id: str = ""
    temperature: float = 0.0
    top_p: float = 1.0
    sampling_seed: int = 0


@dataclass
class DecodeMicrobatchOutput:
    session_id: str
    logits: Optional[np.ndarray]
    sampled_token: Optional[int]
    execution_time_ms: int


def _backend_array(backends):
    arr = (C.c_void_p * len(backends))(*[b.h for b in backends])
    return C.cast(arr, C.POINTER(C.c_void_p)), arr


class DecodePipeline:
    """The serving loop of BackendMicrobatchExecutor.decode_step_batch over a
    fixed set of sessions, pipelined (zrh_decode_pipeline): every step does its
    host bookkeeping, stages its metadata and replays the bucket's captured
    step graph; step() returns the previous step's greedy ids, so the host work
    of step k + 1 overlaps step k on the device.  Ids stay on the device between
    steps (step 0 reads `first_tokens`)."""

    def __init__(self, backends: Sequence["RocmExecutionBackend"], first_tokens: Sequence[int]):
        self.ctx = backends[0].ctx
        self.lib = self.ctx.lib
        self.n = len(backends)
        self._ptrs, self._keep = _backend_array(backends)
        toks = np.ascontiguousarray(first_tokens, np.uint32)
        h = C.c_void_p()
        self.ctx.check(self.lib.zrh_decode_pipeline_create(self._ptrs, self.n, _ptr(toks, C.c_uint32), C.byref(h)))
        self.h = h.value
        self._prev = np.zeros(self.n, np.uint32)
        self._ready = C.c_int(0)

    def step(self) -> Optional[np.ndarray]:
        """Enqueues the next step; returns the previous step's ids (None on the first)."""
        self.ctx.check(self.lib.zrh_decode_pipeline_step(self.h, _ptr(self._prev, C.c_uint32), C.byref(self._ready)))
        return self._prev.copy() if self._ready.value else None

    def finish(self) -> np.ndarray:
        """Waits for the last enqueued step; its ids."""
        out = np.zeros(self.n, np.uint32)
        self.ctx.check(self.lib.zrh_decode_pipeline_finish(self.h, _ptr(out, C.c_uint32)))
        return out

    def info(self) -> dict:
        steps = C.c_uint64()
        st = _lib.StepGraphStats()
        self.ctx.check(self.lib.zrh_decode_pipeline_info(self.h, C.byref(steps), C.byref(st)))
        out = {name: getattr(st, name) for name, _ in _lib.StepGraphStats._fields_}
        out["steps"] = steps.value
        return out

    def close(self):
        if getattr(self, "h", None):
            self.lib.zrh_decode_pipeline_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class BackendMicrobatchExecutor:
    @staticmethod
    def decode_step_batch(requests: List[DecodeMicrobatchRequest], want_logits: bool = False,
                          partials: Optional[np.ndarray] = None, plan=None) -> List[DecodeMicrobatchOutput]:
        """backend.rs:110-151 fast path: one fused microbatch over every session.
        A `plan` (FastPathPlanner.plan_decode) is validated against the
        requests' backend contexts first (validate_decode_contexts, 116-123).
        Greedy requests get `sampled_token` from the device argmax (backend.rs:537-553)."""
        if plan is not None:
            FastPathPlanner.validate_decode_contexts(plan, [r.backend.fast_path_context() for r in requests])
        if not requests:
            raise ZrError(-1, "Decode microbatch requires at least one backend and token")
        ctx = requests[0].backend.ctx
        for r in requests:
            if r.backend.ctx is not ctx:
                raise ZrError(-1, "Fast-path decode batch requires one shared model residency")
        n = len(requests)
        toks = np.ascontiguousarray([r.token for r in requests], np.uint32)
        out_tokens = np.zeros(n, np.uint32)
        logits = np.zeros((n, ctx.geo.vocab), np.float32) if want_logits else None
        ptrs, _keep = _backend_array([r.backend for r in requests])
        stochastic = any(r.temperature > 0.0 and r.top_p > 0.0 for r in requests)
        t0 = time.perf_counter()
        lg = _ptr(logits, C.c_float) if logits is not None else None
        pa = _ptr(partials, C.c_float) if partials is not None else None
        if stochastic:  # sample_fast_path_logits_batch (backend.rs:275-316) on the device logits
            temps = np.ascontiguousarray([r.temperature for r in requests], np.float32)
            tops = np.ascontiguousarray([r.top_p for r in requests], np.float32)
            seeds = np.ascontiguousarray([r.sampling_seed for r in requests], np.uint64)
            ctx.check(ctx.lib.zrh_decode_step_batch_sampled(ptrs, n, _ptr(toks, C.c_uint32), _ptr(temps, C.c_float),
                                                            _ptr(tops, C.c_float), _ptr(seeds, C.c_uint64),
                                                            _ptr(out_tokens, C.c_uint32), lg, pa))
        else:
            ctx.check(ctx.lib.zrh_decode_step_batch(ptrs, n, _ptr(toks, C.c_uint32), _ptr(out_tokens, C.c_uint32),
                                                    lg, pa))
        ms = int((time.perf_counter() - t0) * 1000)
        return [DecodeMicrobatchOutput(r.session_id, logits[i] if logits is not None else None, int(out_tokens[i]), ms)
                for i, r in enumerate(requests)]

    @staticmethod
    def forward_mixed(backends: List[RocmExecutionBackend], chunks: List[Sequence[int]], want_logits: bool = True,
                      partials: Optional[np.ndarray] = None):
        """Mixed chunked-prefill + decode microbatch packed into one varlen tensor."""
        ctx = backends[0].ctx
        q_len = np.ascontiguousarray([len(c) for c in chunks], np.int32)
        toks = np.ascontiguousarray(np.concatenate([np.asarray(c, np.uint32) for c in chunks]), np.uint32)
        n = len(backends)
        out_tokens = np.zeros(n, np.uint32)
        logits = np.zeros((n, ctx.geo.vocab), np.float32) if want_logits else None
        ptrs, _keep = _backend_array(backends)
        ctx.check(ctx.lib.zrh_forward_mixed(ptrs, n, _ptr(q_len, C.c_int), _ptr(toks, C.c_uint32),
                                            _ptr(out_tokens, C.c_uint32),
                                            _ptr(logits, C.c_float) if logits is not None else None,
                                            _ptr(partials, C.c_float) if partials is not None else None))
        return out_tokens, logits
