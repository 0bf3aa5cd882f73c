"""ctypes binding of libzip_rocm.so (include/zip_rocm.h, include/zip_rocm_host.h).

Loading fails loudly when the HIP library has not been built: there is no
CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# ZR_LIBRARY may name another build of the same library (A/B measurements)
LIB_PATH = os.environ.get("ZR_LIBRARY") or os.path.join(HERE, "libzip_rocm.so")

c_int_p = C.POINTER(C.c_int)
c_u32_p = C.POINTER(C.c_uint32)
c_u16_p = C.POINTER(C.c_uint16)
c_f32_p = C.POINTER(C.c_float)
c_void_pp = C.POINTER(C.c_void_p)

ZR_OK = 0
ZR_E_INVALID = -1
ZR_DTYPE_F32 = 0
ZR_DTYPE_BF16 = 1
ZR_FLAG_SPLIT_ACTIVATIONS = 1

STATUS_NAMES = {0: "ZR_OK", -1: "ZR_E_INVALID", -2: "ZR_E_OOM", -3: "ZR_E_HIP", -4: "ZR_E_INVARIANT",
                -5: "ZR_E_UNSUPPORTED", -6: "ZR_E_NODEVICE"}


class ZrError(RuntimeError):
    """A failed zr_* call (AgentError::Execution in the reference)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class DeviceInfo(C.Structure):
    _fields_ = [("device_count", C.c_int), ("device", C.c_int), ("compute_units", C.c_int),
                ("clock_mhz", C.c_int), ("hbm_bytes", C.c_uint64), ("arch", C.c_char * 64)]


class ModelDesc(C.Structure):
    _fields_ = [("hidden", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
                ("num_layers", C.c_int), ("vocab", C.c_int), ("ffn_cols", C.c_int),
                ("shard_start", C.c_int), ("shard_end", C.c_int), ("rms_norm_eps", C.c_float),
                ("rope_base", C.c_float), ("page_tokens", C.c_int), ("kv_dtype", C.c_int),
                ("max_tokens", C.c_int), ("max_seqs", C.c_int), ("max_pages_per_seq", C.c_int),
                ("flags", C.c_int)]


class LayerWeights(C.Structure):
    _fields_ = [("w_q", c_u16_p), ("w_k", c_u16_p), ("w_v", c_u16_p), ("w_o", c_u16_p),
                ("w_gate", c_u16_p), ("w_up", c_u16_p), ("w_down", c_u16_p),
                ("attn_norm", c_f32_p), ("mlp_norm", c_f32_p)]


class Microbatch(C.Structure):
    _fields_ = [("num_seqs", C.c_int), ("q_len", c_int_p), ("kv_before", c_int_p),
                ("first_pos", c_int_p), ("first_offset", c_int_p), ("block_tables", c_int_p),
                ("block_table_stride", C.c_int), ("tokens", c_u32_p)]


class StepGraphStats(C.Structure):
    _fields_ = [("launches", C.c_uint64), ("captures", C.c_int), ("buckets", C.c_int), ("sequences", C.c_int),
                ("items_capacity", C.c_int), ("merge_capacity", C.c_int), ("fused_rope", C.c_int),
                ("metadata_bytes", C.c_size_t)]


class ExecutorContract(C.Structure):
    _fields_ = [("executor_class", C.c_char_p), ("optimization_profile", C.c_char_p),
                ("n_host_kernels", C.c_int), ("host_kernels", C.POINTER(C.c_char_p)),
                ("n_fused_stages", C.c_int), ("fused_stages", C.POINTER(C.c_char_p)),
                ("stage_kernels", C.POINTER(C.c_char_p)), ("collective_residency", C.c_char_p),
                ("prefill_supports_microbatch", C.c_int), ("prefill_requires_static_workspace", C.c_int),
                ("prefill_uses_device_sampling", C.c_int), ("decode_supports_microbatch", C.c_int),
                ("decode_requires_static_workspace", C.c_int), ("decode_uses_device_sampling", C.c_int),
                ("kv_requires_paged_cache", C.c_int), ("kv_append_only_decode", C.c_int),
                ("kv_supports_prefill", C.c_int), ("kv_supports_decode", C.c_int),
                ("collective_tensors_per_layer", C.c_int), ("provider", C.c_char_p),
                ("compatibility_class", C.c_char_p), ("memory_model", C.c_char_p),
                ("supports_decode_microbatch", C.c_int), ("supports_paged_kv", C.c_int),
                ("supports_checkpoint_handoff", C.c_int), ("supports_device_sampling", C.c_int),
                ("fast_path_eligible", C.c_int), ("capture_strategy", C.c_char_p)]


class FastPathContext(C.Structure):
    _fields_ = [("logical_kv_tokens", C.c_int), ("position", C.c_int), ("cached_tokens", C.c_int),
                ("decode_token_ceiling", C.c_int)]


class FastPathPlan(C.Structure):
    _fields_ = [("batch_size_ceiling", C.c_int), ("token_ceiling", C.c_int), ("actual_batch_size", C.c_int),
                ("actual_token_count", C.c_int), ("max_sequence_len", C.c_int), ("page_slots", C.c_int),
                ("field_offset", C.c_size_t * 4), ("field_bytes", C.c_size_t * 4), ("metadata_bytes", C.c_size_t),
                ("workspace_bytes", C.c_size_t), ("workspace_alignment", C.c_size_t),
                ("bucket_label", C.c_char * 64), ("phase", C.c_int), ("capture_strategy", C.c_char * 24),
                ("prefill_strategy", C.c_char * 32), ("layout_hash", C.c_uint64)]


class FastPathBackendContext(C.Structure):
    _fields_ = [("provider", C.c_char_p), ("optimization_profile", C.c_char_p), ("model_id", C.c_char_p),
                ("logical_kv_tokens", C.c_int)]


# (name, restype, argtypes) for every exported symbol declared in include/*.h
SIGNATURES = [
    # zip_rocm.h
    ("zr_probe", C.c_int, [C.c_int, C.POINTER(DeviceInfo)]),
    ("zr_global_last_error", C.c_char_p, []),
    ("zr_context_create", C.c_int, [C.POINTER(ModelDesc), C.c_int, c_void_pp]),
    ("zr_context_destroy", None, [C.c_void_p]),
    ("zr_last_error", C.c_char_p, [C.c_void_p]),
    ("zr_kv_head_map", C.c_int, [C.c_void_p, c_u32_p, C.c_int, c_int_p]),
    ("zr_upload_layer", C.c_int, [C.c_void_p, C.c_int, C.POINTER(LayerWeights)]),
    ("zr_upload_globals", C.c_int, [C.c_void_p, c_u16_p, c_f32_p, c_u16_p]),
    ("zr_kv_pool_create", C.c_int, [C.c_void_p, C.c_int]),
    ("zr_kv_pool_pages", C.c_int, [C.c_void_p]),
    ("zr_kv_pool_bytes", C.c_uint64, [C.c_void_p]),
    ("zr_forward", C.c_int, [C.c_void_p, C.POINTER(Microbatch), c_u32_p, c_f32_p, c_f32_p]),
    ("zr_stage", C.c_int, [C.c_void_p, C.POINTER(Microbatch), c_void_pp]),
    ("zr_staged_destroy", None, [C.c_void_p]),
    ("zr_forward_staged_async", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    ("zr_synchronize", C.c_int, [C.c_void_p]),
    ("zr_graph_capture_staged", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, c_void_pp]),
    ("zr_graph_launch", C.c_int, [C.c_void_p, C.c_void_p]),
    ("zr_graph_destroy", None, [C.c_void_p]),
    ("zr_transfer_cached_bytes", C.c_size_t, [C.c_void_p]),
    ("zr_step_graph_create", C.c_int, [C.c_void_p, c_void_pp]),
    ("zr_step_graph_launch", C.c_int, [C.c_void_p, C.POINTER(Microbatch), C.c_void_p, C.c_void_p, C.c_void_p]),
    ("zr_step_graph_info", C.c_int, [C.c_void_p, C.POINTER(StepGraphStats)]),
    ("zr_forward_replay_info", C.c_int, [C.c_void_p, C.POINTER(StepGraphStats)]),
    ("zr_step_graph_destroy", None, [C.c_void_p]),
    ("zr_pack", C.c_int, [C.c_void_p, C.POINTER(Microbatch), c_int_p, c_int_p, c_int_p, c_int_p, c_int_p]),
    ("zr_rope_kv_write", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int]),
    ("zr_attention", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    ("zr_kv_read_probe", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_double)]),
    ("zr_rope_attention", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int]),
    ("zr_kv_gather", C.c_int, [C.c_void_p, c_int_p, C.c_int, C.c_int, C.c_int, C.c_int, c_f32_p, c_f32_p]),
    ("zr_kv_scatter", C.c_int, [C.c_void_p, c_int_p, C.c_int, C.c_int, C.c_int, C.c_int, c_f32_p, c_f32_p]),
    ("zr_kv_gather_async", C.c_int, [C.c_void_p, c_int_p, C.c_int, C.c_int, C.c_int, C.c_int, c_f32_p, c_f32_p,
                                     c_void_pp]),
    ("zr_kv_upload_async", C.c_int, [C.c_void_p, c_f32_p, c_f32_p, C.c_int, c_void_pp]),
    ("zr_kv_scatter_transfer", C.c_int, [C.c_void_p, C.c_void_p, c_int_p, C.c_int, C.c_int, C.c_int, C.c_int]),
    ("zr_transfer_done", C.c_int, [C.c_void_p]),
    ("zr_transfer_wait", C.c_int, [C.c_void_p]),
    ("zr_transfer_destroy", None, [C.c_void_p]),
    ("zr_kv_export_cbor", C.c_int, [C.c_void_p, c_int_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_longlong, C.c_int,
                                    C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    ("zr_kv_read_pages", C.c_int, [C.c_void_p, C.c_int, c_int_p, C.c_int, C.c_void_p]),
    ("zr_argmax", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    ("zr_argmax_noalloc", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    ("zr_sample", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, c_f32_p, c_f32_p, C.POINTER(C.c_uint64),
                            C.c_void_p]),
    ("zr_sample_last_logits", C.c_int, [C.c_void_p, C.c_int, c_f32_p, c_f32_p, C.POINTER(C.c_uint64), c_u32_p]),
    ("zr_rms_norm", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    ("zr_gemm", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    ("zr_gemm_swiglu", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    ("zr_device_alloc", C.c_int, [C.c_void_p, C.c_size_t, c_void_pp]),
    ("zr_device_free", C.c_int, [C.c_void_p, C.c_void_p]),
    ("zr_host_alloc", C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    ("zr_host_free", C.c_int, [C.c_void_p, C.c_void_p]),
    ("zr_memcpy_h2d", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("zr_memcpy_d2h", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t]),
    ("zr_fill_normal_bf16", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint64, C.c_float]),
    ("zr_kv_pool_fill_normal", C.c_int, [C.c_void_p, C.c_uint64, C.c_float]),
    ("zr_get_executor_contract", C.c_int, [C.POINTER(ExecutorContract)]),
    ("zr_timing_begin", C.c_int, [C.c_void_p, C.c_uint]),
    ("zr_timing_end", C.c_int, [C.c_void_p, C.POINTER(C.c_double), c_int_p]),
    # zip_rocm_host.h
    ("zrh_pool_create", C.c_int, [C.c_void_p, c_int_p, C.c_int, c_void_pp]),
    ("zrh_pool_destroy", None, [C.c_void_p]),
    ("zrh_pool_free_pages", C.c_int, [C.c_void_p]),
    ("zrh_backend_create", C.c_int, [C.c_void_p, C.c_int, c_void_pp]),
    ("zrh_backend_destroy", None, [C.c_void_p]),
    ("zrh_prefill", C.c_int, [C.c_void_p, c_u32_p, C.c_int, c_f32_p, c_u32_p]),
    ("zrh_decode_step", C.c_int, [C.c_void_p, C.c_uint32, c_f32_p, c_u32_p]),
    ("zrh_decode_step_batch", C.c_int, [c_void_pp, C.c_int, c_u32_p, c_u32_p, c_f32_p, c_f32_p]),
    ("zrh_decode_step_batch_sampled", C.c_int, [c_void_pp, C.c_int, c_u32_p, c_f32_p, c_f32_p,
                                                C.POINTER(C.c_uint64), c_u32_p, c_f32_p, c_f32_p]),
    ("zrh_forward_mixed", C.c_int, [c_void_pp, C.c_int, c_int_p, c_u32_p, c_u32_p, c_f32_p, c_f32_p]),
    ("zrh_stage_mixed", C.c_int, [c_void_pp, C.c_int, c_int_p, c_u32_p, c_void_pp]),
    ("zrh_cache_seq_len", C.c_int, [C.c_void_p]),
    ("zrh_sequence_position", C.c_int, [C.c_void_p]),
    ("zrh_logical_kv_tokens", C.c_int, [C.c_void_p]),
    ("zrh_base_position", C.c_int, [C.c_void_p]),
    ("zrh_live_kv_cache_bytes", C.c_uint64, [C.c_void_p]),
    ("zrh_allocated_pages", C.c_int, [C.c_void_p]),
    ("zrh_block_table", C.c_int, [C.c_void_p, c_u32_p, c_int_p, c_int_p, c_int_p, C.c_int]),
    ("zrh_export_kv", C.c_int, [C.c_void_p, C.c_int, c_f32_p, c_f32_p, c_int_p, c_int_p, c_int_p]),
    ("zrh_import_kv", C.c_int, [C.c_void_p, c_f32_p, c_f32_p, C.c_int, C.c_int, C.c_int]),
    ("zrh_export_kv_async", C.c_int, [C.c_void_p, C.c_int, c_f32_p, c_f32_p, c_int_p, c_int_p, c_int_p, c_void_pp]),
    ("zrh_import_kv_transfer", C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    ("zrh_export_kv_cbor", C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t), c_int_p,
                                     c_int_p]),
    ("zrh_import_kv_cbor", C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_int]),
    ("zrh_clear", None, [C.c_void_p]),
    ("zrh_release_pages", C.c_int, [C.c_void_p]),
    ("zrh_get_fast_path_context", C.c_int, [C.c_void_p, C.POINTER(FastPathContext)]),
    ("zrh_fast_path_plan_decode", C.c_int, [C.c_int, C.c_int, C.c_int, C.POINTER(FastPathPlan)]),
    ("zrh_fast_path_stage_decode", C.c_int, [C.POINTER(FastPathPlan), c_void_pp, C.c_int, c_u32_p, c_u32_p,
                                             c_u32_p, c_u32_p]),
    ("zrh_fast_path_plan_prefill", C.c_int, [C.c_int, C.POINTER(FastPathPlan)]),
    ("zrh_fast_path_stage_prefill_positions", C.c_int, [C.POINTER(FastPathPlan), C.c_uint64, C.c_int, c_u32_p]),
    ("zrh_fast_path_validate_decode_contexts", C.c_int, [C.POINTER(FastPathPlan), C.POINTER(FastPathBackendContext),
                                                         C.c_int]),
    ("zrh_decode_pipeline_create", C.c_int, [c_void_pp, C.c_int, c_u32_p, c_void_pp]),
    ("zrh_decode_pipeline_step", C.c_int, [C.c_void_p, c_u32_p, c_int_p]),
    ("zrh_decode_pipeline_finish", C.c_int, [C.c_void_p, c_u32_p]),
    ("zrh_decode_pipeline_info", C.c_int, [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(StepGraphStats)]),
    ("zrh_decode_pipeline_destroy", None, [C.c_void_p]),
    ("zrh_kv_reserve", C.c_int, [C.c_void_p, C.c_int]),
    ("zrh_retain_suffix", C.c_int, [C.c_void_p, C.c_int]),
]

_lib = None


def load():
    """Load libzip_rocm.so; raises if it has not been built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m mesh_amd.build` "
                              "(the rocm provider has no CPU fallback)")
        lib = C.CDLL(LIB_PATH)
        for name, restype, argtypes in SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(status: int, ctx=None) -> int:
    if status != ZR_OK:
        lib = load()
        msg = lib.zr_last_error(ctx) if ctx else lib.zr_global_last_error()
        raise ZrError(status, (msg or b"").decode(errors="replace"))
    return status
