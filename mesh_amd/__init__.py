"""mesh_amd -- MI355X (gfx950) `rocm` execution provider for the zip engine.

The compute path is libzip_rocm.so (hand-written HIP kernels + C ABI,
include/zip_rocm.h); this package is its Python mirror of zip's provider
interface (mesh_amd.provider).
"""
from .provider import (BackendMicrobatchExecutor, DecodeMicrobatchOutput, DecodeMicrobatchRequest,
                       DecodePipeline, DeviceBuffer, DeviceContext, ExecutionProviderKind, FastPathPlanner, KVCacheBlob,
                       KVCacheSnapshot, KVCacheWireSnapshot, KVSequenceState, KVTransfer, ModelGeometry,
                       RocmExecutionBackend,
                       bf16_bits, device_info, executor_contract, probe_provider)

__all__ = ["BackendMicrobatchExecutor", "DecodeMicrobatchOutput", "DecodeMicrobatchRequest", "DecodePipeline",
           "DeviceBuffer",
           "DeviceContext", "ExecutionProviderKind", "FastPathPlanner", "KVCacheBlob", "KVCacheSnapshot",
           "KVCacheWireSnapshot", "KVSequenceState", "KVTransfer", "ModelGeometry", "RocmExecutionBackend", "bf16_bits",
           "device_info", "executor_contract", "probe_provider"]
