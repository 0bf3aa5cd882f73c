// The rocm arm of the executor contract and provider contract descriptor
// (include/zip_rocm.h zr_get_executor_contract): what a Rust
// `ExecutionProviderKind::Rocm` arm reports, read from the library that
// implements it, so the stage -> kernel map cannot drift from the code.
#include <string.h>

#include "zr_internal.h"

namespace {

// FusedKernelStage (engine.rs:124-132) in contract order, snake_case as the
// reference serialises it, with the __global__ kernels of this library that
// implement each stage.
const char* const kStageNames[] = {"norm_qkv", "rope_kv_write", "paged_attention", "residual_mlp",
                                   "device_sampling"};
const char* const kStageKernels[] = {
    "rms_norm_vec_kernel,rms_norm_kernel,gemm_kernel",
    "rope_table_kernel,rope_kv_write_kernel,rope_kv_write_vec_kernel,paged_attention_kernel",
    "paged_attention_kernel,paged_prefill_attention_kernel,attention_merge_kernel",
    "rms_norm_vec_kernel,rms_norm_kernel,gemm_kernel,gemm_swiglu_ksplit_kernel,splitk_reduce_kernel",
    "argmax_partial_kernel,argmax_final_kernel,sample_kernel",
};
const char* const kHostKernels[] = {"host_assisted_sampling"};

}  // namespace

extern "C" zr_status zr_get_executor_contract(zr_executor_contract* out) {
    if (!out) return zr::set_global_err(ZR_E_INVALID, "null argument");
    memset(out, 0, sizeof *out);
    // LocalExecutorContract::for_provider (engine.rs:171-273), as the Cuda arm
    // (240-273) declares it, with prefill microbatches: chunked prefill rows
    // share the decode microbatch here (zrh_forward_mixed).
    out->executor_class = "fast_path";
    out->optimization_profile = "rocm_fused";
    out->n_host_kernels = 1;
    out->host_kernels = kHostKernels;
    out->n_fused_stages = 5;
    out->fused_stages = kStageNames;
    out->stage_kernels = kStageKernels;
    out->collective_residency = "staged_runtime";
    out->prefill_supports_microbatch = 1;
    out->prefill_requires_static_workspace = 1;
    out->prefill_uses_device_sampling = 1;
    out->decode_supports_microbatch = 1;
    out->decode_requires_static_workspace = 1;
    out->decode_uses_device_sampling = 1;
    out->kv_requires_paged_cache = 1;
    out->kv_append_only_decode = 1;
    out->kv_supports_prefill = 1;
    out->kv_supports_decode = 1;
    out->collective_tensors_per_layer = 2;
    // BackendContractDescriptor::for_provider (provider/mod.rs:88-150)
    out->provider = "rocm";
    out->compatibility_class = "rocm_fast_path";
    out->memory_model = "discrete_vram";
    out->supports_decode_microbatch = 1;
    out->supports_paged_kv = 1;
    out->supports_checkpoint_handoff = 1;
    out->supports_device_sampling = 1;
    out->fast_path_eligible = 1;
    // FastPathPlanner::capture_strategy (fast_path.rs:831-837): the fused profile replays
    out->capture_strategy = "replay_preferred";
    return ZR_OK;
}
