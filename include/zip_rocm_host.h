/*
 * zip_rocm_host.h -- host-side `rocm` execution backend over zip_rocm.h.
 *
 * The reference's provider host is Rust (agent/src/inference/backend.rs,
 * forward_pass.rs); this image has no Rust toolchain, so the same host logic
 * is C++ here with a C ABI: one zrh_backend is one session's
 * ProviderExecutionBackend (backend.rs:400-662) = ForwardPass position +
 * DeviceKVCache page tables (forward_pass.rs:899-1243).  The host owns the
 * page tables and positions; the GPU executes through zr_forward.
 *
 * Page tables reproduce the reference bit for bit: session-local page ids
 * with a LIFO free list, span block tables with a first-span start row after
 * retain_suffix, a sliding window of max_seq_len tokens.  Each local page is
 * bound to one global page of the KV pool when it is first allocated.
 */
#ifndef ZIP_ROCM_HOST_H
#define ZIP_ROCM_HOST_H

#include "zip_rocm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Global page allocator of a context's KV pool (LIFO).  initial_order
 * (nullable, n entries) is the initial free list; pages are popped from its
 * end.  NULL means pages come out 0, 1, 2, ...  With ctx == NULL the pool is
 * bookkeeping-only (n pages, no device): page tables, reserve and trim work,
 * compute and KV transfer calls fail with ZR_E_INVALID. */
typedef struct zrh_pool zrh_pool;
zr_status zrh_pool_create(zr_context* ctx, const int* initial_order, int n, zrh_pool** out);
void zrh_pool_destroy(zrh_pool* pool);
int zrh_pool_free_pages(const zrh_pool* pool);

typedef struct zrh_backend zrh_backend;
/* ForwardPass::from_residency (forward_pass.rs:1781-1824); the reference
 * hard-codes max_seq_len 4096 (1795), configs with longer contexts pass 8192. */
zr_status zrh_backend_create(zrh_pool* pool, int max_seq_len, zrh_backend** out);
void zrh_backend_destroy(zrh_backend* b); /* returns its global pages to the pool */

/* ForwardPass::prefill (2089-2112): clears the cache, keeps the last window.
 * logits [vocab] (nullable), greedy (nullable). */
zr_status zrh_prefill(zrh_backend* b, const uint32_t* tokens, int n, float* logits, uint32_t* greedy);
/* ForwardPass::decode_step (2115-2139). */
zr_status zrh_decode_step(zrh_backend* b, uint32_t token, float* logits, uint32_t* greedy);
/* BackendMicrobatchExecutor::decode_step_batch (backend.rs:110-151) on the
 * fast path: one fused microbatch over n sessions of one context.
 * out_tokens [n] greedy, out_logits [n, vocab], out_partials
 * [layers][2][n][hidden] -- each nullable. */
zr_status zrh_decode_step_batch(zrh_backend* const* backends, int n, const uint32_t* tokens, uint32_t* out_tokens,
                                float* out_logits, float* out_partials);
/* decode_step_batch with per-request sampling (DecodeMicrobatchRequest
 * temperature / top_p / sampling_seed, backend.rs:90-105): the fused step,
 * then sample_fast_path_logits_batch (275-316) on the step's device logits
 * (zr_sample semantics; rows with temperature <= 0 or top_p <= 0 keep the
 * argmax).  out_tokens is required.  If sampling fails after the step, the
 * sessions have advanced (the step is not rolled back), as in the reference. */
zr_status zrh_decode_step_batch_sampled(zrh_backend* const* backends, int n, const uint32_t* tokens,
                                        const float* temperature, const float* top_p, const uint64_t* seeds,
                                        uint32_t* out_tokens, float* out_logits, float* out_partials);
/* Mixed chunked-prefill + decode microbatch: session i appends q_len[i]
 * tokens at its current position (tokens packed back to back); logits come
 * from the last row of every session. */
zr_status zrh_forward_mixed(zrh_backend* const* backends, int n, const int* q_len, const uint32_t* tokens,
                            uint32_t* out_tokens, float* out_logits, float* out_partials);
/* Same bookkeeping as zrh_forward_mixed but only stages the microbatch for
 * device-resident replay (zr_forward_staged_async); positions advance. */
zr_status zrh_stage_mixed(zrh_backend* const* backends, int n, const int* q_len, const uint32_t* tokens,
                          zr_staged** out);

int zrh_cache_seq_len(const zrh_backend* b);
int zrh_sequence_position(const zrh_backend* b);
int zrh_logical_kv_tokens(const zrh_backend* b);
int zrh_base_position(const zrh_backend* b);
uint64_t zrh_live_kv_cache_bytes(const zrh_backend* b);
int zrh_allocated_pages(const zrh_backend* b);
/* LiveKVBlockTable of the session (kv_cache.rs:325-438): spans in
 * session-local page ids, plus the global pool page of each span.  Returns
 * the span count (or <0); arrays may be NULL to query the count. */
int zrh_block_table(const zrh_backend* b, uint32_t* page_ids, int* start_tokens, int* token_counts,
                    int* global_pages, int capacity);

/* export_kv_cache (forward_pass.rs:2442-2448 -> 1169-1204) with the segmented
 * retention window: the newest min(seq_len, max(max_cached_tokens, 1)) rows
 * (all rows if max_cached_tokens < 0) gathered from the pool, f32
 * [layers][rows][kv_cols].  *rows = 0 means no snapshot (empty cache). */
zr_status zrh_export_kv(const zrh_backend* b, int max_cached_tokens, float* k, float* v, int* rows,
                        int* base_position, int* next_position);
/* import_kv_cache (2450-2454 -> 1206-1242): clears, scatters the rows into
 * fresh pages, validates cached_tokens and base_position. */
zr_status zrh_import_kv(zrh_backend* b, const float* k, const float* v, int rows, int base_position,
                        int next_position);
/* zrh_export_kv with its copy to k / v in flight (zr_kv_gather_async): the
 * session's pages may be released once this returns; k / v (pinned host
 * memory) hold the rows after zr_transfer_wait(*out).  *out = NULL when there
 * is no snapshot (empty cache). */
zr_status zrh_export_kv_async(const zrh_backend* b, int max_cached_tokens, float* k, float* v, int* rows,
                              int* base_position, int* next_position, zr_transfer** out);
/* zrh_import_kv from a transfer's device buffer (zr_kv_scatter_transfer): an
 * upload (zr_kv_upload_async) or a session's own in-flight export. */
zr_status zrh_import_kv_transfer(zrh_backend* b, zr_transfer* t, int rows, int base_position, int next_position);
/* export_kv_cache -> export_snapshot (forward_pass.rs:1169-1204) as its wire
 * bytes: the KVCacheSnapshot blob (KVCacheBlob::from_cache, kv_cache.rs:77-84,
 * encoding FullSnapshotCbor) = KVCache::to_bytes (880-887) of the newest
 * min(seq_len, max(max_cached_tokens, 1)) rows (all if < 0).  The sequence
 * state goes to *next_position / *cached_tokens (KVSequenceState, 20-26).
 * Empty cache: *out_len = 0, no document (export_snapshot returns None).
 * out == NULL: size query; capacity short: ZR_E_INVALID with *out_len set. */
zr_status zrh_export_kv_cbor(const zrh_backend* b, int max_cached_tokens, uint8_t* out, size_t capacity,
                             size_t* out_len, int* next_position, int* cached_tokens);
/* import_kv_cache -> import_snapshot (1206-1242) from the wire bytes:
 * KVCacheSnapshot::decode_cache (kv_cache.rs:115-141) checks the document
 * against the sequence state (cached_tokens, first cached position), then the
 * rows are scattered into fresh pages as zrh_import_kv does. */
zr_status zrh_import_kv_cbor(zrh_backend* b, const uint8_t* bytes, size_t len, int next_position,
                             int cached_tokens);
/* ForwardPass::clear_cache (2423-2426). */
void zrh_clear(zrh_backend* b);
/* Eviction under KV pressure: every global page bound to the session goes
 * back to the pool; the session restarts empty at position 0. */
zr_status zrh_release_pages(zrh_backend* b);

/* ------------------------------------------------------ fast-path planner --- */
/* FastPathBackendContext (fast_path.rs:102-108) of one session, as
 * ProviderRuntimeCore::fast_path_context builds it (backend.rs:748-755).  The
 * provider ("rocm") and profile ("rocm_fused") are the contract's
 * (zr_get_executor_contract); the model id is the caller's. */
typedef struct {
    int logical_kv_tokens;     /* ForwardPass::logical_kv_tokens */
    int position;              /* next absolute position (DecodeSlotState.position) */
    int cached_tokens;         /* rows in the live window (DecodeSlotState::sequence_len) */
    int decode_token_ceiling;  /* FastPathPlanner::decode_token_ceiling_for_context (676-683); -1: none */
} zrh_fast_path_context;
zr_status zrh_get_fast_path_context(const zrh_backend* b, zrh_fast_path_context* out);

/* FastPathPlanner::plan_decode (fast_path.rs:644-669) for the rocm_fused
 * profile: the first bucket of DECODE_BUCKET_BATCHES x DECODE_BUCKET_KV_TOKENS
 * (15-16) that holds batch_size and total_kv_tokens, with the metadata layout
 * of metadata_fields (839-867): four u32 fields back to back,
 * slot_sequence_lengths[B], slot_positions[B], slot_block_tables[B][page_slots]
 * and slot_mapping[B] (B = batch_size_ceiling, page_slots =
 * ceil(token_ceiling / 16)), and workspace_requirements (869-890) with the
 * fused-profile constants.  A batch no bucket holds is ZR_E_UNSUPPORTED with
 * FastPathInvariantError::UnsupportedBucket's text (146-157); the 256-session
 * step is such a batch and runs without a plan (backend.rs:116-126). */
typedef struct {
    int batch_size_ceiling, token_ceiling;
    int actual_batch_size, actual_token_count, max_sequence_len;
    int page_slots;
    size_t field_offset[4], field_bytes[4]; /* the four metadata fields, in order */
    size_t metadata_bytes;
    size_t workspace_bytes, workspace_alignment;
    char bucket_label[64];                  /* "decode-b{B}-kv{T}-rocm" / "prefill-t{T}-rocm" */
    int phase;                              /* ExecutionPhase: 0 decode, 1 prefill */
    char capture_strategy[24];              /* FastPathPlanner::capture_strategy (831-837): "replay_preferred" */
    char prefill_strategy[32];              /* "single_sequence_buckets" (prefill plans), "" (decode) */
    /* BucketMetadataLayout::layout_hash (892-902) of the bucket key (phase,
     * provider "rocm", profile "rocm_fused", both ceilings) and the fields
     * (name, element size, count, stride).  The reference hashes with Rust's
     * DefaultHasher, a process-local value that never leaves the process; this
     * library hashes the same items with FNV-1a 64 (each integer as 8
     * little-endian bytes, each name's bytes then 0xff).  The value only has
     * to match the plan it was computed for (the drift check). */
    uint64_t layout_hash;
} zrh_fast_path_plan;
zr_status zrh_fast_path_plan_decode(int batch_size, int total_kv_tokens, int max_sequence_len,
                                    zrh_fast_path_plan* out);
/* FastPathPlanner::plan_prefill (fast_path.rs:680-702): the first bucket of
 * PREFILL_BUCKET_TOKENS (17: 128, 512, 2048, 8192, 16384; batch ceiling 1)
 * holding prompt_tokens, built as plan_decode builds its plan (metadata
 * fields over one slot, workspace_requirements, capture strategy) with
 * prefill_strategy SingleSequenceBuckets.  A prompt longer than every bucket
 * is ZR_E_UNSUPPORTED with UnsupportedBucket's text; the coordinator plans
 * a prefill so when the request permits the fast path (coordinator.rs:2164-2172). */
zr_status zrh_fast_path_plan_prefill(int prompt_tokens, zrh_fast_path_plan* out);
/* PrefillWorkspaceLease::stage_positions (fast_path.rs:409-445), which
 * ForwardPass::forward_tokens calls for a leased prefill (forward_pass.rs:2470-2476):
 * resets the lease's positions (plan->token_ceiling words) and writes
 * absolute_position_start + i for i < token_count.  A count beyond the ceiling
 * is CaptureUnsafe ("prefill token count {n} exceeds bucket ceiling {T}"), a
 * position beyond u32 "prefill absolute position exceeded u32 addressable
 * range" (ZR_E_INVALID). */
zr_status zrh_fast_path_stage_prefill_positions(const zrh_fast_path_plan* plan, uint64_t absolute_position_start,
                                                int token_count, uint32_t* positions);
/* FastPathBackendContext (fast_path.rs:102-108) of any provider's backend,
 * as ExecutionBackend::fast_path_context reports it (backend.rs:748-755):
 * ExecutionProviderKind and BackendOptimizationProfile as the reference
 * serialises them ("rocm" / "rocm_fused", "cpu" / "cpu_serial", "cuda" /
 * "cuda_fused", "metal" / "metal_vectorized"), the model id (nullable). */
typedef struct {
    const char* provider;
    const char* optimization_profile;
    const char* model_id;
    int logical_kv_tokens;
} zrh_fast_path_backend_context;
/* FastPathPlanner::validate_decode_contexts (fast_path.rs:704-778), which
 * BackendMicrobatchExecutor::decode_step_batch runs before a planned batch
 * (backend.rs:116-123): the request count equals the plan's batch, every
 * context is the plan's provider and profile, fits the bucket's token
 * ceiling and shares one model id, and the plan's layout hash matches its
 * bucket and fields.  Errors carry CaptureUnsafe / MetadataDrift texts
 * (ZR_E_INVALID). */
zr_status zrh_fast_path_validate_decode_contexts(const zrh_fast_path_plan* plan,
                                                 const zrh_fast_path_backend_context* contexts, int n);

/* DecodeWorkspaceLease::stage (fast_path.rs:263-338) over the slot states of
 * n sessions (DeviceKVCache::decode_slot_state, forward_pass.rs:1065-1074):
 * resets `metadata` (plan->metadata_bytes) and writes the sequence lengths,
 * positions, live block tables (session page ids; unused slots u32::MAX) and
 * slot indices (unused slots u32::MAX); token_ids / positions (nullable,
 * batch_size_ceiling words each) receive the lease's token and position
 * buffers (zero beyond n).  Errors carry the CaptureUnsafe texts (158-164). */
zr_status zrh_fast_path_stage_decode(const zrh_fast_path_plan* plan, zrh_backend* const* backends, int n,
                                     const uint32_t* tokens, uint32_t* metadata, uint32_t* token_ids,
                                     uint32_t* positions);

/* ---------------------------------------------------- decode pipeline --- */
/* The serving loop of BackendMicrobatchExecutor::decode_step_batch
 * (backend.rs:110-151) over a fixed set of n sessions, pipelined.  Each
 * zrh_decode_pipeline_step does the step's host bookkeeping (window trim and
 * page reservation per session, as zrh_decode_step_batch), launches it through
 * a zr_step_graph (one captured graph per bucket, replayed with the step's
 * metadata) and returns the greedy ids of the previous step, waiting for that
 * step only: the host work of step k + 1 overlaps step k on the device.  Ids
 * stay on the device between steps: step 0 reads first_tokens, step k the ids
 * of step k - 1.  Positions advance as each step is enqueued.  A step that
 * fails to enqueue leaves its sessions as they were (steps already enqueued
 * run).  zrh_decode_pipeline_finish waits for the last step and returns its
 * ids.  The sessions must not be used elsewhere while the pipeline lives. */
typedef struct zrh_decode_pipeline zrh_decode_pipeline;
zr_status zrh_decode_pipeline_create(zrh_backend* const* backends, int n, const uint32_t* first_tokens,
                                     zrh_decode_pipeline** out);
/* prev_tokens [n] (nullable) receives the previous step's ids when *prev_ready = 1. */
zr_status zrh_decode_pipeline_step(zrh_decode_pipeline* p, uint32_t* prev_tokens, int* prev_ready);
zr_status zrh_decode_pipeline_finish(zrh_decode_pipeline* p, uint32_t* last_tokens);
zr_status zrh_decode_pipeline_info(const zrh_decode_pipeline* p, uint64_t* steps, zr_step_graph_stats* graph);
void zrh_decode_pipeline_destroy(zrh_decode_pipeline* p);

/* Page-table state machine without compute, for allocator checks:
 * DeviceKVCache::append_layer over all layers (rows appended, window trim
 * included) and DeviceKVCache::retain_suffix. */
zr_status zrh_kv_reserve(zrh_backend* b, int rows);
zr_status zrh_retain_suffix(zrh_backend* b, int keep_rows);

#ifdef __cplusplus
}
#endif
#endif
