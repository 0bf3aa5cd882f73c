/*
 * zip_rocm.h -- C ABI of the MI355X (gfx950) execution provider for zip.
 *
 * This is the thin FFI a `rocm` arm of zip's provider abstraction binds
 * (agent/src/inference/backend.rs:30-88 ExecutionBackend, provider/mod.rs:8-33
 * ExecutionProviderKind).  The host keeps ownership of scheduling and of the
 * paged-KV page tables; every call here executes one worker's share of the
 * forward pass on one GPU with hand-written CDNA4 kernels.
 *
 * Conventions
 *  - Every function returns zr_status (0 = ok).  Failures never abort: the
 *    message is kept per context (zr_last_error) or per thread
 *    (zr_global_last_error) -- the AgentError::Execution / Config split of
 *    agent/src/errors.rs:19-36.
 *  - Plain pointers and sizes only.  "host" arrays are ordinary CPU memory;
 *    "device" pointers come from zr_device_alloc.  Weight uploads accept either.
 *  - One context = one device + one HIP stream; calls on a context are
 *    serialised by the caller (the reference drives a backend through &mut
 *    self from one task, coordinator.rs:2291-2306).  Entry points are
 *    synchronous at return unless named *_async.
 *  - Weights are bf16 bit patterns in the reference's row-major [in, out]
 *    layout (x @ W, forward_pass.rs:89-114); norms are f32.
 *  - The KV pool is global pages of `page_tokens` (16) rows for K and V of
 *    every layer; a page id in a block table indexes all layers
 *    (page tables are per-layer identical, forward_pass.rs:1024-1047).
 */
#ifndef ZIP_ROCM_H
#define ZIP_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int zr_status;
#define ZR_OK 0
#define ZR_E_INVALID (-1)     /* bad argument / shape (AgentError::Execution) */
#define ZR_E_OOM (-2)         /* device or pool memory exhausted */
#define ZR_E_HIP (-3)         /* HIP runtime failure */
#define ZR_E_INVARIANT (-4)   /* page-table / position invariant violated */
#define ZR_E_UNSUPPORTED (-5) /* geometry the kernels do not cover */
#define ZR_E_NODEVICE (-6)    /* no gfx950 device */

#define ZR_DTYPE_F32 0
#define ZR_DTYPE_BF16 1

/* zr_model_desc.flags */
#define ZR_FLAG_SPLIT_ACTIVATIONS 1 /* GEMM A operands as bf16 hi+lo pairs (~fp32) */

/* ------------------------------------------------------------- device --- */
typedef struct {
    int device_count;
    int device;          /* the device described below */
    int compute_units;
    int clock_mhz;
    uint64_t hbm_bytes;
    char arch[64];       /* e.g. "gfx950:sramecc+:xnack-" */
} zr_device_info;

/* runtime.rs:335-385 probe_provider: reports the device, ZR_E_NODEVICE if the
 * selected device is not gfx950. */
zr_status zr_probe(int device, zr_device_info* out);
const char* zr_global_last_error(void);

/* ------------------------------------------------------------ context --- */
typedef struct {
    int hidden, num_heads, num_kv_heads, num_layers, vocab;
    int ffn_cols;                 /* this shard's FFN columns (partition_columns) */
    int shard_start, shard_end;   /* this shard's q-column range (forward_pass.rs:1257) */
    float rms_norm_eps, rope_base;
    int page_tokens;              /* 16 (kv_cache.rs:214) */
    int kv_dtype;                 /* ZR_DTYPE_BF16 or ZR_DTYPE_F32 */
    int max_tokens;               /* rows of one microbatch (sum of q_len) */
    int max_seqs;                 /* sequences of one microbatch */
    int max_pages_per_seq;        /* block-table width */
    int flags;
} zr_model_desc;

typedef struct zr_context zr_context;

/* ForwardPass::from_residency / SharedModelResidency::from_host
 * (forward_pass.rs:1725-1824): validates the shard geometry with the rules of
 * resolve_attention_shard_layout and allocates activations on `device`. */
zr_status zr_context_create(const zr_model_desc* desc, int device, zr_context** out);
void zr_context_destroy(zr_context* ctx);
const char* zr_last_error(const zr_context* ctx);
/* Local q-head -> local kv-head map (build_local_kv_head_indices 2951-2970). */
zr_status zr_kv_head_map(const zr_context* ctx, uint32_t* out, int capacity, int* count);

/* ------------------------------------------------------------ weights --- */
typedef struct {
    const uint16_t* w_q;     /* [hidden, q_cols]  bf16 */
    const uint16_t* w_k;     /* [hidden, kv_cols] */
    const uint16_t* w_v;     /* [hidden, kv_cols] */
    const uint16_t* w_o;     /* [q_cols, hidden] */
    const uint16_t* w_gate;  /* [hidden, ffn_cols] */
    const uint16_t* w_up;    /* [hidden, ffn_cols] */
    const uint16_t* w_down;  /* [ffn_cols, hidden] */
    const float* attn_norm;  /* [hidden] */
    const float* mlp_norm;   /* [hidden] */
} zr_layer_weights;

/* DeviceModelWeights::from_host (forward_pass.rs:1560-1591): w_qkv = [q|k|v]
 * and w_gate_up = [gate|up] column concatenations, repacked into the MFMA
 * fragment layout.  Pointers may be host or device memory. */
zr_status zr_upload_layer(zr_context* ctx, int layer, const zr_layer_weights* w);
zr_status zr_upload_globals(zr_context* ctx, const uint16_t* embedding /* [vocab, hidden] */,
                            const float* final_norm /* [hidden] */,
                            const uint16_t* lm_head /* [hidden, vocab] */);

/* ------------------------------------------------------------ KV pool --- */
/* Allocates n_pages global pages (zero-filled).  Page p of layer l holds K and
 * V for 16 token rows of every local kv head. */
zr_status zr_kv_pool_create(zr_context* ctx, int n_pages);
int zr_kv_pool_pages(const zr_context* ctx);
uint64_t zr_kv_pool_bytes(const zr_context* ctx);

/* ------------------------------------------------------- microbatches --- */
/* One ragged microbatch: decode rows (q_len 1) and prefill chunks (q_len > 1)
 * packed into one varlen token tensor.  All arrays are host memory.
 * Sequence s appends q_len[s] rows after kv_before[s] cached rows (the live
 * window after the sliding-window trim); its first new token has absolute
 * position first_pos[s].  block_tables[s] lists the global pages of the live
 * window AFTER the append, oldest first; the window starts at row
 * first_offset[s] of the first page (a span trimmed by retain_suffix). */
typedef struct {
    int num_seqs;
    const int* q_len;
    const int* kv_before;
    const int* first_pos;
    const int* first_offset;
    const int* block_tables;   /* [num_seqs][block_table_stride] */
    int block_table_stride;
    const uint32_t* tokens;    /* [sum q_len]; may be NULL for staged runs fed on device */
} zr_microbatch;

/* Runs embed -> num_layers x (norm, QKV, RoPE+KV write, paged attention, O,
 * residual, norm, gate_up+SwiGLU, down, residual) -> final norm -> LM head on
 * the last row of every sequence -> greedy argmax
 * (fast_path_decode_microbatch, forward_pass.rs:2143-2319).  Outputs are host
 * arrays, each nullable: out_tokens [num_seqs] greedy ids (first index on
 * ties), out_logits [num_seqs, vocab] f32, out_partials
 * [num_layers][2][sum q_len][hidden] f32 = per-layer pre-all-reduce
 * (o_partial, down_partial) (forward_pass.rs:2265, 2290).  A decode
 * microbatch (one row per sequence, MFMA page layout) asking for out_tokens
 * only is replayed from the context's step graph once its sequence count has
 * run three calls in a row: the same kernels on the same metadata as the
 * eager pass, so the same ids bit for bit, without its per-kernel launches
 * (zr_forward_replay_info). */
zr_status zr_forward(zr_context* ctx, const zr_microbatch* mb, uint32_t* out_tokens,
                     float* out_logits, float* out_partials);

/* Device-resident variant: metadata staged once into device memory.  Every
 * entry below that takes a zr_staged returns ZR_E_INVALID ("staged
 * microbatch of another context") for one staged by another context. */
typedef struct zr_staged zr_staged;
zr_status zr_stage(zr_context* ctx, const zr_microbatch* mb, zr_staged** out);
void zr_staged_destroy(zr_staged* st);
/* Enqueues the forward pass on the context stream without synchronising.
 * d_tokens: device [sum q_len] input ids, or NULL to use the staged ids.
 * d_out_tokens: device [num_seqs] greedy ids (may be d_tokens of a later
 * decode step); d_out_logits nullable device [num_seqs, vocab].
 * Ids fed from device memory are checked on the device (host ids are checked
 * when staged): the next zr_synchronize returns ZR_E_INVALID with
 * "Token {id} out of vocabulary bounds {vocab}" for the first bad id
 * (embed_tokens, tensor_ops.rs:482-490).  That microbatch's outputs and the
 * KV rows it appended are then meaningless; nothing is read out of bounds. */
zr_status zr_forward_staged_async(zr_context* ctx, zr_staged* st, const uint32_t* d_tokens,
                                  uint32_t* d_out_tokens, float* d_out_logits);
/* Waits for the context stream; reports a device-fed id error (above). */
zr_status zr_synchronize(zr_context* ctx);
/* Replay of a staged step (GraphCaptureStrategy::ReplayPreferred, the fused
 * profile's capture strategy, fast_path.rs:831-837): records exactly what
 * zr_forward_staged_async(ctx, st, d_tokens, d_out_tokens, d_out_logits)
 * enqueues -- kernels and, for device-fed ids, the id-check copy; no memset
 * or allocation -- into a HIP graph on the context stream.  zr_graph_launch
 * enqueues the recorded step again (same staged metadata and buffers, which
 * must stay alive), with the same id check at the next zr_synchronize.
 * Capture is refused while per-class timing is on (events recorded by graph
 * nodes do not time).  A graph holds the addresses of the context's buffers
 * too: once one of them has been reallocated (a workspace grown for a larger
 * microbatch, the KV pool re-created, weights uploaded again), zr_graph_launch
 * returns ZR_E_INVALID for graphs captured before; capture again.  Destroy a
 * graph before its context. */
typedef struct zr_graph zr_graph;
zr_status zr_graph_capture_staged(zr_context* ctx, zr_staged* st, const uint32_t* d_tokens,
                                  uint32_t* d_out_tokens, float* d_out_logits, zr_graph** out);
zr_status zr_graph_launch(zr_context* ctx, zr_graph* g);
void zr_graph_destroy(zr_graph* g);

/* A decode step replayed across steps: the fused profile's ReplayPreferred
 * capture (fast_path.rs:831-837) over a bucket workspace that is re-staged
 * every step (DecodeWorkspaceLease, fast_path.rs:263-338, 542-571).  One HIP
 * graph (the pack stage and the forward pass) is captured per bucket -- the
 * sequence count and room for the step's attention work list -- and replayed
 * for every later step that fits it, each launch carrying that step's
 * metadata.  A launch stages the microbatch into a pinned host buffer, copies
 * it into the graph's own device buffers on a copy stream of its own, replays
 * the graph on the context stream and, with h_out_tokens (pinned host memory,
 * nullable), copies the step's greedy ids back.  Two buffer sets alternate, so
 * the host staging of the next step overlaps this one on the device; nothing
 * is allocated per step and no graph holds a memset.  Only decode microbatches
 * of one row per sequence (MFMA page layout); a microbatch that outgrows its
 * bucket gets a new one (synchronously).  d_tokens / d_out_tokens: device
 * [num_seqs] ids in and out (a captured graph per pair; the ids are checked
 * as in zr_forward_staged_async, at the next zr_synchronize).  The outputs
 * are ready after zr_synchronize (or an event the caller records on the
 * stream).  Not with per-class timing on. */
typedef struct zr_step_graph zr_step_graph;
typedef struct {
    uint64_t launches;
    int captures, buckets, sequences;
    int items_capacity, merge_capacity, fused_rope;
    size_t metadata_bytes;   /* staged per step (H2D) */
} zr_step_graph_stats;
zr_status zr_step_graph_create(zr_context* ctx, zr_step_graph** out);
zr_status zr_step_graph_launch(zr_step_graph* g, const zr_microbatch* mb, const uint32_t* d_tokens,
                               uint32_t* d_out_tokens, uint32_t* h_out_tokens);
zr_status zr_step_graph_info(const zr_step_graph* g, zr_step_graph_stats* out);
void zr_step_graph_destroy(zr_step_graph* g);
/* Diagnostic, no counterpart in the reference: the step graph that
 * zr_forward replays decode steps from (one row per sequence, MFMA page
 * layout, greedy ids only -- no logits or partials -- once the same sequence
 * count has run three calls in a row; ZR_FORWARD_REPLAY=0 keeps zr_forward
 * eager).  Zeros before the first replay. */
zr_status zr_forward_replay_info(const zr_context* ctx, zr_step_graph_stats* out);

/* ------------------------------------------------------ op-level entries --- */
/* Ragged packing on the GPU: device outputs cu_q/cu_k [num_seqs+1],
 * positions/slot_mapping/seq_ids [sum q_len] (host arrays, copied back). */
zr_status zr_pack(zr_context* ctx, const zr_microbatch* mb, int* cu_q, int* cu_k, int* positions,
                  int* slot_mapping, int* seq_ids);
/* RoPE on q and k + KV append (the RopeKvWrite stage): d_qkv device
 * [sum q_len, q_cols + 2*kv_cols] f32 projection output; writes RoPE'd q to
 * d_q_out [sum q_len, q_cols] and RoPE'd k / v into the pool at the staged
 * slot mapping for `layer`.  rope=0 skips the rotation (append only). */
zr_status zr_rope_kv_write(zr_context* ctx, zr_staged* st, int layer, const float* d_qkv,
                           float* d_q_out, int rope);
/* GQA paged attention (decode rows and causal chunked prefill) over the
 * staged microbatch for `layer`: d_q device [sum q_len, q_cols] f32 (RoPE'd),
 * d_out device [sum q_len, q_cols] f32. */
zr_status zr_attention(zr_context* ctx, zr_staged* st, int layer, const float* d_q, float* d_out);
/* Diagnostic, no counterpart in the reference: the HBM rate the decode
 * attention launch's access pattern can reach.  Launches `repeats` times
 * (1..10000) a read-only copy of that launch's page stream for the staged
 * microbatch at `layer` -- the same grid, work records, block tables and
 * 16-byte nontemporal page loads in the same order, without Q, softmax, MFMA
 * or output -- and returns the mean launch time in *mean_ms (HIP events on
 * the context stream; synchronises).  Needs the MFMA page layout (head_dim 64
 * or 128) and decode attention items in `st`.  For a bench or a profiler:
 * dividing the launch's K/V bytes by it gives the ceiling that the attention
 * kernel's own rate is measured against. */
zr_status zr_kv_read_probe(zr_context* ctx, zr_staged* st, int layer, int repeats, double* mean_ms);
/* The RopeKvWrite and Attention stages in one launch, for a staged
 * microbatch whose sequences each have one query row (decode; the MFMA page
 * layout): d_qkv as for zr_rope_kv_write, d_out as for zr_attention.  The
 * same q, K / V rows and outputs as zr_rope_kv_write + zr_attention, bit for
 * bit; the forward pass takes this path for such microbatches.  Other
 * microbatches: ZR_E_UNSUPPORTED.  (The RopeKvWrite and PagedAttention stages
 * of FusedKernelStage, engine.rs:124-132; RoPE tensor_ops.rs:509-560, append
 * forward_pass.rs:462-521, attention forward_pass.rs:2838-2895.) */
zr_status zr_rope_attention(zr_context* ctx, zr_staged* st, int layer, const float* d_qkv, float* d_out,
                            int rope);
/* Checkpoint KV handoff gather (build_active_tensors + retain_suffix window,
 * forward_pass.rs:633-680, 1169-1204): rows [first_row, first_row + n_rows)
 * of one sequence's live window, all layers, into dst_k/dst_v
 * [num_layers][n_rows][kv_cols] f32 (host or device memory). */
zr_status zr_kv_gather(zr_context* ctx, const int* block_table, int n_pages, int first_offset,
                       int first_row, int n_rows, float* dst_k, float* dst_v);
/* Snapshot import scatter (import_snapshot, forward_pass.rs:1206-1242):
 * writes rows [0, n_rows) of src_k/src_v [num_layers][n_rows][kv_cols] f32 at
 * logical rows first_row.. of the window described by block_table. */
zr_status zr_kv_scatter(zr_context* ctx, const int* block_table, int n_pages, int first_offset,
                        int first_row, int n_rows, const float* src_k, const float* src_v);

/* ---- KV windows in flight: zr_kv_gather / zr_kv_scatter with the PCIe copy
 * on a stream of its own (one per direction), overlapping the decode steps --
 * the eviction checkpoint and restore of the KV-pressure path (coordinator.rs
 * 871-894, forward_pass.rs:1169-1242 export / import), whose copies the
 * reference makes synchronously.  A transfer owns a device buffer
 * [num_layers][n_rows][kv_cols] K, then V (reused after destroy, never freed
 * before the context).  Host buffers should be pinned (zr_host_alloc) for the
 * copies to overlap.  One host thread per context. */
typedef struct zr_transfer zr_transfer;
/* The gather of zr_kv_gather on the context's stream into the transfer's
 * buffer, then the copy to dst_k / dst_v on the device-to-host stream.
 * Returns at once: the window's pages may be reused as soon as this returns
 * (later launches on the context's stream run after the gather); dst_k /
 * dst_v are valid after zr_transfer_wait. */
zr_status zr_kv_gather_async(zr_context* ctx, const int* block_table, int n_pages, int first_offset,
                             int first_row, int n_rows, float* dst_k, float* dst_v, zr_transfer** out);
/* Copies src_k / src_v [num_layers][n_rows][kv_cols] f32 into a transfer's
 * buffer on the host-to-device stream (a restore, issued ahead of it). */
zr_status zr_kv_upload_async(zr_context* ctx, const float* src_k, const float* src_v, int n_rows,
                             zr_transfer** out);
/* zr_kv_scatter from a transfer's buffer, on the context's stream: after its
 * upload (waited for on the device), or straight from a gather's buffer (its
 * rows are on the device; its copy to the host may still be running).
 * n_rows must be the transfer's. */
zr_status zr_kv_scatter_transfer(zr_context* ctx, zr_transfer* t, const int* block_table, int n_pages,
                                 int first_offset, int first_row, int n_rows);
/* Only the pages the rows touch are copied with the transfer, so
 * block_table may be the session's whole table (n_pages entries). */
/* 1 when the transfer's host copy has finished, 0 while it runs, <0 on error. */
int zr_transfer_done(const zr_transfer* t);
zr_status zr_transfer_wait(zr_transfer* t);
/* Waits for the copy and the last kernel on the buffer, keeps the buffer for
 * reuse (the 8 largest finished buffers are kept; a transfer that fits none
 * frees the smaller ones, and all of them before one retry when device memory
 * runs out).  Destroy every transfer before its context.  No reference
 * counterpart: the reference copies synchronously (forward_pass.rs:1169-1242). */
void zr_transfer_destroy(zr_transfer* t);
/* Bytes of device memory the context keeps in finished transfers' buffers. */
size_t zr_transfer_cached_bytes(const zr_context* ctx);
/* KV snapshot wire format (KVCache::to_bytes, kv_cache.rs:880-887: ciborium
 * 0.2.2 CBOR of the cache DeviceKVCache::export_snapshot builds,
 * forward_pass.rs:1169-1204): gathers rows [first_row, first_row + n_rows)
 * like zr_kv_gather and encodes the document on the device.  base_position is
 * the absolute position of the first exported row; the config map holds this
 * context's layers, the model's kv heads, head_dim and cfg_max_seq_len.
 * out == NULL: only *out_len.  capacity < the document: ZR_E_INVALID with
 * *out_len set.  out is host memory (pinned for full-rate copies). */
zr_status zr_kv_export_cbor(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                            int n_rows, long long base_position, int cfg_max_seq_len, uint8_t* out, size_t capacity,
                            size_t* out_len);
/* Raw page access for bit-exact checks: copies `n_pages` pages of `layer`
 * (K then V, pool dtype, pool layout) into host memory. */
zr_status zr_kv_read_pages(zr_context* ctx, int layer, const int* pages, int n_pages, void* dst);
/* Greedy argmax over rows of a device [rows, cols] f32 matrix (first index on
 * ties; runtime.rs:561-570). */
zr_status zr_argmax(zr_context* ctx, const float* d_x, int rows, int cols, uint32_t* d_out);
/* zr_argmax without allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * fixed-footprint serving loops, harnesses that forbid hipMalloc).  The
 * argmax partials go to a fixed 256 KiB device array of the library (each GPU
 * holds its own copy for the life of the process) instead of the context's
 * workspace, so rows * ceil(cols / 4096) <= 32768 (e.g. 256 rows of 128256
 * logits use 8192); larger inputs return ZR_E_INVALID.  Enqueued on the
 * context stream without synchronising (d_out is ready after
 * zr_synchronize).  Every call on one GPU shares that array: calls that
 * overlap on one GPU (other contexts' streams) race. */
zr_status zr_argmax_noalloc(zr_context* ctx, const float* d_x, int rows, int cols, uint32_t* d_out);
/* Stochastic sampling of device logits [rows, cols] f32, per row with its own
 * temperature, top_p and seed (host arrays): sample_tokens_device_with_seeds
 * (runtime.rs:534-601) as the batched decode path groups it
 * (sample_fast_path_logits_batch, backend.rs:275-316).  temperature <= 0 or
 * top_p <= 0: argmax.  Cumulative sums are exact integer sums of
 * round(exp(y - max) * 2^36) compared with exact integer targets
 * (deterministic; the reference's candle reduction orders are unspecified).
 * cols <= 2^20 (ZR_E_INVALID otherwise).  d_out: device u32 [rows]. */
zr_status zr_sample(zr_context* ctx, const float* d_logits, int rows, int cols, const float* temperature,
                    const float* top_p, const uint64_t* seeds, uint32_t* d_out);
/* The same on the logits of the context's last forward (its first `rows`
 * rows, one per sequence of that microbatch); tokens to host memory.  For
 * ProviderRuntimeCore::sample (forward_pass.rs:2046-2086) on device logits
 * and the batched decode path. */
zr_status zr_sample_last_logits(zr_context* ctx, int rows, const float* temperature, const float* top_p,
                                const uint64_t* seeds, uint32_t* out_tokens);
/* y = rms_norm(x) * gamma (tensor_ops.rs:285-304), device f32 [rows, cols]. */
zr_status zr_rms_norm(zr_context* ctx, const float* d_x, const float* d_gamma, float* d_y, int rows,
                      int cols);
/* C[M,N] = A[M,K] @ W[K,N] with W bf16 [K,N] (host or device, reference
 * layout), A/C device f32 -- the shard projection GEMM on MFMA. */
zr_status zr_gemm(zr_context* ctx, const float* d_a, const uint16_t* w, float* d_c, int m, int n,
                  int k);
/* H[M,F] = silu(A @ Wg) * (A @ Wu) (runtime.rs:927-929 silu_device and the
 * broadcast_mul at forward_pass.rs:2286-2289; host form tensor_ops.rs:268-278)
 * with Wg, Wu bf16 [K,F] (host or device, reference layout), A / H device f32:
 * the gate / up product with SwiGLU in its epilogue exactly as the decode step
 * runs it (F % 32 == 0).  H is the next product's operand expanded to f32. */
zr_status zr_gemm_swiglu(zr_context* ctx, const float* d_a, const uint16_t* w_gate, const uint16_t* w_up,
                         float* d_h, int m, int f, int k);

/* --------------------------------------------------------- device memory --- */
zr_status zr_device_alloc(zr_context* ctx, size_t bytes, void** out);
zr_status zr_device_free(zr_context* ctx, void* p);
/* Pinned host memory (hipHostMalloc), e.g. for KV snapshots that move over
 * PCIe at full rate.  No reference counterpart (the reference keeps snapshots
 * in pageable Rust vectors). */
zr_status zr_host_alloc(zr_context* ctx, size_t bytes, void** out);
zr_status zr_host_free(zr_context* ctx, void* p);
zr_status zr_memcpy_h2d(zr_context* ctx, void* dst, const void* src, size_t bytes);
zr_status zr_memcpy_d2h(zr_context* ctx, void* dst, const void* src, size_t bytes);
/* Fills device bf16 [n] with N(0, std) draws (Box-Muller over a counter-based
 * SplitMix64 stream keyed by seed) -- synthetic random-init weights. */
zr_status zr_fill_normal_bf16(zr_context* ctx, uint16_t* d_dst, size_t n, uint64_t seed, float std);
/* Fills every page of the KV pool with N(0, std) values in the pool dtype. */
zr_status zr_kv_pool_fill_normal(zr_context* ctx, uint64_t seed, float std);

/* ------------------------------------------------------------ contract --- */
/* The rocm arm of LocalExecutorContract::for_provider (engine.rs:171-273;
 * fields of LocalExecutorContract 159-169, ExecutorPhasePlan 141-148,
 * KvRuntimeContract 150-156) and of BackendContractDescriptor::for_provider
 * (provider/mod.rs:88-150), as snake_case strings the reference serialises
 * (engine.rs:102-139).  stage_kernels[i] lists, comma-separated, the kernels
 * of this library that implement fused_stages[i].  All strings are static. */
typedef struct {
    const char* executor_class;          /* "fast_path" (LocalExecutorClass) */
    const char* optimization_profile;    /* "rocm_fused" (BackendOptimizationProfile) */
    int n_host_kernels;
    const char* const* host_kernels;     /* HostKernel */
    int n_fused_stages;
    const char* const* fused_stages;     /* FusedKernelStage, contract order */
    const char* const* stage_kernels;
    const char* collective_residency;    /* "staged_runtime" */
    int prefill_supports_microbatch, prefill_requires_static_workspace, prefill_uses_device_sampling;
    int decode_supports_microbatch, decode_requires_static_workspace, decode_uses_device_sampling;
    int kv_requires_paged_cache, kv_append_only_decode, kv_supports_prefill, kv_supports_decode;
    int collective_tensors_per_layer;
    const char* provider;                /* "rocm" (ExecutionProviderKind) */
    const char* compatibility_class;     /* "rocm_fast_path" (ProviderCompatibilityClass) */
    const char* memory_model;            /* "discrete_vram" (MemoryModel) */
    int supports_decode_microbatch, supports_paged_kv, supports_checkpoint_handoff, supports_device_sampling;
    int fast_path_eligible;
    /* FastPathPlanner::capture_strategy (fast_path.rs:831-837) of the rocm_fused
     * profile: "replay_preferred", as the CudaFused arm; served by
     * zr_graph_capture_staged / zr_step_graph_* (GraphCaptureStrategy). */
    const char* capture_strategy;
} zr_executor_contract;
zr_status zr_get_executor_contract(zr_executor_contract* out);

/* ---------------------------------------------------------- profiling --- */
/* Per-kernel-class timing with HIP events on the context stream (enabled
 * between begin/end) around the launches of the classes set in class_mask
 * (bit c for class c).  Classes: 0 attention, 1 gemm, 2 norm/rope/kv,
 * 3 other (split merges, split-K reduce, argmax, sampling, KV gather/scatter),
 * 4 KV snapshot encode.  No reference counterpart (measurement only). */
zr_status zr_timing_begin(zr_context* ctx, unsigned class_mask);
zr_status zr_timing_end(zr_context* ctx, double* ms_by_class /* [5] */, int* launches_by_class /* [5] */);

#ifdef __cplusplus
}
#endif
#endif
