/*
 * zip_oracle.h -- CPU restatement of the zip engine's hot path (saint0x/mesh).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the test oracle for the HIP provider:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product path (mesh_amd/) never links or calls it.
 *
 * Everything is IEEE f32 as in the reference, with per-element operation order
 * following the reference's host text (agent/src/inference/tensor_ops.rs and
 * forward_pass.rs); see each function's comment for the exact citation.
 *
 * Parity pinning (what checks each part; tests/test_oracle_*.py):
 *   page allocator / block tables  KATs forward_pass.rs:3728-3822, 3458-3507,
 *                                  invariants kv_cache.rs:372-415
 *   shard layout                   KAT forward_pass.rs:3325-3354
 *   packing (cu_seqlens, positions, slot mapping)   closed forms + KATs
 *                                  fast_path.rs:974-1080
 *   attention                      fp64 brute force, L=1 -> v0, equal keys ->
 *                                  mean(V), incremental == full recompute
 *   rms_norm / rope / silu         closed forms (numpy fp64), pos 0 identity,
 *                                  rotation norm preservation
 *   matmul                         KAT tensor_ops.rs:577-590, fp64 brute force
 *   greedy argmax                  KAT tensor_ops.rs:633-639, first index on ties
 *   stochastic sampling            parity unpinned beyond the seed-threshold
 *                                  closed form (no fixture in the reference)
 */
#ifndef ZIP_ORACLE_H
#define ZIP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: 0 ok, negative = error (message via or_last_error()). */
const char* or_last_error(void);

/* ---------------------------------------------------------------- ops --- */
/* tensor_ops.rs:219-240: C[m,n] = A[m,k] @ B[k,n], f32, k-order accumulation. */
int or_matmul(const float* a, const float* b, float* c, int m, int k, int n);
/* tensor_ops.rs:285-304 */
int or_rms_norm(const float* x, const float* gamma, float* out, int rows, int cols, float eps);
/* tensor_ops.rs:268-278 */
void or_silu(const float* x, float* out, int64_t n);
/* tensor_ops.rs:509-560 (runtime.rs:282-301 for the inverse-frequency table) */
int or_apply_rope(const float* x, float* out, int rows, int cols, const uint32_t* positions,
                  int head_dim, float base);
void or_rope_inv_freq(int head_dim, float base, float* inv_freq /* [head_dim/2] */);
/* tensor_ops.rs:461-473: first maximum wins (strict >). */
uint32_t or_sample_greedy(const float* logits, int n);
/* tensor_ops.rs:394-458 (deterministic_sample_threshold at 372-388). */
uint32_t or_sample_token(const float* logits, int n, float temperature, float top_p, uint64_t seed);
float or_sample_threshold(uint64_t seed);
/* The batched decode path's device sampler (runtime.rs:534-601) for one row, in f64 on the f32 scaled
 * logits; *margin (nullable) is the distance from tau / top_p to the nearest cumulative boundary the
 * decision depends on. */
uint32_t or_sample_token_device(const float* logits, int n, float temperature, float top_p, uint64_t seed,
                                double* margin);
/* forward_pass.rs:1317-1372: causal attention with a cached prefix, one head.
 * q [q_rows, d], k/v [kv_rows, d]; row r sees keys [0, prefix + r]. */
int or_causal_attention_with_prefix(const float* q, const float* k, const float* v, float* out,
                                    int q_rows, int kv_rows, int d, float scale, int prefix_len);

/* float -> bf16 (round to nearest even) and back, as stored by a bf16 KV pool. */
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t h);
void or_round_bf16_inplace(float* x, int64_t n);

/* ------------------------------------------------------ shard geometry --- */
/* forward_pass.rs:1257-1315 and 2951-2970 */
typedef struct {
    int head_dim, q_heads_per_kv_head, q_cols, q_head_start, local_q_heads;
    int kv_cols, kv_head_start, local_kv_heads;
} or_shard_layout;
int or_resolve_shard_layout(int hidden, int num_heads, int num_kv_heads, int shard_start,
                            int shard_end, or_shard_layout* out, uint32_t* local_kv_head_indices);
/* artifact_loader.rs:351-366 */
int or_partition_columns(int total_columns, int worker_position, int total_workers);

/* ------------------------------------------- paged KV session (device) --- */
/* One session's DeviceKVCache (forward_pass.rs:899-1243): per-layer paged
 * caches with a LIFO page free list, span block tables and a sliding window. */
typedef struct or_session or_session;
or_session* or_session_new(int num_layers, int kv_cols, int page_rows, int max_seq_len,
                           int kv_round_bf16);
void or_session_free(or_session* s);
/* DeviceKVCache::append_layer (forward_pass.rs:920-957); k/v [rows, kv_cols] */
int or_session_append_layer(or_session* s, int layer, const float* k, const float* v, int rows);
/* DeviceKVCache::retain_suffix (1084-1094) */
int or_session_retain_suffix(or_session* s, int keep_rows);
/* DeviceKVCache::clear (1076-1082) */
void or_session_clear(or_session* s);
int or_session_seq_len(const or_session* s, int layer);
int or_session_base_position(const or_session* s);
int or_session_position(const or_session* s);
void or_session_set_position(or_session* s, int position);
int or_session_allocated_pages(const or_session* s, int layer);
/* live_block_table (forward_pass.rs:682-721, 1024-1048): returns span count or <0.
 * page_ids/start/count may be NULL to query the count. */
int or_session_block_table(const or_session* s, int layer, uint32_t* page_ids, int* start_tokens,
                           int* token_counts, int max_spans);
/* build_active_tensors (forward_pass.rs:633-680): k/v [seq_len, kv_cols] */
int or_session_gather(const or_session* s, int layer, float* k_out, float* v_out);
/* export_snapshot (1169-1204): max_cached_tokens < 0 means no limit.
 * Writes [num_layers][rows][kv_cols]; returns rows (0 = no snapshot). */
int or_session_export(const or_session* s, int max_cached_tokens, float* k_out, float* v_out,
                      int* out_base_position, int* out_next_position);
/* import_snapshot (1206-1242) */
int or_session_import(or_session* s, const float* k, const float* v, int rows, int base_position,
                      int next_position);

/* ---------------------------------------------------------------- model --- */
typedef struct {
    int hidden, num_heads, num_kv_heads, num_layers, vocab, ffn_cols;
    int shard_start, shard_end; /* q-column range of this worker's shard */
    float rms_norm_eps, rope_base;
} or_model_config;
typedef struct or_model or_model;
or_model* or_model_new(const or_model_config* cfg);
void or_model_free(or_model* m);
/* Pointers are borrowed, row-major [in, out] as the reference (x @ W). */
int or_model_set_globals(or_model* m, const float* embedding /*[V,H]*/,
                         const float* final_norm /*[H]*/, const float* lm_head /*[H,V]*/);
int or_model_set_layer(or_model* m, int layer, const float* w_q, const float* w_k,
                       const float* w_v, const float* w_o, const float* w_gate, const float* w_up,
                       const float* w_down, const float* attn_norm, const float* mlp_norm);
/* The same model with bf16 bit-pattern weights (bf16 -> f32 is exact, so the
 * results are bit-identical to the f32 form of the same values); halves the
 * host memory of full-width models. */
int or_model_set_globals_bf16(or_model* m, const uint16_t* embedding, const float* final_norm,
                              const uint16_t* lm_head);
int or_model_set_layer_bf16(or_model* m, int layer, const uint16_t* w_q, const uint16_t* w_k,
                            const uint16_t* w_v, const uint16_t* w_o, const uint16_t* w_gate,
                            const uint16_t* w_up, const uint16_t* w_down, const float* attn_norm,
                            const float* mlp_norm);
/* or_matmul with b given as bf16 bit patterns (bit-identical results). */
int or_matmul_bf16w(const float* a, const uint16_t* b, float* c, int m, int k, int n);


/* ForwardPass::fast_path_decode_microbatch (forward_pass.rs:2143-2319) over B
 * sessions with the same model.  logits [B, V]; partials (nullable)
 * [num_layers][2][B][H] = (o_partial, down_partial) per layer; hidden_out
 * (nullable) [B, H] = final normed hidden. */
int or_decode_microbatch(const or_model* m, or_session** sessions, int batch,
                         const uint32_t* tokens, float* logits, float* partials);
/* ForwardPass::prefill (2089-2112): clears the cache, keeps the last window.
 * logits [V] of the last row. */
/* The same step with the appended K / V row of every (layer, session) taken
 * from force_k / force_v [num_layers][B][kv_cols]: the rows another
 * implementation stored after rounding its own f32 values to bf16.  Two
 * correct f32 evaluations can round a near-tie element to neighbouring bf16
 * values; forcing the stored rows lets the rest of the step be compared
 * without that rounding flip.  own_k / own_v (nullable, same shape) receive
 * this oracle's own f32 rows (before rounding), so the caller can check that
 * every forced element is a valid rounding of a value within f32 noise. */
int or_decode_microbatch_forced(const or_model* m, or_session** sessions, int batch, const uint32_t* tokens,
                                float* logits, float* partials, const float* force_k, const float* force_v,
                                float* own_k, float* own_v);
int or_prefill(const or_model* m, or_session* s, const uint32_t* tokens, int n_tokens,
               float* logits);
/* Chunked prefill at the session's current position (forward_tokens 2456-2528
 * with a non-empty prefix; masked attention 2764-2836 / 1317-1372).
 * logits [V] of the last row (nullable); partials like or_decode_microbatch
 * but [num_layers][2][n_tokens][H]. */
int or_prefill_chunk(const or_model* m, or_session* s, const uint32_t* tokens, int n_tokens,
                     float* logits, float* partials);

/* -------------------------------------------------------------- packing --- */
/* Closed form of the ragged packing metadata (fast_path.rs:263-338, 409-445,
 * forward_pass.rs:1012-1014): per sequence q_len new tokens appended after
 * kv_before cached rows; first_pos = base_position + kv_before.
 * block_tables [nseq][max_pages] global page ids, first_offset = start row of
 * the first span.  Outputs cu_q/cu_k [nseq+1], positions/slot_mapping/seq_ids
 * [total_q]. */
int or_pack(int nseq, const int* q_len, const int* kv_before, const int* first_pos,
            const int* first_offset, const int* block_tables, int max_pages, int page_rows,
            int* cu_q, int* cu_k, int* positions, int* slot_mapping, int* seq_ids);

/* ------------------------------------------------------ KV snapshot CBOR (kv_cbor.c) */
/* Head of major type `major` with argument v (RFC 8949 section 3), shortest form; returns bytes. */
int or_cbor_uint(int major, uint64_t v, uint8_t* out);
/* ciborium's float item for an f32 (narrowest exact of half / single / double); returns bytes. */
int or_cbor_float(float x, uint8_t* out);
/* KVCache::to_bytes (kv_cache.rs:880-887) of an export_snapshot cache: k, v = [num_layers][rows][cols].
 * Returns the byte count (out NULL: count only), -2 when capacity is too small, -1 on bad sizes. */
int64_t or_kv_cbor_encode(const float* k, const float* v, int num_layers, int rows, int cols,
                          int64_t base_position, int cfg_num_layers, int cfg_num_heads, int cfg_head_dim,
                          int cfg_max_seq_len, uint8_t* out, int64_t capacity);

#ifdef __cplusplus
}
#endif
#endif
