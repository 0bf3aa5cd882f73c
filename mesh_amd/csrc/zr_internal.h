// Internal declarations of the zip MI355X provider: context layout, kernel
// launchers and small device helpers shared by the .hip translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/zip_rocm.h"

namespace zr {

constexpr int kPageRows = 16;   // DEFAULT_LIVE_KV_PAGE_TOKENS (kv_cache.rs:214)
constexpr int kWave = 64;       // CDNA wavefront

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

// ---------------------------------------------------------------- helpers
__host__ __device__ inline uint16_t f32_to_bf16_bits(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

// Split x into bf16 hi + lo with x ~= hi + lo to ~2^-16 relative.  The casts
// compile to gfx950's v_cvt_pk_bf16_f32 (round to nearest even): the same bits
// as f32_to_bf16_bits for every input but NaN, without its NaN branch.
__device__ inline void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    const __bf16 h = (__bf16)x;
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (__bf16)(x - (float)h));
}

// x[0..7] as the hi (lo_part false) or lo halves of split_bf16, one bf16x8
// (8 consecutive columns of the fragment-packed operand below are one 16-byte
// run)
__device__ inline bf16x8 to_bf16x8(const float* x, bool lo_part) {
    bf16x8 r;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint16_t hi, lo;
        split_bf16(x[j], hi, lo);
        r[j] = __builtin_bit_cast(__bf16, lo_part ? lo : hi);
    }
    return r;
}

// GEMM A operands (bf16 activations) are stored fragment-packed for the
// 32x32x16 MFMA: the [rows, K] matrix (K a multiple of 32, rows padded to
// 32) is a sequence of 1 KiB fragments (32-row tile mt, 16-column slice kt16)
// in which lane l holds row 32 mt + l % 32, columns 16 kt16 + 8 (l / 32)
// + j, j < 8.  A block of the GEMM then copies every fragment with one
// contiguous 1 KiB load.  Under ZR_FLAG_SPLIT_ACTIVATIONS the lo halves
// follow the hi plane: plane size = a_plane(rows, K).
__host__ __device__ inline size_t a_pack_index(int m, int k, int K) {
    const int kt16 = K >> 4;
    const int lane = (m & 31) + (((k >> 3) & 1) << 5);
    return ((((size_t)(m >> 5) * kt16 + (k >> 4)) << 6) + lane) * 8 + (k & 7);
}
__host__ __device__ inline size_t a_plane(int rows, int K) { return (size_t)((rows + 31) & ~31) * K; }

// --------------------------------------------------------------- context
typedef __attribute__((address_space(3))) void lds_void;

// LDS rings fed by copies into LDS (GEMM operands: buffer_load ... lds;
// prefill K/V pages: global_load_lds).
// Block barrier for the LDS ring: wait until at most N of this wave's vector
// memory ops (its copies of later stages) are outstanding and
// all of its LDS reads have returned, then s_barrier.  __syncthreads() would
// also wait for the later stages' copies (its fence drains vmcnt), which
// serialises the ring.  The empty asm statements keep the compiler from
// moving memory operations across the barrier.
template <int N>
__device__ __forceinline__ void ring_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // vmcnt(N), expcnt(7), lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ring_barrier for `ahead` (block-uniform, 0..MAXA) stages of VM copies
// each issued after the one waited for.
template <int VM, int MAXA>
__device__ __forceinline__ void ring_wait(int ahead) {
    if constexpr (MAXA > 0) {
        if (ahead >= MAXA) {
            ring_barrier<VM * MAXA>();
            return;
        }
        ring_wait<VM, MAXA - 1>(ahead);
    } else {
        ring_barrier<0>();
    }
}

struct StagedMeta;  // device copy of one microbatch's metadata

// KV pool page layout (per layer, per global page: the K block, then the V
// block, one [16 x head_dim] tile per local kv head):
//   K tile: element (t, d) at ((d / 8) * 16 + t) * 8 + d % 8 -- one 1 KiB row of
//           64 lanes x 16 B is the MFMA A-operand fragment (token = lane % 16,
//           8 dims per lane) for 32 dims.
//   V tile: element (t, d) at ((((d / 32) * 4 + t / 4) * 16 + d % 16) * 2
//           + (d / 16) % 2) * 4 + t % 4 -- 4 consecutive tokens of one dim are
//           one P.V MFMA operand lane; dims d and d + 16 sit side by side, so a
//           lane loads both with one 16 B (bf16) load and a wave reads 1 KiB
//           contiguous per 32 dims.
// (f32 pools then reorder each 512-element block: page_order below.)
// Plain layout (pools whose head_dim the MFMA kernels do not take): both tiles
// row-major [16 rows][head_dim].
__device__ inline size_t k_off(int t, int d) { return ((size_t)(d >> 3) * kPageRows + t) * 8 + (d & 7); }
__device__ inline size_t v_off(int t, int d) {
    return (((((size_t)(d >> 5) * 4 + (t >> 2)) * 16 + (d & 15)) * 2 + ((d >> 4) & 1)) * 4) + (t & 3);
}
// f32 pools keep those offsets' 512-element blocks (one 64-lane x 8-element
// wave fragment each: 32 dims of K, or of V, of one kv head's page) but hold
// each lane's 8 elements as two runs of 4, half-major: lane l's elements 0-3
// at 4 l, 4-7 at 256 + 4 l.  Each 16-byte lane load of a wave is then one
// contiguous 1 KiB run, as in a bf16 page (with lane-contiguous 32-byte
// groups every f32 load spanned 2 KiB for 1 KiB of data).
template <typename KV>
__device__ inline size_t page_order(size_t e) {
    if constexpr (sizeof(KV) == 2) {
        return e;
    } else {
        const size_t w = e & 511;
        return (e & ~(size_t)511) | ((w & 4) << 6) | ((w >> 3) << 2) | (w & 3);
    }
}
template <typename KV>
__device__ inline size_t k_off_of(int t, int d, int D, int plain) {
    return plain ? (size_t)t * D + d : page_order<KV>(k_off(t, d));
}
template <typename KV>
__device__ inline size_t v_off_of(int t, int d, int D, int plain) {
    return plain ? (size_t)t * D + d : page_order<KV>(v_off(t, d));
}
template <typename T> __device__ inline void store_elem(T* p, float x);
template <> __device__ inline void store_elem<float>(float* p, float x) { *p = x; }
template <> __device__ inline void store_elem<uint16_t>(uint16_t* p, float x) { *p = f32_to_bf16_bits(x); }
template <typename T> __device__ inline float load_elem(const T* p);
template <> __device__ inline float load_elem<float>(const float* p) { return *p; }
template <> __device__ inline float load_elem<uint16_t>(const uint16_t* p) { return bf16_bits_to_f32(*p); }

struct LayerDev {
    uint16_t* w_qkv = nullptr;     // packed [K=H, N=Q+2Kc]
    uint16_t* w_o = nullptr;       // packed [K=Q, N=H]
    uint16_t* w_gate_up = nullptr; // packed [K=H, N=2F] ([gate|up])
    uint16_t* w_down = nullptr;    // packed [K=F, N=H]
    float* attn_norm = nullptr;
    float* mlp_norm = nullptr;
};

struct TimingState {
    bool enabled = false;
    unsigned class_mask = 0x1F;      // classes that record events
    std::vector<hipEvent_t> pool;    // recycled events
    std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> spans;
    size_t next_event = 0;
};

}  // namespace zr

struct zr_context {
    zr_model_desc desc{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;

    // shard geometry (resolve_attention_shard_layout)
    int head_dim = 0, q_cols = 0, kv_cols = 0, local_q_heads = 0, local_kv_heads = 0;
    int q_per_kv = 0, q_head_start = 0, kv_head_start = 0;
    std::vector<uint32_t> kv_head_map;
    // Page layout of the KV pool.  false: the MFMA fragment layout of the
    // decode / prefill attention kernels (head_dim 64 or 128, q heads per kv
    // head dividing 16).  true (any other even head_dim up to 256, any group):
    // each kv head's K and V tiles are row-major [16 rows][head_dim], read by
    // the generic attention kernel.
    bool plain_kv = false;

    // weights
    std::vector<zr::LayerDev> layers;
    uint16_t* embedding = nullptr;  // [V, H] bf16 (row gather)
    uint16_t* lm_head = nullptr;    // packed [K=H, N=V]
    float* final_norm = nullptr;
    float* inv_freq = nullptr;      // [head_dim/2] host powf table

    // KV pool: layer l, page p at kv_pool + (l * n_pages + p) * page_bytes;
    // K block then V block, each [kv_heads][page layout] in kv dtype.
    void* kv_pool = nullptr;
    int n_pages = 0;
    size_t page_bytes = 0;   // bytes of one page of one layer (K and V)

    // activations (max_tokens rows).  GEMM A operands are bf16 [M, K], followed
    // by the lo half [M, K] under ZR_FLAG_SPLIT_ACTIVATIONS.
    float* hidden = nullptr;     // [T, H] residual stream (f32)
    uint16_t* xa = nullptr;      // normed hidden, A of QKV / gate_up
    float* qkv = nullptr;        // [T, Q + 2Kc]
    float* q_rope = nullptr;     // [T, Q]
    uint16_t* attn_a = nullptr;  // attention output, A of O
    float* proj = nullptr;       // [T, H] O / down projection output (pre-all-reduce partial)
    uint16_t* ffn_a = nullptr;   // SwiGLU output, A of down
    uint16_t* final_a = nullptr; // [S, H] normed last rows, A of the LM head
    float* logits = nullptr;     // [S, V]
    uint32_t* tokens_out = nullptr; // [S]
    float* splitk_ws = nullptr;     // split-K partial workspace
    size_t splitk_ws_floats = 0;
    float* attn_part = nullptr;     // attention split partials
    size_t attn_part_floats = 0;
    float* argmax_ws = nullptr;     // argmax partials
    size_t argmax_ws_floats = 0;
    // bumped whenever a buffer the forward pass reads is freed or moved (a
    // workspace regrown, the KV pool or weights replaced): graphs captured
    // before hold its old address and are refused at launch
    uint64_t buffer_epoch = 0;
    // staged microbatches (zr_stage) not yet destroyed: a graph replays its
    // staged blob, so it is refused once that blob is gone
    std::vector<uint64_t> live_staged;
    uint64_t next_staged_id = 1;

    zr::StagedMeta* scratch_stage = nullptr;  // reused by zr_forward
    // zr_forward's decode steps replayed from a step graph once a sequence
    // count repeats: the graph, ids in / out (device [2][max_seqs]; pinned
    // host [2][max_seqs]) and the run of calls with the current count
    zr_step_graph* fwd_graph = nullptr;
    uint32_t* fwd_ids = nullptr;
    uint32_t* fwd_h_ids = nullptr;
    int fwd_seqs = 0, fwd_repeats = 0;
    float* kv_stage = nullptr;      // KV gather / scatter staging (rows + table)
    size_t kv_stage_floats = 0;
    // KV window copies between HBM and host memory that overlap the compute
    // stream (zr_transfer): one stream per direction, default priority, and
    // the device buffers of finished transfers, kept for reuse (hipFree
    // would synchronise the device)
    hipStream_t d2h_stream = nullptr, h2d_stream = nullptr;
    std::vector<std::pair<float*, size_t>> xfer_free;
    void* cbor_ws = nullptr;        // KV snapshot encoder: chunk sizes / offsets / header tables
    size_t cbor_ws_bytes = 0;
    void* cbor_out = nullptr;       // KV snapshot encoder: the document on the device
    size_t cbor_out_bytes = 0;
    void* sample_ws = nullptr;      // stochastic sampling: per-row parameters
    size_t sample_ws_bytes = 0;
    // Device-fed token ids out of the vocabulary: the embedding kernel keeps
    // the smallest (row << 32 | id) here (all ones = none); a forward pass fed
    // from device memory copies it to the pinned host word, which
    // zr_synchronize checks.
    unsigned long long* d_token_err = nullptr;
    unsigned long long* h_token_err = nullptr;
    bool token_check_pending = false;
    float* noalloc_scratch = nullptr;  // device address of the library's fixed argmax scratch on this device
    zr::TimingState timing;
};

namespace zr {

// Error helpers --------------------------------------------------------
zr_status set_err(zr_context* ctx, zr_status code, const char* fmt, ...);
zr_status set_global_err(zr_status code, const char* fmt, ...);

#define ZR_HIP(ctx, expr)                                                            \
    do {                                                                            \
        hipError_t e__ = (expr);                                                    \
        if (e__ != hipSuccess)                                                      \
            return ::zr::set_err((ctx), ZR_E_HIP, "%s failed: %s (%s:%d)", #expr,   \
                                 hipGetErrorString(e__), __FILE__, __LINE__);       \
    } while (0)

#define ZR_LAUNCH_CHECK(ctx)                                                         \
    do {                                                                            \
        hipError_t e__ = hipGetLastError();                                         \
        if (e__ != hipSuccess)                                                      \
            return ::zr::set_err((ctx), ZR_E_HIP, "kernel launch failed: %s (%s:%d)", \
                                 hipGetErrorString(e__), __FILE__, __LINE__);       \
    } while (0)

// Timing of kernel classes (HIP events on the context stream).
enum { kClassAttention = 0, kClassGemm = 1, kClassNormRopeKv = 2, kClassOther = 3, kClassKvCbor = 4 };
constexpr int kTimingClasses = 5;
void timing_mark_begin(zr_context* ctx, int cls, hipEvent_t* out);
void timing_mark_end(zr_context* ctx, int cls, hipEvent_t begin);

// Staged microbatch metadata (device) ------------------------------------
struct StagedMeta {
    zr_context* ctx = nullptr;
    uint64_t id = 0;          // zr_stage handle id (zr_context::live_staged)
    int num_seqs = 0, total_q = 0, stride = 0;
    int max_kv = 0;           // max kv_after over sequences
    int n_attn_items = 0;     // attention work items (per kv head)
    int n_tiles = 0;          // attention query tiles (per kv head)
    int n_merge = 0;          // tiles with more than one split
    int n_pblocks = 0;        // prefill work units (block, key split) per kv head
    int prefill_kh = 1;       // key halves per prefill workgroup (1: 4 waves, 2: 8 waves)
    int n_part_items = 0;     // partial items: decode items, then prefill (group, split) items
    bool pure_decode = false; // every sequence has one query row (MFMA page layout): RoPE + KV append can run
                              // inside the decode attention kernel
    bool fuse_rope = false;   // ... and the forward pass has them do so
    bool owns = true;
    int grid_items = 0;       // decode attention records the launch covers (n_attn_items, or a bucket's
                              // capacity whose records past n_attn_items are empty)
    int grid_merge = 0;       // merge records the launch covers (likewise)
    // one device allocation holding every array below
    void* dev = nullptr;
    size_t dev_bytes = 0, cap_bytes = 0;
    // device arrays
    int* q_len = nullptr;
    int* kv_before = nullptr;
    int* first_pos = nullptr;
    int* first_offset = nullptr;
    int* block_tables = nullptr;
    uint32_t* tokens = nullptr;
    int* cu_q = nullptr;        // [S+1]   (pack kernel output)
    int* cu_k = nullptr;        // [S+1]
    int* positions = nullptr;   // [T]
    int* slot_mapping = nullptr;// [T]
    int* seq_ids = nullptr;     // [T]
    int* last_rows = nullptr;   // [S] row index of each sequence's last token
    float2* rope_cs = nullptr;  // [T][head_dim / 2] (cos, sin) of position x inv_freq (pack stage output)
    // decode attention: three records per dispatch rank (items longest first),
    //   {seq, first q row, nq, page_begin}, {page_end, kv_before + q0, first_offset, item | kAttnSingle | kAttnLast},
    //   {the pool pages of the item's first 4 pages (the last one repeated past its end)}
    int4* attn_rec = nullptr;
    int4* merge_rec = nullptr;  // [n_merge] tiles the merge kernel combines: {first partial, splits, first q row, nq}
    int4* pblocks = nullptr;    // [n_pblocks] {seq, r0, nrows, pages}, most key tiles first
    int4* psplits = nullptr;    // [n_pblocks] {first key tile, end key tile, item, splits}
    // host copies
    std::vector<int> h_q_len, h_kv_before, h_first_pos, h_first_offset, h_block_tables;
    std::vector<int4> h_items, h_tiles, h_pblocks, h_psplits;
    std::vector<int> h_merge, h_order;
    std::vector<int4> h_attn_rec, h_merge_rec;
    std::vector<uint32_t> h_tokens;
    std::vector<unsigned char> h_blob;
};

// A replayed step's bucket: the staged arrays sit at the same offsets of the
// same device blob every step, sized for the bucket's capacities; records past
// a step's counts are empty (nq = 0).  The host blob is written in place into
// `host` (pinned); nothing is allocated, copied or launched.
struct StageFixed {
    int stride = 0;                  // block-table stride of the blob
    int items_cap = 0;               // decode attention records
    int merge_cap = 0;               // merge records
    bool fuse_rope = false;          // RoPE + KV append inside attention (fixed per bucket)
    unsigned char* host = nullptr;
    size_t host_cap = 0;
    void* dev = nullptr;
    size_t dev_cap = 0;
    bool plan_only = false;          // only the counts (items, merges, partials) for sizing a bucket
};
// Blob bytes of a fixed layout: host part (copied per step) and the whole.
void stage_fixed_bytes(const zr_context* ctx, int S, int total_q, const StageFixed& f, size_t* host_bytes,
                       size_t* dev_bytes);
// Stages a microbatch.  With `fixed`, a microbatch that is not a pure decode
// step or exceeds the bucket's capacities sets *fits = false and returns
// ZR_E_UNSUPPORTED (the caller captures a new bucket).
zr_status stage_microbatch(zr_context* ctx, const zr_microbatch* mb, StagedMeta* st, const StageFixed* fixed = nullptr,
                           bool* fits = nullptr);
// flags of a decode attention record's last field (above them: the item index)
constexpr unsigned kAttnSingle = 1u << 30;  // the item's tile has one split: it writes the final output
constexpr unsigned kAttnLast = 1u << 31;    // the item is its tile's last split (holds the newest rows)

// An f32 [rows, cols] operand held as n split-K slabs `stride` floats apart;
// readers sum the slabs in order (n = 1: a plain array).
struct Slabs {
    const float* ptr = nullptr;
    int n = 1;
    size_t stride = 0;
    Slabs() = default;
    Slabs(const float* p) : ptr(p) {}
    Slabs(const float* p, int n_, size_t s) : ptr(p), n(n_), stride(s) {}
};

// Kernel launchers (one per .hip file) ------------------------------------
zr_status launch_pack(zr_context* ctx, StagedMeta* st);
// check_ids: record out-of-vocabulary ids in ctx->d_token_err (device-fed ids)
zr_status launch_embed(zr_context* ctx, StagedMeta* st, const uint32_t* d_tokens, bool check_ids);
// y = rms_norm(x (+ residual_in)) * gamma.  With residual_in, x_out = x +
// residual_in is written first.  Output as f32 (y_f32) or as the bf16 A operand
// of the next GEMM (y_bf16: hi [rows, cols] then lo when split_lo).
zr_status launch_rms_norm(zr_context* ctx, const float* x, const Slabs& residual, float* x_out,
                          const float* gamma, float* y_f32, uint16_t* y_bf16, int split_lo,
                          const int* row_index, int rows, int cols);
zr_status launch_rope_kv_write(zr_context* ctx, StagedMeta* st, int layer, const Slabs& qkv,
                               float* q_out, int rope);
// out_f32 [T, q_cols] or out_bf16 (A operand of the O projection).
zr_status launch_attention(zr_context* ctx, StagedMeta* st, int layer, const float* q, float* out_f32,
                           uint16_t* out_bf16);
// Pure decode microbatches (st->pure_decode): RoPE + KV append and attention in
// one launch, q and the new K / V rows read from the QKV product's slabs.
// Times `repeats` launches of a read-only copy of the decode attention
// launch's page stream for staged microbatch `st` at `layer` (mean ms).
zr_status launch_kv_read_probe(zr_context* ctx, StagedMeta* st, int layer, int repeats, double* mean_ms);
zr_status launch_attention_rope(zr_context* ctx, StagedMeta* st, int layer, const Slabs& qkv, int rope,
                                float* out_f32, uint16_t* out_bf16);
zr_status launch_kv_copy(zr_context* ctx, int layer_begin, int layer_end, const int* d_table,
                         int first_offset, int first_row, int n_rows, float* k, float* v,
                         int to_pool);
zr_status launch_argmax(zr_context* ctx, const float* x, int rows, int cols, uint32_t* out);
// The same with the partials in the library's fixed device array (no
// allocation; rows x ceil(cols / 4096) <= kNoAllocArgmaxPairs).
constexpr int kNoAllocArgmaxPairs = 32768;
constexpr int kMaxDevices = 64;
zr_status noalloc_scratch_init(zr_context* ctx);
zr_status launch_argmax_noalloc(zr_context* ctx, const float* x, int rows, int cols, uint32_t* out);
// sample_tokens_device_with_seeds per row (sample.hip); parameters are host arrays
zr_status launch_sample(zr_context* ctx, const float* d_logits, int rows, int cols, const float* temperature,
                        const float* top_p, const uint64_t* seeds, uint32_t* d_out);

enum GemmEpilogue { kEpiStore = 0, kEpiSwiGLU = 1 };
struct GemmPlan {
    int KT = 0, NT = 0, row_blocks = 0, col_blocks = 0, splits = 1, kt_per_split = 0;
    bool direct = true;
    size_t ws_floats = 0;
};
GemmPlan gemm_plan(int m, int n, int k, int epilogue);
// C = A @ W (W packed, A bf16 operand).  kEpiStore writes c_f32; kEpiSwiGLU
// writes silu(gate) * up as the bf16 operand c_bf16 (or f32 c_f32).  With
// `deferred` (kEpiStore only) a split-K product is left as its slabs in the
// split-K workspace for the consumer to sum (valid until the next GEMM);
// *deferred then describes C either way.
zr_status launch_gemm(zr_context* ctx, const uint16_t* a, const uint16_t* w_packed, float* c_f32,
                      uint16_t* c_bf16, int m, int n, int k, int epilogue, Slabs* deferred = nullptr);
// f32 [rows, K] -> fragment-packed bf16 hi (+ lo) A operand (K % 32 == 0)
zr_status launch_to_bf16_pair(zr_context* ctx, const float* x, int rows, int K, uint16_t* out, int with_lo);
// fragment-packed bf16 hi (+ lo) [rows, K] -> f32 hi + lo [rows, K]
zr_status launch_from_bf16_pair(zr_context* ctx, const uint16_t* in, int rows, int K, int with_lo, float* y);
zr_status pack_weight(zr_context* ctx, const uint16_t* src /* [K,N] host or device */,
                      int k, int n, uint16_t** out_packed);
// Packs [K, n1] | [K, n2] | ... (column concatenation) into one packed matrix.
zr_status pack_weight_concat(zr_context* ctx, const uint16_t* const* srcs, const int* widths,
                             int count, int k, uint16_t** out_packed);
size_t packed_weight_elems(int k, int n);

zr_status launch_fill_normal_bf16(zr_context* ctx, uint16_t* dst, size_t n, uint64_t seed, float std);
zr_status launch_fill_pool_normal(zr_context* ctx, uint64_t seed, float std);

// KV snapshot wire format (kv_cbor.hip) -----------------------------------
// Fixed byte strings of the KVCache CBOR document around the 2L float arrays:
// entry a < 2L precedes array a (K of layer a / 2 or V), the last follows the
// last array.
struct KvCborLayout {
    std::vector<uint8_t> bytes;
    std::vector<uint32_t> off, len;
};
KvCborLayout kv_cbor_layout(int layers, int rows, int cols, long long base_position, const int cfg[4]);
zr_status launch_kv_cbor(zr_context* ctx, const float* d_k, const float* d_v, int layers, int rows, int cols,
                         long long base_position, const int cfg[4], uint8_t* out, size_t capacity, size_t* out_len);
struct KvCborDoc {
    int layers = 0;
    long long rows = 0, cols = 0, base_position = 0;
    long long cfg[4] = {0, 0, 0, 0};  // num_layers, num_heads, head_dim, max_seq_len
    std::vector<float> k, v;          // [layers][rows][cols]
};
bool kv_cbor_decode(const uint8_t* bytes, size_t len, KvCborDoc* doc, std::string* err);

}  // namespace zr
