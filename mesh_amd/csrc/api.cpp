// C ABI entry points of the zip MI355X provider (include/zip_rocm.h):
// context and weight residency, KV pool, microbatch staging and the decode /
// prefill forward pass (ForwardPass::fast_path_decode_microbatch,
// agent/src/inference/forward_pass.rs:2143-2319).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cstdlib>

#include "zr_internal.h"

namespace zr {

zr_status pack_weight_gate_up(zr_context* ctx, const uint16_t* gate, const uint16_t* up, int k, int f,
                              uint16_t** out);

static thread_local std::string g_err;

zr_status set_err(zr_context* ctx, zr_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    g_err = buf;
    return code;
}

zr_status set_global_err(zr_status code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

// ------------------------------------------------------------- timing
void timing_mark_begin(zr_context* ctx, int cls, hipEvent_t* out) {
    *out = nullptr;
    TimingState& t = ctx->timing;
    if (!t.enabled || !(t.class_mask & (1u << cls))) return;
    if (t.next_event + 2 > t.pool.size()) {
        for (int i = 0; i < 64; ++i) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) return;
            t.pool.push_back(e);
        }
    }
    *out = t.pool[t.next_event++];
    hipEventRecord(*out, ctx->stream);
}

void timing_mark_end(zr_context* ctx, int cls, hipEvent_t begin) {
    TimingState& t = ctx->timing;
    if (!t.enabled || !begin) return;
    hipEvent_t e = t.pool[t.next_event++];
    hipEventRecord(e, ctx->stream);
    t.spans.push_back({cls, {begin, e}});
}

// ------------------------------------------------------------- geometry
// resolve_attention_shard_layout (forward_pass.rs:1257-1315) and
// build_local_kv_head_indices (2951-2970).
static zr_status resolve_geometry(zr_context* ctx) {
    const zr_model_desc& d = ctx->desc;
    if (d.num_heads <= 0 || d.hidden % d.num_heads != 0)
        return set_err(ctx, ZR_E_INVALID, "Unsupported attention geometry: hidden_dim %d num_heads %d", d.hidden,
                       d.num_heads);
    if (d.num_kv_heads <= 0 || d.num_heads % d.num_kv_heads != 0)
        return set_err(ctx, ZR_E_INVALID,
                       "Unsupported grouped-query attention geometry: num_heads %d num_kv_heads %d", d.num_heads,
                       d.num_kv_heads);
    if (d.shard_start >= d.shard_end || d.shard_end > d.hidden || d.shard_start < 0)
        return set_err(ctx, ZR_E_INVALID, "Invalid shard range %d..%d for hidden_dim %d", d.shard_start,
                       d.shard_end, d.hidden);
    const int head_dim = d.hidden / d.num_heads;
    const int qpk = d.num_heads / d.num_kv_heads;
    const int group = qpk * head_dim;
    if (d.hidden % group != 0)
        return set_err(ctx, ZR_E_INVALID, "Hidden dim %d is not divisible by grouped-query shard width %d",
                       d.hidden, group);
    if (d.shard_start % group != 0 || d.shard_end % group != 0)
        return set_err(ctx, ZR_E_INVALID, "Shard range %d..%d is not aligned to grouped-query shard width %d",
                       d.shard_start, d.shard_end, group);
    ctx->head_dim = head_dim;
    ctx->q_per_kv = qpk;
    ctx->q_cols = d.shard_end - d.shard_start;
    const int groups = ctx->q_cols / group;
    ctx->local_q_heads = groups * qpk;
    ctx->local_kv_heads = groups;
    ctx->kv_cols = groups * head_dim;
    ctx->q_head_start = d.shard_start / head_dim;
    ctx->kv_head_start = d.shard_start / group;
    ctx->kv_head_map.clear();
    for (int i = 0; i < ctx->local_q_heads; ++i) {
        const int gq = ctx->q_head_start + i, gk = gq / qpk;
        if (gk < ctx->kv_head_start || gk >= ctx->kv_head_start + ctx->local_kv_heads)
            return set_err(ctx, ZR_E_INVARIANT, "Local KV head ownership mismatch: q_head %d maps to kv_head %d", gq,
                           gk);
        ctx->kv_head_map.push_back((uint32_t)(gk - ctx->kv_head_start));
    }
    // RoPE's rotate-half pairs dims (i, i + d / 2): an even head_dim
    // (tensor_ops.rs:509-520); the generic attention kernel holds up to 256
    // dims per lane group
    if (head_dim % 2 != 0 || head_dim > 256)
        return set_err(ctx, ZR_E_UNSUPPORTED, "head_dim %d not supported (even, at most 256)", head_dim);
    if (ctx->kv_cols % 4 != 0)
        return set_err(ctx, ZR_E_UNSUPPORTED, "kv columns %d not a multiple of 4", ctx->kv_cols);
    if (ctx->q_cols % 32 != 0)
        return set_err(ctx, ZR_E_UNSUPPORTED, "q columns %d not a multiple of 32 (the O projection operand)",
                       ctx->q_cols);
    ctx->plain_kv = !((head_dim == 64 || head_dim == 128) && qpk <= 16 && 16 % qpk == 0);
    return ZR_OK;
}

// Split-K workspace of one GEMM shape (same plan as launch_gemm).
static size_t gemm_ws_floats(int m, int n, int k, int epilogue) { return gemm_plan(m, n, k, epilogue).ws_floats; }

static void destroy_streams(zr_context* ctx) {
    for (hipStream_t* st : {&ctx->stream, &ctx->d2h_stream, &ctx->h2d_stream})
        if (*st) {
            (void)hipStreamDestroy(*st);
            *st = nullptr;
        }
}

static void free_ctx_buffers(zr_context* ctx) {
    void* bufs[] = {ctx->hidden, ctx->xa, ctx->qkv, ctx->q_rope, ctx->attn_a, ctx->proj, ctx->ffn_a,
                    ctx->logits, ctx->final_a, ctx->tokens_out, ctx->splitk_ws, ctx->attn_part,
                    ctx->argmax_ws, ctx->inv_freq, ctx->kv_pool, ctx->embedding, ctx->lm_head,
                    ctx->final_norm, ctx->d_token_err};
    for (void* b : bufs)
        if (b) hipFree(b);
    if (ctx->h_token_err) hipHostFree(ctx->h_token_err);
    for (auto& L : ctx->layers) {
        void* lb[] = {L.w_qkv, L.w_o, L.w_gate_up, L.w_down, L.attn_norm, L.mlp_norm};
        for (void* b : lb)
            if (b) hipFree(b);
    }
}

// ----------------------------------------------------------------- staging
static inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

// Offsets of one staged blob: the host-written inputs and records first, then
// the arrays the pack stage derives on the device.
struct BlobLayout {
    size_t o_qlen, o_kvb, o_fpos, o_foff, o_bt, o_tok, o_arec, o_mrec, o_pblk, o_psplit, host_bytes;
    size_t o_cuq, o_cuk, o_pos, o_slot, o_seq, o_last, o_rcs, total_bytes;
};

static BlobLayout blob_layout(int S, int stride, int total_q, int n_items, int n_merge, int n_pblocks, int head_dim) {
    BlobLayout b;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align16(off + bytes);
        return o;
    };
    b.o_qlen = take(4 * S);
    b.o_kvb = take(4 * S);
    b.o_fpos = take(4 * S);
    b.o_foff = take(4 * S);
    b.o_bt = take(4 * (size_t)S * stride);
    b.o_tok = take(4 * (size_t)std::max(total_q, 1));
    b.o_arec = take(48 * (size_t)std::max(n_items, 1));
    b.o_mrec = take(16 * (size_t)std::max(n_merge, 1));
    b.o_pblk = take(16 * (size_t)std::max(n_pblocks, 1));
    b.o_psplit = take(16 * (size_t)std::max(n_pblocks, 1));
    b.host_bytes = off;
    b.o_cuq = take(4 * (S + 1));
    b.o_cuk = take(4 * (S + 1));
    b.o_pos = take(4 * (size_t)total_q);
    b.o_slot = take(4 * (size_t)total_q);
    b.o_seq = take(4 * (size_t)total_q);
    b.o_last = take(4 * S);
    b.o_rcs = take(8 * (size_t)total_q * (head_dim / 2));
    b.total_bytes = off;
    return b;
}

void stage_fixed_bytes(const zr_context* ctx, int S, int total_q, const StageFixed& f, size_t* host_bytes,
                       size_t* dev_bytes) {
    const BlobLayout b = blob_layout(S, f.stride, total_q, f.items_cap, f.merge_cap, 0, ctx->head_dim);
    *host_bytes = b.host_bytes;
    *dev_bytes = b.total_bytes;
}

zr_status stage_microbatch(zr_context* ctx, const zr_microbatch* mb, StagedMeta* st, const StageFixed* fixed,
                           bool* fits) {
    if (fits) *fits = true;
    auto no_fit = [&](const char* why) {
        if (fits) *fits = false;
        return set_err(ctx, ZR_E_UNSUPPORTED, "microbatch does not fit the step graph's bucket: %s", why);
    };
    if (!mb) return set_err(ctx, ZR_E_INVALID, "null microbatch");
    const int S = mb->num_seqs;
    if (S <= 0 || S > ctx->desc.max_seqs)
        return set_err(ctx, ZR_E_INVALID, "microbatch has %d sequences (capacity %d)", S, ctx->desc.max_seqs);
    if (!mb->q_len || !mb->kv_before || !mb->first_pos || !mb->first_offset || !mb->block_tables)
        return set_err(ctx, ZR_E_INVALID, "microbatch arrays must not be null");
    const int stride = mb->block_table_stride;
    if (stride <= 0 || stride > ctx->desc.max_pages_per_seq)
        return set_err(ctx, ZR_E_INVALID, "block table stride %d outside 1..%d", stride, ctx->desc.max_pages_per_seq);
    if (!ctx->kv_pool) return set_err(ctx, ZR_E_INVALID, "KV pool not created");
    int total_q = 0, max_kv = 0;
    for (int s = 0; s < S; ++s) {
        const int ql = mb->q_len[s], kb = mb->kv_before[s], fo = mb->first_offset[s];
        if (ql <= 0) return set_err(ctx, ZR_E_INVALID, "sequence %d has q_len %d", s, ql);
        if (kb < 0 || fo < 0 || fo >= kPageRows || mb->first_pos[s] < 0)
            return set_err(ctx, ZR_E_INVALID, "sequence %d has kv_before %d first_offset %d first_pos %d", s, kb, fo,
                           mb->first_pos[s]);
        if (mb->first_pos[s] < kb)
            return set_err(ctx, ZR_E_INVARIANT, "sequence %d: first_pos %d precedes %d cached rows", s,
                           mb->first_pos[s], kb);
        const long need = ((long)fo + kb + ql + kPageRows - 1) / kPageRows;
        if (need > stride)
            return set_err(ctx, ZR_E_INVALID, "sequence %d needs %ld pages, block table holds %d", s, need, stride);
        for (long p = 0; p < need; ++p) {
            const int id = mb->block_tables[(size_t)s * stride + p];
            if (id < 0 || id >= ctx->n_pages)
                return set_err(ctx, ZR_E_INVARIANT, "sequence %d page slot %ld holds page %d outside pool of %d", s, p,
                               id, ctx->n_pages);
        }
        total_q += ql;
        max_kv = std::max(max_kv, kb + ql);
    }
    if (total_q > ctx->desc.max_tokens)
        return set_err(ctx, ZR_E_INVALID, "microbatch has %d tokens (capacity %d)", total_q, ctx->desc.max_tokens);
    if (mb->tokens)
        for (int t = 0; t < total_q; ++t)
            if (mb->tokens[t] >= (uint32_t)ctx->desc.vocab)
                return set_err(ctx, ZR_E_INVALID, "Token %u out of vocabulary bounds %d", mb->tokens[t],
                               ctx->desc.vocab);

    if (fixed && stride > fixed->stride) return no_fit("block table stride");
    const int blob_stride = fixed ? fixed->stride : stride;
    st->ctx = ctx;
    st->num_seqs = S;
    st->total_q = total_q;
    st->stride = blob_stride;
    st->max_kv = max_kv;

    // attention tiles / split items (the generic kernel of plain-layout pools
    // takes one workgroup per (row, q head) and needs none)
    const int G = ctx->q_per_kv, qpt = ctx->plain_kv ? 0 : 16 / G;
    st->h_tiles.clear();
    st->h_items.clear();
    st->h_pblocks.clear();
    st->h_psplits.clear();
    // sequences with >= 128 / G rows (prefill chunks) go to the prefill kernel
    // as blocks of 128 / G rows (bf16 pools, G dividing 32)
    int prows = 0;
    if (!ctx->plain_kv && ctx->desc.kv_dtype == ZR_DTYPE_BF16 && G <= 32 && 32 % G == 0) prows = 128 / G;
    if (const char* env = getenv("ZR_ATTN_PREFILL"))
        if (atoi(env) == 0) prows = 0;
    std::vector<int> tile_pages;
    std::vector<int4> pblk;  // prefill blocks {seq, r0, nrows, pages}
    long total_pages = 0, total_ktiles = 0;
    for (int s = 0; s < S && qpt > 0; ++s) {
        const int ql = mb->q_len[s], kb = mb->kv_before[s], fo = mb->first_offset[s];
        if (prows && ql >= prows) {
            for (int r0 = 0; r0 < ql; r0 += prows) {
                const int nr = std::min(prows, ql - r0);
                const int last_visible = kb + r0 + nr - 1;
                const int pages = (fo + last_visible + 1 + kPageRows - 1) / kPageRows;
                pblk.push_back(make_int4(s, r0, nr, pages));
                total_ktiles += (pages + 1) / 2;
            }
            continue;
        }
        for (int q0 = 0; q0 < ql; q0 += qpt) {
            const int nq = std::min(qpt, ql - q0);
            const int last_visible = kb + q0 + nq - 1;  // logical index of the tile's last key
            const int pages = (fo + last_visible + 1 + kPageRows - 1) / kPageRows;
            st->h_tiles.push_back(make_int4(s, q0, nq, 0));
            tile_pages.push_back(pages);
            total_pages += pages;
        }
    }
    // ~96 pages per split at 256 sessions x 8 kv heads x ~1.5k tokens (measured
    // best on MI355X with longest-first dispatch: 64 and 144 tie); at least 8
    // pages, which measured best at 32 sessions (a launch there costs ~8 us
    // plus ~0.45 us per page of a split: 12 pages 0.4 % slower, 16 1.2 %, 24 6 %)
    const long target_wgs = 2048;
    int pps = (int)std::min<long>(4096, std::max<long>(8, (total_pages * ctx->local_kv_heads + target_wgs - 1) / target_wgs));
    // and at most 16 splits per tile, which the merge combines in one round
    // trip; more take its general form (32 sessions at 3.5-4k contexts: 1.98
    // ms per step with 8-page splits, 32 per tile, against 1.76-1.81 with 16)
    {
        int max_pages = 0;
        for (int tp : tile_pages) max_pages = std::max(max_pages, tp);
        pps = std::max(pps, (max_pages + 15) / 16);
    }
    if (const char* env = getenv("ZR_ATTN_PAGES_PER_SPLIT")) pps = std::max(1, atoi(env));
    for (size_t t = 0; t < st->h_tiles.size(); ++t) {
        st->h_tiles[t].w = (int)st->h_items.size();
        for (int pb = 0; pb < tile_pages[t]; pb += pps)
            st->h_items.push_back(make_int4((int)t, pb, std::min(tile_pages[t], pb + pps), 0));
    }
    const int n_decode_tiles = (int)st->h_tiles.size();
    st->n_attn_items = (int)st->h_items.size();
    // A prefill workgroup takes its block's key tiles in steps of `kh`: with
    // kh = 2 its 8 waves are two halves of 4, each half streaming every other
    // tile for all of the block's columns, and the halves' (m, l, O) meet in
    // LDS at the end (no partials, no merge launch).  That halves the longest
    // block's chain of tiles at one 8-wave workgroup per CU instead of two
    // 4-wave ones (the 2108-row mixed microbatch, Llama-3 layer: prefill
    // kernel 89.2 against 96.9 us per layer with one half, rocprofv3 means).
    // ZR_ATTN_PREFILL_KEY_HALVES=1 / 2 forces either form.
    int kh = 2;
    if (const char* env = getenv("ZR_ATTN_PREFILL_KEY_HALVES")) kh = atoi(env) == 1 ? 1 : 2;
    st->prefill_kh = kh;
    // Prefill blocks split along their key tiles (32 keys each) when the
    // blocks alone leave CUs idle: about 512 / kh workgroups (the resident
    // slots: 2 / kh per CU), at least 16 kh key tiles per split.  Blocks that
    // fill the slots by themselves run unsplit (the 2108-row mixed
    // microbatch, 64 blocks x 8 kv heads, with 4-wave workgroups: 7.82-7.88 ms
    // per microbatch against 7.97-8.02 with 33-tile splits, whose merge takes
    // 0.19 of the 0.91 ms of attention + merge per 4 layers; running the
    // prefill kernel on a second stream beside the decode rows' attention
    // measured no faster either way).  A block with several splits writes
    // partials per 16-column group (16 / G rows x G heads, the decode tiles'
    // layout), one item per (group, split) after the decode items, and its
    // groups join the merge list as tiles.
    const long slots = 512 / kh;
    int tps = (int)std::max<long>(16 * kh, (total_ktiles * ctx->local_kv_heads + slots - 1) / slots);
    if ((long)pblk.size() * ctx->local_kv_heads >= slots) tps = 1 << 30;
    if (const char* env = getenv("ZR_ATTN_PREFILL_TILES_PER_SPLIT")) tps = std::max(1, atoi(env));
    if (G > 16) tps = 1 << 30;  // a 16-column group must hold whole rows
    int next_item = st->n_attn_items;
    for (const int4& b : pblk) {
        const int nt = (b.w + 1) / 2;
        const int ns = (nt + tps - 1) / tps;
        if (ns <= 1) {
            st->h_pblocks.push_back(b);
            st->h_psplits.push_back(make_int4(0, nt, -1, 1));
            continue;
        }
        const int rows_per_group = 16 / G;
        const int groups = (b.z + rows_per_group - 1) / rows_per_group;
        for (int sp = 0; sp < ns; ++sp) {
            st->h_pblocks.push_back(b);
            st->h_psplits.push_back(make_int4((int)((long)sp * nt / ns), (int)((long)(sp + 1) * nt / ns),
                                              next_item + sp, ns));
        }
        for (int k = 0; k < groups; ++k)
            st->h_tiles.push_back(make_int4(b.x, b.y + k * rows_per_group,
                                            std::min(rows_per_group, b.z - k * rows_per_group), next_item + k * ns));
        next_item += groups * ns;
    }
    st->n_part_items = next_item;
    st->h_tiles.push_back(make_int4(0, 0, 0, next_item));  // sentinel
    st->n_tiles = (int)st->h_tiles.size() - 1;
    // dispatch order: longest items first, so the short ones fill the tail
    st->h_order.resize(st->n_attn_items);
    for (int i = 0; i < st->n_attn_items; ++i) st->h_order[i] = i;
    std::stable_sort(st->h_order.begin(), st->h_order.end(), [&](int x, int y) {
        return st->h_items[x].z - st->h_items[x].y > st->h_items[y].z - st->h_items[y].y;
    });
    // tiles whose splits need the merge kernel (every prefill group tile has several)
    st->h_merge.clear();
    for (int t = 0; t < st->n_tiles; ++t)
        if (t >= n_decode_tiles || st->h_tiles[t + 1].w - st->h_tiles[t].w > 1) st->h_merge.push_back(t);
    st->n_merge = (int)st->h_merge.size();
    // Per-launch records in the order the kernels read them, so that a
    // workgroup's first page and Q loads wait on one metadata load instead of
    // a chain (rank -> item -> tile -> sequence arrays).
    {
        std::vector<int> cuq(S + 1, 0);
        for (int s = 0; s < S; ++s) cuq[s + 1] = cuq[s] + mb->q_len[s];
        if (st->n_part_items >= (int)kAttnSingle)
            return set_err(ctx, ZR_E_INVALID, "%d attention items exceed the record's index field", st->n_part_items);
        st->h_attn_rec.resize(3 * (size_t)st->n_attn_items);
        for (int r = 0; r < st->n_attn_items; ++r) {
            const int item = st->h_order[r];
            const int4 it = st->h_items[item], tl = st->h_tiles[it.x];
            const int first = tl.w, end = st->h_tiles[it.x + 1].w;
            const int seq = tl.x;
            unsigned meta = (unsigned)item;
            if (end - first == 1) meta |= kAttnSingle;
            if (item == end - 1) meta |= kAttnLast;
            const int* bt = mb->block_tables + (size_t)seq * stride;
            auto pid = [&](int k) { return it.y + k < it.z ? bt[it.y + k] : 0; };
            st->h_attn_rec[3 * r] = make_int4(seq, cuq[seq] + tl.y, tl.z, it.y);
            st->h_attn_rec[3 * r + 1] =
                make_int4(it.z, mb->kv_before[seq] + tl.y, mb->first_offset[seq], (int)meta);
            st->h_attn_rec[3 * r + 2] = make_int4(pid(0), pid(1), pid(2), pid(3));
        }
        st->h_merge_rec.resize(st->n_merge);
        for (int i = 0; i < st->n_merge; ++i) {
            const int t = st->h_merge[i];
            const int4 tl = st->h_tiles[t];
            st->h_merge_rec[i] = make_int4(tl.w, st->h_tiles[t + 1].w - tl.w, cuq[tl.x] + tl.y, tl.z);
        }
    }
    // prefill work units: most key tiles first
    {
        std::vector<int> ord(st->h_pblocks.size());
        for (size_t i = 0; i < ord.size(); ++i) ord[i] = (int)i;
        std::stable_sort(ord.begin(), ord.end(), [&](int x, int y) {
            return st->h_psplits[x].y - st->h_psplits[x].x > st->h_psplits[y].y - st->h_psplits[y].x;
        });
        std::vector<int4> b2(ord.size()), s2(ord.size());
        for (size_t i = 0; i < ord.size(); ++i) {
            b2[i] = st->h_pblocks[ord[i]];
            s2[i] = st->h_psplits[ord[i]];
        }
        st->h_pblocks.swap(b2);
        st->h_psplits.swap(s2);
    }
    st->n_pblocks = (int)st->h_pblocks.size();
    // every sequence one query row in the MFMA page layout: the decode kernel
    // can take RoPE + KV append too (launch_attention_rope).  The forward pass
    // does so when splits stream >= 48 pages: the q slab loads and the last
    // split's append then add little to a split (256 Llama-3 sessions, ~96
    // pages per split: 17.9 -> 17.3 ms per step), where 8- to 12-page splits
    // (32 TinyLlama sessions) lose more than the RoPE launch costs
    // (1.49 -> 1.59 ms).  ZR_ATTN_FUSE_ROPE=1 / 0 forces either path.
    st->pure_decode = !ctx->plain_kv && S > 0 && st->n_pblocks == 0;
    for (int s = 0; s < S && st->pure_decode; ++s) st->pure_decode = mb->q_len[s] == 1;
    st->fuse_rope = st->pure_decode && pps >= 48;
    if (const char* env = getenv("ZR_ATTN_FUSE_ROPE")) st->fuse_rope = st->pure_decode && atoi(env) != 0;
    st->grid_items = st->n_attn_items;
    st->grid_merge = st->n_merge;
    if (fixed) {
        if (!st->pure_decode || st->n_pblocks > 0) return no_fit("not a decode step of one row per sequence");
        if (fixed->plan_only) return ZR_OK;
        if (st->n_attn_items > fixed->items_cap) return no_fit("attention items");
        if (st->n_merge > fixed->merge_cap) return no_fit("split merges");
        st->fuse_rope = fixed->fuse_rope;
        st->grid_items = fixed->items_cap;
        st->grid_merge = fixed->merge_cap;
    }

    const size_t need_part = (size_t)st->n_part_items * ctx->local_kv_heads * 16 * (ctx->head_dim + 2);
    if (fixed && need_part > ctx->attn_part_floats) return no_fit("attention partial workspace");
    if (need_part > ctx->attn_part_floats) {
        hipStreamSynchronize(ctx->stream);
        if (ctx->attn_part) hipFree(ctx->attn_part);
        ++ctx->buffer_epoch;
        ctx->attn_part = nullptr;
        ctx->attn_part_floats = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->attn_part, need_part * sizeof(float)));
        ctx->attn_part_floats = need_part;
    }

    // one blob: inputs, derived arrays, attention items
    const BlobLayout L = blob_layout(S, blob_stride, total_q, st->grid_items, st->grid_merge, st->n_pblocks,
                                     ctx->head_dim);
    const size_t host_bytes = L.host_bytes, total_bytes = L.total_bytes;
    unsigned char* hb;
    if (fixed) {
        if (total_bytes > fixed->dev_cap || host_bytes > fixed->host_cap)
            return set_err(ctx, ZR_E_INVARIANT, "step graph blob of %zu bytes holds %zu", fixed->dev_cap, total_bytes);
        st->dev = fixed->dev;
        st->cap_bytes = fixed->dev_cap;
        st->owns = false;
        hb = fixed->host;
    } else {
        if (total_bytes > st->cap_bytes) {
            hipStreamSynchronize(ctx->stream);
            if (st->dev) hipFree(st->dev);
            st->dev = nullptr;
            st->cap_bytes = 0;
            ZR_HIP(ctx, hipMalloc(&st->dev, total_bytes));
            st->cap_bytes = total_bytes;
        }
        st->h_blob.assign(host_bytes, 0);
        hb = st->h_blob.data();
    }
    st->dev_bytes = total_bytes;
    memcpy(hb + L.o_qlen, mb->q_len, 4 * S);
    memcpy(hb + L.o_kvb, mb->kv_before, 4 * S);
    memcpy(hb + L.o_fpos, mb->first_pos, 4 * S);
    memcpy(hb + L.o_foff, mb->first_offset, 4 * S);
    if (blob_stride == stride) {
        memcpy(hb + L.o_bt, mb->block_tables, 4 * (size_t)S * stride);
    } else {  // a bucket's wider table: each row's pages, the rest of the row zero (pool page 0)
        int* bt = (int*)(hb + L.o_bt);
        for (int s = 0; s < S; ++s) {
            memcpy(bt + (size_t)s * blob_stride, mb->block_tables + (size_t)s * stride, 4 * (size_t)stride);
            memset(bt + (size_t)s * blob_stride + stride, 0, 4 * (size_t)(blob_stride - stride));
        }
    }
    if (mb->tokens) memcpy(hb + L.o_tok, mb->tokens, 4 * (size_t)total_q);
    if (st->n_attn_items) memcpy(hb + L.o_arec, st->h_attn_rec.data(), 48 * (size_t)st->n_attn_items);
    if (st->grid_items > st->n_attn_items)  // empty records (nq = 0): their workgroups return at once
        memset(hb + L.o_arec + 48 * (size_t)st->n_attn_items, 0, 48 * (size_t)(st->grid_items - st->n_attn_items));
    if (st->n_merge) memcpy(hb + L.o_mrec, st->h_merge_rec.data(), 16 * (size_t)st->n_merge);
    if (st->grid_merge > st->n_merge)
        memset(hb + L.o_mrec + 16 * (size_t)st->n_merge, 0, 16 * (size_t)(st->grid_merge - st->n_merge));
    if (st->n_pblocks) memcpy(hb + L.o_pblk, st->h_pblocks.data(), 16 * (size_t)st->n_pblocks);
    if (st->n_pblocks) memcpy(hb + L.o_psplit, st->h_psplits.data(), 16 * (size_t)st->n_pblocks);
    unsigned char* db = (unsigned char*)st->dev;
    st->q_len = (int*)(db + L.o_qlen);
    st->kv_before = (int*)(db + L.o_kvb);
    st->first_pos = (int*)(db + L.o_fpos);
    st->first_offset = (int*)(db + L.o_foff);
    st->block_tables = (int*)(db + L.o_bt);
    st->tokens = (uint32_t*)(db + L.o_tok);
    st->attn_rec = (int4*)(db + L.o_arec);
    st->merge_rec = (int4*)(db + L.o_mrec);
    st->pblocks = (int4*)(db + L.o_pblk);
    st->psplits = (int4*)(db + L.o_psplit);
    st->cu_q = (int*)(db + L.o_cuq);
    st->cu_k = (int*)(db + L.o_cuk);
    st->positions = (int*)(db + L.o_pos);
    st->slot_mapping = (int*)(db + L.o_slot);
    st->seq_ids = (int*)(db + L.o_seq);
    st->last_rows = (int*)(db + L.o_last);
    st->rope_cs = (float2*)(db + L.o_rcs);
    st->h_q_len.assign(mb->q_len, mb->q_len + S);
    st->h_kv_before.assign(mb->kv_before, mb->kv_before + S);
    if (fixed) return ZR_OK;  // the step graph copies the host blob and runs the pack stage
    ZR_HIP(ctx, hipMemcpyAsync(st->dev, hb, host_bytes, hipMemcpyHostToDevice, ctx->stream));
    return launch_pack(ctx, st);
}

// ----------------------------------------------------------- forward pass
static zr_status check_ready(zr_context* ctx) {
    if (!ctx->embedding || !ctx->lm_head || !ctx->final_norm)
        return set_err(ctx, ZR_E_INVALID, "global weights not uploaded");
    for (int l = 0; l < ctx->desc.num_layers; ++l)
        if (!ctx->layers[l].w_qkv) return set_err(ctx, ZR_E_INVALID, "layer %d weights not uploaded", l);
    if (!ctx->kv_pool) return set_err(ctx, ZR_E_INVALID, "KV pool not created");
    return ZR_OK;
}

static zr_status run_forward(zr_context* ctx, StagedMeta* st, const uint32_t* d_tokens, uint32_t* d_out_tokens,
                             float* d_out_logits, float* h_partials) {
    zr_status rc = check_ready(ctx);
    if (rc) return rc;
    const zr_model_desc& d = ctx->desc;
    const int T = st->total_q, S = st->num_seqs, H = d.hidden, F = d.ffn_cols;
    (void)S;
    const int QKV = ctx->q_cols + 2 * ctx->kv_cols;
    if ((rc = launch_embed(ctx, st, d_tokens ? d_tokens : st->tokens, d_tokens != nullptr))) return rc;
    const int lo = (d.flags & ZR_FLAG_SPLIT_ACTIVATIONS) ? 1 : 0;
    // split-K products are left as slabs for the next kernel to sum, except
    // where the caller asked for the per-layer partials (those are copied out)
    Slabs down(nullptr);
    for (int l = 0; l < d.num_layers; ++l) {
        const LayerDev& L = ctx->layers[l];
        Slabs* defer = h_partials ? nullptr : &down;
        // hidden += previous down partial; xa = rms_norm(hidden) * attn_norm
        if ((rc = launch_rms_norm(ctx, ctx->hidden, l > 0 ? down : Slabs(nullptr), ctx->hidden, L.attn_norm, nullptr,
                                  ctx->xa, lo, nullptr, T, H)))
            return rc;
        Slabs qkv(ctx->qkv);
        if ((rc = launch_gemm(ctx, ctx->xa, L.w_qkv, ctx->qkv, nullptr, T, QKV, H, kEpiStore, &qkv))) return rc;
        if (st->fuse_rope) {  // RoPE + KV append inside the decode attention launch
            if ((rc = launch_attention_rope(ctx, st, l, qkv, 1, nullptr, ctx->attn_a))) return rc;
        } else {
            if ((rc = launch_rope_kv_write(ctx, st, l, qkv, ctx->q_rope, 1))) return rc;
            if ((rc = launch_attention(ctx, st, l, ctx->q_rope, nullptr, ctx->attn_a))) return rc;
        }
        Slabs o(ctx->proj);
        if ((rc = launch_gemm(ctx, ctx->attn_a, L.w_o, ctx->proj, nullptr, T, H, ctx->q_cols, kEpiStore,
                              h_partials ? nullptr : &o)))
            return rc;
        if (h_partials)
            ZR_HIP(ctx, hipMemcpyAsync(h_partials + ((size_t)l * 2 + 0) * T * H, ctx->proj, sizeof(float) * T * H,
                                       hipMemcpyDeviceToHost, ctx->stream));
        // post_attn = hidden + o_partial (identity all-reduce at one worker)
        if ((rc = launch_rms_norm(ctx, ctx->hidden, o, ctx->hidden, L.mlp_norm, nullptr, ctx->xa, lo, nullptr,
                                  T, H)))
            return rc;
        if ((rc = launch_gemm(ctx, ctx->xa, L.w_gate_up, nullptr, ctx->ffn_a, T, 2 * F, H, kEpiSwiGLU))) return rc;
        down = Slabs(ctx->proj);
        if ((rc = launch_gemm(ctx, ctx->ffn_a, L.w_down, ctx->proj, nullptr, T, H, F, kEpiStore, defer))) return rc;
        if (h_partials)
            ZR_HIP(ctx, hipMemcpyAsync(h_partials + ((size_t)l * 2 + 1) * T * H, ctx->proj, sizeof(float) * T * H,
                                       hipMemcpyDeviceToHost, ctx->stream));
    }
    // final residual + norm on the last row of every sequence, LM head, argmax
    if ((rc = launch_rms_norm(ctx, ctx->hidden, down, ctx->hidden, ctx->final_norm, nullptr, ctx->final_a, lo,
                              st->last_rows, S, H)))
        return rc;
    float* logits = ctx->logits;
    if ((rc = launch_gemm(ctx, ctx->final_a, ctx->lm_head, logits, nullptr, S, d.vocab, H, kEpiStore))) return rc;
    if ((rc = launch_argmax(ctx, logits, S, d.vocab, d_out_tokens ? d_out_tokens : ctx->tokens_out))) return rc;
    if (d_out_logits)
        ZR_HIP(ctx, hipMemcpyAsync(d_out_logits, logits, sizeof(float) * S * d.vocab, hipMemcpyDeviceToDevice,
                                   ctx->stream));
    if (d_tokens) {  // the id check of device-fed tokens, read by zr_synchronize
        ZR_HIP(ctx, hipMemcpyAsync(ctx->h_token_err, ctx->d_token_err, sizeof(unsigned long long),
                                   hipMemcpyDeviceToHost, ctx->stream));
        ctx->token_check_pending = true;
    }
    return ZR_OK;
}

}  // namespace zr

using namespace zr;

// ============================================================ C ABI ======
extern "C" {

const char* zr_global_last_error(void) { return g_err.c_str(); }
const char* zr_last_error(const zr_context* ctx) { return ctx ? ctx->err.c_str() : g_err.c_str(); }

zr_status zr_probe(int device, zr_device_info* out) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return set_global_err(ZR_E_NODEVICE, "no HIP device available (%s)", hipGetErrorString(e));
    if (device < 0 || device >= count) return set_global_err(ZR_E_INVALID, "device %d outside 0..%d", device, count - 1);
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return set_global_err(ZR_E_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (out) {
        memset(out, 0, sizeof *out);
        out->device_count = count;
        out->device = device;
        out->compute_units = p.multiProcessorCount;
        out->clock_mhz = p.clockRate / 1000;
        out->hbm_bytes = p.totalGlobalMem;
        snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    }
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return set_global_err(ZR_E_NODEVICE, "device %d is %s, this provider is built for gfx950", device,
                              p.gcnArchName);
    return ZR_OK;
}

zr_status zr_context_create(const zr_model_desc* desc, int device, zr_context** out) {
    if (!desc || !out) return set_global_err(ZR_E_INVALID, "null argument");
    *out = nullptr;
    zr_status rc = ZR_OK;
    zr_context* ctx = new zr_context();
    ctx->desc = *desc;
    ctx->device = device;
    const zr_model_desc& d = ctx->desc;
    if (d.page_tokens != kPageRows) rc = set_err(ctx, ZR_E_UNSUPPORTED, "page_tokens must be 16, got %d", d.page_tokens);
    else if (d.kv_dtype != ZR_DTYPE_BF16 && d.kv_dtype != ZR_DTYPE_F32) rc = set_err(ctx, ZR_E_INVALID, "kv_dtype %d", d.kv_dtype);
    else if (d.num_layers <= 0 || d.vocab <= 0 || d.ffn_cols <= 0 || d.max_tokens <= 0 || d.max_seqs <= 0 ||
             d.max_pages_per_seq <= 0)
        rc = set_err(ctx, ZR_E_INVALID, "model descriptor has a non-positive size");
    else if (d.hidden % 32 != 0 || d.ffn_cols % 32 != 0)
        rc = set_err(ctx, ZR_E_UNSUPPORTED, "hidden %d / ffn %d must be multiples of 32", d.hidden, d.ffn_cols);
    if (!rc) rc = resolve_geometry(ctx);
    if (!rc) {
        // The GEMM kernels address each operand with 32-bit buffer offsets
        // (launch_gemm): every packed weight and every A operand at max_tokens
        // rows (bf16 hi + lo planes) stays below 2 GiB, refused here rather
        // than mid-step.
        const int H = d.hidden, Q = ctx->q_cols, KVc = ctx->kv_cols, F = d.ffn_cols;
        const struct {
            const char* name;
            int k, n;
        } w[] = {{"w_qkv", H, Q + 2 * KVc}, {"w_o", Q, H}, {"w_gate_up", H, 2 * F}, {"w_down", F, H},
                 {"lm_head", H, d.vocab}};
        for (const auto& x : w)
            if (!rc && 2 * packed_weight_elems(x.k, x.n) > 0x7fffffffull)
                rc = set_err(ctx, ZR_E_UNSUPPORTED, "packed %s [%d, %d] exceeds the GEMM's 2 GiB operand limit", x.name,
                             x.k, x.n);
        const int widest_k = std::max(H, std::max(Q, F));
        if (!rc && 2 * 2 * a_plane(d.max_tokens, widest_k) > 0x7fffffffull)
            rc = set_err(ctx, ZR_E_UNSUPPORTED, "max_tokens %d x K %d activations exceed the GEMM's 2 GiB operand limit",
                         d.max_tokens, widest_k);
    }
    if (!rc) {
        rc = zr_probe(device, nullptr);  // geometry errors are reported before device errors
        if (rc) ctx->err = g_err;
    }
    if (rc) {
        set_global_err(rc, "%s", ctx->err.c_str());
        delete ctx;
        return rc;
    }
    auto fail = [&](hipError_t e, const char* what) {
        set_global_err(ZR_E_HIP, "%s: %s", what, hipGetErrorString(e));
        free_ctx_buffers(ctx);
        destroy_streams(ctx);
        delete ctx;
        return e == hipErrorOutOfMemory ? ZR_E_OOM : ZR_E_HIP;
    };
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return fail(e, "hipSetDevice");
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->d2h_stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->h2d_stream, hipStreamNonBlocking);
    if (e != hipSuccess) return fail(e, "hipStreamCreate");
    const size_t T = d.max_tokens, S = d.max_seqs, H = d.hidden, Q = ctx->q_cols, KV = ctx->kv_cols, F = d.ffn_cols;
    struct {
        void** p;
        size_t bytes;
    } allocs[] = {
        {(void**)&ctx->hidden, 4 * T * H},
        {(void**)&ctx->xa, 2 * 2 * a_plane((int)T, (int)H)},
        {(void**)&ctx->qkv, 4 * T * (Q + 2 * KV)},   {(void**)&ctx->q_rope, 4 * T * Q},
        {(void**)&ctx->attn_a, 2 * 2 * a_plane((int)T, (int)Q)},
        {(void**)&ctx->proj, 4 * T * H},
        {(void**)&ctx->ffn_a, 2 * 2 * a_plane((int)T, (int)F)},
        {(void**)&ctx->logits, 4 * S * d.vocab},
        {(void**)&ctx->final_a, 2 * 2 * a_plane((int)S, (int)H)},
        {(void**)&ctx->tokens_out, 4 * S},
        {(void**)&ctx->inv_freq, 4 * (size_t)ctx->head_dim / 2},
        {(void**)&ctx->d_token_err, sizeof(unsigned long long)},
    };
    for (auto& a : allocs) {
        e = hipMalloc(a.p, a.bytes);
        if (e != hipSuccess) return fail(e, "hipMalloc activations");
    }
    // split-K workspace: max over every row count a microbatch can have (the
    // plan changes with m, so no grid of sample sizes bounds it): 1..T rows
    // for the layer GEMMs, 1..S for the LM head
    size_t ws = 0;
    for (size_t m = 1; m <= T; ++m) {
        const int mm = (int)m;
        ws = std::max(ws, gemm_ws_floats(mm, (int)(Q + 2 * KV), (int)H, kEpiStore));
        ws = std::max(ws, gemm_ws_floats(mm, (int)H, (int)Q, kEpiStore));
        ws = std::max(ws, gemm_ws_floats(mm, (int)(2 * F), (int)H, kEpiSwiGLU));
        ws = std::max(ws, gemm_ws_floats(mm, (int)H, (int)F, kEpiStore));
        if (m <= S) ws = std::max(ws, gemm_ws_floats(mm, d.vocab, (int)H, kEpiStore));
    }
    ws = std::max<size_t>(ws, 1);
    e = hipMalloc(&ctx->splitk_ws, ws * 4);
    if (e != hipSuccess) return fail(e, "hipMalloc split-K workspace");
    ctx->splitk_ws_floats = ws;
    ctx->argmax_ws_floats = S * ((d.vocab + 4095) / 4096) * 2;
    e = hipMalloc(&ctx->argmax_ws, ctx->argmax_ws_floats * 4);
    if (e != hipSuccess) return fail(e, "hipMalloc argmax workspace");
    // RoPE inverse frequencies with the host powf, exactly as the reference
    // builds them (runtime.rs:282-301): 1 / base^(2i / d) in f32.
    std::vector<float> inv(ctx->head_dim / 2);
    for (int i = 0; i < ctx->head_dim / 2; ++i)
        inv[i] = 1.0f / powf(d.rope_base, (float)i * 2.0f / (float)ctx->head_dim);
    e = hipMemcpy(ctx->inv_freq, inv.data(), inv.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(e, "hipMemcpy inv_freq");
    if (zr_status src = noalloc_scratch_init(ctx)) {
        const std::string why = ctx->err;
        set_global_err(src, "%s", why.c_str());
        free_ctx_buffers(ctx);
        destroy_streams(ctx);
        delete ctx;
        return src;
    }
    e = hipHostMalloc((void**)&ctx->h_token_err, sizeof(unsigned long long), hipHostMallocDefault);
    if (e != hipSuccess) return fail(e, "hipHostMalloc token check word");
    *ctx->h_token_err = ~0ull;
    e = hipMemcpy(ctx->d_token_err, ctx->h_token_err, sizeof(unsigned long long), hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(e, "hipMemcpy token check word");
    ctx->layers.resize(d.num_layers);
    ctx->scratch_stage = new StagedMeta();
    *out = ctx;
    return ZR_OK;
}

void zr_context_destroy(zr_context* ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    for (hipStream_t st : {ctx->stream, ctx->d2h_stream, ctx->h2d_stream})
        if (st) hipStreamSynchronize(st);
    if (ctx->fwd_graph) zr_step_graph_destroy(ctx->fwd_graph);
    if (ctx->fwd_ids) (void)hipFree(ctx->fwd_ids);
    if (ctx->fwd_h_ids) (void)hipHostFree(ctx->fwd_h_ids);
    for (auto& fb : ctx->xfer_free) (void)hipFree(fb.first);
    ctx->xfer_free.clear();
    if (ctx->scratch_stage) {
        if (ctx->scratch_stage->dev) hipFree(ctx->scratch_stage->dev);
        delete ctx->scratch_stage;
    }
    for (hipEvent_t e : ctx->timing.pool) hipEventDestroy(e);
    if (ctx->kv_stage) (void)hipFree(ctx->kv_stage);
    if (ctx->cbor_ws) (void)hipFree(ctx->cbor_ws);
    if (ctx->cbor_out) (void)hipFree(ctx->cbor_out);
    if (ctx->sample_ws) (void)hipFree(ctx->sample_ws);
    free_ctx_buffers(ctx);
    destroy_streams(ctx);
    delete ctx;
}

zr_status zr_kv_head_map(const zr_context* ctx, uint32_t* out, int capacity, int* count) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    if (count) *count = (int)ctx->kv_head_map.size();
    if (out) {
        if (capacity < (int)ctx->kv_head_map.size()) return set_global_err(ZR_E_INVALID, "capacity too small");
        std::copy(ctx->kv_head_map.begin(), ctx->kv_head_map.end(), out);
    }
    return ZR_OK;
}

zr_status zr_upload_layer(zr_context* ctx, int layer, const zr_layer_weights* w) {
    if (!ctx || !w) return set_global_err(ZR_E_INVALID, "null argument");
    if (layer < 0 || layer >= ctx->desc.num_layers) return set_err(ctx, ZR_E_INVALID, "Invalid layer index: %d", layer);
    if (!w->w_q || !w->w_k || !w->w_v || !w->w_o || !w->w_gate || !w->w_up || !w->w_down || !w->attn_norm ||
        !w->mlp_norm)
        return set_err(ctx, ZR_E_INVALID, "layer %d: null weight pointer", layer);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    LayerDev& L = ctx->layers[layer];
    LayerDev fresh;
    const int H = ctx->desc.hidden, F = ctx->desc.ffn_cols;
    const uint16_t* qkv[3] = {w->w_q, w->w_k, w->w_v};
    const int widths[3] = {ctx->q_cols, ctx->kv_cols, ctx->kv_cols};
    zr_status rc = pack_weight_concat(ctx, qkv, widths, 3, H, &fresh.w_qkv);
    if (!rc) rc = pack_weight(ctx, w->w_o, ctx->q_cols, H, &fresh.w_o);
    if (!rc) rc = pack_weight_gate_up(ctx, w->w_gate, w->w_up, H, F, &fresh.w_gate_up);
    if (!rc) rc = pack_weight(ctx, w->w_down, F, H, &fresh.w_down);
    if (!rc) {
        hipError_t e = hipMalloc(&fresh.attn_norm, 4 * (size_t)H);
        if (e == hipSuccess) e = hipMalloc(&fresh.mlp_norm, 4 * (size_t)H);
        if (e == hipSuccess) e = hipMemcpy(fresh.attn_norm, w->attn_norm, 4 * (size_t)H, hipMemcpyDefault);
        if (e == hipSuccess) e = hipMemcpy(fresh.mlp_norm, w->mlp_norm, 4 * (size_t)H, hipMemcpyDefault);
        if (e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "norm upload: %s", hipGetErrorString(e));
    }
    if (rc) {
        void* lb[] = {fresh.w_qkv, fresh.w_o, fresh.w_gate_up, fresh.w_down, fresh.attn_norm, fresh.mlp_norm};
        for (void* b : lb)
            if (b) hipFree(b);
        return rc;
    }
    void* old[] = {L.w_qkv, L.w_o, L.w_gate_up, L.w_down, L.attn_norm, L.mlp_norm};
    for (void* b : old)
        if (b) hipFree(b);
    if (L.w_qkv) ++ctx->buffer_epoch;
    L = fresh;
    return ZR_OK;
}

zr_status zr_upload_globals(zr_context* ctx, const uint16_t* embedding, const float* final_norm,
                            const uint16_t* lm_head) {
    if (!ctx || !embedding || !final_norm || !lm_head) return set_global_err(ZR_E_INVALID, "null argument");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    const size_t H = ctx->desc.hidden, V = ctx->desc.vocab;
    uint16_t* emb = nullptr;
    float* fn = nullptr;
    uint16_t* head = nullptr;
    hipError_t e = hipMalloc(&emb, 2 * V * H);
    if (e == hipSuccess) e = hipMemcpy(emb, embedding, 2 * V * H, hipMemcpyDefault);
    if (e == hipSuccess) e = hipMalloc(&fn, 4 * H);
    if (e == hipSuccess) e = hipMemcpy(fn, final_norm, 4 * H, hipMemcpyDefault);
    zr_status rc = e == hipSuccess ? ZR_OK : set_err(ctx, ZR_E_HIP, "global upload: %s", hipGetErrorString(e));
    if (!rc) rc = pack_weight(ctx, lm_head, (int)H, (int)V, &head);
    if (rc) {
        if (emb) hipFree(emb);
        if (fn) hipFree(fn);
        if (head) hipFree(head);
        return rc;
    }
    if (ctx->embedding) ++ctx->buffer_epoch;
    if (ctx->embedding) hipFree(ctx->embedding);
    if (ctx->final_norm) hipFree(ctx->final_norm);
    if (ctx->lm_head) hipFree(ctx->lm_head);
    ctx->embedding = emb;
    ctx->final_norm = fn;
    ctx->lm_head = head;
    return ZR_OK;
}

zr_status zr_kv_pool_create(zr_context* ctx, int n_pages) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    if (n_pages <= 0) return set_err(ctx, ZR_E_INVALID, "n_pages %d", n_pages);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    const size_t esz = ctx->desc.kv_dtype == ZR_DTYPE_BF16 ? 2 : 4;
    const size_t page_bytes = (size_t)2 * ctx->kv_cols * kPageRows * esz;
    const size_t total = page_bytes * n_pages * ctx->desc.num_layers;
    if (ctx->kv_pool) {
        hipStreamSynchronize(ctx->stream);
        hipFree(ctx->kv_pool);
        ++ctx->buffer_epoch;
        ctx->kv_pool = nullptr;
        ctx->n_pages = 0;
    }
    hipError_t e = hipMalloc(&ctx->kv_pool, total);
    if (e != hipSuccess)
        return set_err(ctx, e == hipErrorOutOfMemory ? ZR_E_OOM : ZR_E_HIP, "KV pool of %zu bytes: %s", total,
                       hipGetErrorString(e));
    ZR_HIP(ctx, hipMemsetAsync(ctx->kv_pool, 0, total, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ctx->n_pages = n_pages;
    ctx->page_bytes = page_bytes;
    return ZR_OK;
}

int zr_kv_pool_pages(const zr_context* ctx) { return ctx ? ctx->n_pages : 0; }
uint64_t zr_kv_pool_bytes(const zr_context* ctx) {
    return ctx ? (uint64_t)ctx->page_bytes * ctx->n_pages * ctx->desc.num_layers : 0;
}

zr_status zr_stage(zr_context* ctx, const zr_microbatch* mb, zr_staged** out) {
    if (!ctx || !out) return set_global_err(ZR_E_INVALID, "null argument");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    StagedMeta* st = new StagedMeta();
    zr_status rc = stage_microbatch(ctx, mb, st);
    if (rc) {
        if (st->dev) hipFree(st->dev);
        delete st;
        return rc;
    }
    st->id = ctx->next_staged_id++;
    ctx->live_staged.push_back(st->id);
    *out = (zr_staged*)st;
    return ZR_OK;
}

void zr_staged_destroy(zr_staged* s) {
    StagedMeta* st = (StagedMeta*)s;
    if (!st) return;
    if (st->ctx) {
        hipStreamSynchronize(st->ctx->stream);
        auto& live = st->ctx->live_staged;
        live.erase(std::remove(live.begin(), live.end(), st->id), live.end());
    }
    if (st->dev) hipFree(st->dev);
    delete st;
}

zr_status zr_forward_staged_async(zr_context* ctx, zr_staged* s, const uint32_t* d_tokens, uint32_t* d_out_tokens,
                                  float* d_out_logits) {
    StagedMeta* st = (StagedMeta*)s;
    if (!ctx || !st || st->ctx != ctx) return set_global_err(ZR_E_INVALID, "staged microbatch of another context");
    return run_forward(ctx, st, d_tokens, d_out_tokens, d_out_logits, nullptr);
}

zr_status zr_synchronize(zr_context* ctx) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->token_check_pending) {
        ctx->token_check_pending = false;
        const unsigned long long bad = *ctx->h_token_err;
        if (bad != ~0ull) {
            const unsigned long long none = ~0ull;
            *ctx->h_token_err = none;
            ZR_HIP(ctx, hipMemcpy(ctx->d_token_err, &none, sizeof none, hipMemcpyHostToDevice));
            // embed_tokens (tensor_ops.rs:482-490)
            return set_err(ctx, ZR_E_INVALID, "Token %u out of vocabulary bounds %d", (unsigned)(bad & 0xffffffffu),
                           ctx->desc.vocab);
        }
    }
    return ZR_OK;
}

struct zr_graph {
    zr_context* ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool token_check = false;  // the step copies the device id-check word to the host
    uint64_t buffer_epoch = 0; // the context's buffer epoch at capture
    uint64_t staged_id = 0;    // the staged microbatch the graph replays
};

zr_status zr_graph_capture_staged(zr_context* ctx, zr_staged* s, const uint32_t* d_tokens, uint32_t* d_out_tokens,
                                  float* d_out_logits, zr_graph** out) {
    StagedMeta* st = (StagedMeta*)s;
    if (!ctx || !st || !out) return set_global_err(ZR_E_INVALID, "null argument");
    if (st->ctx != ctx) return set_err(ctx, ZR_E_INVALID, "staged microbatch of another context");
    // HIP events recorded by graph nodes do not time (hipEventElapsedTime
    // reports an invalid handle for them), so timing stays eager-only
    if (ctx->timing.enabled) return set_err(ctx, ZR_E_INVALID, "graph capture with per-class timing on");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    // a step pending on the stream finishes first; its id check stays pending
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const bool pending = ctx->token_check_pending;
    ZR_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    zr_status rc = run_forward(ctx, st, d_tokens, d_out_tokens, d_out_logits, nullptr);
    hipGraph_t graph = nullptr;
    const hipError_t e_end = hipStreamEndCapture(ctx->stream, &graph);
    ctx->token_check_pending = pending;  // nothing ran yet
    if (!rc && e_end != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "graph capture: %s", hipGetErrorString(e_end));
    hipGraphExec_t exec = nullptr;
    if (!rc) {
        const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "graph instantiate: %s", hipGetErrorString(e));
    }
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipGetLastError();
        return rc;
    }
    zr_graph* g = new zr_graph;
    g->ctx = ctx;
    g->graph = graph;
    g->exec = exec;
    g->token_check = d_tokens != nullptr;
    g->buffer_epoch = ctx->buffer_epoch;
    g->staged_id = st->id;
    *out = g;
    return ZR_OK;
}

zr_status zr_graph_launch(zr_context* ctx, zr_graph* g) {
    if (!ctx || !g) return set_global_err(ZR_E_INVALID, "null argument");
    if (g->ctx != ctx) return set_err(ctx, ZR_E_INVALID, "graph of another context");
    if (g->buffer_epoch != ctx->buffer_epoch)
        return set_err(ctx, ZR_E_INVALID,
                       "graph captured before a workspace, the KV pool or weights were reallocated: capture it again");
    if (std::find(ctx->live_staged.begin(), ctx->live_staged.end(), g->staged_id) == ctx->live_staged.end())
        return set_err(ctx, ZR_E_INVALID, "the graph's staged microbatch was destroyed: stage and capture again");
    ZR_HIP(ctx, hipGraphLaunch(g->exec, ctx->stream));
    if (g->token_check) ctx->token_check_pending = true;
    return ZR_OK;
}

void zr_graph_destroy(zr_graph* g) {
    if (!g) return;
    if (g->ctx && g->ctx->stream) (void)hipStreamSynchronize(g->ctx->stream);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

}  // extern "C"

// ------------------------------------------------------------ step graphs
// One decode step captured per bucket and replayed for every later step that
// fits the bucket, each launch with its own metadata.  Two blobs alternate:
// step i stages into pinned host buffer i % 2 (after that buffer's previous
// copy has finished), a copy stream moves it into device blob i % 2 once the
// replay that last read the blob (step i - 2) has finished, and the replay of
// step i waits for that copy.  The host staging of step i + 1 overlaps step i
// on the device.
struct zr_step_graph {
    zr_context* ctx = nullptr;
    hipStream_t copy = nullptr;
    bool valid = false;          // a bucket is set up
    int S = 0;                   // sequences of the bucket
    uint64_t epoch = 0;          // the context's buffer epoch at set-up
    StageFixed fixed[2];
    size_t host_bytes = 0;       // host part of a blob (copied per step)
    unsigned char* pinned[2] = {nullptr, nullptr};
    void* dev[2] = {nullptr, nullptr};
    size_t host_cap = 0, dev_cap = 0;
    hipEvent_t copied[2] = {nullptr, nullptr};    // the copy into blob b has finished
    hipEvent_t replayed[2] = {nullptr, nullptr};  // the replay that read blob b has finished
    bool copy_pending[2] = {false, false}, replay_pending[2] = {false, false};
    StagedMeta st[2];
    struct Exec {
        const uint32_t* in;
        uint32_t* out;
        int blob;
        hipGraph_t graph;
        hipGraphExec_t exec;
    };
    std::vector<Exec> execs;
    uint64_t launches = 0;
    int captures = 0, buckets = 0;
};

namespace {

void step_graph_drop_execs(zr_step_graph* g) {
    for (auto& e : g->execs) {
        if (e.exec) (void)hipGraphExecDestroy(e.exec);
        if (e.graph) (void)hipGraphDestroy(e.graph);
    }
    g->execs.clear();
}

zr_status step_graph_quiesce(zr_step_graph* g) {
    zr_context* ctx = g->ctx;
    ZR_HIP(ctx, hipStreamSynchronize(g->copy));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int b = 0; b < 2; ++b) g->copy_pending[b] = g->replay_pending[b] = false;
    return ZR_OK;
}

// Sizes a bucket for the sequence count and the counts of `mb` with room to
// grow: records for 1.25x the step's attention items (+64) and merges (+16),
// the context's widest block table, and the step's RoPE placement.
zr_status step_graph_setup(zr_step_graph* g, const zr_microbatch* mb) {
    zr_context* ctx = g->ctx;
    StagedMeta probe;
    StageFixed plan;
    plan.plan_only = true;
    plan.stride = ctx->desc.max_pages_per_seq;
    bool fits = true;
    zr_status rc = stage_microbatch(ctx, mb, &probe, &plan, &fits);
    if (rc) return rc;  // not a decode step of one row per sequence, or invalid
    if ((rc = step_graph_quiesce(g))) return rc;
    step_graph_drop_execs(g);
    g->valid = false;
    StageFixed f;
    f.stride = ctx->desc.max_pages_per_seq;
    f.items_cap = (probe.n_attn_items + std::max(64, probe.n_attn_items / 4) + 7) / 8 * 8;
    f.merge_cap = probe.n_merge + std::max(16, probe.n_merge / 4);
    f.fuse_rope = probe.fuse_rope;
    // partials of every item a step of the bucket can hold (decode items only)
    const size_t need_part = (size_t)f.items_cap * ctx->local_kv_heads * 16 * (ctx->head_dim + 2);
    if (need_part > ctx->attn_part_floats) {
        if (ctx->attn_part) hipFree(ctx->attn_part);
        ++ctx->buffer_epoch;
        ctx->attn_part = nullptr;
        ctx->attn_part_floats = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->attn_part, need_part * sizeof(float)));
        ctx->attn_part_floats = need_part;
    }
    size_t hbytes = 0, dbytes = 0;
    stage_fixed_bytes(ctx, mb->num_seqs, probe.total_q, f, &hbytes, &dbytes);
    for (int b = 0; b < 2; ++b) {
        if (hbytes > g->host_cap) {
            if (g->pinned[b]) (void)hipHostFree(g->pinned[b]);
            g->pinned[b] = nullptr;
            ZR_HIP(ctx, hipHostMalloc((void**)&g->pinned[b], hbytes, hipHostMallocDefault));
        }
        if (dbytes > g->dev_cap) {
            if (g->dev[b]) (void)hipFree(g->dev[b]);
            g->dev[b] = nullptr;
            ZR_HIP(ctx, hipMalloc(&g->dev[b], dbytes));
        }
    }
    g->host_cap = std::max(g->host_cap, hbytes);
    g->dev_cap = std::max(g->dev_cap, dbytes);
    for (int b = 0; b < 2; ++b) {
        g->fixed[b] = f;
        g->fixed[b].host = g->pinned[b];
        g->fixed[b].host_cap = g->host_cap;
        g->fixed[b].dev = g->dev[b];
        g->fixed[b].dev_cap = g->dev_cap;
    }
    g->host_bytes = hbytes;
    g->S = mb->num_seqs;
    g->epoch = ctx->buffer_epoch;
    g->valid = true;
    ++g->buckets;
    return ZR_OK;
}

zr_status step_graph_capture(zr_step_graph* g, int b, const uint32_t* in, uint32_t* out, hipGraphExec_t* exec_out) {
    zr_context* ctx = g->ctx;
    for (auto& e : g->execs)
        if (e.in == in && e.out == out && e.blob == b) {
            *exec_out = e.exec;
            return ZR_OK;
        }
    // a capture starts on an idle stream (once per bucket and token pair)
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    const bool pending = ctx->token_check_pending;
    ZR_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    zr_status rc = launch_pack(ctx, &g->st[b]);
    if (!rc) rc = run_forward(ctx, &g->st[b], in, out, nullptr, nullptr);
    hipGraph_t graph = nullptr;
    const hipError_t e_end = hipStreamEndCapture(ctx->stream, &graph);
    ctx->token_check_pending = pending;  // nothing ran yet
    if (!rc && e_end != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "step graph capture: %s", hipGetErrorString(e_end));
    hipGraphExec_t exec = nullptr;
    if (!rc) {
        const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "step graph instantiate: %s", hipGetErrorString(e));
    }
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        (void)hipGetLastError();
        return rc;
    }
    g->execs.push_back({in, out, b, graph, exec});
    ++g->captures;
    *exec_out = exec;
    return ZR_OK;
}

}  // namespace

extern "C" {

zr_status zr_step_graph_create(zr_context* ctx, zr_step_graph** out) {
    if (!ctx || !out) return set_global_err(ZR_E_INVALID, "null argument");
    if (ctx->plain_kv) return set_err(ctx, ZR_E_UNSUPPORTED, "step graphs need the MFMA page layout");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    zr_step_graph* g = new zr_step_graph();
    g->ctx = ctx;
    hipError_t e = hipStreamCreateWithFlags(&g->copy, hipStreamNonBlocking);
    for (int b = 0; b < 2 && e == hipSuccess; ++b) {
        e = hipEventCreateWithFlags(&g->copied[b], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&g->replayed[b], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        zr_step_graph_destroy(g);
        return set_err(ctx, ZR_E_HIP, "step graph: %s", hipGetErrorString(e));
    }
    *out = g;
    return ZR_OK;
}

zr_status zr_step_graph_launch(zr_step_graph* g, const zr_microbatch* mb, const uint32_t* d_tokens,
                               uint32_t* d_out_tokens, uint32_t* h_out_tokens) {
    if (!g || !mb || !d_tokens || !d_out_tokens) return set_global_err(ZR_E_INVALID, "null argument");
    zr_context* ctx = g->ctx;
    zr_status rc = check_ready(ctx);
    if (rc) return rc;
    if (ctx->timing.enabled) return set_err(ctx, ZR_E_INVALID, "step graph launch with per-class timing on");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    if (!g->valid || g->epoch != ctx->buffer_epoch || g->S != mb->num_seqs)
        if ((rc = step_graph_setup(g, mb))) return rc;
    const int b = (int)(g->launches & 1);
    if (g->copy_pending[b]) {  // pinned buffer b is free once its last copy has finished
        ZR_HIP(ctx, hipEventSynchronize(g->copied[b]));
        g->copy_pending[b] = false;
    }
    bool fits = true;
    rc = stage_microbatch(ctx, mb, &g->st[b], &g->fixed[b], &fits);
    if (rc && !fits) {  // a new bucket, sized for this step
        if ((rc = step_graph_setup(g, mb))) return rc;
        rc = stage_microbatch(ctx, mb, &g->st[b], &g->fixed[b], &fits);
    }
    if (rc) return rc;
    if (g->replay_pending[b]) ZR_HIP(ctx, hipStreamWaitEvent(g->copy, g->replayed[b], 0));
    ZR_HIP(ctx, hipMemcpyAsync(g->dev[b], g->pinned[b], g->host_bytes, hipMemcpyHostToDevice, g->copy));
    ZR_HIP(ctx, hipEventRecord(g->copied[b], g->copy));
    g->copy_pending[b] = true;
    hipGraphExec_t exec = nullptr;
    if ((rc = step_graph_capture(g, b, d_tokens, d_out_tokens, &exec))) return rc;
    ZR_HIP(ctx, hipStreamWaitEvent(ctx->stream, g->copied[b], 0));
    ZR_HIP(ctx, hipGraphLaunch(exec, ctx->stream));
    ZR_HIP(ctx, hipEventRecord(g->replayed[b], ctx->stream));
    g->replay_pending[b] = true;
    ctx->token_check_pending = true;  // the replay copies the id-check word (device-fed ids)
    if (h_out_tokens)
        ZR_HIP(ctx, hipMemcpyAsync(h_out_tokens, d_out_tokens, 4 * (size_t)mb->num_seqs, hipMemcpyDeviceToHost,
                                   ctx->stream));
    ++g->launches;
    return ZR_OK;
}

zr_status zr_step_graph_info(const zr_step_graph* g, zr_step_graph_stats* out) {
    if (!g || !out) return set_global_err(ZR_E_INVALID, "null argument");
    out->launches = g->launches;
    out->captures = g->captures;
    out->buckets = g->buckets;
    out->sequences = g->S;
    out->items_capacity = g->valid ? g->fixed[0].items_cap : 0;
    out->merge_capacity = g->valid ? g->fixed[0].merge_cap : 0;
    out->fused_rope = g->valid && g->fixed[0].fuse_rope;
    out->metadata_bytes = g->host_bytes;
    return ZR_OK;
}

void zr_step_graph_destroy(zr_step_graph* g) {
    if (!g) return;
    if (g->copy) (void)hipStreamSynchronize(g->copy);
    if (g->ctx && g->ctx->stream) (void)hipStreamSynchronize(g->ctx->stream);
    step_graph_drop_execs(g);
    for (int b = 0; b < 2; ++b) {
        if (g->pinned[b]) (void)hipHostFree(g->pinned[b]);
        if (g->dev[b]) (void)hipFree(g->dev[b]);
        if (g->copied[b]) (void)hipEventDestroy(g->copied[b]);
        if (g->replayed[b]) (void)hipEventDestroy(g->replayed[b]);
        g->st[b].dev = nullptr;  // the blob belongs to the step graph
    }
    if (g->copy) (void)hipStreamDestroy(g->copy);
    delete g;
}

// A decode step of one row per sequence whose caller wants only the greedy
// ids, replayed from the context's step graph (the kernels and metadata of
// the eager forward pass, captured once per bucket): the ids go up, the graph
// replays, the ids come back.  Taken once the same sequence count has run
// kForwardReplayAfter times in a row, so that a steady decode loop replays
// and batches that change every step (sessions joining and leaving) do not
// capture a graph per step.  ZR_FORWARD_REPLAY=0 keeps every step eager.
constexpr int kForwardReplayAfter = 3;

static bool forward_replay_fits(const zr_context* ctx, const zr_microbatch* mb) {
    if (ctx->plain_kv || ctx->timing.enabled || mb->num_seqs < 1 || mb->num_seqs > ctx->desc.max_seqs) return false;
    for (int s = 0; s < mb->num_seqs; ++s)
        if (mb->q_len[s] != 1) return false;
    static const bool off = [] {
        const char* e = getenv("ZR_FORWARD_REPLAY");
        return e && atoi(e) == 0;
    }();
    return !off;
}

static zr_status forward_replayed(zr_context* ctx, const zr_microbatch* mb, uint32_t* out_tokens) {
    const int S = mb->num_seqs, cap = ctx->desc.max_seqs;
    zr_status rc = ZR_OK;
    if (!ctx->fwd_graph && (rc = zr_step_graph_create(ctx, &ctx->fwd_graph))) return rc;
    if (!ctx->fwd_ids) ZR_HIP(ctx, hipMalloc((void**)&ctx->fwd_ids, 8 * (size_t)cap));
    if (!ctx->fwd_h_ids) ZR_HIP(ctx, hipHostMalloc((void**)&ctx->fwd_h_ids, 8 * (size_t)cap, hipHostMallocDefault));
    // (the previous call synchronised, so the pinned ids are free)
    memcpy(ctx->fwd_h_ids, mb->tokens, 4 * (size_t)S);
    ZR_HIP(ctx, hipMemcpyAsync(ctx->fwd_ids, ctx->fwd_h_ids, 4 * (size_t)S, hipMemcpyHostToDevice, ctx->stream));
    rc = zr_step_graph_launch(ctx->fwd_graph, mb, ctx->fwd_ids, ctx->fwd_ids + cap, ctx->fwd_h_ids + cap);
    if (rc) {
        (void)hipStreamSynchronize(ctx->stream);
        return rc;
    }
    if ((rc = zr_synchronize(ctx))) return rc;
    memcpy(out_tokens, ctx->fwd_h_ids + cap, 4 * (size_t)S);
    return ZR_OK;
}

zr_status zr_forward_replay_info(const zr_context* ctx, zr_step_graph_stats* out) {
    if (!ctx || !out) return set_global_err(ZR_E_INVALID, "null argument");
    if (!ctx->fwd_graph) {
        *out = zr_step_graph_stats{};
        return ZR_OK;
    }
    return zr_step_graph_info(ctx->fwd_graph, out);
}

zr_status zr_forward(zr_context* ctx, const zr_microbatch* mb, uint32_t* out_tokens, float* out_logits,
                     float* out_partials) {
    if (!ctx || !mb) return set_global_err(ZR_E_INVALID, "null argument");
    if (!mb->tokens) return set_err(ctx, ZR_E_INVALID, "zr_forward needs host token ids");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    if (mb->num_seqs == ctx->fwd_seqs) {
        ++ctx->fwd_repeats;
    } else {
        ctx->fwd_seqs = mb->num_seqs;
        ctx->fwd_repeats = 1;
    }
    if (out_tokens && !out_logits && !out_partials && ctx->fwd_repeats >= kForwardReplayAfter &&
        forward_replay_fits(ctx, mb))
        return forward_replayed(ctx, mb, out_tokens);
    StagedMeta* st = ctx->scratch_stage;
    zr_status rc = stage_microbatch(ctx, mb, st);
    if (!rc) rc = run_forward(ctx, st, nullptr, ctx->tokens_out, nullptr, out_partials);
    if (!rc && out_tokens)
        ZR_HIP(ctx, hipMemcpyAsync(out_tokens, ctx->tokens_out, 4 * (size_t)mb->num_seqs, hipMemcpyDeviceToHost,
                                   ctx->stream));
    if (!rc && out_logits)
        ZR_HIP(ctx, hipMemcpyAsync(out_logits, ctx->logits, 4 * (size_t)mb->num_seqs * ctx->desc.vocab,
                                   hipMemcpyDeviceToHost, ctx->stream));
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "forward: %s", hipGetErrorString(e));
    return rc;
}

// ------------------------------------------------------- op-level entries
zr_status zr_pack(zr_context* ctx, const zr_microbatch* mb, int* cu_q, int* cu_k, int* positions, int* slot_mapping,
                  int* seq_ids) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    StagedMeta* st = ctx->scratch_stage;
    zr_status rc = stage_microbatch(ctx, mb, st);
    if (rc) return rc;
    const int S = st->num_seqs, T = st->total_q;
    if (cu_q) ZR_HIP(ctx, hipMemcpyAsync(cu_q, st->cu_q, 4 * (S + 1), hipMemcpyDeviceToHost, ctx->stream));
    if (cu_k) ZR_HIP(ctx, hipMemcpyAsync(cu_k, st->cu_k, 4 * (S + 1), hipMemcpyDeviceToHost, ctx->stream));
    if (positions) ZR_HIP(ctx, hipMemcpyAsync(positions, st->positions, 4 * (size_t)T, hipMemcpyDeviceToHost, ctx->stream));
    if (slot_mapping)
        ZR_HIP(ctx, hipMemcpyAsync(slot_mapping, st->slot_mapping, 4 * (size_t)T, hipMemcpyDeviceToHost, ctx->stream));
    if (seq_ids) ZR_HIP(ctx, hipMemcpyAsync(seq_ids, st->seq_ids, 4 * (size_t)T, hipMemcpyDeviceToHost, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

// A staged microbatch's arrays index this context's pool and workspaces: one
// staged by another context is refused before anything launches.
static zr_status staged_for(zr_context* ctx, const StagedMeta* st) {
    if (st->ctx != ctx) return set_err(ctx, ZR_E_INVALID, "staged microbatch of another context");
    return ZR_OK;
}

zr_status zr_rope_kv_write(zr_context* ctx, zr_staged* s, int layer, const float* d_qkv, float* d_q_out, int rope) {
    StagedMeta* st = (StagedMeta*)s;
    if (!ctx || !st || !d_qkv || !d_q_out) return set_global_err(ZR_E_INVALID, "null argument");
    if (zr_status rc = staged_for(ctx, st)) return rc;
    if (layer < 0 || layer >= ctx->desc.num_layers) return set_err(ctx, ZR_E_INVALID, "Invalid layer index: %d", layer);
    zr_status rc = launch_rope_kv_write(ctx, st, layer, d_qkv, d_q_out, rope);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_rope_attention(zr_context* ctx, zr_staged* s, int layer, const float* d_qkv, float* d_out, int rope) {
    StagedMeta* st = (StagedMeta*)s;
    if (!ctx || !st || !d_qkv || !d_out) return set_global_err(ZR_E_INVALID, "null argument");
    if (zr_status rc = staged_for(ctx, st)) return rc;
    if (layer < 0 || layer >= ctx->desc.num_layers) return set_err(ctx, ZR_E_INVALID, "Invalid layer index: %d", layer);
    zr_status rc = launch_attention_rope(ctx, st, layer, Slabs(d_qkv), rope, d_out, nullptr);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_attention(zr_context* ctx, zr_staged* s, int layer, const float* d_q, float* d_out) {
    StagedMeta* st = (StagedMeta*)s;
    if (!ctx || !st || !d_q || !d_out) return set_global_err(ZR_E_INVALID, "null argument");
    if (zr_status rc = staged_for(ctx, st)) return rc;
    if (layer < 0 || layer >= ctx->desc.num_layers) return set_err(ctx, ZR_E_INVALID, "Invalid layer index: %d", layer);
    zr_status rc = launch_attention(ctx, st, layer, d_q, d_out, nullptr);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_kv_read_probe(zr_context* ctx, zr_staged* s, int layer, int repeats, double* mean_ms) {
    StagedMeta* st = (StagedMeta*)s;
    if (!ctx || !st || !mean_ms) return set_global_err(ZR_E_INVALID, "null argument");
    if (zr_status rc = staged_for(ctx, st)) return rc;
    if (layer < 0 || layer >= ctx->desc.num_layers) return set_err(ctx, ZR_E_INVALID, "Invalid layer index: %d", layer);
    if (repeats <= 0 || repeats > 10000) return set_err(ctx, ZR_E_INVALID, "repeats %d outside 1..10000", repeats);
    if (!ctx->kv_pool) return set_err(ctx, ZR_E_INVALID, "KV pool not created");
    return launch_kv_read_probe(ctx, st, layer, repeats, mean_ms);
}

// the page window of a gather / scatter lies inside the table and the pool
static zr_status kv_copy_check(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                               int n_rows) {
    if (!ctx->kv_pool) return set_err(ctx, ZR_E_INVALID, "KV pool not created");
    if (first_offset < 0 || first_offset >= kPageRows || first_row < 0)
        return set_err(ctx, ZR_E_INVALID, "first_offset %d first_row %d", first_offset, first_row);
    const long last = (long)first_offset + first_row + n_rows - 1;
    if (last / kPageRows >= n_pages)
        return set_err(ctx, ZR_E_INVALID, "rows up to %ld exceed %d pages", last, n_pages);
    for (long p = (first_offset + first_row) / kPageRows; p <= last / kPageRows; ++p)
        if (block_table[p] < 0 || block_table[p] >= ctx->n_pages)
            return set_err(ctx, ZR_E_INVARIANT, "page slot %ld holds page %d outside pool of %d", p, block_table[p],
                           ctx->n_pages);
    return ZR_OK;
}

static zr_status kv_copy_entry(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                               int n_rows, float* k, float* v, int to_pool, float** d_rows = nullptr) {
    if (!ctx || !block_table || (!d_rows && (!k || !v))) return set_global_err(ZR_E_INVALID, "null argument");
    if (!ctx->kv_pool) return set_err(ctx, ZR_E_INVALID, "KV pool not created");
    if (n_rows <= 0) return ZR_OK;
    if (zr_status rc = kv_copy_check(ctx, block_table, n_pages, first_offset, first_row, n_rows)) return rc;
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    const int L = ctx->desc.num_layers;
    const size_t elems = (size_t)L * n_rows * ctx->kv_cols;
    // persistent staging (grown on demand): the table and the K / V rows
    const size_t need = 2 * elems + (size_t)n_pages;
    if (need > ctx->kv_stage_floats) {
        ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->kv_stage) (void)hipFree(ctx->kv_stage);
        ctx->kv_stage = nullptr;
        ctx->kv_stage_floats = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->kv_stage, need * sizeof(float)));
        ctx->kv_stage_floats = need;
    }
    float* d_k = ctx->kv_stage;
    float* d_v = d_k + elems;
    int* d_table = (int*)(d_v + elems);
    hipError_t e = hipMemcpyAsync(d_table, block_table, 4 * (size_t)n_pages, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess && to_pool) e = hipMemcpyAsync(d_k, k, 4 * elems, hipMemcpyDefault, ctx->stream);
    if (e == hipSuccess && to_pool) e = hipMemcpyAsync(d_v, v, 4 * elems, hipMemcpyDefault, ctx->stream);
    zr_status rc = e == hipSuccess ? ZR_OK : set_err(ctx, ZR_E_HIP, "kv copy staging: %s", hipGetErrorString(e));
    if (!rc) rc = launch_kv_copy(ctx, 0, L, d_table, first_offset, first_row, n_rows, d_k, d_v, to_pool);
    if (d_rows) {  // gather into the device staging only ([L][rows][Kc] K, then V)
        *d_rows = d_k;
        return rc;
    }
    if (!rc && !to_pool) {
        e = hipMemcpyAsync(k, d_k, 4 * elems, hipMemcpyDefault, ctx->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(v, d_v, 4 * elems, hipMemcpyDefault, ctx->stream);
        if (e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "kv gather copy-out: %s", hipGetErrorString(e));
    }
    e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "kv copy: %s", hipGetErrorString(e));
    return rc;
}

}  // extern "C"

// One session window's KV in a device buffer of its own, on its way to or
// from host memory on a copy stream: K [layers][rows][kv_cols], then V, then
// room for a page table.  `used` is recorded after the last compute-stream
// kernel on the buffer; `copied` after the host copy.
struct zr_transfer {
    zr_context* ctx = nullptr;
    float* buf = nullptr;
    size_t floats = 0;
    int rows = 0;
    bool to_host = false;
    hipEvent_t copied = nullptr;
    hipEvent_t used = nullptr;
};

namespace zr {

// a transfer with a buffer of >= floats: the smallest finished one that fits, else a new allocation
// Finished transfers' buffers kept for reuse: at most this many (the
// smallest beyond it are freed when a transfer is destroyed).
constexpr size_t kXferKeep = 8;

// Frees the kept buffers smaller than `floats` (all of them with floats = max).
static void xfer_release_below(zr_context* ctx, size_t floats) {
    auto& fl = ctx->xfer_free;
    for (size_t i = 0; i < fl.size();) {
        if (fl[i].second < floats) {
            (void)hipFree(fl[i].first);
            fl.erase(fl.begin() + i);
        } else {
            ++i;
        }
    }
}

static zr_status xfer_new(zr_context* ctx, size_t floats, zr_transfer** out) {
    zr_transfer* t = new zr_transfer();
    t->ctx = ctx;
    int best = -1;
    for (int i = 0; i < (int)ctx->xfer_free.size(); ++i)
        if (ctx->xfer_free[i].second >= floats && (best < 0 || ctx->xfer_free[i].second < ctx->xfer_free[best].second))
            best = i;
    hipError_t e = hipSuccess;
    if (best >= 0) {
        t->buf = ctx->xfer_free[best].first;
        t->floats = ctx->xfer_free[best].second;
        ctx->xfer_free.erase(ctx->xfer_free.begin() + best);
    } else {
        // none fits: the kept buffers too small for this window go first, and
        // when device memory is short every kept buffer before one retry
        xfer_release_below(ctx, floats);
        e = hipMalloc(&t->buf, floats * sizeof(float));
        if (e == hipErrorOutOfMemory) {
            (void)hipGetLastError();
            xfer_release_below(ctx, ~(size_t)0);
            e = hipMalloc(&t->buf, floats * sizeof(float));
        }
        if (e != hipSuccess) t->buf = nullptr;
        t->floats = floats;
    }
    if (e == hipSuccess) e = hipEventCreateWithFlags(&t->copied, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&t->used, hipEventDisableTiming);
    if (e != hipSuccess) {
        if (t->buf && best < 0) (void)hipFree(t->buf);
        else if (t->buf) ctx->xfer_free.emplace_back(t->buf, t->floats);
        if (t->copied) (void)hipEventDestroy(t->copied);
        if (t->used) (void)hipEventDestroy(t->used);
        delete t;
        return set_err(ctx, e == hipErrorOutOfMemory ? ZR_E_OOM : ZR_E_HIP, "KV transfer buffer: %s",
                       hipGetErrorString(e));
    }
    *out = t;
    return ZR_OK;
}

}  // namespace zr

extern "C" {

zr_status zr_kv_gather_async(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                             int n_rows, float* dst_k, float* dst_v, zr_transfer** out) {
    if (!ctx || !block_table || !dst_k || !dst_v || !out) return set_global_err(ZR_E_INVALID, "null argument");
    *out = nullptr;
    if (n_rows <= 0) return set_err(ctx, ZR_E_INVALID, "a KV transfer needs rows (%d)", n_rows);
    if (zr_status rc = kv_copy_check(ctx, block_table, n_pages, first_offset, first_row, n_rows)) return rc;
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    const int L = ctx->desc.num_layers;
    const size_t elems = (size_t)L * n_rows * ctx->kv_cols;
    zr_transfer* t = nullptr;
    if (zr_status rc = xfer_new(ctx, 2 * elems + (size_t)n_pages, &t)) return rc;
    t->rows = n_rows;
    t->to_host = true;
    float* d_k = t->buf;
    float* d_v = d_k + elems;
    int* d_table = (int*)(d_v + elems);
    // the gather on the compute stream (the session's pages may be handed out
    // right after this call: later kernels run after it), the copy-out on the
    // device-to-host stream once the gather is done
    hipError_t e = hipMemcpyAsync(d_table, block_table, 4 * (size_t)n_pages, hipMemcpyHostToDevice, ctx->stream);
    zr_status rc = e == hipSuccess ? ZR_OK : set_err(ctx, ZR_E_HIP, "kv transfer table: %s", hipGetErrorString(e));
    if (!rc) rc = launch_kv_copy(ctx, 0, L, d_table, first_offset, first_row, n_rows, d_k, d_v, 0);
    if (!rc) {
        e = hipEventRecord(t->used, ctx->stream);
        if (e == hipSuccess) e = hipStreamWaitEvent(ctx->d2h_stream, t->used, 0);
        if (e == hipSuccess) e = hipMemcpyAsync(dst_k, d_k, 4 * elems, hipMemcpyDeviceToHost, ctx->d2h_stream);
        if (e == hipSuccess) e = hipMemcpyAsync(dst_v, d_v, 4 * elems, hipMemcpyDeviceToHost, ctx->d2h_stream);
        if (e == hipSuccess) e = hipEventRecord(t->copied, ctx->d2h_stream);
        if (e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "kv transfer copy-out: %s", hipGetErrorString(e));
    }
    if (rc) {
        zr_transfer_destroy(t);
        return rc;
    }
    *out = t;
    return ZR_OK;
}

zr_status zr_kv_upload_async(zr_context* ctx, const float* src_k, const float* src_v, int n_rows, zr_transfer** out) {
    if (!ctx || !src_k || !src_v || !out) return set_global_err(ZR_E_INVALID, "null argument");
    *out = nullptr;
    if (n_rows <= 0) return set_err(ctx, ZR_E_INVALID, "a KV transfer needs rows (%d)", n_rows);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    const size_t elems = (size_t)ctx->desc.num_layers * n_rows * ctx->kv_cols;
    zr_transfer* t = nullptr;
    // room for the page table of any placement of the rows (a partial first page)
    if (zr_status rc = xfer_new(ctx, 2 * elems + (size_t)n_rows / kPageRows + 2, &t)) return rc;
    t->rows = n_rows;
    hipError_t e = hipMemcpyAsync(t->buf, src_k, 4 * elems, hipMemcpyHostToDevice, ctx->h2d_stream);
    if (e == hipSuccess) e = hipMemcpyAsync(t->buf + elems, src_v, 4 * elems, hipMemcpyHostToDevice, ctx->h2d_stream);
    if (e == hipSuccess) e = hipEventRecord(t->copied, ctx->h2d_stream);
    if (e == hipSuccess) e = hipEventRecord(t->used, ctx->h2d_stream);
    if (e != hipSuccess) {
        zr_status rc = set_err(ctx, ZR_E_HIP, "kv transfer upload: %s", hipGetErrorString(e));
        zr_transfer_destroy(t);
        return rc;
    }
    *out = t;
    return ZR_OK;
}

zr_status zr_kv_scatter_transfer(zr_context* ctx, zr_transfer* t, const int* block_table, int n_pages,
                                 int first_offset, int first_row, int n_rows) {
    if (!ctx || !t || !block_table) return set_global_err(ZR_E_INVALID, "null argument");
    if (t->ctx != ctx) return set_err(ctx, ZR_E_INVALID, "KV transfer of another context");
    if (n_rows != t->rows) return set_err(ctx, ZR_E_INVALID, "KV transfer holds %d rows, not %d", t->rows, n_rows);
    if (zr_status rc = kv_copy_check(ctx, block_table, n_pages, first_offset, first_row, n_rows)) return rc;
    const int L = ctx->desc.num_layers;
    const size_t elems = (size_t)L * n_rows * ctx->kv_cols;
    // only the pages the rows touch travel with the transfer (at most
    // n_rows / 16 + 2: the room every transfer keeps), addressed from the
    // first of them
    const int p0 = (first_offset + first_row) / kPageRows;
    const int p1 = (first_offset + first_row + n_rows - 1) / kPageRows;
    const int used_pages = p1 - p0 + 1;
    if (2 * elems + (size_t)used_pages > t->floats)
        return set_err(ctx, ZR_E_INVALID, "page table of %d pages does not fit the KV transfer", used_pages);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    float* d_k = t->buf;
    float* d_v = d_k + elems;
    int* d_table = (int*)(d_v + elems);
    // an upload is waited for; a gather's rows are on the device already (an
    // earlier launch on this stream), its copy-out only reads them
    hipError_t e = hipMemcpyAsync(d_table, block_table + p0, 4 * (size_t)used_pages, hipMemcpyHostToDevice,
                                  ctx->stream);
    if (e == hipSuccess && !t->to_host) e = hipStreamWaitEvent(ctx->stream, t->copied, 0);
    if (e != hipSuccess) return set_err(ctx, ZR_E_HIP, "kv transfer scatter: %s", hipGetErrorString(e));
    const int sliced_offset = (first_offset + first_row) - p0 * kPageRows;
    if (zr_status rc = launch_kv_copy(ctx, 0, L, d_table, sliced_offset, 0, n_rows, d_k, d_v, 1)) return rc;
    ZR_HIP(ctx, hipEventRecord(t->used, ctx->stream));
    return ZR_OK;
}

int zr_transfer_done(const zr_transfer* t) {
    if (!t) return set_global_err(ZR_E_INVALID, "null argument");
    const hipError_t e = hipEventQuery(t->copied);
    if (e == hipSuccess) return 1;
    if (e == hipErrorNotReady) return 0;
    return set_err(t->ctx, ZR_E_HIP, "KV transfer: %s", hipGetErrorString(e));
}

zr_status zr_transfer_wait(zr_transfer* t) {
    if (!t) return set_global_err(ZR_E_INVALID, "null argument");
    ZR_HIP(t->ctx, hipEventSynchronize(t->copied));
    return ZR_OK;
}

void zr_transfer_destroy(zr_transfer* t) {
    if (!t) return;
    // the buffer is reused once its host copy and its last kernel are done
    (void)hipEventSynchronize(t->copied);
    (void)hipEventSynchronize(t->used);
    if (t->buf) {
        auto& fl = t->ctx->xfer_free;
        fl.emplace_back(t->buf, t->floats);
        while (fl.size() > kXferKeep) {  // keep the largest
            size_t smallest = 0;
            for (size_t i = 1; i < fl.size(); ++i)
                if (fl[i].second < fl[smallest].second) smallest = i;
            (void)hipFree(fl[smallest].first);
            fl.erase(fl.begin() + smallest);
        }
    }
    (void)hipEventDestroy(t->copied);
    (void)hipEventDestroy(t->used);
    delete t;
}

size_t zr_transfer_cached_bytes(const zr_context* ctx) {
    if (!ctx) return 0;
    size_t floats = 0;
    for (const auto& fb : ctx->xfer_free) floats += fb.second;
    return floats * sizeof(float);
}

zr_status zr_kv_gather(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                       int n_rows, float* dst_k, float* dst_v) {
    return kv_copy_entry(ctx, block_table, n_pages, first_offset, first_row, n_rows, dst_k, dst_v, 0);
}

zr_status zr_kv_scatter(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                        int n_rows, const float* src_k, const float* src_v) {
    return kv_copy_entry(ctx, block_table, n_pages, first_offset, first_row, n_rows, (float*)src_k, (float*)src_v, 1);
}

zr_status zr_kv_export_cbor(zr_context* ctx, const int* block_table, int n_pages, int first_offset, int first_row,
                            int n_rows, long long base_position, int cfg_max_seq_len, uint8_t* out, size_t capacity,
                            size_t* out_len) {
    if (!ctx || !block_table || !out_len) return set_global_err(ZR_E_INVALID, "null argument");
    if (n_rows <= 0) return set_err(ctx, ZR_E_INVALID, "empty KV export has no CBOR document");
    if (base_position < 0 || cfg_max_seq_len < 0) return set_err(ctx, ZR_E_INVALID, "negative position or length");
    float* d_k = nullptr;
    zr_status rc = kv_copy_entry(ctx, block_table, n_pages, first_offset, first_row, n_rows, nullptr, nullptr, 0, &d_k);
    if (rc) return rc;
    const int L = ctx->desc.num_layers;
    const float* d_v = d_k + (size_t)L * n_rows * ctx->kv_cols;
    // KVCacheConfig of the device cache (forward_pass.rs:1791-1796): the model's kv heads and head_dim
    const int cfg[4] = {L, ctx->desc.num_kv_heads, ctx->head_dim, cfg_max_seq_len};
    return launch_kv_cbor(ctx, d_k, d_v, L, n_rows, ctx->kv_cols, base_position, cfg, out, capacity, out_len);
}

zr_status zr_kv_read_pages(zr_context* ctx, int layer, const int* pages, int n_pages, void* dst) {
    if (!ctx || !pages || !dst) return set_global_err(ZR_E_INVALID, "null argument");
    if (layer < 0 || layer >= ctx->desc.num_layers) return set_err(ctx, ZR_E_INVALID, "Invalid layer index: %d", layer);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    for (int i = 0; i < n_pages; ++i) {
        if (pages[i] < 0 || pages[i] >= ctx->n_pages) return set_err(ctx, ZR_E_INVALID, "page %d outside pool", pages[i]);
        const char* src = (const char*)ctx->kv_pool + ((size_t)layer * ctx->n_pages + pages[i]) * ctx->page_bytes;
        ZR_HIP(ctx, hipMemcpyAsync((char*)dst + (size_t)i * ctx->page_bytes, src, ctx->page_bytes,
                                   hipMemcpyDeviceToHost, ctx->stream));
    }
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

zr_status zr_argmax(zr_context* ctx, const float* d_x, int rows, int cols, uint32_t* d_out) {
    if (!ctx || !d_x || !d_out) return set_global_err(ZR_E_INVALID, "null argument");
    if (rows <= 0 || cols <= 0) return set_err(ctx, ZR_E_INVALID, "Device sampling received an empty logits tensor");
    const size_t need = (size_t)rows * ((cols + 4095) / 4096) * 2;
    if (need > ctx->argmax_ws_floats) {
        hipStreamSynchronize(ctx->stream);
        hipFree(ctx->argmax_ws);
        ++ctx->buffer_epoch;
        ctx->argmax_ws = nullptr;
        ctx->argmax_ws_floats = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->argmax_ws, need * 4));
        ctx->argmax_ws_floats = need;
    }
    zr_status rc = launch_argmax(ctx, d_x, rows, cols, d_out);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_argmax_noalloc(zr_context* ctx, const float* d_x, int rows, int cols, uint32_t* d_out) {
    if (!ctx || !d_x || !d_out) return set_global_err(ZR_E_INVALID, "null argument");
    if (rows <= 0 || cols <= 0) return set_err(ctx, ZR_E_INVALID, "Device sampling received an empty logits tensor");
    return launch_argmax_noalloc(ctx, d_x, rows, cols, d_out);
}

zr_status zr_sample(zr_context* ctx, const float* d_logits, int rows, int cols, const float* temperature,
                    const float* top_p, const uint64_t* seeds, uint32_t* d_out) {
    if (!ctx || !d_logits || !temperature || !top_p || !seeds || !d_out)
        return set_global_err(ZR_E_INVALID, "null argument");
    if (rows <= 0 || cols <= 0) return set_err(ctx, ZR_E_INVALID, "Device sampling received an empty logits tensor");
    zr_status rc = launch_sample(ctx, d_logits, rows, cols, temperature, top_p, seeds, d_out);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_sample_last_logits(zr_context* ctx, int rows, const float* temperature, const float* top_p,
                                const uint64_t* seeds, uint32_t* out_tokens) {
    if (!ctx || !out_tokens) return set_global_err(ZR_E_INVALID, "null argument");
    if (!ctx->logits || !ctx->tokens_out) return set_err(ctx, ZR_E_INVALID, "no logits to sample");
    if (rows <= 0 || rows > ctx->desc.max_seqs)
        return set_err(ctx, ZR_E_INVALID, "Device sampling received %d rows", rows);
    zr_status rc = launch_sample(ctx, ctx->logits, rows, ctx->desc.vocab, temperature, top_p, seeds, ctx->tokens_out);
    if (rc) return rc;
    ZR_HIP(ctx, hipMemcpyAsync(out_tokens, ctx->tokens_out, 4 * (size_t)rows, hipMemcpyDeviceToHost, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

zr_status zr_rms_norm(zr_context* ctx, const float* d_x, const float* d_gamma, float* d_y, int rows, int cols) {
    if (!ctx || !d_x || !d_gamma || !d_y) return set_global_err(ZR_E_INVALID, "null argument");
    zr_status rc = launch_rms_norm(ctx, d_x, nullptr, nullptr, d_gamma, d_y, nullptr, 0, nullptr, rows, cols);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

// Op-level product of a packed weight with a device f32 A [m, k]: A is padded
// to the packed K (a multiple of 32; the packed weights are zero beyond k) and
// converted to the bf16 (hi + lo) operand.  kEpiStore writes C [m, n] to d_out;
// kEpiSwiGLU writes its bf16 operand and expands it to f32 [m, n / 2] in d_out.
// Takes ownership of `packed`.
static zr_status run_gemm_op(zr_context* ctx, const float* d_a, uint16_t* packed, float* d_out, int m, int n, int k,
                             int epilogue) {
    const int lo = (ctx->desc.flags & ZR_FLAG_SPLIT_ACTIVATIONS) ? 1 : 0;
    const int kp = (k + 31) / 32 * 32;
    const size_t need = gemm_ws_floats(m, n, kp, epilogue);
    float* saved_ws = ctx->splitk_ws;
    size_t saved_n = ctx->splitk_ws_floats;
    float* tmp_ws = nullptr;
    float* a_pad = nullptr;
    uint16_t* a16 = nullptr;
    uint16_t* h16 = nullptr;
    zr_status rc = ZR_OK;
    hipError_t e = hipMalloc(&a16, (size_t)2 * 2 * a_plane(m, kp));
    if (e == hipSuccess) e = hipMalloc(&a_pad, (size_t)4 * m * kp);
    if (e == hipSuccess && epilogue == kEpiSwiGLU) e = hipMalloc(&h16, (size_t)2 * 2 * a_plane(m, n / 2));
    if (e == hipSuccess) e = hipMemsetAsync(a_pad, 0, (size_t)4 * m * kp, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(a_pad, 4 * (size_t)kp, d_a, 4 * (size_t)k, 4 * (size_t)k, m, hipMemcpyDeviceToDevice,
                             ctx->stream);
    if (e == hipSuccess && need > saved_n) {
        e = hipMalloc(&tmp_ws, need * 4);
        if (e == hipSuccess) {
            ctx->splitk_ws = tmp_ws;
            ctx->splitk_ws_floats = need;
        }
    }
    if (e != hipSuccess) rc = set_err(ctx, ZR_E_OOM, "gemm workspace: %s", hipGetErrorString(e));
    if (!rc) rc = launch_to_bf16_pair(ctx, a_pad, m, kp, a16, lo);
    if (!rc && epilogue == kEpiSwiGLU) {
        rc = launch_gemm(ctx, a16, packed, nullptr, h16, m, n, kp, kEpiSwiGLU);
        if (!rc) rc = launch_from_bf16_pair(ctx, h16, m, n / 2, lo, d_out);
    } else if (!rc) {
        rc = launch_gemm(ctx, a16, packed, d_out, nullptr, m, n, kp, kEpiStore);
    }
    e = hipStreamSynchronize(ctx->stream);
    if (!rc && e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "gemm: %s", hipGetErrorString(e));
    ctx->splitk_ws = saved_ws;
    ctx->splitk_ws_floats = saved_n;
    if (tmp_ws) (void)hipFree(tmp_ws);
    if (h16) (void)hipFree(h16);
    if (a_pad) (void)hipFree(a_pad);
    if (a16) (void)hipFree(a16);
    (void)hipFree(packed);
    return rc;
}

zr_status zr_gemm(zr_context* ctx, const float* d_a, const uint16_t* w, float* d_c, int m, int n, int k) {
    if (!ctx || !d_a || !w || !d_c) return set_global_err(ZR_E_INVALID, "null argument");
    if (m <= 0 || n <= 0 || k <= 0) return set_err(ctx, ZR_E_INVALID, "Matmul shape mismatch: %dx%d @ %dx%d", m, k, k, n);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    uint16_t* packed = nullptr;
    zr_status rc = pack_weight(ctx, w, k, n, &packed);
    if (rc) return rc;
    return run_gemm_op(ctx, d_a, packed, d_c, m, n, k, kEpiStore);
}

zr_status zr_gemm_swiglu(zr_context* ctx, const float* d_a, const uint16_t* w_gate, const uint16_t* w_up, float* d_h,
                         int m, int f, int k) {
    if (!ctx || !d_a || !w_gate || !w_up || !d_h) return set_global_err(ZR_E_INVALID, "null argument");
    if (m <= 0 || f <= 0 || k <= 0)
        return set_err(ctx, ZR_E_INVALID, "Matmul shape mismatch: %dx%d @ %dx%d", m, k, k, 2 * f);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    uint16_t* packed = nullptr;
    zr_status rc = pack_weight_gate_up(ctx, w_gate, w_up, k, f, &packed);
    if (rc) return rc;
    return run_gemm_op(ctx, d_a, packed, d_h, m, 2 * f, k, kEpiSwiGLU);
}

zr_status zr_device_alloc(zr_context* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return set_global_err(ZR_E_INVALID, "null argument");
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    if (e != hipSuccess) return set_err(ctx, e == hipErrorOutOfMemory ? ZR_E_OOM : ZR_E_HIP, "hipMalloc(%zu): %s",
                                        bytes, hipGetErrorString(e));
    return ZR_OK;
}

zr_status zr_host_alloc(zr_context* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return set_global_err(ZR_E_INVALID, "null argument");
    *out = nullptr;
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, bytes > 0 ? bytes : 1, hipHostMallocDefault);
    if (e != hipSuccess) return set_err(ctx, ZR_E_OOM, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
    *out = p;
    return ZR_OK;
}

zr_status zr_host_free(zr_context* ctx, void* p) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    if (p) ZR_HIP(ctx, hipHostFree(p));
    return ZR_OK;
}

zr_status zr_device_free(zr_context* ctx, void* p) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    if (p) {
        hipStreamSynchronize(ctx->stream);
        ZR_HIP(ctx, hipFree(p));
    }
    return ZR_OK;
}

zr_status zr_memcpy_h2d(zr_context* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    ZR_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

zr_status zr_memcpy_d2h(zr_context* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    ZR_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

zr_status zr_fill_normal_bf16(zr_context* ctx, uint16_t* d_dst, size_t n, uint64_t seed, float std) {
    if (!ctx || !d_dst) return set_global_err(ZR_E_INVALID, "null argument");
    zr_status rc = launch_fill_normal_bf16(ctx, d_dst, n, seed, std);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_kv_pool_fill_normal(zr_context* ctx, uint64_t seed, float std) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    if (!ctx->kv_pool) return set_err(ctx, ZR_E_INVALID, "KV pool not created");
    zr_status rc = launch_fill_pool_normal(ctx, seed, std);
    if (!rc) ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return rc;
}

zr_status zr_timing_begin(zr_context* ctx, unsigned class_mask) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ctx->timing.enabled = true;
    ctx->timing.class_mask = class_mask;
    ctx->timing.spans.clear();
    ctx->timing.next_event = 0;
    return ZR_OK;
}

zr_status zr_timing_end(zr_context* ctx, double* ms_by_class, int* launches_by_class) {
    if (!ctx) return set_global_err(ZR_E_INVALID, "null context");
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    double ms[kTimingClasses] = {};
    int n[kTimingClasses] = {};
    for (auto& sp : ctx->timing.spans) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, sp.second.first, sp.second.second) == hipSuccess) {
            ms[sp.first] += t;
            n[sp.first] += 1;
        }
    }
    ctx->timing.enabled = false;
    ctx->timing.spans.clear();
    ctx->timing.next_event = 0;
    if (ms_by_class) memcpy(ms_by_class, ms, sizeof ms);
    if (launches_by_class) memcpy(launches_by_class, n, sizeof n);
    return ZR_OK;
}

}  // extern "C"
