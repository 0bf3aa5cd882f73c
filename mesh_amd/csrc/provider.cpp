// Host-side rocm execution backend (include/zip_rocm_host.h): the session page
// tables, positions and microbatch assembly that the reference keeps in its
// Rust provider host (forward_pass.rs:303-1243, 2089-2319; backend.rs:110-151).
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "../../include/zip_rocm_host.h"
#include "zr_internal.h"

using zr::kPageRows;
using zr::set_err;
using zr::set_global_err;

struct zrh_pool {
    zr_context* ctx = nullptr;
    std::vector<int> free_list;  // LIFO: pop_back
    // Global pages popped while a host call is open, in pop order, so that a
    // failed call can give them back (PoolTxn).
    std::vector<int> popped;
    int txn_depth = 0;
};

namespace {

struct PageEntry {
    int global = -1;
    int used_rows = 0;
    bool active = false;
};

struct Span {
    int page_index, start_row, row_count;
};

// One session's DeviceKVCache with a single canonical block table: the
// reference keeps one allocator per layer, but every layer evolves
// identically (checked by DeviceKVCache::live_block_table, 1024-1048), so the
// device pool stores all layers of a page at one page id.
struct SessionKV {
    std::vector<PageEntry> pages;
    std::vector<int> free_pages;  // LIFO of local page indices
    std::vector<Span> spans;
    int seq_len = 0;
    int base_position = 0;
};

}  // namespace

struct zrh_backend {
    zrh_pool* pool = nullptr;
    zr_context* ctx = nullptr;
    int max_seq_len = 4096;
    int position = 0;  // ForwardPass.position (forward_pass.rs:1774)
    SessionKV kv;
};

namespace {

// A host call that fails leaves the pool as it found it.  Sessions restore
// their saved page tables on failure, and the global pages that were bound to
// them during the call go back onto the free list in reverse pop order, which
// restores the LIFO order exactly.  Calls nest (a chunked prefill runs one
// microbatch per chunk): each rolls back only what was popped after its mark.
class PoolTxn {
  public:
    explicit PoolTxn(zrh_pool* pool) : pool_(pool), mark_(pool ? pool->popped.size() : 0) {
        if (pool_) ++pool_->txn_depth;
    }
    ~PoolTxn() {
        if (pool_ && --pool_->txn_depth == 0) pool_->popped.clear();
    }
    PoolTxn(const PoolTxn&) = delete;
    PoolTxn& operator=(const PoolTxn&) = delete;
    void rollback() {
        if (!pool_) return;
        while (pool_->popped.size() > mark_) {
            pool_->free_list.push_back(pool_->popped.back());
            pool_->popped.pop_back();
        }
    }

  private:
    zrh_pool* pool_;
    size_t mark_;
};

zr_status fail(zrh_backend* b, zr_status code, const char* msg, int a = 0, int c = 0, int d = 0) {
    return set_err(b ? b->ctx : nullptr, code, msg, a, c, d);
}

// allocate_page (forward_pass.rs:396-424): LIFO reuse, else a new local page
// bound to a fresh global page of the pool.
zr_status allocate_page(zrh_backend* b, int* out) {
    SessionKV& kv = b->kv;
    if (!kv.free_pages.empty()) {
        const int idx = kv.free_pages.back();
        kv.free_pages.pop_back();
        if (kv.pages[idx].active)
            return fail(b, ZR_E_INVARIANT, "Device KV allocator attempted to reuse page %d while it was Active", idx);
        kv.pages[idx].used_rows = 0;
        kv.pages[idx].active = true;
        *out = idx;
        return ZR_OK;
    }
    if (b->pool->free_list.empty())
        return fail(b, ZR_E_OOM, "KV pool exhausted: no free global page for local page %d", (int)kv.pages.size());
    PageEntry pe;
    pe.global = b->pool->free_list.back();
    b->pool->free_list.pop_back();
    if (b->pool->txn_depth) b->pool->popped.push_back(pe.global);
    pe.active = true;
    kv.pages.push_back(pe);
    *out = (int)kv.pages.size() - 1;
    return ZR_OK;
}

// release_page (426-446)
zr_status release_page(zrh_backend* b, int idx) {
    SessionKV& kv = b->kv;
    if (idx < 0 || idx >= (int)kv.pages.size()) return fail(b, ZR_E_INVARIANT, "Invalid device KV page index %d", idx);
    if (!kv.pages[idx].active) return fail(b, ZR_E_INVARIANT, "Device KV allocator double-freed page %d", idx);
    kv.pages[idx].used_rows = 0;
    kv.pages[idx].active = false;
    kv.free_pages.push_back(idx);
    return ZR_OK;
}

// reclaim_unused_pages (448-460)
zr_status reclaim_unused(zrh_backend* b) {
    SessionKV& kv = b->kv;
    std::vector<char> referenced(kv.pages.size(), 0);
    for (const Span& s : kv.spans) referenced[s.page_index] = 1;
    for (int p = 0; p < (int)kv.pages.size(); ++p)
        if (!referenced[p] && kv.pages[p].used_rows != 0) {
            zr_status rc = release_page(b, p);
            if (rc) return rc;
        }
    return ZR_OK;
}

// DeviceLayerKVCache::clear (840-850): free list re-seeded 0..n
void clear_kv(SessionKV& kv) {
    for (PageEntry& p : kv.pages) {
        p.used_rows = 0;
        p.active = false;
    }
    kv.free_pages.clear();
    for (int p = 0; p < (int)kv.pages.size(); ++p) kv.free_pages.push_back(p);
    kv.spans.clear();
    kv.seq_len = 0;
    kv.base_position = 0;
}

// DeviceKVCache::retain_suffix (1084-1094) over DeviceLayerKVCache::retain_suffix (852-881)
zr_status retain_suffix(zrh_backend* b, int keep) {
    SessionKV& kv = b->kv;
    if (keep < 0) keep = 0;
    const int seq = kv.seq_len;
    if (seq <= keep) return ZR_OK;
    if (keep == 0) {
        const int base = kv.base_position;
        clear_kv(kv);
        kv.base_position = base + seq;
        return ZR_OK;
    }
    int drop = seq - keep;
    while (drop > 0) {
        if (kv.spans.empty()) return fail(b, ZR_E_INVARIANT, "Device KV block table unexpectedly empty");
        Span& front = kv.spans.front();
        if (drop >= front.row_count) {
            drop -= front.row_count;
            const int idx = front.page_index;
            kv.spans.erase(kv.spans.begin());
            zr_status rc = release_page(b, idx);
            if (rc) return rc;
            continue;
        }
        front.start_row += drop;
        front.row_count -= drop;
        drop = 0;
    }
    kv.seq_len = keep;
    kv.base_position += seq - keep;
    return reclaim_unused(b);
}

// ensure_writable_tail (353-394) + the row bookkeeping of append (462-521)
zr_status reserve_rows(zrh_backend* b, int rows) {
    SessionKV& kv = b->kv;
    int done = 0;
    while (done < rows) {
        int idx;
        if (kv.spans.empty()) {
            zr_status rc = allocate_page(b, &idx);
            if (rc) return rc;
            kv.spans.push_back({idx, 0, 0});
        } else {
            const Span tail = kv.spans.back();
            const PageEntry& tp = kv.pages[tail.page_index];
            if (tail.start_row + tail.row_count != tp.used_rows)
                return fail(b, ZR_E_INVARIANT, "Device KV tail span for page %d is inconsistent: span end %d vs used_rows %d",
                            tail.page_index, tail.start_row + tail.row_count, tp.used_rows);
            if (kPageRows - tp.used_rows > 0) {
                idx = tail.page_index;
            } else {
                zr_status rc = allocate_page(b, &idx);
                if (rc) return rc;
                kv.spans.push_back({idx, 0, 0});
            }
        }
        PageEntry& pg = kv.pages[idx];
        const int n = std::min(kPageRows - pg.used_rows, rows - done);
        pg.used_rows += n;
        kv.spans.back().row_count += n;
        kv.seq_len += n;
        done += n;
    }
    return ZR_OK;
}

// DeviceKVCache::append_layer (920-957) applied to every layer at once.
zr_status append_rows(zrh_backend* b, int rows) {
    const int max_seq = std::max(b->max_seq_len, 1);
    if (rows > max_seq) rows = max_seq;
    if (b->kv.seq_len + rows > max_seq) {
        const int drop = b->kv.seq_len + rows - max_seq;
        zr_status rc = retain_suffix(b, std::max(0, b->kv.seq_len - drop));
        if (rc) return rc;
    }
    return reserve_rows(b, rows);
}

// Canonical device table of the live window: global pages oldest first,
// first-span start row.  Interior spans must be full pages from row 0 (the
// invariant the kernels' row = first_offset + logical index relies on).
zr_status device_table(zrh_backend* b, std::vector<int>& table, int* first_offset) {
    const SessionKV& kv = b->kv;
    table.clear();
    *first_offset = kv.spans.empty() ? 0 : kv.spans.front().start_row;
    for (size_t i = 0; i < kv.spans.size(); ++i) {
        const Span& s = kv.spans[i];
        if (i > 0 && s.start_row != 0)
            return fail(b, ZR_E_INVARIANT, "span %d starts at row %d", (int)i, s.start_row);
        if (i + 1 < kv.spans.size() && s.start_row + s.row_count != kPageRows)
            return fail(b, ZR_E_INVARIANT, "interior span %d ends at row %d", (int)i, s.start_row + s.row_count);
        table.push_back(kv.pages[s.page_index].global);
    }
    return ZR_OK;
}

struct Assembled {
    std::vector<int> q_len, kv_before, first_pos, first_offset, tables;
    int stride = 0;
};

// One microbatch row per session: trim the window for the incoming rows, then
// reserve them (attention_output 1446-1452 / the batched decode 2703-2723).
// Saved session state of one microbatch, restored when the call fails.
struct Saved {
    std::vector<SessionKV> kv;
    std::vector<int> pos;
    void restore(zrh_backend* const* backends, int n, PoolTxn& txn) {
        for (int i = 0; i < n && i < (int)kv.size(); ++i) {
            backends[i]->kv = kv[i];
            backends[i]->position = pos[i];
        }
        txn.rollback();
    }
};

// Every session of a microbatch draws from the same pool (one pool per
// context), so one PoolTxn covers the call.
zr_status assemble(zrh_backend* const* backends, int n, const int* q_len, bool decode_only, Assembled& out,
                   Saved& saved, PoolTxn& txn) {
    if (n <= 0 || !backends || !backends[0])
        return set_global_err(ZR_E_INVALID, "Decode microbatch requires at least one backend and token");
    zr_context* ctx = backends[0]->ctx;
    std::vector<std::vector<int>> tables(n);
    saved.kv.clear();
    saved.pos.clear();
    for (int i = 0; i < n; ++i) {
        zrh_backend* b = backends[i];
        if (!b || b->ctx != ctx) return set_err(ctx, ZR_E_INVALID, "microbatch mixes contexts");
        if (b->pool != backends[0]->pool) return set_err(ctx, ZR_E_INVALID, "microbatch mixes KV pools");
        for (int j = 0; j < i; ++j)
            if (backends[j] == b) return set_err(ctx, ZR_E_INVALID, "session %d appears twice in one microbatch", i);
        saved.kv.push_back(b->kv);
        saved.pos.push_back(b->position);
    }
    out = Assembled();
    zr_status rc = ZR_OK;
    for (int i = 0; i < n && !rc; ++i) {
        zrh_backend* b = backends[i];
        const int ql = q_len[i];
        if (ql <= 0) rc = set_err(ctx, ZR_E_INVALID, "session %d has q_len %d", i, ql);
        else if (ql > std::max(b->max_seq_len, 1))
            rc = set_err(ctx, ZR_E_INVALID, "chunk of %d tokens exceeds the %d-token window", ql, b->max_seq_len);
        else if (decode_only && b->position == 0)
            rc = set_err(ctx, ZR_E_INVALID, "Decode microbatch requested before prompt prefill");
        else if (b->kv.base_position + b->kv.seq_len != b->position)
            rc = set_err(ctx, ZR_E_INVARIANT, "Forward pass position %d diverged from KV cache next position %d",
                         b->position, b->kv.base_position + b->kv.seq_len);
        if (rc) break;
        const int max_seq = std::max(b->max_seq_len, 1);
        if (b->kv.seq_len + ql > max_seq) {
            const int drop = b->kv.seq_len + ql - max_seq;
            rc = retain_suffix(b, std::max(0, b->kv.seq_len - drop));
            if (rc) break;
        }
        const int prefix = b->kv.seq_len;
        if (b->position != b->kv.base_position + prefix) {
            rc = set_err(ctx, ZR_E_INVARIANT, "Non-contiguous attention positions: expected %d, got %d",
                         b->kv.base_position + prefix, b->position);
            break;
        }
        rc = reserve_rows(b, ql);
        if (rc) break;
        int foff = 0;
        rc = device_table(b, tables[i], &foff);
        if (rc) break;
        out.q_len.push_back(ql);
        out.kv_before.push_back(prefix);
        out.first_pos.push_back(b->position);
        out.first_offset.push_back(foff);
        out.stride = std::max(out.stride, (int)tables[i].size());
    }
    if (rc) {
        saved.restore(backends, n, txn);
        return rc;
    }
    out.tables.assign((size_t)n * out.stride, 0);
    for (int i = 0; i < n; ++i) std::copy(tables[i].begin(), tables[i].end(), out.tables.begin() + (size_t)i * out.stride);
    return ZR_OK;
}

zr_microbatch as_microbatch(const Assembled& a, const uint32_t* tokens) {
    zr_microbatch mb;
    mb.num_seqs = (int)a.q_len.size();
    mb.q_len = a.q_len.data();
    mb.kv_before = a.kv_before.data();
    mb.first_pos = a.first_pos.data();
    mb.first_offset = a.first_offset.data();
    mb.block_tables = a.tables.data();
    mb.block_table_stride = a.stride;
    mb.tokens = tokens;
    return mb;
}

zr_status run_mixed(zrh_backend* const* backends, int n, const int* q_len, const uint32_t* tokens, bool decode_only,
                    uint32_t* out_tokens, float* out_logits, float* out_partials) {
    if (n <= 0 || !backends || !backends[0])
        return set_global_err(ZR_E_INVALID, "Decode microbatch requires at least one backend and token");
    PoolTxn txn(backends[0]->pool);
    Assembled a;
    Saved saved;
    zr_status rc = assemble(backends, n, q_len, decode_only, a, saved, txn);
    if (rc) return rc;
    // the page tables of a bookkeeping-only pool are assembled (and rolled
    // back) like any other; only the compute needs a device
    if (!backends[0]->ctx) rc = set_global_err(ZR_E_INVALID, "bookkeeping-only pool has no device context");
    zr_microbatch mb = as_microbatch(a, tokens);
    if (!rc) rc = zr_forward(backends[0]->ctx, &mb, out_tokens, out_logits, out_partials);
    if (rc) {
        saved.restore(backends, n, txn);
        return rc;
    }
    for (int i = 0; i < n; ++i) backends[i]->position += q_len[i];
    return ZR_OK;
}

}  // namespace

extern "C" {

zr_status zrh_pool_create(zr_context* ctx, const int* initial_order, int n, zrh_pool** out) {
    if (!out) return set_global_err(ZR_E_INVALID, "null argument");
    // ctx == NULL: a bookkeeping-only pool of n pages (page tables without a device)
    const int pages = ctx ? zr_kv_pool_pages(ctx) : n;
    if (pages <= 0) return set_err(ctx, ZR_E_INVALID, ctx ? "KV pool not created" : "pool of %d pages", n);
    zrh_pool* p = new zrh_pool();
    p->ctx = ctx;
    if (initial_order) {
        if (n != pages) {
            delete p;
            return set_err(ctx, ZR_E_INVALID, "initial order has %d pages, pool has %d", n, pages);
        }
        std::vector<char> seen(pages, 0);
        for (int i = 0; i < n; ++i) {
            if (initial_order[i] < 0 || initial_order[i] >= pages || seen[initial_order[i]]) {
                delete p;
                return set_err(ctx, ZR_E_INVALID, "initial order is not a permutation of the pool pages");
            }
            seen[initial_order[i]] = 1;
        }
        p->free_list.assign(initial_order, initial_order + n);
    } else {
        for (int i = pages - 1; i >= 0; --i) p->free_list.push_back(i);
    }
    *out = p;
    return ZR_OK;
}

void zrh_pool_destroy(zrh_pool* pool) { delete pool; }
int zrh_pool_free_pages(const zrh_pool* pool) { return pool ? (int)pool->free_list.size() : 0; }

zr_status zrh_backend_create(zrh_pool* pool, int max_seq_len, zrh_backend** out) {
    if (!pool || !out) return set_global_err(ZR_E_INVALID, "null argument");
    zrh_backend* b = new zrh_backend();
    b->pool = pool;
    b->ctx = pool->ctx;
    b->max_seq_len = max_seq_len;
    *out = b;
    return ZR_OK;
}

void zrh_backend_destroy(zrh_backend* b) {
    if (!b) return;
    zrh_release_pages(b);
    delete b;
}

zr_status zrh_prefill(zrh_backend* b, const uint32_t* tokens, int n, float* logits, uint32_t* greedy) {
    if (!b || !tokens) return set_global_err(ZR_E_INVALID, "null argument");
    if (n <= 0) return set_err(b->ctx, ZR_E_INVALID, "Cannot prefill an empty prompt without an explicit BOS policy");
    PoolTxn txn(b->pool);
    const SessionKV saved = b->kv;
    const int saved_pos = b->position;
    // clear_cache + keep the last window (forward_pass.rs:2101-2105)
    clear_kv(b->kv);
    b->position = 0;
    const int window = std::max(b->max_seq_len, 1);
    const int start = n > window ? n - window : 0;
    b->kv.base_position = start;
    b->position = start;
    // prompts longer than the context's row capacity run as causal chunks
    // with the earlier chunks as cached prefix (the same attention rows)
    const int cap = std::max(b->ctx ? b->ctx->desc.max_tokens : window, 1);
    uint32_t tok;
    zr_status rc = ZR_OK;
    for (int off = start; off < n && !rc; off += cap) {
        const int ql = std::min(cap, n - off);
        const bool last = off + ql >= n;
        rc = run_mixed(&b, 1, &ql, tokens + off, false, last && greedy ? greedy : &tok, last ? logits : nullptr,
                       nullptr);
    }
    if (rc) {
        b->kv = saved;
        b->position = saved_pos;
        txn.rollback();
    }
    return rc;
}

zr_status zrh_decode_step(zrh_backend* b, uint32_t token, float* logits, uint32_t* greedy) {
    if (!b) return set_global_err(ZR_E_INVALID, "null argument");
    if (b->position == 0) return set_err(b->ctx, ZR_E_INVALID, "Decode step requested before prompt prefill");
    const int one = 1;
    uint32_t tok;
    return run_mixed(&b, 1, &one, &token, true, greedy ? greedy : &tok, logits, nullptr);
}

zr_status zrh_decode_step_batch(zrh_backend* const* backends, int n, const uint32_t* tokens, uint32_t* out_tokens,
                                float* out_logits, float* out_partials) {
    if (!backends || !tokens || n <= 0) return set_global_err(ZR_E_INVALID, "Decode microbatch requires at least one backend and token");
    std::vector<int> ones(n, 1);
    return run_mixed(backends, n, ones.data(), tokens, true, out_tokens, out_logits, out_partials);
}

zr_status zrh_decode_step_batch_sampled(zrh_backend* const* backends, int n, const uint32_t* tokens,
                                        const float* temperature, const float* top_p, const uint64_t* seeds,
                                        uint32_t* out_tokens, float* out_logits, float* out_partials) {
    if (!backends || !tokens || n <= 0) return set_global_err(ZR_E_INVALID, "Decode microbatch requires at least one backend and token");
    if (!temperature || !top_p || !seeds || !out_tokens) return set_global_err(ZR_E_INVALID, "null argument");
    std::vector<int> ones(n, 1);
    zr_status rc = run_mixed(backends, n, ones.data(), tokens, true, out_tokens, out_logits, out_partials);
    if (rc) return rc;
    bool stochastic = false;
    for (int i = 0; i < n; ++i) stochastic |= temperature[i] > 0.0f && top_p[i] > 0.0f;
    if (!stochastic) return ZR_OK;  // the argmax of the forward is the answer
    // the step itself succeeded; a sampling failure is reported as such (backend.rs:137-151)
    rc = zr_sample_last_logits(backends[0]->ctx, n, temperature, top_p, seeds, out_tokens);
    if (rc) {
        const std::string why = zr_last_error(backends[0]->ctx);
        set_err(backends[0]->ctx, rc, "Device stochastic sampling failed: %s", why.c_str());
    }
    return rc;
}

zr_status zrh_forward_mixed(zrh_backend* const* backends, int n, const int* q_len, const uint32_t* tokens,
                            uint32_t* out_tokens, float* out_logits, float* out_partials) {
    if (!backends || !tokens || !q_len || n <= 0) return set_global_err(ZR_E_INVALID, "null argument");
    return run_mixed(backends, n, q_len, tokens, false, out_tokens, out_logits, out_partials);
}

zr_status zrh_stage_mixed(zrh_backend* const* backends, int n, const int* q_len, const uint32_t* tokens,
                          zr_staged** out) {
    if (!backends || !backends[0] || !q_len || !out || n <= 0) return set_global_err(ZR_E_INVALID, "null argument");
    PoolTxn txn(backends[0]->pool);
    Assembled a;
    Saved saved;
    zr_status rc = assemble(backends, n, q_len, false, a, saved, txn);
    if (rc) return rc;
    if (!backends[0]->ctx) rc = set_global_err(ZR_E_INVALID, "bookkeeping-only pool has no device context");
    zr_microbatch mb = as_microbatch(a, tokens);
    if (!rc) rc = zr_stage(backends[0]->ctx, &mb, out);
    if (rc) {
        saved.restore(backends, n, txn);
        return rc;
    }
    for (int i = 0; i < n; ++i) backends[i]->position += q_len[i];
    return ZR_OK;
}

int zrh_cache_seq_len(const zrh_backend* b) { return b ? b->kv.seq_len : 0; }
int zrh_sequence_position(const zrh_backend* b) { return b ? b->position : 0; }
int zrh_logical_kv_tokens(const zrh_backend* b) { return b ? b->position - b->kv.base_position : 0; }
int zrh_base_position(const zrh_backend* b) { return b ? b->kv.base_position : 0; }
int zrh_allocated_pages(const zrh_backend* b) { return b ? (int)b->kv.pages.size() : 0; }

uint64_t zrh_live_kv_cache_bytes(const zrh_backend* b) {
    // DeviceLayerKVCache::memory_usage (883-891) summed over layers, at the
    // pool's element size.
    if (!b || !b->ctx) return 0;
    const zr_context* ctx = b->ctx;
    const uint64_t esz = ctx->desc.kv_dtype == ZR_DTYPE_BF16 ? 2 : 4;
    return (uint64_t)b->kv.pages.size() * kPageRows * ctx->kv_cols * esz * 2 * ctx->desc.num_layers;
}

int zrh_block_table(const zrh_backend* b, uint32_t* page_ids, int* start_tokens, int* token_counts, int* global_pages,
                    int capacity) {
    if (!b) return set_global_err(ZR_E_INVALID, "null backend");
    const SessionKV& kv = b->kv;
    const int n = (int)kv.spans.size();
    if (page_ids || start_tokens || token_counts || global_pages) {
        if (capacity < n) return set_err(b->ctx, ZR_E_INVALID, "block table has %d spans > capacity %d", n, capacity);
        for (int i = 0; i < n; ++i) {
            const Span& s = kv.spans[i];
            if (page_ids) page_ids[i] = (uint32_t)s.page_index;
            if (start_tokens) start_tokens[i] = s.start_row;
            if (token_counts) token_counts[i] = s.row_count;
            if (global_pages) global_pages[i] = kv.pages[s.page_index].global;
        }
    }
    return n;
}

extern "C++" {
// export_kv_cache's checks and window; `gather` copies rows [first, first + keep)
template <typename Gather>
static zr_status export_rows(zrh_backend* b, int max_cached_tokens, int* rows, int* base_position,
                             int* next_position, bool have_buffers, Gather gather) {
    const SessionKV& kv = b->kv;
    if (kv.base_position + kv.seq_len != b->position)
        return set_err(b->ctx, ZR_E_INVARIANT, "Device KV export next_position %d does not match cache next position %d",
                       b->position, kv.base_position + kv.seq_len);
    if (next_position) *next_position = b->position;
    *rows = 0;
    if (base_position) *base_position = kv.base_position;
    if (kv.seq_len == 0) return ZR_OK;
    int keep = kv.seq_len;
    if (max_cached_tokens >= 0) keep = std::min(keep, std::max(max_cached_tokens, 1));
    if (!have_buffers) return set_err(b->ctx, ZR_E_INVALID, "null export buffers");
    if (!b->ctx) return set_global_err(ZR_E_INVALID, "bookkeeping-only pool has no device context");
    std::vector<int> table;
    int foff = 0;
    zr_status rc = device_table(b, table, &foff);
    if (!rc) rc = gather(table, foff, kv.seq_len - keep, keep);
    if (rc) return rc;
    *rows = keep;
    if (base_position) *base_position = kv.base_position + (kv.seq_len - keep);
    return ZR_OK;
}
}  // extern "C++"

zr_status zrh_export_kv_async(const zrh_backend* cb, int max_cached_tokens, float* k, float* v, int* rows,
                              int* base_position, int* next_position, zr_transfer** out) {
    zrh_backend* b = (zrh_backend*)cb;
    if (!b || !rows || !out) return set_global_err(ZR_E_INVALID, "null argument");
    *out = nullptr;
    return export_rows(b, max_cached_tokens, rows, base_position, next_position, k && v,
                       [&](const std::vector<int>& table, int foff, int first, int keep) {
                           return zr_kv_gather_async(b->ctx, table.data(), (int)table.size(), foff, first, keep, k, v,
                                                     out);
                       });
}

zr_status zrh_export_kv(const zrh_backend* cb, int max_cached_tokens, float* k, float* v, int* rows,
                        int* base_position, int* next_position) {
    zrh_backend* b = (zrh_backend*)cb;
    if (!b || !rows) return set_global_err(ZR_E_INVALID, "null argument");
    return export_rows(b, max_cached_tokens, rows, base_position, next_position, k && v,
                       [&](const std::vector<int>& table, int foff, int first, int keep) {
                           return zr_kv_gather(b->ctx, table.data(), (int)table.size(), foff, first, keep, k, v);
                       });
}

extern "C++" {
// import_kv_cache's checks, page binding and rollback; `scatter` writes the rows
template <typename Scatter>
static zr_status import_rows(zrh_backend* b, int rows, int base_position, int next_position, bool have_rows,
                             Scatter scatter) {
    if (rows < 0 || rows > next_position)
        return set_err(b->ctx, ZR_E_INVALID, "KV sequence state is invalid: cached_tokens %d exceeds next_position %d",
                       rows, next_position);
    if (base_position != next_position - rows)
        return set_err(b->ctx, ZR_E_INVALID, "KV snapshot base position mismatch: payload starts at %d, sequence metadata says %d",
                       base_position, next_position - rows);
    PoolTxn txn(b->pool);
    const SessionKV saved = b->kv;
    const int saved_pos = b->position;
    clear_kv(b->kv);
    b->kv.base_position = base_position;
    zr_status rc = ZR_OK;
    if (rows > 0) {
        if (!have_rows) rc = set_err(b->ctx, ZR_E_INVALID, "null import buffers");
        const int max_seq = std::max(b->max_seq_len, 1);
        const int keep = std::min(rows, max_seq);
        if (!rc) rc = append_rows(b, keep);
        if (!rc && b->kv.seq_len != rows)
            rc = set_err(b->ctx, ZR_E_INVARIANT, "Recovered device KV cache length %d does not match snapshot cached token count %d",
                         b->kv.seq_len, rows);
        // page tables of a bookkeeping-only pool are built (and rolled back); the copy needs a device
        if (!rc && !b->ctx) rc = set_global_err(ZR_E_INVALID, "bookkeeping-only pool has no device context");
        std::vector<int> table;
        int foff = 0;
        if (!rc) rc = device_table(b, table, &foff);
        if (!rc) rc = scatter(table, foff);
    }
    if (!rc && b->kv.base_position != next_position - rows)
        rc = set_err(b->ctx, ZR_E_INVARIANT, "Recovered device KV cache base position %d does not match snapshot first cached position %d",
                     b->kv.base_position, next_position - rows);
    if (rc) {
        b->kv = saved;
        b->position = saved_pos;
        txn.rollback();
        return rc;
    }
    b->position = next_position;
    return ZR_OK;
}
}  // extern "C++"

zr_status zrh_import_kv(zrh_backend* b, const float* k, const float* v, int rows, int base_position,
                        int next_position) {
    if (!b) return set_global_err(ZR_E_INVALID, "null argument");
    return import_rows(b, rows, base_position, next_position, k && v, [&](const std::vector<int>& table, int foff) {
        return zr_kv_scatter(b->ctx, table.data(), (int)table.size(), foff, 0, rows, k, v);
    });
}

zr_status zrh_import_kv_transfer(zrh_backend* b, zr_transfer* t, int rows, int base_position, int next_position) {
    if (!b || !t) return set_global_err(ZR_E_INVALID, "null argument");
    return import_rows(b, rows, base_position, next_position, true, [&](const std::vector<int>& table, int foff) {
        return zr_kv_scatter_transfer(b->ctx, t, table.data(), (int)table.size(), foff, 0, rows);
    });
}

zr_status zrh_export_kv_cbor(const zrh_backend* cb, int max_cached_tokens, uint8_t* out, size_t capacity,
                             size_t* out_len, int* next_position, int* cached_tokens) {
    zrh_backend* b = (zrh_backend*)cb;
    if (!b || !out_len) return set_global_err(ZR_E_INVALID, "null argument");
    const SessionKV& kv = b->kv;
    if (kv.base_position + kv.seq_len != b->position)
        return set_err(b->ctx, ZR_E_INVARIANT, "Device KV export next_position %d does not match cache next position %d",
                       b->position, kv.base_position + kv.seq_len);
    if (next_position) *next_position = b->position;
    if (cached_tokens) *cached_tokens = 0;
    *out_len = 0;
    if (kv.seq_len == 0) return ZR_OK;
    if (!b->ctx) return set_global_err(ZR_E_INVALID, "bookkeeping-only pool has no device context");
    int keep = kv.seq_len;
    if (max_cached_tokens >= 0) keep = std::min(keep, std::max(max_cached_tokens, 1));
    std::vector<int> table;
    int foff = 0;
    zr_status rc = device_table(b, table, &foff);
    // the retained rows start at base_position + dropped rows (KVCache::retain_suffix, kv_cache.rs:847-872)
    if (!rc)
        rc = zr_kv_export_cbor(b->ctx, table.data(), (int)table.size(), foff, kv.seq_len - keep, keep,
                               (long long)kv.base_position + (kv.seq_len - keep), b->max_seq_len, out, capacity,
                               out_len);
    if (rc) return rc;
    if (cached_tokens) *cached_tokens = keep;
    return ZR_OK;
}

zr_status zrh_import_kv_cbor(zrh_backend* b, const uint8_t* bytes, size_t len, int next_position,
                             int cached_tokens) {
    if (!b || (!bytes && len)) return set_global_err(ZR_E_INVALID, "null argument");
    zr_context* ctx = b->ctx;
    // KVSequenceState::validate (kv_cache.rs:50-58)
    if (cached_tokens < 0 || cached_tokens > next_position)
        return set_err(ctx, ZR_E_INVALID, "KV sequence state is invalid: cached_tokens %d exceeds next_position %d",
                       cached_tokens, next_position);
    zr::KvCborDoc doc;
    std::string err;
    if (!zr::kv_cbor_decode(bytes, len, &doc, &err))
        return set_err(ctx, ZR_E_INVALID, "Failed to deserialize KV cache: %s", err.c_str());
    // KVCacheSnapshot::validate_with_cache (kv_cache.rs:121-141)
    if (doc.rows != cached_tokens)
        return set_err(ctx, ZR_E_INVALID, "KV snapshot cached token mismatch: payload has %lld tokens, sequence metadata says %d",
                       doc.rows, cached_tokens);
    if (doc.base_position != (long long)next_position - cached_tokens)
        return set_err(ctx, ZR_E_INVALID, "KV snapshot base position mismatch: payload starts at %lld, sequence metadata says %d",
                       doc.base_position, next_position - cached_tokens);
    if (doc.rows > 0 && ctx) {
        if (doc.layers != ctx->desc.num_layers)
            return set_err(ctx, ZR_E_INVALID, "KV snapshot has %d layers, the model has %d", doc.layers,
                           ctx->desc.num_layers);
        if (doc.cols != ctx->kv_cols)
            return set_err(ctx, ZR_E_INVALID, "KV cache append width mismatch: snapshot rows of %lld, cache rows of %d",
                           doc.cols, ctx->kv_cols);
    }
    return zrh_import_kv(b, doc.rows ? doc.k.data() : nullptr, doc.rows ? doc.v.data() : nullptr, (int)doc.rows,
                         (int)doc.base_position, next_position);
}

void zrh_clear(zrh_backend* b) {
    if (!b) return;
    clear_kv(b->kv);
    b->position = 0;
}

zr_status zrh_release_pages(zrh_backend* b) {
    if (!b) return set_global_err(ZR_E_INVALID, "null backend");
    for (const PageEntry& p : b->kv.pages)
        if (p.global >= 0) b->pool->free_list.push_back(p.global);
    b->kv = SessionKV();
    b->position = 0;
    return ZR_OK;
}

// ------------------------------------------------------------ fast path
// Buckets of fast_path.rs:15-16 (decode), in the planner's search order.
static const int kDecodeBucketBatches[] = {1, 2, 4, 8};
static const int kDecodeBucketKvTokens[] = {2048, 8192, 16384, 32768, 65536};

zr_status zrh_get_fast_path_context(const zrh_backend* b, zrh_fast_path_context* out) {
    if (!b || !out) return set_global_err(ZR_E_INVALID, "null argument");
    out->logical_kv_tokens = b->position - b->kv.base_position;
    out->position = b->position;
    out->cached_tokens = b->kv.seq_len;
    out->decode_token_ceiling = -1;
    for (int t : kDecodeBucketKvTokens)
        if (out->logical_kv_tokens <= t) {
            out->decode_token_ceiling = t;
            break;
        }
    return ZR_OK;
}

}  // extern "C"

// FNV-1a 64 over the layout's items (zrh_fast_path_plan.layout_hash).
struct LayoutHasher {
    uint64_t h = 0xcbf29ce484222325ull;
    void byte(uint8_t b) { h = (h ^ b) * 0x100000001b3ull; }
    void u64(uint64_t v) {
        for (int i = 0; i < 8; ++i) byte((uint8_t)(v >> (8 * i)));
    }
    void str(const char* s) {
        for (; *s; ++s) byte((uint8_t)*s);
        byte(0xff);
    }
};

static const char* const kMetadataFieldNames[4] = {"slot_sequence_lengths", "slot_positions", "slot_block_tables",
                                                   "slot_mapping"};

static uint64_t plan_layout_hash(const zrh_fast_path_plan* p) {
    LayoutHasher h;
    h.u64((uint64_t)p->phase);
    h.str("rocm");
    h.str("rocm_fused");
    h.u64((uint64_t)p->batch_size_ceiling);
    h.u64((uint64_t)p->token_ceiling);
    for (int f = 0; f < 4; ++f) {
        h.str(kMetadataFieldNames[f]);
        h.u64(sizeof(uint32_t));
        h.u64(p->field_bytes[f] / sizeof(uint32_t));
        h.u64(p->field_bytes[f]);
    }
    return h.h;
}

// FastPathPlanner::build_plan (fast_path.rs:780-829) for the rocm_fused profile.
static void build_plan(int phase, int bb, int bt, int batch, int tokens, int max_seq, zrh_fast_path_plan* out) {
    memset(out, 0, sizeof *out);
    out->phase = phase;
    out->batch_size_ceiling = bb;
    out->token_ceiling = bt;
    out->actual_batch_size = batch;
    out->actual_token_count = tokens;
    out->max_sequence_len = max_seq;
    out->page_slots = (bt + kPageRows - 1) / kPageRows;
    // metadata_fields (839-867): the same four u32 fields for either phase
    const size_t widths[4] = {(size_t)bb, (size_t)bb, (size_t)bb * out->page_slots, (size_t)bb};
    size_t off = 0;
    for (int f = 0; f < 4; ++f) {
        out->field_offset[f] = off;
        out->field_bytes[f] = widths[f] * sizeof(uint32_t);
        off += out->field_bytes[f];
    }
    out->metadata_bytes = off;
    // workspace_requirements (869-890): the fused profile's 96 B per token and 32 KiB per slot
    out->workspace_bytes = off + (size_t)bt * 96 + (size_t)bb * 32 * 1024;
    out->workspace_alignment = 256;
    if (phase == 0)
        snprintf(out->bucket_label, sizeof out->bucket_label, "decode-b%d-kv%d-rocm", bb, bt);
    else
        snprintf(out->bucket_label, sizeof out->bucket_label, "prefill-t%d-rocm", bt);
    snprintf(out->capture_strategy, sizeof out->capture_strategy, "replay_preferred");
    if (phase == 1) snprintf(out->prefill_strategy, sizeof out->prefill_strategy, "single_sequence_buckets");
    out->layout_hash = plan_layout_hash(out);
}

// Buckets of fast_path.rs:17 (prefill).
static const int kPrefillBucketTokens[] = {128, 512, 2048, 8192, 16384};

extern "C" {

zr_status zrh_fast_path_plan_decode(int batch_size, int total_kv_tokens, int max_sequence_len,
                                    zrh_fast_path_plan* out) {
    if (!out) return set_global_err(ZR_E_INVALID, "null argument");
    if (batch_size < 0 || total_kv_tokens < 0 || max_sequence_len < 0)
        return set_global_err(ZR_E_INVALID, "negative batch size or token count");
    int bb = -1, bt = -1;
    for (int b : kDecodeBucketBatches) {
        for (int t : kDecodeBucketKvTokens)
            if (batch_size <= b && total_kv_tokens <= t) {
                bb = b;
                bt = t;
                break;
            }
        if (bb >= 0) break;
    }
    if (bb < 0)
        return set_global_err(ZR_E_UNSUPPORTED, "no stable Decode bucket supports batch_size=%d token_count=%d for RocmFused",
                              batch_size, total_kv_tokens);
    build_plan(0, bb, bt, batch_size, total_kv_tokens, max_sequence_len, out);
    return ZR_OK;
}

zr_status zrh_fast_path_plan_prefill(int prompt_tokens, zrh_fast_path_plan* out) {
    if (!out) return set_global_err(ZR_E_INVALID, "null argument");
    if (prompt_tokens < 0) return set_global_err(ZR_E_INVALID, "negative token count");
    for (int t : kPrefillBucketTokens)
        if (prompt_tokens <= t) {
            build_plan(1, 1, t, 1, prompt_tokens, prompt_tokens, out);
            return ZR_OK;
        }
    return set_global_err(ZR_E_UNSUPPORTED, "no stable Prefill bucket supports batch_size=1 token_count=%d for RocmFused",
                          prompt_tokens);
}

zr_status zrh_fast_path_stage_prefill_positions(const zrh_fast_path_plan* plan, uint64_t absolute_position_start,
                                                int token_count, uint32_t* positions) {
    if (!plan || !positions || token_count < 0) return set_global_err(ZR_E_INVALID, "null argument or negative count");
    if (plan->phase != 1)
        return set_global_err(ZR_E_INVALID, "prefill workspace checkout requires prefill plan, got Decode");
    if (token_count > plan->token_ceiling)
        return set_global_err(ZR_E_INVALID,
                              "fast-path capture invariant failed for prefill-t%d-rocm: prefill token count %d exceeds "
                              "bucket ceiling %d",
                              plan->token_ceiling, token_count, plan->token_ceiling);
    std::fill(positions, positions + plan->token_ceiling, 0u);  // PrefillWorkspaceBuffers::reset
    for (int i = 0; i < token_count; ++i) {
        const uint64_t p = absolute_position_start + (uint64_t)i;
        if (p < absolute_position_start || p > 0xFFFFFFFFull)
            return set_global_err(ZR_E_INVALID, "prefill absolute position exceeded u32 addressable range");
        positions[i] = (uint32_t)p;
    }
    return ZR_OK;
}

zr_status zrh_fast_path_validate_decode_contexts(const zrh_fast_path_plan* plan,
                                                 const zrh_fast_path_backend_context* contexts, int n) {
    if (!plan || (n > 0 && !contexts) || n < 0) return set_global_err(ZR_E_INVALID, "null argument");
    const char* label = plan->bucket_label;
    auto unsafe = [&](const char* fmt, auto... args) {
        char detail[256];
        snprintf(detail, sizeof detail, fmt, args...);
        return set_global_err(ZR_E_INVALID, "fast-path capture invariant failed for %s: %s", label, detail);
    };
    if (n != plan->actual_batch_size)
        return unsafe("planned batch size %d but executor received %d requests", plan->actual_batch_size, n);
    if (n == 0) return ZR_OK;
    auto is_plan_kind = [](const zrh_fast_path_backend_context& c) {
        return c.provider && c.optimization_profile && strcmp(c.provider, "rocm") == 0 &&
               strcmp(c.optimization_profile, "rocm_fused") == 0;
    };
    if (!is_plan_kind(contexts[0])) return unsafe("%s", "primary backend context does not match planned provider/profile");
    const char* primary_model = contexts[0].model_id;
    for (int i = 0; i < n; ++i) {
        const zrh_fast_path_backend_context& c = contexts[i];
        if (!is_plan_kind(c))
            return unsafe("%s", "mixed provider/profile contexts cannot reuse a single fast-path bucket");
        if (c.logical_kv_tokens > plan->token_ceiling)
            return unsafe("session KV footprint %d exceeds bucket token ceiling %d", c.logical_kv_tokens,
                          plan->token_ceiling);
        if (primary_model && c.model_id && strcmp(primary_model, c.model_id) != 0)
            return unsafe("%s", "mixed model residencies cannot share one replay-valid bucket");
    }
    const uint64_t observed = plan_layout_hash(plan);
    if (observed != plan->layout_hash)
        return set_global_err(ZR_E_INVALID, "fast-path metadata drift for %s: expected layout hash %llu, observed %llu",
                              label, (unsigned long long)plan->layout_hash, (unsigned long long)observed);
    return ZR_OK;
}

zr_status zrh_fast_path_stage_decode(const zrh_fast_path_plan* plan, zrh_backend* const* backends, int n,
                                     const uint32_t* tokens, uint32_t* metadata, uint32_t* token_ids,
                                     uint32_t* positions) {
    if (!plan || !metadata || (n > 0 && (!backends || !tokens))) return set_global_err(ZR_E_INVALID, "null argument");
    const int B = plan->batch_size_ceiling, slots = plan->page_slots;
    zr_context* ctx = n > 0 && backends[0] ? backends[0]->ctx : nullptr;
    if (n > B)
        return set_err(ctx, ZR_E_INVALID, "fast-path capture invariant failed for %s: runtime batch size %d exceeds bucket ceiling %d",
                       plan->bucket_label, n, B);
    // reset (DecodeWorkspaceBuffers::reset): lengths and positions 0, tables and mapping u32::MAX
    uint32_t* seq_lens = metadata + plan->field_offset[0] / 4;
    uint32_t* slot_pos = metadata + plan->field_offset[1] / 4;
    uint32_t* tables = metadata + plan->field_offset[2] / 4;
    uint32_t* mapping = metadata + plan->field_offset[3] / 4;
    std::fill(seq_lens, seq_lens + B, 0u);
    std::fill(slot_pos, slot_pos + B, 0u);
    std::fill(tables, tables + (size_t)B * slots, 0xFFFFFFFFu);
    std::fill(mapping, mapping + B, 0xFFFFFFFFu);
    if (token_ids) std::fill(token_ids, token_ids + B, 0u);
    if (positions) std::fill(positions, positions + B, 0u);
    if (token_ids) std::copy(tokens, tokens + n, token_ids);
    for (int i = 0; i < n; ++i) {
        const zrh_backend* b = backends[i];
        if (!b) return set_global_err(ZR_E_INVALID, "null backend in slot %d", i);
        // decode_slot_state (forward_pass.rs:1065-1074)
        if (b->kv.base_position + b->kv.seq_len != b->position)
            return set_err(b->ctx, ZR_E_INVARIANT, "Forward pass position %d diverged from KV cache next position %d",
                           b->position, b->kv.base_position + b->kv.seq_len);
        const int seq = b->kv.seq_len;
        if (seq > plan->token_ceiling)
            return set_err(b->ctx, ZR_E_INVALID,
                           "fast-path capture invariant failed for %s: slot %d sequence length %d exceeds bucket token ceiling %d",
                           plan->bucket_label, i, seq, plan->token_ceiling);
        if ((int)b->kv.spans.size() > slots)
            return set_err(b->ctx, ZR_E_INVALID,
                           "fast-path capture invariant failed for %s: slot %d block table length %d exceeds workspace capacity %d",
                           plan->bucket_label, i, (int)b->kv.spans.size(), slots);
        if (positions) positions[i] = (uint32_t)b->position;
        seq_lens[i] = (uint32_t)seq;
        slot_pos[i] = (uint32_t)b->position;
        mapping[i] = (uint32_t)i;
        for (size_t p = 0; p < b->kv.spans.size(); ++p)
            tables[(size_t)i * slots + p] = (uint32_t)b->kv.spans[p].page_index;
    }
    return ZR_OK;
}

// ------------------------------------------------------ decode pipeline
}  // extern "C"

struct zrh_decode_pipeline {
    std::vector<zrh_backend*> backends;
    zr_context* ctx = nullptr;
    zr_step_graph* graph = nullptr;
    uint32_t* d_tok[2] = {nullptr, nullptr};  // ids in / out, alternating
    uint32_t* h_tok[2] = {nullptr, nullptr};  // pinned copies of each step's ids
    hipEvent_t done[2] = {nullptr, nullptr};  // the step's id copy has landed
    uint64_t steps = 0;
};

extern "C" {

zr_status zrh_decode_pipeline_create(zrh_backend* const* backends, int n, const uint32_t* first_tokens,
                                     zrh_decode_pipeline** out) {
    if (!backends || !first_tokens || !out || n <= 0 || !backends[0])
        return set_global_err(ZR_E_INVALID, "Decode microbatch requires at least one backend and token");
    zr_context* ctx = backends[0]->ctx;
    if (!ctx) return set_global_err(ZR_E_INVALID, "bookkeeping-only pool has no device context");
    for (int i = 0; i < n; ++i) {
        if (!backends[i] || backends[i]->ctx != ctx) return set_err(ctx, ZR_E_INVALID, "microbatch mixes contexts");
        for (int j = 0; j < i; ++j)
            if (backends[j] == backends[i])
                return set_err(ctx, ZR_E_INVALID, "session %d appears twice in one microbatch", i);
    }
    if (n > ctx->desc.max_seqs || n > ctx->desc.max_tokens)
        return set_err(ctx, ZR_E_INVALID, "microbatch has %d sequences (capacity %d)", n,
                       std::min(ctx->desc.max_seqs, ctx->desc.max_tokens));
    for (int i = 0; i < n; ++i)
        if (first_tokens[i] >= (uint32_t)ctx->desc.vocab)
            return set_err(ctx, ZR_E_INVALID, "Token %u out of vocabulary bounds %d", first_tokens[i], ctx->desc.vocab);
    ZR_HIP(ctx, hipSetDevice(ctx->device));
    zrh_decode_pipeline* p = new zrh_decode_pipeline();
    p->backends.assign(backends, backends + n);
    p->ctx = ctx;
    zr_status rc = zr_step_graph_create(ctx, &p->graph);
    hipError_t e = hipSuccess;
    for (int b = 0; b < 2 && !rc && e == hipSuccess; ++b) {
        e = hipMalloc((void**)&p->d_tok[b], 4 * (size_t)n);
        if (e == hipSuccess) e = hipHostMalloc((void**)&p->h_tok[b], 4 * (size_t)n, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&p->done[b], hipEventDisableTiming);
    }
    if (!rc && e == hipSuccess)
        e = hipMemcpy(p->d_tok[0], first_tokens, 4 * (size_t)n, hipMemcpyHostToDevice);
    if (!rc && e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "decode pipeline: %s", hipGetErrorString(e));
    if (rc) {
        zrh_decode_pipeline_destroy(p);
        return rc;
    }
    *out = p;
    return ZR_OK;
}

zr_status zrh_decode_pipeline_step(zrh_decode_pipeline* p, uint32_t* prev_tokens, int* prev_ready) {
    if (!p) return set_global_err(ZR_E_INVALID, "null argument");
    zr_context* ctx = p->ctx;
    const int n = (int)p->backends.size();
    if (prev_ready) *prev_ready = 0;
    const uint64_t i = p->steps;
    zrh_backend* const* bs = p->backends.data();
    // the decode rows of BackendMicrobatchExecutor::decode_step_batch:
    // window trim and page reservation per session (attention_output 1446-1452)
    PoolTxn txn(bs[0]->pool);
    Assembled a;
    Saved saved;
    std::vector<int> ones(n, 1);
    zr_status rc = assemble(bs, n, ones.data(), true, a, saved, txn);
    if (rc) return rc;
    zr_microbatch mb = as_microbatch(a, nullptr);
    rc = zr_step_graph_launch(p->graph, &mb, p->d_tok[i & 1], p->d_tok[(i + 1) & 1], p->h_tok[i & 1]);
    if (!rc) {
        const hipError_t e = hipEventRecord(p->done[i & 1], ctx->stream);
        if (e != hipSuccess) rc = set_err(ctx, ZR_E_HIP, "decode pipeline: %s", hipGetErrorString(e));
    }
    if (rc) {
        saved.restore(bs, n, txn);
        return rc;
    }
    for (int s = 0; s < n; ++s) bs[s]->position += 1;
    p->steps = i + 1;
    if (i > 0) {  // the previous step's ids: the host waits for that step only
        ZR_HIP(ctx, hipEventSynchronize(p->done[(i - 1) & 1]));
        if (prev_tokens) memcpy(prev_tokens, p->h_tok[(i - 1) & 1], 4 * (size_t)n);
        if (prev_ready) *prev_ready = 1;
    }
    return ZR_OK;
}

zr_status zrh_decode_pipeline_finish(zrh_decode_pipeline* p, uint32_t* last_tokens) {
    if (!p) return set_global_err(ZR_E_INVALID, "null argument");
    if (p->steps == 0) return set_err(p->ctx, ZR_E_INVALID, "decode pipeline has run no step");
    zr_status rc = zr_synchronize(p->ctx);  // also reports a device-fed id out of the vocabulary
    if (rc) return rc;
    if (last_tokens) memcpy(last_tokens, p->h_tok[(p->steps - 1) & 1], 4 * p->backends.size());
    return ZR_OK;
}

zr_status zrh_decode_pipeline_info(const zrh_decode_pipeline* p, uint64_t* steps, zr_step_graph_stats* graph) {
    if (!p) return set_global_err(ZR_E_INVALID, "null argument");
    if (steps) *steps = p->steps;
    return graph ? zr_step_graph_info(p->graph, graph) : ZR_OK;
}

void zrh_decode_pipeline_destroy(zrh_decode_pipeline* p) {
    if (!p) return;
    if (p->ctx && p->ctx->stream) (void)hipStreamSynchronize(p->ctx->stream);
    if (p->graph) zr_step_graph_destroy(p->graph);
    for (int b = 0; b < 2; ++b) {
        if (p->d_tok[b]) (void)hipFree(p->d_tok[b]);
        if (p->h_tok[b]) (void)hipHostFree(p->h_tok[b]);
        if (p->done[b]) (void)hipEventDestroy(p->done[b]);
    }
    delete p;
}

zr_status zrh_kv_reserve(zrh_backend* b, int rows) {
    if (!b) return set_global_err(ZR_E_INVALID, "null backend");
    if (rows <= 0) return set_err(b->ctx, ZR_E_INVALID, "Device KV append received an empty key shape");
    PoolTxn txn(b->pool);
    const SessionKV saved = b->kv;
    zr_status rc = append_rows(b, rows);
    if (rc) {
        b->kv = saved;
        txn.rollback();
        return rc;
    }
    b->position = b->kv.base_position + b->kv.seq_len;
    return ZR_OK;
}

zr_status zrh_retain_suffix(zrh_backend* b, int keep_rows) {
    if (!b) return set_global_err(ZR_E_INVALID, "null backend");
    const SessionKV saved = b->kv;
    zr_status rc = retain_suffix(b, keep_rows);
    if (rc) {
        b->kv = saved;
        return rc;
    }
    b->position = b->kv.base_position + b->kv.seq_len;
    return ZR_OK;
}

}  // extern "C"
