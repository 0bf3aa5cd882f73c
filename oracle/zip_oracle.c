/*
 * zip_oracle.c -- CPU restatement of the zip engine's hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the test oracle; see zip_oracle.h).  Plain C11 + OpenMP,
 * f32 throughout (except or_sample_token_device, which states an f32 rule of
 * unspecified evaluation order in f64), built with -ffp-contract=off so every
 * multiply and add rounds as the reference's Rust f32 code does.  OpenMP only splits independent output
 * elements; it never reorders an accumulation.
 */
#include "zip_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static char g_err[512];

static int fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
#pragma omp critical(oracle_err)
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return -1;
}

const char* or_last_error(void) { return g_err; }

/* ============================================================ ops ======= */

/* tensor_ops.rs:219-240.  The reference loops i, k, j with out[i][j] +=
 * a[i][k] * b[k][j]: every output element accumulates over k in order, which
 * this keeps exactly.  Tiles of 16 rows x 256 columns run in parallel and
 * reuse each weight block from cache; no accumulation is reordered. */
int or_matmul(const float* a, const float* b, float* c, int m, int k, int n) {
    if (m < 0 || k < 0 || n < 0) return fail("Matmul shape mismatch: %dx%d @ %dx%d", m, k, k, n);
    memset(c, 0, sizeof(float) * (size_t)m * (size_t)n);
    const int ib = 16, jb = 256;
    const int nib = (m + ib - 1) / ib, njb = (n + jb - 1) / jb;
#pragma omp parallel for collapse(2) schedule(static)
    for (int it = 0; it < nib; ++it) {
        for (int blk = 0; blk < njb; ++blk) {
            const int i0 = it * ib, i1 = i0 + ib < m ? i0 + ib : m;
            const int j0 = blk * jb, j1 = j0 + jb < n ? j0 + jb : n;
            for (int kk = 0; kk < k; ++kk) {
                const float* b_row = b + (size_t)kk * n;
                for (int i = i0; i < i1; ++i) {
                    const float a_ik = a[(size_t)i * k + kk];
                    float* out_row = c + (size_t)i * n;
                    for (int j = j0; j < j1; ++j) out_row[j] += a_ik * b_row[j];
                }
            }
        }
    }
    return 0;
}

/* tensor_ops.rs:285-304 */
int or_rms_norm(const float* x, const float* gamma, float* out, int rows, int cols, float eps) {
    if (cols <= 0) return fail("RMS norm dimension mismatch: cols %d", cols);
#pragma omp parallel for schedule(static) if (rows > 8)
    for (int r = 0; r < rows; ++r) {
        const float* s = x + (size_t)r * cols;
        float sum = 0.0f;
        for (int c = 0; c < cols; ++c) sum += s[c] * s[c];
        const float mean_square = sum / (float)cols;
        const float inv_rms = 1.0f / sqrtf(mean_square + eps);
        float* o = out + (size_t)r * cols;
        for (int c = 0; c < cols; ++c) o[c] = s[c] * inv_rms * gamma[c];
    }
    return 0;
}

/* tensor_ops.rs:268-278 */
void or_silu(const float* x, float* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* runtime.rs:282-301 / tensor_ops.rs:524-527: 1 / base^(2i/d) in f32. */
void or_rope_inv_freq(int head_dim, float base, float* inv_freq) {
    for (int i = 0; i < head_dim / 2; ++i)
        inv_freq[i] = 1.0f / powf(base, (float)i * 2.0f / (float)head_dim);
}

/* tensor_ops.rs:509-560: rotate-half RoPE per head with absolute positions. */
int or_apply_rope(const float* x, float* out, int rows, int cols, const uint32_t* positions,
                  int head_dim, float base) {
    if (head_dim % 2 != 0) return fail("RoPE requires even head_dim, got %d", head_dim);
    if (cols % head_dim != 0)
        return fail("RoPE head_dim %d does not divide tensor width %d", head_dim, cols);
    const int half = head_dim / 2;
    float inv_freq[1024];
    if (half > 1024) return fail("RoPE head_dim %d too large", head_dim);
    or_rope_inv_freq(head_dim, base, inv_freq);
    const int num_heads = cols / head_dim;
    for (int r = 0; r < rows; ++r) {
        const float position = (float)positions[r];
        for (int h = 0; h < num_heads; ++h) {
            const size_t off = (size_t)r * cols + (size_t)h * head_dim;
            for (int d = 0; d < half; ++d) {
                const float theta = position * inv_freq[d];
                const float c = cosf(theta), s = sinf(theta);
                const float left = x[off + d], right = x[off + half + d];
                out[off + d] = left * c - right * s;
                out[off + half + d] = left * s + right * c;
            }
        }
    }
    return 0;
}

/* tensor_ops.rs:461-473 */
uint32_t or_sample_greedy(const float* logits, int n) {
    int max_idx = 0;
    float max_val = -INFINITY;
    for (int i = 0; i < n; ++i)
        if (logits[i] > max_val) {
            max_val = logits[i];
            max_idx = i;
        }
    return (uint32_t)max_idx;
}

/* tensor_ops.rs:372-388: SplitMix64 finaliser -> 24-bit threshold. */
float or_sample_threshold(uint64_t seed) {
    uint64_t x = seed + 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    x ^= x >> 31;
    const uint32_t upper = (uint32_t)(x >> 40);
    double t = (double)upper / (double)(1ull << 24);
    const double hi = 1.0 - 2.220446049250313e-16;
    if (t < 0.0) t = 0.0;
    if (t > hi) t = hi;
    return (float)t;
}

typedef struct {
    int idx;
    float p;
} idx_prob;

/* Rust's sort_by is a stable merge sort: equal probabilities keep index order. */
static void stable_sort_desc(idx_prob* v, int n, idx_prob* tmp) {
    for (int width = 1; width < n; width *= 2) {
        for (int lo = 0; lo < n; lo += 2 * width) {
            int mid = lo + width < n ? lo + width : n;
            int hi = lo + 2 * width < n ? lo + 2 * width : n;
            int i = lo, j = mid, k = lo;
            while (i < mid && j < hi) tmp[k++] = (v[j].p > v[i].p) ? v[j++] : v[i++];
            while (i < mid) tmp[k++] = v[i++];
            while (j < hi) tmp[k++] = v[j++];
        }
        memcpy(v, tmp, sizeof(idx_prob) * (size_t)n);
    }
}

/* tensor_ops.rs:394-458 */
uint32_t or_sample_token(const float* logits, int n, float temperature, float top_p, uint64_t seed) {
    float* scaled = (float*)malloc(sizeof(float) * (size_t)n);
    float* probs = (float*)malloc(sizeof(float) * (size_t)n);
    idx_prob* ip = (idx_prob*)malloc(sizeof(idx_prob) * (size_t)n);
    idx_prob* tmp = (idx_prob*)malloc(sizeof(idx_prob) * (size_t)n);
    for (int i = 0; i < n; ++i)
        scaled[i] = (temperature != 1.0f && temperature > 0.0f) ? logits[i] / temperature : logits[i];
    float max_val = -INFINITY;
    for (int i = 0; i < n; ++i) max_val = fmaxf(max_val, scaled[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; ++i) {
        probs[i] = expf(scaled[i] - max_val);
        sum += probs[i];
    }
    for (int i = 0; i < n; ++i) probs[i] = probs[i] / sum;
    for (int i = 0; i < n; ++i) ip[i] = (idx_prob){i, probs[i]};
    stable_sort_desc(ip, n, tmp);
    float cumsum = 0.0f;
    int cutoff = n;
    for (int i = 0; i < n; ++i) {
        cumsum += ip[i].p;
        if (cumsum >= top_p) {
            cutoff = i + 1;
            break;
        }
    }
    float selected_sum = 0.0f;
    for (int i = 0; i < cutoff; ++i) selected_sum += ip[i].p;
    const float r = or_sample_threshold(seed);
    uint32_t result = n > 0 ? (uint32_t)ip[0].idx : 0;
    if (top_p >= 1.0f) {
        float c = 0.0f;
        for (int i = 0; i < n; ++i) {
            c += probs[i];
            if (r < c) {
                result = (uint32_t)i;
                goto done;
            }
        }
        goto done;
    }
    {
        float c = 0.0f;
        for (int i = 0; i < cutoff; ++i) {
            c += ip[i].p / selected_sum;
            if (r < c) {
                result = (uint32_t)ip[i].idx;
                goto done;
            }
        }
    }
done:
    free(scaled);
    free(probs);
    free(ip);
    free(tmp);
    return result;
}

typedef struct {
    int idx;
    double p;
} idx_prob64;

static void stable_sort_desc64(idx_prob64* v, int n, idx_prob64* tmp) {
    for (int width = 1; width < n; width *= 2) {
        for (int lo = 0; lo < n; lo += 2 * width) {
            int mid = lo + width < n ? lo + width : n;
            int hi = lo + 2 * width < n ? lo + 2 * width : n;
            int i = lo, j = mid, k = lo;
            while (i < mid && j < hi) tmp[k++] = (v[j].p > v[i].p) ? v[j++] : v[i++];
            while (i < mid) tmp[k++] = v[i++];
            while (j < hi) tmp[k++] = v[j++];
        }
        memcpy(v, tmp, sizeof(idx_prob64) * (size_t)n);
    }
}

/* runtime.rs:534-601 (sample_tokens_device_with_seeds), the batched decode
 * path's sampler (backend.rs:275-316), for one row: temperature scaling as
 * affine(1 / T) (f32(x * f32(1 / T)), 555-563), softmax, then
 * top_p >= 1: the first index whose cumulative probability reaches tau;
 * top_p < 1: probabilities sorted descending (ties in index order), kept
 * while the cumulative sum before them is below top_p (apply_top_p_device,
 * 461-482), renormalised, first crossing of tau in sorted order.  No
 * crossing: position 0 (argmax of an all-zero mask, 517-518).  tau = the
 * SplitMix64 threshold of the seed (483-497).  temperature <= 0 or
 * top_p <= 0: argmax, first index on ties.
 * The reference leaves the reduction orders of its softmax sum and cumsums to
 * the candle kernels, so no f32 evaluation order is the reference's: the
 * softmax and the cumulative sums are evaluated here in f64 on the f32 scaled
 * logits (accurate to ~1e-12 at 128k columns, where a sequential f32 cumsum
 * drifts by ~1e-4), and *margin receives the f64 distance from tau and top_p
 * to the nearest cumulative boundary the decision depends on (0 when the
 * sampled element has an unequal near-tie, below).  An f32 evaluation in any
 * order returns this token whenever its rounding error stays below that
 * margin. */
uint32_t or_sample_token_device(const float* logits, int n, float temperature, float top_p, uint64_t seed,
                                double* margin) {
    if (margin) *margin = INFINITY;
    if (temperature <= 0.0f || top_p <= 0.0f) return or_sample_greedy(logits, n);
    const float mul = 1.0f / temperature;
    double* probs = (double*)malloc(sizeof(double) * (size_t)n);
    float max_val = -INFINITY;
    for (int i = 0; i < n; ++i) {
        const float x = temperature == 1.0f ? logits[i] : logits[i] * mul;
        probs[i] = x;
        max_val = fmaxf(max_val, x);
    }
    double sum = 0.0;
    for (int i = 0; i < n; ++i) {
        probs[i] = exp(probs[i] - (double)max_val);
        sum += probs[i];
    }
    for (int i = 0; i < n; ++i) probs[i] /= sum;
    const double tau = (double)or_sample_threshold(seed);
    uint32_t result = 0;
    if (top_p >= 1.0f) {
        double c = 0.0, best = INFINITY;
        int found = 0;
        for (int i = 0; i < n; ++i) {
            c += probs[i];
            if (fabs(c - tau) < best) best = fabs(c - tau);
            if (!found && c >= tau) {
                result = (uint32_t)i;
                found = 1;
            }
        }
        if (margin) *margin = best;
        free(probs);
        return result;
    }
    idx_prob64* ip = (idx_prob64*)malloc(sizeof(idx_prob64) * (size_t)n);
    idx_prob64* tmp = (idx_prob64*)malloc(sizeof(idx_prob64) * (size_t)n);
    for (int i = 0; i < n; ++i) ip[i] = (idx_prob64){i, probs[i]};
    stable_sort_desc64(ip, n, tmp);
    /* keep sorted position j while the sum before it is below top_p */
    double before = 0.0, denom = 0.0, mp = INFINITY;
    int kept = 0;
    for (int j = 0; j < n; ++j) {
        if (fabs(before - (double)top_p) < mp) mp = fabs(before - (double)top_p);
        if (before < (double)top_p) {
            kept = j + 1;
            denom += ip[j].p;
        }
        before += ip[j].p;
    }
    double c = 0.0, mt = INFINITY;
    int found = 0, jr = 0;
    for (int j = 0; j < kept; ++j) {
        c += ip[j].p;
        if (fabs(c / denom - tau) < mt) mt = fabs(c / denom - tau);
        if (!found && c / denom >= tau) {
            jr = j;
            found = 1;
        }
    }
    result = (uint32_t)ip[jr].idx;
    /* The sampled element's identity: an element whose probability lies within
     * an f32 evaluation's relative error of it (expf, the division, and the
     * rounding of y - max, ~1.2e-7 per unit of |y - max|) may sort on either
     * side of it there, and then sits at the crossing instead.  Equal scaled
     * logits give equal probabilities in every evaluation (ties in column
     * order), so only unequal near-ties make the token ambiguous: margin 0. */
    {
        const int id = ip[jr].idx;
        const float yj = temperature == 1.0f ? logits[id] : logits[id] * mul;
        const double pj = ip[jr].p, tol = 1e-6 * (1.0 + fabs((double)yj - (double)max_val)) * pj;
        for (int q = jr - 1; q >= 0 && ip[q].p - pj <= tol; --q)
            if (ip[q].p != pj) mt = 0.0;
        for (int q = jr + 1; q < n && pj - ip[q].p <= tol; ++q)
            if (ip[q].p != pj) mt = 0.0;
    }
    if (margin) *margin = mp < mt ? mp : mt;
    free(probs);
    free(ip);
    free(tmp);
    return result;
}

/* forward_pass.rs:1317-1372 */
int or_causal_attention_with_prefix(const float* q, const float* k, const float* v, float* out,
                                    int q_rows, int kv_rows, int d, float scale, int prefix_len) {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(kv_rows > 0 ? kv_rows : 1));
    for (int r = 0; r < q_rows; ++r) {
        const int max_k = prefix_len + r + 1;
        if (max_k > kv_rows) {
            free(scores);
            return fail("Attention prefix exceeds cached sequence: prefix %d query_row %d cache_rows %d",
                        prefix_len, r, kv_rows);
        }
        const float* qs = q + (size_t)r * d;
        float max_score = -INFINITY;
        for (int t = 0; t < max_k; ++t) {
            const float* ks = k + (size_t)t * d;
            float dot = 0.0f;
            for (int i = 0; i < d; ++i) dot += qs[i] * ks[i];
            const float s = dot * scale;
            max_score = fmaxf(max_score, s);
            scores[t] = s;
        }
        float exp_sum = 0.0f;
        for (int t = 0; t < max_k; ++t) {
            scores[t] = expf(scores[t] - max_score);
            exp_sum += scores[t];
        }
        float* o = out + (size_t)r * d;
        for (int i = 0; i < d; ++i) o[i] = 0.0f;
        for (int t = 0; t < max_k; ++t) {
            const float w = scores[t] / exp_sum;
            const float* vs = v + (size_t)t * d;
            for (int i = 0; i < d; ++i) o[i] += w * vs[i];
        }
    }
    free(scores);
    return 0;
}

uint16_t or_f32_to_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void or_round_bf16_inplace(float* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = or_bf16_to_f32(or_f32_to_bf16(x[i]));
}

/* ================================================== shard geometry ====== */

/* forward_pass.rs:1257-1315 and build_local_kv_head_indices 2951-2970 */
int or_resolve_shard_layout(int hidden, int num_heads, int num_kv_heads, int shard_start,
                            int shard_end, or_shard_layout* out, uint32_t* local_kv_head_indices) {
    if (num_heads <= 0 || hidden % num_heads != 0)
        return fail("Unsupported attention geometry: hidden_dim %d num_heads %d", hidden, num_heads);
    if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
        return fail("Unsupported grouped-query attention geometry: num_heads %d num_kv_heads %d",
                    num_heads, num_kv_heads);
    if (shard_start >= shard_end || shard_end > hidden)
        return fail("Invalid shard range %d..%d for hidden_dim %d", shard_start, shard_end, hidden);
    const int head_dim = hidden / num_heads;
    const int qpk = num_heads / num_kv_heads;
    const int group = qpk * head_dim;
    if (hidden % group != 0)
        return fail("Hidden dim %d is not divisible by grouped-query shard width %d", hidden, group);
    if (shard_start % group != 0 || shard_end % group != 0)
        return fail("Shard range %d..%d is not aligned to grouped-query shard width %d", shard_start,
                    shard_end, group);
    or_shard_layout l;
    l.head_dim = head_dim;
    l.q_heads_per_kv_head = qpk;
    l.q_cols = shard_end - shard_start;
    const int groups = l.q_cols / group;
    l.local_q_heads = groups * qpk;
    l.q_head_start = shard_start / head_dim;
    l.kv_head_start = shard_start / group;
    l.local_kv_heads = groups;
    l.kv_cols = groups * head_dim;
    if (local_kv_head_indices) {
        for (int i = 0; i < l.local_q_heads; ++i) {
            const int gq = l.q_head_start + i;
            const int gk = gq / qpk;
            if (gk < l.kv_head_start || gk >= l.kv_head_start + l.local_kv_heads)
                return fail("Local KV head ownership mismatch: q_head %d maps to kv_head %d", gq, gk);
            local_kv_head_indices[i] = (uint32_t)(gk - l.kv_head_start);
        }
    }
    if (out) *out = l;
    return 0;
}

/* artifact_loader.rs:351-366 */
int or_partition_columns(int total_columns, int worker_position, int total_workers) {
    if (total_workers == 0) return total_columns;
    const int per = total_columns / total_workers, rem = total_columns % total_workers;
    return worker_position < rem ? per + 1 : per;
}

/* ============================================ paged KV session ========== */

typedef struct {
    int page_index, start_row, row_count;
} span_t;

typedef struct {
    float* keys;   /* [page_rows, cols] */
    float* values; /* [page_rows, cols] */
    int used_rows;
    int active;
} page_t;

typedef struct {
    page_t* pages;
    int n_pages, cap_pages;
    int* free_pages;
    int n_free, cap_free;
    span_t* spans;
    int n_spans, cap_spans;
    int seq_len;
} layer_t;

struct or_session {
    int num_layers, cols, page_rows, max_seq_len, kv_round_bf16;
    layer_t* layers;
    int base_position;
    int position;
};

#define GROW(ptr, n, cap, type)                                            \
    do {                                                                   \
        if ((n) >= (cap)) {                                                \
            (cap) = (cap) ? (cap) * 2 : 8;                                 \
            (ptr) = (type*)realloc((ptr), sizeof(type) * (size_t)(cap));   \
        }                                                                  \
    } while (0)

or_session* or_session_new(int num_layers, int kv_cols, int page_rows, int max_seq_len,
                           int kv_round_bf16) {
    if (num_layers <= 0 || kv_cols <= 0 || page_rows <= 0) {
        fail("invalid session geometry");
        return NULL;
    }
    or_session* s = (or_session*)calloc(1, sizeof(or_session));
    s->num_layers = num_layers;
    s->cols = kv_cols;
    s->page_rows = page_rows;
    s->max_seq_len = max_seq_len;
    s->kv_round_bf16 = kv_round_bf16;
    s->layers = (layer_t*)calloc((size_t)num_layers, sizeof(layer_t));
    return s;
}

void or_session_free(or_session* s) {
    if (!s) return;
    for (int l = 0; l < s->num_layers; ++l) {
        layer_t* L = &s->layers[l];
        for (int p = 0; p < L->n_pages; ++p) {
            free(L->pages[p].keys);
            free(L->pages[p].values);
        }
        free(L->pages);
        free(L->free_pages);
        free(L->spans);
    }
    free(s->layers);
    free(s);
}

/* allocate_page (forward_pass.rs:396-424): pop the LIFO free list, else grow. */
static int layer_allocate_page(or_session* s, layer_t* L) {
    if (L->n_free > 0) {
        const int idx = L->free_pages[--L->n_free];
        if (idx < 0 || idx >= L->n_pages) return fail("Invalid free device KV page index %d", idx);
        if (L->pages[idx].active)
            return fail("Device KV allocator attempted to reuse page %d while it was Active", idx);
        L->pages[idx].used_rows = 0;
        L->pages[idx].active = 1;
        return idx;
    }
    GROW(L->pages, L->n_pages, L->cap_pages, page_t);
    page_t* p = &L->pages[L->n_pages];
    const size_t n = (size_t)s->page_rows * (size_t)s->cols;
    p->keys = (float*)calloc(n, sizeof(float));
    p->values = (float*)calloc(n, sizeof(float));
    p->used_rows = 0;
    p->active = 1;
    return L->n_pages++;
}

/* release_page (426-446) */
static int layer_release_page(layer_t* L, int idx) {
    if (idx < 0 || idx >= L->n_pages) return fail("Invalid device KV page index %d", idx);
    if (!L->pages[idx].active) return fail("Device KV allocator double-freed page %d", idx);
    L->pages[idx].used_rows = 0;
    L->pages[idx].active = 0;
    GROW(L->free_pages, L->n_free, L->cap_free, int);
    L->free_pages[L->n_free++] = idx;
    return 0;
}

/* reclaim_unused_pages (448-460) */
static int layer_reclaim(layer_t* L) {
    for (int p = 0; p < L->n_pages; ++p) {
        int referenced = 0;
        for (int i = 0; i < L->n_spans; ++i)
            if (L->spans[i].page_index == p) {
                referenced = 1;
                break;
            }
        if (!referenced && L->pages[p].used_rows != 0)
            if (layer_release_page(L, p) < 0) return -1;
    }
    return 0;
}

/* ensure_writable_tail (353-394) */
static int layer_ensure_writable_tail(or_session* s, layer_t* L) {
    if (L->n_spans == 0) {
        const int idx = layer_allocate_page(s, L);
        if (idx < 0) return idx;
        GROW(L->spans, L->n_spans, L->cap_spans, span_t);
        L->spans[L->n_spans++] = (span_t){idx, 0, 0};
        return idx;
    }
    const span_t tail = L->spans[L->n_spans - 1];
    if (tail.page_index < 0 || tail.page_index >= L->n_pages)
        return fail("Invalid device KV page index %d", tail.page_index);
    const page_t* tp = &L->pages[tail.page_index];
    if (tail.start_row + tail.row_count != tp->used_rows)
        return fail("Device KV tail span for page %d is inconsistent: span end %d vs used_rows %d",
                    tail.page_index, tail.start_row + tail.row_count, tp->used_rows);
    if (s->page_rows - tp->used_rows > 0) return tail.page_index;
    const int idx = layer_allocate_page(s, L);
    if (idx < 0) return idx;
    GROW(L->spans, L->n_spans, L->cap_spans, span_t);
    L->spans[L->n_spans++] = (span_t){idx, 0, 0};
    return idx;
}

/* DeviceLayerKVCache::append (462-521) */
static int layer_append(or_session* s, layer_t* L, const float* k, const float* v, int rows) {
    int appended = 0;
    const int cols = s->cols;
    while (appended < rows) {
        const int idx = layer_ensure_writable_tail(s, L);
        if (idx < 0) return idx;
        page_t* p = &L->pages[idx];
        int copy_rows = s->page_rows - p->used_rows;
        if (copy_rows > rows - appended) copy_rows = rows - appended;
        for (int r = 0; r < copy_rows; ++r) {
            float* kd = p->keys + (size_t)(p->used_rows + r) * cols;
            float* vd = p->values + (size_t)(p->used_rows + r) * cols;
            memcpy(kd, k + (size_t)(appended + r) * cols, sizeof(float) * (size_t)cols);
            memcpy(vd, v + (size_t)(appended + r) * cols, sizeof(float) * (size_t)cols);
            if (s->kv_round_bf16) {
                or_round_bf16_inplace(kd, cols);
                or_round_bf16_inplace(vd, cols);
            }
        }
        p->used_rows += copy_rows;
        span_t* tail = &L->spans[L->n_spans - 1];
        if (tail->page_index != idx)
            return fail("Device KV tail span/page mismatch: span page %d vs active page %d",
                        tail->page_index, idx);
        tail->row_count += copy_rows;
        appended += copy_rows;
        L->seq_len += copy_rows;
    }
    return 0;
}

/* DeviceLayerKVCache::clear (840-850): the free list is re-seeded 0..n, so the
 * next allocation pops the highest page index. */
static void layer_clear(layer_t* L) {
    for (int p = 0; p < L->n_pages; ++p) {
        L->pages[p].used_rows = 0;
        L->pages[p].active = 0;
    }
    L->n_free = 0;
    for (int p = 0; p < L->n_pages; ++p) {
        GROW(L->free_pages, L->n_free, L->cap_free, int);
        L->free_pages[L->n_free++] = p;
    }
    L->n_spans = 0;
    L->seq_len = 0;
}

/* DeviceLayerKVCache::retain_suffix (852-881) */
static int layer_retain_suffix(layer_t* L, int keep) {
    if (L->seq_len <= keep) return 0;
    if (keep == 0) {
        layer_clear(L);
        return 0;
    }
    int drop = L->seq_len - keep;
    while (drop > 0) {
        if (L->n_spans == 0) return fail("Device KV block table unexpectedly empty");
        span_t* front = &L->spans[0];
        if (drop >= front->row_count) {
            drop -= front->row_count;
            const int idx = front->page_index;
            memmove(L->spans, L->spans + 1, sizeof(span_t) * (size_t)(L->n_spans - 1));
            L->n_spans--;
            if (layer_release_page(L, idx) < 0) return -1;
            continue;
        }
        front->start_row += drop;
        front->row_count -= drop;
        drop = 0;
    }
    L->seq_len = keep;
    return layer_reclaim(L);
}

static int session_seq_len0(const or_session* s) { return s->layers[0].seq_len; }

/* DeviceKVCache::retain_suffix (1084-1094) */
int or_session_retain_suffix(or_session* s, int keep_rows) {
    const int seq_len = session_seq_len0(s);
    if (keep_rows < 0) keep_rows = 0;
    if (seq_len <= keep_rows) return 0;
    for (int l = 0; l < s->num_layers; ++l)
        if (layer_retain_suffix(&s->layers[l], keep_rows) < 0) return -1;
    s->base_position += seq_len - keep_rows;
    return 0;
}

/* DeviceKVCache::clear (1076-1082) */
void or_session_clear(or_session* s) {
    for (int l = 0; l < s->num_layers; ++l) layer_clear(&s->layers[l]);
    s->base_position = 0;
}

/* DeviceKVCache::append_layer (920-957) */
int or_session_append_layer(or_session* s, int layer, const float* k, const float* v, int rows) {
    if (layer < 0 || layer >= s->num_layers) return fail("Invalid layer index: %d", layer);
    if (rows <= 0) return fail("Device KV append received an empty key shape");
    const int max_seq = s->max_seq_len > 1 ? s->max_seq_len : 1;
    if (rows > max_seq) {
        const int start = rows - max_seq;
        k += (size_t)start * s->cols;
        v += (size_t)start * s->cols;
        rows = max_seq;
    }
    const int cur = s->layers[layer].seq_len;
    if (cur + rows > max_seq) {
        const int drop = cur + rows - max_seq;
        const int keep = cur - drop > 0 ? cur - drop : 0;
        if (or_session_retain_suffix(s, keep) < 0) return -1;
    }
    return layer_append(s, &s->layers[layer], k, v, rows);
}

int or_session_seq_len(const or_session* s, int layer) {
    if (layer < 0 || layer >= s->num_layers) return fail("Invalid layer index: %d", layer);
    return s->layers[layer].seq_len;
}
int or_session_base_position(const or_session* s) { return s->base_position; }
int or_session_position(const or_session* s) { return s->position; }
void or_session_set_position(or_session* s, int position) { s->position = position; }
int or_session_allocated_pages(const or_session* s, int layer) {
    if (layer < 0 || layer >= s->num_layers) return fail("Invalid layer index: %d", layer);
    return s->layers[layer].n_pages;
}

/* DeviceLayerKVCache::live_block_table (682-721) with the LiveKVBlockTable
 * contract checks of kv_cache.rs:372-415 and the cross-layer equality check of
 * DeviceKVCache::live_block_table (1024-1048). */
int or_session_block_table(const or_session* s, int layer, uint32_t* page_ids, int* start_tokens,
                           int* token_counts, int max_spans) {
    if (layer < 0 || layer >= s->num_layers) return fail("Invalid layer index: %d", layer);
    const layer_t* L = &s->layers[layer];
    int total = 0;
    for (int i = 0; i < L->n_spans; ++i) {
        const span_t sp = L->spans[i];
        if (sp.row_count == 0) return fail("Live KV block table span %d is empty", i);
        if (sp.start_row >= s->page_rows)
            return fail("Live KV block table span %d starts outside page bounds", i);
        if (sp.start_row + sp.row_count > s->page_rows)
            return fail("Live KV block table span %d exceeds page bounds", i);
        if (!L->pages[sp.page_index].active)
            return fail("Device KV block table span %d references non-active page %d", i,
                        sp.page_index);
        if (sp.start_row + sp.row_count > L->pages[sp.page_index].used_rows)
            return fail("Device KV block table span %d exceeds page %d used rows", i, sp.page_index);
        total += sp.row_count;
    }
    if (total != L->seq_len)
        return fail("Live KV block table token mismatch: spans cover %d, cached_tokens says %d",
                    total, L->seq_len);
    const layer_t* L0 = &s->layers[0];
    if (L0->n_spans != L->n_spans || L0->seq_len != L->seq_len)
        return fail("Device KV layer %d diverged from layer 0", layer);
    for (int i = 0; i < L->n_spans; ++i)
        if (memcmp(&L0->spans[i], &L->spans[i], sizeof(span_t)) != 0)
            return fail("Device KV layer %d block table diverged from canonical layer 0 layout", layer);
    if (page_ids || start_tokens || token_counts) {
        if (L->n_spans > max_spans) return fail("block table has %d spans > %d", L->n_spans, max_spans);
        for (int i = 0; i < L->n_spans; ++i) {
            if (page_ids) page_ids[i] = (uint32_t)L->spans[i].page_index;
            if (start_tokens) start_tokens[i] = L->spans[i].start_row;
            if (token_counts) token_counts[i] = L->spans[i].row_count;
        }
    }
    return L->n_spans;
}

/* build_active_tensors (633-680) */
int or_session_gather(const or_session* s, int layer, float* k_out, float* v_out) {
    if (layer < 0 || layer >= s->num_layers) return fail("Invalid layer index: %d", layer);
    const layer_t* L = &s->layers[layer];
    if (L->seq_len == 0 || L->n_spans == 0)
        return fail("Requested device KV state before cache initialization");
    int row = 0;
    const int cols = s->cols;
    for (int i = 0; i < L->n_spans; ++i) {
        const span_t sp = L->spans[i];
        const page_t* p = &L->pages[sp.page_index];
        const size_t n = (size_t)sp.row_count * cols;
        if (k_out) memcpy(k_out + (size_t)row * cols, p->keys + (size_t)sp.start_row * cols, n * 4);
        if (v_out) memcpy(v_out + (size_t)row * cols, p->values + (size_t)sp.start_row * cols, n * 4);
        row += sp.row_count;
    }
    return row;
}

/* export_snapshot (1169-1204).  The host KVCache then applies
 * retain_suffix(max(limit, 1)) (kv_cache.rs:847-868): keep the newest rows,
 * advance the base position by the dropped count. */
int or_session_export(const or_session* s, int max_cached_tokens, float* k_out, float* v_out,
                      int* out_base_position, int* out_next_position) {
    const int seq_len = session_seq_len0(s);
    const int next = s->base_position + seq_len;
    if (out_next_position) *out_next_position = next;
    if (seq_len == 0) {
        if (out_base_position) *out_base_position = s->base_position;
        return 0;
    }
    int keep = seq_len;
    if (max_cached_tokens >= 0) {
        const int limit = max_cached_tokens > 1 ? max_cached_tokens : 1;
        if (keep > limit) keep = limit;
    }
    const int drop = seq_len - keep;
    float* tk = (float*)malloc(sizeof(float) * (size_t)seq_len * s->cols);
    float* tv = (float*)malloc(sizeof(float) * (size_t)seq_len * s->cols);
    for (int l = 0; l < s->num_layers; ++l) {
        if (or_session_gather(s, l, tk, tv) < 0) {
            free(tk);
            free(tv);
            return -1;
        }
        const size_t n = (size_t)keep * s->cols;
        memcpy(k_out + (size_t)l * n, tk + (size_t)drop * s->cols, n * 4);
        memcpy(v_out + (size_t)l * n, tv + (size_t)drop * s->cols, n * 4);
    }
    free(tk);
    free(tv);
    if (out_base_position) *out_base_position = s->base_position + drop;
    return keep;
}

/* import_snapshot (1206-1242) and ForwardPass::import_kv_cache_snapshot
 * (2450-2454). */
int or_session_import(or_session* s, const float* k, const float* v, int rows, int base_position,
                      int next_position) {
    if (rows > next_position) return fail("KV sequence state is invalid: cached_tokens %d exceeds next_position %d", rows, next_position);
    if (base_position != next_position - rows)
        return fail("KV snapshot base position mismatch: payload starts at %d, sequence metadata says %d",
                    base_position, next_position - rows);
    or_session_clear(s);
    s->base_position = base_position;
    if (rows > 0)
        for (int l = 0; l < s->num_layers; ++l) {
            const size_t n = (size_t)rows * s->cols;
            if (or_session_append_layer(s, l, k + (size_t)l * n, v + (size_t)l * n, rows) < 0)
                return -1;
        }
    if (session_seq_len0(s) != rows)
        return fail("Recovered device KV cache length %d does not match snapshot cached token count %d",
                    session_seq_len0(s), rows);
    if (s->base_position != next_position - rows)
        return fail("Recovered device KV cache base position mismatch");
    s->position = next_position;
    return 0;
}

/* =========================================================== model ====== */

/* A weight matrix [in, out] held as f32 values or as bf16 bit patterns.
 * bf16 -> f32 is exact, so both forms give bit-identical products. */
typedef struct {
    const float* f;
    const uint16_t* h;
} wmat;

typedef struct {
    wmat w_q, w_k, w_v, w_o, w_gate, w_up, w_down;
    const float *attn_norm, *mlp_norm;
} layer_w;

struct or_model {
    or_model_config cfg;
    or_shard_layout lay;
    uint32_t* kv_idx;
    wmat embedding, lm_head;
    const float* final_norm;
    layer_w* layers;
};

/* or_matmul with b as bf16 bit patterns: the same loop order and the same f32
 * products (the upcast is exact), so the result is bit-identical to
 * or_matmul on the f32 values of b. */
int or_matmul_bf16w(const float* a, const uint16_t* b, float* c, int m, int k, int n) {
    if (m < 0 || k < 0 || n < 0) return fail("Matmul shape mismatch: %dx%d @ %dx%d", m, k, k, n);
    memset(c, 0, sizeof(float) * (size_t)m * (size_t)n);
    const int ib = 16, jb = 256;
    const int nib = (m + ib - 1) / ib, njb = (n + jb - 1) / jb;
#pragma omp parallel for collapse(2) schedule(static)
    for (int it = 0; it < nib; ++it) {
        for (int blk = 0; blk < njb; ++blk) {
            const int i0 = it * ib, i1 = i0 + ib < m ? i0 + ib : m;
            const int j0 = blk * jb, j1 = j0 + jb < n ? j0 + jb : n;
            float bf[256];
            for (int kk = 0; kk < k; ++kk) {
                const uint16_t* b_row = b + (size_t)kk * n;
                for (int j = j0; j < j1; ++j) bf[j - j0] = or_bf16_to_f32(b_row[j]);
                for (int i = i0; i < i1; ++i) {
                    const float a_ik = a[(size_t)i * k + kk];
                    float* out_row = c + (size_t)i * n;
                    for (int j = j0; j < j1; ++j) out_row[j] += a_ik * bf[j - j0];
                }
            }
        }
    }
    return 0;
}



or_model* or_model_new(const or_model_config* cfg) {
    or_shard_layout lay;
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(cfg->num_heads > 0 ? cfg->num_heads : 1));
    if (or_resolve_shard_layout(cfg->hidden, cfg->num_heads, cfg->num_kv_heads, cfg->shard_start,
                                cfg->shard_end, &lay, idx) < 0) {
        free(idx);
        return NULL;
    }
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->cfg = *cfg;
    m->lay = lay;
    m->kv_idx = idx;
    m->layers = (layer_w*)calloc((size_t)cfg->num_layers, sizeof(layer_w));
    return m;
}

void or_model_free(or_model* m) {
    if (!m) return;
    free(m->kv_idx);
    free(m->layers);
    free(m);
}

static int mm(const float* a, wmat b, float* c, int rows, int k, int n) {
    return b.h ? or_matmul_bf16w(a, b.h, c, rows, k, n) : or_matmul(a, b.f, c, rows, k, n);
}

int or_model_set_globals(or_model* m, const float* embedding, const float* final_norm,
                         const float* lm_head) {
    m->embedding = (wmat){embedding, NULL};
    m->final_norm = final_norm;
    m->lm_head = (wmat){lm_head, NULL};
    return 0;
}

int or_model_set_globals_bf16(or_model* m, const uint16_t* embedding, const float* final_norm,
                              const uint16_t* lm_head) {
    m->embedding = (wmat){NULL, embedding};
    m->final_norm = final_norm;
    m->lm_head = (wmat){NULL, lm_head};
    return 0;
}

int or_model_set_layer(or_model* m, int layer, const float* w_q, const float* w_k,
                       const float* w_v, const float* w_o, const float* w_gate, const float* w_up,
                       const float* w_down, const float* attn_norm, const float* mlp_norm) {
    if (layer < 0 || layer >= m->cfg.num_layers) return fail("Invalid layer index: %d", layer);
    m->layers[layer] = (layer_w){{w_q, NULL}, {w_k, NULL}, {w_v, NULL}, {w_o, NULL}, {w_gate, NULL},
                                 {w_up, NULL}, {w_down, NULL}, attn_norm, mlp_norm};
    return 0;
}

int or_model_set_layer_bf16(or_model* m, int layer, const uint16_t* w_q, const uint16_t* w_k,
                            const uint16_t* w_v, const uint16_t* w_o, const uint16_t* w_gate,
                            const uint16_t* w_up, const uint16_t* w_down, const float* attn_norm,
                            const float* mlp_norm) {
    if (layer < 0 || layer >= m->cfg.num_layers) return fail("Invalid layer index: %d", layer);
    m->layers[layer] = (layer_w){{NULL, w_q}, {NULL, w_k}, {NULL, w_v}, {NULL, w_o}, {NULL, w_gate},
                                 {NULL, w_up}, {NULL, w_down}, attn_norm, mlp_norm};
    return 0;
}

/* tensor_ops.rs:482-500 */
static int embed(const or_model* m, const uint32_t* tokens, int n, float* out) {
    const int H = m->cfg.hidden;
    for (int i = 0; i < n; ++i) {
        if ((int)tokens[i] >= m->cfg.vocab || (int)tokens[i] < 0)
            return fail("Token %u out of vocabulary bounds %d", tokens[i], m->cfg.vocab);
        float* dst = out + (size_t)i * H;
        if (m->embedding.h) {
            const uint16_t* src = m->embedding.h + (size_t)tokens[i] * H;
            for (int j = 0; j < H; ++j) dst[j] = or_bf16_to_f32(src[j]);
        } else {
            memcpy(dst, m->embedding.f + (size_t)tokens[i] * H, sizeof(float) * (size_t)H);
        }
    }
    return 0;
}

/* Attention for one session over its cached rows after appending `rows` new
 * rows at cache_prefix_len (forward_pass.rs:1410-1499 host text; the device
 * single-query path 2838-2895 is the rows == 1 case).  q_rope [rows, q_cols]
 * (row stride q_stride), out [rows, q_cols]. */
static int session_attention(const or_model* m, or_session* s, int layer, const float* q_rope,
                             int q_stride, int rows, int prefix, float* out) {
    const or_shard_layout* lay = &m->lay;
    const int d = lay->head_dim, kvc = lay->kv_cols;
    const int seq = s->layers[layer].seq_len;
    float* K = (float*)malloc(sizeof(float) * (size_t)seq * kvc);
    float* V = (float*)malloc(sizeof(float) * (size_t)seq * kvc);
    float* kh = (float*)malloc(sizeof(float) * (size_t)seq * d);
    float* vh = (float*)malloc(sizeof(float) * (size_t)seq * d);
    float* qh = (float*)malloc(sizeof(float) * (size_t)rows * d);
    float* oh = (float*)malloc(sizeof(float) * (size_t)rows * d);
    int rc = or_session_gather(s, layer, K, V);
    const float scale = 1.0f / sqrtf((float)d);
    for (int h = 0; rc >= 0 && h < lay->local_q_heads; ++h) {
        const int kvh = (int)m->kv_idx[h];
        for (int t = 0; t < seq; ++t) {
            memcpy(kh + (size_t)t * d, K + (size_t)t * kvc + (size_t)kvh * d, sizeof(float) * d);
            memcpy(vh + (size_t)t * d, V + (size_t)t * kvc + (size_t)kvh * d, sizeof(float) * d);
        }
        for (int r = 0; r < rows; ++r)
            memcpy(qh + (size_t)r * d, q_rope + (size_t)r * q_stride + (size_t)h * d, sizeof(float) * d);
        rc = or_causal_attention_with_prefix(qh, kh, vh, oh, rows, seq, d, scale, prefix);
        for (int r = 0; rc >= 0 && r < rows; ++r)
            memcpy(out + (size_t)r * lay->q_cols + (size_t)h * d, oh + (size_t)r * d, sizeof(float) * d);
    }
    free(K);
    free(V);
    free(kh);
    free(vh);
    free(qh);
    free(oh);
    return rc < 0 ? -1 : 0;
}

typedef struct {
    float *normed, *q, *k, *v, *qr, *kr, *attn, *o, *gate, *up, *mlp, *down;
} scratch_t;

static void scratch_alloc(scratch_t* w, const or_model* m, int rows) {
    const size_t H = (size_t)m->cfg.hidden, Q = (size_t)m->lay.q_cols, KV = (size_t)m->lay.kv_cols;
    const size_t F = (size_t)m->cfg.ffn_cols, R = (size_t)rows;
    w->normed = (float*)malloc(4 * R * H);
    w->q = (float*)malloc(4 * R * Q);
    w->k = (float*)malloc(4 * R * KV);
    w->v = (float*)malloc(4 * R * KV);
    w->qr = (float*)malloc(4 * R * Q);
    w->kr = (float*)malloc(4 * R * KV);
    w->attn = (float*)malloc(4 * R * Q);
    w->o = (float*)malloc(4 * R * H);
    w->gate = (float*)malloc(4 * R * F);
    w->up = (float*)malloc(4 * R * F);
    w->mlp = (float*)malloc(4 * R * F);
    w->down = (float*)malloc(4 * R * H);
}

static void scratch_free(scratch_t* w) {
    free(w->normed); free(w->q); free(w->k); free(w->v); free(w->qr); free(w->kr);
    free(w->attn); free(w->o); free(w->gate); free(w->up); free(w->mlp); free(w->down);
}

/* MLP half of a layer (forward_pass.rs:2279-2307): post_attn = hidden + o;
 * hidden = post_attn + down(silu(gate) * up). */
static int mlp_block(const or_model* m, const layer_w* Lw, float* hidden, scratch_t* w, int rows,
                     float* part_o, float* part_down) {
    const int H = m->cfg.hidden, F = m->cfg.ffn_cols;
    const size_t RH = (size_t)rows * H;
    if (part_o) memcpy(part_o, w->o, 4 * RH);
    for (size_t i = 0; i < RH; ++i) hidden[i] = hidden[i] + w->o[i];
    if (or_rms_norm(hidden, Lw->mlp_norm, w->normed, rows, H, m->cfg.rms_norm_eps) < 0) return -1;
    if (mm(w->normed, Lw->w_gate, w->gate, rows, H, F) < 0) return -1;
    if (mm(w->normed, Lw->w_up, w->up, rows, H, F) < 0) return -1;
    or_silu(w->gate, w->mlp, (int64_t)rows * F);
    for (size_t i = 0; i < (size_t)rows * F; ++i) w->mlp[i] = w->mlp[i] * w->up[i];
    if (mm(w->mlp, Lw->w_down, w->down, rows, F, H) < 0) return -1;
    if (part_down) memcpy(part_down, w->down, 4 * RH);
    for (size_t i = 0; i < RH; ++i) hidden[i] = hidden[i] + w->down[i];
    return 0;
}

static int decode_microbatch(const or_model* m, or_session** sessions, int batch, const uint32_t* tokens,
                             float* logits, float* partials, const float* force_k, const float* force_v,
                             float* own_k, float* own_v);

/* ForwardPass::fast_path_decode_microbatch (2143-2319) with
 * attention_output_device_batch_from_backends (2612-2740). */
int or_decode_microbatch(const or_model* m, or_session** sessions, int batch,
                         const uint32_t* tokens, float* logits, float* partials) {
    return decode_microbatch(m, sessions, batch, tokens, logits, partials, NULL, NULL, NULL, NULL);
}

int or_decode_microbatch_forced(const or_model* m, or_session** sessions, int batch, const uint32_t* tokens,
                                float* logits, float* partials, const float* force_k, const float* force_v,
                                float* own_k, float* own_v) {
    if (!force_k || !force_v) return fail("forced decode needs the stored K and V rows");
    return decode_microbatch(m, sessions, batch, tokens, logits, partials, force_k, force_v, own_k, own_v);
}

static int decode_microbatch(const or_model* m, or_session** sessions, int batch, const uint32_t* tokens,
                             float* logits, float* partials, const float* force_k, const float* force_v,
                             float* own_k, float* own_v) {
    if (batch <= 0) return fail("Decode microbatch requires at least one backend and token");
    const int H = m->cfg.hidden, Q = m->lay.q_cols, KV = m->lay.kv_cols, d = m->lay.head_dim;
    uint32_t* positions = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)batch);
    for (int b = 0; b < batch; ++b) {
        or_session* s = sessions[b];
        if (s->position == 0) {
            free(positions);
            return fail("Decode microbatch requested before prompt prefill");
        }
        if (s->base_position + session_seq_len0(s) != s->position) {
            free(positions);
            return fail("Forward pass position %d diverged from KV cache next position %d",
                        s->position, s->base_position + session_seq_len0(s));
        }
        positions[b] = (uint32_t)s->position;
    }
    float* hidden = (float*)malloc(sizeof(float) * (size_t)batch * H);
    scratch_t w;
    scratch_alloc(&w, m, batch);
    int rc = embed(m, tokens, batch, hidden);
    for (int l = 0; rc >= 0 && l < m->cfg.num_layers; ++l) {
        const layer_w* Lw = &m->layers[l];
        rc = or_rms_norm(hidden, Lw->attn_norm, w.normed, batch, H, m->cfg.rms_norm_eps);
        if (rc >= 0) rc = mm(w.normed, Lw->w_q, w.q, batch, H, Q);
        if (rc >= 0) rc = mm(w.normed, Lw->w_k, w.k, batch, H, KV);
        if (rc >= 0) rc = mm(w.normed, Lw->w_v, w.v, batch, H, KV);
        if (rc >= 0) rc = or_apply_rope(w.q, w.qr, batch, Q, positions, d, m->cfg.rope_base);
        if (rc >= 0) rc = or_apply_rope(w.k, w.kr, batch, KV, positions, d, m->cfg.rope_base);
        /* sessions are independent: each one's trim / append / attention
         * runs in the reference's order, sessions in parallel */
        int bad = 0;
        if (rc >= 0) {
#pragma omp parallel for schedule(dynamic, 1) reduction(| : bad)
            for (int b = 0; b < batch; ++b) {
                or_session* s = sessions[b];
                int src = 0;
                const int cur = s->layers[l].seq_len;
                const int max_seq = s->max_seq_len > 1 ? s->max_seq_len : 1;
                if (cur + 1 > max_seq) {
                    const int drop = cur + 1 - max_seq;
                    src = or_session_retain_suffix(s, cur - drop > 0 ? cur - drop : 0);
                }
                const int prefix = s->layers[l].seq_len;
                if (src >= 0 && (int)positions[b] != s->base_position + prefix)
                    src = fail("Non-contiguous attention positions: expected %d, got %u",
                               s->base_position + prefix, positions[b]);
                const float* kr = w.kr + (size_t)b * KV;
                const float* vr = w.v + (size_t)b * KV;
                if (force_k) {
                    /* the row another implementation stored is appended in
                     * place of this oracle's own, which is handed back (f32,
                     * before any bf16 rounding) for the caller to judge */
                    const size_t o = ((size_t)l * batch + b) * KV;
                    if (own_k) memcpy(own_k + o, kr, sizeof(float) * (size_t)KV);
                    if (own_v) memcpy(own_v + o, vr, sizeof(float) * (size_t)KV);
                    kr = force_k + o;
                    vr = force_v + o;
                }
                if (src >= 0) src = or_session_append_layer(s, l, kr, vr, 1);
                if (src >= 0)
                    src = session_attention(m, s, l, w.qr + (size_t)b * Q, Q, 1, prefix,
                                            w.attn + (size_t)b * Q);
                if (src < 0) bad |= 1;
            }
        }
        if (bad) rc = -1;
        if (rc >= 0) rc = mm(w.attn, Lw->w_o, w.o, batch, Q, H);
        if (rc >= 0) {
            float* po = partials ? partials + ((size_t)l * 2 + 0) * (size_t)batch * H : NULL;
            float* pd = partials ? partials + ((size_t)l * 2 + 1) * (size_t)batch * H : NULL;
            rc = mlp_block(m, Lw, hidden, &w, batch, po, pd);
        }
    }
    if (rc >= 0) rc = or_rms_norm(hidden, m->final_norm, w.normed, batch, H, m->cfg.rms_norm_eps);
    if (rc >= 0 && logits) rc = mm(w.normed, m->lm_head, logits, batch, H, m->cfg.vocab);
    if (rc >= 0)
        for (int b = 0; b < batch; ++b) sessions[b]->position += 1;
    scratch_free(&w);
    free(hidden);
    free(positions);
    return rc < 0 ? -1 : 0;
}

/* forward_tokens (2456-2528) for one session starting at its next position;
 * the attention block follows the host attention_output (1410-1499): trim the
 * window for the incoming rows first, then attend with the prefix mask. */
static int forward_tokens(const or_model* m, or_session* s, const uint32_t* tokens, int n,
                          int start_pos, float* logits, float* partials) {
    const int H = m->cfg.hidden, Q = m->lay.q_cols, KV = m->lay.kv_cols, d = m->lay.head_dim;
    uint32_t* positions = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)n);
    for (int i = 0; i < n; ++i) positions[i] = (uint32_t)(start_pos + i);
    float* hidden = (float*)malloc(sizeof(float) * (size_t)n * H);
    scratch_t w;
    scratch_alloc(&w, m, n);
    int rc = embed(m, tokens, n, hidden);
    for (int l = 0; rc >= 0 && l < m->cfg.num_layers; ++l) {
        const layer_w* Lw = &m->layers[l];
        rc = or_rms_norm(hidden, Lw->attn_norm, w.normed, n, H, m->cfg.rms_norm_eps);
        if (rc >= 0) rc = mm(w.normed, Lw->w_q, w.q, n, H, Q);
        if (rc >= 0) rc = mm(w.normed, Lw->w_k, w.k, n, H, KV);
        if (rc >= 0) rc = mm(w.normed, Lw->w_v, w.v, n, H, KV);
        if (rc < 0) break;
        const int cur = s->layers[l].seq_len;
        const int max_seq = s->max_seq_len > 1 ? s->max_seq_len : 1;
        if (cur + n > max_seq) {
            const int drop = cur + n - max_seq;
            rc = or_session_retain_suffix(s, cur - drop > 0 ? cur - drop : 0);
            if (rc < 0) break;
        }
        const int prefix = s->layers[l].seq_len;
        if (start_pos != s->base_position + prefix) {
            rc = fail("Non-contiguous attention positions: expected %d, got %d",
                      s->base_position + prefix, start_pos);
            break;
        }
        rc = or_apply_rope(w.q, w.qr, n, Q, positions, d, m->cfg.rope_base);
        if (rc >= 0) rc = or_apply_rope(w.k, w.kr, n, KV, positions, d, m->cfg.rope_base);
        if (rc >= 0) rc = or_session_append_layer(s, l, w.kr, w.v, n);
        if (rc >= 0) rc = session_attention(m, s, l, w.qr, Q, n, prefix, w.attn);
        if (rc >= 0) rc = mm(w.attn, Lw->w_o, w.o, n, Q, H);
        if (rc >= 0) {
            float* po = partials ? partials + ((size_t)l * 2 + 0) * (size_t)n * H : NULL;
            float* pd = partials ? partials + ((size_t)l * 2 + 1) * (size_t)n * H : NULL;
            rc = mlp_block(m, Lw, hidden, &w, n, po, pd);
        }
    }
    if (rc >= 0) rc = or_rms_norm(hidden, m->final_norm, w.normed, n, H, m->cfg.rms_norm_eps);
    if (rc >= 0 && logits)
        rc = mm(w.normed + (size_t)(n - 1) * H, m->lm_head, logits, 1, H, m->cfg.vocab);
    scratch_free(&w);
    free(hidden);
    free(positions);
    return rc < 0 ? -1 : 0;
}

/* ForwardPass::prefill (2089-2112) */
int or_prefill(const or_model* m, or_session* s, const uint32_t* tokens, int n_tokens,
               float* logits) {
    if (n_tokens <= 0) return fail("Cannot prefill an empty prompt without an explicit BOS policy");
    or_session_clear(s);
    s->position = 0;
    const int window = s->max_seq_len > 1 ? s->max_seq_len : 1;
    const int start = n_tokens > window ? n_tokens - window : 0;
    s->base_position = start;
    if (forward_tokens(m, s, tokens + start, n_tokens - start, start, logits, NULL) < 0) return -1;
    s->position = n_tokens;
    return 0;
}

int or_prefill_chunk(const or_model* m, or_session* s, const uint32_t* tokens, int n_tokens,
                     float* logits, float* partials) {
    if (n_tokens <= 0) return fail("Forward pass requires at least one token");
    if (s->base_position + session_seq_len0(s) != s->position)
        return fail("Forward pass position %d diverged from KV cache next position %d", s->position,
                    s->base_position + session_seq_len0(s));
    if (forward_tokens(m, s, tokens, n_tokens, s->position, logits, partials) < 0) return -1;
    s->position += n_tokens;
    return 0;
}

/* ========================================================= packing ====== */

int or_pack(int nseq, const int* q_len, const int* kv_before, const int* first_pos,
            const int* first_offset, const int* block_tables, int max_pages, int page_rows,
            int* cu_q, int* cu_k, int* positions, int* slot_mapping, int* seq_ids) {
    cu_q[0] = 0;
    cu_k[0] = 0;
    for (int s = 0; s < nseq; ++s) {
        cu_q[s + 1] = cu_q[s] + q_len[s];
        cu_k[s + 1] = cu_k[s] + kv_before[s] + q_len[s];
    }
    for (int s = 0; s < nseq; ++s) {
        for (int i = 0; i < q_len[s]; ++i) {
            const int t = cu_q[s] + i;
            const int row = first_offset[s] + kv_before[s] + i;
            const int pg = row / page_rows;
            if (pg >= max_pages) return fail("sequence %d row %d beyond block table capacity", s, row);
            positions[t] = first_pos[s] + i;
            slot_mapping[t] = block_tables[(size_t)s * max_pages + pg] * page_rows + row % page_rows;
            seq_ids[t] = s;
        }
    }
    return 0;
}
