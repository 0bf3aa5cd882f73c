// GQA paged attention for decode rows and causal chunked prefill.
//
// Reference semantics: single-query decode attention
// (forward_pass.rs:2838-2895) and masked multi-query attention with a cached
// prefix (forward_pass.rs:2764-2836, host text 1317-1372):
//   o = softmax(q . K^T / sqrt(d)) . V, query row r of a chunk sees keys
//   [0, prefix + r].
//
// Work decomposition.  A workgroup is one wavefront (64 lanes).  It owns one
// kv head of one "tile" and a contiguous range of KV pages (a split):
//   tile   = up to 16 / G queries of one sequence, so the 16 MFMA columns are
//            (query, q-head-of-this-kv-head) pairs -- every K/V page is read
//            once and serves all of them (the reference instead materialises
//            a GQA-expanded copy per q head, forward_pass.rs:783-828).
//   split  = pages [page_begin, page_end) of the tile's visible window.
// Each split writes (m, l, o[d]) per column; attention_reduce merges splits.
//
// Per page (16 tokens), with lane l, column c = l % 16, quad q4 = l / 16:
//   S^T[t][c] = sum_d K[t][d] Q[c][d]     mfma 16x16x32 bf16, K as A operand
//                                          (one 1 KiB coalesced load per 32 dims)
//   lane holds S^T[t = 4*q4 + i][c], i < 4 -> online softmax in registers
//   O^T[d][c] += sum_t V^T[d][t] P^T[t][c] mfma 16x16x16 bf16; P^T is exactly
//                                          the lane's own score registers.
// Precision: Q and P enter the MFMA as bf16 hi + lo pairs (x = hi + lo to
// 2^-16), K/V are exact in bf16 pools; f32 pools also split K/V into hi + lo
// (three products per MFMA pair).  Accumulation is f32 throughout.
#include "zr_internal.h"

namespace zr {

__device__ inline float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

template <typename KV, int D> struct PageRegs;

// bf16 pool: K fragment per 32 dims = 8 bf16 (16 B), V fragment per 16 dims = 4 bf16 (8 B)
template <int D> struct PageRegs<uint16_t, D> {
    bf16x8 k[D / 32];
    bf16x4 v[D / 16];
    __device__ inline void load(const uint16_t* kp, const uint16_t* vp, int lane) {
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb)
            k[kb] = *(const bf16x8*)(kp + ((size_t)kb * kWave + lane) * 8);
        const int q4 = lane >> 4, c = lane & 15;
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
            v[db] = *(const bf16x4*)(vp + ((size_t)q4 * D + db * 16 + c) * 4);
    }
};

template <int D> struct PageRegs<float, D> {
    f32x4 k[D / 32][2];
    f32x4 v[D / 16];
    __device__ inline void load(const float* kp, const float* vp, int lane) {
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            const f32x4* src = (const f32x4*)(kp + ((size_t)kb * kWave + lane) * 8);
            k[kb][0] = src[0];
            k[kb][1] = src[1];
        }
        const int q4 = lane >> 4, c = lane & 15;
#pragma unroll
        for (int db = 0; db < D / 16; ++db) v[db] = *(const f32x4*)(vp + ((size_t)q4 * D + db * 16 + c) * 4);
    }
};

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

__device__ inline bf16x4 to_bf16x4(const float* x, bool lo_part) {
    bf16x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint16_t hi, lo;
        split_bf16(x[j], hi, lo);
        r[j] = __builtin_bit_cast(__bf16, lo_part ? lo : hi);
    }
    return r;
}

template <int D>
__device__ inline f32x4 qk_mfma(const PageRegs<uint16_t, D>& pg, const bf16x8* qhi, const bf16x8* qlo) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pg.k[kb], qhi[kb], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pg.k[kb], qlo[kb], s, 0, 0, 0);
    }
    return s;
}

template <int D>
__device__ inline f32x4 qk_mfma(const PageRegs<float, D>& pg, const bf16x8* qhi, const bf16x8* qlo) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        float kf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kf[j] = pg.k[kb][0][j];
            kf[4 + j] = pg.k[kb][1][j];
        }
        const bf16x8 khi = to_bf16x8(kf, false), klo = to_bf16x8(kf, true);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, qhi[kb], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, qlo[kb], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klo, qhi[kb], s, 0, 0, 0);
    }
    return s;
}

template <int D>
__device__ inline void pv_mfma(const PageRegs<uint16_t, D>& pg, bf16x4 phi, bf16x4 plo, f32x4* o) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pg.v[db], phi, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pg.v[db], plo, o[db], 0, 0, 0);
    }
}

template <int D>
__device__ inline void pv_mfma(const PageRegs<float, D>& pg, bf16x4 phi, bf16x4 plo, f32x4* o) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        float vf[4] = {pg.v[db][0], pg.v[db][1], pg.v[db][2], pg.v[db][3]};
        const bf16x4 vhi = to_bf16x4(vf, false), vlo = to_bf16x4(vf, true);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vhi, phi, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vhi, plo, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vlo, phi, o[db], 0, 0, 0);
    }
}

struct AttnArgs {
    const float* q;          // [T, q_cols]
    int q_cols;
    const void* pool;        // layer base of the pool
    size_t page_elems;       // elements of one page (K + V, all kv heads)
    const int* block_tables;
    int stride;
    const int* first_offset;
    const int* kv_before;
    const int* cu_q;
    const int4* items;       // {tile, page_begin, page_end, unused}
    const int4* tiles;       // {seq, q0, nq, first_item}
    int G;                   // q heads per kv head
    int kv_heads;
    float scale_log2;        // log2(e) / sqrt(d)
    float* part;             // [items][kv_heads][16][D + 2]
};

template <typename KV, int D>
__global__ __launch_bounds__(64) void paged_attention_kernel(AttnArgs a) {
    const int lane = threadIdx.x;
    const int item = blockIdx.x, kvh = blockIdx.y;
    const int4 it = a.items[item];
    const int4 tl = a.tiles[it.x];
    const int seq = tl.x, q0 = tl.y, nq = tl.z;
    const int c = lane & 15, q4 = lane >> 4;
    const int qi = c / a.G, g = c - qi * a.G;
    const bool col_valid = qi < nq && c < (16 / a.G) * a.G;
    const int kvb = a.kv_before[seq];
    const int foff = a.first_offset[seq];
    // last visible logical key index of this column (causal: prefix + row)
    const int jmax = kvb + q0 + (col_valid ? qi : 0);

    // Q^T as the MFMA B operand: lane holds Q[c][32*kb + 8*q4 + j]
    bf16x8 qhi[D / 32], qlo[D / 32];
    {
        const int row = a.cu_q[seq] + q0 + (col_valid ? qi : 0);
        const float* qp = a.q + (size_t)row * a.q_cols + (size_t)(kvh * a.G + g) * D;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = col_valid ? qp[kb * 32 + q4 * 8 + j] : 0.0f;
            qhi[kb] = to_bf16x8(x, false);
            qlo[kb] = to_bf16x8(x, true);
        }
    }

    const KV* pool = (const KV*)a.pool;
    const int* bt = a.block_tables + (size_t)seq * a.stride;
    const size_t kv_tile = (size_t)kPageRows * D;            // one head's K (or V) tile
    const size_t v_block = (size_t)a.kv_heads * kv_tile;      // V block offset inside a page

    f32x4 o[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.0f;

    PageRegs<KV, D> cur, nxt;
    int p = it.y;
    const int pend = it.z;
    {
        const KV* base = pool + (size_t)bt[p] * a.page_elems + (size_t)kvh * kv_tile;
        cur.load(base, base + v_block, lane);
    }
    for (; p < pend; ++p) {
        if (p + 1 < pend) {
            const KV* base = pool + (size_t)bt[p + 1] * a.page_elems + (size_t)kvh * kv_tile;
            nxt.load(base, base + v_block, lane);
        }
        const f32x4 s = qk_mfma<D>(cur, qhi, qlo);
        float sc[4];
        float pmax = -INFINITY;
        const int jbase = p * kPageRows + q4 * 4 - foff;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = jbase + i;
            const bool ok = j >= 0 && j <= jmax;
            sc[i] = ok ? s[i] * a.scale_log2 : -INFINITY;
            pmax = fmaxf(pmax, sc[i]);
        }
        pmax = fmaxf(pmax, shfl_xor(pmax, 16));
        pmax = fmaxf(pmax, shfl_xor(pmax, 32));
        const float m_new = fmaxf(m, pmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m - m_use);
        float pr[4];
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pr[i] = exp2f(sc[i] - m_use);
            psum += pr[i];
        }
        lsum = lsum * alpha + psum;
        m = m_new;
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[db][i] *= alpha;
        pv_mfma<D>(cur, to_bf16x4(pr, false), to_bf16x4(pr, true), o);
        if (p + 1 < pend) cur = nxt;
    }
    lsum += shfl_xor(lsum, 16);
    lsum += shfl_xor(lsum, 32);

    float* out = a.part + (((size_t)item * a.kv_heads + kvh) * 16 + c) * (D + 2);
    if (q4 == 0) {
        out[0] = m;
        out[1] = lsum;
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[2 + db * 16 + q4 * 4 + i] = o[db][i];
}

// Merge the splits of one (tile, kv head): o = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
template <int D>
__global__ __launch_bounds__(256) void attention_reduce_kernel(const float* __restrict__ part,
                                                               const int4* __restrict__ tiles,
                                                               const int* __restrict__ cu_q, int G,
                                                               int kv_heads, int q_cols,
                                                               float* __restrict__ out) {
    const int tile = blockIdx.x, kvh = blockIdx.y;
    const int4 tl = tiles[tile];
    const int seq = tl.x, q0 = tl.y, nq = tl.z, first = tl.w;
    const int nparts = tiles[tile + 1].w - first;
    const int qpt = 16 / G;
    for (int e = threadIdx.x; e < 16 * D; e += blockDim.x) {
        const int c = e / D, d = e % D;
        const int qi = c / G, g = c - qi * G;
        if (qi >= nq || qi >= qpt) continue;
        float M = -INFINITY;
        for (int s = 0; s < nparts; ++s)
            M = fmaxf(M, part[(((size_t)(first + s) * kv_heads + kvh) * 16 + c) * (D + 2)]);
        float L = 0.0f, acc = 0.0f;
        for (int s = 0; s < nparts; ++s) {
            const float* ps = part + (((size_t)(first + s) * kv_heads + kvh) * 16 + c) * (D + 2);
            const float w = ps[0] == -INFINITY ? 0.0f : exp2f(ps[0] - M);
            L += ps[1] * w;
            acc += ps[2 + d] * w;
        }
        const int row = cu_q[seq] + q0 + qi;
        out[(size_t)row * q_cols + (size_t)(kvh * G + g) * D + d] = acc / L;
    }
}

template <typename KV, int D>
static zr_status launch_attn_t(zr_context* ctx, StagedMeta* st, int layer, const float* q, float* out) {
    AttnArgs a;
    a.q = q;
    a.q_cols = ctx->q_cols;
    a.page_elems = (size_t)2 * ctx->kv_cols * kPageRows;
    a.pool = (const KV*)ctx->kv_pool + (size_t)layer * ctx->n_pages * a.page_elems;
    a.block_tables = st->block_tables;
    a.stride = st->stride;
    a.first_offset = st->first_offset;
    a.kv_before = st->kv_before;
    a.cu_q = st->cu_q;
    a.items = st->attn_items;
    a.tiles = st->attn_tiles;
    a.G = ctx->q_per_kv;
    a.kv_heads = ctx->local_kv_heads;
    a.scale_log2 = 1.4426950408889634f / sqrtf((float)D);
    a.part = ctx->attn_part;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassAttention, &ev);
    hipLaunchKernelGGL((paged_attention_kernel<KV, D>), dim3(st->n_attn_items, ctx->local_kv_heads),
                       dim3(64), 0, ctx->stream, a);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassAttention, ev);
    timing_mark_begin(ctx, kClassOther, &ev);
    hipLaunchKernelGGL((attention_reduce_kernel<D>), dim3(st->n_tiles, ctx->local_kv_heads), dim3(256), 0,
                       ctx->stream, ctx->attn_part, st->attn_tiles, st->cu_q, ctx->q_per_kv,
                       ctx->local_kv_heads, ctx->q_cols, out);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassOther, ev);
    return ZR_OK;
}

zr_status launch_attention(zr_context* ctx, StagedMeta* st, int layer, const float* q, float* out) {
    if (st->n_attn_items == 0) return ZR_OK;
    const size_t need = (size_t)st->n_attn_items * ctx->local_kv_heads * 16 * (ctx->head_dim + 2);
    if (need > ctx->attn_part_floats)
        return set_err(ctx, ZR_E_OOM, "attention partial workspace too small: need %zu floats, have %zu",
                       need, ctx->attn_part_floats);
    zr_status rc;
    const bool bf = ctx->desc.kv_dtype == ZR_DTYPE_BF16;
    switch (ctx->head_dim) {
        case 64: rc = bf ? launch_attn_t<uint16_t, 64>(ctx, st, layer, q, out) : launch_attn_t<float, 64>(ctx, st, layer, q, out); break;
        case 128: rc = bf ? launch_attn_t<uint16_t, 128>(ctx, st, layer, q, out) : launch_attn_t<float, 128>(ctx, st, layer, q, out); break;
        default: return set_err(ctx, ZR_E_UNSUPPORTED, "head_dim %d not supported (64, 128)", ctx->head_dim);
    }
    return rc;
}

}  // namespace zr
