// GQA paged attention for decode rows and causal chunked prefill.
//
// Reference semantics: single-query decode attention
// (forward_pass.rs:2838-2895) and masked multi-query attention with a cached
// prefix (forward_pass.rs:2764-2836, host text 1317-1372):
//   o = softmax(q . K^T / sqrt(d)) . V, query row r of a chunk sees keys
//   [0, prefix + r].
//
// Two kernels share one launch slot: sequences with at least 128 / G query
// rows in a bf16 pool (prefill chunks) run paged_prefill_attention_kernel
// (further below); every other row (decode rows, short chunks, f32 pools)
// runs paged_attention_kernel.
//
// Work decomposition.  A workgroup is one wavefront (64 lanes).  It owns one
// kv head of one "tile" and a contiguous range of KV pages (a split):
//   tile   = up to 16 / G queries of one sequence, so the 16 MFMA columns are
//            (query, q-head-of-this-kv-head) pairs -- every K/V page is read
//            once and serves all of them (the reference instead materialises
//            a GQA-expanded copy per q head, forward_pass.rs:783-828).
//   split  = pages [page_begin, page_end) of the tile's visible window.
// Each split writes (m, l, o[d]) per column; attention_merge_kernel merges splits.
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

// Every page of the pool is read once per launch (one workgroup per kv head
// and page run), so the loads carry the nontemporal hint: the lines are
// streamed through L2 with low retention instead of displacing what the other
// waves on the XCD still read (256-session Llama-3-8B step: attention 9.55-9.78
// -> 8.81-8.99 ms per step; 32-session TinyLlama step unchanged).
template <typename KV, int D> struct PageRegs;

// bf16 pool: K fragment per 32 dims = 8 bf16 (16 B); V per 32 dims = 8 bf16
// (16 B): tokens 4 q4 .. 4 q4 + 3 of dims 32 vb + c, then of 32 vb + 16 + c.
// Both are one 1 KiB contiguous wave load.
template <int D> struct PageRegs<uint16_t, D> {
    bf16x8 k[D / 32];
    bf16x8 v[D / 32];
    __device__ inline void load(const uint16_t* kp, const uint16_t* vp, int lane) {
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb)
            k[kb] = __builtin_nontemporal_load((const bf16x8*)(kp + ((size_t)kb * kWave + lane) * 8));
#pragma unroll
        for (int vb = 0; vb < D / 32; ++vb)
            v[vb] = __builtin_nontemporal_load((const bf16x8*)(vp + ((size_t)vb * kWave + lane) * 8));
    }
};

// f32 pool (page_order): the same 8 values per lane and 32 dims, as two
// 16 B halves that each come from one contiguous 1 KiB wave run (K: dims
// 8 g + [0, 4) then + [4, 8); V: dim d then d + 16, 4 tokens each).
template <int D> struct PageRegs<float, D> {
    f32x4 k[D / 32][2];
    f32x4 v[D / 32][2];
    __device__ inline void load(const float* kp, const float* vp, int lane) {
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            const f32x4* src = (const f32x4*)(kp + (size_t)kb * kWave * 8) + lane;
            k[kb][0] = __builtin_nontemporal_load(src);
            k[kb][1] = __builtin_nontemporal_load(src + kWave);
        }
#pragma unroll
        for (int vb = 0; vb < D / 32; ++vb) {
            const f32x4* src = (const f32x4*)(vp + (size_t)vb * kWave * 8) + lane;
            v[vb][0] = __builtin_nontemporal_load(src);
            v[vb][1] = __builtin_nontemporal_load(src + kWave);
        }
    }
};

// x[0..7] as bf16 hi + lo fragments, two values per v_cvt_pk_bf16_f32 (the
// same bits as split_bf16)
__device__ inline void split_bf16x8(const float* x, bf16x8& hi, bf16x8& lo) {
    typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2;
    typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x2 v = {x[2 * j], x[2 * j + 1]};
        const bf16x2 h = __builtin_convertvector(v, bf16x2);
        const bf16x2 l = __builtin_convertvector(v - __builtin_convertvector(h, f32x2), bf16x2);
        hi[2 * j] = h[0];
        hi[2 * j + 1] = h[1];
        lo[2 * j] = l[0];
        lo[2 * j + 1] = l[1];
    }
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

// qhi / qlo point at [D / 32][64] fragment arrays (LDS); lane selects its slot.
template <int D>
__device__ inline f32x4 qk_mfma(const PageRegs<uint16_t, D>& pg, const bf16x8* qhi, const bf16x8* qlo, int lane) {
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pg.k[kb], qhi[kb * 64 + lane], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pg.k[kb], qlo[kb * 64 + lane], s, 0, 0, 0);
    }
    return s;
}

template <int D>
__device__ inline f32x4 qk_mfma(const PageRegs<float, D>& pg, const bf16x8* qhi, const bf16x8* qlo, int lane) {
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
        const bf16x8 qh = qhi[kb * 64 + lane];
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, qh, s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(khi, qlo[kb * 64 + lane], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(klo, qh, s, 0, 0, 0);
    }
    return s;
}

// O^T += V^T P^T over a page pair (32 tokens) on the 16x16x32 MFMA: lane l
// supplies tokens 4*q4 .. 4*q4+3 of page A then of page B for both operands,
// which is exactly its own score registers for P^T and, for V^T, the matching
// 4-token halves of its two pages' V fragments (dims 16 db + c).
template <int D>
__device__ inline void pv_mfma2(const PageRegs<uint16_t, D>& pa, const PageRegs<uint16_t, D>& pb, bf16x8 phi,
                                bf16x8 plo, f32x4* o) {
#pragma unroll
    for (int vb = 0; vb < D / 32; ++vb) {
        const bf16x8 v0 = __builtin_shufflevector(pa.v[vb], pb.v[vb], 0, 1, 2, 3, 8, 9, 10, 11);
        const bf16x8 v1 = __builtin_shufflevector(pa.v[vb], pb.v[vb], 4, 5, 6, 7, 12, 13, 14, 15);
        o[2 * vb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, phi, o[2 * vb], 0, 0, 0);
        o[2 * vb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, plo, o[2 * vb], 0, 0, 0);
        o[2 * vb + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, phi, o[2 * vb + 1], 0, 0, 0);
        o[2 * vb + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, plo, o[2 * vb + 1], 0, 0, 0);
    }
}

template <int D>
__device__ inline void pv_mfma2(const PageRegs<float, D>& pa, const PageRegs<float, D>& pb, bf16x8 phi, bf16x8 plo,
                                f32x4* o) {
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
        const f32x4 va = pa.v[db >> 1][db & 1], vbv = pb.v[db >> 1][db & 1];
        float vf[8] = {va[0], va[1], va[2], va[3], vbv[0], vbv[1], vbv[2], vbv[3]};
        const bf16x8 vhi = to_bf16x8(vf, false), vlo = to_bf16x8(vf, true);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vhi, phi, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vhi, plo, o[db], 0, 0, 0);
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vlo, phi, o[db], 0, 0, 0);
    }
}

// max over the lanes {l, l^16, l^32, l^48} (the four quads holding one column),
// with gfx950's VALU lane swaps.
__device__ inline float quad_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

struct AttnArgs {
    const float* q;          // [T, q_cols]
    int q_cols;
    const void* pool;        // layer base of the pool
    size_t page_elems;       // elements of one page (K + V, all kv heads)
    const int* block_tables;
    int stride;
    const int4* rec;         // three records per dispatch rank (longest item first): {seq, first q row, nq,
                             // page_begin}, {page_end, kv_before + q0, first_offset, item | kAttnSingle | kAttnLast},
                             // {pool pages of the item's first 4 pages}
    int n_items;
    int G;                   // q heads per kv head
    int kv_heads;
    float scale_log2;        // log2(e) / sqrt(d)
    float* part;             // [items][kv_heads][16][D + 2]
    float* out_f32;          // final output of single-split tiles ([T, q_cols]) ...
    uint16_t* out_bf16;      // ... or as the bf16 A operand (lo half at out_lo_offset)
    size_t out_lo_offset;
    // FUSE (pure decode microbatches): q and the new K / V rows come from the
    // QKV product's split-K slabs, rotated with the step's (cos, sin) table,
    // and each tile's last split appends its kv head's K / V row to the page
    const float* qkv;        // slab 0 of [T, qkv_stride]
    int qkv_n;               // slabs, summed in slab order
    size_t qkv_slab;         // floats from one slab to the next
    int qkv_stride;          // q_cols + 2 kv_cols
    int kv_cols;
    const int* slot;         // [T] pool slot of each row's new K / V
    const float2* rope_cs;   // [T][D / 2] (cos, sin), or null: no rotation
};

template <typename KV, int D, int RING, bool FUSE>
__global__ __launch_bounds__(64) void paged_attention_kernel(AttnArgs a) {
    const int lane = threadIdx.x;
    // Workgroups go to the 8 XCDs round-robin (XCD = blockIdx % 8).  Block
    // b = 8 kv_heads grp + 8 kvh + x runs kv head kvh of dispatch rank
    // 8 grp + x, so every kv head of one item -- all of its pages' bytes --
    // is read through the same XCD (its L2 and its address translation).
    const int per_grp = 8 * a.kv_heads;
    const int rem = blockIdx.x % per_grp;
    const int kvh = rem >> 3;
    const int rank = (blockIdx.x / per_grp) * 8 + (rem & 7);
    if (rank >= a.n_items) return;
    // everything the workgroup needs to start its loads, in one record
    const int4 r0 = a.rec[3 * rank], r1 = a.rec[3 * rank + 1], r2 = a.rec[3 * rank + 2];
    const int seq = r0.x, row0 = r0.y, nq = r0.z, page_b = r0.w, page_e = r1.x, foff = r1.z;
    if (nq == 0) return;  // an empty record past a replayed bucket's items
    const unsigned meta = (unsigned)r1.w;
    const int item = (int)(meta & (kAttnSingle - 1));
    const int c = lane & 15, q4 = lane >> 4;
    const int qi = c / a.G, g = c - qi * a.G;
    const bool col_valid = qi < nq && c < (16 / a.G) * a.G;
    // last visible logical key index of this column (causal: prefix + row)
    const int jmax = r1.y + (col_valid ? qi : 0);

    // Q^T as the MFMA B operand (lane holds Q[c][32*kb + 8*q4 + j]) as bf16
    // hi + lo fragments, parked in LDS to keep registers for the page ring.
    __shared__ bf16x8 qs[2][D / 32][64];
    const bf16x8* qhi = qs[0][0];
    const bf16x8* qlo = qs[1][0];

    const KV* pool = (const KV*)a.pool;
    const int* bt = a.block_tables + (size_t)seq * a.stride;
    const size_t kv_tile = (size_t)kPageRows * D;            // one head's K (or V) tile
    const size_t v_block = (size_t)a.kv_heads * kv_tile;      // V block offset inside a page

    f32x4 o[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.0f;

    // a page pair (p, p + 1): S^T = K Q^T for both, one online-softmax step
    // over 32 tokens, O^T += V^T P^T.  has_b == false masks page B (odd tail).
    auto process2 = [&](const PageRegs<KV, D>& pa, const PageRegs<KV, D>& pb, int p, bool has_b) {
        const f32x4 sa = qk_mfma<D>(pa, qhi, qlo, lane);
        const f32x4 sb = qk_mfma<D>(pb, qhi, qlo, lane);
        float sc[8];
        float pmax = -INFINITY;
        const int jbase = p * kPageRows + q4 * 4 - foff;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ja = jbase + i, jb = jbase + kPageRows + i;
            sc[i] = (ja >= 0 && ja <= jmax) ? sa[i] * a.scale_log2 : -INFINITY;
            sc[4 + i] = (has_b && jb <= jmax) ? sb[i] * a.scale_log2 : -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) pmax = fmaxf(pmax, sc[i]);
        pmax = quad_max(pmax);
        const float m_new = fmaxf(m, pmax);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m - m_use);
        float pr[8];
        float psum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pr[i] = exp2f(sc[i] - m_use);
            psum += pr[i];
        }
        lsum = lsum * alpha + psum;
        m = m_new;
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[db][i] *= alpha;
        pv_mfma2<D>(pa, pb, to_bf16x8(pr, false), to_bf16x8(pr, true), o);
    };

    // Register ring of RING page sets, consumed in pairs: RING - 2 pages are
    // in flight while a pair is computed.
    static_assert(RING % 2 == 0 && RING >= 4, "ring of page pairs");
    PageRegs<KV, D> ring[RING];
    auto load_page = [&](PageRegs<KV, D>& r, int pool_page) {
        const KV* base = pool + (size_t)pool_page * a.page_elems + (size_t)kvh * kv_tile;
        r.load(base, base + v_block, lane);
    };
    auto load_or_shared = [&](PageRegs<KV, D>& r, int p) {
        const int pg = bt[min(p, page_e - 1)];
        load_page(r, p < page_e ? pg : 0);
    };
    // Every ring slot is loaded unconditionally (past the split's end, and in
    // the record past a short item's end, pool page 0, which every wave
    // shares, so those loads hit L2; the values are never used: 32-session
    // TinyLlama step attention -1.4% against reloading the split's last page,
    // a third of whose loads fall past the end of an 8-page split with this
    // ring): with no conditional loads the compiler
    // can wait for exactly the slot it computes on (in-order vmcnt) instead
    // of conservatively draining the newest pages' loads too.  The pool
    // pages of the first RING - 2 come from the record: no block-table load
    // stands before them.
    static_assert(RING - 2 <= 4, "the record holds the first 4 pages");
    const int first_pages[4] = {r2.x, r2.y, r2.z, r2.w};
    auto load_first_pages = [&]() {
#pragma unroll
        for (int r = 0; r < RING - 2; ++r) load_page(ring[r], first_pages[r]);
    };
    // Q row of this lane's column, fetched before the first pages so that its
    // wait (in-order vmcnt) does not also wait for them
    f32x4 qx[D / 32][2];
    if constexpr (FUSE) {
        // RoPE + KV append of the decode row (the scalar RoPE kernel's
        // operations in its order: slabs summed in slab order, then
        // a c - b s, a s + b c per rotate-half pair, no contraction).  A
        // decode tile holds one query: column c < G is q head kvh G + c.
        const int row = row0;
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        // Every column reads a q head of the row (g < G), so the loads need
        // no guard: columns past the tile are zeroed after the sums.  The
        // slabs are read nontemporal, like the pages (256-session step:
        // launch 275.4-277.9 -> 272.8-273.5 us).
        const float* qp = a.qkv + (size_t)row * a.qkv_stride + (size_t)(kvh * a.G + g) * D + q4 * 8;
        // (cos, sin) of the lane's dims 32 kb + 8 q4 + j for kb < D / 64 (the
        // rotate-half partner of block kb is kb + D / 64), fetched together
        // with the slabs: one round trip for both
        float cv[D / 64][8], sv[D / 64][8];
        if (a.rope_cs) {
            const float2* cs = a.rope_cs + (size_t)row * (D / 2) + q4 * 8;
#pragma unroll
            for (int kb = 0; kb < D / 64; ++kb)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float4 pr = ((const float4*)(cs + kb * 32))[w];
                    cv[kb][2 * w] = pr.x;
                    sv[kb][2 * w] = pr.y;
                    cv[kb][2 * w + 1] = pr.z;
                    sv[kb][2 * w + 1] = pr.w;
                }
        }
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            qx[kb][0] = __builtin_nontemporal_load((const f32x4*)(qp + kb * 32));
            qx[kb][1] = __builtin_nontemporal_load((const f32x4*)(qp + kb * 32 + 4));
        }
        constexpr int CH = D == 64 ? 8 : 4;  // slabs per batch of loads
        // The tile's last split appends the new row.  Lane e (and e + 64 ...)
        // handles K pair (e, e + D / 2) for e < D / 2, else V dim e - D / 2;
        // its values of the first NB slabs, K's (cos, sin) and the row's
        // slot come in the same round trip as q's slabs.
        const bool last = meta & kAttnLast;
        constexpr int NE = (D / 2 + D + 63) / 64, NB = 1 + CH;
        const float* kr = a.qkv + (size_t)row * a.qkv_stride + a.q_cols + (size_t)kvh * D;
        const float* vr = kr + a.kv_cols;
        float ax[NE][NB], ay[NE][NB];
        float2 kcs = make_float2(1.f, 0.f);
        int sl = 0;
        if (last) {
            sl = a.slot[row];
#pragma unroll
            for (int i = 0; i < NE; ++i) {
                const int e = lane + 64 * i;
#pragma unroll
                for (int u = 0; u < NB; ++u)
                    if (u < a.qkv_n) {
                        if (e < D / 2) {
                            ax[i][u] = kr[(size_t)u * a.qkv_slab + e];
                            ay[i][u] = kr[(size_t)u * a.qkv_slab + e + D / 2];
                        } else if (e < D / 2 + D) {
                            ax[i][u] = vr[(size_t)u * a.qkv_slab + e - D / 2];
                        }
                    }
            }
            if (a.rope_cs && lane < D / 2) kcs = a.rope_cs[(size_t)row * (D / 2) + lane];
        }
        for (int s0 = 1; s0 < a.qkv_n; s0 += CH) {
            f32x4 t[CH][D / 32][2];
#pragma unroll
            for (int u = 0; u < CH; ++u)
#pragma unroll
                for (int kb = 0; kb < D / 32; ++kb)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        t[u][kb][h] = s0 + u < a.qkv_n ? __builtin_nontemporal_load((const f32x4*)(
                                                              qp + (size_t)(s0 + u) * a.qkv_slab + kb * 32 + 4 * h))
                                                        : zero;
#pragma unroll
            for (int u = 0; u < CH; ++u)
                if (s0 + u < a.qkv_n)
#pragma unroll
                    for (int kb = 0; kb < D / 32; ++kb) {
                        qx[kb][0] += t[u][kb][0];
                        qx[kb][1] += t[u][kb][1];
                    }
        }
        if (!col_valid)
#pragma unroll
            for (int kb = 0; kb < D / 32; ++kb) qx[kb][0] = qx[kb][1] = zero;
        if (a.rope_cs) {
#pragma clang fp contract(off)
#pragma unroll
            for (int kb = 0; kb < D / 64; ++kb)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = qx[kb][j >> 2][j & 3], y = qx[kb + D / 64][j >> 2][j & 3];
                    qx[kb][j >> 2][j & 3] = x * cv[kb][j] - y * sv[kb][j];
                    qx[kb + D / 64][j >> 2][j & 3] = x * sv[kb][j] + y * cv[kb][j];
                }
        }
        // the appended row's values, complete before any page load goes out
        // (the same operations in the same order as the RoPE kernel: slabs
        // summed in slab order, then x c - y s, x s + y c)
        float av[NE][2];
        if (last) {
#pragma clang fp contract(off)
#pragma unroll
            for (int i = 0; i < NE; ++i) {
                const int e = lane + 64 * i;
                float x = ax[i][0], y = ay[i][0];
#pragma unroll
                for (int u = 1; u < NB; ++u)
                    if (u < a.qkv_n) {
                        x += ax[i][u];
                        if (e < D / 2) y += ay[i][u];
                    }
                for (int u = NB; u < a.qkv_n; ++u) {
                    if (e < D / 2) {
                        x += kr[(size_t)u * a.qkv_slab + e];
                        y += kr[(size_t)u * a.qkv_slab + e + D / 2];
                    } else if (e < D / 2 + D) {
                        x += vr[(size_t)u * a.qkv_slab + e - D / 2];
                    }
                }
                if (e < D / 2 && a.rope_cs) {
                    const float nx = x * kcs.x - y * kcs.y;
                    const float ny = x * kcs.y + y * kcs.x;
                    x = nx;
                    y = ny;
                }
                av[i][0] = x;
                av[i][1] = y;
            }
        }
        // the first ring pages go out before the append's wait when none of
        // them can hold the new row (it sits in the split's last page)
        const bool early = !last || page_e - page_b > RING - 2;
        if (early) load_first_pages();
        if (last) {
            const int r = sl % kPageRows;
            KV* kt = (KV*)a.pool + (size_t)(sl / kPageRows) * a.page_elems + (size_t)kvh * kv_tile;
            KV* vt = kt + v_block;
#pragma unroll
            for (int i = 0; i < NE; ++i) {
                const int e = lane + 64 * i;
                if (e < D / 2) {
                    store_elem(kt + page_order<KV>(k_off(r, e)), av[i][0]);
                    store_elem(kt + page_order<KV>(k_off(r, e + D / 2)), av[i][1]);
                } else if (e < D / 2 + D) {
                    store_elem(vt + page_order<KV>(v_off(r, e - D / 2)), av[i][0]);
                }
            }
            ring_barrier<0>();  // the row is written before its page is read
        }
        if (!early) load_first_pages();
    } else {
        const int row = row0 + (col_valid ? qi : 0);
        const float* qp = a.q + (size_t)row * a.q_cols + (size_t)(kvh * a.G + g) * D + q4 * 8;
#pragma unroll
        for (int kb = 0; kb < D / 32; ++kb) {
            qx[kb][0] = col_valid ? *(const f32x4*)(qp + kb * 32) : f32x4{0.f, 0.f, 0.f, 0.f};
            qx[kb][1] = col_valid ? *(const f32x4*)(qp + kb * 32 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
        load_first_pages();
    }
    const int pend = page_e;
#pragma unroll
    for (int kb = 0; kb < D / 32; ++kb) {
        const float x[8] = {qx[kb][0][0], qx[kb][0][1], qx[kb][0][2], qx[kb][0][3],
                            qx[kb][1][0], qx[kb][1][1], qx[kb][1][2], qx[kb][1][3]};
        qs[0][kb][lane] = to_bf16x8(x, false);
        qs[1][kb][lane] = to_bf16x8(x, true);
    }
    for (int p = page_b; p < pend; p += RING) {
#pragma unroll
        for (int r = 0; r < RING; r += 2) {
            const int pp = p + r;
            if (pp >= pend) break;
            load_or_shared(ring[(r + RING - 2) % RING], pp + RING - 2);
            load_or_shared(ring[(r + RING - 1) % RING], pp + RING - 1);
            const bool has_b = pp + 1 < pend;
            process2(ring[r], has_b ? ring[r + 1] : ring[r], pp, has_b);
        }
    }
    lsum += shfl_xor(lsum, 16);
    lsum += shfl_xor(lsum, 32);

    if (!col_valid) return;
    if (meta & kAttnSingle) {
        // the tile has one split: normalise and write the final output here
        const int row = row0 + qi;
        const float inv = 1.0f / lsum;
        if (a.out_bf16) {
            // Lane (c, q4) holds dims 16 db + 4 q4 + [0, 4); lane (c, q4 ^ 1)
            // the neighbouring 4.  One exchange per float gives the even-q4
            // lane dims 16 db + 4 q4 + [0, 8) of an even block db and the odd
            // one the same run of block db + 1: one 16-byte run of the
            // fragment-packed operand per plane.  The partner has the same
            // column, so the same col_valid.
            static_assert(D % 32 == 0, "pairs of 16-dim blocks");
            const bool odd = q4 & 1;
#pragma unroll
            for (int db = 0; db < D / 16; db += 2) {
                float x[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float mine = (odd ? o[db + 1][i] : o[db][i]) * inv;
                    const float theirs = shfl_xor((odd ? o[db][i] : o[db + 1][i]) * inv, 16);
                    x[i] = odd ? theirs : mine;
                    x[4 + i] = odd ? mine : theirs;
                }
                const int d0 = odd ? 16 * (db + 1) + 4 * (q4 - 1) : 16 * db + 4 * q4;
                // nontemporal: the lines need not stay in L2 beside the page
                // stream (256-session step: launch 276.5-277.8 -> 271.1-271.7 us)
                const size_t o_idx = a_pack_index(row, (kvh * a.G + g) * D + d0, a.q_cols);
                __builtin_nontemporal_store(to_bf16x8(x, false), (bf16x8*)(a.out_bf16 + o_idx));
                if (a.out_lo_offset)
                    __builtin_nontemporal_store(to_bf16x8(x, true), (bf16x8*)(a.out_bf16 + a.out_lo_offset + o_idx));
            }
            return;
        }
#pragma unroll
        for (int db = 0; db < D / 16; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a.out_f32[(size_t)row * a.q_cols + (kvh * a.G + g) * D + db * 16 + q4 * 4 + i] = o[db][i] * inv;
        return;
    }
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

// ------------------------------------------------------------ prefill blocks
// Sequences with at least 128 / G query rows (prefill chunks) run here, bf16
// pools only.  A workgroup of 4 waves owns one kv head of one block of
// 128 / G query rows: 128 columns = (row, q head of the kv head) pairs, 32
// per wave.  Every 32-key tile (two pages) of the block's visible window is
// copied once into an LDS ring with global_load_lds (the pool's page layout,
// no registers) and serves all 128 columns, where the decode tiles above
// would read each page once per 16 columns.
// Per tile and wave, on v_mfma_f32_32x32x16_bf16 (lane l, h = l / 32):
//   S[key][col] = sum_d K[key][d] Q[col][d]: K (A operand) is one 16 B LDS read
//     per lane and 16 dims (key l % 32, dims 16 ks + 8 h .. + 7 = one chunk of
//     the page's K layout); Q^T (B operand) as bf16 hi + lo in registers.
//     The lane gets S[8 (i / 4) + 4 h + i % 4][l % 32], i < 16.
//   online softmax per column: 16 keys in the lane, the other 16 in lane l ^ 32.
//   O[d][col] += sum_key V[key][d] P[key][col]: the summation index k = 8 h + j
//     of k-step ks2 stands for key 16 ks2 + 8 (j / 4) + 4 h + j % 4, so P's B
//     fragment is the lane's own scores i = 8 ks2 + j (hi + lo), and V^T's A
//     fragment is two 8-byte runs of the page's V layout (rows 4 h .. 4 h + 3
//     and 8 + 4 h .. of dim 32 db + l % 32).
// Causal mask: column (row r, head g) sees logical keys j <= kv_before + r.
struct PrefillArgs {
    const float* q;          // [T, q_cols]
    int q_cols;
    const uint16_t* pool;    // layer base of the pool (bf16)
    size_t page_elems;
    int stride;              // block table row stride (the table is a kernel argument)
    const int* first_offset;
    const int* kv_before;
    const int* cu_q;
    const int4* blocks;      // per work unit: {seq, r0, nrows, pages}, most key tiles first
    const int4* splits;      // per work unit: {first key tile, end key tile, partial item, splits of the block}
    int n_blocks;
    float* part;             // [items][kv_heads][16][D + 2] partials of blocks with splits > 1
    int G;                   // q heads per kv head (divides 32)
    int kv_heads;
    float scale_log2;        // log2(e) / sqrt(d)
    float* out_f32;
    uint16_t* out_bf16;
    size_t out_lo_offset;
};

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

__device__ inline float pair_max(float x) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ inline float pair_sum(float x) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int D, int STAGES, int KH>
__global__ __launch_bounds__(256 * KH, 2 / KH) void paged_prefill_attention_kernel(PrefillArgs a,
                                                                               const int* __restrict__ block_tables) {
    constexpr int NW = 4;            // column waves (32 columns each)
    constexpr int CHUNKS = 8 * D;   // 16 B chunks per tile: 2 pages x (K, V) x 16 rows x D bf16
    constexpr int VM = D / 32;      // global_load_lds per wave per stage (1 KiB each)
    static_assert(CHUNKS == NW * VM * 64, "stage copy split");
    static_assert(KH == 1 || KH == 2, "key halves");
    // a stage holds KH consecutive key tiles, tile h for the waves of half h
    __shared__ bf16x8 lds[STAGES][KH][CHUNKS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = wave / NW, wq = wave - half * NW;  // key half, column wave
    // block-uniform values in scalar registers
    const int rank = __builtin_amdgcn_readfirstlane(blockIdx.x / a.kv_heads);
    const int kvh = blockIdx.x - rank * a.kv_heads;
    const int4 blk = a.blocks[rank];
    const int4 spl = a.splits[rank];
    const int seq = __builtin_amdgcn_readfirstlane(blk.x), r0 = __builtin_amdgcn_readfirstlane(blk.y);
    const int nrows = __builtin_amdgcn_readfirstlane(blk.z), npages = __builtin_amdgcn_readfirstlane(blk.w);
    const int kt0 = __builtin_amdgcn_readfirstlane(spl.x), kt1 = __builtin_amdgcn_readfirstlane(spl.y);
    const int h = lane >> 5;
    const int col = lane & 31;
    const int rpw = 32 / a.G;  // query rows per column wave
    const int rloc = wq * rpw + col / a.G, g = col - (col / a.G) * a.G;
    const bool valid = rloc < nrows;
    const int kvb = __builtin_amdgcn_readfirstlane(a.kv_before[seq]);
    const int foff = __builtin_amdgcn_readfirstlane(a.first_offset[seq]);
    const int jmax = kvb + r0 + (valid ? rloc : 0);  // last visible logical key of this column
    const int grow = __builtin_amdgcn_readfirstlane(a.cu_q[seq]) + r0 + (valid ? rloc : 0);

    const uint16_t* pool = a.pool;
    // (a restrict kernel argument: nothing here writes it, so its reads are scalar loads)
    const int* bt = block_tables + (size_t)seq * a.stride;
    const size_t kv_tile = (size_t)kPageRows * D;
    const size_t v_block = (size_t)a.kv_heads * kv_tile;
    // Key tiles [kt0, kt1) go in steps of KH: step p holds tile kt0 + KH p + h
    // for the waves of half h.  A half stages its own tile of each step into
    // ring slot `slot` from the pool pages of the tile's two pages (pg0, pg1):
    // chunk group f = i NW + wq is (page pp, K or V, 1 KiB group); a page past
    // the window's end repeats the last page (its keys are masked, and a tile
    // past kt1 is copied the same way and skipped), so every wave issues VM
    // copies per stage.  The page ids are read a step ahead (tile_pages), so
    // no scalar load waits in front of a stage's copies.
    auto tile_pages = [&](int kt, int& pg0, int& pg1) {
        pg0 = __builtin_amdgcn_readfirstlane(bt[min(2 * kt, npages - 1)]);
        pg1 = __builtin_amdgcn_readfirstlane(bt[min(2 * kt + 1, npages - 1)]);
    };
    // Copies are buffer loads into LDS over one page: the page's base in the
    // (scalar) buffer descriptor, the lane's 16 B as the vector offset, the
    // K / V block, kv head and 1 KiB group as a scalar offset.
    const uint32_t page_bytes = (uint32_t)(a.page_elems * 2);
    const int voff = lane * 16;
    auto issue = [&](int slot, int pg0, int pg1) {
        const __amdgpu_buffer_rsrc_t r0 =
            __builtin_amdgcn_make_buffer_rsrc((void*)(pool + (size_t)pg0 * a.page_elems), 0, page_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t r1 =
            __builtin_amdgcn_make_buffer_rsrc((void*)(pool + (size_t)pg1 * a.page_elems), 0, page_bytes, 0x00020000);
#pragma unroll
        for (int i = 0; i < VM; ++i) {
            const int f = i * NW + wq;
            const int pp = f / (2 * VM), kv = (f / VM) & 1, grp = f % VM;
            const int soff = (int)(((kv ? v_block : 0) + (size_t)kvh * kv_tile) * 2) + grp * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(pp ? r1 : r0, (lds_void*)&lds[slot][half][f * 64], 16, voff, soff,
                                                     0, 0);
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[db][i] = 0.0f;
    float m = -INFINITY, lsum = 0.0f;

    // a tile needs the causal mask only if it may hold a key before the
    // window (first_offset) or after the block's first row's last visible key
    const int ntiles = kt1 - kt0;
    const int nsteps = (ntiles + KH - 1) / KH;
    const int jfree = kvb + r0;  // keys <= jfree are visible to every row of the block
    int npg0 = 0, npg1 = 0;  // pool pages of this half's tile of the next step to stage
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nsteps) {
            tile_pages(kt0 + KH * s + half, npg0, npg1);
            issue(s, npg0, npg1);
        }
    tile_pages(kt0 + KH * (STAGES - 1) + half, npg0, npg1);
    // Q^T fragments (B operand): lane holds Q[col][16 ks + 8 h + j] * log2(e) / sqrt(d)
    // as hi + lo (scores come out in log2 units).  Loaded after the first
    // stages' copies are issued, so both latencies overlap.
    bf16x8 qh[D / 16], ql[D / 16];
    {
        const float* qp = a.q + (size_t)grow * a.q_cols + (size_t)(kvh * a.G + g) * D + 8 * h;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            float x[8];
            const f32x4 x0 = valid ? *(const f32x4*)(qp + 16 * ks) : f32x4{0.f, 0.f, 0.f, 0.f};
            const f32x4 x1 = valid ? *(const f32x4*)(qp + 16 * ks + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[j] = x0[j] * a.scale_log2;
                x[4 + j] = x1[j] * a.scale_log2;
            }
            qh[ks] = to_bf16x8(x, false);
            ql[ks] = to_bf16x8(x, true);
        }
    }
    // One tile of a half in two parts.  phase_s: the tile's LDS fragments,
    // read in two batches ahead of their consumers (K before the S = K Q^T
    // MFMAs, V before the softmax, whose VALU work covers their return), and
    // S.  phase_p: the causal mask where needed, the online softmax step and
    // O += V^T P, on registers only.
    f32x16 s;
    bf16x8 vfr[2][D / 32];
    int s_it = 0;        // key tile held in s / vfr
    bool s_act = false;  // ... and whether it is one of the block's tiles
    auto phase_s = [&](int t) {
        s_it = kt0 + KH * t + half;
        s_act = KH == 1 || s_it < kt1;
        if (!s_act) {
            // (s and vfr are written on every path, so the previous tile's
            // values are not kept alive through this one)
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
                for (int db = 0; db < D / 32; ++db) vfr[ks2][db] = bf16x8{};
            return;
        }
        const bf16x8* st = lds[t % STAGES][half];
        const int kbase = ((lane >> 4) & 1) * 2 * (2 * D) + (lane & 15);  // page pp = (l % 32) / 16, row l % 16
        bf16x8 kf[D / 16];
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) kf[ks] = st[kbase + (2 * ks + h) * 16];
        __builtin_amdgcn_sched_barrier(0);  // the K reads stay ahead of the MFMAs
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qh[ks], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], ql[ks], s, 0, 0, 0);
        }
        const bf16x4* sv = (const bf16x4*)st;
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ++ks2) {
            const int vbase = (2 * ks2 + 1) * 4 * D;  // 8-byte units of page ks2's V block
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
                // unit of (rows 4 q .. 4 q + 3, dim d): ((d / 32 * 4 + q) * 16 + d % 16) * 2 + d / 16 % 2
                const int u = ((db * 4 + h) * 16 + (lane & 15)) * 2 + ((lane >> 4) & 1);
                const bf16x4 v0 = sv[vbase + u], v1 = sv[vbase + u + 2 * 16 * 2];
                vfr[ks2][db] = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // the V reads go out before the softmax
    };
    auto phase_p = [&]() {
        if (!s_act) return;
        const int it = s_it;
        // the causal mask only on tiles that can hold a key before the window
        // or past the block's first row (a uniform branch, kept out of the
        // common path)
        if (it * 32 - foff < 0 || it * 32 + 31 - foff > jfree) {
            asm volatile("" ::: "memory");
            const int jbase = it * 32 + 4 * h - foff;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int j = jbase + 8 * (i >> 2) + (i & 3);
                if (j < 0 || j > jmax) s[i] = -INFINITY;
            }
        }
        float tmax = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, s[i]);
        tmax = pair_max(tmax);
        // Lazy rescale: a column keeps its running max m until a tile's max
        // exceeds it by more than 8 (log2 units), so P <= 2^8 and O and l are
        // rescaled only when some column of the wave moves that far (the first
        // tile with a visible key, then rarely).  The result is the same
        // softmax: O and l share the scale.
        if (__any(tmax > m + 8.0f)) {
            // only the lanes whose max moves rescale (alpha 0 while m = -inf);
            // the others keep alpha = 1 exactly, also a column with no visible
            // key yet (m = -inf, where m - m would be NaN)
            const bool up = tmax > m + 8.0f;
            const float alpha = up ? __builtin_amdgcn_exp2f(m - tmax) : 1.0f;
            if (up) m = tmax;
            lsum *= alpha;
#pragma unroll
            for (int db = 0; db < D / 32; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        }
        const float m_use = m == -INFINITY ? 0.0f : m;
        float pr[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            pr[i] = __builtin_amdgcn_exp2f(s[i] - m_use);
            lsum += pr[i];
        }
        // O += V^T P over the tile's two pages (k-steps ks2)
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ++ks2) {
            bf16x8 ph, pl;
            split_bf16x8(pr + 8 * ks2, ph, pl);
#pragma unroll
            for (int db = 0; db < D / 32; ++db) {
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[ks2][db], ph, o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[ks2][db], pl, o[db], 0, 0, 0);
            }
        }
    };
    // the page ids of the step after the one just staged, read once this
    // step's LDS reads have been issued and waited for (scalar loads return
    // out of order: one in flight would turn every LDS wait into a full
    // drain); the next ring barrier waits for them
    auto prefetch_pages = [&](int t) {
        __builtin_amdgcn_sched_barrier(0);
        if (t + STAGES - 1 < nsteps) tile_pages(kt0 + KH * (t + STAGES) + half, npg0, npg1);
    };
    // One loop for both forms: with KH = 2 each half takes every other key
    // tile (kt0 + 2 t + half) of the block.  (A second barrier per step that
    // offset the halves into MFMA-bound and VALU-bound phases measured slower
    // once the copies were descriptor-based: mixed 2108-row microbatch, prefill
    // kernel 90.9-91.1 against 87.4-87.7 us per layer without it.)
    for (int t = 0; t < nsteps; ++t) {
        ring_wait<VM, STAGES - 2>(min(STAGES - 2, nsteps - 1 - t));
        if (t + STAGES - 1 < nsteps) issue((t + STAGES - 1) % STAGES, npg0, npg1);
        phase_s(t);
        phase_p();
        prefetch_pages(t);
    }
    lsum = pair_sum(lsum);
    if constexpr (KH == 2) {
        // The halves' (m, l, O) of each column meet in LDS (the ring is free:
        // every wave has passed its last ring wait and LDS read): half 1
        // writes, half 0 rescales both to the larger m and adds.  A half with
        // no visible key in its tiles (m = -inf, l = 0, O = 0) gets weight 0.
        constexpr int CW = 2 + 16 * (D / 32);  // floats per column lane
        static_assert((size_t)NW * CW * 64 * 4 <= sizeof(lds), "combine buffer");
        float* cmb = (float*)&lds[0][0][0] + (size_t)wq * CW * 64 + lane;  // [wq][j][lane]
        __syncthreads();
        if (half == 1) {
            cmb[0] = m;
            cmb[64] = lsum;
#pragma unroll
            for (int db = 0; db < D / 32; ++db)
#pragma unroll
                for (int i = 0; i < 16; ++i) cmb[(2 + db * 16 + i) * 64] = o[db][i];
        }
        __syncthreads();
        if (half == 1) return;
        const float m1 = cmb[0], l1 = cmb[64];
        const float mm = fmaxf(m, m1);
        const float a0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mm);
        const float a1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
        m = mm;
        lsum = lsum * a0 + l1 * a1;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[db][i] = o[db][i] * a0 + cmb[(2 + db * 16 + i) * 64] * a1;
    }
    if (!valid) return;
    if (spl.w > 1) {
        // one split of several: (m, l, o) of this column into the item of its
        // 16-column group (16 / G rows x G heads, the decode tiles' layout);
        // attention_merge_kernel combines the splits
        const int item = spl.z + ((wq * 32 + col) >> 4) * spl.w;
        float* out = a.part + (((size_t)item * a.kv_heads + kvh) * 16 + (col & 15)) * (D + 2);
        if (h == 0) {
            out[0] = m;
            out[1] = lsum;
        }
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) out[2 + db * 32 + 8 * (i >> 2) + 4 * h + (i & 3)] = o[db][i];
        return;
    }
    const float inv = 1.0f / lsum;
    const int ocol0 = (kvh * a.G + g) * D;
    if (a.out_bf16) {
        // Lane (col, h) holds dims 32 db + 16 p + 4 h + [0, 4) (o[db][8 p + i])
        // and 32 db + 16 p + 8 + 4 h + [0, 4) (o[db][8 p + 4 + i]) of its row;
        // its partner lane (col, 1 - h) the other two quarters.  One
        // permlane32 swap per float gives lane h the 8 consecutive dims
        // 32 db + 16 p + 8 h + [0, 8), which are one 16-byte run of the
        // fragment-packed operand (hi plane, then lo): one store each instead
        // of eight 2-byte stores.  The partner has the same column, so the
        // same `valid`.
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                float x[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[db][8 * p + i] * inv),
                                                                     __float_as_uint(o[db][8 * p + 4 + i] * inv), false,
                                                                     false);
                    x[i] = __uint_as_float(sw[0]);
                    x[4 + i] = __uint_as_float(sw[1]);
                }
                const size_t oi = a_pack_index(grow, ocol0 + db * 32 + 16 * p + 8 * h, a.q_cols);
                *(bf16x8*)(a.out_bf16 + oi) = to_bf16x8(x, false);
                if (a.out_lo_offset) *(bf16x8*)(a.out_bf16 + a.out_lo_offset + oi) = to_bf16x8(x, true);
            }
        return;
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            const int d = db * 32 + 8 * i4 + 4 * h;
            const f32x4 v = {o[db][4 * i4] * inv, o[db][4 * i4 + 1] * inv, o[db][4 * i4 + 2] * inv,
                             o[db][4 * i4 + 3] * inv};
            *(f32x4*)(a.out_f32 + (size_t)grow * a.q_cols + ocol0 + d) = v;
        }
}

// Merge the splits of one (tile, kv head) with more than one split:
// o = sum_s o_s w_s with w_s = 2^(m_s - M) / sum_r l_r 2^(m_r - M), M the
// max over splits (m in log2 units).  The weights of up to kChunk splits are
// computed once per chunk into LDS; each thread then accumulates fixed
// output elements, consecutive threads reading consecutive columns.
template <int D>
__global__ __launch_bounds__(256) void attention_merge_kernel(const float* __restrict__ part,
                                                              const int4* __restrict__ merge_rec, int G,
                                                              int kv_heads, int q_cols, float* __restrict__ out,
                                                              uint16_t* __restrict__ out_bf16, size_t lo_offset) {
    constexpr int kChunk = 64;
    constexpr int kPer = 16 * D / 256;  // output elements per thread (16 columns max)
    __shared__ float sw[kChunk][16];
    __shared__ float sred[16][16];
    __shared__ float sM[16], sLinv[16];
    // {first partial, splits, first q row, nq} of the tile
    const int4 mr = merge_rec[blockIdx.x];
    const int kvh = blockIdx.y;
    const int first = mr.x, nparts = mr.y, row0 = mr.z, nq = mr.w;
    if (nq <= 0) return;  // an empty record past a replayed bucket's merges
    const int ncols = min(nq, 16 / G) * G;
    const size_t pstride = (size_t)kv_heads * 16 * (D + 2);
    const float* base = part + ((size_t)first * kv_heads + kvh) * 16 * (D + 2);
    const int tid = threadIdx.x;
    if (nparts <= 16) {
        // One round trip: thread (column tid / 16, dims D / 16 from (tid % 16) D / 16)
        // loads (m, l) and its dims of every split at once (partial rows are
        // 8-byte aligned), then combines them in registers -- the same
        // operations in the same order as the general path below.
        constexpr int DT = D / 16, P2 = DT / 2;
        const int c = tid >> 4, d0 = (tid & 15) * DT;
        if (c >= ncols) return;
        const float* pc = base + (size_t)c * (D + 2);
        float2 ml[16], ov[16][P2];
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < nparts) {
                ml[s] = *(const float2*)(pc + s * pstride);
#pragma unroll
                for (int k = 0; k < P2; ++k) ov[s][k] = *(const float2*)(pc + s * pstride + 2 + d0 + 2 * k);
            }
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < nparts) M = fmaxf(M, ml[s].x);
        float L = 0.0f;
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < nparts && ml[s].x != -INFINITY) L = L + __fmul_rn(ml[s].y, exp2f(ml[s].x - M));
        const float Linv = 1.0f / L;
        float acc[DT];
#pragma unroll
        for (int j = 0; j < DT; ++j) acc[j] = 0.0f;
#pragma unroll
        for (int s = 0; s < 16; ++s)
            if (s < nparts) {
                const float w = ml[s].x != -INFINITY ? exp2f(ml[s].x - M) * Linv : 0.0f;
#pragma unroll
                for (int k = 0; k < P2; ++k) {
                    acc[2 * k] = fmaf(ov[s][k].x, w, acc[2 * k]);
                    acc[2 * k + 1] = fmaf(ov[s][k].y, w, acc[2 * k + 1]);
                }
            }
        const int qi = c / G, g = c - qi * G;
        const int row = row0 + qi;
        if (out_bf16) {
            // the thread's DT consecutive dims (d0 a multiple of DT) are one
            // contiguous run of the fragment-packed operand: one store per plane
            static_assert(DT == 4 || DT == 8, "runs of 4 or 8 dims");
            const size_t o = a_pack_index(row, (kvh * G + g) * D + d0, q_cols);
            if constexpr (DT == 8) {
                *(bf16x8*)(out_bf16 + o) = to_bf16x8(acc, false);
                if (lo_offset) *(bf16x8*)(out_bf16 + lo_offset + o) = to_bf16x8(acc, true);
            } else {
                ushort4 hi, lo;
                split_bf16(acc[0], hi.x, lo.x);
                split_bf16(acc[1], hi.y, lo.y);
                split_bf16(acc[2], hi.z, lo.z);
                split_bf16(acc[3], hi.w, lo.w);
                *(ushort4*)(out_bf16 + o) = hi;
                if (lo_offset) *(ushort4*)(out_bf16 + lo_offset + o) = lo;
            }
        } else {
#pragma unroll
            for (int j = 0; j < DT; ++j) out[(size_t)row * q_cols + (kvh * G + g) * D + d0 + j] = acc[j];
        }
        return;
    }
    // column max over splits: 16 threads per column
    {
        const int c = tid & 15, pl = tid >> 4;
        float M = -INFINITY;
        if (c < ncols)
            for (int s = pl; s < nparts; s += 16) M = fmaxf(M, base[s * pstride + (size_t)c * (D + 2)]);
        sred[pl][c] = M;
        __syncthreads();
        if (tid < 16) {
            float m = sred[0][tid];
#pragma unroll
            for (int i = 1; i < 16; ++i) m = fmaxf(m, sred[i][tid]);
            sM[tid] = m;
        }
        __syncthreads();
        const float Mc = sM[c];
        float L = 0.0f;
        if (c < ncols)
            for (int s = pl; s < nparts; s += 16) {
                const float* ps = base + s * pstride + (size_t)c * (D + 2);
                const float mv = ps[0];
                if (mv != -INFINITY) L += ps[1] * exp2f(mv - Mc);
            }
        sred[pl][c] = L;
        __syncthreads();
        if (tid < 16) {
            float l = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) l += sred[i][tid];
            sLinv[tid] = 1.0f / l;
        }
        __syncthreads();
    }
    float acc[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) acc[j] = 0.0f;
    for (int s0 = 0; s0 < nparts; s0 += kChunk) {
        const int ns = min(kChunk, nparts - s0);
        for (int t = tid; t < ns * 16; t += 256) {
            const int s = t >> 4, c = t & 15;
            float w = 0.0f;
            if (c < ncols) {
                const float mv = base[(s0 + s) * pstride + (size_t)c * (D + 2)];
                if (mv != -INFINITY) w = exp2f(mv - sM[c]) * sLinv[c];
            }
            sw[s][c] = w;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int e = tid + j * 256;
            const int c = e / D, d = e - c * D;
            if (c < ncols) {
                const float* ps = base + (size_t)s0 * pstride + (size_t)c * (D + 2) + 2 + d;
                float v = acc[j];
                for (int s = 0; s < ns; ++s) v += ps[s * pstride] * sw[s][c];
                acc[j] = v;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * 256;
        const int c = e / D, d = e - c * D;
        if (c >= ncols) continue;
        const int qi = c / G, g = c - qi * G;
        const int row = row0 + qi;
        const int col = (kvh * G + g) * D + d;
        if (out_bf16) {
            uint16_t hi, lo;
            split_bf16(acc[j], hi, lo);
            const size_t o = a_pack_index(row, col, q_cols);
            out_bf16[o] = hi;
            if (lo_offset) out_bf16[lo_offset + o] = lo;
        } else {
            out[(size_t)row * q_cols + col] = acc[j];
        }
    }
}

template <typename KV, int D>
static zr_status launch_attn_t(zr_context* ctx, StagedMeta* st, int layer, const float* q, float* out,
                               uint16_t* out_bf16, const Slabs* qkv = nullptr, int rope = 0) {
    AttnArgs a;
    a.q = q;
    a.qkv = qkv ? qkv->ptr : nullptr;
    a.qkv_n = qkv ? qkv->n : 1;
    a.qkv_slab = qkv ? qkv->stride : 0;
    a.qkv_stride = ctx->q_cols + 2 * ctx->kv_cols;
    a.kv_cols = ctx->kv_cols;
    a.slot = st->slot_mapping;
    a.rope_cs = rope ? st->rope_cs : nullptr;
    a.q_cols = ctx->q_cols;
    a.page_elems = (size_t)2 * ctx->kv_cols * kPageRows;
    a.pool = (const KV*)ctx->kv_pool + (size_t)layer * ctx->n_pages * a.page_elems;
    a.block_tables = st->block_tables;
    a.stride = st->stride;
    a.rec = st->attn_rec;
    a.n_items = st->grid_items;
    a.G = ctx->q_per_kv;
    a.kv_heads = ctx->local_kv_heads;
    a.scale_log2 = 1.4426950408889634f / sqrtf((float)D);
    a.part = ctx->attn_part;
    a.out_f32 = out;
    a.out_bf16 = out_bf16;
    a.out_lo_offset = (ctx->desc.flags & ZR_FLAG_SPLIT_ACTIVATIONS) ? a_plane(st->total_q, ctx->q_cols) : 0;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassAttention, &ev);
    if (st->grid_items > 0) {
        // bf16 pages: a 6-page ring, one wave per SIMD (measured: a 4-page ring
        // at two waves per SIMD spills and loses ~20%); f32 pages: 4 pages
        const dim3 grid(((st->grid_items + 7) / 8) * 8 * ctx->local_kv_heads);
        if (qkv)
            hipLaunchKernelGGL((paged_attention_kernel<KV, D, sizeof(KV) == 4 ? 4 : 6, true>), grid, dim3(64), 0,
                               ctx->stream, a);
        else
            hipLaunchKernelGGL((paged_attention_kernel<KV, D, sizeof(KV) == 4 ? 4 : 6, false>), grid, dim3(64), 0,
                               ctx->stream, a);
        ZR_LAUNCH_CHECK(ctx);
    }
    if constexpr (sizeof(KV) == 2) {
        if (st->n_pblocks > 0) {
            PrefillArgs pa;
            pa.q = q;
            pa.q_cols = a.q_cols;
            pa.pool = (const uint16_t*)a.pool;
            pa.page_elems = a.page_elems;
            pa.stride = a.stride;
            pa.first_offset = st->first_offset;
            pa.kv_before = st->kv_before;
            pa.cu_q = st->cu_q;
            pa.blocks = st->pblocks;
            pa.splits = st->psplits;
            pa.n_blocks = st->n_pblocks;
            pa.part = ctx->attn_part;
            pa.G = a.G;
            pa.kv_heads = a.kv_heads;
            pa.scale_log2 = a.scale_log2;
            pa.out_f32 = out;
            pa.out_bf16 = out_bf16;
            pa.out_lo_offset = a.out_lo_offset;
            // one workgroup per (block, kv head): kv head = block index mod kv_heads, so
            // with kv_heads dividing 8 a kv head's pages stay on the XCDs it maps to
            if (st->prefill_kh == 2)
                hipLaunchKernelGGL((paged_prefill_attention_kernel<D, 4, 2>), dim3(st->n_pblocks * ctx->local_kv_heads),
                                   dim3(512), 0, ctx->stream, pa, st->block_tables);
            else
                hipLaunchKernelGGL((paged_prefill_attention_kernel<D, 4, 1>), dim3(st->n_pblocks * ctx->local_kv_heads),
                                   dim3(256), 0, ctx->stream, pa, st->block_tables);
            ZR_LAUNCH_CHECK(ctx);
        }
    }
    timing_mark_end(ctx, kClassAttention, ev);
    if (st->grid_merge > 0) {
        timing_mark_begin(ctx, kClassOther, &ev);
        hipLaunchKernelGGL((attention_merge_kernel<D>), dim3(st->grid_merge, ctx->local_kv_heads), dim3(256), 0,
                           ctx->stream, ctx->attn_part, st->merge_rec, ctx->q_per_kv, ctx->local_kv_heads,
                           ctx->q_cols, out, out_bf16, a.out_lo_offset);
        ZR_LAUNCH_CHECK(ctx);
        timing_mark_end(ctx, kClassOther, ev);
    }
    return ZR_OK;
}

// ------------------------------------------------------- any head_dim
// Pools in the plain layout (head_dim other than 64 / 128, or q heads per kv
// head not dividing 16): one wave per (query row, q head).  The wave walks
// the visible keys 64 at a time (a key per lane: the lane's score over D from
// its K row; rows of a page are contiguous), keeps an online softmax across
// the wave and accumulates P.V with lanes over the dims (up to 4 per lane).
// Row i of a sequence with `prefix` cached rows sees keys [0, prefix + i]: a
// decode row sees its whole window, a prefill chunk the causal prefix
// (forward_pass.rs:2764-2895, 1317-1372).
struct GenericAttnArgs {
    const float* q;
    int q_cols;
    const void* pool;          // layer base of the pool
    size_t page_elems;
    const int* block_tables;
    int stride;
    const int* first_offset;
    const int* kv_before;
    const int* cu_q;
    const int* seq_ids;
    int D, G, kv_heads;
    float scale;               // 1 / sqrt(D)
    float* out_f32;
    uint16_t* out_bf16;
    size_t out_lo_offset;
};

__device__ inline float load_kv(const float* p) { return *p; }
__device__ inline float load_kv(const uint16_t* p) { return bf16_bits_to_f32(*p); }

__device__ inline float wave_max64(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ inline float wave_sum64(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <typename KV>
__global__ __launch_bounds__(64) void paged_attention_generic_kernel(GenericAttnArgs a) {
    __shared__ float qs[256];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int D = a.D;
    const int s = a.seq_ids[t];
    const int i = t - a.cu_q[s];
    const int L = a.kv_before[s] + i + 1;
    const int fo = a.first_offset[s];
    const int* bt = a.block_tables + (size_t)s * a.stride;
    const int kvh = h / a.G;
    const KV* pool = (const KV*)a.pool;
    const size_t k_head = (size_t)kvh * kPageRows * D;
    const size_t v_head = (size_t)a.kv_heads * kPageRows * D + k_head;
    for (int d = lane; d < D; d += 64) qs[d] = a.q[(size_t)t * a.q_cols + h * D + d];
    __syncthreads();
    float m = -INFINITY, l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < L; k0 += 64) {
        const int key = k0 + lane;
        float sc = -INFINITY;
        if (key < L) {
            const int row = fo + key;
            const KV* kr = pool + (size_t)bt[row / kPageRows] * a.page_elems + k_head + (size_t)(row % kPageRows) * D;
            float acc = 0.0f;
            for (int d = 0; d < D; ++d) acc += qs[d] * load_kv(kr + d);
            sc = acc * a.scale;
        }
        const float mn = fmaxf(m, wave_max64(sc));  // finite: key k0 is visible
        const float alpha = expf(m - mn);           // 0 on the first chunk (m = -inf)
        const float p = key < L ? expf(sc - mn) : 0.0f;
        l = l * alpha + wave_sum64(p);
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] *= alpha;
        const int nk = min(64, L - k0);
        for (int kk = 0; kk < nk; ++kk) {
            const float pk = __shfl(p, kk, 64);
            const int row = fo + k0 + kk;
            const KV* vr = pool + (size_t)bt[row / kPageRows] * a.page_elems + v_head + (size_t)(row % kPageRows) * D;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (lane + 64 * j < D) o[j] += pk * load_kv(vr + lane + 64 * j);
        }
        m = mn;
    }
    const float inv_l = 1.0f / l;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = lane + 64 * j;
        if (d >= D) continue;
        const float y = o[j] * inv_l;
        const int c = h * D + d;
        if (a.out_bf16) {
            uint16_t hi, lo;
            split_bf16(y, hi, lo);
            const size_t idx = a_pack_index(t, c, a.q_cols);
            a.out_bf16[idx] = hi;
            if (a.out_lo_offset) a.out_bf16[a.out_lo_offset + idx] = lo;
        } else {
            a.out_f32[(size_t)t * a.q_cols + c] = y;
        }
    }
}

template <typename KV>
static zr_status launch_attn_generic(zr_context* ctx, StagedMeta* st, int layer, const float* q, float* out,
                                     uint16_t* out_bf16) {
    GenericAttnArgs a;
    a.q = q;
    a.q_cols = ctx->q_cols;
    a.page_elems = (size_t)2 * ctx->kv_cols * kPageRows;
    a.pool = (const KV*)ctx->kv_pool + (size_t)layer * ctx->n_pages * a.page_elems;
    a.block_tables = st->block_tables;
    a.stride = st->stride;
    a.first_offset = st->first_offset;
    a.kv_before = st->kv_before;
    a.cu_q = st->cu_q;
    a.seq_ids = st->seq_ids;
    a.D = ctx->head_dim;
    a.G = ctx->q_per_kv;
    a.kv_heads = ctx->local_kv_heads;
    a.scale = 1.0f / sqrtf((float)ctx->head_dim);
    a.out_f32 = out;
    a.out_bf16 = out_bf16;
    a.out_lo_offset = (ctx->desc.flags & ZR_FLAG_SPLIT_ACTIVATIONS) ? a_plane(st->total_q, ctx->q_cols) : 0;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassAttention, &ev);
    hipLaunchKernelGGL(paged_attention_generic_kernel<KV>, dim3(st->total_q, ctx->local_q_heads), dim3(64), 0,
                       ctx->stream, a);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassAttention, ev);
    return ZR_OK;
}

// XOR of every 32-bit word a page set holds (keeps the probe's loads live)
__device__ inline unsigned xor4(uint4 w) { return w.x ^ w.y ^ w.z ^ w.w; }
template <int D>
__device__ inline unsigned page_fold(const PageRegs<uint16_t, D>& r) {
    unsigned x = 0;
#pragma unroll
    for (int b = 0; b < D / 32; ++b) x ^= xor4(__builtin_bit_cast(uint4, r.k[b])) ^ xor4(__builtin_bit_cast(uint4, r.v[b]));
    return x;
}
template <int D>
__device__ inline unsigned page_fold(const PageRegs<float, D>& r) {
    unsigned x = 0;
#pragma unroll
    for (int b = 0; b < D / 32; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            x ^= xor4(__builtin_bit_cast(uint4, r.k[b][h])) ^ xor4(__builtin_bit_cast(uint4, r.v[b][h]));
    return x;
}

// Read-only twin of paged_attention_kernel's page stream, for measuring the
// HBM rate its access pattern can reach: the same grid and block -> (item,
// kv head) mapping, the same work records and block tables, the same
// nontemporal 16-byte loads of each page's K and V tiles through a ring of
// RING page sets loaded in the same order (the first RING - 2 from the
// record, then two ahead per pair), and no Q, softmax, MFMA or output: each
// page set is folded into one XOR word, and each workgroup writes one.
template <typename KV, int D, int RING>
__global__ __launch_bounds__(64) void kv_read_probe_kernel(AttnArgs a, unsigned* out) {
    const int lane = threadIdx.x;
    const int per_grp = 8 * a.kv_heads;
    const int rem = blockIdx.x % per_grp;
    const int kvh = rem >> 3;
    const int rank = (blockIdx.x / per_grp) * 8 + (rem & 7);
    unsigned acc = 0;
    if (rank < a.n_items) {
        const int4 r0 = a.rec[3 * rank], r1 = a.rec[3 * rank + 1], r2 = a.rec[3 * rank + 2];
        const int seq = r0.x, nq = r0.z, page_b = r0.w, page_e = r1.x;
        if (nq > 0) {
            const KV* pool = (const KV*)a.pool;
            const int* bt = a.block_tables + (size_t)seq * a.stride;
            const size_t kv_tile = (size_t)kPageRows * D;
            const size_t v_block = (size_t)a.kv_heads * kv_tile;
            PageRegs<KV, D> ring[RING];
            auto load_page = [&](PageRegs<KV, D>& r, int pool_page) {
                const KV* base = pool + (size_t)pool_page * a.page_elems + (size_t)kvh * kv_tile;
                r.load(base, base + v_block, lane);
            };
            auto load_or_shared = [&](PageRegs<KV, D>& r, int p) {
                const int pg = bt[min(p, page_e - 1)];
                load_page(r, p < page_e ? pg : 0);
            };
            auto fold = [&](const PageRegs<KV, D>& r) { acc ^= page_fold(r); };
            static_assert(RING - 2 <= 4, "the record holds the first 4 pages");
            const int first_pages[4] = {r2.x, r2.y, r2.z, r2.w};
#pragma unroll
            for (int r = 0; r < RING - 2; ++r) load_page(ring[r], first_pages[r]);
            for (int p = page_b; p < page_e; p += RING) {
#pragma unroll
                for (int r = 0; r < RING; r += 2) {
                    const int pp = p + r;
                    if (pp >= page_e) break;
                    load_or_shared(ring[(r + RING - 2) % RING], pp + RING - 2);
                    load_or_shared(ring[(r + RING - 1) % RING], pp + RING - 1);
                    fold(ring[r]);
                    if (pp + 1 < page_e) fold(ring[r + 1]);
                }
            }
        }
    }
    if (lane == 0) out[blockIdx.x] = acc;
}

template <typename KV, int D>
static zr_status launch_kv_read_probe_t(zr_context* ctx, StagedMeta* st, int layer, int repeats, double* mean_ms) {
    AttnArgs a{};
    a.page_elems = (size_t)2 * ctx->kv_cols * kPageRows;
    a.pool = (const KV*)ctx->kv_pool + (size_t)layer * ctx->n_pages * a.page_elems;
    a.block_tables = st->block_tables;
    a.stride = st->stride;
    a.rec = st->attn_rec;
    a.n_items = st->grid_items;
    a.kv_heads = ctx->local_kv_heads;
    const dim3 grid(((st->grid_items + 7) / 8) * 8 * ctx->local_kv_heads);
    // one word per workgroup, in the attention partials' workspace
    if ((size_t)grid.x > ctx->attn_part_floats)
        return set_err(ctx, ZR_E_OOM, "attention partial workspace too small for %u probe words", grid.x);
    hipEvent_t e0, e1;
    ZR_HIP(ctx, hipEventCreate(&e0));
    hipError_t e = hipEventCreate(&e1);
    if (e != hipSuccess) {
        (void)hipEventDestroy(e0);
        return set_err(ctx, ZR_E_HIP, "hipEventCreate: %s", hipGetErrorString(e));
    }
    e = hipEventRecord(e0, ctx->stream);
    for (int i = 0; i < repeats && e == hipSuccess; ++i) {
        hipLaunchKernelGGL((kv_read_probe_kernel<KV, D, sizeof(KV) == 4 ? 4 : 6>), grid, dim3(64), 0, ctx->stream, a,
                           (unsigned*)ctx->attn_part);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(e1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (e != hipSuccess) return set_err(ctx, ZR_E_HIP, "KV read probe: %s", hipGetErrorString(e));
    *mean_ms = (double)ms / repeats;
    return ZR_OK;
}

zr_status launch_kv_read_probe(zr_context* ctx, StagedMeta* st, int layer, int repeats, double* mean_ms) {
    if (ctx->plain_kv || (ctx->head_dim != 64 && ctx->head_dim != 128))
        return set_err(ctx, ZR_E_UNSUPPORTED, "the KV read probe follows the MFMA page layout (head_dim 64 or 128)");
    if (st->grid_items == 0) return set_err(ctx, ZR_E_INVALID, "the staged microbatch has no decode attention items");
    const bool bf = ctx->desc.kv_dtype == ZR_DTYPE_BF16;
    if (ctx->head_dim == 64)
        return bf ? launch_kv_read_probe_t<uint16_t, 64>(ctx, st, layer, repeats, mean_ms)
                  : launch_kv_read_probe_t<float, 64>(ctx, st, layer, repeats, mean_ms);
    return bf ? launch_kv_read_probe_t<uint16_t, 128>(ctx, st, layer, repeats, mean_ms)
              : launch_kv_read_probe_t<float, 128>(ctx, st, layer, repeats, mean_ms);
}

zr_status launch_attention(zr_context* ctx, StagedMeta* st, int layer, const float* q, float* out,
                           uint16_t* out_bf16) {
    if (st->total_q == 0) return ZR_OK;
    if (ctx->plain_kv) {
        if (ctx->head_dim > 256) return set_err(ctx, ZR_E_UNSUPPORTED, "head_dim %d above 256", ctx->head_dim);
        return ctx->desc.kv_dtype == ZR_DTYPE_BF16
                   ? launch_attn_generic<uint16_t>(ctx, st, layer, q, out, out_bf16)
                   : launch_attn_generic<float>(ctx, st, layer, q, out, out_bf16);
    }
    if (st->grid_items == 0 && st->n_pblocks == 0) return ZR_OK;
    const size_t need = (size_t)st->n_part_items * ctx->local_kv_heads * 16 * (ctx->head_dim + 2);
    if (need > ctx->attn_part_floats)
        return set_err(ctx, ZR_E_OOM, "attention partial workspace too small: need %zu floats, have %zu",
                       need, ctx->attn_part_floats);
    zr_status rc;
    const bool bf = ctx->desc.kv_dtype == ZR_DTYPE_BF16;
    switch (ctx->head_dim) {
        case 64: rc = bf ? launch_attn_t<uint16_t, 64>(ctx, st, layer, q, out, out_bf16) : launch_attn_t<float, 64>(ctx, st, layer, q, out, out_bf16); break;
        case 128: rc = bf ? launch_attn_t<uint16_t, 128>(ctx, st, layer, q, out, out_bf16) : launch_attn_t<float, 128>(ctx, st, layer, q, out, out_bf16); break;
        default: return set_err(ctx, ZR_E_UNSUPPORTED, "head_dim %d not supported (64, 128)", ctx->head_dim);
    }
    return rc;
}

zr_status launch_attention_rope(zr_context* ctx, StagedMeta* st, int layer, const Slabs& qkv, int rope,
                                float* out, uint16_t* out_bf16) {
    if (!st->pure_decode)
        return set_err(ctx, ZR_E_UNSUPPORTED, "RoPE inside attention needs a microbatch of one-row decode sequences");
    if (st->grid_items == 0) return ZR_OK;
    const size_t need = (size_t)st->n_part_items * ctx->local_kv_heads * 16 * (ctx->head_dim + 2);
    if (need > ctx->attn_part_floats)
        return set_err(ctx, ZR_E_OOM, "attention partial workspace too small: need %zu floats, have %zu",
                       need, ctx->attn_part_floats);
    const bool bf = ctx->desc.kv_dtype == ZR_DTYPE_BF16;
    switch (ctx->head_dim) {  // pure_decode implies the MFMA page layout: head_dim 64 or 128
        case 64:
            return bf ? launch_attn_t<uint16_t, 64>(ctx, st, layer, nullptr, out, out_bf16, &qkv, rope)
                      : launch_attn_t<float, 64>(ctx, st, layer, nullptr, out, out_bf16, &qkv, rope);
        case 128:
            return bf ? launch_attn_t<uint16_t, 128>(ctx, st, layer, nullptr, out, out_bf16, &qkv, rope)
                      : launch_attn_t<float, 128>(ctx, st, layer, nullptr, out, out_bf16, &qkv, rope);
        default: return set_err(ctx, ZR_E_UNSUPPORTED, "head_dim %d not supported (64, 128)", ctx->head_dim);
    }
}

}  // namespace zr
