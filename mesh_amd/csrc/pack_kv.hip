// Ragged-batch packing, fused RoPE + paged-KV append, and the KV handoff
// gather/scatter kernels.  The KV pool's page layouts (MFMA fragment, with
// f32 pools' page_order, and plain) are k_off / v_off / page_order /
// k_off_of / v_off_of in zr_internal.h.
#include "zr_internal.h"

namespace zr {

// ------------------------------------------------------------------ pack
// One workgroup: exclusive scans of q_len and kv_after, then per-token
// positions / slot mapping / sequence ids
// (DecodeWorkspaceLease::stage_with_slot_reader, fast_path.rs:263-338;
// PrefillWorkspaceLease::stage_positions, fast_path.rs:409-445).
__global__ __launch_bounds__(1024) void pack_kernel(int S, const int* __restrict__ q_len,
                                                    const int* __restrict__ kv_before,
                                                    const int* __restrict__ first_pos,
                                                    const int* __restrict__ first_offset,
                                                    const int* __restrict__ bt, int stride,
                                                    int* __restrict__ cu_q, int* __restrict__ cu_k,
                                                    int* __restrict__ positions, int* __restrict__ slot,
                                                    int* __restrict__ seq_ids, int* __restrict__ last_rows) {
    __shared__ int sq[1024], sk[1024];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int per = (S + nt - 1) / nt;
    const int s0 = tid * per, s1 = min(S, s0 + per);
    int lq = 0, lk = 0;
    for (int s = s0; s < s1; ++s) {
        lq += q_len[s];
        lk += kv_before[s] + q_len[s];
    }
    sq[tid] = lq;
    sk[tid] = lk;
    __syncthreads();
    // Hillis-Steele inclusive scan over the per-thread sums
    for (int off = 1; off < nt; off <<= 1) {
        int aq = tid >= off ? sq[tid - off] : 0;
        int ak = tid >= off ? sk[tid - off] : 0;
        __syncthreads();
        sq[tid] += aq;
        sk[tid] += ak;
        __syncthreads();
    }
    int bq = sq[tid] - lq, bk = sk[tid] - lk;
    if (tid == 0) {
        cu_q[0] = 0;
        cu_k[0] = 0;
    }
    for (int s = s0; s < s1; ++s) {
        bq += q_len[s];
        bk += kv_before[s] + q_len[s];
        cu_q[s + 1] = bq;
        cu_k[s + 1] = bk;
        last_rows[s] = bq - 1;
    }
    __syncthreads();
    __threadfence_block();
    const int total = sq[nt - 1];
    for (int t = tid; t < total; t += nt) {
        // binary search: largest s with cu_q[s] <= t
        int lo = 0, hi = S - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (cu_q[mid] <= t) lo = mid; else hi = mid - 1;
        }
        const int s = lo, i = t - cu_q[s];
        const int row = first_offset[s] + kv_before[s] + i;
        positions[t] = first_pos[s] + i;
        slot[t] = bt[(size_t)s * stride + row / kPageRows] * kPageRows + row % kPageRows;
        seq_ids[t] = s;
    }
}

// RoPE angles of the step, shared by every layer: (cos, sin) of
// theta = f32(position) * inv_freq[i] in f32 (tensor_ops.rs:509-560,
// runtime.rs:935-1005), one entry per (row, rotation pair).
__global__ __launch_bounds__(256) void rope_table_kernel(int rows, int half, const int* __restrict__ positions,
                                                         const float* __restrict__ inv_freq, float2* __restrict__ cs) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * half) return;
    const int t = idx / half, i = idx - t * half;
    const float theta = (float)positions[t] * inv_freq[i];
    cs[idx] = make_float2(cosf(theta), sinf(theta));
}

zr_status launch_pack(zr_context* ctx, StagedMeta* st) {
    hipLaunchKernelGGL(pack_kernel, dim3(1), dim3(1024), 0, ctx->stream, st->num_seqs, st->q_len,
                       st->kv_before, st->first_pos, st->first_offset, st->block_tables, st->stride,
                       st->cu_q, st->cu_k, st->positions, st->slot_mapping, st->seq_ids, st->last_rows);
    ZR_LAUNCH_CHECK(ctx);
    const int half = ctx->head_dim / 2, n = st->total_q * half;
    if (n > 0) {
        hipLaunchKernelGGL(rope_table_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, st->total_q, half,
                           st->positions, ctx->inv_freq, st->rope_cs);
        ZR_LAUNCH_CHECK(ctx);
    }
    return ZR_OK;
}

// ---------------------------------------------------------- RoPE + append
// One workgroup per token row.  RoPE follows tensor_ops.rs:509-560 /
// runtime.rs:935-1005 (rotate-half; (cos, sin) of theta = position * inv_freq
// in f32 from the step's table, rope_table_kernel) and the KV append is
// DeviceLayerKVCache::append (forward_pass.rs:462-521) at the slot the host
// reserved.
constexpr int kSlabsAhead = 16;  // split-K slabs whose loads go out together (the GEMM splits at most 16 ways)

template <typename KV>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(
    const float* __restrict__ qkv, int qkv_n, size_t qkv_slab, int qkv_stride, float* __restrict__ q_out,
    int q_cols, int kv_cols,
    int D, const int* __restrict__ slot, const float2* __restrict__ rope_cs,
    KV* __restrict__ layer_pool, size_t page_elems, int rope, int plain) {
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    const int half = D / 2;
    const float* row = qkv + (size_t)t * qkv_stride;
    const int s = slot[t];
    const int page = s / kPageRows, r = s % kPageRows;
    KV* kpage = layer_pool + (size_t)page * page_elems;
    const int kv_heads = kv_cols / D;
    KV* vpage = kpage + (size_t)kv_heads * kPageRows * D;
    // q: q_cols / 2 rotation pairs, k: kv_cols / 2 pairs, v: kv_cols copies
    const int nq = q_cols / 2, nk = kv_cols / 2;
    for (int j = blockIdx.y * blockDim.x + threadIdx.x; j < nq + nk + kv_cols; j += gridDim.y * blockDim.x) {
        if (j < nq + nk) {
            const bool is_q = j < nq;
            const int jj = is_q ? j : j - nq;
            const int head = jj / half, i = jj % half;
            const float* src = row + (is_q ? 0 : q_cols) + head * D;
            // every slab's pair (up to kSlabsAhead) and the (cos, sin) are
            // loaded before the first add: one round trip, summed in slab order
            const float2 cs = rope ? rope_cs[(size_t)t * half + i] : make_float2(1.f, 0.f);
            float la[kSlabsAhead], lb[kSlabsAhead];
#pragma unroll
            for (int sl = 0; sl < kSlabsAhead; ++sl)
                if (sl < qkv_n) {
                    la[sl] = src[sl * qkv_slab + i];
                    lb[sl] = src[sl * qkv_slab + i + half];
                }
            float a = la[0], b = lb[0];
#pragma unroll
            for (int sl = 1; sl < kSlabsAhead; ++sl)
                if (sl < qkv_n) {
                    a += la[sl];
                    b += lb[sl];
                }
            for (int sl = kSlabsAhead; sl < qkv_n; ++sl) {
                a += src[sl * qkv_slab + i];
                b += src[sl * qkv_slab + i + half];
            }
            if (rope) {
                const float c = cs.x, sn = cs.y;
                const float na = a * c - b * sn;
                const float nb = a * sn + b * c;
                a = na;
                b = nb;
            }
            if (is_q) {
                q_out[(size_t)t * q_cols + head * D + i] = a;
                q_out[(size_t)t * q_cols + head * D + i + half] = b;
            } else {
                KV* kt = kpage + (size_t)head * kPageRows * D;
                store_elem(kt + k_off_of<KV>(r, i, D, plain), a);
                store_elem(kt + k_off_of<KV>(r, i + half, D, plain), b);
            }
        } else {
            const int c = j - nq - nk;
            const int head = c / D, d = c % D;
            KV* vt = vpage + (size_t)head * kPageRows * D;
            const float* src = row + q_cols + kv_cols + c;
            float lv[kSlabsAhead];
#pragma unroll
            for (int sl = 0; sl < kSlabsAhead; ++sl)
                if (sl < qkv_n) lv[sl] = src[sl * qkv_slab];
            float vv = lv[0];
#pragma unroll
            for (int sl = 1; sl < kSlabsAhead; ++sl)
                if (sl < qkv_n) vv += lv[sl];
            for (int sl = kSlabsAhead; sl < qkv_n; ++sl) vv += src[sl * qkv_slab];
            store_elem(vt + v_off_of<KV>(r, d, D, plain), vv);
        }
    }
}

// The same stage for head_dim % 8 == 0 in float4 runs, one item per lane of
// one-wave workgroups (row, y): 4 consecutive rotation pairs of one q / k
// head -- float4 loads of both halves from every split-K slab, issued 8 slabs
// at a time and summed in slab order, and the lane's own 4 (cos, sin) pairs
// from the table loaded while they are in flight -- or 4 consecutive V
// elements.  Bit-identical to the scalar kernel.
template <typename KV>
__global__ __launch_bounds__(64) void rope_kv_write_vec_kernel(
    const float* __restrict__ qkv, int qkv_n, size_t qkv_slab, int qkv_stride, float* __restrict__ q_out,
    int q_cols, int kv_cols,
    int D, const int* __restrict__ slot, const float2* __restrict__ rope_cs,
    KV* __restrict__ layer_pool, size_t page_elems, int rope, int plain) {
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    const int half = D / 2, g4 = half / 4;
    const int kv_heads = kv_cols / D, q_heads = q_cols / D;
    const int n_rot = (q_heads + kv_heads) * g4, n_v = kv_cols / 4;
    const int j = blockIdx.y * blockDim.x + threadIdx.x;
    if (j >= n_rot + n_v) return;
    const float* row = qkv + (size_t)t * qkv_stride;
    const int s = slot[t];
    const int page = s / kPageRows, r = s % kPageRows;
    KV* kpage = layer_pool + (size_t)page * page_elems;
    KV* vpage = kpage + (size_t)kv_heads * kPageRows * D;
    auto add4 = [](float4& x, const float4& y) {
        x.x += y.x;
        x.y += y.y;
        x.z += y.z;
        x.w += y.w;
    };
    if (j < n_rot) {
        const int head = j / g4, i0 = (j - head * g4) * 4;
        const bool is_q = head < q_heads;
        const int hh = is_q ? head : head - q_heads;
        const float* src = row + (is_q ? 0 : q_cols) + hh * D + i0;
        float4 a4 = *(const float4*)src, b4 = *(const float4*)(src + half);
        float c[4] = {1.f, 1.f, 1.f, 1.f}, sv[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 1; s0 < qkv_n; s0 += 8) {
            float4 qa[8], qb[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const bool ok = s0 + u < qkv_n;
                qa[u] = ok ? *(const float4*)(src + (s0 + u) * qkv_slab) : make_float4(0.f, 0.f, 0.f, 0.f);
                qb[u] = ok ? *(const float4*)(src + (s0 + u) * qkv_slab + half) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
            if (rope && s0 == 1) {
                const float4* cs4 = (const float4*)(rope_cs + (size_t)t * half + i0);
                const float4 p0 = cs4[0], p1 = cs4[1];
                c[0] = p0.x, sv[0] = p0.y, c[1] = p0.z, sv[1] = p0.w;
                c[2] = p1.x, sv[2] = p1.y, c[3] = p1.z, sv[3] = p1.w;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s0 + u < qkv_n) {
                    add4(a4, qa[u]);
                    add4(b4, qb[u]);
                }
        }
        if (rope && qkv_n == 1) {
            const float4* cs4 = (const float4*)(rope_cs + (size_t)t * half + i0);
            const float4 p0 = cs4[0], p1 = cs4[1];
            c[0] = p0.x, sv[0] = p0.y, c[1] = p0.z, sv[1] = p0.w;
            c[2] = p1.x, sv[2] = p1.y, c[3] = p1.z, sv[3] = p1.w;
        }
        float a[4] = {a4.x, a4.y, a4.z, a4.w}, b[4] = {b4.x, b4.y, b4.z, b4.w};
        if (rope) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float na = a[u] * c[u] - b[u] * sv[u];
                const float nb = a[u] * sv[u] + b[u] * c[u];
                a[u] = na;
                b[u] = nb;
            }
        }
        if (is_q) {
            float* qo = q_out + (size_t)t * q_cols + hh * D + i0;
            *(float4*)qo = make_float4(a[0], a[1], a[2], a[3]);
            *(float4*)(qo + half) = make_float4(b[0], b[1], b[2], b[3]);
        } else {
            KV* kt = kpage + (size_t)hh * kPageRows * D;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                store_elem(kt + k_off_of<KV>(r, i0 + u, D, plain), a[u]);
                store_elem(kt + k_off_of<KV>(r, half + i0 + u, D, plain), b[u]);
            }
        }
    } else {
        const int cidx = (j - n_rot) * 4;
        const int head = cidx / D, d = cidx - head * D;
        KV* vt = vpage + (size_t)head * kPageRows * D;
        const float* src = row + q_cols + kv_cols + cidx;
        float4 v4 = *(const float4*)src;
        for (int s0 = 1; s0 < qkv_n; s0 += 8) {
            float4 q[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                q[u] = s0 + u < qkv_n ? *(const float4*)(src + (s0 + u) * qkv_slab) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s0 + u < qkv_n) add4(v4, q[u]);
        }
        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) store_elem(vt + v_off_of<KV>(r, d + u, D, plain), vv[u]);
    }
}

static inline size_t page_elems_of(const zr_context* ctx) {
    return (size_t)2 * ctx->kv_cols * kPageRows;
}

zr_status launch_rope_kv_write(zr_context* ctx, StagedMeta* st, int layer, const Slabs& qkv,
                               float* q_out, int rope) {
    if (st->total_q == 0) return ZR_OK;
    const size_t pe = page_elems_of(ctx);
    const int stride = ctx->q_cols + 2 * ctx->kv_cols;
    // one thread per rotation pair / V element: q_cols / 2 + kv_cols / 2 + kv_cols per token
    const int items = ctx->q_cols / 2 + ctx->kv_cols / 2 + ctx->kv_cols;
    const dim3 grid(st->total_q, (items + 255) / 256);
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassNormRopeKv, &ev);
    // float4 runs need 4 | D / 2 and 16 B aligned rows and slabs.  Measured
    // on the decode steps: at 256 rows the float4 kernel takes 4 % off the
    // norm / RoPE class; at 32 rows (16 split-K slabs) one pair per thread,
    // spread over 4x more waves, is 2 % faster per step.
    const bool vec = ctx->head_dim % 8 == 0 && stride % 4 == 0 && qkv.stride % 4 == 0 && st->total_q >= 128;
    if (vec) {
        // one float4 item per lane: (q + kv heads) x D / 8 rotations + kv_cols / 4 V runs per row,
        // one-wave workgroups so that small batches still spread over the CUs
        const int vitems = (ctx->q_cols + ctx->kv_cols) / 8 + ctx->kv_cols / 4;
        const dim3 vgrid(st->total_q, (vitems + 63) / 64);
        if (ctx->desc.kv_dtype == ZR_DTYPE_BF16)
            hipLaunchKernelGGL(rope_kv_write_vec_kernel<uint16_t>, vgrid, dim3(64), 0, ctx->stream,
                               qkv.ptr, qkv.n, qkv.stride, stride, q_out, ctx->q_cols, ctx->kv_cols, ctx->head_dim,
                               st->slot_mapping, st->rope_cs,
                               (uint16_t*)ctx->kv_pool + (size_t)layer * ctx->n_pages * pe, pe, rope,
                               ctx->plain_kv ? 1 : 0);
        else
            hipLaunchKernelGGL(rope_kv_write_vec_kernel<float>, vgrid, dim3(64), 0, ctx->stream,
                               qkv.ptr, qkv.n, qkv.stride, stride, q_out, ctx->q_cols, ctx->kv_cols, ctx->head_dim,
                               st->slot_mapping, st->rope_cs,
                               (float*)ctx->kv_pool + (size_t)layer * ctx->n_pages * pe, pe, rope,
                               ctx->plain_kv ? 1 : 0);
    } else if (ctx->desc.kv_dtype == ZR_DTYPE_BF16) {
        uint16_t* pool = (uint16_t*)ctx->kv_pool + (size_t)layer * ctx->n_pages * pe;
        hipLaunchKernelGGL(rope_kv_write_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream,
                           qkv.ptr, qkv.n, qkv.stride, stride, q_out, ctx->q_cols, ctx->kv_cols, ctx->head_dim,
                           st->slot_mapping, st->rope_cs, pool, pe, rope, ctx->plain_kv ? 1 : 0);
    } else {
        float* pool = (float*)ctx->kv_pool + (size_t)layer * ctx->n_pages * pe;
        hipLaunchKernelGGL(rope_kv_write_kernel<float>, grid, dim3(256), 0, ctx->stream,
                           qkv.ptr, qkv.n, qkv.stride, stride, q_out, ctx->q_cols, ctx->kv_cols, ctx->head_dim,
                           st->slot_mapping, st->rope_cs, pool, pe, rope, ctx->plain_kv ? 1 : 0);
    }
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassNormRopeKv, ev);
    return ZR_OK;
}

// ------------------------------------------------------ gather / scatter
// Logical window row j of a sequence lives at physical row first_offset + j of
// its page list (interior spans are full pages; only the first span may start
// mid-page after retain_suffix).  One workgroup per (page of the range, layer)
// moves the page's K block, then its V block, through an LDS tile that holds
// the page's 16 rows row-major in the pool dtype, each row padded by 16 B:
//   row side:  whole rows as float4 runs (the block's 16 rows are contiguous
//              in the [layers][rows][kv_cols] f32 arrays);
//   page side: the block's 8-element groups, contiguous in the pool layout
//              (16 B in bf16 pools), consecutive threads on consecutive
//              groups, so a wave moves 1 KiB segments;
//     K group (g, r):  row r, dims 8 g .. 8 g + 7 of one head (a thread reads
//                      them from one LDS row; consecutive rows are 16 B apart
//                      modulo 256 B, so a wave's group reads do not conflict);
//     V groups:        a thread takes 4 consecutive groups (rows 4 q .. 4 q + 3
//                      of dims d .. d + 3 and d + 16 .. d + 19, one 64 B run).
// Only rows [first_row, first_row + n_rows) are copied.  A scatter loads only
// those rows into LDS and writes the V quads cut by the range element by
// element, leaving the page's other rows untouched.
template <typename KV>
struct alignas(8 * sizeof(KV)) Group8 {
    KV x[8];
};

// Group g of a K or V block: its elements 8 g .. 8 g + 7 in the bf16 order
// (k_off / v_off), which f32 pools hold as two runs of 4, 256 elements apart
// (page_order).
template <typename KV>
__device__ inline Group8<KV> get_group(const KV* blk, size_t g) {
    if constexpr (sizeof(KV) == 2) {
        return ((const Group8<KV>*)blk)[g];
    } else {
        const KV* p = blk + page_order<KV>(8 * g);
        const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 256);
        Group8<KV> r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.x[i] = a[i];
            r.x[4 + i] = b[i];
        }
        return r;
    }
}
template <typename KV>
__device__ inline void put_group(KV* blk, size_t g, const Group8<KV>& x) {
    if constexpr (sizeof(KV) == 2) {
        ((Group8<KV>*)blk)[g] = x;
    } else {
        KV* p = blk + page_order<KV>(8 * g);
        *(f32x4*)p = f32x4{x.x[0], x.x[1], x.x[2], x.x[3]};
        *(f32x4*)(p + 256) = f32x4{x.x[4], x.x[5], x.x[6], x.x[7]};
    }
}
template <typename KV>
__device__ inline KV* group_elem(KV* blk, size_t g, int i) {
    return blk + page_order<KV>(8 * g + i);
}

template <typename KV>
__device__ inline void store4(KV* p, f32x4 x);
template <>
__device__ inline void store4<float>(float* p, f32x4 x) {
    *(f32x4*)p = x;
}
template <>
__device__ inline void store4<uint16_t>(uint16_t* p, f32x4 x) {
    ushort4 h;
    h.x = f32_to_bf16_bits(x[0]);
    h.y = f32_to_bf16_bits(x[1]);
    h.z = f32_to_bf16_bits(x[2]);
    h.w = f32_to_bf16_bits(x[3]);
    *(ushort4*)p = h;
}
template <typename KV>
__device__ inline f32x4 load4(const KV* p);
template <>
__device__ inline f32x4 load4<float>(const float* p) {
    return *(const f32x4*)p;
}
template <>
__device__ inline f32x4 load4<uint16_t>(const uint16_t* p) {
    const ushort4 h = *(const ushort4*)p;
    return f32x4{bf16_bits_to_f32(h.x), bf16_bits_to_f32(h.y), bf16_bits_to_f32(h.z), bf16_bits_to_f32(h.w)};
}

template <typename KV>
constexpr int kv_tile_pitch(int kv_cols) {
    return kv_cols + 16 / (int)sizeof(KV);  // elements: 16 B of padding per row
}

template <typename KV>
__global__ __launch_bounds__(256) void kv_copy_kernel(KV* __restrict__ pool, size_t page_elems, int n_pages_pool,
                                                      int layer_begin, const int* __restrict__ table,
                                                      int first_offset, int first_row, int n_rows, int kv_heads,
                                                      int D, float* __restrict__ k, float* __restrict__ v,
                                                      int to_pool, int plain) {
    extern __shared__ __align__(16) unsigned char kv_lds[];
    KV* tile = (KV*)kv_lds;
    const int slot = blockIdx.x, l = blockIdx.y;
    const int p0 = (first_offset + first_row) / kPageRows;
    const int page = table[p0 + slot];
    const int rbase = (p0 + slot) * kPageRows - first_offset - first_row;  // output row of page row 0
    const int r_lo = max(0, -rbase), r_hi = min(kPageRows, n_rows - rbase);
    const int kv_cols = kv_heads * D;
    const int pitch = kv_tile_pitch<KV>(kv_cols);
    const int c4 = kv_cols / 4;
    const int tile8 = kPageRows * D / 8;      // 8-element groups of one head's K (or V) tile
    KV* kblk = pool + ((size_t)(layer_begin + l) * n_pages_pool + page) * page_elems;
    if (plain) {
        // row-major [kv_head][16 rows][D] tiles: element by element, page side in order
        for (int which = 0; which < 2; ++which) {
            KV* blk = kblk + (size_t)which * kv_cols * kPageRows;
            float* rows = (which ? v : k) + (size_t)l * n_rows * kv_cols;
            for (int e = threadIdx.x; e < kv_cols * kPageRows; e += blockDim.x) {
                const int h = e / (kPageRows * D), rem = e - h * (kPageRows * D);
                const int r = rem / D, d = rem - r * D;
                if (r < r_lo || r >= r_hi) continue;
                float* x = rows + (size_t)(rbase + r) * kv_cols + h * D + d;
                if (to_pool)
                    store_elem(blk + e, *x);
                else
                    *x = load_elem(blk + e);
            }
        }
        return;
    }
    for (int which = 0; which < 2; ++which) {
        KV* blk = kblk + (size_t)which * kv_cols * kPageRows;
        // row r of the page is row rbase + r >= 0 of layer l's f32 rows (r_lo <= r < r_hi)
        float* rows = (which ? v : k) + (size_t)l * n_rows * kv_cols;
        if (which) __syncthreads();  // the K block's LDS reads are done
        if (to_pool) {
            for (int i = threadIdx.x; i < (r_hi - r_lo) * c4; i += blockDim.x) {
                const int r = r_lo + i / c4, c = (i - (i / c4) * c4) * 4;
                store4(tile + r * pitch + c, *(const f32x4*)(rows + (size_t)(rbase + r) * kv_cols + c));
            }
            __syncthreads();
        }
        if (!which) {
            for (int gi = threadIdx.x; gi < kv_heads * tile8; gi += blockDim.x) {
                const int h = gi / tile8, cg = gi - h * tile8;
                const int g = cg >> 4, r = cg & 15;  // K group cg = g * 16 + r
                KV* t = tile + r * pitch + h * D + 8 * g;
                if (to_pool) {
                    if (r >= r_lo && r < r_hi) put_group(blk, gi, *(const Group8<KV>*)t);
                } else {
                    *(Group8<KV>*)t = get_group(blk, gi);
                }
            }
        } else {
            // V group cg = ((d / 32) * 4 + q) * 16 + dd holds rows 4 q + i of dims d (i) and d + 16 (4 + i)
            for (int qi = threadIdx.x; qi < kv_heads * D / 2; qi += blockDim.x) {
                const int h = qi / (D / 2), cg0 = (qi - h * (D / 2)) * 4;
                const int q = (cg0 >> 4) & 3, d0 = (cg0 >> 6) * 32 + (cg0 & 15);
                const int r0 = 4 * q;
                const size_t g0 = (size_t)h * tile8 + cg0;  // groups g0 .. g0 + 3
                KV* t = tile + r0 * pitch + h * D + d0;
                if (!to_pool) {
                    Group8<KV> gr[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) gr[j] = get_group(blk, g0 + j);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            t[i * pitch + j] = gr[j].x[i];
                            t[i * pitch + 16 + j] = gr[j].x[4 + i];
                        }
                } else if (r0 >= r_lo && r0 + 3 < r_hi) {
                    Group8<KV> gr[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            gr[j].x[i] = t[i * pitch + j];
                            gr[j].x[4 + i] = t[i * pitch + 16 + j];
                        }
#pragma unroll
                    for (int j = 0; j < 4; ++j) put_group(blk, g0 + j, gr[j]);
                } else if (r0 + 3 >= r_lo && r0 < r_hi) {
                    for (int j = 0; j < 4; ++j)
                        for (int i = 0; i < 4; ++i) {
                            if (r0 + i < r_lo || r0 + i >= r_hi) continue;
                            *group_elem(blk, g0 + j, i) = t[i * pitch + j];
                            *group_elem(blk, g0 + j, 4 + i) = t[i * pitch + 16 + j];
                        }
                }
            }
        }
        if (!to_pool) {
            __syncthreads();
            for (int i = threadIdx.x; i < (r_hi - r_lo) * c4; i += blockDim.x) {
                const int r = r_lo + i / c4, c = (i - (i / c4) * c4) * 4;
                *(f32x4*)(rows + (size_t)(rbase + r) * kv_cols + c) = load4(tile + r * pitch + c);
            }
        }
    }
}

template <typename KV>
static zr_status kv_copy_launch(zr_context* ctx, dim3 grid, int layer_begin, const int* d_table, int first_offset,
                                int first_row, int n_rows, float* k, float* v, int to_pool) {
    const size_t lds = ctx->plain_kv ? 0 : (size_t)kPageRows * kv_tile_pitch<KV>(ctx->kv_cols) * sizeof(KV);
    if (lds > 160 * 1024)
        return set_err(ctx, ZR_E_UNSUPPORTED, "KV copy tile of %zu bytes exceeds LDS (%d kv columns)", lds,
                       ctx->kv_cols);
    if (lds > 64 * 1024) {
        const hipError_t e =
            hipFuncSetAttribute((const void*)kv_copy_kernel<KV>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return set_err(ctx, ZR_E_HIP, "KV copy LDS attribute: %s", hipGetErrorString(e));
    }
    hipLaunchKernelGGL(kv_copy_kernel<KV>, grid, dim3(256), lds, ctx->stream, (KV*)ctx->kv_pool, page_elems_of(ctx),
                       ctx->n_pages, layer_begin, d_table, first_offset, first_row, n_rows,
                       ctx->kv_cols / ctx->head_dim, ctx->head_dim, k, v, to_pool, ctx->plain_kv ? 1 : 0);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

zr_status launch_kv_copy(zr_context* ctx, int layer_begin, int layer_end, const int* d_table,
                         int first_offset, int first_row, int n_rows, float* k, float* v, int to_pool) {
    if (n_rows <= 0 || layer_end <= layer_begin) return ZR_OK;
    if (ctx->kv_cols % 4 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "kv columns %d not a multiple of 4", ctx->kv_cols);
    const int p0 = (first_offset + first_row) / kPageRows;
    const int p1 = (first_offset + first_row + n_rows - 1) / kPageRows;
    dim3 grid(p1 - p0 + 1, layer_end - layer_begin);
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassOther, &ev);  // not on the decode path: class "other" holds it alone there
    const zr_status rc =
        ctx->desc.kv_dtype == ZR_DTYPE_BF16
            ? kv_copy_launch<uint16_t>(ctx, grid, layer_begin, d_table, first_offset, first_row, n_rows, k, v, to_pool)
            : kv_copy_launch<float>(ctx, grid, layer_begin, d_table, first_offset, first_row, n_rows, k, v, to_pool);
    if (rc) return rc;
    timing_mark_end(ctx, kClassOther, ev);
    return ZR_OK;
}

// --------------------------------------------------------- synthetic fill
// Counter-based SplitMix64 -> two uniforms -> Box-Muller normal.
__device__ inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ inline float normal_at(uint64_t seed, uint64_t i) {
    const uint64_t r = splitmix64(seed * 0x100000001B3ull + i);
    const float u1 = ((float)(uint32_t)(r >> 40) + 1.0f) * (1.0f / 16777217.0f);
    const float u2 = (float)(uint32_t)(r & 0xFFFFFF) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
}

__global__ void fill_normal_bf16_kernel(uint16_t* dst, size_t n, uint64_t seed, float std) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = f32_to_bf16_bits(normal_at(seed, i) * std);
}

__global__ void fill_normal_f32_kernel(float* dst, size_t n, uint64_t seed, float std) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = normal_at(seed, i) * std;
}

zr_status launch_fill_normal_bf16(zr_context* ctx, uint16_t* dst, size_t n, uint64_t seed, float std) {
    hipLaunchKernelGGL(fill_normal_bf16_kernel, dim3(4096), dim3(256), 0, ctx->stream, dst, n, seed, std);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

zr_status launch_fill_pool_normal(zr_context* ctx, uint64_t seed, float std) {
    const size_t n = (size_t)ctx->desc.num_layers * ctx->n_pages * page_elems_of(ctx);
    if (ctx->desc.kv_dtype == ZR_DTYPE_BF16)
        hipLaunchKernelGGL(fill_normal_bf16_kernel, dim3(8192), dim3(256), 0, ctx->stream,
                           (uint16_t*)ctx->kv_pool, n, seed, std);
    else
        hipLaunchKernelGGL(fill_normal_f32_kernel, dim3(8192), dim3(256), 0, ctx->stream,
                           (float*)ctx->kv_pool, n, seed, std);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

}  // namespace zr
