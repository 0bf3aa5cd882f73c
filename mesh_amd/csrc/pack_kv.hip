// Ragged-batch packing, fused RoPE + paged-KV append, and the KV handoff
// gather/scatter kernels.
//
// KV pool layout (per layer, per global page, K block then V block, one
// [16 x head_dim] tile per local kv head, element type = pool dtype):
//   K tile: element (t, d) at ((d / 8) * 16 + t) * 8 + d % 8
//           -> one 1 KiB row of 64 lanes x 16 B is exactly the MFMA A-operand
//              fragment (token = lane % 16, 8 dims per lane) for 32 dims.
//   V tile: element (t, d) at ((((d / 32) * 4 + t / 4) * 16 + d % 16) * 2
//           + (d / 16) % 2) * 4 + t % 4
//           -> 4 consecutive tokens of one dim are one P.V MFMA operand
//              lane; dims d and d + 16 sit next to each other, so a lane
//              loads both with one 16 B (bf16) load and a wave reads 1 KiB
//              contiguous per 32 dims.
#include "zr_internal.h"

namespace zr {

__device__ inline size_t k_off(int t, int d) { return ((size_t)(d >> 3) * kPageRows + t) * 8 + (d & 7); }
__device__ inline size_t v_off(int t, int d, int) {
    return (((((size_t)(d >> 5) * 4 + (t >> 2)) * 16 + (d & 15)) * 2 + ((d >> 4) & 1)) * 4) + (t & 3);
}

template <typename T> __device__ inline void store_elem(T* p, float x);
template <> __device__ inline void store_elem<float>(float* p, float x) { *p = x; }
template <> __device__ inline void store_elem<uint16_t>(uint16_t* p, float x) { *p = f32_to_bf16_bits(x); }
template <typename T> __device__ inline float load_elem(const T* p);
template <> __device__ inline float load_elem<float>(const float* p) { return *p; }
template <> __device__ inline float load_elem<uint16_t>(const uint16_t* p) { return bf16_bits_to_f32(*p); }

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

zr_status launch_pack(zr_context* ctx, StagedMeta* st) {
    hipLaunchKernelGGL(pack_kernel, dim3(1), dim3(1024), 0, ctx->stream, st->num_seqs, st->q_len,
                       st->kv_before, st->first_pos, st->first_offset, st->block_tables, st->stride,
                       st->cu_q, st->cu_k, st->positions, st->slot_mapping, st->seq_ids, st->last_rows);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

// ---------------------------------------------------------- RoPE + append
// One workgroup per token row.  RoPE follows tensor_ops.rs:509-560 /
// runtime.rs:935-1005 (rotate-half, theta = position * inv_freq in f32) and
// the KV append is DeviceLayerKVCache::append (forward_pass.rs:462-521) at the
// slot the host reserved.
template <typename KV>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(
    const float* __restrict__ qkv, int qkv_n, size_t qkv_slab, int qkv_stride, float* __restrict__ q_out,
    int q_cols, int kv_cols,
    int D, const int* __restrict__ positions, const int* __restrict__ slot,
    const float* __restrict__ inv_freq, KV* __restrict__ layer_pool, size_t page_elems, int rope) {
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    const int half = D / 2;
    const float pos = (float)positions[t];
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
            float a = src[i], b = src[i + half];
#pragma unroll 4
            for (int sl = 1; sl < qkv_n; ++sl) {
                a += src[sl * qkv_slab + i];
                b += src[sl * qkv_slab + i + half];
            }
            if (rope) {
                const float theta = pos * inv_freq[i];
                const float c = cosf(theta), sn = sinf(theta);
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
                store_elem(kt + k_off(r, i), a);
                store_elem(kt + k_off(r, i + half), b);
            }
        } else {
            const int c = j - nq - nk;
            const int head = c / D, d = c % D;
            KV* vt = vpage + (size_t)head * kPageRows * D;
            float vv = row[q_cols + kv_cols + c];
#pragma unroll 4
            for (int sl = 1; sl < qkv_n; ++sl) vv += row[sl * qkv_slab + q_cols + kv_cols + c];
            store_elem(vt + v_off(r, d, D), vv);
        }
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
    if (ctx->desc.kv_dtype == ZR_DTYPE_BF16) {
        uint16_t* pool = (uint16_t*)ctx->kv_pool + (size_t)layer * ctx->n_pages * pe;
        hipLaunchKernelGGL(rope_kv_write_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream,
                           qkv.ptr, qkv.n, qkv.stride, stride, q_out, ctx->q_cols, ctx->kv_cols, ctx->head_dim, st->positions,
                           st->slot_mapping, ctx->inv_freq, pool, pe, rope);
    } else {
        float* pool = (float*)ctx->kv_pool + (size_t)layer * ctx->n_pages * pe;
        hipLaunchKernelGGL(rope_kv_write_kernel<float>, grid, dim3(256), 0, ctx->stream,
                           qkv.ptr, qkv.n, qkv.stride, stride, q_out, ctx->q_cols, ctx->kv_cols, ctx->head_dim, st->positions,
                           st->slot_mapping, ctx->inv_freq, pool, pe, rope);
    }
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassNormRopeKv, ev);
    return ZR_OK;
}

// ------------------------------------------------------ gather / scatter
// Logical window row j of a sequence lives at physical row first_offset + j of
// its page list (interior spans are full pages; only the first span may start
// mid-page after retain_suffix).  One workgroup per (page of the range, layer);
// its threads sweep the page's 8-element groups, which are contiguous in the
// pool layout (16 B in bf16 pools):
//   K group (g, r):    row r, dims 8 g .. 8 g + 7 of one head;
//   V group (q, dd):   rows 4 q .. 4 q + 3 of dims d and d + 16, d = 32 (g / 4) + dd.
// Consecutive threads take consecutive groups, so the page side is read or
// written in whole 1 KiB wave segments and each row side in 128 B runs.  Only
// rows [first_row, first_row + n_rows) are copied: a scatter writes the other
// rows of a boundary V group element by element, leaving them untouched.
template <typename KV>
struct alignas(8 * sizeof(KV)) Group8 {
    KV x[8];
};

template <typename KV>
__global__ __launch_bounds__(256) void kv_copy_kernel(KV* __restrict__ pool, size_t page_elems, int n_pages_pool,
                                                      int layer_begin, const int* __restrict__ table,
                                                      int first_offset, int first_row, int n_rows, int kv_heads,
                                                      int D, float* __restrict__ k, float* __restrict__ v,
                                                      int to_pool) {
    const int slot = blockIdx.x, l = blockIdx.y;
    const int p0 = (first_offset + first_row) / kPageRows;
    const int page = table[p0 + slot];
    const int rbase = (p0 + slot) * kPageRows - first_offset - first_row;  // output row of page row 0
    const int r_lo = max(0, -rbase), r_hi = min(kPageRows, n_rows - rbase);
    const size_t kv_cols = (size_t)kv_heads * D;
    const int tile = kPageRows * D;           // elements of one head's K (or V) tile
    const int groups = kv_heads * tile / 8;   // 8-element groups per K (or V) block
    Group8<KV>* kp = (Group8<KV>*)(pool + ((size_t)(layer_begin + l) * n_pages_pool + page) * page_elems);
    Group8<KV>* vp = kp + groups;
    // output row of page row r (r_lo <= r < r_hi, so rbase + r >= 0)
    auto krow = [&](int r) { return k + ((size_t)l * n_rows + (rbase + r)) * kv_cols; };
    auto vrow = [&](int r) { return v + ((size_t)l * n_rows + (rbase + r)) * kv_cols; };
    for (int gi = threadIdx.x; gi < groups; gi += blockDim.x) {
        const int h = gi / (tile / 8), cg = gi - h * (tile / 8);
        // K: group cg = g * 16 + r
        {
            const int g = cg >> 4, r = cg & 15;
            if (r >= r_lo && r < r_hi) {
                float* row = krow(r) + (size_t)h * D + 8 * g;
                if (to_pool) {
                    Group8<KV> gr;
#pragma unroll
                    for (int j = 0; j < 8; ++j) store_elem(&gr.x[j], row[j]);
                    kp[gi] = gr;
                } else {
                    const Group8<KV> gr = kp[gi];
#pragma unroll
                    for (int j = 0; j < 8; ++j) row[j] = load_elem(&gr.x[j]);
                }
            }
        }
    }
    // V: group cg = ((d / 32) * 4 + q) * 16 + dd holds rows 4 q + i of dims d (i)
    // and d + 16 (4 + i).  A thread takes 4 consecutive groups (dims d .. d + 3,
    // one 64 B run of the page) and moves the 4 rows as float4 runs of dims
    // d .. d + 3 and d + 16 .. d + 19; a quad cut by the row range goes element
    // by element.
    const int quads = kv_heads * D / 2;
    for (int qi = threadIdx.x; qi < quads; qi += blockDim.x) {
        const int h = qi / (D / 2), cg0 = (qi - h * (D / 2)) * 4;
        const int q = (cg0 >> 4) & 3, d0 = (cg0 >> 6) * 32 + (cg0 & 15);
        const int r0 = 4 * q;
        if (r0 + 3 < r_lo || r0 >= r_hi) continue;
        Group8<KV>* gp = vp + (size_t)h * (tile / 8) + cg0;
        const size_t c0 = (size_t)h * D + d0;  // column of dim d0
        if (r0 >= r_lo && r0 + 3 < r_hi) {
            if (to_pool) {
                f32x4 lo4[4], hi4[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo4[i] = *(const f32x4*)(vrow(r0 + i) + c0);
                    hi4[i] = *(const f32x4*)(vrow(r0 + i) + c0 + 16);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    Group8<KV> gr;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        store_elem(&gr.x[i], lo4[i][j]);
                        store_elem(&gr.x[4 + i], hi4[i][j]);
                    }
                    gp[j] = gr;
                }
            } else {
                Group8<KV> gr[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) gr[j] = gp[j];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    *(f32x4*)(vrow(r0 + i) + c0) = f32x4{load_elem(&gr[0].x[i]), load_elem(&gr[1].x[i]),
                                                        load_elem(&gr[2].x[i]), load_elem(&gr[3].x[i])};
                    *(f32x4*)(vrow(r0 + i) + c0 + 16) =
                        f32x4{load_elem(&gr[0].x[4 + i]), load_elem(&gr[1].x[4 + i]), load_elem(&gr[2].x[4 + i]),
                              load_elem(&gr[3].x[4 + i])};
                }
            }
        } else {
            for (int j = 0; j < 4; ++j) {
                KV* e = gp[j].x;
                for (int i = 0; i < 4; ++i) {
                    if (r0 + i < r_lo || r0 + i >= r_hi) continue;
                    if (to_pool) {
                        store_elem(&e[i], vrow(r0 + i)[c0 + j]);
                        store_elem(&e[4 + i], vrow(r0 + i)[c0 + 16 + j]);
                    } else {
                        vrow(r0 + i)[c0 + j] = load_elem(&e[i]);
                        vrow(r0 + i)[c0 + 16 + j] = load_elem(&e[4 + i]);
                    }
                }
            }
        }
    }
}

zr_status launch_kv_copy(zr_context* ctx, int layer_begin, int layer_end, const int* d_table,
                         int first_offset, int first_row, int n_rows, float* k, float* v, int to_pool) {
    if (n_rows <= 0 || layer_end <= layer_begin) return ZR_OK;
    const size_t pe = page_elems_of(ctx);
    const int p0 = (first_offset + first_row) / kPageRows;
    const int p1 = (first_offset + first_row + n_rows - 1) / kPageRows;
    dim3 grid(p1 - p0 + 1, layer_end - layer_begin);
    const int kvh = ctx->kv_cols / ctx->head_dim;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassOther, &ev);  // not on the decode path: class "other" holds it alone there
    if (ctx->desc.kv_dtype == ZR_DTYPE_BF16)
        hipLaunchKernelGGL(kv_copy_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream,
                           (uint16_t*)ctx->kv_pool, pe, ctx->n_pages, layer_begin, d_table, first_offset,
                           first_row, n_rows, kvh, ctx->head_dim, k, v, to_pool);
    else
        hipLaunchKernelGGL(kv_copy_kernel<float>, grid, dim3(256), 0, ctx->stream, (float*)ctx->kv_pool,
                           pe, ctx->n_pages, layer_begin, d_table, first_offset, first_row, n_rows, kvh,
                           ctx->head_dim, k, v, to_pool);
    ZR_LAUNCH_CHECK(ctx);
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
