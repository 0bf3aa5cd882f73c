// Stochastic sampling on the device: the batched decode path's sampler,
// sample_tokens_device_with_seeds (runtime.rs:534-601, called per group of
// rows by sample_fast_path_logits_batch, backend.rs:275-316).
//
// Per row (one 1024-thread workgroup):
//   temperature <= 0 or top_p <= 0: argmax of the raw logits (first index).
//   s = x * f32(1 / T) (affine, 534-601; x itself when T == 1); p = softmax(s).
//   top_p >= 1: the first index whose cumulative probability reaches tau.
//   top_p < 1: in the order (p descending, index ascending) keep an element
//     while the probability before it is below top_p (apply_top_p_device,
//     461-482); renormalise; the first kept element whose cumulative share
//     reaches tau.  No crossing: position 0.
//   tau = k / 2^24, k the top 24 bits of the SplitMix64 finaliser of the
//   seed (deterministic_sample_threshold, 483-497), computed on the host.
// Cumulative sums are exact integer sums of w = round(p * 2^36), so a row's
// token does not depend on the reduction order (the reference's candle
// cumsum / sum orders are not specified either); "reaches" compares
// integers: cum >= tau * 2^36 = k * 2^12, and cum * 2^24 >= k * denom for
// the renormalised share.  The order above is never materialised: the
// element where a cumulative sum crosses a target is found by a radix select
// over the probabilities' bit patterns (11 + 11 + 10 bits; per-digit bucket
// weight sums in LDS), then by rank among equal probabilities.
#include "zr_internal.h"

// Every pass recomputes p = exp(x * mul - m) / s and must get the same bits:
// no contraction into fused multiply-adds anywhere in this file.
#pragma clang fp contract(off)

namespace zr {

namespace {

constexpr int kSampleThreads = 1024;
constexpr double kFixScale = 68719476736.0;  // 2^36

struct SampleRowArgs {
    float mul;      // 1 / T (f32), used when scale != 0
    float top_p;
    uint32_t k;     // tau = k / 2^24
    int mode;       // 0 argmax, 1 full distribution, 2 nucleus
    int scale;      // T != 1
    int pad[3];
};

__device__ inline uint64_t fix_weight(float p) { return (uint64_t)((double)p * kFixScale + 0.5); }

// Block-wide exclusive scan of one u64 per thread; *total = the sum.
__device__ inline uint64_t block_exscan(uint64_t x, uint64_t* wtot, uint64_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t incl = x;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    __syncthreads();  // wtot may still be read by a previous call
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    uint64_t base = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kSampleThreads / 64; ++w) {
        if (w < wave) base += wtot[w];
        all += wtot[w];
    }
    *total = all;
    return base + incl - x;
}

struct RowView {
    const float* x;
    int cols;
    int c0, c1;      // this thread's contiguous columns (passes that need index order)
    float mul, m, s; // scaling, max, sum of exp
    int scale;
    // passes whose result does not depend on the order visit columns
    // tid, tid + 1024, ... so that a wave reads 256 contiguous bytes
    __device__ inline float scaled(int i) const { return scale ? x[i] * mul : x[i]; }
    __device__ inline float p(int i) const {
        return expf(scaled(i) - m) / s;
    }
};

// The element (in the order p descending, index ascending) at which the
// inclusive cumulative weight first reaches `target` (>= 1, <= total):
// returns its column.  *c_incl receives its inclusive cumulative weight.
__device__ int select_crossing(const RowView& rv, uint64_t target, uint64_t* c_incl, uint64_t* hsum,
                               uint64_t* wtot, int* found) {
    const int tid = threadIdx.x;
    uint32_t mask = 0, value = 0;
    uint64_t acc = 0;  // weight of the elements ordered before the current key range
    const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
#pragma unroll
    for (int pass = 0; pass < 3; ++pass) {
        const int sh = shifts[pass], nb = 1 << widths[pass];
        for (int b = tid; b < 2048; b += kSampleThreads) hsum[b] = 0;
        __syncthreads();
        // elements of weight 0 never cross a target >= 1: they are skipped
        for (int i = tid; i < rv.cols; i += kSampleThreads) {
            const float p = rv.p(i);
            const uint32_t key = __float_as_uint(p);
            const uint64_t w = fix_weight(p);
            if ((key & mask) == value && w) atomicAdd((unsigned long long*)&hsum[(key >> sh) & (nb - 1)], w);
        }
        __syncthreads();
        // descending buckets: thread t owns buckets nb-1-2t and nb-2-2t
        uint64_t mine = 0;
        const int bhi = nb - 1 - 2 * tid, blo = bhi - 1;
        if (bhi >= 0) mine += hsum[bhi];
        if (blo >= 0) mine += hsum[blo];
        uint64_t total;
        const uint64_t ex = acc + block_exscan(mine, wtot, &total);  // weight before bucket bhi
        if (tid == 0) *found = -1;
        __syncthreads();
        if (bhi >= 0 && ex < target && target <= ex + hsum[bhi]) *found = bhi;
        if (blo >= 0 && ex + hsum[bhi] < target && target <= ex + hsum[bhi] + hsum[blo]) *found = blo;
        __syncthreads();
        const int bstar = *found;
        __syncthreads();
        // weight of the buckets above b*: recompute from the owner's prefix
        if (bstar >= 0 && (tid == (nb - 1 - bstar) / 2)) {
            wtot[16] = ex + ((bstar == blo) ? hsum[bhi] : 0);
        }
        __syncthreads();
        if (bstar < 0) return -1;  // total below target (not reached by callers)
        acc = wtot[16];
        mask |= (uint32_t)(nb - 1) << sh;
        value |= (uint32_t)bstar << sh;
        __syncthreads();
    }
    // value = the crossing element's probability bits; acc = weight of larger ones;
    // rank among the equal ones (index order): t = ceil((target - acc) / w)
    const uint64_t w = fix_weight(__uint_as_float(value));
    const uint64_t t = w ? (target - acc + w - 1) / w : 1;
    uint64_t cnt = 0;
    for (int i = rv.c0; i < rv.c1; ++i) cnt += __float_as_uint(rv.p(i)) == value;
    uint64_t total;
    const uint64_t ex = block_exscan(cnt, wtot, &total);
    if (tid == 0) *found = -1;
    __syncthreads();
    if (ex < t && t <= ex + cnt) {
        uint64_t r = ex;
        for (int i = rv.c0; i < rv.c1; ++i)
            if (__float_as_uint(rv.p(i)) == value && ++r == t) {
                *found = i;
                break;
            }
    }
    __syncthreads();
    *c_incl = acc + t * w;
    return *found;
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(const float* __restrict__ logits, int cols,
                                                                const SampleRowArgs* __restrict__ rows,
                                                                uint32_t* __restrict__ out) {
    __shared__ uint64_t hsum[2048];
    __shared__ uint64_t wtot[17];
    __shared__ float fred[kSampleThreads / 64];
    __shared__ int ired[kSampleThreads / 64];
    __shared__ int found;
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SampleRowArgs a = rows[r];
    RowView rv;
    rv.x = logits + (size_t)r * cols;
    rv.cols = cols;
    const int per = (cols + kSampleThreads - 1) / kSampleThreads;
    rv.c0 = min(cols, tid * per);
    rv.c1 = min(cols, rv.c0 + per);
    rv.mul = a.mul;
    rv.scale = a.scale;
    if (a.mode == 0) {  // argmax of the raw logits, first index on ties
        float bv = -INFINITY;
        int bi = cols;
        for (int i = rv.c0; i < rv.c1; ++i)
            if (rv.x[i] > bv) {
                bv = rv.x[i];
                bi = i;
            }
        if (bi == cols && rv.c0 < rv.c1) bi = rv.c0;  // all -inf
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            const float v2 = __shfl_xor(bv, o, 64);
            const int i2 = __shfl_xor(bi, o, 64);
            if (v2 > bv || (v2 == bv && i2 < bi)) {
                bv = v2;
                bi = i2;
            }
        }
        if (lane == 0) {
            fred[wave] = bv;
            ired[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < kSampleThreads / 64; ++w)
                if (fred[w] > bv || (fred[w] == bv && ired[w] < bi)) {
                    bv = fred[w];
                    bi = ired[w];
                }
            out[r] = (uint32_t)(bi < cols ? bi : 0);
        }
        return;
    }
    // softmax statistics (fixed reduction order)
    float m = -INFINITY;
    for (int i = tid; i < cols; i += kSampleThreads) m = fmaxf(m, rv.scaled(i));
#pragma unroll
    for (int o = 32; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) fred[wave] = m;
    __syncthreads();
    m = -INFINITY;
    for (int w = 0; w < kSampleThreads / 64; ++w) m = fmaxf(m, fred[w]);
    __syncthreads();
    rv.m = m;
    float s = 0.0f;
    for (int i = tid; i < cols; i += kSampleThreads) s += expf(rv.scaled(i) - m);
#pragma unroll
    for (int o = 32; o; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) fred[wave] = s;
    __syncthreads();
    s = 0.0f;
    for (int w = 0; w < kSampleThreads / 64; ++w) s += fred[w];
    __syncthreads();
    rv.s = s;
    uint64_t seg = 0, total;
    if (a.mode == 1) {
        for (int i = rv.c0; i < rv.c1; ++i) seg += fix_weight(rv.p(i));
        const uint64_t ex = block_exscan(seg, wtot, &total);
        // first index whose cumulative weight reaches tau * 2^36 = k * 2^12
        const uint64_t target = (uint64_t)a.k << 12;
        if (tid == 0) found = target == 0 ? 0 : -1;
        __syncthreads();
        if (target > 0 && ex < target && target <= ex + seg) {
            uint64_t c = ex;
            for (int i = rv.c0; i < rv.c1; ++i) {
                c += fix_weight(rv.p(i));
                if (c >= target) {
                    found = i;
                    break;
                }
            }
        }
        __syncthreads();
        if (tid == 0) out[r] = (uint32_t)(found < 0 ? 0 : found);
        return;
    }
    for (int i = tid; i < cols; i += kSampleThreads) seg += fix_weight(rv.p(i));
    (void)block_exscan(seg, wtot, &total);
    // nucleus: the last kept element is the first whose inclusive cumulative
    // weight reaches top_p (all kept when the total stays below it)
    uint64_t p_int = (uint64_t)ceil((double)a.top_p * kFixScale);
    if (p_int < 1) p_int = 1;
    uint64_t denom = total;
    if (p_int <= total) {
        uint64_t c;
        select_crossing(rv, p_int, &c, hsum, wtot, &found);
        denom = c;
    }
    // sampled: first kept element with cum * 2^24 >= k * denom
    uint64_t t2 = ((uint64_t)a.k * denom + (1ull << 24) - 1) >> 24;
    if (t2 < 1) t2 = 1;
    uint64_t c2;
    const int col = select_crossing(rv, t2, &c2, hsum, wtot, &found);
    if (tid == 0) out[r] = (uint32_t)(col < 0 ? 0 : col);
}

}  // namespace

// Host: per-row parameters (deterministic_sample_threshold in double, as the
// reference computes it) and the launch.  temperature / top_p / seeds are
// host arrays of `rows`; logits and out are device memory.
zr_status launch_sample(zr_context* ctx, const float* d_logits, int rows, int cols, const float* temperature,
                        const float* top_p, const uint64_t* seeds, uint32_t* d_out) {
    if (rows <= 0) return ZR_OK;
    if (cols <= 0) return set_err(ctx, ZR_E_INVALID, "Device sampling received an empty logits tensor");
    std::vector<SampleRowArgs> h(rows);
    for (int r = 0; r < rows; ++r) {
        SampleRowArgs& a = h[r];
        const float T = temperature[r], P = top_p[r];
        a.mode = (T <= 0.0f || P <= 0.0f) ? 0 : (P >= 1.0f ? 1 : 2);
        a.scale = T != 1.0f;
        a.mul = 1.0f / T;
        a.top_p = P;
        uint64_t x = seeds[r] + 0x9E3779B97F4A7C15ull;  // SplitMix64 finaliser
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        x ^= x >> 31;
        a.k = (uint32_t)(x >> 40);  // tau = k / 2^24 < 1 - eps: the clamp never binds
        a.pad[0] = a.pad[1] = a.pad[2] = 0;
    }
    const size_t bytes = sizeof(SampleRowArgs) * (size_t)rows;
    if (bytes > ctx->sample_ws_bytes) {
        ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->sample_ws) (void)hipFree(ctx->sample_ws);
        ctx->sample_ws = nullptr;
        ctx->sample_ws_bytes = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->sample_ws, bytes));
        ctx->sample_ws_bytes = bytes;
    }
    ZR_HIP(ctx, hipMemcpyAsync(ctx->sample_ws, h.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassOther, &ev);
    hipLaunchKernelGGL(sample_kernel, dim3(rows), dim3(kSampleThreads), 0, ctx->stream, d_logits, cols,
                       (const SampleRowArgs*)ctx->sample_ws, d_out);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassOther, ev);
    // the host parameters must outlive the copy
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

}  // namespace zr
