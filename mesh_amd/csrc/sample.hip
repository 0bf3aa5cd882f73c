// Stochastic sampling on the device: the batched decode path's sampler,
// sample_tokens_device_with_seeds (runtime.rs:534-601, called per group of
// rows by sample_fast_path_logits_batch, backend.rs:275-316).
//
// Per row (one 1024-thread workgroup):
//   temperature <= 0 or top_p <= 0: argmax of the raw logits (first index).
//   y = x * f32(1 / T) (affine, 534-601; x itself when T == 1); p = softmax(y).
//   top_p >= 1: the first index whose cumulative probability reaches tau.
//   top_p < 1: in the order (p descending, index ascending) keep an element
//     while the probability before it is below top_p (apply_top_p_device,
//     461-482); renormalise; the first kept element whose cumulative share
//     reaches tau.  No crossing: position 0.
//   tau = k / 2^24, k the top 24 bits of the SplitMix64 finaliser of the
//   seed (deterministic_sample_threshold, 483-497), computed on the host.
// Arithmetic: e = expf(y - max) in f32 and its weight w = round(e * 2^36)
// (0 below 2^-37); p = e / sum(e), so with W = sum(w) every comparison of a
// cumulative probability becomes one of exact integers: cum >= tau * W is
// cum >= ceil(k * W / 2^24); before < top_p * W makes the last kept element
// the first with cum >= ceil(top_p * W); the renormalised share reaches tau
// at cum >= ceil(k * denom / 2^24).  A row's token therefore does not depend
// on any reduction order (the reference's candle sum / cumsum orders are not
// specified either), and the softmax denominator is never formed.
//
// Every pass over a row reads it coalesced (float4 per lane, four loads in
// flight per thread) and recomputes e from the logit; the row is never
// materialised in another form.  Passes:
//   greedy: one pass (max, first index).
//   max of y: one pass, then
//   full distribution: one pass of weight sums over 16 contiguous ranges
//     (one per wave), then the range holding the crossing.
//   nucleus: the (p descending, index ascending) order is never built.  One
//     pass histograms e by exponent and two mantissa bits (weight sums), which
//     fixes the bucket of the top_p crossing and the range of buckets the
//     sampled crossing can fall in; when those buckets hold at most 8192
//     elements (bounded by weight sum / smallest weight), one pass collects
//     them into LDS, they are sorted by (e, -index) (by rank up to 1024 of
//     them, a bitonic network beyond) and both crossings are read off the
//     sorted run.  Otherwise each crossing is
//     refined on its own: further passes over the next 11 and 10 bits,
//     collection of the bucket, and, for a run of more than 8192 equal
//     probabilities, rank in index order by per-tile counts.
#include "zr_internal.h"

// Every pass recomputes e = expf(x * mul - m) and must get the same bits:
// no contraction into fused multiply-adds anywhere in this file.
#pragma clang fp contract(off)

namespace zr {

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kCap = 8192;                     // candidates resolved in LDS
constexpr int kMaxCols = 1 << 20;              // weight sums stay below 2^57
constexpr uint32_t kMinKey = 90u << 23;        // e < 2^-37 weighs 0
constexpr uint32_t kOneKey = 127u << 23;       // e == 1
constexpr int kL1Base = (int)(kMinKey >> 21);  // first level: bits 21..31, offset
constexpr int kL1Buckets = 256;
constexpr float kLog2E = 1.44269504088896341f;

struct SampleRowArgs {
    float mul;      // f32(1 / T); 1 when T == 1 (x * 1 == x exactly)
    uint32_t k;     // tau = k / 2^24
    int mode;       // 0 argmax, 1 full distribution, 2 nucleus
    uint32_t tp_m;  // top_p = tp_m / 2^tp_q exactly (nucleus)
    int tp_q;
    int pad[3];
};

// round(e * 2^36), halves up, from the bits of e in [0, 1]: 0 below 2^-37
// (and for anything above 1 or not a number).  Equal to
// (uint64_t)((double)e * 2^36 + 0.5).  Branch free: with s = 127 - exponent,
// q = floor(2 e 2^36) = (mant << 14) >> s and the rounded value is (q + 1) >> 1.
__device__ inline uint64_t fix_weight(uint32_t b) {
    const uint32_t eb = b >> 23;
    const uint32_t s = min(127u - min(eb, 127u), 63u);
    const uint64_t q = ((uint64_t)((b & 0x7FFFFFu) | 0x800000u) << 14) >> s;
    const uint64_t w = (q + 1) >> 1;
    return eb > 127u ? 0 : w;
}

// ceil(a * b / 2^q) for a * b < 2^120.
__device__ inline uint64_t ceil_mul_shr(uint64_t a, uint64_t b, int q) {
    const unsigned __int128 p = (unsigned __int128)a * b;
    if (q >= 120) return p ? 1 : 0;
    return (uint64_t)((p + (((unsigned __int128)1 << q) - 1)) >> q);
}

__device__ inline int l1_bucket(uint32_t key) { return (int)(key >> 21) - kL1Base; }
__device__ inline uint64_t l1_min_weight(int b) { return fix_weight((uint32_t)(b + kL1Base) << 21); }

struct Row {
    const float* x;
    int cols, vec;   // vec: cols % 4 == 0 and x 16-byte aligned
    float mul, m;
    __device__ inline float scaled(float v) const { return v * mul; }
    __device__ inline float diff(float v) const { return scaled(v) - m; }
    // e = 2^((y - max) * log2(e)) with the hardware exp2 (1 ulp; results
    // below 2^-126 may flush to 0, far below the smallest weighted e):
    // relative error below (1 + |y - max|) * 1.2e-7
    __device__ inline uint32_t key_of_diff(float d) const {
        return __float_as_uint(__builtin_amdgcn_exp2f(d * kLog2E));
    }
    __device__ inline uint32_t key(float v) const { return key_of_diff(diff(v)); }
    __device__ inline int tiles() const {
        return vec ? ((cols >> 2) + kThreads - 1) / kThreads : (cols + kThreads - 1) / kThreads;
    }
};

// Visits every column once: f(column, logit, tile).  Lane l of tile t holds
// columns 4 * (1024 t + l) .. + 3 (vec) or 1024 t + l, so within a tile the
// column order is the thread order; a thread sees its tiles in ascending order.
template <class F>
__device__ inline void sweep(const Row& R, F&& f) {
    const int tid = threadIdx.x;
    if (R.vec) {
        // two groups of four float4 loads in flight: the next group is
        // issued before the current one is processed
        const float4* x4 = reinterpret_cast<const float4*>(R.x);
        const int nv = R.cols >> 2;
        float4 cur[4], nxt[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = tid + u * kThreads;
            cur[u] = j < nv ? x4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (int j0 = tid; j0 < nv; j0 += 4 * kThreads) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = j0 + (4 + u) * kThreads;
                nxt[u] = j < nv ? x4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = j0 + u * kThreads;
                if (j < nv) {
                    const int t = j / kThreads;
                    f(4 * j, cur[u].x, t);
                    f(4 * j + 1, cur[u].y, t);
                    f(4 * j + 2, cur[u].z, t);
                    f(4 * j + 3, cur[u].w, t);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) cur[u] = nxt[u];
        }
    } else {
        for (int i0 = tid; i0 < R.cols; i0 += 4 * kThreads) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * kThreads;
                v[u] = i < R.cols ? R.x[i] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * kThreads;
                if (i < R.cols) f(i, v[u], i / kThreads);
            }
        }
    }
}

// Wave w covers the contiguous columns [w * span, (w + 1) * span) (span a
// multiple of 4), its lanes reading consecutive float4 (or floats), four
// loads in flight per lane: f(column, logit).
template <class F>
__device__ inline void sweep_wave_range(const Row& R, int span, F&& f) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = wave * span, c1 = min(R.cols, c0 + span);
    if (R.vec) {
        const float4* x4 = reinterpret_cast<const float4*>(R.x);
        const int j1 = c1 >> 2;
        for (int jb = (c0 >> 2) + lane; jb < j1; jb += 4 * 64) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = jb + u * 64;
                v[u] = j < j1 ? x4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = jb + u * 64;
                if (j < j1) {
                    f(4 * j, v[u].x);
                    f(4 * j + 1, v[u].y);
                    f(4 * j + 2, v[u].z);
                    f(4 * j + 3, v[u].w);
                }
            }
        }
    } else {
        for (int ib = c0 + lane; ib < c1; ib += 4 * 64) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = ib + u * 64;
                v[u] = i < c1 ? R.x[i] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = ib + u * 64;
                if (i < c1) f(i, v[u]);
            }
        }
    }
}

struct Shared {
    uint64_t hist[2048];         // second / third level, tile sums, tile counts
    uint64_t hist1[kL1Buckets];  // first level weight sums
    uint64_t pre1[kL1Buckets];   // weight of the first-level buckets above each
    uint64_t off[kL1Buckets];    // running-weight offset of collected buckets
    uint64_t cand[kCap];         // (e bits << 32) | (~column), sorted descending
    uint64_t wtot[kWaves];
    float fm[kWaves];
    int fi[kWaves];
    int ncand, bucket, found, first;
    uint64_t acc, bsum, total, cin;
};

// Block-wide exclusive scan of one u64 per thread; *total = the sum.
__device__ inline uint64_t block_exscan(uint64_t x, Shared& S, uint64_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t incl = x;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    __syncthreads();  // wtot may still be read by a previous call
    if (lane == 63) S.wtot[wave] = incl;
    __syncthreads();
    uint64_t base = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        if (w < wave) base += S.wtot[w];
        all += S.wtot[w];
    }
    *total = all;
    return base + incl - x;
}

// The entry of h (nb entries, visited in descending index order when desc,
// ascending otherwise) where the running weight, starting at acc, first
// reaches target.  S.bucket = its index (-1: never), S.acc = the weight
// before it, S.bsum = its weight; S.total = acc + all weight.
__device__ __attribute__((always_inline)) inline void hist_cross(const uint64_t* h, int nb, bool desc,
                                                                 uint64_t target, uint64_t acc, Shared& S) {
    const int tid = threadIdx.x, per = (nb + kThreads - 1) / kThreads;
    uint64_t mine = 0;
    for (int q = 0; q < per; ++q) {
        const int pos = tid * per + q;
        if (pos < nb) mine += h[desc ? nb - 1 - pos : pos];
    }
    uint64_t total;
    uint64_t ex = acc + block_exscan(mine, S, &total);
    if (tid == 0) {
        S.bucket = -1;
        S.total = acc + total;
    }
    __syncthreads();
    if (ex < target && target <= ex + mine) {
        for (int q = 0; q < per; ++q) {
            const int pos = tid * per + q;
            const int b = desc ? nb - 1 - pos : pos;
            const uint64_t w = h[b];
            if (target <= ex + w) {
                S.bucket = b;
                S.acc = ex;
                S.bsum = w;
                break;
            }
            ex += w;
        }
    }
    __syncthreads();
}

// Tile t: the thread order is the column order.  q(logit) gives each
// column's amount; returns the column where the running amount first reaches
// target (>= 1), -1 if it never does.
template <class Q>
__device__ __attribute__((always_inline)) inline int tile_find(const Row& R, int t, uint64_t target, Q&& q,
                                                               Shared& S) {
    const int tid = threadIdx.x;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    int n = 0, base = 0;
    if (R.vec) {
        const int j = t * kThreads + tid;
        if (j < (R.cols >> 2)) {
            const float4 f = reinterpret_cast<const float4*>(R.x)[j];
            v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
            n = 4;
        }
        base = 4 * j;
    } else {
        const int i = t * kThreads + tid;
        if (i < R.cols) {
            v[0] = R.x[i];
            n = 1;
        }
        base = i;
    }
    uint64_t a[4] = {0, 0, 0, 0}, sum = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (e < n) sum += (a[e] = q(v[e]));
    uint64_t total;
    const uint64_t ex = block_exscan(sum, S, &total);
    if (tid == 0) S.found = -1;
    __syncthreads();
    if (ex < target && target <= ex + sum) {
        uint64_t c = ex;
        int hit = -1;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            c += a[e];
            if (hit < 0 && e < n && c >= target) hit = e;
        }
        S.found = base + hit;
    }
    __syncthreads();
    return S.found;
}

// A window [lo, hi] of y - max holding every element whose key lies in
// [klo, khi] (keys of weight > 0): key(d) is monotone in d and within
// (1 + |d|) * 1.2e-7 of exp(d), far inside the 1e-3 slack.
struct DWindow {
    float lo, hi;
};
__device__ inline DWindow d_window(uint32_t klo, uint32_t khi) {
    const float a = logf(__uint_as_float(klo)), b = logf(__uint_as_float(khi));
    return {a - (1e-3f + 1e-4f * fabsf(a)), b + (1e-3f + 1e-4f * fabsf(b))};
}

// Columns [start, start + len): each thread sums q over a contiguous chunk;
// returns the column where the running amount first reaches target (>= 1),
// -1 if it never does.
template <class Q>
__device__ __attribute__((always_inline)) inline int range_find(const Row& R, int start, int len, uint64_t target,
                                                                Q&& q, Shared& S) {
    const int tid = threadIdx.x, per = (len + kThreads - 1) / kThreads;
    const int lo = min(len, tid * per), hi = min(len, lo + per);
    uint64_t sum = 0;
    for (int i = lo; i < hi; ++i) sum += q(R.x[start + i]);
    uint64_t total;
    const uint64_t ex = block_exscan(sum, S, &total);
    if (tid == 0) S.found = -1;
    __syncthreads();
    if (ex < target && target <= ex + sum) {
        uint64_t c = ex;
        for (int i = lo; i < hi; ++i) {
            c += q(R.x[start + i]);
            if (c >= target) {
                S.found = start + i;
                break;
            }
        }
    }
    __syncthreads();
    return S.found;
}

// Collects the elements of weight > 0 whose key lies in [klo1, khi1] or
// [klo2, khi2] (at most kCap of them) and sorts them descending by
// (key, ~column); returns their number.  The exact key is computed only
// inside the y windows of the two ranges.  The entries are distinct (the
// column is part of each), so up to 1024 of them are placed by rank; larger
// sets go through a bitonic network.  S.hist is scratch here.
__device__ __attribute__((always_inline)) inline int collect_sorted(const Row& R, uint32_t klo1, uint32_t khi1,
                                                                    uint32_t klo2, uint32_t khi2, Shared& S) {
    const int tid = threadIdx.x;
    klo1 = klo1 < kMinKey ? kMinKey : klo1;
    klo2 = klo2 < kMinKey ? kMinKey : klo2;
    khi1 = khi1 > kOneKey ? kOneKey : khi1;
    khi2 = khi2 > kOneKey ? kOneKey : khi2;
    const DWindow w1 = d_window(klo1, khi1), w2 = d_window(klo2, khi2);
    const bool use1 = klo1 <= khi1, use2 = klo2 <= khi2;
    if (tid == 0) S.ncand = 0;
    __syncthreads();
    sweep(R, [&](int i, float v, int) {
        const float d = R.diff(v);
        if ((use1 && d >= w1.lo && d <= w1.hi) || (use2 && d >= w2.lo && d <= w2.hi)) {
            const uint32_t key = R.key_of_diff(d);
            if ((use1 && key >= klo1 && key <= khi1) || (use2 && key >= klo2 && key <= khi2)) {
                const int slot = atomicAdd(&S.ncand, 1);
                if (slot < kCap) S.cand[slot] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
            }
        }
    });
    __syncthreads();
    const int n = min(S.ncand, kCap);
    if (n <= kThreads) {
        const uint64_t mine = tid < n ? S.cand[tid] : 0;
        int rank = 0;
        if (tid < n)
            for (int j = 0; j < n; ++j) rank += S.cand[j] > mine;
        if (tid < n) S.hist[rank] = mine;
        __syncthreads();
        if (tid < n) S.cand[tid] = S.hist[tid];
        __syncthreads();
        return n;
    }
    int n2 = 2;
    while (n2 < n) n2 <<= 1;
    for (int q = n + tid; q < n2; q += kThreads) S.cand[q] = 0;
    __syncthreads();
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < n2; i += kThreads) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = S.cand[i], b = S.cand[ixj];
                    if ((i & k) == 0 ? a < b : a > b) {
                        S.cand[i] = b;
                        S.cand[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    return n;
}

// Over the sorted candidates (n of them, each thread a contiguous chunk), the
// running weight of candidate i is base(i) + (weight of candidates 0..i),
// base(i) = S.off[first-level bucket of i] when per_bucket, else acc.  Finds
// the first candidate whose running weight reaches target: returns its
// column (-1: none) and *c_incl its running weight.
__device__ __attribute__((always_inline)) inline int cand_cross(int n, bool per_bucket, uint64_t acc,
                                                                uint64_t target, Shared& S, uint64_t* c_incl) {
    const int tid = threadIdx.x, per = (n + kThreads - 1) / kThreads;
    const int lo = min(n, tid * per), hi = min(n, lo + per);
    uint64_t sum = 0;
    for (int q = lo; q < hi; ++q) sum += fix_weight((uint32_t)(S.cand[q] >> 32));
    uint64_t total;
    uint64_t run = block_exscan(sum, S, &total);
    if (tid == 0) S.first = INT_MAX;
    __syncthreads();
    int mine = INT_MAX;
    uint64_t cmine = 0;
    for (int q = lo; q < hi; ++q) {
        const uint32_t key = (uint32_t)(S.cand[q] >> 32);
        run += fix_weight(key);
        const uint64_t c = (per_bucket ? S.off[l1_bucket(key)] : acc) + run;
        if (c >= target) {
            mine = q;
            cmine = c;
            break;
        }
    }
    if (mine != INT_MAX) atomicMin(&S.first, mine);
    __syncthreads();
    if (mine != INT_MAX && mine == S.first) {
        S.found = (int)~(uint32_t)S.cand[mine];
        S.cin = cmine;
    }
    if (tid == 0 && S.first == INT_MAX) S.found = -1;
    __syncthreads();
    *c_incl = S.cin;
    return S.found;
}

// One crossing refined on its own: the element, in the order (e descending,
// column ascending), at which the running weight first reaches target
// (1 <= target <= total weight).  cs caches the last collected bucket.
struct CandState {
    uint32_t mask, value;
    int n;  // -1: empty
};

__device__ __attribute__((always_inline)) inline int refine_cross(const Row& R, uint64_t target, Shared& S,
                                                                  CandState& cs, uint64_t* c_incl) {
    const int tid = threadIdx.x;
    hist_cross(S.hist1, kL1Buckets, true, target, 0, S);
    if (S.bucket < 0) return -1;
    uint32_t mask = 0xFFE00000u, value = (uint32_t)(S.bucket + kL1Base) << 21;
    uint64_t acc = S.acc, bsum = S.bsum;
    int level = 1;
    // elements in a bucket <= its weight / the weight of its smallest key
    while (bsum / fix_weight(value) > (uint64_t)kCap && level < 3) {
        const int sh = level == 1 ? 10 : 0, nb = level == 1 ? 2048 : 1024;
        for (int b = tid; b < nb; b += kThreads) S.hist[b] = 0;
        __syncthreads();
        sweep(R, [&](int, float v, int) {
            const uint32_t key = R.key(v);
            if ((key & mask) == value)
                atomicAdd((unsigned long long*)&S.hist[(key >> sh) & (nb - 1)],
                          (unsigned long long)fix_weight(key));
        });
        __syncthreads();
        hist_cross(S.hist, nb, true, target, acc, S);
        if (S.bucket < 0) return -1;
        acc = S.acc;
        bsum = S.bsum;
        mask |= (uint32_t)(nb - 1) << sh;
        value |= (uint32_t)S.bucket << sh;
        ++level;
    }
    if (bsum / fix_weight(value) > (uint64_t)kCap) {
        // a run of more than kCap equal probabilities: the t-th of them in column order
        const uint64_t w = fix_weight(value);
        const uint64_t t = (target - acc + w - 1) / w;
        for (int b = tid; b < 2048; b += kThreads) S.hist[b] = 0;
        __syncthreads();
        int cur = -1;
        uint64_t run = 0;
        sweep(R, [&](int, float v, int tile) {
            if (tile != cur) {
                if (run) atomicAdd((unsigned long long*)&S.hist[cur], (unsigned long long)run);
                cur = tile;
                run = 0;
            }
            run += R.key(v) == value;
        });
        if (run) atomicAdd((unsigned long long*)&S.hist[cur], (unsigned long long)run);
        __syncthreads();
        hist_cross(S.hist, R.tiles(), false, t, 0, S);
        if (S.bucket < 0) return -1;
        const int tile = S.bucket;
        const uint64_t before = S.acc;
        const int col = tile_find(R, tile, t - before, [&](float v) -> uint64_t { return R.key(v) == value; }, S);
        *c_incl = acc + t * w;
        return col;
    }
    if (!(cs.n >= 0 && cs.mask == mask && cs.value == value)) {
        cs.n = collect_sorted(R, value, value | ~mask, 1u, 0u, S);
        cs.mask = mask;
        cs.value = value;
    }
    return cand_cross(cs.n, false, acc, target, S, c_incl);
}

__global__ __launch_bounds__(kThreads) void sample_kernel(const float* __restrict__ logits, int cols, int vec,
                                                          const SampleRowArgs* __restrict__ rows,
                                                          uint32_t* __restrict__ out) {
    __shared__ Shared S;
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SampleRowArgs a = rows[r];
    Row R;
    R.x = logits + (size_t)r * cols;
    R.cols = cols;
    R.vec = vec;
    R.mul = a.mul;
    R.m = 0.f;
    if (a.mode == 0) {  // argmax of the raw logits, first index on ties
        float bv = -INFINITY;
        int bi = INT_MAX;
        sweep(R, [&](int i, float v, int) {
            if (v > bv || bi == INT_MAX) {
                bv = v;
                bi = i;
            }
        });
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
            S.fm[wave] = bv;
            S.fi[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < kWaves; ++w)
                if (S.fm[w] > bv || (S.fm[w] == bv && S.fi[w] < bi)) {
                    bv = S.fm[w];
                    bi = S.fi[w];
                }
            out[r] = (uint32_t)(bi < cols ? bi : 0);
        }
        return;
    }
    // max of the scaled logits
    float mt = -INFINITY;
    sweep(R, [&](int, float v, int) { mt = fmaxf(mt, R.scaled(v)); });
#pragma unroll
    for (int o = 32; o; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o, 64));
    if (lane == 0) S.fm[wave] = mt;
    __syncthreads();
    float m = -INFINITY;
    for (int w = 0; w < kWaves; ++w) m = fmaxf(m, S.fm[w]);
    R.m = m;
    if (a.mode == 1) {
        // first column whose running weight reaches ceil(k * W / 2^24): each
        // wave sums a contiguous range, the crossing range is scanned
        const int span = (((cols + kWaves - 1) / kWaves) + 3) & ~3;
        uint64_t sum = 0;
        sweep_wave_range(R, span, [&](int, float v) { sum += fix_weight(R.key(v)); });
#pragma unroll
        for (int o = 32; o; o >>= 1) sum += __shfl_xor(sum, o, 64);
        if (lane == 0) S.hist[wave] = sum;
        __syncthreads();
        hist_cross(S.hist, kWaves, false, 0, 0, S);
        const uint64_t target = ceil_mul_shr(a.k, S.total, 24);
        int col = -1;
        if (target > 0) {
            hist_cross(S.hist, kWaves, false, target, 0, S);
            if (S.bucket >= 0) {
                const int start = S.bucket * span;
                col = range_find(R, start, min(cols - start, span), target - S.acc,
                                 [&](float v) { return fix_weight(R.key(v)); }, S);
            }
        }
        if (tid == 0) out[r] = (uint32_t)(col < 0 ? 0 : col);
        return;
    }
    // nucleus: the first-level histogram and each bucket's preceding weight
    for (int b = tid; b < kL1Buckets; b += kThreads) S.hist1[b] = 0;
    __syncthreads();
    sweep(R, [&](int, float v, int) {
        const uint32_t key = R.key(v);
        const uint64_t w = fix_weight(key);
        if (w) atomicAdd((unsigned long long*)&S.hist1[l1_bucket(key)], (unsigned long long)w);
    });
    __syncthreads();
    uint64_t total;
    {
        const int b = kL1Buckets - 1 - tid;  // descending
        const uint64_t mine = b >= 0 ? S.hist1[b] : 0;
        const uint64_t ex = block_exscan(mine, S, &total);
        if (b >= 0) S.pre1[b] = ex;
    }
    if (tid == 0) S.bucket = -1;
    __syncthreads();
    if (total == 0) {
        if (tid == 0) out[r] = 0;
        return;
    }
    // the last kept element: first with cum >= P (none when P > W: all kept);
    // the first-level buckets holding running weight P, then the range the
    // sampled target ceil(k * denom / 2^24) can reach, denom within bucket b1
    const uint64_t P = ceil_mul_shr(a.tp_m, total, a.tp_q);
    auto holds = [&](int b, uint64_t t) { return S.hist1[b] && S.pre1[b] < t && t <= S.pre1[b] + S.hist1[b]; };
    if (tid < kL1Buckets && P <= total && holds(tid, P)) S.bucket = tid;
    __syncthreads();
    const int b1 = S.bucket;
    const uint64_t dlo = b1 < 0 ? total : S.pre1[b1] + 1, dhi = b1 < 0 ? total : S.pre1[b1] + S.hist1[b1];
    uint64_t t2lo = ceil_mul_shr(a.k, dlo, 24), t2hi = ceil_mul_shr(a.k, dhi, 24);
    t2lo = t2lo < 1 ? 1 : t2lo;
    t2hi = t2hi < 1 ? 1 : t2hi;
    if (tid == 0) {
        S.first = -1;  // bh
        S.found = -1;  // bl
        S.acc = 0;     // element bound
    }
    __syncthreads();
    if (tid < kL1Buckets) {
        if (holds(tid, t2lo)) S.first = tid;
        if (holds(tid, t2hi)) S.found = tid;
    }
    __syncthreads();
    const int bh = S.first, bl = S.found;  // bl <= bh
    auto in_set = [&](int b) { return b == b1 || (b >= bl && b <= bh); };
    // elements in a bucket <= its weight / the weight of its smallest key
    if (tid < kL1Buckets && in_set(tid) && S.hist1[tid])
        atomicAdd((unsigned long long*)&S.acc, (unsigned long long)(S.hist1[tid] / l1_min_weight(tid)));
    __syncthreads();
    const uint64_t bound = S.acc;
    int col;
    if (bl >= 0 && bh >= 0 && bound <= (uint64_t)kCap) {
        // both crossings from one collected, sorted run
        // the set is b1 and bl..bh (b1 <= bl): one key range when adjacent
        const uint32_t lo_b1 = (uint32_t)(b1 + kL1Base) << 21, lo_bl = (uint32_t)(bl + kL1Base) << 21;
        const uint32_t hi_bh = ((uint32_t)(bh + kL1Base + 1) << 21) - 1;
        int n;
        if (b1 < 0 || b1 >= bl - 1)
            n = collect_sorted(R, b1 < 0 ? lo_bl : (b1 < bl ? lo_b1 : lo_bl), hi_bh, 1u, 0u, S);
        else
            n = collect_sorted(R, lo_b1, lo_b1 + (1u << 21) - 1, lo_bl, hi_bh, S);
        {
            // running-weight offset of each collected bucket: its preceding
            // weight less the collected weight of the buckets above it
            const int b = kL1Buckets - 1 - tid;  // descending
            const uint64_t mine = b >= 0 && in_set(b) ? S.hist1[b] : 0;
            uint64_t all;
            const uint64_t before = block_exscan(mine, S, &all);
            if (b >= 0 && in_set(b)) S.off[b] = S.pre1[b] - before;
            __syncthreads();
        }
        uint64_t denom = total;
        if (b1 >= 0) {
            uint64_t c = 0;
            if (cand_cross(n, true, 0, P, S, &c) >= 0) denom = c;
        }
        uint64_t t2 = ceil_mul_shr(a.k, denom, 24);
        t2 = t2 < 1 ? 1 : t2;
        uint64_t c2 = 0;
        col = cand_cross(n, true, 0, t2, S, &c2);
    } else {
        CandState cs{0u, 0u, -1};
        uint64_t denom = total;
        if (P <= total) {
            uint64_t c = 0;
            if (refine_cross(R, P, S, cs, &c) >= 0) denom = c;
        }
        uint64_t t2 = ceil_mul_shr(a.k, denom, 24);
        t2 = t2 < 1 ? 1 : t2;
        uint64_t c2 = 0;
        col = refine_cross(R, t2, S, cs, &c2);
    }
    if (tid == 0) out[r] = (uint32_t)(col < 0 ? 0 : col);
}

}  // namespace

// Host: per-row parameters (deterministic_sample_threshold in double, as the
// reference computes it; top_p as an exact fraction) and the launch.
// temperature / top_p / seeds are host arrays of `rows`; logits and out are
// device memory.
zr_status launch_sample(zr_context* ctx, const float* d_logits, int rows, int cols, const float* temperature,
                        const float* top_p, const uint64_t* seeds, uint32_t* d_out) {
    if (rows <= 0) return ZR_OK;
    if (cols <= 0) return set_err(ctx, ZR_E_INVALID, "Device sampling received an empty logits tensor");
    if (cols > kMaxCols)
        return set_err(ctx, ZR_E_INVALID, "Device sampling supports at most %d columns, got %d", kMaxCols, cols);
    std::vector<SampleRowArgs> h(rows);
    for (int r = 0; r < rows; ++r) {
        SampleRowArgs& a = h[r];
        const float T = temperature[r], P = top_p[r];
        a.mode = (T <= 0.0f || P <= 0.0f) ? 0 : (P >= 1.0f ? 1 : 2);
        a.mul = T != 1.0f ? 1.0f / T : 1.0f;
        a.tp_m = 0;
        a.tp_q = 0;
        if (a.mode == 2) {  // 0 < P < 1: P = f * 2^e, f in [0.5, 1) with 24 bits
            int e = 0;
            const float f = std::frexp(P, &e);
            a.tp_m = (uint32_t)std::ldexp(f, 24);
            a.tp_q = 24 - e;
        }
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
    const int vec = (cols % 4 == 0) && ((uintptr_t)d_logits % 16 == 0);
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassOther, &ev);
    hipLaunchKernelGGL(sample_kernel, dim3(rows), dim3(kThreads), 0, ctx->stream, d_logits, cols, vec,
                       (const SampleRowArgs*)ctx->sample_ws, d_out);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassOther, ev);
    // the host parameters must outlive the copy
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

}  // namespace zr
