// KV snapshot wire format on the device.
//
// export: the bytes KVCache::to_bytes (kv_cache.rs:880-887; ciborium 0.2.2,
// Cargo.lock:627-629) writes for the cache DeviceKVCache::export_snapshot
// (forward_pass.rs:1169-1204) builds, encoded from the gathered K / V rows.
// import: a host decoder of the same document (import_snapshot,
// forward_pass.rs:1206-1242, reads it back through KVCache::from_bytes,
// kv_cache.rs:889-895).
//
// Document (serde derive: a struct is a definite map of field-name text ->
// value in declaration order; None = null; usize = unsigned integer; Vec =
// definite array; RFC 8949 heads in their shortest form):
//   {"layers": [ per layer l:
//      {"keys":   {"data": [f32 x rows*cols], "rows": r, "cols": c},
//       "values": {"data": [...], "rows": r, "cols": c},
//       "seq_len": r, "layer_idx": l} ],
//    "base_position": b,
//    "config": {"num_layers", "num_heads", "head_dim", "max_seq_len"}}
// (KVCache kv_cache.rs:664-672, LayerKVCache 505-515, Tensor2D
// tensor_ops.rs:23-31, KVCacheConfig kv_cache.rs:190-200.)
// Each f32 is widened to f64 and written as the narrowest IEEE float that
// converts back to the same bits: half (0xf9) when the value is exactly a
// binary16, else single (0xfa).  NaN (never in a valid cache): quieted, half
// when the quieted payload fits its 10 bits, else double (0xfb).
//
// The float stream is the 2L arrays in document order (K of layer 0, V of
// layer 0, K of layer 1, ...).  Everything between two arrays (and before
// the first, after the last) is a fixed byte string built on the host.  The
// device pass is a byte-size count per 2048-float chunk, an exclusive scan of
// the chunk sizes, and a write pass that lays each chunk's bytes out in LDS
// (chunk-local scan over its threads) and stores them with 16 B vector
// stores into the chunk's slot of the output.
#include "zr_internal.h"

#include <cstring>
#include <vector>

namespace zr {

namespace {

constexpr int kCborThreads = 256;
constexpr int kCborPerThread = 8;
constexpr int kCborChunk = kCborThreads * kCborPerThread;  // floats per block
constexpr int kCborStage = 22528;                           // LDS bytes of one chunk (bound checked on the host)

// binary16 bits of an f32 when the value is exactly a binary16 (see header).
__host__ __device__ inline bool cbor_half(uint32_t u, uint32_t* h) {
    const uint32_t s = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a == 0) {
        *h = s;
        return true;
    }
    if (a >= 0x7f800000u) {
        if (a == 0x7f800000u) {
            *h = s | 0x7c00u;
            return true;
        }
        const uint32_t m = (a & 0x7fffffu) | 0x400000u;  // quieted NaN
        if (m & 0x1fffu) return false;
        *h = s | 0x7c00u | (m >> 13);
        return true;
    }
    if (a < 0x00800000u) return false;  // f32 subnormal: below every binary16
    const int e = (int)(a >> 23) - 127;
    const uint32_t sig = (a & 0x7fffffu) | 0x800000u;  // value = sig * 2^(e - 23)
    if (e > 15) return false;
    if (e >= -14) {
        if (sig & 0x1fffu) return false;
        *h = s | ((uint32_t)(e + 15) << 10) | ((sig >> 13) & 0x3ffu);
        return true;
    }
    if (e < -24) return false;
    const int sh = -(e + 1);  // binary16 subnormal k * 2^-24 with k = sig >> sh
    if (sig & ((1u << sh) - 1u)) return false;
    *h = s | (sig >> sh);
    return true;
}

__host__ __device__ inline int cbor_float_size(uint32_t u) {
    uint32_t h;
    if (cbor_half(u, &h)) return 3;
    return (u & 0x7fffffffu) > 0x7f800000u ? 9 : 5;
}

__device__ inline void cbor_float_write(uint32_t u, uint8_t* o) {
    uint32_t h;
    if (cbor_half(u, &h)) {
        o[0] = 0xf9;
        o[1] = (uint8_t)(h >> 8);
        o[2] = (uint8_t)h;
    } else if ((u & 0x7fffffffu) <= 0x7f800000u) {
        o[0] = 0xfa;
        o[1] = (uint8_t)(u >> 24);
        o[2] = (uint8_t)(u >> 16);
        o[3] = (uint8_t)(u >> 8);
        o[4] = (uint8_t)u;
    } else {
        const uint64_t d = ((uint64_t)(u >> 31) << 63) | 0x7ff0000000000000ull |
                           ((uint64_t)((u & 0x7fffffu) | 0x400000u) << 29);
        o[0] = 0xfb;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[1 + i] = (uint8_t)(d >> (56 - 8 * i));
    }
}

struct CborArgs {
    const float* k;            // [L][n]
    const float* v;            // [L][n]
    long long n;               // floats per array (rows * cols, a multiple of 16)
    long long total;           // 2 L n
    int arrays;                // 2 L
    const uint8_t* hdr;        // prefix byte strings, then the suffix
    const uint32_t* hdr_off;   // [arrays + 1]
    const uint32_t* hdr_len;   // [arrays + 1]
    uint32_t* chunk_bytes;     // [chunks]
    unsigned long long* chunk_off;  // [chunks]: offset inside the chunk's group of 1024
    unsigned long long* group_off;  // [groups + 1]: group offsets, then the document size
    uint8_t* out;
};

// This thread's 8 floats (one array: n is a multiple of 16) and their bytes,
// including the prefix of an array that starts here and the suffix after the
// last float of the stream.
struct ThreadSpan {
    long long i0;
    int count;
    int array;
    long long within;
};

__device__ inline ThreadSpan thread_span(const CborArgs& a, long long chunk) {
    ThreadSpan t;
    t.i0 = chunk * kCborChunk + (long long)threadIdx.x * kCborPerThread;
    const long long left = a.total - t.i0;
    t.count = left <= 0 ? 0 : (left < kCborPerThread ? (int)left : kCborPerThread);
    t.array = t.count ? (int)(t.i0 / a.n) : 0;
    t.within = t.count ? t.i0 - (long long)t.array * a.n : 0;
    return t;
}

__device__ inline void load_floats(const CborArgs& a, const ThreadSpan& t, uint32_t* u) {
    const float* src = ((t.array & 1) ? a.v : a.k) + (long long)(t.array >> 1) * a.n + t.within;
    const uint4* s4 = (const uint4*)src;
#pragma unroll
    for (int q = 0; q < kCborPerThread / 4; ++q) {
        const uint4 w = s4[q];
        u[4 * q] = w.x;
        u[4 * q + 1] = w.y;
        u[4 * q + 2] = w.z;
        u[4 * q + 3] = w.w;
    }
}

__device__ inline uint32_t thread_bytes(const CborArgs& a, const ThreadSpan& t, const uint32_t* u) {
    if (!t.count) return 0;
    uint32_t b = t.within == 0 ? a.hdr_len[t.array] : 0u;
#pragma unroll
    for (int j = 0; j < kCborPerThread; ++j) b += cbor_float_size(u[j]);
    if (t.i0 + kCborPerThread >= a.total) b += a.hdr_len[a.arrays];
    return b;
}

__device__ inline uint32_t block_sum(uint32_t x, uint32_t* red) {
#pragma unroll
    for (int o = 32; o; o >>= 1) x += __shfl_xor(x, o, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < kCborThreads / 64; ++w) s += red[w];
    return s;
}

__global__ __launch_bounds__(kCborThreads) void cbor_count_kernel(CborArgs a) {
    __shared__ uint32_t red[kCborThreads / 64];
    const ThreadSpan t = thread_span(a, blockIdx.x);
    uint32_t u[kCborPerThread];
    if (t.count) load_floats(a, t, u);
    const uint32_t b = block_sum(thread_bytes(a, t, u), red);
    if (threadIdx.x == 0) a.chunk_bytes[blockIdx.x] = b;
}

// Exclusive scan of the chunk sizes in two levels: each 1024-thread block
// scans 1024 chunks (chunk_off = offset inside its group) and writes the
// group's total; one block then scans the group totals (group_off, and the
// document size at group_off[groups]).
__device__ inline unsigned long long block_exclusive_1024(unsigned long long x, unsigned long long* wtot,
                                                         unsigned long long* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned long long incl = x;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wtot[wave] = incl;
    __syncthreads();
    unsigned long long base = 0, all = 0;
    for (int w = 0; w < 16; ++w) {
        if (w < wave) base += wtot[w];
        all += wtot[w];
    }
    *total = all;
    return base + incl - x;
}

__global__ __launch_bounds__(1024) void cbor_scan_groups_kernel(const uint32_t* __restrict__ bytes, int chunks,
                                                                unsigned long long* __restrict__ off,
                                                                unsigned long long* __restrict__ group_tot) {
    __shared__ unsigned long long wtot[16];
    const int c = blockIdx.x * 1024 + threadIdx.x;
    unsigned long long total;
    const unsigned long long ex = block_exclusive_1024(c < chunks ? bytes[c] : 0u, wtot, &total);
    if (c < chunks) off[c] = ex;
    if (threadIdx.x == 0) group_tot[blockIdx.x] = total;
}

__global__ __launch_bounds__(1024) void cbor_scan_top_kernel(const unsigned long long* __restrict__ group_tot,
                                                             int groups, unsigned long long* __restrict__ group_off) {
    __shared__ unsigned long long wtot[16];
    unsigned long long run = 0;
    for (int g0 = 0; g0 < groups; g0 += 1024) {  // block-uniform loop
        const int g = g0 + threadIdx.x;
        unsigned long long total;
        const unsigned long long ex = block_exclusive_1024(g < groups ? group_tot[g] : 0ull, wtot, &total);
        if (g < groups) group_off[g] = run + ex;
        run += total;
        __syncthreads();
    }
    if (threadIdx.x == 0) group_off[groups] = run;
}

// One block per chunk.  A thread whose 8 floats are all halves (the common
// case for bf16-valued rows) and hold no header bytes builds its 24 bytes as
// 6 little-endian words (f9 hi lo per float), shifts them to the LDS word
// grid and stores whole words (edge words, shared with the neighbours, byte
// by byte); other threads store byte by byte.  The chunk then leaves LDS in
// 16 B vector stores.
__global__ __launch_bounds__(kCborThreads) void cbor_write_kernel(CborArgs a) {
    __shared__ __align__(16) uint8_t stage[kCborStage + 16];
    __shared__ uint32_t wsum[kCborThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = blockIdx.x;
    const unsigned long long g = a.chunk_off[c] + a.group_off[c >> 10];
    uint32_t u[kCborPerThread];
    const ThreadSpan t = thread_span(a, c);
    if (t.count) load_floats(a, t, u);
    const uint32_t mine = thread_bytes(a, t, u);
    uint32_t incl = mine;  // exclusive scan of `mine` over the block
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kCborThreads / 64; ++w) {
        if (w < wave) base += wsum[w];
        total += wsum[w];
    }
    const uint32_t shift = (uint32_t)(g & 15u);  // stage byte s <-> output byte (g & ~15) + s
    const uint32_t off = shift + base + (incl - mine);
    uint32_t hv[kCborPerThread];
    bool all_half = t.count && t.within != 0 && t.i0 + kCborPerThread < a.total;
#pragma unroll
    for (int j = 0; j < kCborPerThread; ++j) {
        uint32_t h = 0;
        all_half = cbor_half(u[j], &h) && all_half;
        hv[j] = h;
    }
    if (all_half) {
        constexpr int NW = 3 * kCborPerThread / 4;
        uint32_t w[NW];
#pragma unroll
        for (int q = 0; q < kCborPerThread / 4; ++q) {  // f9 a1 a0 f9 | b1 b0 f9 c1 | c0 f9 d1 d0
            const uint32_t h0 = hv[4 * q], h1 = hv[4 * q + 1], h2 = hv[4 * q + 2], h3 = hv[4 * q + 3];
            w[3 * q] = 0xf9u | ((h0 >> 8) << 8) | ((h0 & 0xffu) << 16) | (0xf9u << 24);
            w[3 * q + 1] = (h1 >> 8) | ((h1 & 0xffu) << 8) | (0xf9u << 16) | ((h2 >> 8) << 24);
            w[3 * q + 2] = (h2 & 0xffu) | (0xf9u << 8) | ((h3 >> 8) << 16) | ((h3 & 0xffu) << 24);
        }
        const uint32_t sb = off & 3u, wb = off >> 2;
        uint32_t* sw = (uint32_t*)stage;
        if (sb == 0) {
#pragma unroll
            for (int i = 0; i < NW; ++i) sw[wb + i] = w[i];
        } else {
            const uint32_t lsh = 8 * sb, rsh = 32 - lsh;
            const uint32_t first = w[0] << lsh;  // bytes sb..3 of word wb are ours
            for (uint32_t b = sb; b < 4; ++b) stage[(wb << 2) + b] = (uint8_t)(first >> (8 * b));
#pragma unroll
            for (int k = 1; k < NW; ++k) sw[wb + k] = (w[k] << lsh) | (w[k - 1] >> rsh);
            const uint32_t last = w[NW - 1] >> rsh;  // bytes 0..sb-1 of word wb + NW are ours
            for (uint32_t b = 0; b < sb; ++b) stage[((wb + NW) << 2) + b] = (uint8_t)(last >> (8 * b));
        }
    } else if (t.count) {
        uint8_t* o = stage + off;
        if (t.within == 0) {
            const uint8_t* h = a.hdr + a.hdr_off[t.array];
            for (uint32_t i = 0; i < a.hdr_len[t.array]; ++i) *o++ = h[i];
        }
#pragma unroll
        for (int j = 0; j < kCborPerThread; ++j) {
            cbor_float_write(u[j], o);
            o += cbor_float_size(u[j]);
        }
        if (t.i0 + kCborPerThread >= a.total) {
            const uint8_t* h = a.hdr + a.hdr_off[a.arrays];
            for (uint32_t i = 0; i < a.hdr_len[a.arrays]; ++i) *o++ = h[i];
        }
    }
    __syncthreads();
    // 16 B segments of [shift, shift + total); partial end segments byte by byte
    const uint32_t end = shift + total;
    const uint32_t segs = (end + 15) / 16;
    uint8_t* dst = a.out + (g & ~15ull);
    for (uint32_t q = threadIdx.x; q < segs; q += kCborThreads) {
        const uint32_t s0 = q * 16;
        if (s0 >= shift && s0 + 16 <= end) {
            *(uint4*)(dst + s0) = *(const uint4*)(stage + s0);
        } else {
            for (uint32_t s = max(s0, shift); s < min(s0 + 16, end); ++s) dst[s] = stage[s];
        }
    }
}

// ------------------------------------------------------------ host side --

struct CborWriter {
    std::vector<uint8_t> b;
    void head(int major, uint64_t v) {
        const uint8_t m = (uint8_t)(major << 5);
        if (v <= 23) {
            b.push_back((uint8_t)(m | v));
            return;
        }
        const int n = v <= 0xffu ? 1 : v <= 0xffffu ? 2 : v <= 0xffffffffu ? 4 : 8;
        b.push_back((uint8_t)(m | (n == 1 ? 24 : n == 2 ? 25 : n == 4 ? 26 : 27)));
        for (int i = n - 1; i >= 0; --i) b.push_back((uint8_t)(v >> (8 * i)));
    }
    void text(const char* s) {
        const size_t n = strlen(s);
        head(3, n);
        b.insert(b.end(), s, s + n);
    }
    void uint_field(const char* name, uint64_t v) {
        text(name);
        head(0, v);
    }
};

}  // namespace

KvCborLayout kv_cbor_layout(int layers, int rows, int cols, long long base_position, const int cfg[4]) {
    KvCborLayout lay;
    const uint64_t n = (uint64_t)rows * (uint64_t)cols;
    auto tensor_tail = [&](CborWriter& w) {  // after the data array
        w.uint_field("rows", (uint64_t)rows);
        w.uint_field("cols", (uint64_t)cols);
    };
    auto add = [&](CborWriter& w) {
        lay.off.push_back((uint32_t)lay.bytes.size());
        lay.len.push_back((uint32_t)w.b.size());
        lay.bytes.insert(lay.bytes.end(), w.b.begin(), w.b.end());
    };
    for (int l = 0; l < layers; ++l) {
        CborWriter k;  // before K data of layer l
        if (l == 0) {
            k.head(5, 3);
            k.text("layers");
            k.head(4, (uint64_t)layers);
        } else {
            tensor_tail(k);
            k.uint_field("seq_len", (uint64_t)rows);
            k.uint_field("layer_idx", (uint64_t)(l - 1));
        }
        k.head(5, 4);
        k.text("keys");
        k.head(5, 3);
        k.text("data");
        k.head(4, n);
        add(k);
        CborWriter v;  // between K and V data
        tensor_tail(v);
        v.text("values");
        v.head(5, 3);
        v.text("data");
        v.head(4, n);
        add(v);
    }
    CborWriter s;  // after the last V data
    tensor_tail(s);
    s.uint_field("seq_len", (uint64_t)rows);
    s.uint_field("layer_idx", (uint64_t)(layers - 1));
    s.uint_field("base_position", (uint64_t)base_position);
    s.text("config");
    s.head(5, 4);
    s.uint_field("num_layers", (uint64_t)cfg[0]);
    s.uint_field("num_heads", (uint64_t)cfg[1]);
    s.uint_field("head_dim", (uint64_t)cfg[2]);
    s.uint_field("max_seq_len", (uint64_t)cfg[3]);
    add(s);
    return lay;
}

// Encodes the gathered rows d_k / d_v ([layers][rows][cols] f32 on the
// device).  out == nullptr: only *out_len.  Returns ZR_E_INVALID (with
// *out_len set) when capacity is short.
zr_status launch_kv_cbor(zr_context* ctx, const float* d_k, const float* d_v, int layers, int rows, int cols,
                         long long base_position, const int cfg[4], uint8_t* out, size_t capacity,
                         size_t* out_len) {
    if (rows <= 0 || layers <= 0) return set_err(ctx, ZR_E_INVALID, "empty KV export has no CBOR document");
    if (cols % kCborPerThread != 0)
        return set_err(ctx, ZR_E_UNSUPPORTED, "KV row width %d is not a multiple of %d", cols, kCborPerThread);
    const KvCborLayout lay = kv_cbor_layout(layers, rows, cols, base_position, cfg);
    const long long n = (long long)rows * cols;
    const long long total = 2LL * layers * n;
    const long long chunks = (total + kCborChunk - 1) / kCborChunk;
    if (chunks > (1LL << 30)) return set_err(ctx, ZR_E_UNSUPPORTED, "KV export of %lld floats too large", total);
    // bound on one chunk's bytes: floats at 9 B, the prefixes of the arrays that start in it, the suffix
    uint32_t max_pre = 0;
    for (size_t i = 0; i + 1 < lay.len.size(); ++i) max_pre = std::max(max_pre, lay.len[i]);
    const long long starts = kCborChunk / n + 2;
    if ((long long)kCborChunk * 9 + starts * max_pre + lay.len.back() > kCborStage)
        return set_err(ctx, ZR_E_UNSUPPORTED, "KV rows of %lld floats per layer too short for the CBOR chunking", n);
    // workspace: chunk sizes, offsets, header tables (grown on demand)
    const size_t tab = lay.off.size();
    const long long groups = (chunks + 1023) / 1024;
    const size_t need = 64 + (size_t)chunks * 12 + (2 * (size_t)groups + 1) * 8 + tab * 8 + lay.bytes.size();
    if (need > ctx->cbor_ws_bytes) {
        ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (ctx->cbor_ws) (void)hipFree(ctx->cbor_ws);
        ctx->cbor_ws = nullptr;
        ctx->cbor_ws_bytes = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->cbor_ws, need));
        ctx->cbor_ws_bytes = need;
    }
    uint8_t* ws = (uint8_t*)ctx->cbor_ws;
    unsigned long long* d_off = (unsigned long long*)ws;
    unsigned long long* d_gtot = d_off + chunks;
    unsigned long long* d_goff = d_gtot + groups;
    uint32_t* d_bytes = (uint32_t*)(d_goff + groups + 1);
    uint32_t* d_hoff = d_bytes + chunks;
    uint32_t* d_hlen = d_hoff + tab;
    uint8_t* d_hdr = (uint8_t*)(d_hlen + tab);
    std::vector<uint32_t> tables(2 * tab);
    memcpy(tables.data(), lay.off.data(), tab * 4);
    memcpy(tables.data() + tab, lay.len.data(), tab * 4);
    ZR_HIP(ctx, hipMemcpyAsync(d_hoff, tables.data(), tables.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    ZR_HIP(ctx, hipMemcpyAsync(d_hdr, lay.bytes.data(), lay.bytes.size(), hipMemcpyHostToDevice, ctx->stream));

    CborArgs a;
    a.k = d_k;
    a.v = d_v;
    a.n = n;
    a.total = total;
    a.arrays = 2 * layers;
    a.hdr = d_hdr;
    a.hdr_off = d_hoff;
    a.hdr_len = d_hlen;
    a.chunk_bytes = d_bytes;
    a.chunk_off = d_off;
    a.group_off = d_goff;
    a.out = nullptr;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassKvCbor, &ev);
    hipLaunchKernelGGL(cbor_count_kernel, dim3((unsigned)chunks), dim3(kCborThreads), 0, ctx->stream, a);
    ZR_LAUNCH_CHECK(ctx);
    hipLaunchKernelGGL(cbor_scan_groups_kernel, dim3((unsigned)groups), dim3(1024), 0, ctx->stream, d_bytes,
                       (int)chunks, d_off, d_gtot);
    ZR_LAUNCH_CHECK(ctx);
    hipLaunchKernelGGL(cbor_scan_top_kernel, dim3(1), dim3(1024), 0, ctx->stream, d_gtot, (int)groups, d_goff);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassKvCbor, ev);
    unsigned long long doc = 0;
    ZR_HIP(ctx, hipMemcpyAsync(&doc, d_goff + groups, 8, hipMemcpyDeviceToHost, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (out_len) *out_len = (size_t)doc;
    if (!out) return ZR_OK;
    if (capacity < doc)
        return set_err(ctx, ZR_E_INVALID, "CBOR buffer of %zu bytes is too small: the snapshot needs %llu", capacity,
                       doc);
    if (doc + 16 > ctx->cbor_out_bytes) {
        if (ctx->cbor_out) (void)hipFree(ctx->cbor_out);
        ctx->cbor_out = nullptr;
        ctx->cbor_out_bytes = 0;
        ZR_HIP(ctx, hipMalloc(&ctx->cbor_out, doc + 16));
        ctx->cbor_out_bytes = doc + 16;
    }
    a.out = (uint8_t*)ctx->cbor_out;
    timing_mark_begin(ctx, kClassKvCbor, &ev);
    hipLaunchKernelGGL(cbor_write_kernel, dim3((unsigned)chunks), dim3(kCborThreads), 0, ctx->stream, a);
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassKvCbor, ev);
    ZR_HIP(ctx, hipMemcpyAsync(out, ctx->cbor_out, doc, hipMemcpyDeviceToHost, ctx->stream));
    ZR_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ZR_OK;
}

// ------------------------------------------------------------- decoder --
// Strict reader of the document above as serde / ciborium would accept it for
// these structs: struct fields in any order, unknown fields skipped, floats
// of any width, integers of any width for usize fields, definite lengths.

namespace {

struct CborReader {
    const uint8_t* p;
    size_t n, i = 0;
    const char* err = nullptr;
    bool fail(const char* m) {
        if (!err) err = m;
        return false;
    }
    bool head(int* major, uint64_t* arg, int* info) {
        if (i >= n) return fail("truncated CBOR document");
        const uint8_t b = p[i++];
        *major = b >> 5;
        *info = b & 31;
        if (*info < 24) {
            *arg = (uint64_t)*info;
            return true;
        }
        const int len = *info == 24 ? 1 : *info == 25 ? 2 : *info == 26 ? 4 : *info == 27 ? 8 : 0;
        if (!len) return fail("indefinite or reserved CBOR length");
        if (i + len > n) return fail("truncated CBOR document");
        uint64_t v = 0;
        for (int k = 0; k < len; ++k) v = (v << 8) | p[i++];
        *arg = v;
        return true;
    }
    bool uint(uint64_t* v) {
        int m, info;
        if (!head(&m, v, &info)) return false;
        return m == 0 ? true : fail("expected an unsigned integer");
    }
    bool text(std::string* s) {
        int m, info;
        uint64_t len;
        if (!head(&m, &len, &info)) return false;
        if (m != 3) return fail("expected a text key");
        if (i + len > n) return fail("truncated CBOR document");
        s->assign((const char*)p + i, (size_t)len);
        i += (size_t)len;
        return true;
    }
    bool map(uint64_t* count) {
        int m, info;
        if (!head(&m, count, &info)) return false;
        return m == 5 ? true : fail("expected a map");
    }
    bool is_null() {
        if (i < n && p[i] == 0xf6) {
            ++i;
            return true;
        }
        return false;
    }
    bool f32(float* out) {
        if (i >= n) return fail("truncated CBOR document");
        const uint8_t b = p[i];
        const int len = b == 0xf9 ? 2 : b == 0xfa ? 4 : b == 0xfb ? 8 : 0;
        if (!len) return fail("expected a float");
        if (i + 1 + len > n) return fail("truncated CBOR document");
        uint64_t v = 0;
        for (int k = 0; k < len; ++k) v = (v << 8) | p[i + 1 + k];
        i += 1 + len;
        if (len == 4) {
            uint32_t u = (uint32_t)v;
            memcpy(out, &u, 4);
        } else if (len == 8) {
            double d;
            memcpy(&d, &v, 8);
            *out = (float)d;
        } else {
            const uint32_t h = (uint32_t)v, s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
            uint32_t u;
            if (e == 0x1f)
                u = s | 0x7f800000u | (m << 13);
            else if (e)
                u = s | ((e + 112) << 23) | (m << 13);
            else if (m == 0)
                u = s;
            else {  // binary16 subnormal m * 2^-24, normal in binary32
                int sh = 0;
                uint32_t mm = m;
                while (!(mm & 0x400u)) {
                    mm <<= 1;
                    ++sh;
                }
                u = s | ((uint32_t)(113 - sh) << 23) | ((mm & 0x3ffu) << 13);
            }
            memcpy(out, &u, 4);
        }
        return true;
    }
    bool skip(int depth = 0) {  // one data item
        if (depth > 64) return fail("CBOR nesting too deep");
        int m, info;
        uint64_t arg;
        if (!head(&m, &arg, &info)) return false;
        switch (m) {
            case 0:
            case 1:
                return true;
            case 2:
            case 3:
                if (i + arg > n) return fail("truncated CBOR document");
                i += (size_t)arg;
                return true;
            case 4:
                for (uint64_t k = 0; k < arg; ++k)
                    if (!skip(depth + 1)) return false;
                return true;
            case 5:
                for (uint64_t k = 0; k < arg; ++k)
                    if (!skip(depth + 1) || !skip(depth + 1)) return false;
                return true;
            case 6:
                return skip(depth + 1);
            default:  // simple values and floats: head() consumed the payload
                return true;
        }
    }
    // Tensor2D {data, rows, cols} into dst (rows * cols floats appended)
    bool tensor(std::vector<float>* dst, uint64_t* rows, uint64_t* cols) {
        uint64_t fields;
        if (!map(&fields)) return false;
        bool has_data = false, has_rows = false, has_cols = false;
        size_t start = dst->size();
        for (uint64_t f = 0; f < fields; ++f) {
            std::string key;
            if (!text(&key)) return false;
            if (key == "data") {
                int m, info;
                uint64_t count;
                if (!head(&m, &count, &info)) return false;
                if (m != 4) return fail("Tensor2D data is not an array");
                if (count > (n - i)) return fail("truncated CBOR document");
                dst->resize(start + (size_t)count);
                float* d = dst->data() + start;
                for (uint64_t k = 0; k < count; ++k)
                    if (!f32(d + k)) return false;
                has_data = true;
            } else if (key == "rows") {
                if (!uint(rows)) return false;
                has_rows = true;
            } else if (key == "cols") {
                if (!uint(cols)) return false;
                has_cols = true;
            } else if (!skip()) {
                return false;
            }
        }
        if (!has_data || !has_rows || !has_cols) return fail("Tensor2D misses a field");
        if (dst->size() - start != *rows * *cols) return fail("Tensor2D data length differs from rows x cols");
        return true;
    }
};

}  // namespace

bool kv_cbor_decode(const uint8_t* bytes, size_t len, KvCborDoc* doc, std::string* err) {
    CborReader r{bytes, len};
    uint64_t fields;
    bool ok = r.map(&fields);
    bool has_layers = false;
    doc->base_position = 0;  // #[serde(default)]
    doc->rows = 0;
    doc->cols = 0;
    doc->layers = 0;
    for (uint64_t f = 0; ok && f < fields; ++f) {
        std::string key;
        if (!(ok = r.text(&key))) break;
        if (key == "layers") {
            int m, info;
            uint64_t count;
            if (!(ok = r.head(&m, &count, &info))) break;
            if (m != 4) {
                ok = r.fail("layers is not an array");
                break;
            }
            doc->layers = (int)count;
            for (uint64_t l = 0; ok && l < count; ++l) {
                uint64_t lf;
                if (!(ok = r.map(&lf))) break;
                uint64_t seq_len = 0, layer_idx = l, kr = 0, kc = 0, vr = 0, vc = 0;
                bool kp = false, vp = false, has_seq = false;
                for (uint64_t g = 0; ok && g < lf; ++g) {
                    std::string k2;
                    if (!(ok = r.text(&k2))) break;
                    if (k2 == "keys") {
                        if (!r.is_null()) {
                            ok = r.tensor(&doc->k, &kr, &kc);
                            kp = true;
                        }
                    } else if (k2 == "values") {
                        if (!r.is_null()) {
                            ok = r.tensor(&doc->v, &vr, &vc);
                            vp = true;
                        }
                    } else if (k2 == "seq_len") {
                        ok = r.uint(&seq_len);
                        has_seq = true;
                    } else if (k2 == "layer_idx") {
                        ok = r.uint(&layer_idx);
                    } else {
                        ok = r.skip();
                    }
                }
                if (!ok) break;
                if (!has_seq) {
                    ok = r.fail("LayerKVCache misses seq_len");
                    break;
                }
                // LayerKVCache::validate (kv_cache.rs:587-622)
                if (kp != vp) {
                    ok = r.fail("KV cache invariant violated: keys/values presence diverged");
                    break;
                }
                if (kp && (kr != vr || kc != vc || seq_len != kr)) {
                    ok = r.fail("KV cache invariant violated: keys / values / seq_len shapes differ");
                    break;
                }
                if (!kp && seq_len != 0) {
                    ok = r.fail("KV cache invariant violated: empty tensors with nonzero seq_len");
                    break;
                }
                // KVCache::validate: one seq_len for all layers; one width
                if (l == 0) {
                    doc->rows = (long long)seq_len;
                    doc->cols = kp ? (long long)kc : 0;
                } else if ((long long)seq_len != doc->rows || (kp && (long long)kc != doc->cols)) {
                    ok = r.fail("KV cache invariant violated across layers");
                    break;
                }
            }
            has_layers = ok;
        } else if (key == "base_position") {
            uint64_t b;
            ok = r.uint(&b);
            doc->base_position = (long long)b;
        } else if (key == "config") {
            uint64_t cf;
            if (!(ok = r.map(&cf))) break;
            for (uint64_t g = 0; ok && g < cf; ++g) {
                std::string k2;
                uint64_t v = 0;
                if (!(ok = r.text(&k2))) break;
                if (!(ok = r.uint(&v))) break;
                if (k2 == "num_layers") doc->cfg[0] = (long long)v;
                else if (k2 == "num_heads") doc->cfg[1] = (long long)v;
                else if (k2 == "head_dim") doc->cfg[2] = (long long)v;
                else if (k2 == "max_seq_len") doc->cfg[3] = (long long)v;
            }
        } else {
            ok = r.skip();
        }
    }
    if (ok && !has_layers) ok = r.fail("KVCache misses layers");
    if (ok && r.i != len) ok = r.fail("trailing bytes after the CBOR document");
    if (!ok && err) *err = r.err ? r.err : "malformed CBOR document";
    return ok;
}

}  // namespace zr
