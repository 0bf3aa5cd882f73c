// Shard projection GEMMs on MFMA: C[M,N] = A[M,K] @ W[K,N].
//
// W (bf16 weights, reference [in, out] layout) is repacked once at upload into
// MFMA B-operand fragments: fragment (nt, kt) is 64 lanes x 8 bf16 where lane l
// holds W[32*kt + 8*(l/16) + j][16*nt + l%16], j < 8, stored contiguously and
// fragments of one 16-column tile consecutive along K.  A wavefront streams
// its weights as perfectly coalesced 1 KiB loads, each element read once.
// A (f32 activations, L2-resident) is converted to bf16 -- or to a hi + lo
// pair under ZR_FLAG_SPLIT_ACTIVATIONS -- while it is staged through LDS.
// Matmul semantics: forward_pass.rs:1696-1714 (w_qkv / w_gate_up column
// concatenations), 2265 (O), 2290 (down), 2311 (LM head); f32 accumulation.
// The gate|up concatenation is interleaved per 16 columns so one 32-column
// pair holds matching gate and up values for the SwiGLU epilogue
// (silu(g) * u, forward_pass.rs:2286-2289).
#include "zr_internal.h"

#include <algorithm>

namespace zr {

size_t packed_weight_elems(int k, int n) {
    const size_t kt = (size_t)(k + 31) / 32, nt = (size_t)(n + 15) / 16;
    return kt * nt * 512;
}

// dst n-tile `nt_dst + i` takes source columns [16 * i, 16 * i + 16) of src
// [K, n_src] (zero outside); tile_stride lets gate/up interleave.
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ src, int K,
                                                          int n_src, int KT, int nt_dst0,
                                                          int tile_step, int n_tiles,
                                                          uint16_t* __restrict__ dst) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // one lane of one fragment
    const size_t total = (size_t)n_tiles * KT * 64;
    if (gid >= total) return;
    const int lane = (int)(gid % 64);
    const size_t frag = gid / 64;
    const int kt = (int)(frag % KT);
    const int i = (int)(frag / KT);
    const int nt = nt_dst0 + i * tile_step;
    const int n = i * 16 + (lane & 15);
    uint16_t* out = dst + (((size_t)nt * KT + kt) * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int k = kt * 32 + (lane >> 4) * 8 + j;
        out[j] = (k < K && n < n_src) ? src[(size_t)k * n_src + n] : (uint16_t)0;
    }
}

static zr_status pack_into(zr_context* ctx, const uint16_t* src, int k, int n, int KT, int nt0,
                           int step, uint16_t* dst) {
    const size_t bytes = (size_t)k * n * 2;
    uint16_t* tmp = nullptr;
    ZR_HIP(ctx, hipMalloc(&tmp, bytes));
    hipError_t e = hipMemcpyAsync(tmp, src, bytes, hipMemcpyDefault, ctx->stream);
    if (e == hipSuccess) {
        const int n_tiles = (n + 15) / 16;
        const size_t total = (size_t)n_tiles * KT * 64;
        hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream,
                           tmp, k, n, KT, nt0, step, n_tiles, dst);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    hipFree(tmp);
    if (e != hipSuccess) return set_err(ctx, ZR_E_HIP, "weight pack failed: %s", hipGetErrorString(e));
    return ZR_OK;
}

zr_status pack_weight(zr_context* ctx, const uint16_t* src, int k, int n, uint16_t** out) {
    const int* widths = &n;
    return pack_weight_concat(ctx, &src, widths, 1, k, out);
}

zr_status pack_weight_concat(zr_context* ctx, const uint16_t* const* srcs, const int* widths, int count,
                             int k, uint16_t** out) {
    int n_total = 0;
    for (int i = 0; i < count; ++i) {
        if (count > 1 && widths[i] % 16 != 0)
            return set_err(ctx, ZR_E_UNSUPPORTED, "concatenated projection width %d is not a multiple of 16",
                           widths[i]);
        n_total += widths[i];
    }
    const int KT = (k + 31) / 32;
    uint16_t* dst = nullptr;
    ZR_HIP(ctx, hipMalloc(&dst, packed_weight_elems(k, n_total) * 2));
    int nt0 = 0;
    for (int i = 0; i < count; ++i) {
        zr_status rc = pack_into(ctx, srcs[i], k, widths[i], KT, nt0, 1, dst);
        if (rc != ZR_OK) {
            hipFree(dst);
            return rc;
        }
        nt0 += (widths[i] + 15) / 16;
    }
    *out = dst;
    return ZR_OK;
}

// Interleaved [gate | up]: tile 2b = gate columns [16b, 16b+16), tile 2b+1 = up.
zr_status pack_weight_gate_up(zr_context* ctx, const uint16_t* gate, const uint16_t* up, int k, int f,
                              uint16_t** out) {
    if (f % 16 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "ffn width %d is not a multiple of 16", f);
    const int KT = (k + 31) / 32;
    uint16_t* dst = nullptr;
    ZR_HIP(ctx, hipMalloc(&dst, packed_weight_elems(k, 2 * f) * 2));
    zr_status rc = pack_into(ctx, gate, k, f, KT, 0, 2, dst);
    if (rc == ZR_OK) rc = pack_into(ctx, up, k, f, KT, 1, 2, dst);
    if (rc != ZR_OK) {
        hipFree(dst);
        return rc;
    }
    *out = dst;
    return ZR_OK;
}

// ------------------------------------------------------------------ GEMM
// Block = 4 wavefronts; block tile = (16*WM) rows x (4*WN*16) columns; each
// wave owns WN 16-column tiles and every row tile.  grid = (column blocks,
// K splits, row blocks).  HL = 2 feeds activations as hi + lo bf16 pairs.
template <int WM, int WN, int HL, int KCH>
__global__ __launch_bounds__(256) void gemm_kernel(const float* __restrict__ A, int M, int K,
                                                   const bf16x8* __restrict__ Wp, int KT, int NT,
                                                   float* __restrict__ C, int N, int kt_per_split,
                                                   size_t split_stride) {
    __shared__ bf16x8 lds[WM * KCH * HL * 64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nt0 = (blockIdx.x * 4 + wave) * WN;
    const int m0 = blockIdx.z * WM * 16;
    const int z = blockIdx.y;
    const int kt_begin = z * kt_per_split;
    const int kt_end = min(KT, kt_begin + kt_per_split);

    f32x4 acc[WM][WN];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) acc[mt][wn] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kc = kt_begin; kc < kt_end; kc += KCH) {
        // weights of this chunk first: they are the HBM stream
        bf16x8 b[KCH][WN];
#pragma unroll
        for (int ktl = 0; ktl < KCH; ++ktl)
#pragma unroll
            for (int wn = 0; wn < WN; ++wn) {
                const int nt = nt0 + wn, kt = kc + ktl;
                if (nt < NT && kt < kt_end)
                    b[ktl][wn] = Wp[((size_t)nt * KT + kt) * 64 + lane];
                else
                    b[ktl][wn] = bf16x8{};
            }
        __syncthreads();  // previous chunk finished reading LDS
        for (int gidx = threadIdx.x; gidx < WM * 16 * KCH * 4; gidx += 256) {
            const int row = gidx / (KCH * 4), rem = gidx - row * (KCH * 4);
            const int ktl = rem >> 2, q4 = rem & 3;
            const int m = m0 + row, k = (kc + ktl) * 32 + q4 * 8;
            float x[8];
            if (m < M && kc + ktl < kt_end && k < K) {
                const f32x4* src = (const f32x4*)(A + (size_t)m * K + k);
                const f32x4 lo4 = src[0], hi4 = src[1];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[j] = lo4[j];
                    x[4 + j] = hi4[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = 0.0f;
            }
            bf16x8 vh, vl;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint16_t h, l;
                split_bf16(x[j], h, l);
                vh[j] = __builtin_bit_cast(__bf16, h);
                vl[j] = __builtin_bit_cast(__bf16, l);
            }
            const int base = (((row >> 4) * KCH + ktl) * HL) * 64 + q4 * 16 + (row & 15);
            lds[base] = vh;
            if (HL == 2) lds[base + 64] = vl;
        }
        __syncthreads();
#pragma unroll
        for (int ktl = 0; ktl < KCH; ++ktl) {
#pragma unroll
            for (int mt = 0; mt < WM; ++mt) {
                const bf16x8 ah = lds[((mt * KCH + ktl) * HL) * 64 + lane];
#pragma unroll
                for (int wn = 0; wn < WN; ++wn)
                    acc[mt][wn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b[ktl][wn], acc[mt][wn], 0, 0, 0);
                if (HL == 2) {
                    const bf16x8 al = lds[((mt * KCH + ktl) * HL) * 64 + 64 + lane];
#pragma unroll
                    for (int wn = 0; wn < WN; ++wn)
                        acc[mt][wn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b[ktl][wn], acc[mt][wn], 0, 0, 0);
                }
            }
        }
    }
    float* out = C + (size_t)z * split_stride;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) {
            const int n = (nt0 + wn) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + mt * 16 + (lane >> 4) * 4 + i;
                if (m < M && n < N) out[(size_t)m * N + n] = acc[mt][wn][i];
            }
        }
}

// Sum of split-K slabs [S][M][N] with the epilogue.
// kEpiStore:  out[m][n] = sum
// kEpiSwiGLU: N = 2F interleaved per 16 columns; out[m][j] = silu(g) * u, out [M, F]
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int S, int M,
                                                            int N, size_t split_stride, int epilogue,
                                                            float* __restrict__ out) {
#pragma clang fp contract(off)
    const int n_out = epilogue == kEpiSwiGLU ? N / 2 : N;
    const size_t total = (size_t)M * n_out;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(idx / n_out), j = (int)(idx % n_out);
        if (epilogue == kEpiSwiGLU) {
            const int gc = (j >> 4) * 32 + (j & 15);
            float g = 0.0f, u = 0.0f;
            for (int s = 0; s < S; ++s) {
                g += ws[s * split_stride + (size_t)m * N + gc];
                u += ws[s * split_stride + (size_t)m * N + gc + 16];
            }
            out[idx] = g / (1.0f + expf(-g)) * u;
        } else {
            float v = 0.0f;
            for (int s = 0; s < S; ++s) v += ws[s * split_stride + (size_t)m * N + j];
            out[idx] = v;
        }
    }
}

template <int WM, int WN, int HL>
static void gemm_launch(dim3 grid, hipStream_t stream, const float* a, int m, int k, const uint16_t* w,
                        int KT, int NT, float* c, int n, int kt_per_split, size_t split_stride) {
    constexpr int KCH = std::min(8, std::max(1, 64 / (WM * HL)));
    hipLaunchKernelGGL((gemm_kernel<WM, WN, HL, KCH>), grid, dim3(256), 0, stream, a, m, k, (const bf16x8*)w, KT,
                       NT, c, n, kt_per_split, split_stride);
}

zr_status launch_gemm(zr_context* ctx, const float* a, const uint16_t* w_packed, float* c, int m, int n,
                      int k, int epilogue) {
    if (m <= 0) return ZR_OK;
    if (k % 8 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM K=%d must be a multiple of 8", k);
    const int KT = (k + 31) / 32, NT = (n + 15) / 16;
    constexpr int WN = 2;
    const int wm = m <= 16 ? 1 : m <= 32 ? 2 : m <= 64 ? 4 : m <= 128 ? 8 : 16;
    const int row_blocks = (m + wm * 16 - 1) / (wm * 16);
    const int col_blocks = (NT + 4 * WN - 1) / (4 * WN);
    // split K until the grid covers the chip ~2x, keeping >= 8 k-tiles per split
    int splits = 1;
    const int target = 2 * 256;
    while (col_blocks * row_blocks * splits < target && KT / (splits * 2) >= 8) splits *= 2;
    const int kt_per_split = (KT + splits - 1) / splits;
    splits = (KT + kt_per_split - 1) / kt_per_split;
    const bool direct = splits == 1 && epilogue == kEpiStore;
    const size_t split_stride = (size_t)m * n;
    if (!direct && (size_t)splits * split_stride > ctx->splitk_ws_floats)
        return set_err(ctx, ZR_E_OOM, "split-K workspace too small (%d x %d x %d)", splits, m, n);
    float* dst = direct ? c : ctx->splitk_ws;
    const bool split_act = (ctx->desc.flags & ZR_FLAG_SPLIT_ACTIVATIONS) != 0;
    dim3 grid(col_blocks, splits, row_blocks);
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassGemm, &ev);
#define ZR_GEMM_CASE(WMV)                                                                                    \
    case WMV:                                                                                                \
        if (split_act)                                                                                       \
            gemm_launch<WMV, WN, 2>(grid, ctx->stream, a, m, k, w_packed, KT, NT, dst, n, kt_per_split,     \
                                    split_stride);                                                          \
        else                                                                                                 \
            gemm_launch<WMV, WN, 1>(grid, ctx->stream, a, m, k, w_packed, KT, NT, dst, n, kt_per_split,     \
                                    split_stride);                                                          \
        break;
    switch (wm) {
        ZR_GEMM_CASE(1)
        ZR_GEMM_CASE(2)
        ZR_GEMM_CASE(4)
        ZR_GEMM_CASE(8)
        ZR_GEMM_CASE(16)
    }
#undef ZR_GEMM_CASE
    ZR_LAUNCH_CHECK(ctx);
    if (!direct) {
        const size_t n_out = epilogue == kEpiSwiGLU ? (size_t)n / 2 : (size_t)n;
        const size_t total = (size_t)m * n_out;
        const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65535);
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, ctx->stream, ctx->splitk_ws, splits,
                           m, n, split_stride, epilogue, c);
        ZR_LAUNCH_CHECK(ctx);
    }
    timing_mark_end(ctx, kClassGemm, ev);
    return ZR_OK;
}

}  // namespace zr
