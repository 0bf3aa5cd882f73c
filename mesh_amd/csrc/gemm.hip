// Shard projection GEMMs on MFMA: C[M,N] = A[M,K] @ W[K,N].
//
// W (bf16 weights, reference [in, out] layout) is repacked once at upload into
// MFMA B-operand fragments: fragment (nt, kt) is 64 lanes x 8 bf16 where lane l
// holds W[32*kt + 8*(l/16) + j][16*nt + l%16], j < 8, stored contiguously and
// fragments of one 16-column tile consecutive along K.  A wavefront streams
// its weights as perfectly coalesced 1 KiB loads, each element read once per
// row block, through a register ring PF k-steps deep.
// A (activations) arrives as bf16 [M, K] -- or a hi + lo bf16 pair under
// ZR_FLAG_SPLIT_ACTIVATIONS -- written by the producing kernel; a block
// stages its A rows through a double-buffered LDS tile shared by the waves
// that own different column slices.
// Matmul semantics: forward_pass.rs:1696-1714 (w_qkv / w_gate_up column
// concatenations), 2265 (O), 2290 (down), 2311 (LM head); f32 accumulation.
// The gate|up concatenation is interleaved per 16 columns so one 32-column
// pair holds matching gate and up values for the SwiGLU epilogue
// (silu(g) * u, forward_pass.rs:2286-2289).
#include "zr_internal.h"

#include <algorithm>
#include <cstdlib>

namespace zr {

size_t packed_weight_elems(int k, int n) {
    const size_t kt = (size_t)(k + 31) / 32, nt = (size_t)(n + 15) / 16;
    return kt * nt * 512;
}

// dst n-tile `nt_dst0 + i * tile_step` takes source columns [16 i, 16 i + 16)
// of src [K, n_src] (zero outside).
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ src, int K,
                                                          int n_src, int KT, int nt_dst0,
                                                          int tile_step, int n_tiles,
                                                          uint16_t* __restrict__ dst) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
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
// Block = WAVES_M x WAVES_N wavefronts; wave tile = (16 WM) rows x (16 WN)
// columns; block tile BM x BN.  grid = (column blocks, K splits, row blocks).
// Per k-step of 32: one barrier; the next A slice is loaded to registers
// before the MFMAs and written to the other LDS buffer after them; the
// weight fragments of k-step kt + PF are requested as soon as step kt's are
// consumed.
template <int WM, int WN, int WAVES_M, int WAVES_N, int PF, int HL>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm_kernel(
    const uint16_t* __restrict__ A, int M, int K, const bf16x8* __restrict__ Wp, int KT, int NT,
    float* __restrict__ C, int N, int kt_per_split, size_t split_stride) {
    constexpr int BM = WAVES_M * WM * 16;
    constexpr int NTHR = WAVES_M * WAVES_N * 64;
    constexpr int A_CHUNKS = BM * 4 * HL;  // 16-byte chunks of one k-step of A
    constexpr int A_PER_T = (A_CHUNKS + NTHR - 1) / NTHR;
    __shared__ bf16x8 lds[2][HL][BM / 16][64];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm_idx = wave / WAVES_N, wn_idx = wave % WAVES_N;
    const int m0 = blockIdx.z * BM;
    const int nt0 = blockIdx.x * (WAVES_N * WN) + wn_idx * WN;
    const int kt_begin = blockIdx.y * kt_per_split;
    const int kt_end = min(KT, kt_begin + kt_per_split);
    const size_t MK = (size_t)M * K;

    bf16x8 areg[A_PER_T];
    auto load_a = [&](int kt) {
#pragma unroll
        for (int j = 0; j < A_PER_T; ++j) {
            const int c = tid + j * NTHR;
            bf16x8 v = bf16x8{};
            if (c < A_CHUNKS) {
                const int hl = c / (BM * 4), r = c - hl * (BM * 4);
                const int m = r >> 2, q = r & 3;
                const int k = kt * 32 + q * 8;
                if (m0 + m < M && kt < kt_end && k < K)
                    v = *(const bf16x8*)(A + hl * MK + (size_t)(m0 + m) * K + k);
            }
            areg[j] = v;
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int j = 0; j < A_PER_T; ++j) {
            const int c = tid + j * NTHR;
            if (c < A_CHUNKS) {
                const int hl = c / (BM * 4), r = c - hl * (BM * 4);
                const int m = r >> 2, q = r & 3;
                lds[buf][hl][m >> 4][q * 16 + (m & 15)] = areg[j];
            }
        }
    };

    bf16x8 bring[PF][WN];
    auto load_b = [&](bf16x8* dst, int kt) {
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) {
            const int nt = nt0 + wn;
            dst[wn] = (nt < NT && kt < kt_end) ? Wp[((size_t)nt * KT + kt) * 64 + lane] : bf16x8{};
        }
    };

    f32x4 acc[WM][WN];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) acc[mt][wn] = f32x4{0.f, 0.f, 0.f, 0.f};

    load_a(kt_begin);
    store_a(0);
#pragma unroll
    for (int s = 0; s < PF; ++s) load_b(bring[s], kt_begin + s);

    int buf = 0;
    for (int kb = kt_begin; kb < kt_end; kb += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const int kt = kb + s;
            if (kt < kt_end) {  // uniform across the block
                load_a(kt + 1);
                __syncthreads();
#pragma unroll
                for (int mt = 0; mt < WM; ++mt) {
                    const bf16x8 ah = lds[buf][0][wm_idx * WM + mt][lane];
#pragma unroll
                    for (int wn = 0; wn < WN; ++wn)
                        acc[mt][wn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bring[s][wn], acc[mt][wn], 0, 0, 0);
                    if (HL == 2) {
                        const bf16x8 al = lds[buf][HL - 1][wm_idx * WM + mt][lane];
#pragma unroll
                        for (int wn = 0; wn < WN; ++wn)
                            acc[mt][wn] =
                                __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bring[s][wn], acc[mt][wn], 0, 0, 0);
                    }
                }
                load_b(bring[s], kt + PF);
                buf ^= 1;
                store_a(buf);
            }
        }
    }

    float* out = C + (size_t)blockIdx.y * split_stride;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) {
            const int n = (nt0 + wn) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + (wm_idx * WM + mt) * 16 + (lane >> 4) * 4 + i;
                if (m < M && n < N) out[(size_t)m * N + n] = acc[mt][wn][i];
            }
        }
}

// ------------------------------------------------- GEMM, LDS-DMA pipeline
// `s_waitcnt vmcnt(n)` with expcnt / lgkmcnt left unconstrained (gfx9
// encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

typedef __attribute__((address_space(3))) void lds_void;

// Both operands go global -> LDS with `global_load_lds_dwordx4` (no
// registers, no per-lane address math beyond one pointer): every 1 KiB MFMA
// fragment of a k-step -- A rows (hi, then lo) and packed weight tiles -- is
// one wave instruction, spread evenly over the block's waves.  STAGES-deep
// LDS ring: at step i a wave waits (vmcnt) for its own copies of stage i,
// the block barrier publishes the stage to every wave and retires the slot
// read at step i-1, which then takes stage i + STAGES - 1.  The compiler
// does not order LDS reads after these copies, hence the explicit waits.
// Block tile BM x BN = (16 WAVES_M WM) x (16 WAVES_N WN); wave tile
// (16 WM) x (16 WN).  Grid: 1-D, decoded so that the row blocks of one
// (column block, split) pair are dispatched 8 apart -- on the same XCD, one
// after the other -- and share that weight tile through its L2.
template <int WM, int WN, int WAVES_M, int WAVES_N, int HL, int STAGES>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm_dma_kernel(
    const uint16_t* __restrict__ A, int M, int K, const bf16x8* __restrict__ Wp, int KT, int NT,
    float* __restrict__ C, int N, int kt_per_split, int splits, int row_blocks, int col_blocks,
    size_t split_stride) {
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BMT = WAVES_M * WM, BNT = WAVES_N * WN;
    constexpr int FA = HL * BMT, FB = BNT, FS = FA + FB;
    constexpr int PW = (FS + NW - 1) / NW;  // copies per wave per stage
    constexpr int FSP = PW * NW;            // fragments per stage incl. padding
    static_assert(STAGES >= 2 && STAGES <= 4, "stages");
    static_assert(PW * (STAGES - 2) < 64, "vmcnt range");
    __shared__ bf16x8 lds[STAGES][FSP][64];

    const int b = blockIdx.x;
    const int j = b >> 3;
    const int rb = j % row_blocks;
    const int g = (j / row_blocks) * 8 + (b & 7);
    if (g >= col_blocks * splits) return;  // padding block of the XCD mapping
    const int cb = g / splits, split = g - cb * splits;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm_idx = wave / WAVES_N, wn_idx = wave - wm_idx * WAVES_N;
    const int m0 = rb * BMT * 16;
    const int nt_blk = cb * BNT;
    const int kt_begin = split * kt_per_split;
    const int nsteps = min(KT, kt_begin + kt_per_split) - kt_begin;
    const size_t MK = (size_t)M * K;

    auto issue = [&](int slot, int kt) {
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            int f = i * NW + wave;
            const int fs = f < FS ? f : f - FS;  // padding rows repeat a real fragment
            const void* src;
            if (fs < FA) {
                const int hl = fs / BMT, mt = fs - hl * BMT;
                const int row = min(m0 + mt * 16 + (lane & 15), M - 1);
                const int kc = min(kt * 32 + (lane >> 4) * 8, K - 8);
                src = A + (size_t)hl * MK + (size_t)row * K + kc;
            } else {
                const int nt = min(nt_blk + (fs - FA), NT - 1);
                src = Wp + ((size_t)nt * KT + kt) * 64 + lane;
            }
            __builtin_amdgcn_global_load_lds(src, (lds_void*)&lds[slot][f][0], 16, 0, 0);
        }
    };

    f32x4 acc[WM][WN];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) acc[mt][wn] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nsteps) issue(s, kt_begin + s);

    int slot = 0;
    for (int i = 0; i < nsteps; ++i) {
        const int ahead = min(STAGES - 2, nsteps - 1 - i);  // stages issued after stage i
        if (STAGES >= 4 && ahead >= 2)
            wait_vmcnt<PW * (STAGES >= 4 ? 2 : 0)>();
        else if (STAGES >= 3 && ahead == 1)
            wait_vmcnt<PW * (STAGES >= 3 ? 1 : 0)>();
        else
            wait_vmcnt<0>();
        __syncthreads();
        if (i + STAGES - 1 < nsteps) {
            int ns = slot + STAGES - 1;
            if (ns >= STAGES) ns -= STAGES;
            issue(ns, kt_begin + i + STAGES - 1);
        }
        const bf16x8* sa = &lds[slot][0][0];
        const bf16x8* sb = &lds[slot][FA][0];
        bf16x8 bf[WN];
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) bf[wn] = sb[(wn_idx * WN + wn) * 64 + lane];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int hl = 0; hl < HL; ++hl) {
                const bf16x8 af = sa[(hl * BMT + wm_idx * WM + mt) * 64 + lane];
#pragma unroll
                for (int wn = 0; wn < WN; ++wn)
                    acc[mt][wn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[wn], acc[mt][wn], 0, 0, 0);
            }
        if (++slot == STAGES) slot = 0;
    }

    float* out = C + (size_t)split * split_stride;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) {
            const int n = (nt_blk + wn_idx * WN + wn) * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + (wm_idx * WM + mt) * 16 + (lane >> 4) * 4 + i;
                if (m < M && n < N) out[(size_t)m * N + n] = acc[mt][wn][i];
            }
        }
}

// Sum of split-K slabs [S][M][N] with the epilogue.
// kEpiStore:  out_f32[m][n] = sum
// kEpiSwiGLU: N = 2F interleaved per 16 columns; h = silu(g) * u written as
//             bf16 hi (+ lo) [M, F] (the next GEMM's A operand) or f32.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int S, int M, int N,
                                                            size_t split_stride, int epilogue,
                                                            float* __restrict__ out_f32,
                                                            uint16_t* __restrict__ out_bf16, int out_lo) {
#pragma clang fp contract(off)
    const int n_out = epilogue == kEpiSwiGLU ? N / 2 : N;
    const size_t total = (size_t)M * n_out;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(idx / n_out), j = (int)(idx % n_out);
        float v;
        if (epilogue == kEpiSwiGLU) {
            const int gc = (j >> 4) * 32 + (j & 15);
            float g = 0.0f, u = 0.0f;
            for (int s = 0; s < S; ++s) {
                g += ws[s * split_stride + (size_t)m * N + gc];
                u += ws[s * split_stride + (size_t)m * N + gc + 16];
            }
            v = g / (1.0f + expf(-g)) * u;
        } else {
            v = 0.0f;
            for (int s = 0; s < S; ++s) v += ws[s * split_stride + (size_t)m * N + j];
        }
        if (out_bf16) {
            uint16_t hi, lo;
            split_bf16(v, hi, lo);
            out_bf16[idx] = hi;
            if (out_lo) out_bf16[total + idx] = lo;
        } else {
            out_f32[idx] = v;
        }
    }
}

// f32 [M, K] -> bf16 hi (+ lo) [M, K] (A operand of zr_gemm)
__global__ __launch_bounds__(256) void to_bf16_pair_kernel(const float* __restrict__ x, size_t n,
                                                           uint16_t* __restrict__ out, int with_lo) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint16_t hi, lo;
        split_bf16(x[i], hi, lo);
        out[i] = hi;
        if (with_lo) out[n + i] = lo;
    }
}

zr_status launch_to_bf16_pair(zr_context* ctx, const float* x, size_t n, uint16_t* out, int with_lo) {
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 16384);
    hipLaunchKernelGGL(to_bf16_pair_kernel, dim3(blocks), dim3(256), 0, ctx->stream, x, n, out, with_lo);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

// Tile configurations (wave tile WM x WN 16x16 tiles; WAVES_M x WAVES_N waves).
// family 0: register-ring kernel (gemm_kernel), for M <= 64 where the step
//           streams weights; family 1: LDS-DMA kernel (gemm_dma_kernel), for
//           M >= 128 where the hi + lo MFMA work dominates.
struct GemmCfg {
    int family, wm, wn, waves_m, waves_n, stages;
    int bm() const { return waves_m * wm * 16; }
    int bn() const { return waves_n * wn * 16; }
};

static bool dma_enabled() {
    static const bool on = !(getenv("ZR_GEMM_DMA") && atoi(getenv("ZR_GEMM_DMA")) == 0);
    return on;
}

// Measured on MI355X over the decode shapes with weights streamed from HBM:
// 2x2 wave tiles with 8 waves suit M <= 64; from 128 rows the LDS-DMA kernel
// with 128 x 256 block tiles (8 waves, 3 stages) wins, and for very wide N
// (the LM head) 4 waves with 2 stages, two blocks per CU.
static GemmCfg pick_cfg(int m, int n) {
    if (m <= 16) return {0, 1, 2, 1, 8, 0};
    if (m <= 32) return {0, 2, 2, 1, 8, 0};
    if (m <= 64) return {0, 4, 2, 1, 8, 0};
    if (!dma_enabled()) return m <= 128 ? GemmCfg{0, 4, 4, 2, 4, 0} : GemmCfg{0, 8, 4, 2, 4, 0};
    if (n >= 65536) return {1, 4, 8, 2, 2, 2};
    return {1, 4, 4, 2, 4, 3};
}

GemmPlan gemm_plan(int m, int n, int k, int epilogue) {
    GemmPlan p;
    const GemmCfg c = pick_cfg(m, n);
    p.KT = (k + 31) / 32;
    p.NT = (n + 15) / 16;
    p.row_blocks = (m + c.bm() - 1) / c.bm();
    p.col_blocks = (p.NT + c.bn() / 16 - 1) / (c.bn() / 16);
    int splits = 1;
    if (c.family == 0) {
        // split K while the grid has fewer than ~1.5 blocks per CU, keeping at
        // least 4 k-steps per split
        static const int target =
            getenv("ZR_GEMM_TARGET_BLOCKS") ? atoi(getenv("ZR_GEMM_TARGET_BLOCKS")) : 384;
        while (p.col_blocks * p.row_blocks * splits * 2 <= target && p.KT / (splits * 2) >= 4) splits *= 2;
    } else {
        // one resident block per CU (LDS-bound): split K while the grid still
        // fits one pass over the CUs, keeping at least 4 k-steps per split
        static const int cus = [] {
            int v = 256;
            int dev = 0;
            if (hipGetDevice(&dev) == hipSuccess)
                (void)hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
            return v > 0 ? v : 256;
        }();
        while (p.col_blocks * p.row_blocks * splits * 2 <= cus && p.KT / (splits * 2) >= 4) splits *= 2;
    }
    p.kt_per_split = (p.KT + splits - 1) / splits;
    p.splits = (p.KT + p.kt_per_split - 1) / p.kt_per_split;
    p.direct = p.splits == 1 && epilogue == kEpiStore;
    p.ws_floats = p.direct ? 0 : (size_t)p.splits * m * n;
    return p;
}

template <int WM, int WN, int WAVES_M, int WAVES_N, int HL>
static void gemm_launch(const GemmPlan& p, hipStream_t stream, const uint16_t* a, int m, int k,
                        const uint16_t* w, float* c, int n, size_t split_stride) {
    constexpr int PF = 4;
    dim3 grid(p.col_blocks, p.splits, p.row_blocks);
    hipLaunchKernelGGL((gemm_kernel<WM, WN, WAVES_M, WAVES_N, PF, HL>), grid, dim3(WAVES_M * WAVES_N * 64), 0,
                       stream, a, m, k, (const bf16x8*)w, p.KT, p.NT, c, n, p.kt_per_split, split_stride);
}

template <int WM, int WN, int WAVES_M, int WAVES_N, int STAGES, int HL>
static void gemm_dma_launch(const GemmPlan& p, hipStream_t stream, const uint16_t* a, int m, int k,
                            const uint16_t* w, float* c, int n, size_t split_stride) {
    const int groups = p.col_blocks * p.splits;
    const unsigned blocks = 8u * (unsigned)p.row_blocks * (unsigned)((groups + 7) / 8);
    hipLaunchKernelGGL((gemm_dma_kernel<WM, WN, WAVES_M, WAVES_N, HL, STAGES>), dim3(blocks),
                       dim3(WAVES_M * WAVES_N * 64), 0, stream, a, m, k, (const bf16x8*)w, p.KT, p.NT, c, n,
                       p.kt_per_split, p.splits, p.row_blocks, p.col_blocks, split_stride);
}

zr_status launch_gemm(zr_context* ctx, const uint16_t* a, const uint16_t* w_packed, float* c_f32,
                      uint16_t* c_bf16, int m, int n, int k, int epilogue, Slabs* deferred) {
    if (deferred && (epilogue != kEpiStore || !c_f32 || c_bf16))
        return set_err(ctx, ZR_E_INVARIANT, "deferred split-K needs an f32 store epilogue");
    if (m <= 0) return ZR_OK;
    if (k % 8 != 0 || k < 8) return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM K=%d must be a multiple of 8", k);
    const GemmPlan p = gemm_plan(m, n, k, epilogue);
    const GemmCfg cfg = pick_cfg(m, n);
    const bool direct = p.direct && c_f32 && !c_bf16;
    const size_t split_stride = (size_t)m * n;
    if (!direct && (size_t)p.splits * split_stride > ctx->splitk_ws_floats)
        return set_err(ctx, ZR_E_OOM, "split-K workspace too small (%d x %d x %d)", p.splits, m, n);
    float* dst = direct ? c_f32 : ctx->splitk_ws;
    const bool split_act = (ctx->desc.flags & ZR_FLAG_SPLIT_ACTIVATIONS) != 0;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassGemm, &ev);
    bool launched = false;
#define ZR_GEMM_CASE(WMV, WNV, WAM, WAN)                                                              \
    if (!launched && cfg.family == 0 && cfg.wm == WMV && cfg.wn == WNV && cfg.waves_m == WAM &&        \
        cfg.waves_n == WAN) {                                                                         \
        if (split_act)                                                                                \
            gemm_launch<WMV, WNV, WAM, WAN, 2>(p, ctx->stream, a, m, k, w_packed, dst, n, split_stride); \
        else                                                                                          \
            gemm_launch<WMV, WNV, WAM, WAN, 1>(p, ctx->stream, a, m, k, w_packed, dst, n, split_stride); \
        launched = true;                                                                              \
    }
#define ZR_GEMM_DMA_CASE(WMV, WNV, WAM, WAN, ST)                                                      \
    if (!launched && cfg.family == 1 && cfg.wm == WMV && cfg.wn == WNV && cfg.waves_m == WAM &&        \
        cfg.waves_n == WAN && cfg.stages == ST) {                                                     \
        if (split_act)                                                                                \
            gemm_dma_launch<WMV, WNV, WAM, WAN, ST, 2>(p, ctx->stream, a, m, k, w_packed, dst, n,      \
                                                       split_stride);                                 \
        else                                                                                          \
            gemm_dma_launch<WMV, WNV, WAM, WAN, ST, 1>(p, ctx->stream, a, m, k, w_packed, dst, n,      \
                                                       split_stride);                                 \
        launched = true;                                                                              \
    }
    ZR_GEMM_CASE(1, 2, 1, 8)
    ZR_GEMM_CASE(2, 2, 1, 8)
    ZR_GEMM_CASE(4, 2, 1, 8)
    ZR_GEMM_CASE(4, 4, 2, 4)
    ZR_GEMM_CASE(8, 4, 2, 4)
    ZR_GEMM_DMA_CASE(4, 4, 2, 4, 3)
    ZR_GEMM_DMA_CASE(4, 8, 2, 2, 2)
#undef ZR_GEMM_CASE
#undef ZR_GEMM_DMA_CASE
    if (!launched) return set_err(ctx, ZR_E_INVARIANT, "no GEMM kernel for the selected tile configuration");
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassGemm, ev);
    if (deferred) {
        *deferred = direct ? Slabs(c_f32) : Slabs(ctx->splitk_ws, p.splits, split_stride);
        return ZR_OK;
    }
    if (!direct) {
        timing_mark_begin(ctx, kClassOther, &ev);
        const size_t n_out = epilogue == kEpiSwiGLU ? (size_t)n / 2 : (size_t)n;
        const size_t total = (size_t)m * n_out;
        const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65535);
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, ctx->stream, ctx->splitk_ws, p.splits,
                           m, n, split_stride, epilogue, c_f32, c_bf16, split_act ? 1 : 0);
        ZR_LAUNCH_CHECK(ctx);
        timing_mark_end(ctx, kClassOther, ev);
    }
    return ZR_OK;
}

}  // namespace zr
