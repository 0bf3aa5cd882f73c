// Shard projection GEMMs on MFMA: C[M,N] = A[M,K] @ W[K,N].
//
// W (bf16 weights, reference [in, out] layout) is repacked once at upload into
// MFMA B-operand fragments of v_mfma_f32_32x32x16_bf16 (on gfx950 it issues
// at the rate of 16x16x32 with twice the work): fragment (nt, kt16) is 64
// lanes x 8 bf16, lane l holding W[16 kt16 + 8 (l / 32) + j][32 nt + l % 32],
// j < 8, stored contiguously; fragments of one 32-column tile are consecutive
// along K (kt16 < 2 ceil(K / 32), zero padded).  A wavefront streams its
// weights as perfectly coalesced 1 KiB loads.
// A (activations) arrives fragment-packed (a_pack_index: 1 KiB fragments of
// 32 rows x 16 columns) as bf16 -- or a hi + lo bf16 pair under
// ZR_FLAG_SPLIT_ACTIVATIONS -- written that way by the producing kernel.
// Matmul semantics: forward_pass.rs:1696-1714 (w_qkv / w_gate_up column
// concatenations), 2265 (O), 2290 (down), 2311 (LM head); f32 accumulation.
// The gate|up concatenation is interleaved per 32 columns so one 64-column
// pair holds matching gate and up values for the SwiGLU epilogue
// (silu(g) * u, forward_pass.rs:2286-2289).
#include "zr_internal.h"

#include <algorithm>
#include <cstdlib>

namespace zr {

size_t packed_weight_elems(int k, int n) {
    const size_t kt16 = 2 * (size_t)((k + 31) / 32), nt = (size_t)(n + 31) / 32;
    return kt16 * nt * 512;
}

// dst 32-column tile `nt_dst0 + i * tile_step` takes source columns
// [32 i, 32 i + 32) of src [K, n_src] (zero outside).
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint16_t* __restrict__ src, int K, int n_src,
                                                          int KT16, int nt_dst0, int tile_step, int n_tiles,
                                                          uint16_t* __restrict__ dst) {
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)n_tiles * KT16 * 64;
    if (gid >= total) return;
    const int lane = (int)(gid % 64);
    const size_t frag = gid / 64;
    const int kt = (int)(frag % KT16);
    const int i = (int)(frag / KT16);
    const int nt = nt_dst0 + i * tile_step;
    const int n = i * 32 + (lane & 31);
    uint16_t* out = dst + (((size_t)nt * KT16 + kt) * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int k = kt * 16 + (lane >> 5) * 8 + j;
        out[j] = (k < K && n < n_src) ? src[(size_t)k * n_src + n] : (uint16_t)0;
    }
}

static zr_status pack_into(zr_context* ctx, const uint16_t* src, int k, int n, int nt0, int step, uint16_t* dst) {
    const size_t bytes = (size_t)k * n * 2;
    const int KT16 = 2 * ((k + 31) / 32);
    uint16_t* tmp = nullptr;
    ZR_HIP(ctx, hipMalloc(&tmp, bytes));
    hipError_t e = hipMemcpyAsync(tmp, src, bytes, hipMemcpyDefault, ctx->stream);
    if (e == hipSuccess) {
        const int n_tiles = (n + 31) / 32;
        const size_t total = (size_t)n_tiles * KT16 * 64;
        hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream,
                           tmp, k, n, KT16, nt0, step, n_tiles, dst);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
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
        if (count > 1 && widths[i] % 32 != 0)
            return set_err(ctx, ZR_E_UNSUPPORTED, "concatenated projection width %d is not a multiple of 32",
                           widths[i]);
        n_total += widths[i];
    }
    uint16_t* dst = nullptr;
    ZR_HIP(ctx, hipMalloc(&dst, packed_weight_elems(k, n_total) * 2));
    int nt0 = 0;
    for (int i = 0; i < count; ++i) {
        zr_status rc = pack_into(ctx, srcs[i], k, widths[i], nt0, 1, dst);
        if (rc != ZR_OK) {
            (void)hipFree(dst);
            return rc;
        }
        nt0 += (widths[i] + 31) / 32;
    }
    *out = dst;
    return ZR_OK;
}

// Interleaved [gate | up]: tile 2b = gate columns [32b, 32b+32), tile 2b+1 = up.
zr_status pack_weight_gate_up(zr_context* ctx, const uint16_t* gate, const uint16_t* up, int k, int f,
                              uint16_t** out) {
    if (f % 32 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "ffn width %d is not a multiple of 32", f);
    uint16_t* dst = nullptr;
    ZR_HIP(ctx, hipMalloc(&dst, packed_weight_elems(k, 2 * f) * 2));
    zr_status rc = pack_into(ctx, gate, k, f, 0, 2, dst);
    if (rc == ZR_OK) rc = pack_into(ctx, up, k, f, 1, 2, dst);
    if (rc != ZR_OK) {
        (void)hipFree(dst);
        return rc;
    }
    *out = dst;
    return ZR_OK;
}

// silu(g) * u = g / (1 + e^-g) * u (runtime.rs:927-929, forward_pass.rs:2286-2289),
// one rounding per operation as written.
__device__ inline float swiglu(float g, float u) {
#pragma clang fp contract(off)
    return g / (1.0f + expf(-g)) * u;
}

// ------------------------------------------------------------------ GEMM
// v_mfma_f32_32x32x16_bf16: A fragment lane l holds A[row l % 32][k 8 (l / 32)
// + j]; the product lane l, element i is C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].
// Block tile BM x BN = (32 WAVES_M WM) x (32 WAVES_N WN); wave tile
// (32 WM) x (32 WN); a k-step covers 32 of K (two MFMA k-halves).
// Both operands go global -> LDS with `buffer_load_dwordx4 ... lds` (no
// registers): every 1 KiB MFMA fragment of a k-step -- A rows (hi, then lo)
// and weight tiles -- is one wave instruction, spread evenly over the
// block's waves.  STAGES-deep ring: halfway through step i a wave waits
// (vmcnt) for its own copies of stage i + 1, the block barrier publishes that
// stage to every wave and retires slot i (all of its reads have returned),
// and the copies of stage i + STAGES go into slot i.  The compiler does not
// order LDS reads after these copies, hence the explicit waits; on gfx950 a
// copy into LDS retires with vmcnt only (an lgkmcnt(0) wait does not cover
// it, measured), so the ring waits on vmcnt.  (Measured on
// the decode shapes: 4 or 5 stages instead of 3, streaming the weights into
// per-wave registers, staging both operands through registers + ds_write,
// or two k-steps per stage, are each no faster; the per-half register
// pipeline below is 3-8 % faster than reading each fragment just before
// its MFMAs.)
// Grid: 1-D, decoded so that the row blocks of one (column block, split)
// pair are dispatched 8 apart -- on the same XCD, one after the other -- and
// share that weight tile through its L2.
// SWIGLU = 1: single split; column tiles come in gate / up pairs (tile 2b is
// gate, 2b + 1 up, WN even) and silu(g) * u is written straight to H as the
// next GEMM's fragment-packed bf16 hi (+ lo when h_lo) operand [M, N / 2].
template <int WM, int WN, int WAVES_M, int WAVES_N, int HL, int STAGES, int SWIGLU>
__global__ __launch_bounds__(WAVES_M* WAVES_N * 64) void gemm_kernel(
    const uint16_t* __restrict__ A, int M, int K, const bf16x8* __restrict__ Wp, int KT, int NT,
    float* __restrict__ C, int N, int kt_per_split, int splits, int row_blocks, int col_blocks,
    size_t split_stride, uint16_t* __restrict__ H, int h_lo) {
    static_assert(!SWIGLU || WN % 2 == 0, "gate / up tile pairs");
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BMT = WAVES_M * WM, BNT = WAVES_N * WN;
    constexpr int FA = HL * BMT * 2, FB = BNT * 2, FS = FA + FB;
    constexpr int PW = (FS + NW - 1) / NW;  // LDS copies per wave per stage
    constexpr int FSP = PW * NW;            // fragments per stage incl. padding
    constexpr int VM = PW;                  // vector-memory ops per wave per stage
    static_assert(STAGES >= 2 && STAGES <= 6, "stages");
    static_assert(VM * (STAGES - 2) < 64, "vmcnt range");
    typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
    __shared__ bf16x8 lds[STAGES][FSP][64];

    const int b = blockIdx.x;
    const int j = b >> 3;
    const int rb = j % row_blocks;
    const int g = (j / row_blocks) * 8 + (b & 7);
    if (g >= col_blocks * splits) return;  // padding block of the XCD mapping
    const int cb = g / splits, split = g - cb * splits;

    // the wave index is uniform: readfirstlane keeps it (and every copy
    // offset derived from it) in scalar registers
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wm_idx = wave / WAVES_N, wn_idx = wave - wm_idx * WAVES_N;
    const int m0 = rb * BMT * 32;
    const int nt_blk = cb * BNT;
    const int KT16 = 2 * KT;
    const int MT = (M + 31) / 32;  // row tiles of the packed A operand
    const int kt_begin = split * kt_per_split;
    const int nsteps = min(KT, kt_begin + kt_per_split) - kt_begin;

    // Copies are buffer loads into LDS: the lane's 16 B of a 1 KiB fragment
    // is a constant vector offset, the fragment's byte offset a scalar, so
    // the per-step address arithmetic stays in the scalar unit.  Offsets are
    // 32-bit: packed operands stay below 2 GiB (zr_context_create refuses
    // geometries past it; launch_gemm checks again).
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_w = __builtin_amdgcn_make_buffer_rsrc((void*)Wp, 0, 0x7fffffff, 0x00020000);
    const int voff = lane * 16;
    auto issue = [&](int slot, int kt) {
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            int f = i * NW + wave;
            const int fs = f < FS ? f : f - FS;  // padding rows repeat a real fragment
            if (fs < FA) {
                // fragment-packed A: row tile (clamped into the operand), k-slice 2 kt + kh
                const int kh = fs & 1, r = fs >> 1;
                const int hl = r / BMT, mt = min(m0 / 32 + (r - hl * BMT), MT - 1);
                const int off = (((hl * MT + mt) * KT16 + 2 * kt + kh) << 10);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_void*)&lds[slot][f][0], 16, voff, off, 0, 0);
            } else {
                const int fb = fs - FA;
                const int nt = min(nt_blk + (fb >> 1), NT - 1);
                const int off = ((nt * KT16 + 2 * kt + (fb & 1)) << 10);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_w, (lds_void*)&lds[slot][f][0], 16, voff, off, 0, 0);
            }
        }
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int wn = 0; wn < WN; ++wn)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][wn][i] = 0.0f;

    // fragments of one k-half (16 k) in registers: kh 0 / kh 1 alternate so
    // that one half's LDS reads are in flight while the other's MFMAs run
    auto load_frags = [&](int slot, int kh, bf16x8* fa, bf16x8* fb) {
#pragma unroll
        for (int wn = 0; wn < WN; ++wn) fb[wn] = lds[slot][FA + (wn_idx * WN + wn) * 2 + kh][lane];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int hl = 0; hl < HL; ++hl)
                fa[mt * HL + hl] = lds[slot][((hl * BMT + wm_idx * WM + mt) << 1) + kh][lane];
    };
    constexpr int NM = WM * HL * WN;  // MFMAs per k-half
    auto mfmas = [&](const bf16x8* fa, const bf16x8* fb, int t0, int t1) {
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            if (t < t0 || t >= t1) continue;
            const int mt = t / (HL * WN), hl = (t / WN) % HL, wn = t % WN;
            acc[mt][wn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[mt * HL + hl], fb[wn], acc[mt][wn], 0, 0, 0);
        }
    };
    bf16x8 fa0[WM * HL], fb0[WN], fa1[WM * HL], fb1[WN];

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nsteps) issue(s, kt_begin + s);
    if (nsteps > 0) {
        ring_wait<VM, STAGES - 2>(min(STAGES - 2, nsteps - 1));
        if (STAGES - 1 < nsteps) issue(STAGES - 1, kt_begin + STAGES - 1);
        load_frags(0, 0, fa0, fb0);
    }
    // Step i: first MFMA of kh 0, the kh 1 reads, the other kh 0 MFMAs; the
    // ring barrier for step i + 1 (its copies landed, slot i free) and the
    // copy of stage i + STAGES into slot i; first MFMA of kh 1, the kh 0 reads
    // of step i + 1, the other kh 1 MFMAs.  The scheduling barriers keep the
    // reads where they are.  After the last step the barrier and the reads
    // are idle (the slot's data is not used).  Each accumulator still sums
    // (kh 0, hi), (kh 0, lo), (kh 1, hi), (kh 1, lo) per k-step, in k order.
    for (int i0 = 0; i0 < nsteps; i0 += STAGES) {
#pragma unroll
        for (int u = 0; u < STAGES; ++u) {
            const int i = i0 + u;
            if (i >= nsteps) break;
            mfmas(fa0, fb0, 0, 1);
            __builtin_amdgcn_sched_barrier(0);
            load_frags(u, 1, fa1, fb1);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(fa0, fb0, 1, NM);
            ring_wait<VM, STAGES - 2>(max(0, min(STAGES - 2, nsteps - 2 - i)));
            if (i + STAGES < nsteps) issue(u, kt_begin + i + STAGES);
            mfmas(fa1, fb1, 0, 1);
            __builtin_amdgcn_sched_barrier(0);
            load_frags((u + 1) % STAGES, 0, fa0, fb0);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(fa1, fb1, 1, NM);
        }
    }

    if constexpr (SWIGLU) {
        // Each 32 x 32 tile of H (silu(g) * u of a gate / up tile pair) goes
        // through a per-wave LDS tile (row pitch 33): written in the product's
        // layout (lane = column), read back as 8 consecutive columns of a row
        // per lane, which is one 16-byte run of the fragment-packed operand.
        // One store per plane and 8 values instead of 8 2-byte stores
        // (256-session decode step: the 2-byte stores cost 0.33 ms of GEMM).
        // F = N / 2 is a multiple of 32 (the planner's SwiGLU requires N % 64
        // == 0), so a run is either whole or past F.
        constexpr int TP = 32 * 33;
        static_assert((size_t)NW * TP * sizeof(float) <= sizeof(lds), "transpose tiles fit the ring");
        const int F = N / 2;
        const size_t plane = a_plane(M, F);
        float* tp = (float*)&lds[0][0][0] + wave * TP;
        __syncthreads();  // every wave is past its last ring read
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int p = 0; p < WN / 2; ++p) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    tp[(8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * 33 + (lane & 31)] =
                        swiglu(acc[mt][2 * p][i], acc[mt][2 * p + 1][i]);
                __syncthreads();
                const int j0 = ((nt_blk + wn_idx * WN + 2 * p) >> 1) * 32;
                const int mb = m0 + (wm_idx * WM + mt) * 32;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int r = (lane + 64 * t) >> 2, grp = lane & 3;
                    const int m = mb + r, j = j0 + 8 * grp;
                    if (m < M && j < F) {
                        float x[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = tp[r * 33 + 8 * grp + e];
                        const size_t o = a_pack_index(m, j, F);
                        *(bf16x8*)(H + o) = to_bf16x8(x, false);
                        if (h_lo) *(bf16x8*)(H + plane + o) = to_bf16x8(x, true);
                    }
                }
                __syncthreads();  // the tile is read before the next one is written
            }
    } else {
        float* out = C + (size_t)split * split_stride;
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int wn = 0; wn < WN; ++wn) {
                const int n = (nt_blk + wn_idx * WN + wn) * 32 + (lane & 31);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int m = m0 + (wm_idx * WM + mt) * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                    if (m < M && n < N) out[(size_t)m * N + n] = acc[mt][wn][i];
                }
            }
    }
}

// gate/up + SwiGLU for at most 32 rows in one launch: K split over the 4
// waves of a workgroup instead of over workgroups (no slabs, no reduce
// kernel).  A workgroup owns one gate / up tile pair (64 columns of the
// interleaved product, 32 columns of H); wave w takes k-steps w, w + 4, ...
// through a ring of its own in LDS: it copies a step's 8 fragments (A hi / lo
// and both weight tiles, two k-halves each) with `buffer_load ... lds` and
// reads only what it copied, so its own vmcnt wait orders the ring and the
// waves never wait for one another until the end.  Each wave accumulates its
// steps in k order ((kh 0, hi), (kh 0, lo), (kh 1, hi), (kh 1, lo) per step);
// the four partial sums then meet in LDS and are added in wave order, and
// silu(g) * u goes to H as the next GEMM's fragment-packed bf16 hi (+ lo).
// Requires M <= 32 and KT % 4 == 0 (every wave the same number of steps).
// ring_wait without the block barrier: only this wave's copies order its ring
template <int N>
__device__ __forceinline__ void wave_copies_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // vmcnt(N), expcnt(7), lgkmcnt(0)
    asm volatile("" ::: "memory");
}
template <int VM, int MAXA>
__device__ __forceinline__ void wave_ring_wait(int ahead) {
    if constexpr (MAXA > 0) {
        if (ahead >= MAXA) {
            wave_copies_wait<VM * MAXA>();
            return;
        }
        wave_ring_wait<VM, MAXA - 1>(ahead);
    } else {
        wave_copies_wait<0>();
    }
}

template <int STAGES, int HL, int MT>
__global__ __launch_bounds__(256) void gemm_swiglu_ksplit_kernel(const uint16_t* __restrict__ A, int M, int K,
                                                                const bf16x8* __restrict__ Wp, int KT, int N,
                                                                uint16_t* __restrict__ H, int h_lo) {
    constexpr int FW = 2 * HL * MT + 4;  // fragments per k-step: A (hl, row tile, kh), then weights (tile, kh)
    typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
    __shared__ bf16x8 lds[4][STAGES][FW][64];
    const int pair = blockIdx.x;  // weight tiles 2 pair (gate), 2 pair + 1 (up)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int KT16 = 2 * KT;
    const int nsteps = KT / 4;
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsrc_w = __builtin_amdgcn_make_buffer_rsrc((void*)Wp, 0, 0x7fffffff, 0x00020000);
    const int voff = lane * 16;
    auto issue = [&](int slot, int step) {
        const int kt = step * 4 + wave;
#pragma unroll
        for (int hl = 0; hl < HL; ++hl)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int kh = 0; kh < 2; ++kh)  // row tile mt of the packed A operand (hi plane, then lo)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_void*)&lds[wave][slot][(hl * MT + mt) * 2 + kh][0],
                                                             16, voff, (((hl * MT + mt) * KT16 + 2 * kt + kh) << 10), 0,
                                                             0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_w,
                                                         (lds_void*)&lds[wave][slot][2 * HL * MT + t * 2 + kh][0], 16,
                                                         voff, (((2 * pair + t) * KT16 + 2 * kt + kh) << 10), 0, 0);
    };
    f32x16 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mt][t][i] = 0.0f;
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nsteps) issue(s, s);
    for (int i0 = 0; i0 < nsteps; i0 += STAGES) {
#pragma unroll
        for (int u = 0; u < STAGES; ++u) {
            const int i = i0 + u;
            if (i >= nsteps) break;
            // this wave's copies of step i have landed (later steps may still be in flight)
            wave_ring_wait<FW, STAGES - 2>(max(0, min(STAGES - 2, nsteps - 1 - i)));
            if (i + STAGES - 1 < nsteps) issue((u + STAGES - 1) % STAGES, i + STAGES - 1);
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const bf16x8 bg = lds[wave][u][2 * HL * MT + kh][lane], bu = lds[wave][u][2 * HL * MT + 2 + kh][lane];
#pragma unroll
                for (int hl = 0; hl < HL; ++hl)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const bf16x8 a = lds[wave][u][(hl * MT + mt) * 2 + kh][lane];
                        acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bg, acc[mt][0], 0, 0, 0);
                        acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bu, acc[mt][1], 0, 0, 0);
                    }
            }
        }
    }
    // the four partial sums meet in LDS (the ring is free once every wave is past its last step)
    __syncthreads();
    float* red = (float*)&lds[0][0][0][0];  // [wave][row tile][tile][i][lane]
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) red[(((wave * MT + mt) * 2 + t) * 16 + i) * 64 + lane] = acc[mt][t][i];
    __syncthreads();
    // thread (i-group tid / 64, lane): elements i = 4 (tid / 64) .. + 3 of each row tile's accumulators
    const int F = N / 2;
    const size_t plane = a_plane(M, F);
    const int j = pair * 32 + (lane & 31);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 4 * wave + q;
            const int m = 32 * mt + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            float g = red[((mt * 2 + 0) * 16 + i) * 64 + lane], up = red[((mt * 2 + 1) * 16 + i) * 64 + lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                g += red[(((w * MT + mt) * 2 + 0) * 16 + i) * 64 + lane];
                up += red[(((w * MT + mt) * 2 + 1) * 16 + i) * 64 + lane];
            }
            if (m < M && j < F) {
                uint16_t hi, lo;
                split_bf16(swiglu(g, up), hi, lo);
                const size_t o = a_pack_index(m, j, F);
                H[o] = hi;
                if (h_lo) H[plane + o] = lo;
            }
        }
}

// Sum of split-K slabs [S][M][N] with the epilogue.
// kEpiStore:  out_f32[m][n] = sum
// kEpiSwiGLU: N = 2F interleaved per 32 columns; h = silu(g) * u written as
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
            const int gc = (j >> 5) * 64 + (j & 31);
            float g = 0.0f, u = 0.0f;
            for (int s = 0; s < S; ++s) {
                g += ws[s * split_stride + (size_t)m * N + gc];
                u += ws[s * split_stride + (size_t)m * N + gc + 32];
            }
            v = swiglu(g, u);
        } else {
            v = 0.0f;
            for (int s = 0; s < S; ++s) v += ws[s * split_stride + (size_t)m * N + j];
        }
        if (out_bf16) {  // fragment-packed A operand of the next GEMM
            uint16_t hi, lo;
            split_bf16(v, hi, lo);
            const size_t o = a_pack_index(m, j, n_out);
            out_bf16[o] = hi;
            if (out_lo) out_bf16[a_plane(M, n_out) + o] = lo;
        } else {
            out_f32[idx] = v;
        }
    }
}

// f32 [rows, K] -> fragment-packed bf16 hi (+ lo) (A operand of zr_gemm)
__global__ __launch_bounds__(256) void to_bf16_pair_kernel(const float* __restrict__ x, int rows, int K,
                                                           uint16_t* __restrict__ out, int with_lo) {
    const size_t n = (size_t)rows * K, plane = a_plane(rows, K);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint16_t hi, lo;
        split_bf16(x[i], hi, lo);
        const size_t o = a_pack_index((int)(i / K), (int)(i % K), K);
        out[o] = hi;
        if (with_lo) out[plane + o] = lo;
    }
}

// fragment-packed bf16 hi (+ lo) [rows, K] -> f32 hi + lo (the value a GEMM
// operand stands for)
__global__ __launch_bounds__(256) void from_bf16_pair_kernel(const uint16_t* __restrict__ in, int rows, int K,
                                                             int with_lo, float* __restrict__ y) {
    const size_t n = (size_t)rows * K, plane = a_plane(rows, K);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const size_t o = a_pack_index((int)(i / K), (int)(i % K), K);
        const float hi = __uint_as_float((uint32_t)in[o] << 16);
        y[i] = with_lo ? hi + __uint_as_float((uint32_t)in[plane + o] << 16) : hi;
    }
}

zr_status launch_from_bf16_pair(zr_context* ctx, const uint16_t* in, int rows, int K, int with_lo, float* y) {
    if (K % 32 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM operand width %d is not a multiple of 32", K);
    const size_t n = (size_t)rows * K;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 16384);
    hipLaunchKernelGGL(from_bf16_pair_kernel, dim3(blocks), dim3(256), 0, ctx->stream, in, rows, K, with_lo, y);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

zr_status launch_to_bf16_pair(zr_context* ctx, const float* x, int rows, int K, uint16_t* out, int with_lo) {
    if (K % 32 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM operand width %d is not a multiple of 32", K);
    const size_t n = (size_t)rows * K;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 16384);
    hipLaunchKernelGGL(to_bf16_pair_kernel, dim3(blocks), dim3(256), 0, ctx->stream, x, rows, K, out, with_lo);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

// Tile configurations: wave tile WM x WN 32x32 tiles, WAVES_M x WAVES_N waves.
struct GemmCfg {
    int wm, wn, waves_m, waves_n, stages;
    bool small;  // many blocks per CU (weight streaming) rather than one
    int bm() const { return waves_m * wm * 32; }
    int bn() const { return waves_n * wn * 32; }
};

static int device_cus() {
    static const int cus = [] {
        int v = 256, dev = 0;
        if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
        return v > 0 ? v : 256;
    }();
    return cus;
}

// Measured on MI355X over the decode shapes with weights streamed from HBM
// (split activations): 32 x 128 tiles for <= 32 rows; 128-row tiles with
// 256 columns, or 512 for wide / deep products and the LM head.
static GemmCfg pick_cfg(int m, int n, int k, int epilogue = kEpiStore) {
    // A vocabulary-wide head over 129-256 rows (the 256-session decode step):
    // 256 x 256 tiles in 16-wave blocks, four waves per SIMD (128256 columns,
    // weights streamed from HBM: 319 us against 339 us with 8-wave 256 x 256
    // blocks).  The same blocks for the other decode products measured no
    // faster (gate / up) or slower; 64-row tiles, two blocks per CU, are
    // faster only while the weights sit in the last-level cache.
    if (m > 128 && m <= 256 && epilogue == kEpiStore && n >= 65536) return {2, 2, 4, 4, 3, false};
    // SwiGLU fused into the GEMM (one split, gate / up tile pairs in a wave) once
    // 128-row tiles fill the CUs; small row counts reduce split-K slabs instead.
    // 128 x 512 tiles once they alone fill two passes over the CUs (prefill-sized
    // row counts: gate/up at 2108 rows 838-850 us against 910-1117 with 128 x 256).
    if (epilogue == kEpiSwiGLU && m > 64) {
        const int wide_tiles = ((m + 127) / 128) * ((n + 511) / 512);
        if (wide_tiles >= 2 * device_cus()) return {2, 4, 2, 4, 3, false};
        // 65-128 rows: 64 x 256 tiles (two row blocks share each weight tile)
        // fill twice the CUs of one 128-row block (decode steps at 96 / 128
        // sessions -4.7 / -4.2 %); at 256 rows they are slower (GEMMs 7.5
        // against 6.8 ms per step)
        if (m <= 128) return {2, 2, 1, 4, 3, false};
        // 129-256 rows: the same 128 x 256 tiles in 16-wave blocks (32 x 64
        // wave tiles, four waves per SIMD to cover the copies' latency):
        // GEMM class 7.33-7.36 against 7.47-7.50 ms per 256-session step with
        // 8 waves.  The store products measured slower in 16-wave blocks.
        if (m <= 256) return {1, 2, 4, 4, 3, false};
        return {2, 2, 2, 4, 3, false};
    }
    // <= 32 rows: a 4-deep ring and one pass of splits over the CUs (TinyLlama
    // shapes at 32 rows, back to back with weights from HBM: QKV 4.84 us
    // against 5.27 with 3 stages and three blocks per CU, gate/up 15.6 against
    // 17.1 (2 slabs instead of 8 for the SwiGLU reduce), down 6.96 against
    // 7.48, LM head 26.8 unsplit against 28.2 + its reduce; O unchanged)
    if (m <= 32) return {1, 1, 1, 4, 4, false};
    // 33-64 rows the same way on 64-row tiles (the tensor-parallel shard step
    // at 64 sessions: 12.6k -> 13.4k tokens/s against ~3 blocks per CU and 3
    // stages, whose 16 slabs each consumer read back)
    if (m <= 64) return {2, 1, 1, 4, 4, false};
    // and the 65-128-row store products (QKV, O, down) on two or more 64-row
    // tiles: fewer split-K slabs for their consumers (decode steps at 96 / 128
    // sessions 10.5 -> 10.2 / 12.4 -> 11.3 ms; at 128 sessions the attention,
    // with RoPE inside, sums q from 2 QKV slabs instead of 10).  At 256 rows
    // the same plan costs the GEMMs what it saves their consumers.
    if (m <= 128 && epilogue == kEpiStore && n < 65536) return {2, 1, 1, 4, 4, false};
    // vocabulary-wide heads: 256-row tiles read each weight tile once
    if (n >= 65536) return m > 128 ? GemmCfg{2, 4, 4, 2, 3, false} : GemmCfg{2, 4, 2, 4, 3, false};
    if (n >= 16384) return {2, 4, 2, 4, 3, false};
    return {2, 2, 2, 4, 3, false};
}

static bool swiglu_fused(int m, int epilogue) { return epilogue == kEpiSwiGLU && m > 64; }

// <= 64 rows of gate / up: SwiGLU in one launch with K split over the waves of
// a workgroup (gemm_swiglu_ksplit_kernel; two 32-row tiles above 32 rows)
static bool swiglu_ksplit(int m, int n, int k, int epilogue) {
    return epilogue == kEpiSwiGLU && m <= 64 && n % 64 == 0 && ((k + 31) / 32) % 4 == 0;
}

GemmPlan gemm_plan(int m, int n, int k, int epilogue) {
    GemmPlan p;
    if (swiglu_ksplit(m, n, k, epilogue)) {
        p.KT = (k + 31) / 32;
        p.NT = (n + 31) / 32;
        p.row_blocks = 1;
        p.col_blocks = p.NT / 2;
        p.kt_per_split = p.KT;
        return p;  // one launch, no workspace
    }
    const GemmCfg c = pick_cfg(m, n, k, epilogue);
    p.KT = (k + 31) / 32;
    p.NT = (n + 31) / 32;
    p.row_blocks = (m + c.bm() - 1) / c.bm();
    p.col_blocks = (p.NT + c.bn() / 32 - 1) / (c.bn() / 32);
    // split K as far as the grid fits one pass over the CUs (one resident
    // block per CU for the large tiles, about three for the small
    // weight-streaming tiles), >= 4 k-steps per split, at most 16 splits
    const int tiles = p.col_blocks * p.row_blocks;
    const int budget = c.small ? 3 * device_cus() : device_cus();
    int splits = swiglu_fused(m, epilogue) ? 1 : std::max(1, std::min(std::min(16, budget / tiles), p.KT / 4));
    if (!swiglu_fused(m, epilogue) && !c.small && tiles > budget) {
        // More tiles than one pass: up to 4 splits when they fill the last
        // pass better.  Cost in passes of unsplit blocks: ceil(tiles S / CUs) / S,
        // plus per extra split one more f32 slab written and read back
        // (8 M N bytes at ~5 TB/s) against one pass of the hi + lo MFMA work
        // (4 BM BN K per CU at ~1.2 PFLOP/s): 480 tiles / (K CUs).  At 2108 rows
        // this picks S = 3 for O (K 4096) and 4 for down (K 14336): -20 to -30 %
        // per GEMM; QKV's slabs cost more than its tail (S = 1).
        const double slab = 480.0 * tiles / ((double)k * budget);
        double best = 1e30;
        for (int s = 1; s <= 4 && s <= std::max(1, p.KT / 4); ++s) {
            const double cost = (double)(((size_t)tiles * s + budget - 1) / budget) / s + slab * (s - 1);
            if (cost < best - 1e-9) {
                best = cost;
                splits = s;
            }
        }
    }
    p.kt_per_split = (p.KT + splits - 1) / splits;
    p.splits = (p.KT + p.kt_per_split - 1) / p.kt_per_split;
    p.direct = p.splits == 1 && (epilogue == kEpiStore || swiglu_fused(m, epilogue));
    p.ws_floats = p.direct ? 0 : (size_t)p.splits * m * n;
    return p;
}

template <int WM, int WN, int WAVES_M, int WAVES_N, int STAGES, int HL, int SWIGLU = 0>
static void gemm_launch(const GemmPlan& p, hipStream_t stream, const uint16_t* a, int m, int k, const uint16_t* w,
                        float* c, int n, size_t split_stride, uint16_t* h = nullptr, int h_lo = 0) {
    const int groups = p.col_blocks * p.splits;
    const unsigned blocks = 8u * (unsigned)p.row_blocks * (unsigned)((groups + 7) / 8);
    hipLaunchKernelGGL((gemm_kernel<WM, WN, WAVES_M, WAVES_N, HL, STAGES, SWIGLU>), dim3(blocks),
                       dim3(WAVES_M * WAVES_N * 64), 0, stream, a, m, k, (const bf16x8*)w, p.KT, p.NT, c, n,
                       p.kt_per_split, p.splits, p.row_blocks, p.col_blocks, split_stride, h, h_lo);
}

zr_status launch_gemm(zr_context* ctx, const uint16_t* a, const uint16_t* w_packed, float* c_f32,
                      uint16_t* c_bf16, int m, int n, int k, int epilogue, Slabs* deferred) {
    if (deferred && (epilogue != kEpiStore || !c_f32 || c_bf16))
        return set_err(ctx, ZR_E_INVARIANT, "deferred split-K needs an f32 store epilogue");
    if (m <= 0) return ZR_OK;
    if (k % 32 != 0) return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM K=%d must be a multiple of 32", k);
    // the kernel addresses its operands with 32-bit buffer offsets
    const size_t a_bytes = 2 * 2 * a_plane(m, k), w_bytes = 2 * packed_weight_elems(k, n);
    if (a_bytes > 0x7fffffffull || w_bytes > 0x7fffffffull)
        return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM operands of %zu / %zu bytes exceed 2 GiB", a_bytes, w_bytes);
    const bool split_act = (ctx->desc.flags & ZR_FLAG_SPLIT_ACTIVATIONS) != 0;
    if (swiglu_ksplit(m, n, k, epilogue) && (!c_bf16 || c_f32 || deferred))
        return set_err(ctx, ZR_E_INVARIANT, "K-split SwiGLU (M=%d) writes the bf16 operand only", m);
    if (swiglu_ksplit(m, n, k, epilogue)) {
        const GemmPlan p = gemm_plan(m, n, k, epilogue);
        hipEvent_t ev;
        timing_mark_begin(ctx, kClassGemm, &ev);
#define ZR_KSPLIT(HLV, MTV)                                                                                     \
    hipLaunchKernelGGL((gemm_swiglu_ksplit_kernel<3, HLV, MTV>), dim3(p.col_blocks), dim3(256), 0, ctx->stream, a, \
                       m, k, (const bf16x8*)w_packed, p.KT, n, c_bf16, HLV - 1)
        if (split_act) {
            if (m > 32)
                ZR_KSPLIT(2, 2);
            else
                ZR_KSPLIT(2, 1);
        } else {
            if (m > 32)
                ZR_KSPLIT(1, 2);
            else
                ZR_KSPLIT(1, 1);
        }
#undef ZR_KSPLIT
        ZR_LAUNCH_CHECK(ctx);
        timing_mark_end(ctx, kClassGemm, ev);
        return ZR_OK;
    }
    const GemmPlan p = gemm_plan(m, n, k, epilogue);
    const GemmCfg cfg = pick_cfg(m, n, k, epilogue);
    if (swiglu_fused(m, epilogue) && (!c_bf16 || c_f32 || n % 64 != 0))
        return set_err(ctx, ZR_E_INVARIANT, "fused SwiGLU writes the bf16 operand only (N=%d)", n);
    const bool fused = swiglu_fused(m, epilogue);
    const bool direct = (p.direct && c_f32 && !c_bf16 && epilogue == kEpiStore) || fused;
    const size_t split_stride = (size_t)m * n;
    if (!direct && (size_t)p.splits * split_stride > ctx->splitk_ws_floats)
        return set_err(ctx, ZR_E_OOM, "split-K workspace too small (%d x %d x %d)", p.splits, m, n);
    float* dst = direct ? c_f32 : ctx->splitk_ws;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassGemm, &ev);
    bool launched = false;
#define ZR_GEMM_FUSED_CASE(WMV, WNV, WAM, WAN, ST)                                                     \
    if (fused && !launched && cfg.wm == WMV && cfg.wn == WNV && cfg.waves_m == WAM &&                  \
        cfg.waves_n == WAN && cfg.stages == ST) {                                                      \
        if (split_act)                                                                                 \
            gemm_launch<WMV, WNV, WAM, WAN, ST, 2, 1>(p, ctx->stream, a, m, k, w_packed, nullptr, n, 0, c_bf16, 1); \
        else                                                                                           \
            gemm_launch<WMV, WNV, WAM, WAN, ST, 1, 1>(p, ctx->stream, a, m, k, w_packed, nullptr, n, 0, c_bf16, 0); \
        launched = true;                                                                               \
    }
    ZR_GEMM_FUSED_CASE(2, 4, 2, 4, 3)
    ZR_GEMM_FUSED_CASE(2, 2, 2, 4, 3)
    ZR_GEMM_FUSED_CASE(2, 2, 1, 4, 3)
    ZR_GEMM_FUSED_CASE(1, 2, 4, 4, 3)
#undef ZR_GEMM_FUSED_CASE
#define ZR_GEMM_CASE(WMV, WNV, WAM, WAN, ST)                                                           \
    if (!fused && !launched && cfg.wm == WMV && cfg.wn == WNV && cfg.waves_m == WAM &&                 \
        cfg.waves_n == WAN && cfg.stages == ST) {                                                      \
        if (split_act)                                                                                 \
            gemm_launch<WMV, WNV, WAM, WAN, ST, 2>(p, ctx->stream, a, m, k, w_packed, dst, n, split_stride); \
        else                                                                                           \
            gemm_launch<WMV, WNV, WAM, WAN, ST, 1>(p, ctx->stream, a, m, k, w_packed, dst, n, split_stride); \
        launched = true;                                                                               \
    }
    ZR_GEMM_CASE(1, 1, 1, 4, 4)
    ZR_GEMM_CASE(2, 1, 1, 4, 3)
    ZR_GEMM_CASE(2, 1, 1, 4, 4)
    ZR_GEMM_CASE(2, 2, 4, 4, 3)
    ZR_GEMM_CASE(2, 4, 4, 2, 3)
    ZR_GEMM_CASE(2, 4, 2, 4, 3)
    ZR_GEMM_CASE(2, 2, 2, 4, 3)
#undef ZR_GEMM_CASE
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
