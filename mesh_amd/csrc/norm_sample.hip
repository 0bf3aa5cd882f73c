// Embedding gather, RMSNorm with a fused residual add, and greedy argmax.
#include <mutex>

#include "zr_internal.h"

namespace zr {

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Row gather of the bf16 embedding table into the f32 residual stream
// (forward_pass.rs:2230-2237; embed_tokens tensor_ops.rs:482-500).  Host ids
// are validated before staging.  Ids fed from device memory are checked here:
// the first out-of-vocabulary one (lowest row) is recorded in *err as
// (row << 32 | id) for the host to report, and its row gathers row 0 so that
// nothing is read out of bounds.
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t* __restrict__ tokens,
                                                    const uint16_t* __restrict__ table, int H, int V,
                                                    float* __restrict__ hidden, unsigned long long* err) {
    const int t = blockIdx.x;
    uint32_t id = tokens[t];
    if (id >= (uint32_t)V) {
        if (err && threadIdx.x == 0) atomicMin(err, ((unsigned long long)t << 32) | id);
        id = 0;
    }
    const uint16_t* src = table + (size_t)id * H;
    float* dst = hidden + (size_t)t * H;
    for (int i = threadIdx.x; i < H; i += blockDim.x) dst[i] = bf16_bits_to_f32(src[i]);
}

zr_status launch_embed(zr_context* ctx, StagedMeta* st, const uint32_t* d_tokens, bool check_ids) {
    if (st->total_q == 0) return ZR_OK;
    hipLaunchKernelGGL(embed_kernel, dim3(st->total_q), dim3(256), 0, ctx->stream, d_tokens,
                       ctx->embedding, ctx->desc.hidden, ctx->desc.vocab, ctx->hidden,
                       check_ids ? ctx->d_token_err : nullptr);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

// y = rms_norm(x (+ residual)) * gamma (tensor_ops.rs:285-304,
// runtime.rs:919-925).  With a residual, x_out = x + residual is written
// first (the broadcast_add of forward_pass.rs:2279 / 2304); the residual may
// arrive as res_n split-K slabs res_stride floats apart, summed in slab order
// (the same sum the split-K reduce forms).  row_index selects source rows
// (the last token of every sequence for the LM head).
__device__ inline float sum_slabs(const float* p, size_t i, int n, size_t stride) {
    float v = p[i];
    for (int s = 1; s < n; ++s) v += p[s * stride + i];
    return v;
}

__global__ __launch_bounds__(256) void rms_norm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ residual_in, int res_n,
                                                       size_t res_stride, float* __restrict__ x_out,
                                                       const float* __restrict__ gamma,
                                                       float* __restrict__ y_f32,
                                                       uint16_t* __restrict__ y_bf16, int split_lo,
                                                       size_t lo_offset,
                                                       const int* __restrict__ row_index, int cols,
                                                       float eps) {
    __shared__ float red[4];
    const int r = blockIdx.x;
    const int src = row_index ? row_index[r] : r;
    const float* xr = x + (size_t)src * cols;
    float* xo = x_out ? x_out + (size_t)src * cols : nullptr;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        float v = xr[i];
        if (residual_in) {
            v = v + sum_slabs(residual_in, (size_t)src * cols + i, res_n, res_stride);
            xo[i] = v;
        }
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = red[0] + red[1] + red[2] + red[3];
    const float inv_rms = 1.0f / sqrtf(total / (float)cols + eps);
    const float* xs = residual_in ? xo : xr;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        const float v = xs[i] * inv_rms * gamma[i];
        if (y_bf16) {
            uint16_t hi, lo;
            split_bf16(v, hi, lo);
            const size_t o = a_pack_index(r, i, cols);
            y_bf16[o] = hi;
            if (split_lo) y_bf16[lo_offset + o] = lo;
        } else {
            y_f32[(size_t)r * cols + i] = v;
        }
    }
}

// Same contract for cols % 4 == 0 and cols <= 4 NT NV: every thread of the
// NT-thread block keeps its NV float4 of the row in registers, so the row is
// read once.
template <int NV, int NT>
__global__ __launch_bounds__(NT) void rms_norm_vec_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ residual_in, int res_n,
                                                           size_t res_stride, float* __restrict__ x_out,
                                                           const float* __restrict__ gamma,
                                                           float* __restrict__ y_f32,
                                                           uint16_t* __restrict__ y_bf16, int split_lo,
                                                           size_t lo_offset,
                                                           const int* __restrict__ row_index, int cols,
                                                           float eps) {
    __shared__ float red[NT / 64];
    const int r = blockIdx.x;
    const int src = row_index ? row_index[r] : r;
    const int n4 = cols >> 2;
    const size_t base = (size_t)src * cols;
    float4 v[NV];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i4 = threadIdx.x + j * NT;
        if (i4 < n4) {
            float4 a = *(const float4*)(x + base + 4 * (size_t)i4);
            if (residual_in) {
                // slabs summed in slab order, their loads issued 16 at a time
                // (one round trip for the split-K products of a decode step)
                const float* rp = residual_in + base + 4 * (size_t)i4;
                float4 rr = *(const float4*)rp;
                for (int s0 = 1; s0 < res_n; s0 += 16) {
                    float4 q[16];
#pragma unroll
                    for (int u = 0; u < 16; ++u)
                        q[u] = s0 + u < res_n ? *(const float4*)(rp + (size_t)(s0 + u) * res_stride)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int u = 0; u < 16; ++u)
                        if (s0 + u < res_n) {
                            rr.x += q[u].x;
                            rr.y += q[u].y;
                            rr.z += q[u].z;
                            rr.w += q[u].w;
                        }
                }
                a.x = a.x + rr.x;
                a.y = a.y + rr.y;
                a.z = a.z + rr.z;
                a.w = a.w + rr.w;
                *(float4*)(x_out + base + 4 * (size_t)i4) = a;
            }
            v[j] = a;
            ss += a.x * a.x;
            ss += a.y * a.y;
            ss += a.z * a.z;
            ss += a.w * a.w;
        }
    }
    // gamma is fetched while the row sum is reduced
    float4 gv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i4 = threadIdx.x + j * NT;
        gv[j] = i4 < n4 ? *(const float4*)(gamma + 4 * (size_t)i4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) total += red[w];
    const float inv_rms = 1.0f / sqrtf(total / (float)cols + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i4 = threadIdx.x + j * NT;
        if (i4 >= n4) continue;
        const float4 g = gv[j];
        float y[4] = {v[j].x * inv_rms * g.x, v[j].y * inv_rms * g.y, v[j].z * inv_rms * g.z,
                      v[j].w * inv_rms * g.w};
        if (y_bf16) {
            ushort4 hi, lo;
            split_bf16(y[0], hi.x, lo.x);
            split_bf16(y[1], hi.y, lo.y);
            split_bf16(y[2], hi.z, lo.z);
            split_bf16(y[3], hi.w, lo.w);
            const size_t o = a_pack_index(r, 4 * i4, cols);  // 4 consecutive columns stay adjacent
            *(ushort4*)(y_bf16 + o) = hi;
            if (split_lo) *(ushort4*)(y_bf16 + lo_offset + o) = lo;
        } else {
            *(float4*)(y_f32 + (size_t)r * cols + 4 * (size_t)i4) = make_float4(y[0], y[1], y[2], y[3]);
        }
    }
}

zr_status launch_rms_norm(zr_context* ctx, const float* x, const Slabs& residual, float* x_out,
                          const float* gamma, float* y_f32, uint16_t* y_bf16, int split_lo,
                          const int* row_index, int rows, int cols) {
    if (rows <= 0) return ZR_OK;
    hipEvent_t ev;
    timing_mark_begin(ctx, kClassNormRopeKv, &ev);
    if (y_bf16 && cols % 32 != 0)
        return set_err(ctx, ZR_E_UNSUPPORTED, "GEMM operand width %d is not a multiple of 32", cols);
    const size_t lo_off = a_plane(rows, cols);
    // 1024-thread blocks (one float4 or two per thread): every row's loads,
    // split-K slabs included, spread over 16 waves
    const bool vec = cols % 4 == 0;
    const int nv1024 = (cols + 4095) / 4096, nv256 = (cols + 1023) / 1024;
#define ZR_RMS_ARGS                                                                                     \
    x, residual.ptr, residual.n, residual.stride, x_out, gamma, y_f32, y_bf16, split_lo, lo_off, row_index, \
        cols, ctx->desc.rms_norm_eps
    if (vec && nv1024 == 1)
        hipLaunchKernelGGL((rms_norm_vec_kernel<1, 1024>), dim3(rows), dim3(1024), 0, ctx->stream, ZR_RMS_ARGS);
    else if (vec && nv1024 == 2)
        hipLaunchKernelGGL((rms_norm_vec_kernel<2, 1024>), dim3(rows), dim3(1024), 0, ctx->stream, ZR_RMS_ARGS);
    else if (vec && nv256 == 1)
        hipLaunchKernelGGL((rms_norm_vec_kernel<1, 256>), dim3(rows), dim3(256), 0, ctx->stream, ZR_RMS_ARGS);
    else if (vec && nv256 == 2)
        hipLaunchKernelGGL((rms_norm_vec_kernel<2, 256>), dim3(rows), dim3(256), 0, ctx->stream, ZR_RMS_ARGS);
    else if (vec && nv256 <= 4)
        hipLaunchKernelGGL((rms_norm_vec_kernel<4, 256>), dim3(rows), dim3(256), 0, ctx->stream, ZR_RMS_ARGS);
    else if (vec && nv256 <= 8)
        hipLaunchKernelGGL((rms_norm_vec_kernel<8, 256>), dim3(rows), dim3(256), 0, ctx->stream, ZR_RMS_ARGS);
    else
        hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(256), 0, ctx->stream, ZR_RMS_ARGS);
#undef ZR_RMS_ARGS
    ZR_LAUNCH_CHECK(ctx);
    timing_mark_end(ctx, kClassNormRopeKv, ev);
    return ZR_OK;
}

// Greedy argmax, two stages; ties keep the lowest index
// (sample_greedy tensor_ops.rs:461-473; device argmax runtime.rs:561-570).
__device__ inline void better(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

constexpr int kArgmaxChunk = 4096;

// vec: cols % 4 == 0 and x 16-byte aligned; a thread then issues its four
// float4 loads of the chunk (4096 columns = 256 threads x 4 x 4) at once.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ x, int cols,
                                                             int chunks, int vec, float* __restrict__ ws) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int r = blockIdx.y, ch = blockIdx.x;
    const int c0 = ch * kArgmaxChunk, c1 = min(cols, c0 + kArgmaxChunk);
    const float* xr = x + (size_t)r * cols;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (vec) {
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        const int j0 = c0 >> 2, j1 = c1 >> 2;
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + (int)threadIdx.x + u * 256;
            v[u] = j < j1 ? x4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = j0 + (int)threadIdx.x + u * 256;
            if (j < j1) {
                better(bv, bi, v[u].x, 4 * j);
                better(bv, bi, v[u].y, 4 * j + 1);
                better(bv, bi, v[u].z, 4 * j + 2);
                better(bv, bi, v[u].w, 4 * j + 3);
            }
        }
    } else {
        for (int i = c0 + threadIdx.x; i < c1; i += blockDim.x) better(bv, bi, xr[i], i);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        better(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        bv = sv[0];
        bi = si[0];
        for (int w = 1; w < 4; ++w) better(bv, bi, sv[w], si[w]);
        ws[((size_t)r * chunks + ch) * 2] = bv;
        ws[((size_t)r * chunks + ch) * 2 + 1] = __int_as_float(bi);
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ ws, int chunks,
                                                          uint32_t* __restrict__ out) {
    const int r = blockIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int ch = threadIdx.x; ch < chunks; ch += 64)
        better(bv, bi, ws[((size_t)r * chunks + ch) * 2], __float_as_int(ws[((size_t)r * chunks + ch) * 2 + 1]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        better(bv, bi, ov, oi);
    }
    // a row of all -inf/NaN keeps index 0, as the reference's initial max_idx
    if (threadIdx.x == 0) out[r] = bi == 0x7fffffff ? 0u : (uint32_t)bi;
}

// Both argmax kernels over `ws` (rows x chunks (value, index) pairs).
static zr_status argmax_into(zr_context* ctx, const float* x, int rows, int cols, uint32_t* out, float* ws,
                             size_t ws_floats) {
    if (rows <= 0) return ZR_OK;
    const int chunks = (cols + kArgmaxChunk - 1) / kArgmaxChunk;
    if ((size_t)rows * chunks * 2 > ws_floats) return set_err(ctx, ZR_E_OOM, "argmax workspace too small");
    static_assert(kArgmaxChunk == 256 * 4 * 4, "one float4 group per thread");
    const int vec = (cols % 4 == 0) && ((uintptr_t)x % 16 == 0);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(chunks, rows), dim3(256), 0, ctx->stream, x, cols, chunks, vec,
                       ws);
    ZR_LAUNCH_CHECK(ctx);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(rows), dim3(64), 0, ctx->stream, ws, chunks, out);
    ZR_LAUNCH_CHECK(ctx);
    return ZR_OK;
}

zr_status launch_argmax(zr_context* ctx, const float* x, int rows, int cols, uint32_t* out) {
    return argmax_into(ctx, x, rows, cols, out, ctx->argmax_ws, ctx->argmax_ws_floats);
}

// ----------------------------------------------- argmax without allocation
// The partials of zr_argmax_noalloc live in this fixed array of the library
// (each device holds its own copy for the life of the process).  Host code
// never passes `scratch` itself to a kernel: its device address is resolved
// once per device with hipGetSymbolAddress (noalloc_scratch_init, called by
// zr_context_create with the device current) and kept in g_scratch_dev.
static __device__ __align__(256) float scratch[2 * kNoAllocArgmaxPairs];

static std::mutex g_scratch_mu;
static float* g_scratch_dev[kMaxDevices];

zr_status noalloc_scratch_init(zr_context* ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return set_err(ctx, ZR_E_UNSUPPORTED, "device %d beyond the %d devices the library tracks", ctx->device,
                       kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[ctx->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_err(ctx, ZR_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", ctx->device,
                           hipGetErrorString(e));
        g_scratch_dev[ctx->device] = (float*)p;
    }
    ctx->noalloc_scratch = g_scratch_dev[ctx->device];
    return ZR_OK;
}

zr_status launch_argmax_noalloc(zr_context* ctx, const float* x, int rows, int cols, uint32_t* out) {
    if (!ctx->noalloc_scratch) return set_err(ctx, ZR_E_INVARIANT, "argmax scratch not resolved for this device");
    const size_t pairs = (size_t)rows * (size_t)((cols + kArgmaxChunk - 1) / kArgmaxChunk);
    if (pairs > (size_t)kNoAllocArgmaxPairs)
        return set_err(ctx, ZR_E_INVALID,
                       "zr_argmax_noalloc: %d rows x %d columns need %zu partials; the fixed scratch holds %d "
                       "(rows x ceil(cols / %d) <= %d)",
                       rows, cols, pairs, kNoAllocArgmaxPairs, kArgmaxChunk, kNoAllocArgmaxPairs);
    return argmax_into(ctx, x, rows, cols, out, ctx->noalloc_scratch, 2 * (size_t)kNoAllocArgmaxPairs);
}

}  // namespace zr
