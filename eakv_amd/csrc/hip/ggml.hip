// ggml.hip — the ggml block type of reference include/eakv_ggml.h:27-31
// (block_q4_1_eakv: 32 split-packed nibble bytes, f32 d, f32 m; 64 values
// in 40 bytes) on gfx950: quantize a row, dequantize a row, dot rows with
// f32 vectors (reference src/ggml_type.c:21-242).  Where the reference's
// AVX-512 and scalar paths differ, these follow the AVX-512 path (fused
// d*n + m, 16 lane accumulators reduced by the 16-lane tree).
#include "common.h"

namespace {

// Row to blocks, 16 lanes per block (lane l: elements 4l..4l+3).  min/max
// as the strict scan of ggml_type.c:79-85; d = range/15 (0 for a constant
// block), id = range > 0 ? 15/range : 0, q = clamp(trunc(0.5 + (x - min)*id),
// 0, 15) (ggml_type.c:47-50, :79-87); byte k = q(x[k]) | q(x[k+32]) << 4.
template <bool VEC>
__global__ __launch_bounds__(256) void ggml_quantize_kernel(const float *__restrict__ src,
                                                            uint8_t *__restrict__ dst, int64_t nb)
{
    const int lane16 = threadIdx.x & 15;
    const int slot_shift = (threadIdx.x & 63) & ~15;
    for (int64_t b = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4); b < nb;
         b += (int64_t)gridDim.x * 16) {
        const float *xp = src + b * 64 + lane16 * 4;
        float4 x;
        if (VEC) {
            x = *reinterpret_cast<const float4 *>(xp);
        } else {
            x.x = xp[0]; x.y = xp[1]; x.z = xp[2]; x.w = xp[3];
        }
        float mn, mx;
        group_minmax(x, slot_shift, mn, mx);
        const float range = __fsub_rn(mx, mn);
        const float d = range / 15.0f;
        const float id = range > 0.0f ? 15.0f / range : 0.0f;
        const uint32_t mine = q4(x.x, mn, id) | (q4(x.y, mn, id) << 8) |
                              (q4(x.z, mn, id) << 16) | (q4(x.w, mn, id) << 24);
        const uint32_t hi = (uint32_t)__shfl_xor((int)mine, 8, 16);
        uint8_t *blk = dst + b * 40;
        if (lane16 < 8) *reinterpret_cast<uint32_t *>(blk + lane16 * 4) = mine | (hi << 4);
        if (lane16 == 0) {
            *reinterpret_cast<float *>(blk + 32) = d;
            *reinterpret_cast<float *>(blk + 36) = mn;
        }
    }
}

// Blocks to a row, 8 lanes per block: lane i takes qs bytes 4i..4i+3 and
// writes values 4i..4i+3 (low nibbles) and 32+4i.. (high nibbles), each
// fma(n, d, m) (ggml_type.c:105-125).
template <bool VEC>
__global__ __launch_bounds__(256) void ggml_dequantize_kernel(const uint8_t *__restrict__ src,
                                                              float *__restrict__ dst, int64_t nb)
{
    const int64_t n8 = nb * 8;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < n8;
         t += (int64_t)gridDim.x * 256) {
        const int64_t b = t >> 3;
        const int i = (int)(t & 7);
        const uint8_t *blk = src + b * 40;
        const uint32_t x = *reinterpret_cast<const uint32_t *>(blk + 4 * i);
        const float d = *reinterpret_cast<const float *>(blk + 32);
        const float m = *reinterpret_cast<const float *>(blk + 36);
        float4 lo, hi;
        lo.x = fmaf((float)(x & 15u), d, m);
        lo.y = fmaf((float)((x >> 8) & 15u), d, m);
        lo.z = fmaf((float)((x >> 16) & 15u), d, m);
        lo.w = fmaf((float)((x >> 24) & 15u), d, m);
        hi.x = fmaf((float)((x >> 4) & 15u), d, m);
        hi.y = fmaf((float)((x >> 12) & 15u), d, m);
        hi.z = fmaf((float)((x >> 20) & 15u), d, m);
        hi.w = fmaf((float)(x >> 28), d, m);
        float *o = dst + b * 64;
        if (VEC) {
            reinterpret_cast<float4 *>(o)[i] = lo;
            reinterpret_cast<float4 *>(o)[8 + i] = hi;
        } else {
            o[4 * i] = lo.x; o[4 * i + 1] = lo.y; o[4 * i + 2] = lo.z; o[4 * i + 3] = lo.w;
            o[32 + 4 * i] = hi.x; o[33 + 4 * i] = hi.y; o[34 + 4 * i] = hi.z;
            o[35 + 4 * i] = hi.w;
        }
    }
}

// Row r (< nrc) of blocks at vx + r*bx dotted with the f32 row at vy + r*by
// into s + r*bs (byte strides), 16 lanes per row: lane l keeps the
// accumulator of AVX-512 lane l of ggml_type.c:151-178, taking per block
// for c = 0, 1 value c*16 + l (low nibble of byte c*16 + l) then value
// c*16 + 32 + l (its high nibble), acc = fma(fma(n, d, m), y, acc); the 16
// accumulators are summed by the 16-lane tree.
__global__ __launch_bounds__(256) void ggml_vec_dot_kernel(int nb, float *s, size_t bs,
                                                           const uint8_t *vx, size_t bx,
                                                           const uint8_t *vy, size_t by, int nrc)
{
    const int l = threadIdx.x & 15;
    for (int64_t r = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4); r < nrc;
         r += (int64_t)gridDim.x * 16) {
        const uint8_t *x = vx + r * bx;
        const float *y = reinterpret_cast<const float *>(vy + r * by);
        float acc = 0.0f;
        for (int i = 0; i < nb; i++) {
            const uint8_t *blk = x + (int64_t)i * 40;
            const float d = *reinterpret_cast<const float *>(blk + 32);
            const float m = *reinterpret_cast<const float *>(blk + 36);
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t q = blk[c * 16 + l];
                acc = fmaf(fmaf((float)(q & 15u), d, m), y[i * 64 + c * 16 + l], acc);
                acc = fmaf(fmaf((float)(q >> 4), d, m), y[i * 64 + c * 16 + 32 + l], acc);
            }
        }
        float a[16];
#pragma unroll
        for (int j = 0; j < 16; j++) a[j] = __shfl(acc, j, 16);
        if (l == 0) *reinterpret_cast<float *>(reinterpret_cast<char *>(s) + r * bs) = reduce16(a);
    }
}

int grid_for(int64_t threads)
{
    int64_t b = (threads + 255) / 256;
    return (int)(b < 1 ? 1 : b > 8192 ? 8192 : b);
}

}  // namespace

extern "C" int eakvd_ggml_quantize_row(const float *src, void *dst, int64_t k, void *stream)
{
    const int64_t nb = k / 64;
    if (nb <= 0) return 0;
    const dim3 grid(grid_for(nb * 16));
    if ((uintptr_t)src % 16 == 0)
        hipLaunchKernelGGL(ggml_quantize_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream,
                           src, (uint8_t *)dst, nb);
    else
        hipLaunchKernelGGL(ggml_quantize_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream,
                           src, (uint8_t *)dst, nb);
    return (int)hipGetLastError();
}

extern "C" int eakvd_ggml_dequantize_row(const void *src, float *dst, int64_t k, void *stream)
{
    const int64_t nb = k / 64;
    if (nb <= 0) return 0;
    const dim3 grid(grid_for(nb * 8));
    if ((uintptr_t)dst % 16 == 0)
        hipLaunchKernelGGL(ggml_dequantize_kernel<true>, grid, dim3(256), 0,
                           (hipStream_t)stream, (const uint8_t *)src, dst, nb);
    else
        hipLaunchKernelGGL(ggml_dequantize_kernel<false>, grid, dim3(256), 0,
                           (hipStream_t)stream, (const uint8_t *)src, dst, nb);
    return (int)hipGetLastError();
}

extern "C" int eakvd_ggml_vec_dot(int n, float *s, size_t bs, const void *vx, size_t bx,
                                  const void *vy, size_t by, int nrc, void *stream)
{
    if (nrc <= 0) return 0;
    hipLaunchKernelGGL(ggml_vec_dot_kernel, dim3(grid_for((int64_t)nrc * 16)), dim3(256), 0,
                       (hipStream_t)stream, n / 64, s, bs, (const uint8_t *)vx, bx,
                       (const uint8_t *)vy, by, nrc);
    return (int)hipGetLastError();
}
