// ggml.hip — the ggml block type of reference include/eakv_ggml.h:27-31
// (block_q4_1_eakv: 32 split-packed nibble bytes, f32 d, f32 m; 64 values
// in 40 bytes) on gfx950: quantize a row, dequantize a row, dot rows with
// f32 vectors (reference src/ggml_type.c:21-242).  Where the reference's
// AVX-512 and scalar paths differ, these follow the AVX-512 path (fused
// d*n + m, 16 lane accumulators reduced by the 16-lane tree).
#include "common.h"

namespace {

// Row to blocks, 8 lanes per block (lane j: elements 4j..4j+3 and
// 32+4j..32+4j+3, so it packs its own four bytes).  min/max as the strict
// scan of ggml_type.c:79-85; d = range/15 (0 for a constant block),
// id = range > 0 ? 15/range : 0, q = clamp(trunc(0.5 + (x - min)*id), 0, 15)
// (ggml_type.c:47-50, :79-87); byte k = q(x[k]) | q(x[k+32]) << 4.  Each
// lane loads its next block before it quantizes the current one.  Loads and
// stores are non-temporal, each byte being touched once (65,536 rows of 4096:
// 199.6-200.3 against 221.4-222.9 us per call with the default policy).
template <bool VEC>
__device__ __forceinline__ void load_block8(const float *bp, int l8, float4 &lo, float4 &hi)
{
    const float *a = bp + l8 * 4, *c = bp + 32 + l8 * 4;
    if (VEC) {
        const v4f x = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(a));
        const v4f y = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(c));
        lo = make_float4(x[0], x[1], x[2], x[3]);
        hi = make_float4(y[0], y[1], y[2], y[3]);
    } else {
        lo = make_float4(a[0], a[1], a[2], a[3]);
        hi = make_float4(c[0], c[1], c[2], c[3]);
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void ggml_quantize_kernel(const float *__restrict__ src,
                                                            uint8_t *__restrict__ dst, int64_t nb)
{
    const int l8 = threadIdx.x & 7;
    const int gbase = (threadIdx.x & 63) & ~7;
    const int64_t step = (int64_t)gridDim.x * 32;
    // the 8 lanes of a block share its trip count
    int64_t b = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    float4 lo, hi;
    if (b < nb) load_block8<VEC>(src + b * 64, l8, lo, hi);
    while (b < nb) {
        const int64_t bn = b + step;
        float4 nlo = lo, nhi = hi;
        if (bn < nb) load_block8<VEC>(src + bn * 64, l8, nlo, nhi);
        float mn, mx;
        group_minmax8(lo, hi, gbase, mn, mx);
        const float range = __fsub_rn(mx, mn);
        const float d = range / 15.0f;
        const float id = range > 0.0f ? 15.0f / range : 0.0f;
        const float f = q4_factor(id);
        const uint32_t b0 = q4(lo.x, mn, f) | (q4(hi.x, mn, f) << 4);
        const uint32_t b1 = q4(lo.y, mn, f) | (q4(hi.y, mn, f) << 4);
        const uint32_t b2 = q4(lo.z, mn, f) | (q4(hi.z, mn, f) << 4);
        const uint32_t b3 = q4(lo.w, mn, f) | (q4(hi.w, mn, f) << 4);
        uint8_t *blk = dst + b * 40;
        __builtin_nontemporal_store(b0 | (b1 << 8) | (b2 << 16) | (b3 << 24),
                                    reinterpret_cast<uint32_t *>(blk + l8 * 4));
        if (l8 == 0) {
            __builtin_nontemporal_store(d, reinterpret_cast<float *>(blk + 32));
            __builtin_nontemporal_store(mn, reinterpret_cast<float *>(blk + 36));
        }
        b = bn;
        lo = nlo;
        hi = nhi;
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
            // non-temporal: 1 GiB of f32 out, 199.6-201.7 against
            // 264.9-269.7 us per call (65,536 rows of 4096) with the default
            // policy
            __builtin_nontemporal_store(v4f{lo.x, lo.y, lo.z, lo.w}, reinterpret_cast<v4f *>(o) + i);
            __builtin_nontemporal_store(v4f{hi.x, hi.y, hi.z, hi.w},
                                        reinterpret_cast<v4f *>(o) + 8 + i);
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
        // four blocks' loads in flight (65,536 rows of 4096: 215.9-217.2
        // against 229.6-229.8 us per call; eight: 222.4-222.9)
#pragma unroll 4
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

// One pass over the threads up to 65,535 blocks (the dequantizer at 65,536
// rows of 4096: 184.2-184.5 against 199.7-200.3 us per call with at most
// 8192 blocks and eight blocks' work per lane)
int grid_for(int64_t threads)
{
    int64_t b = (threads + 255) / 256;
    return (int)(b < 1 ? 1 : b > 65535 ? 65535 : b);
}

}  // namespace

extern "C" int eakvd_ggml_quantize_row(const float *src, void *dst, int64_t k, void *stream)
{
    const int64_t nb = k / 64;
    if (nb <= 0) return 0;
    // 32 blocks per workgroup, one pass up to 2^16 workgroups
    const int64_t wg = (nb + 31) / 32;
    const dim3 grid((unsigned)(wg < 65536 ? wg : 65536));
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
