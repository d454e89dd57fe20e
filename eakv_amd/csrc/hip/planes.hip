// planes.hip — whole-plane kernels on a cache's (layer, kv) blocks:
// dequantization to f32 and the integrity check.  Both stream the planes
// once and are bound by HBM bandwidth.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../eakvd.h"

namespace {

// Dequantize groups [g0, g0 + n) of one block into out (64 f32 per group,
// in group order): value = fma(nibble, scale, bias), byte k of a group
// holding dim k in its low nibble and dim k + 32 in its high nibble, as
// reference kernels/dequantize_avx512.ea:10-89.  Eight lanes per group:
// lane i takes bytes 4i..4i+3 (one dword) and writes dims 4i..4i+3 (low
// nibbles) and 32+4i..32+4i+3 (high nibbles): a group's 32 bytes are read
// and its 256 output bytes written by consecutive lanes.
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t *__restrict__ w,
                                                         const float *__restrict__ sc,
                                                         const float *__restrict__ bi,
                                                         int64_t g0, int64_t n,
                                                         float *__restrict__ out)
{
    const int64_t n8 = n * 8;
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < n8; t += step) {
        const int64_t gi = t >> 3;
        const int i = (int)(t & 7);
        const int64_t g = g0 + gi;
        const uint32_t x = *(const uint32_t *)(w + g * 32 + 4 * i);
        const float s = sc[g], b = bi[g];
        float4 lo, hi;
        lo.x = fmaf((float)(x & 15u), s, b);
        lo.y = fmaf((float)((x >> 8) & 15u), s, b);
        lo.z = fmaf((float)((x >> 16) & 15u), s, b);
        lo.w = fmaf((float)((x >> 24) & 15u), s, b);
        hi.x = fmaf((float)((x >> 4) & 15u), s, b);
        hi.y = fmaf((float)((x >> 12) & 15u), s, b);
        hi.z = fmaf((float)((x >> 20) & 15u), s, b);
        hi.w = fmaf((float)(x >> 28), s, b);
        float4 *o = (float4 *)(out + gi * 64);
        o[i] = lo;
        o[8 + i] = hi;
    }
}

// The integrity check of reference kernels/validate.ea:14-71 on the first n
// groups of every block, one block per grid row y: the code of a group is
// 1 if its scale is NaN, else 2 if its bias is NaN, else 3 if its scale is
// negative, else 0; NaN is read from the bits as the reference does
// (positive: bits > 0x7f800000; negative: bits in 0xff800001..0xffffffff).
// The reference returns the code of the first failing group; here each
// failing group offers the key g*4 + code and the block's minimum wins
// (atomic min of the key into res[y], which starts at all ones).
__device__ __forceinline__ bool nan_bits(int32_t v)
{
    return v > 2139095040 || (v < 0 && v > -8388608);
}

__global__ __launch_bounds__(256) void validate_kernel(const uint8_t *__restrict__ base,
                                                       int64_t block_bytes, int64_t s_off,
                                                       int64_t b_off, int64_t n,
                                                       unsigned long long *__restrict__ res)
{
    const uint8_t *blk = base + (int64_t)blockIdx.y * block_bytes;
    const int32_t *sb = (const int32_t *)(blk + s_off);
    const int32_t *bb = (const int32_t *)(blk + b_off);
    unsigned long long key = ~0ull;
    auto check = [&](int64_t g, int32_t s, int32_t b) {
        const int code = nan_bits(s) ? 1 : nan_bits(b) ? 2 : __int_as_float(s) < 0.0f ? 3 : 0;
        if (code) {
            const unsigned long long k = (unsigned long long)g * 4 + (unsigned long long)code;
            key = k < key ? k : key;
        }
    };
    // four groups per lane and iteration, as 16-byte loads (the planes are
    // 256-byte aligned); the last n % 4 groups one at a time
    const int64_t n4 = n / 4;
    const int64_t step = (int64_t)gridDim.x * 256;
    for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < n4; j += step) {
        const int4 s = reinterpret_cast<const int4 *>(sb)[j];
        const int4 b = reinterpret_cast<const int4 *>(bb)[j];
        check(4 * j, s.x, b.x);
        check(4 * j + 1, s.y, b.y);
        check(4 * j + 2, s.z, b.z);
        check(4 * j + 3, s.w, b.w);
    }
    if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
        const int64_t g = 4 * n4 + threadIdx.x;
        check(g, sb[g], bb[g]);
    }
    // the block's minimum: across the wave, then the waves
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(key, off, 64);
        key = o < key ? o : key;
    }
    __shared__ unsigned long long wmin[4];
    if ((threadIdx.x & 63) == 0) wmin[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = wmin[0];
        for (int i = 1; i < 4; i++) m = wmin[i] < m ? wmin[i] : m;
        if (m != ~0ull) atomicMin(res + blockIdx.y, m);
    }
}

}  // namespace

extern "C" int eakvd_dequantize(const eakvd_geom *g, const uint8_t *base, int layer, int kv,
                                int64_t g0, int64_t n, float *out, void *stream)
{
    if (n <= 0) return 0;
    const uint8_t *blk = base + ((int64_t)layer * 2 + kv) * g->block_bytes;
    // one pass where the grid allows (a 32K plane of 8 kv heads: 16,416
    // blocks, 25.2-25.3 against 30.7-30.8 us with the grid held to 4096
    // blocks and four groups per lane)
    const int64_t nb = (n * 8 + 255) / 256;
    const unsigned gx = (unsigned)(nb < 65535 ? nb : 65535);
    hipLaunchKernelGGL(dequantize_kernel, dim3(gx), dim3(256), 0,
                       (hipStream_t)stream, blk, (const float *)(blk + g->s_off),
                       (const float *)(blk + g->b_off), g0, n, out);
    return (int)hipGetLastError();
}

extern "C" int eakvd_validate(const eakvd_geom *g, const uint8_t *base, int n_blocks,
                              int64_t n, unsigned long long *res, void *stream)
{
    hipError_t e = hipMemsetAsync(res, 0xff, (size_t)n_blocks * sizeof(*res),
                                  (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
    if (n <= 0 || n_blocks <= 0) return 0;
    // one pass over a block's groups (up to 1024 x 256 lanes of four groups;
    // the 64 blocks of a 32K cache: 39.0-39.6 against 40.4-40.8 us with 64
    // blocks per row walking eight steps)
    const int64_t nbx = ((n + 3) / 4 + 255) / 256;
    const int gx = (int)(nbx < 1 ? 1 : nbx > 1024 ? 1024 : nbx);
    hipLaunchKernelGGL(validate_kernel, dim3(gx, n_blocks), dim3(256), 0, (hipStream_t)stream,
                       base, g->block_bytes, g->s_off, g->b_off, n, res);
    return (int)hipGetLastError();
}
