// quantize.hip — Q4_1 group-64 split-packed quantization on gfx950.
//
// Bit-exact restatement of reference kernels/quantize_simd.ea:9-59 (the
// quantizer driven by src/cache.c:60-151):
//   min/max: strict </> scan from element 0 (first occurrence wins; NaN
//            elements after element 0 are skipped; a NaN element 0 makes
//            min = max = NaN)
//   scale  = range > 0 ? range/15 : 1,  inv = range > 0 ? 15/range : 0
//   bias   = min
//   q(x)   = clamp(to_i32((x - min)*inv + 0.5), 0, 15), two roundings,
//            to_i32 with x86 cvttss2si semantics (NaN / out of range ->
//            INT32_MIN, then clamped to 0)
//   byte k = q(x[k+32])*16 + q(x[k])
//
// Work split: 8 lanes per group; lane j holds elements 4j..4j+3 (its four
// low nibbles) and 32+4j..32+4j+3 (their high nibbles), so it packs its own
// four bytes.  A wave covers 8 groups (2 KB of f32) with two 16-byte loads
// per lane; each lane loads its next group before it quantizes the current
// one.  The group min and max combine across the 8 lanes by DPP moves.
#include "common.h"

namespace {

constexpr int64_t kQuantBlocks = 8192;
constexpr int64_t kOnePass = 32768;

// One group: the reference's min/max, scale, bias and nibbles; lane j's
// four packed bytes, and (lane 0) the scale and bias.
struct QOut {
    uint32_t word;
    float scale, bias;
};

__device__ __forceinline__ QOut quantize_group8(const float4 &lo, const float4 &hi, int gbase)
{
    float mn, mx;
    group_minmax8(lo, hi, gbase, mn, mx);
    const float range = __fsub_rn(mx, mn);
    QOut o;
    o.scale = 1.0f;
    o.bias = mn;
    float inv = 0.0f;
    if (range > 0.0f) {
        o.scale = range / 15.0f;
        inv = 15.0f / range;
    }
    const uint32_t b0 = q4(lo.x, mn, inv) | (q4(hi.x, mn, inv) << 4);
    const uint32_t b1 = q4(lo.y, mn, inv) | (q4(hi.y, mn, inv) << 4);
    const uint32_t b2 = q4(lo.z, mn, inv) | (q4(hi.z, mn, inv) << 4);
    const uint32_t b3 = q4(lo.w, mn, inv) | (q4(hi.w, mn, inv) << 4);
    o.word = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    return o;
}

template <bool VEC>
__device__ __forceinline__ void load_group8(const float *gp, int l8, float4 &lo, float4 &hi)
{
    const float *a = gp + l8 * 4, *b = gp + 32 + l8 * 4;
    if (VEC) {
        lo = *reinterpret_cast<const float4 *>(a);
        hi = *reinterpret_cast<const float4 *>(b);
    } else {
        lo = make_float4(a[0], a[1], a[2], a[3]);
        hi = make_float4(b[0], b[1], b[2], b[3]);
    }
}

template <int NT, bool VEC>
__global__ __launch_bounds__(NT) void quantize8_kernel(eakvd_geom g, eakvd_quant_job job)
{
    const int l8 = threadIdx.x & 7;
    const int slot = threadIdx.x >> 3;
    const int gbase = (threadIdx.x & 63) & ~7;
    const int64_t slots = NT / 8;
    const int64_t per_cache = (int64_t)job.n_planes * job.nh;
    const int64_t gstep = (int64_t)gridDim.x * slots;

    for (int64_t row = blockIdx.y; row < job.n_rows; row += gridDim.y) {
        const int c = (int)(row / per_cache);
        const int64_t rem = row % per_cache;
        const int plane = job.plane0 + (int)(rem / job.nh);
        const int64_t h = rem % job.nh;
        uint8_t *blk = job.base[c] + (int64_t)plane * g.block_bytes;
        float *sp = (float *)(blk + g.s_off);
        float *bp = (float *)(blk + g.b_off);
        const int64_t gdst0 = h * g.gph + job.g_off[c];
        const float *srow = job.src + row * job.row_stride;

        // the 8 lanes of a group share its trip count, so the DPP moves and
        // shuffles above only ever read lanes of the same group
        int64_t gi = (int64_t)blockIdx.x * slots + slot;
        float4 lo, hi;
        if (gi < job.n_g) load_group8<VEC>(srow + gi * 64, l8, lo, hi);
        while (gi < job.n_g) {
            const int64_t gn = gi + gstep;
            float4 nlo = lo, nhi = hi;
            if (gn < job.n_g) load_group8<VEC>(srow + gn * 64, l8, nlo, nhi);
            const QOut o = quantize_group8(lo, hi, gbase);
            const int64_t gd = gdst0 + gi;
            *reinterpret_cast<uint32_t *>(blk + gd * 32 + l8 * 4) = o.word;
            if (l8 == 0) {
                sp[gd] = o.scale;
                bp[gd] = o.bias;
            }
            gi = gn;
            lo = nlo;
            hi = nhi;
        }
    }
}

}  // namespace

extern "C" int eakvd_quantize(const eakvd_geom *g, const eakvd_quant_job *job,
                              void *stream)
{
    if (job->n_rows <= 0 || job->n_g <= 0) return 0;
    const hipStream_t st = (hipStream_t)stream;
    const int64_t gy = job->n_rows < 65535 ? job->n_rows : 65535;
    // float4 loads need 16-byte aligned rows
    const bool vec = ((uintptr_t)job->src % 16 == 0) && (job->row_stride % 4 == 0);
    if (job->n_g <= 8) {
        // a token or two per row (appends): one block of 64 lanes per row
        const dim3 grid(1, (unsigned)gy);
        if (vec)
            hipLaunchKernelGGL((quantize8_kernel<64, true>), grid, dim3(64), 0, st, *g, *job);
        else
            hipLaunchKernelGGL((quantize8_kernel<64, false>), grid, dim3(64), 0, st, *g, *job);
    } else {
        // blocks of 32 groups: one pass over the rows where that takes at
        // least kOnePass blocks (long rows), else about kQuantBlocks blocks
        // (a few passes each)
        const int64_t need = (job->n_g + 31) / 32;
        const int64_t target = need * gy >= kOnePass ? need * gy : kQuantBlocks;
        int64_t gx = (target + gy - 1) / gy;
        if (gx > need) gx = need;
        if (gx < 1) gx = 1;
        const dim3 grid((unsigned)gx, (unsigned)gy);
        if (vec)
            hipLaunchKernelGGL((quantize8_kernel<256, true>), grid, dim3(256), 0, st, *g, *job);
        else
            hipLaunchKernelGGL((quantize8_kernel<256, false>), grid, dim3(256), 0, st, *g, *job);
    }
    return (int)hipGetLastError();
}
