// quantize.hip — Q4_1 group-64 split-packed quantization on gfx950.
//
// Bit-exact restatement of reference kernels/quantize_simd.ea:9-59 (the
// quantizer driven by src/cache.c:60-151):
//   min/max: strict </> scan from element 0 (first occurrence wins; NaN
//            elements after element 0 are skipped; a NaN element 0 makes
//            min = max = NaN)
//   scale  = range > 0 ? range/15 : 1,  inv = range > 0 ? 15/range : 0
//   bias   = min
//   q(x)   = clamp(to_i32((x - min)*inv + 0.5), 0, 15), each step rounded,
//            to_i32 with x86 cvttss2si semantics (NaN / out of range ->
//            INT32_MIN, then clamped to 0); one v_cvt_i32_f32 gives the same
//            nibble for every value a group can produce (q4, common.h)
//   byte k = q(x[k+32])*16 + q(x[k])
//
// Work split: 8 lanes per group; lane j holds elements 4j..4j+3 (its four
// low nibbles) and 32+4j..32+4j+3 (their high nibbles), so it packs its own
// four bytes.  A wave covers 8 groups (2 KB of f32) with two 16-byte loads
// per lane.  The group min and max combine across the 8 lanes by DPP moves.
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
    const float f = q4_factor(inv);
    const uint32_t b0 = q4(lo.x, mn, f) | (q4(hi.x, mn, f) << 4);
    const uint32_t b1 = q4(lo.y, mn, f) | (q4(hi.y, mn, f) << 4);
    const uint32_t b2 = q4(lo.z, mn, f) | (q4(hi.z, mn, f) << 4);
    const uint32_t b3 = q4(lo.w, mn, f) | (q4(hi.w, mn, f) << 4);
    o.word = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    return o;
}

// Every source and output byte is touched once: the 16-byte loads of aligned
// rows and the stores are non-temporal (64Q/8KV d128 128K rows, 537 MB of f32 per launch from
// HBM: 102.7-103.0 against 107.0-108.1 us per launch with the default
// policy and one group per lane; 32Q/8KV d128 32K rows: 29.4-29.5 against
// 31.1-31.5 us).
template <bool VEC>
__device__ __forceinline__ void load_group8(const float *gp, int l8, float4 &lo, float4 &hi)
{
    const float *a = gp + l8 * 4, *b = gp + 32 + l8 * 4;
    if (VEC) {
        const v4f x = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(a));
        const v4f y = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(b));
        lo = make_float4(x[0], x[1], x[2], x[3]);
        hi = make_float4(y[0], y[1], y[2], y[3]);
    } else {
        lo = make_float4(a[0], a[1], a[2], a[3]);
        hi = make_float4(b[0], b[1], b[2], b[3]);
    }
}

// One group per lane at most (gridDim.x * NT/8 >= n_g, the launch shape of
// long rows) or a loop in which each lane loads its next group before it
// quantizes the current one.
template <int NT, bool VEC>
__global__ __launch_bounds__(NT) void quantize8_kernel(eakvd_geom g, eakvd_quant_job job)
{
    const int l8 = threadIdx.x & 7;
    const int slot = threadIdx.x >> 3;
    const int gbase = (threadIdx.x & 63) & ~7;
    const int64_t slots = NT / 8;
    // rows, heads and planes per cache fit 32 bits (the host checks n_rows)
    const uint32_t per_cache = (uint32_t)job.n_planes * (uint32_t)job.nh;
    const uint32_t nh = (uint32_t)job.nh;
    const int64_t gstep = (int64_t)gridDim.x * slots;

    for (int64_t row = blockIdx.y; row < job.n_rows; row += gridDim.y) {
        const uint32_t r = (uint32_t)row;
        const uint32_t c = r / per_cache;
        const uint32_t rem = r - c * per_cache;
        const uint32_t pl = rem / nh;
        const uint32_t h = rem - pl * nh;
        uint8_t *blk = job.base[c] + (int64_t)(job.plane0 + (int)pl) * g.block_bytes;
        float *sp = (float *)(blk + g.s_off);
        float *bp = (float *)(blk + g.b_off);
        const int64_t gdst0 = (int64_t)h * g.gph + job.g_off[c];
        const float *srow = job.src + row * job.row_stride;

        // the 8 lanes of a group share its trip count, so the DPP moves and
        // shuffles of the min/max only ever read lanes of the same group
        int64_t gi = (int64_t)blockIdx.x * slots + slot;
        auto put = [&](const QOut &o, int64_t gq) {
            const int64_t gd = gdst0 + gq;
            __builtin_nontemporal_store(o.word, reinterpret_cast<uint32_t *>(blk + gd * 32 + l8 * 4));
            if (l8 == 0) {
                __builtin_nontemporal_store(o.scale, sp + gd);
                __builtin_nontemporal_store(o.bias, bp + gd);
            }
        };
        if (gstep >= job.n_g) {
            if (gi < job.n_g) {
                float4 lo, hi;
                load_group8<VEC>(srow + gi * 64, l8, lo, hi);
                put(quantize_group8(lo, hi, gbase), gi);
            }
            continue;
        }
        float4 lo, hi;
        if (gi < job.n_g) load_group8<VEC>(srow + gi * 64, l8, lo, hi);
        while (gi < job.n_g) {
            const int64_t gn = gi + gstep;
            float4 nlo = lo, nhi = hi;
            if (gn < job.n_g) load_group8<VEC>(srow + gn * 64, l8, nlo, nhi);
            put(quantize_group8(lo, hi, gbase), gi);
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
    if (job->n_rows > INT32_MAX) return (int)hipErrorInvalidValue;
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
        // blocks of 32 groups: two groups per lane where one pass over the
        // rows takes at least kOnePass blocks (long rows), else about
        // kQuantBlocks blocks (one pass or a few, each lane loading its next
        // group before it quantizes the current one)
        const int64_t need = (job->n_g + 31) / 32;
        const int64_t target = need * gy >= kOnePass ? need * gy / 2 : kQuantBlocks;
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
