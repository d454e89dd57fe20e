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
// Work split: 16 lanes per group, each lane one float4 (elements 4l..4l+3,
// so lanes 0-7 carry the low-nibble half and lanes 8-15 the high half).
// A wave covers 4 groups = 1 KB of contiguous f32 per load instruction.
#include "common.h"

namespace {

template <int NT, bool VEC>
__global__ __launch_bounds__(NT) void quantize_kernel(eakvd_geom g,
                                                      eakvd_quant_job job)
{
    const int lane16 = threadIdx.x & 15;
    const int slot = threadIdx.x >> 4;
    const int slot_shift = (threadIdx.x & 63) & ~15;
    const int64_t slots = NT / 16;
    const int64_t per_cache = (int64_t)job.n_planes * job.nh;

    for (int64_t row = blockIdx.y; row < job.n_rows; row += gridDim.y) {
        const int c = (int)(row / per_cache);
        const int64_t rem = row % per_cache;
        const int plane = job.plane0 + (int)(rem / job.nh);
        const int64_t h = rem % job.nh;
        uint8_t *blk = job.base[c] + (int64_t)plane * g.block_bytes;
        uint8_t *wp = blk;
        float *sp = (float *)(blk + g.s_off);
        float *bp = (float *)(blk + g.b_off);
        const int64_t gdst0 = h * g.gph + job.g_off[c];
        const float *srow = job.src + row * job.row_stride;

        for (int64_t gi = (int64_t)blockIdx.x * slots + slot; gi < job.n_g;
             gi += (int64_t)gridDim.x * slots) {
            const float *xp = srow + gi * 64 + lane16 * 4;
            float4 x;
            if (VEC) {
                x = *reinterpret_cast<const float4 *>(xp);
            } else {
                x.x = xp[0]; x.y = xp[1]; x.z = xp[2]; x.w = xp[3];
            }

            float mn, mx;
            group_minmax(x, slot_shift, mn, mx);

            const float range = __fsub_rn(mx, mn);
            float scale = 1.0f, inv = 0.0f;
            if (range > 0.0f) {
                scale = range / 15.0f;
                inv = 15.0f / range;
            }

            const uint32_t q0 = q4(x.x, mn, inv), q1 = q4(x.y, mn, inv);
            const uint32_t q2 = q4(x.z, mn, inv), q3 = q4(x.w, mn, inv);
            const uint32_t mine = q0 | (q1 << 8) | (q2 << 16) | (q3 << 24);
            const uint32_t hi = (uint32_t)__shfl_xor((int)mine, 8, 16);

            const int64_t gd = gdst0 + gi;
            if (lane16 < 8) {
                *reinterpret_cast<uint32_t *>(wp + gd * 32 + lane16 * 4) =
                    mine | (hi << 4);
            }
            if (lane16 == 0) {
                sp[gd] = scale;
                bp[gd] = mn;
            }
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
    if (job->n_g <= 4) {
        const dim3 grid(1, (unsigned)gy);
        if (vec)
            hipLaunchKernelGGL((quantize_kernel<64, true>), grid, dim3(64), 0,
                               st, *g, *job);
        else
            hipLaunchKernelGGL((quantize_kernel<64, false>), grid, dim3(64), 0,
                               st, *g, *job);
    } else {
        // about 8 K blocks of 16 groups per pass over the rows
        int64_t need = (job->n_g + 15) / 16;
        int64_t gx = (8192 + gy - 1) / gy;
        if (gx > need) gx = need;
        if (gx < 1) gx = 1;
        const dim3 grid((unsigned)gx, (unsigned)gy);
        if (vec)
            hipLaunchKernelGGL((quantize_kernel<256, true>), grid, dim3(256), 0,
                               st, *g, *job);
        else
            hipLaunchKernelGGL((quantize_kernel<256, false>), grid, dim3(256), 0,
                               st, *g, *job);
    }
    return (int)hipGetLastError();
}
