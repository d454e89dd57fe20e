// common.h — device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../eakvd.h"

#define EAKV_WAVE 64

// Plane pointers of block (layer, kv) of a cache at `base`.
struct Planes {
    const uint8_t *w;
    const float *s;
    const float *b;
};

__device__ __host__ __forceinline__ Planes planes_of(const eakvd_geom &g,
                                                     const uint8_t *base,
                                                     int layer, int kv)
{
    const uint8_t *blk = base + (int64_t)(layer * 2 + kv) * g.block_bytes;
    Planes p;
    p.w = blk;
    p.s = (const float *)(blk + g.s_off);
    p.b = (const float *)(blk + g.b_off);
    return p;
}

// Byte i (0..15) of a 16-byte vector.
__device__ __forceinline__ uint32_t byte_of(const uint4 &v, int i)
{
    uint32_t w = i < 4 ? v.x : (i < 8 ? v.y : (i < 12 ? v.z : v.w));
    return (w >> (8 * (i & 3))) & 0xffu;
}

// Reference reduce_add over 16 lanes, pairwise halving tree (the order the
// CPU restatement fixes): v8[i]=a[i]+a[i+8], v4, v2, then v2[0]+v2[1].
__device__ __forceinline__ float reduce16(const float *a)
{
    float v8[8], v4[4], v2[2];
#pragma unroll
    for (int i = 0; i < 8; i++) v8[i] = __fadd_rn(a[i], a[i + 8]);
#pragma unroll
    for (int i = 0; i < 4; i++) v4[i] = __fadd_rn(v8[i], v8[i + 4]);
#pragma unroll
    for (int i = 0; i < 2; i++) v2[i] = __fadd_rn(v4[i], v4[i + 2]);
    return __fadd_rn(v2[0], v2[1]);
}

// Wave64 reductions (butterfly; every lane ends with the same value).
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, 64));
    return v;
}

static inline int ceil_div_i(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define EAKV_LOG2E 1.4426950408889634f
