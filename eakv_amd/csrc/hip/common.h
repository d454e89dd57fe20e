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

// Byte J of x as a float, one v_cvt_f32_ubyteJ (the compiler otherwise
// extracts the byte with a separate v_bfe_u32 first).
template <int J>
__device__ __forceinline__ float ubyte_f32(uint32_t x)
{
    float r;
    if constexpr (J == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(x));
    else if constexpr (J == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(x));
    else if constexpr (J == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(x));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(x));
    return r;
}

// Chunk partials cross blocks through device-scope (sc1) stores and loads: they
// write through to, and read from, the device's coherence point, so no L2
// writeback or invalidate (a whole-cache operation per XCD, costlier than
// the kernel when every block pays it) is needed between blocks.
__device__ __forceinline__ void st_dev(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p)
{
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Compute units of the current device (looked up once; 256 if unknown).
static inline int cu_count()
{
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0, v = 0;
        n_cu = hipGetDevice(&dev) == hipSuccess &&
                       hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                           hipSuccess && v > 0
                   ? v : 256;
    }
    return n_cu;
}

// ---- Q4 group quantization pieces shared by the cache quantizer (q4) and
// the ggml block type (all of them: 16 lanes per 64-value group, lane l
// holding elements 4l..4l+3 as a float4; slot_shift = the group's first
// lane in the wave).

// f32 -> i32 with x86 cvttss2si semantics (NaN / out of range -> INT32_MIN).
__device__ __forceinline__ int to_i32_x86(float v)
{
    return (v >= -2147483648.0f && v < 2147483648.0f) ? (int)v : (int)0x80000000;
}

// q(x) = clamp(to_i32((x - mn)*inv + 0.5), 0, 15), each step rounded.
__device__ __forceinline__ uint32_t q4(float x, float mn, float inv)
{
    float v = __fadd_rn(__fmul_rn(__fsub_rn(x, mn), inv), 0.5f);
    int q = to_i32_x86(v);
    q = q < 0 ? 0 : (q > 15 ? 15 : q);
    return (uint32_t)q;
}

// First element (in index order 4*lane16 + i) of the group that compares
// equal to zero; its value carries the sign a strict scan keeps.
__device__ __forceinline__ float first_zero(const float4 &x, int slot_shift)
{
    float mine = x.x == 0.0f ? x.x
               : (x.y == 0.0f ? x.y : (x.z == 0.0f ? x.z : x.w));
    bool has = (x.x == 0.0f) | (x.y == 0.0f) | (x.z == 0.0f) | (x.w == 0.0f);
    uint64_t m = __ballot(has);
    uint32_t sm = (uint32_t)(m >> slot_shift) & 0xffffu;
    int src = __ffs((int)sm) - 1;
    if (src < 0) src = 0;
    return __shfl(mine, src, 16);
}

// min and max of a group as a strict </> scan from element 0 finds them:
// the first occurrence wins (so +0 / -0 as they come first), NaN elements
// after element 0 are skipped, a NaN element 0 gives min = max = NaN.
__device__ __forceinline__ void group_minmax(const float4 &x, int slot_shift, float &mn,
                                             float &mx)
{
    mn = fminf(fminf(x.x, x.y), fminf(x.z, x.w));
    mx = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, o, 16));
        mx = fmaxf(mx, __shfl_xor(mx, o, 16));
    }
    if (mn == 0.0f || mx == 0.0f) {
        const float z = first_zero(x, slot_shift);
        if (mn == 0.0f) mn = z;
        if (mx == 0.0f) mx = z;
    }
    const float x0 = __shfl(x.x, 0, 16);
    if (x0 != x0) { mn = x0; mx = x0; }
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define EAKV_LOG2E 1.4426950408889634f
