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
// two adjacent floats (8-byte aligned) in one device-scope store
__device__ __forceinline__ void st_dev2(float *p, float a, float b)
{
    const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// two adjacent floats (8-byte aligned) in one device-scope load
__device__ __forceinline__ float2 ld_dev2(const float *p)
{
    const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<float *>(p)),
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
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

// ---- Q4 group quantization pieces shared by the cache quantizer and the
// ggml block type (8 lanes per 64-value group).
//
// The reference's nibble is q = clamp(to_i32((x - mn)*inv + 0.5), 0, 15),
// each step rounded, to_i32 with x86 cvttss2si semantics (NaN and values
// outside the int32 range -> INT32_MIN), inv = range > 0 ? 15/range : 0.
// Over the values a group can produce, one v_cvt_i32_f32 (truncation, NaN
// -> 0) gives the same nibble:
//   inv finite and > 0: every non-NaN element lies in [mn, mx], so x - mn
//     rounds into [0, range] and (x - mn)*inv to at most
//     RN(range * RN(15/range)) <= 15 + 2^-20; v lies in [0.5, 16) and
//     truncates to 0..15 with the clamp idle.  A NaN element gives v = NaN
//     -> 0, the reference's INT32_MIN clamped.
//   inv = 0 (range 0, NaN or +inf): v = 0.5 or NaN -> 0, as the reference.
//   inv = +inf (15/range overflows: range < 15/FLT_MAX): the reference's v
//     is +inf (x > mn) or NaN (x = mn: 0*inf), every nibble 0.  q4_factor
//     turns that inv into NaN, so every v is NaN -> 0.
// (The range test and clamp cost three more instructions per element.)
__device__ __forceinline__ float q4_factor(float inv)
{
    return inv == __builtin_inff() ? __builtin_nanf("") : inv;
}

// q4(x, mn, q4_factor(inv)): the reference's nibble of x.
__device__ __forceinline__ uint32_t q4(float x, float mn, float f)
{
    const float v = __fadd_rn(__fmul_rn(__fsub_rn(x, mn), f), 0.5f);
    int q;
    // the instruction itself, whose NaN result is defined (0), where C's
    // float-to-int conversion leaves NaN undefined
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(v));
    return (uint32_t)q;
}

// DPP moves within 8-lane groups: the mirror of each half row (lane i and
// 7 - i), and the quad permutations xor 2 and xor 1.
constexpr int kDppHalfMirror = 0x141, kDppXor2 = 0x4E, kDppXor1 = 0xB1;
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// The first element of the group, in index order, that compares equal to
// zero (the group has one): the low halves of lanes 0-7 hold elements 0-31,
// the high halves 32-63.  gbase: the group's first lane in the wave.
__device__ __forceinline__ float first_zero8(const float4 &lo, const float4 &hi, int gbase)
{
    const float zl = lo.x == 0.0f ? lo.x : (lo.y == 0.0f ? lo.y : (lo.z == 0.0f ? lo.z : lo.w));
    const float zh = hi.x == 0.0f ? hi.x : (hi.y == 0.0f ? hi.y : (hi.z == 0.0f ? hi.z : hi.w));
    const bool hl = (lo.x == 0.0f) | (lo.y == 0.0f) | (lo.z == 0.0f) | (lo.w == 0.0f);
    const bool hh = (hi.x == 0.0f) | (hi.y == 0.0f) | (hi.z == 0.0f) | (hi.w == 0.0f);
    const uint32_t bl = (uint32_t)(__ballot(hl) >> gbase) & 0xffu;
    const uint32_t bh = (uint32_t)(__ballot(hh) >> gbase) & 0xffu;
    const int sl = bl ? __ffs((int)bl) - 1 : 0;
    const int sh = bh ? __ffs((int)bh) - 1 : 0;
    const float vl = __shfl(zl, sl, 8), vh = __shfl(zh, sh, 8);
    return bl ? vl : vh;
}

// min and max of a 64-value group held by 8 lanes (lane j: elements 4j..4j+3
// in lo, 32+4j..32+4j+3 in hi; gbase = the group's first lane in the wave)
// as a strict </> scan from element 0 finds them: the first occurrence wins
// (so +0 / -0 as they come first), NaN elements after element 0 are
// skipped, a NaN element 0 gives min = max = NaN.  Every lane of the group
// gets both; the groups of a wave must run the same branches together
// (their lanes share a trip count).
__device__ __forceinline__ void group_minmax8(const float4 &lo, const float4 &hi, int gbase,
                                              float &mn, float &mx)
{
    mn = fminf(fminf(fminf(lo.x, lo.y), fminf(lo.z, lo.w)),
               fminf(fminf(hi.x, hi.y), fminf(hi.z, hi.w)));
    mx = fmaxf(fmaxf(fmaxf(lo.x, lo.y), fmaxf(lo.z, lo.w)),
               fmaxf(fmaxf(hi.x, hi.y), fmaxf(hi.z, hi.w)));
    mn = fminf(mn, dpp_f<kDppHalfMirror>(mn));
    mx = fmaxf(mx, dpp_f<kDppHalfMirror>(mx));
    mn = fminf(mn, dpp_f<kDppXor2>(mn));
    mx = fmaxf(mx, dpp_f<kDppXor2>(mx));
    mn = fminf(mn, dpp_f<kDppXor1>(mn));
    mx = fmaxf(mx, dpp_f<kDppXor1>(mx));
    // a zero min or max: the first zero's sign, as a strict scan keeps it
    if (mn == 0.0f || mx == 0.0f) {
        const float z = first_zero8(lo, hi, gbase);
        if (mn == 0.0f) mn = z;
        if (mx == 0.0f) mx = z;
    }
    // a NaN element 0 makes min = max = that NaN
    if (__ballot((threadIdx.x & 7) == 0 && lo.x != lo.x) != 0) {
        const float x0 = __shfl(lo.x, 0, 8);
        if (x0 != x0) {
            mn = x0;
            mx = x0;
        }
    }
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define EAKV_LOG2E 1.4426950408889634f
