// synth.hip — seeded synthetic KV / query generator on the device, for the
// benchmark and the full-size tests (libeakv_synth.so; not part of the eakv
// API).  Value (row, pos, dim) depends only on (seed, row, pos, dim), so any
// slice of a cache — a whole layer, one appended token — can be regenerated
// independently and identically.
//
//   v = N(0,1) * sigma * chan[row][dim] * (1 + drift_amp*sin(pos/drift_period))
//   with probability outlier_p, v = +-outlier_v instead
// N(0,1) by Box-Muller from a splitmix64 hash of the counter.
#include <hip/hip_runtime.h>
#include <stdint.h>

extern "C" {
typedef struct {
    uint64_t     seed;
    int64_t      row0;         // hash id of the first row
    int64_t      pos0;         // position of the first token
    float        sigma;
    const float *chan;         // device [n_rows][d] or NULL
    float        drift_amp, drift_period;
    float        outlier_p, outlier_v;
} eakv_synth_params;
}

namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void synth_kernel(float *__restrict__ out,
                                                    int64_t n, int64_t n_tok,
                                                    int d, eakv_synth_params p)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        const int dim = (int)(i % d);
        const int64_t rt = i / d;
        const int64_t tok = rt % n_tok, r = rt / n_tok;
        const int64_t pos = p.pos0 + tok;
        const uint64_t ctr = ((uint64_t)(p.row0 + r) << 40) ^
                             ((uint64_t)pos << 12) ^ (uint64_t)dim;
        const uint64_t h = mix64(p.seed ^ mix64(ctr));
        const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);
        const float u2 = (float)((h >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
        float v = sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795865f * u2);
        v *= p.sigma;
        if (p.chan) v *= p.chan[r * d + dim];
        if (p.drift_amp != 0.0f)
            v *= 1.0f + p.drift_amp * sinf((float)pos / p.drift_period);
        if (p.outlier_p > 0.0f) {
            const uint64_t h2 = mix64(h ^ 0xD1B54A32D192ED03ull);
            const float u3 = (float)(h2 >> 40) * (1.0f / 16777216.0f);
            if (u3 < p.outlier_p) v = (h2 & 1) ? p.outlier_v : -p.outlier_v;
        }
        out[i] = v;
    }
}

}  // namespace

// out[r][t][i] for r < n_rows, t < n_tok, i < d.
extern "C" int eakv_synth_fill(float *out, int64_t n_rows, int64_t n_tok, int d,
                               const eakv_synth_params *p, void *stream)
{
    const int64_t n = n_rows * n_tok * d;
    if (n <= 0) return 0;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(synth_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, out, n, n_tok, d, *p);
    return (int)hipGetLastError();
}

namespace {

// Plain streaming copy, 16 B per lane per iteration: the known-size kernel
// that HBM byte counters (FETCH_SIZE, WRITE_SIZE) are calibrated against.
__global__ __launch_bounds__(256) void copy_kernel(uint4 *__restrict__ dst,
                                                   const uint4 *__restrict__ src,
                                                   int64_t n16)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16;
         i += (int64_t)gridDim.x * 256)
        dst[i] = src[i];
}

// Plain streaming read, two 16-byte non-temporal loads in flight per lane,
// the words xor-folded into one word per thread: the device's sustained read
// rate for one contiguous region, the practical ceiling of a bandwidth-bound
// pass.  The non-temporal hint is worth about 7% (335.8 MB passes, 3 blocks
// per CU: 6.78-6.80 against 6.29-6.39 TB/s), as on the fused kernel's plane
// loads.
__global__ __launch_bounds__(256) void read_kernel(const uint4 *__restrict__ src, int64_t n16,
                                                   unsigned *__restrict__ sink)
{
    const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t nt = (int64_t)gridDim.x * 256;
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *s4 = reinterpret_cast<const u32x4 *>(src);
    unsigned a = 0;
    for (int64_t i = tid; i < n16; i += 2 * nt) {
        const u32x4 u = __builtin_nontemporal_load(&s4[i]);
        const u32x4 v = i + nt < n16 ? __builtin_nontemporal_load(&s4[i + nt])
                                     : u32x4{0, 0, 0, 0};
        a ^= u.x ^ u.y ^ u.z ^ u.w ^ v.x ^ v.y ^ v.z ^ v.w;
    }
    sink[tid] = a;
}

// The caller's row softmax of the reference's unfused workload (scores ->
// softmax -> output; the reference leaves it to the caller): one block of
// 1024 threads per row, w = exp(s - max) * (1 / sum), the max starting at
// -1e6 as in the reference's fused kernel.  Rows of up to 16384 values stay
// in registers (one read, one write); longer rows are read three times.
// Used to time that workload, not for parity.
__device__ __forceinline__ float block_max(float m, float *red)
{
    for (int k = 32; k >= 1; k >>= 1) m = fmaxf(m, __shfl_xor(m, k, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int i = 1; i < 16; i++) m = fmaxf(m, red[i]);
    __syncthreads();
    return m;
}

__device__ __forceinline__ float block_sum(float v, float *red)
{
    for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0];
    for (int i = 1; i < 16; i++) v += red[i];
    __syncthreads();
    return v;
}

template <int PER>
__global__ __launch_bounds__(1024) void softmax_kernel(const float *__restrict__ s,
                                                       float *__restrict__ w, int L)
{
    __shared__ float red[16];
    const float *r = s + (int64_t)blockIdx.x * L;
    float *o = w + (int64_t)blockIdx.x * L;
    const int t = threadIdx.x;
    if constexpr (PER > 0) {
        float v[PER];
        float m = -1000000.0f;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = t + 1024 * k;
            v[k] = i < L ? r[i] : -INFINITY;
            m = fmaxf(m, v[k]);
        }
        m = block_max(m, red);
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            v[k] = expf(v[k] - m);
            sum += v[k];
        }
        const float inv = 1.0f / block_sum(sum, red);
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = t + 1024 * k;
            if (i < L) o[i] = v[k] * inv;
        }
    } else {
        float m = -1000000.0f;
        for (int i = t; i < L; i += 1024) m = fmaxf(m, r[i]);
        m = block_max(m, red);
        float sum = 0.0f;
        for (int i = t; i < L; i += 1024) sum += expf(r[i] - m);
        const float inv = 1.0f / block_sum(sum, red);
        for (int i = t; i < L; i += 1024) o[i] = expf(r[i] - m) * inv;
    }
}

}  // namespace

// Row softmax of scores[n_rows][L] into w (device pointers).
extern "C" int eakv_synth_softmax(const float *scores, float *w, int n_rows, int L, void *stream)
{
    if (n_rows <= 0 || L <= 0) return 0;
    const hipStream_t st = (hipStream_t)stream;
    const dim3 g((unsigned)n_rows), b(1024);
    if (L <= 2048)
        hipLaunchKernelGGL(softmax_kernel<2>, g, b, 0, st, scores, w, L);
    else if (L <= 4096)
        hipLaunchKernelGGL(softmax_kernel<4>, g, b, 0, st, scores, w, L);
    else if (L <= 8192)
        hipLaunchKernelGGL(softmax_kernel<8>, g, b, 0, st, scores, w, L);
    else if (L <= 16384)
        hipLaunchKernelGGL(softmax_kernel<16>, g, b, 0, st, scores, w, L);
    else
        hipLaunchKernelGGL(softmax_kernel<0>, g, b, 0, st, scores, w, L);
    return (int)hipGetLastError();
}

namespace {

// scores[h][t] = (q[h] . k[h][t]) / sqrt(d) on f32 rows k[(h*L + t)*d ..],
// one thread per (h, t), the dims in order (a plain dot, no quantization).
__global__ __launch_bounds__(256) void dot_kernel(const float *__restrict__ k,
                                                  const float *__restrict__ q,
                                                  float *__restrict__ scores, int nh, int L,
                                                  int d, float rs)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)nh * L) return;
    const int h = (int)(i / L);
    const float4 *kr = reinterpret_cast<const float4 *>(k + i * d);
    const float4 *qr = reinterpret_cast<const float4 *>(q + (int64_t)h * d);
    float sum = 0.0f;
    for (int c = 0; c < d / 4; c++) {
        const float4 a = kr[c], b = qr[c];
        sum = fmaf(a.x, b.x, sum);
        sum = fmaf(a.y, b.y, sum);
        sum = fmaf(a.z, b.z, sum);
        sum = fmaf(a.w, b.w, sum);
    }
    scores[i] = sum * rs;
}

}  // namespace

// The reference benchmark's dot baselines (benchmarks/bench_libeakv.c:76-122)
// on the device: scores[nh][L] = q[nh][d] . k[nh][L][d] / sqrt(d), d a
// multiple of 4, all pointers 16-byte aligned.
extern "C" int eakv_synth_dot_scores(const float *k, const float *q, float *scores, int nh,
                                     int L, int d, void *stream)
{
    if (nh <= 0 || L <= 0) return 0;
    if ((d & 3) || ((uintptr_t)k & 15) || ((uintptr_t)q & 15)) return (int)hipErrorInvalidValue;
    const int64_t n = (int64_t)nh * L;
    hipLaunchKernelGGL(dot_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, k, q, scores, nh, L, d, 1.0f / sqrtf((float)d));
    return (int)hipGetLastError();
}

// Compute units of the current device (0 if the query fails).
extern "C" int eakv_synth_cu_count(void)
{
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return v;
}

// Reads src[0, n_bytes) once (n_bytes a multiple of 16, src 16-aligned) with
// `blocks` blocks of 256 threads; sink receives blocks * 256 words.
extern "C" int eakv_synth_read(const void *src, int64_t n_bytes, unsigned *sink, int blocks,
                               void *stream)
{
    if (n_bytes <= 0 || blocks <= 0) return 0;
    if ((n_bytes & 15) || ((uintptr_t)src & 15)) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(read_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const uint4 *)src, n_bytes / 16, sink);
    return (int)hipGetLastError();
}

// dst[0, n_bytes) = src[0, n_bytes); n_bytes a multiple of 16, both 16-aligned.
extern "C" int eakv_synth_copy(void *dst, const void *src, int64_t n_bytes,
                               void *stream)
{
    if (n_bytes <= 0) return 0;
    if ((n_bytes & 15) || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15))
        return (int)hipErrorInvalidValue;
    const int64_t n16 = n_bytes / 16;
    int64_t blocks = (n16 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (uint4 *)dst, (const uint4 *)src, n16);
    return (int)hipGetLastError();
}

namespace {

// One wave sleeps until the device's real-time counter has advanced `ticks`
// past its first reading, or after `max_iter` sleeps, whichever comes
// first: every launch ends.
__global__ __launch_bounds__(64) void hold_kernel(uint64_t ticks, int max_iter)
{
    const uint64_t t0 = wall_clock64();
    for (int i = 0; i < max_iter; i++) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(64);
    }
}

}  // namespace

// Occupies `stream` for about `us` microseconds (at most 100 ms) with one
// sleeping wave, so that the calls the host enqueues behind it wait in the
// stream's queue and then run back to back: the device time of a run of short
// calls without the host's issue rate in it.
extern "C" int eakv_synth_hold(int us, void *stream)
{
    if (us <= 0) return 0;
    if (us > 100000) us = 100000;
    // s_sleep 64 is about 64 x 64 clocks, 1.7-4 us; the cap ends the launch
    // within a few times the request even if the counter does not advance.
    const int max_iter = us + 1000;
    int dev = 0, khz = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess ||
        khz <= 0)
        khz = 100000;
    hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (uint64_t)us * (uint64_t)khz / 1000, max_iter);
    return (int)hipGetLastError();
}
