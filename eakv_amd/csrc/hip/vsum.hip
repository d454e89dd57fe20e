// vsum.hip — unfused V weighted sum on the packed cache (MHA and GQA,
// d=64/128).
//
// Restates reference kernels/fused_v_sum.ea:83-163, fused_v_sum_64.ea:55-110,
// fused_k_score_gqa.ea:106-305 and fused_k_score_gqa_64.ea:79-209: per
// (q head, dim) the product terms are o = fma(fma(nibble, s, b), w[t], o).
// The reference runs one chain over all t; here the sequence is split over
// token slots and chunks (each a sequential chain) and the partial sums are
// added in a fixed order, so results are deterministic and agree with the
// single chain to rounding.
//
// Layout: a lane owns one packed dword of a token (8 dims: 4 low nibbles and
// the 4 high nibbles 32 dims further), D/8 lanes per token, 256/(D/8) token
// slots per block.  V is dequantized once per token and reused by every q
// head of its group (at most 8 per pass).
#include "common.h"

namespace {

constexpr int kHeadsPerPass = 8;

template <int D>
__global__ __launch_bounds__(256) void v_sum_kernel(
    const uint8_t *__restrict__ vw, const float *__restrict__ vs,
    const float *__restrict__ vb, int64_t gph, int L,
    const float *__restrict__ w, int n_q, int qpk, int chunk,
    float *__restrict__ partial)
{
    constexpr int GPD = D / 64;
    constexpr int LPT = D / 8;
    constexpr int SLOTS = 256 / LPT;
    __shared__ float red[SLOTS * D];

    const int kvh = blockIdx.y;
    const int ch = blockIdx.x;
    const int lt = threadIdx.x % LPT;
    const int slot = threadIdx.x / LPT;
    const int grp = lt / 8, dj = lt % 8;
    const int t_begin = ch * chunk;
    const int t_end = min(L, t_begin + chunk);
    // dims of this lane: lo e -> 64*grp + 4*dj + e, hi e -> +32
    const int dim_lo = 64 * grp + 4 * dj;

    for (int hb = 0; hb < qpk; hb += kHeadsPerPass) {
        const int nh = min(kHeadsPerPass, qpk - hb);
        float acc[kHeadsPerPass][8];
#pragma unroll
        for (int o = 0; o < kHeadsPerPass; o++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[o][e] = 0.0f;

        for (int t = t_begin + slot; t < t_end; t += SLOTS) {
            const int64_t g = (int64_t)kvh * gph + (int64_t)t * GPD + grp;
            const uint32_t word =
                *reinterpret_cast<const uint32_t *>(vw + g * 32 + dj * 4);
            const float s = vs[g], b = vb[g];
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[e] = fmaf((float)((word >> (8 * e)) & 15u), s, b);
                v[4 + e] = fmaf((float)((word >> (8 * e + 4)) & 15u), s, b);
            }
#pragma unroll
            for (int o = 0; o < kHeadsPerPass; o++) {
                if (o < nh) {
                    const int qh = kvh * qpk + hb + o;
                    const float wt = w[(int64_t)qh * L + t];
#pragma unroll
                    for (int e = 0; e < 8; e++)
                        acc[o][e] = fmaf(v[e], wt, acc[o][e]);
                }
            }
        }

        // o is unrolled so acc stays in registers; nh is block-uniform, so
        // the barriers below are reached by every thread or by none.
#pragma unroll
        for (int o = 0; o < kHeadsPerPass; o++) {
            if (o >= nh) break;
            float *r = red + slot * D;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                r[dim_lo + e] = acc[o][e];
                r[dim_lo + 32 + e] = acc[o][4 + e];
            }
            __syncthreads();
            if (threadIdx.x < D) {
                float sum = red[threadIdx.x];
                for (int sl = 1; sl < SLOTS; sl++)
                    sum = __fadd_rn(sum, red[sl * D + threadIdx.x]);
                const int qh = kvh * qpk + hb + o;
                partial[((int64_t)ch * n_q + qh) * D + threadIdx.x] = sum;
            }
            __syncthreads();
        }
    }
}

// out[i] = sum over chunks in order of partial[c][i]
__global__ __launch_bounds__(256) void chunk_sum_kernel(
    const float *__restrict__ partial, int n_chunks, int64_t n_out,
    float *__restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n_out) return;
    float sum = partial[i];
    for (int c = 1; c < n_chunks; c++)
        sum = __fadd_rn(sum, partial[(int64_t)c * n_out + i]);
    out[i] = sum;
}

int v_sum_chunk(int seq_len, int n_kv)
{
    // about 2048 blocks over the kv heads, at least 64 tokens per block
    int64_t c = ((int64_t)seq_len * n_kv + 2047) / 2048;
    c = (c + 63) / 64 * 64;
    if (c < 64) c = 64;
    return (int)c;
}

}  // namespace

extern "C" size_t eakvd_v_sum_work_bytes(const eakvd_geom *g, int seq_len,
                                         int n_q)
{
    if (seq_len <= 0) return 0;
    const int chunk = v_sum_chunk(seq_len, g->n_kv_heads);
    const int n_chunks = ceil_div_i(seq_len, chunk);
    return (size_t)n_chunks * n_q * g->head_dim * sizeof(float);
}

extern "C" int eakvd_v_sum(const eakvd_geom *g, const uint8_t *base,
                           int layer, int seq_len, const float *w, int n_q,
                           int n_kv, float *out, void *work, void *stream)
{
    const hipStream_t st = (hipStream_t)stream;
    const int64_t n_out = (int64_t)n_q * g->head_dim;
    if (seq_len <= 0)
        return (int)hipMemsetAsync(out, 0, n_out * sizeof(float), st);
    const Planes p = planes_of(*g, base, layer, 1);
    // the chunk is sized from the cache's head count so that the work size
    // does not depend on n_kv
    const int chunk = v_sum_chunk(seq_len, g->n_kv_heads);
    const int n_chunks = ceil_div_i(seq_len, chunk);
    const int qpk = n_q / n_kv;
    float *partial = (float *)work;
    const dim3 grid((unsigned)n_chunks, (unsigned)n_kv);
    if (g->head_dim == 64)
        hipLaunchKernelGGL(v_sum_kernel<64>, grid, dim3(256), 0, st, p.w, p.s,
                           p.b, g->gph, seq_len, w, n_q, qpk, chunk, partial);
    else
        hipLaunchKernelGGL(v_sum_kernel<128>, grid, dim3(256), 0, st, p.w,
                           p.s, p.b, g->gph, seq_len, w, n_q, qpk, chunk,
                           partial);
    hipLaunchKernelGGL(chunk_sum_kernel, dim3((unsigned)ceil_div_i(n_out, 256)),
                       dim3(256), 0, st, partial, n_chunks, n_out, out);
    return (int)hipGetLastError();
}
