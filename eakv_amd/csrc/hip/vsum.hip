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
// head of its group (HP per pass: 1, 2, 4 or 8, the smallest that covers
// the group up to 8, so registers are spent only on heads that exist).  A lane takes kBatch tokens of its
// slot at a time and issues all their loads (V word, scale, bias, weights)
// before the arithmetic, so kBatch loads per lane are in flight; a block
// covers a chunk of kChunk tokens of one kv head and writes one partial per
// q head, which chunk_sum_kernel adds in a fixed order.
#include "common.h"

namespace {

constexpr int kBatch = 8;
constexpr int kChunk = 256;

template <int D, int HP>
__global__ __launch_bounds__(256) void v_sum_kernel(
    const uint8_t *__restrict__ vw, const float *__restrict__ vs,
    const float *__restrict__ vb, int64_t gph, int L,
    const float *__restrict__ w, int n_q, int qpk, float *__restrict__ partial)
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
    const int t_begin = ch * kChunk;
    const int t_end = min(L, t_begin + kChunk);
    // dims of this lane: lo e -> 64*grp + 4*dj + e, hi e -> +32
    const int dim_lo = 64 * grp + 4 * dj;

    for (int hb = 0; hb < qpk; hb += HP) {
        const int nh = min(HP, qpk - hb);
        const float *wq = w + (int64_t)(kvh * qpk + hb) * L;
        float acc[HP][8];
#pragma unroll
        for (int o = 0; o < HP; o++)
#pragma unroll
            for (int e = 0; e < 8; e++) acc[o][e] = 0.0f;

        for (int t0 = t_begin + slot; t0 < t_end; t0 += SLOTS * kBatch) {
            uint32_t word[kBatch];
            float sc[kBatch], bi[kBatch], wt[kBatch][HP];
#pragma unroll
            for (int u = 0; u < kBatch; u++) {
                const int t = t0 + u * SLOTS;
                const bool in = t < t_end;
                const int tt = in ? t : t_begin;
                const int64_t g = (int64_t)kvh * gph + (int64_t)tt * GPD + grp;
                word[u] = *reinterpret_cast<const uint32_t *>(vw + g * 32 + dj * 4);
                sc[u] = vs[g];
                bi[u] = vb[g];
#pragma unroll
                for (int o = 0; o < HP; o++)
                    wt[u][o] = (in && o < nh) ? wq[(int64_t)o * L + tt] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kBatch; u++) {
                if (t0 + u * SLOTS >= t_end) break;
                float v[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[e] = fmaf((float)((word[u] >> (8 * e)) & 15u), sc[u], bi[u]);
                    v[4 + e] = fmaf((float)((word[u] >> (8 * e + 4)) & 15u), sc[u], bi[u]);
                }
#pragma unroll
                for (int o = 0; o < HP; o++) {
                    if (o < nh) {
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[o][e] = fmaf(v[e], wt[u][o], acc[o][e]);
                    }
                }
            }
        }

        // o is unrolled so acc stays in registers; nh is block-uniform, so
        // the barriers below are reached by every thread or by none.
#pragma unroll
        for (int o = 0; o < HP; o++) {
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

// out[i] = the sum over chunks of partial[c][i], in a fixed order: a block
// takes 32 outputs; thread (i, part) adds chunks part, part + 8, ... in
// order, kSumBatch at a time with their loads in flight (32 consecutive
// outputs per row of threads: coalesced), and the 8 part sums of an output
// are then added in part order.
constexpr int kSumParts = 8;
constexpr int kSumBatch = 16;

__global__ __launch_bounds__(256) void chunk_sum_kernel(
    const float *__restrict__ partial, int n_chunks, int64_t n_out,
    float *__restrict__ out)
{
    __shared__ float red[kSumParts][32];
    const int o = threadIdx.x & 31, part = threadIdx.x >> 5;
    const int64_t i = (int64_t)blockIdx.x * 32 + o;
    const int64_t ic = i < n_out ? i : n_out - 1;
    float sum = 0.0f;
    for (int c0 = part; c0 < n_chunks; c0 += kSumParts * kSumBatch) {
        float p[kSumBatch];
#pragma unroll
        for (int j = 0; j < kSumBatch; j++) {
            const int c = c0 + j * kSumParts;
            p[j] = c < n_chunks ? partial[(int64_t)c * n_out + ic] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kSumBatch; j++)
            if (c0 + j * kSumParts < n_chunks) sum = __fadd_rn(sum, p[j]);
    }
    red[part][o] = sum;
    __syncthreads();
    if (part == 0 && i < n_out) {
        float t = red[0][o];
#pragma unroll
        for (int k = 1; k < kSumParts; k++) t = __fadd_rn(t, red[k][o]);
        out[i] = t;
    }
}

__global__ __launch_bounds__(256) void zero_kernel(float *__restrict__ out, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = 0.0f;
}

}  // namespace

extern "C" size_t eakvd_v_sum_work_bytes(const eakvd_geom *g, int seq_len,
                                         int n_q)
{
    if (seq_len <= 0) return 0;
    const int n_chunks = ceil_div_i(seq_len, kChunk);
    const size_t valu = (size_t)n_chunks * n_q * g->head_dim * sizeof(float);
    const size_t mfma = eakvd_v_sum_mfma_work_bytes(g, seq_len, n_q);
    return valu > mfma ? valu : mfma;
}

extern "C" int eakvd_v_sum(const eakvd_geom *g, const uint8_t *base,
                           int layer, int seq_len, const float *w, int n_q,
                           int n_kv, float *out, void *work, void *stream)
{
    const hipStream_t st = (hipStream_t)stream;
    const int64_t n_out = (int64_t)n_q * g->head_dim;
    if (seq_len <= 0) {
        // zeros by a kernel, not a memset: the call may be captured in a graph
        hipLaunchKernelGGL(zero_kernel, dim3((unsigned)ceil_div_i(n_out, 256)), dim3(256), 0,
                           st, out, n_out);
        return (int)hipGetLastError();
    }
    // the matrix-core program where it applies (up to 8 q heads per kv head)
    const int r = eakvd_v_sum_mfma(g, base, layer, seq_len, w, n_q, n_kv, out, work, stream);
    if (r >= 0) return r;
    const Planes p = planes_of(*g, base, layer, 1);
    const int n_chunks = ceil_div_i(seq_len, kChunk);
    const int qpk = n_q / n_kv;
    float *partial = (float *)work;
    const dim3 grid((unsigned)n_chunks, (unsigned)n_kv);
    auto kern = g->head_dim == 64
                    ? (qpk <= 1 ? v_sum_kernel<64, 1> : qpk <= 2 ? v_sum_kernel<64, 2>
                       : qpk <= 4 ? v_sum_kernel<64, 4> : v_sum_kernel<64, 8>)
                    : (qpk <= 1 ? v_sum_kernel<128, 1> : qpk <= 2 ? v_sum_kernel<128, 2>
                       : qpk <= 4 ? v_sum_kernel<128, 4> : v_sum_kernel<128, 8>);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, p.w, p.s, p.b, g->gph, seq_len, w, n_q,
                       qpk, partial);
    hipLaunchKernelGGL(chunk_sum_kernel, dim3((unsigned)ceil_div_i(n_out, 32)),
                       dim3(256), 0, st, partial, n_chunks, n_out, out);
    return (int)hipGetLastError();
}
