// kscore.hip — unfused K-score on the packed cache (MHA and GQA, d=64/128).
//
// Restates reference kernels/fused_k_score.ea:161-235,
// fused_k_score_64.ea:100-153, fused_k_score_gqa.ea:7-99 and
// fused_k_score_gqa_64.ea:6-73 with the same arithmetic per (q head, token):
//   k     = fma(nibble, scale, bias)                       (dequant, 1 rounding)
//   acc_i = fma chain over chunks c of k[c*16+i]*q[c*16+i]  (16 lanes)
//   score = reduce_add(acc) * (1/sqrt(d))
// Chunk c of a token covers dims c*16..c*16+15: group c/4, bytes
// (c&1)*16..+15, low nibbles for c%4 < 2.
//
// Layout: one lane per token.  A token's 32*gpd packed bytes are read as
// uint4 vectors; its dequantized values are computed once and dotted with
// every q head of its group (the reference GQA loop flip).  The q vectors are
// wave-uniform and are read through the scalar cache.
#include "common.h"

namespace {

template <int D>
__global__ __launch_bounds__(256) void k_score_kernel(
    const uint8_t *__restrict__ kw, const float *__restrict__ ks,
    const float *__restrict__ kb, int64_t gph, int L,
    const float *__restrict__ q, int qpk, float *__restrict__ scores, float rs)
{
    constexpr int GPD = D / 64;
    constexpr int NC = D / 16;
    const int kvh = blockIdx.y;
    const int t = blockIdx.x * 256 + threadIdx.x;
    if (t >= L) return;

    const int64_t g0 = (int64_t)kvh * gph + (int64_t)t * GPD;
    const uint4 *src = reinterpret_cast<const uint4 *>(kw + g0 * 32);
    uint4 raw[2 * GPD];
#pragma unroll
    for (int i = 0; i < 2 * GPD; i++) raw[i] = src[i];
    float sc[GPD], bi[GPD];
#pragma unroll
    for (int j = 0; j < GPD; j++) {
        sc[j] = ks[g0 + j];
        bi[j] = kb[g0 + j];
    }

    float k[D];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int grp = c >> 2, cc = c & 3;
        const uint4 &v = raw[grp * 2 + (cc & 1)];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            uint32_t b = byte_of(v, i);
            uint32_t n = cc < 2 ? (b & 15u) : (b >> 4);
            k[c * 16 + i] = fmaf((float)n, sc[grp], bi[grp]);
        }
    }

    for (int o = 0; o < qpk; o++) {
        const int qh = kvh * qpk + o;
        const float *qv = q + (int64_t)qh * D;
        float acc[16];
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                acc[i] = fmaf(k[c * 16 + i], qv[c * 16 + i], acc[i]);
        scores[(int64_t)qh * L + t] = __fmul_rn(reduce16(acc), rs);
    }
}

}  // namespace

extern "C" int eakvd_k_score(const eakvd_geom *g, const uint8_t *base,
                             int layer, int seq_len, const float *q, int n_q,
                             int n_kv, float *scores, void *stream)
{
    if (seq_len <= 0) return 0;
    const Planes p = planes_of(*g, base, layer, 0);
    const hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)ceil_div_i(seq_len, 256), (unsigned)n_kv);
    const int qpk = n_q / n_kv;
    const float rs = 1.0f / sqrtf((float)g->head_dim);
    if (g->head_dim == 64)
        hipLaunchKernelGGL(k_score_kernel<64>, grid, dim3(256), 0, st, p.w,
                           p.s, p.b, g->gph, seq_len, q, qpk, scores, rs);
    else
        hipLaunchKernelGGL(k_score_kernel<128>, grid, dim3(256), 0, st, p.w,
                           p.s, p.b, g->gph, seq_len, q, qpk, scores, rs);
    return (int)hipGetLastError();
}
