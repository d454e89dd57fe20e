// fused.hip — fused decode attention on the packed cache: K-score, softmax
// and V-sum in one pass over K and V, for a batch of same-shape caches.
//
// Semantics: reference kernels/fused_attention.ea:190-373 (two passes:
// max with init -1e6, w = exp(s - max), sum, o = fma(deq_v, w, o),
// out = o * (1/sum)), extended per q head to GQA and d=64.
//
// Work split (flash-decoding): one block per (sequence, kv head, chunk of
// CHUNK tokens).  Inside a block
//   A  one lane per token: K dequantized once (fma(nib, s, b)) and scored
//      against every q head of the group with the reference arithmetic
//      (16-lane fma chains, halving-tree reduce, * 1/sqrt(d));
//   B  chunk max m per head, p = exp(s - m), l = sum p (fixed order);
//   C  V: a lane owns one packed dword (8 dims) of a token, o += deq * p;
//   D  token slots summed in a fixed order, partial (m, l, o[D]) stored.
// A combine kernel merges the chunks of each (sequence, q head) in chunk
// order: M = max(-1e6, m_c), out = sum o_c e^(m_c-M) / sum l_c e^(m_c-M).
#include "common.h"

namespace {

constexpr int kChunk = 512;      // tokens per block
constexpr int kHeadsLds = 16;    // q heads per pass

template <int D>
__global__ __launch_bounds__(256) void fused_kernel(
    eakvd_geom g, eakvd_batch bt, int layer, const float *__restrict__ q,
    int n_q, int qpk, int max_chunks, float rs, float *__restrict__ part)
{
    constexpr int GPD = D / 64;
    constexpr int NC = D / 16;
    constexpr int LPT = D / 8;
    constexpr int SLOTS = 256 / LPT;
    __shared__ float sc[kHeadsLds][kChunk];
    __shared__ float red[SLOTS * D];
    __shared__ float wred[4];
    __shared__ float mh[kHeadsLds], lh[kHeadsLds];

    const int ch = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
    const int L = bt.seq_len[s];
    const int t0 = ch * kChunk;
    if (t0 >= L) return;
    const int nt = min(kChunk, L - t0);
    const Planes K = planes_of(g, bt.base[s], layer, 0);
    const Planes V = planes_of(g, bt.base[s], layer, 1);
    const float *qs = q + (int64_t)s * n_q * D;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    for (int hb = 0; hb < qpk; hb += kHeadsLds) {
        const int nh = min(kHeadsLds, qpk - hb);

        // ---- A: scores
        for (int i = tid; i < nt; i += 256) {
            const int t = t0 + i;
            const int64_t g0 = (int64_t)kvh * g.gph + (int64_t)t * GPD;
            const uint4 *src = reinterpret_cast<const uint4 *>(K.w + g0 * 32);
            uint4 raw[2 * GPD];
#pragma unroll
            for (int r = 0; r < 2 * GPD; r++) raw[r] = src[r];
            float kd[D];
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int grp = c >> 2, cc = c & 3;
                const float ss = K.s[g0 + grp], bb = K.b[g0 + grp];
                const uint4 &v = raw[grp * 2 + (cc & 1)];
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    uint32_t by = byte_of(v, e);
                    uint32_t n = cc < 2 ? (by & 15u) : (by >> 4);
                    kd[c * 16 + e] = fmaf((float)n, ss, bb);
                }
            }
            for (int o = 0; o < nh; o++) {
                const float *qv = qs + (int64_t)(kvh * qpk + hb + o) * D;
                float acc[16];
#pragma unroll
                for (int e = 0; e < 16; e++) acc[e] = 0.0f;
#pragma unroll
                for (int c = 0; c < NC; c++)
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        acc[e] = fmaf(kd[c * 16 + e], qv[c * 16 + e], acc[e]);
                sc[o][i] = __fmul_rn(reduce16(acc), rs);
            }
        }
        __syncthreads();

        // ---- B: chunk max, p = exp(s - m), l = sum p
        for (int o = 0; o < nh; o++) {
            float m = -INFINITY;
            for (int i = tid; i < nt; i += 256) m = fmaxf(m, sc[o][i]);
            m = wave_max(m);
            if (lane == 0) wred[wv] = m;
            __syncthreads();
            m = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
            __syncthreads();
            float l = 0.0f;
            for (int i = tid; i < nt; i += 256) {
                const float p = expf(__fsub_rn(sc[o][i], m));
                sc[o][i] = p;
                l = __fadd_rn(l, p);
            }
            l = wave_sum(l);
            if (lane == 0) wred[wv] = l;
            __syncthreads();
            if (tid == 0) {
                mh[o] = m;
                lh[o] = __fadd_rn(__fadd_rn(wred[0], wred[1]),
                                  __fadd_rn(wred[2], wred[3]));
            }
            __syncthreads();
        }

        // ---- C: V accumulation
        const int lt = tid % LPT, slot = tid / LPT;
        const int grp = lt / 8, dj = lt % 8;
        const int dim_lo = 64 * grp + 4 * dj;
        for (int ob = 0; ob < nh; ob += 8) {
            const int nb = min(8, nh - ob);
            float acc[8][8];
#pragma unroll
            for (int o = 0; o < 8; o++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[o][e] = 0.0f;
            for (int i = slot; i < nt; i += SLOTS) {
                const int64_t gg =
                    (int64_t)kvh * g.gph + (int64_t)(t0 + i) * GPD + grp;
                const uint32_t word =
                    *reinterpret_cast<const uint32_t *>(V.w + gg * 32 + dj * 4);
                const float ss = V.s[gg], bb = V.b[gg];
                float v[8];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[e] = fmaf((float)((word >> (8 * e)) & 15u), ss, bb);
                    v[4 + e] = fmaf((float)((word >> (8 * e + 4)) & 15u), ss, bb);
                }
#pragma unroll
                for (int o = 0; o < 8; o++) {
                    if (o < nb) {
                        const float p = sc[ob + o][i];
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            acc[o][e] = fmaf(v[e], p, acc[o][e]);
                    }
                }
            }
            // ---- D: sum token slots, store partial
            // o is unrolled so acc stays in registers; nb is block-uniform,
            // so the barriers below are reached by every thread or by none.
#pragma unroll
            for (int o = 0; o < 8; o++) {
                if (o >= nb) break;
                float *r = red + slot * D;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    r[dim_lo + e] = acc[o][e];
                    r[dim_lo + 32 + e] = acc[o][4 + e];
                }
                __syncthreads();
                const int qh = kvh * qpk + hb + ob + o;
                float *dst =
                    part + (((int64_t)s * n_q + qh) * max_chunks + ch) * (D + 2);
                if (tid < D) {
                    float sum = red[tid];
                    for (int sl = 1; sl < SLOTS; sl++)
                        sum = __fadd_rn(sum, red[sl * D + tid]);
                    dst[2 + tid] = sum;
                }
                if (tid == 0) {
                    dst[0] = mh[ob + o];
                    dst[1] = lh[ob + o];
                }
                __syncthreads();
            }
        }
        __syncthreads();
    }
}

// One block per (sequence, q head); thread i handles output dim i.
template <int D>
__global__ __launch_bounds__(D) void combine_kernel(
    eakvd_batch bt, int n_q, int max_chunks, const float *__restrict__ part,
    float *__restrict__ out)
{
    const int qh = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    const int n_chunks = (bt.seq_len[s] + kChunk - 1) / kChunk;
    const float *p = part + ((int64_t)s * n_q + qh) * max_chunks * (D + 2);
    float M = 0.0f - 1000000.0f;
    for (int c = 0; c < n_chunks; c++) M = fmaxf(M, p[c * (D + 2)]);
    float l = 0.0f, o = 0.0f;
    for (int c = 0; c < n_chunks; c++) {
        const float *pc = p + c * (D + 2);
        const float f = expf(__fsub_rn(pc[0], M));
        l = fmaf(pc[1], f, l);
        o = fmaf(pc[2 + i], f, o);
    }
    out[((int64_t)s * n_q + qh) * D + i] = __fmul_rn(o, 1.0f / l);
}

int max_chunks_of(const eakvd_batch *b)
{
    int mx = 0;
    for (int i = 0; i < b->n_seq; i++)
        mx = b->seq_len[i] > mx ? b->seq_len[i] : mx;
    return (mx + kChunk - 1) / kChunk;
}

}  // namespace

extern "C" size_t eakvd_fused_work_bytes(const eakvd_geom *g,
                                         const eakvd_batch *b, int n_q)
{
    return (size_t)b->n_seq * n_q * max_chunks_of(b) * (g->head_dim + 2) *
           sizeof(float);
}

extern "C" int eakvd_fused(const eakvd_geom *g, const eakvd_batch *b,
                           int layer, const float *q, int n_q, int n_kv,
                           float *out, void *work, void *stream)
{
    const hipStream_t st = (hipStream_t)stream;
    const int mc = max_chunks_of(b);
    const int qpk = n_q / n_kv;
    const float rs = 1.0f / sqrtf((float)g->head_dim);
    float *part = (float *)work;
    if (mc > 0) {
        const dim3 grid((unsigned)mc, (unsigned)n_kv, (unsigned)b->n_seq);
        if (g->head_dim == 64)
            hipLaunchKernelGGL(fused_kernel<64>, grid, dim3(256), 0, st, *g,
                               *b, layer, q, n_q, qpk, mc, rs, part);
        else
            hipLaunchKernelGGL(fused_kernel<128>, grid, dim3(256), 0, st, *g,
                               *b, layer, q, n_q, qpk, mc, rs, part);
    }
    const dim3 cgrid((unsigned)n_q, (unsigned)b->n_seq);
    if (g->head_dim == 64)
        hipLaunchKernelGGL(combine_kernel<64>, cgrid, dim3(64), 0, st, *b, n_q,
                           mc, part, out);
    else
        hipLaunchKernelGGL(combine_kernel<128>, cgrid, dim3(128), 0, st, *b,
                           n_q, mc, part, out);
    return (int)hipGetLastError();
}
