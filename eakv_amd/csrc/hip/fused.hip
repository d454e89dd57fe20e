// fused.hip — fused decode attention on the packed cache: K-score, softmax
// and V-sum in one pass over K and V, for a batch of same-shape caches.
//
// Semantics: reference kernels/fused_attention.ea:190-373 (max with init
// -1e6, w = exp(s - max), sum, o = sum deq_v * w, out = o * (1/sum)),
// extended per q head to GQA and d=64.  Each q head h reads kv head
// h / (n_q/n_kv).
//
// Work split (flash-decoding): one block per (sequence, kv head, chunk).
// Chunk partials (m, l, o[D]) are merged in chunk order by the last block of
// each (sequence, kv head) to finish (an atomic count, no spinning), so one
// launch produces the output.
//
// Two block programs:
//
// mfma_kernel (groups of up to 4 q heads per kv head): 4 waves x 512 tokens.
//   K phase, 16 tokens per step: one v_mfma_i32_16x16x64_i8 per 64-dim group.
//     A = the q heads as 32-bit fixed point split into four signed bytes
//         (rows 4h+p: head h, byte p), B = the token's nibbles as int8 (the
//         packed bytes masked, no conversion).  The exact integer dots are
//         recombined in f64 and  score = (s0*dot0 + s1*dot1)/sqrt(d)
//         + (b0*sum q0 + b1*sum q1)/sqrt(d), rounded once to f32.
//   V phase, 8 (d=128) or 16 (d=64) tokens per step:
//     v_mfma_f32_4x4x1f32 outer products: block (group, token slot), rows =
//     4 heads with A = p*scale, columns = 4 dims with B = nibble; the bias
//     enters as sum p*bias per (head, group).  p = exp(score - chunk max).
//   Waves are merged in LDS, then chunks across blocks.
// valu_kernel (wider groups): one lane per token for K with the reference
//   arithmetic, then V by dims; same partial/merge scheme.
#include "common.h"

namespace {

// ------------------------------------------------------------------ MFMA

constexpr int kWaves = 4;
constexpr int kTW = 1024;               // tokens per wave per chunk
constexpr int kChunkM = kWaves * kTW;   // tokens per block
constexpr int kTT = 64;                 // tokens per tile (one pipeline stage)
constexpr float kTau = 8.0f;            // lazy-rescale headroom, e^8

__device__ __forceinline__ int sext8(int v) { return (int)(int8_t)(v & 0xff); }

// byte p (0 = most significant) of the balanced base-256 digits of z,
// |z| <= 2^30: z = d3*2^24 + d2*2^16 + d1*2^8 + d0, every digit in [-128,127]
__device__ __forceinline__ int digit_of(int z, int p)
{
    const int d0 = sext8(z);
    const int z1 = (z - d0) >> 8;
    const int d1 = sext8(z1);
    const int z2 = (z1 - d1) >> 8;
    const int d2 = sext8(z2);
    const int d3 = (z2 - d2) >> 8;
    return p == 0 ? d3 : (p == 1 ? d2 : (p == 2 ? d1 : d0));
}

// One lane's share of a kTT-token tile: the packed K bytes and K scale/bias
// of its MFMA sub-tiles, and the packed V bytes and V scale/bias of its
// V steps.
template <int D>
struct Tile {
    static constexpr int GPD = D / 64;
    static constexpr int NK = kTT / 16;          // K sub-tiles of 16 tokens
    static constexpr int TS = 16 / GPD;          // V token slots per step
    static constexpr int NV = kTT / TS;          // V steps
    uint2 kw[NK][GPD];
    float ks[NK][GPD], kb[NK][GPD];
    uint2 vw[NV];
    float vs[NV], vb[NV];
};

template <int D>
__device__ __forceinline__ void load_tile(Tile<D> &T, const Planes &K,
                                          const Planes &V, int64_t hbase,
                                          int t, int we, int tl, int qq,
                                          int ts, int grp, int x)
{
    constexpr int GPD = D / 64;
#pragma unroll
    for (int k = 0; k < Tile<D>::NK; k++) {
        const int tok = min(t + 16 * k + tl, we - 1);
        const int64_t gk = hbase + (int64_t)tok * GPD;
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
            T.kw[k][gg] = *reinterpret_cast<const uint2 *>(K.w + (gk + gg) * 32 + qq * 8);
        if (GPD == 2) {
            const float2 sv = *reinterpret_cast<const float2 *>(K.s + gk);
            const float2 bv = *reinterpret_cast<const float2 *>(K.b + gk);
            T.ks[k][0] = sv.x; T.ks[k][GPD - 1] = sv.y;
            T.kb[k][0] = bv.x; T.kb[k][GPD - 1] = bv.y;
        } else {
            T.ks[k][0] = K.s[gk];
            T.kb[k][0] = K.b[gk];
        }
    }
#pragma unroll
    for (int j = 0; j < Tile<D>::NV; j++) {
        const int tok = min(t + Tile<D>::TS * j + ts, we - 1);
        const int64_t gv = hbase + (int64_t)tok * GPD + grp;
        T.vw[j] = *reinterpret_cast<const uint2 *>(V.w + gv * 32 + x * 8);
        T.vs[j] = V.s[gv];
        T.vb[j] = V.b[gv];
    }
}

template <int D>
__global__ __launch_bounds__(256, 2) void mfma_kernel(
    eakvd_geom g, eakvd_batch bt, int layer, const float *__restrict__ q,
    int n_q, int qpk, int n_kv, int max_chunks, float rs,
    float *__restrict__ part, unsigned *__restrict__ cnt,
    float *__restrict__ out)
{
    constexpr int GPD = D / 64;
    constexpr int TS = Tile<D>::TS;
    constexpr int NK = Tile<D>::NK;
    constexpr int NV = Tile<D>::NV;
    __shared__ float p_lds[kWaves][2][4][kTT];
    __shared__ float o_lds[kWaves][4][D];
    __shared__ float m_lds[kWaves][4], l_lds[kWaves][4];
    __shared__ int last_flag;

    const int ch = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
    const int L = bt.seq_len[s];
    const int t0 = ch * kChunkM;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int G = qpk;                                  // 1..4
    float *outs = out + ((int64_t)s * n_q + (int64_t)kvh * qpk) * D;
    if (t0 >= L) {
        // an empty context gives 0 * (1/0) = NaN, as the reference
        if (L == 0 && ch == 0)
            for (int i = tid; i < G * D; i += 256) outs[i] = __builtin_nanf("");
        return;
    }
    const int wb = t0 + w * kTW;
    const int we = min(L, wb + kTW);
    const Planes K = planes_of(g, bt.base[s], layer, 0);
    const Planes V = planes_of(g, bt.base[s], layer, 1);
    const int64_t hbase = (int64_t)kvh * g.gph;
    const float *qs = q + ((int64_t)s * n_q + (int64_t)kvh * qpk) * D;

    // ---- q -> A operands.  Lane l: row i = l%16 (head ha = i/4, digit
    // pa = i%4), k-block qq = l/16; k-slot j of group gg holds dim
    // 64gg + 8qq + j (j < 8, low nibbles) or 64gg + 32 + 8qq + (j-8).
    const int ha = (l & 15) >> 2, pa = l & 3, qq = l >> 4;
    float qv[GPD][16];
    float amax = 0.0f;
    double qsum[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) {
        qsum[gg] = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int dim = 64 * gg + (j < 8 ? 8 * qq + j : 32 + 8 * qq + j - 8);
            const float v = ha < G ? qs[ha * D + dim] : 0.0f;
            qv[gg][j] = v;
            amax = fmaxf(amax, fabsf(v));
            qsum[gg] += (double)v;
        }
    }
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    int ex;
    frexpf(amax, &ex);            // amax < 2^ex, so |q * 2^(30-ex)| < 2^30
    const int esh = 30 - ex;
    v4i A[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) {
        uint32_t wd[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int z = (int)rintf(ldexpf(qv[gg][j], esh));
            wd[j >> 2] |= (uint32_t)(digit_of(z, pa) & 0xff) << (8 * (j & 3));
        }
        A[gg] = v4i{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
        qsum[gg] += __shfl_xor(qsum[gg], 16, 64);
        qsum[gg] += __shfl_xor(qsum[gg], 32, 64);
    }
    // constants of the head whose scores this lane receives (ho = l/16)
    const int ho = l >> 4, tl = l & 15;
    const int esh_o = __shfl(esh, 4 * ho, 64);
    const double cs = (double)rs * ldexp(1.0, -esh_o);
    double bq[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) bq[gg] = (double)rs * __shfl(qsum[gg], 4 * ho, 64);

    // V lane roles: l = grp*4*TS + ts*4 + x; block (grp, ts) = token slot ts
    // of group grp, x = head (A row) and dim column (B).  Column x of
    // accumulator m is dim 64grp + 32(m>=8) + 8x + m%8.
    const int x = l & 3, ts = (l >> 2) % TS, grp = (l >> 2) / TS;

    v4f acc[16];
#pragma unroll
    for (int m = 0; m < 16; m++) acc[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float bacc = 0.0f, lsum = 0.0f;
    float mrun[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};

    Tile<D> cur, nxt;
    if (wb < we) load_tile<D>(cur, K, V, hbase, wb, we, tl, qq, ts, grp, x);
    int buf = 0;
    for (int t = wb; t < we; t += kTT) {
        if (t + kTT < we) load_tile<D>(nxt, K, V, hbase, t + kTT, we, tl, qq, ts, grp, x);

        // ---- K: scores of this lane's head ho for tokens t + 16k + tl
        float sc[NK];
        float mt = -INFINITY;
#pragma unroll
        for (int k = 0; k < NK; k++) {
            double a = 0.0;
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) {
                const uint2 raw = cur.kw[k][gg];
                const v4i B = v4i{(int)(raw.x & 0x0F0F0F0Fu), (int)(raw.y & 0x0F0F0F0Fu),
                                  (int)((raw.x >> 4) & 0x0F0F0F0Fu),
                                  (int)((raw.y >> 4) & 0x0F0F0F0Fu)};
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[gg], B,
                                                                    v4i{0, 0, 0, 0}, 0, 0, 0);
                const double dot = ((double)d[0] * 16777216.0 + (double)d[1] * 65536.0) +
                                   ((double)d[2] * 256.0 + (double)d[3]);
                a += cs * ((double)cur.ks[k][gg] * dot) + (double)cur.kb[k][gg] * bq[gg];
            }
            sc[k] = t + 16 * k + tl < we ? (float)a : -INFINITY;
            mt = fmaxf(mt, sc[k]);
        }
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) mt = fmaxf(mt, __shfl_xor(mt, o, 64));

        // ---- lazy rescale: move the running max only when a head's tile max
        // exceeds it by more than kTau, so p = exp(s - mrun) stays <= e^kTau
        float mth[4];
        bool up = false;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            mth[r] = __shfl(mt, 16 * r, 64);
            up |= mth[r] > mrun[r] + kTau;
        }
        if (up) {
            float f[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float mn = mth[r] > mrun[r] + kTau ? mth[r] : mrun[r];
                f[r] = exp2f((mrun[r] - mn) * EAKV_LOG2E);
                mrun[r] = mn;
            }
#pragma unroll
            for (int m = 0; m < 16; m++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[m][r] *= f[r];
            const float fx = x == 0 ? f[0] : (x == 1 ? f[1] : (x == 2 ? f[2] : f[3]));
            bacc *= fx;
            lsum *= fx;
        }
        const float mho = ho == 0 ? mrun[0] : (ho == 1 ? mrun[1] : (ho == 2 ? mrun[2] : mrun[3]));
#pragma unroll
        for (int k = 0; k < NK; k++)
            p_lds[w][buf][ho][16 * k + tl] = exp2f((sc[k] - mho) * EAKV_LOG2E);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- V: p*scale rows x 4 dims columns per 4x4x1 block
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const float p = x < G ? p_lds[w][buf][x][TS * j + ts] : 0.0f;
            const float a = p * cur.vs[j];
            bacc = fmaf(p, cur.vb[j], bacc);
            lsum += grp == 0 ? p : 0.0f;
            const uint2 raw = cur.vw[j];
            const uint32_t lo0 = raw.x & 0x0F0F0F0Fu, lo1 = raw.y & 0x0F0F0F0Fu;
            const uint32_t hi0 = (raw.x >> 4) & 0x0F0F0F0Fu, hi1 = (raw.y >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int m = 0; m < 16; m++) {
                const uint32_t wd = m < 8 ? (m < 4 ? lo0 : lo1) : (m < 12 ? hi0 : hi1);
                const float nb = (float)((wd >> (8 * (m & 3))) & 0xffu);
                acc[m] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, nb, acc[m], 0, 0, 0);
            }
        }
        cur = nxt;
        buf ^= 1;
    }

    // sum the token slots (lane bits 2 .. 2+log2(TS)-1)
#pragma unroll
    for (int o = 4; o < 4 * TS; o <<= 1) {
#pragma unroll
        for (int m = 0; m < 16; m++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[m][r] += __shfl_xor(acc[m][r], o, 64);
        bacc += __shfl_xor(bacc, o, 64);
        lsum += __shfl_xor(lsum, o, 64);
    }
    float bsum[4];
#pragma unroll
    for (int r = 0; r < 4; r++) bsum[r] = __shfl(bacc, grp * 4 * TS + r, 64);
    if (ts == 0) {
#pragma unroll
        for (int m = 0; m < 16; m++) {
            const int dim = 64 * grp + (m >= 8 ? 32 : 0) + 8 * x + (m & 7);
#pragma unroll
            for (int r = 0; r < 4; r++) o_lds[w][r][dim] = acc[m][r] + bsum[r];
        }
    }
    if (l < 4) {
        m_lds[w][l] = mrun[l];
        l_lds[w][l] = lsum;
    }
    __syncthreads();

    // ---- merge the waves into this chunk's partial
    for (int i = tid; i < G * D; i += 256) {
        const int h = i / D, dim = i % D;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kWaves; ww++) M = fmaxf(M, m_lds[ww][h]);
        float lt = 0.0f, ot = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ww++) {
            const float f = exp2f((m_lds[ww][h] - M) * EAKV_LOG2E);
            lt = fmaf(l_lds[ww][h], f, lt);
            ot = fmaf(o_lds[ww][h][dim], f, ot);
        }
        float *dst = part + (((int64_t)s * n_q + kvh * qpk + h) * max_chunks + ch) * (D + 2);
        dst[2 + dim] = ot;
        if (dim == 0) {
            dst[0] = M;
            dst[1] = lt;
        }
    }

    // ---- the last chunk of this (sequence, kv head) merges all chunks
    __syncthreads();
    const int n_chunks = (L + kChunkM - 1) / kChunkM;
    unsigned *c = cnt + s * n_kv + kvh;
    if (tid == 0) {
        __threadfence();
        last_flag = atomicAdd(c, 1u) == (unsigned)(n_chunks - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    for (int i = tid; i < G * D; i += 256) {
        const int h = i / D, dim = i % D;
        const float *p = part + ((int64_t)s * n_q + kvh * qpk + h) * max_chunks * (D + 2);
        float M = 0.0f - 1000000.0f;
        for (int cc = 0; cc < n_chunks; cc++) M = fmaxf(M, p[cc * (D + 2)]);
        float lt = 0.0f, ot = 0.0f;
        for (int cc = 0; cc < n_chunks; cc++) {
            const float *pc = p + cc * (D + 2);
            const float f = expf(pc[0] - M);
            lt = fmaf(pc[1], f, lt);
            ot = fmaf(pc[2 + dim], f, ot);
        }
        outs[i] = ot * (1.0f / lt);
    }
    if (tid == 0) *c = 0u;
}

// ------------------------------------------------------------------ VALU

constexpr int kChunkV = 512;      // tokens per block
constexpr int kHeadsLds = 16;     // q heads per pass

template <int D>
__global__ __launch_bounds__(256) void valu_kernel(
    eakvd_geom g, eakvd_batch bt, int layer, const float *__restrict__ q,
    int n_q, int qpk, int max_chunks, float rs, float *__restrict__ part)
{
    constexpr int GPD = D / 64;
    constexpr int NC = D / 16;
    constexpr int LPT = D / 8;
    constexpr int SLOTS = 256 / LPT;
    __shared__ float sc[kHeadsLds][kChunkV];
    __shared__ float red[SLOTS * D];
    __shared__ float wred[4];
    __shared__ float mh[kHeadsLds], lh[kHeadsLds];

    const int ch = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
    const int L = bt.seq_len[s];
    const int t0 = ch * kChunkV;
    if (t0 >= L) return;
    const int nt = min(kChunkV, L - t0);
    const Planes K = planes_of(g, bt.base[s], layer, 0);
    const Planes V = planes_of(g, bt.base[s], layer, 1);
    const float *qs = q + (int64_t)s * n_q * D;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;

    for (int hb = 0; hb < qpk; hb += kHeadsLds) {
        const int nh = min(kHeadsLds, qpk - hb);

        // K: one lane per token, reference arithmetic
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
                float a[16];
#pragma unroll
                for (int e = 0; e < 16; e++) a[e] = 0.0f;
#pragma unroll
                for (int c = 0; c < NC; c++)
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        a[e] = fmaf(kd[c * 16 + e], qv[c * 16 + e], a[e]);
                sc[o][i] = __fmul_rn(reduce16(a), rs);
            }
        }
        __syncthreads();

        // chunk max, p = exp(s - m), l = sum p
        for (int o = 0; o < nh; o++) {
            float m = -INFINITY;
            for (int i = tid; i < nt; i += 256) m = fmaxf(m, sc[o][i]);
            m = wave_max(m);
            if (lane == 0) wred[wv] = m;
            __syncthreads();
            m = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
            __syncthreads();
            float lsum = 0.0f;
            for (int i = tid; i < nt; i += 256) {
                const float p = expf(__fsub_rn(sc[o][i], m));
                sc[o][i] = p;
                lsum = __fadd_rn(lsum, p);
            }
            lsum = wave_sum(lsum);
            if (lane == 0) wred[wv] = lsum;
            __syncthreads();
            if (tid == 0) {
                mh[o] = m;
                lh[o] = __fadd_rn(__fadd_rn(wred[0], wred[1]),
                                  __fadd_rn(wred[2], wred[3]));
            }
            __syncthreads();
        }

        // V: a lane owns one packed dword (8 dims) of a token
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
                        for (int e = 0; e < 8; e++) acc[o][e] = fmaf(v[e], p, acc[o][e]);
                    }
                }
            }
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
                float *dst = part + (((int64_t)s * n_q + qh) * max_chunks + ch) * (D + 2);
                if (tid < D) {
                    float sum = red[tid];
                    for (int sl = 1; sl < SLOTS; sl++) sum = __fadd_rn(sum, red[sl * D + tid]);
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

// One block per (sequence, q head): merge the VALU path's chunks.
template <int D>
__global__ __launch_bounds__(D) void combine_kernel(
    eakvd_batch bt, int n_q, int max_chunks, const float *__restrict__ part,
    float *__restrict__ out)
{
    const int qh = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    const int n_chunks = (bt.seq_len[s] + kChunkV - 1) / kChunkV;
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

int max_len(const eakvd_batch *b)
{
    int mx = 0;
    for (int i = 0; i < b->n_seq; i++) mx = b->seq_len[i] > mx ? b->seq_len[i] : mx;
    return mx;
}

}  // namespace

extern "C" size_t eakvd_fused_work_bytes(const eakvd_geom *g,
                                         const eakvd_batch *b, int n_q)
{
    // sized for the finer (VALU) chunking, which covers both programs
    const int mc = (max_len(b) + kChunkV - 1) / kChunkV;
    return (size_t)b->n_seq * n_q * mc * (g->head_dim + 2) * sizeof(float);
}

extern "C" int eakvd_fused(const eakvd_geom *g, const eakvd_batch *b,
                           int layer, const float *q, int n_q, int n_kv,
                           float *out, void *work, unsigned *counters,
                           void *stream)
{
    const hipStream_t st = (hipStream_t)stream;
    const int qpk = n_q / n_kv;
    const float rs = 1.0f / sqrtf((float)g->head_dim);
    float *part = (float *)work;
    const int ml = max_len(b);
    if (qpk <= 4) {
        const int mc = ml > 0 ? (ml + kChunkM - 1) / kChunkM : 1;
        const dim3 grid((unsigned)mc, (unsigned)n_kv, (unsigned)b->n_seq);
        if (g->head_dim == 64)
            hipLaunchKernelGGL(mfma_kernel<64>, grid, dim3(256), 0, st, *g, *b, layer,
                               q, n_q, qpk, n_kv, mc, rs, part, counters, out);
        else
            hipLaunchKernelGGL(mfma_kernel<128>, grid, dim3(256), 0, st, *g, *b, layer,
                               q, n_q, qpk, n_kv, mc, rs, part, counters, out);
        return (int)hipGetLastError();
    }
    const int mc = (ml + kChunkV - 1) / kChunkV;
    if (mc > 0) {
        const dim3 grid((unsigned)mc, (unsigned)n_kv, (unsigned)b->n_seq);
        if (g->head_dim == 64)
            hipLaunchKernelGGL(valu_kernel<64>, grid, dim3(256), 0, st, *g, *b,
                               layer, q, n_q, qpk, mc, rs, part);
        else
            hipLaunchKernelGGL(valu_kernel<128>, grid, dim3(256), 0, st, *g, *b,
                               layer, q, n_q, qpk, mc, rs, part);
    }
    const dim3 cgrid((unsigned)n_q, (unsigned)b->n_seq);
    if (g->head_dim == 64)
        hipLaunchKernelGGL(combine_kernel<64>, cgrid, dim3(64), 0, st, *b, n_q, mc,
                           part, out);
    else
        hipLaunchKernelGGL(combine_kernel<128>, cgrid, dim3(128), 0, st, *b, n_q,
                           mc, part, out);
    return (int)hipGetLastError();
}
