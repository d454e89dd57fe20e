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
// mfma_kernel (up to 4 q heads per kv head): 4 waves x 1024 tokens per block.
//   Each wave walks its tokens in 32-token tiles, two tiles in flight
//   (ping-pong registers, buffer loads issued one tile ahead).  Per tile:
//   K, 16 tokens per v_mfma_i32_16x16x64_i8 and 64-dim group:
//     A = the q heads as 32-bit fixed point split into four signed bytes
//         (rows 4h+p: head h, byte p), B = the token's nibbles as int8 (the
//         packed bytes masked, no conversion).  The exact integer dot of each
//         byte row is recombined in f32 with weights 2^24, 2^16, 2^8, 1
//         (times 2^-e/sqrt(d)), and score = s*dot + b*sum(q)/sqrt(d).
//   Online softmax with a lazy running max: the running max of a head moves
//     only when a tile max exceeds it by more than kTau, so every
//     p = exp(score - max) stays <= e^kTau and the accumulators are rescaled
//     rarely.
//   V, v_mfma_f32_4x4x1f32 outer products: block (group, token slot), rows =
//     4 heads with A = p*scale, columns = 4 dims with B = nibble as float;
//     the bias enters as sum p*bias per (head, group).  p moves from the score
//     layout (lane = head x token) to the V layout through LDS.
//   Waves are merged in LDS, then chunks across blocks.
// valu_kernel (wider groups): one lane per token for K with the reference
//   arithmetic, then V by dims; same partial/merge scheme.
#include "common.h"

namespace {

// ------------------------------------------------------------------ MFMA

constexpr int kWaves = 4;
constexpr int kTW = 1024;               // tokens per wave per chunk
constexpr int kChunkM = kWaves * kTW;   // tokens per block
#ifndef EAKV_FUSED_TT
#define EAKV_FUSED_TT 32
#endif
constexpr int kTT = EAKV_FUSED_TT;      // tokens per tile (one pipeline stage)
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

// Buffer resources of the six planes (scalar registers) and this lane's byte
// offsets at the wave's first token.  A tile is read with buffer loads:
// resource + lane offset + uniform tile offset + immediate, so a tile costs
// no per-lane address arithmetic.  Reads past a plane's end return 0.
struct LaneOffs {
    __amdgpu_buffer_rsrc_t kw, vw, ks, kb, vs, vb;
    uint32_t kwo, kso, vwo, vso;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const void *p, int64_t bytes)
{
    // dword3 0x00020000: raw (untyped) 32-bit buffer on gfx9-family parts
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint2 ldb64(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, (int)so, 0);
    return uint2{v[0], v[1]};
}

__device__ __forceinline__ float ldf(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0));
}

// The tile at token offset dt of the wave.  A tile can run up to kTT - 1
// tokens past the wave's last token; those reads stay inside the plane (or
// return 0 beyond it) and their scores are masked to -inf, so their weight is
// exactly 0.
template <int D>
__device__ __forceinline__ void load_tile(Tile<D> &T, const LaneOffs &P, int dt)
{
    constexpr int GPD = D / 64;
    constexpr int TS = Tile<D>::TS;
    // dt is the same in every lane; readfirstlane makes that visible, so the
    // tile offsets go to the scalar soffset operand
    const uint32_t du = (uint32_t)__builtin_amdgcn_readfirstlane(dt);
    const uint32_t ws = du * GPD * 32, ss = du * GPD * 4;
#pragma unroll
    for (int k = 0; k < Tile<D>::NK; k++) {
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
            T.kw[k][gg] = ldb64(P.kw, P.kwo + (16 * k * GPD + gg) * 32, ws);
        if (GPD == 2) {
            const uint2 sv = ldb64(P.ks, P.kso + 16 * k * GPD * 4, ss);
            const uint2 bv = ldb64(P.kb, P.kso + 16 * k * GPD * 4, ss);
            T.ks[k][0] = __uint_as_float(sv.x); T.ks[k][GPD - 1] = __uint_as_float(sv.y);
            T.kb[k][0] = __uint_as_float(bv.x); T.kb[k][GPD - 1] = __uint_as_float(bv.y);
        } else {
            T.ks[k][0] = ldf(P.ks, P.kso + 16 * k * 4, ss);
            T.kb[k][0] = ldf(P.kb, P.kso + 16 * k * 4, ss);
        }
    }
#pragma unroll
    for (int j = 0; j < Tile<D>::NV; j++) {
        T.vw[j] = ldb64(P.vw, P.vwo + TS * j * GPD * 32, ws);
        T.vs[j] = ldf(P.vs, P.vso + TS * j * GPD * 4, ss);
        T.vb[j] = ldf(P.vb, P.vso + TS * j * GPD * 4, ss);
    }
}

// State carried across the tiles of one wave.  The running maxima are
// wave-uniform scalars.
template <int D>
struct WaveState {
    v4f acc[16];
    float bacc, lsum;
    float m0, m1, m2, m3;
};

__device__ __forceinline__ float sel4(int i, float a, float b, float c, float d)
{
    float r = a;
    r = i == 1 ? b : r;
    r = i == 2 ? c : r;
    r = i == 3 ? d : r;
    return r;
}

// x & 0x0F0F0F0F hidden from the optimizer, so that extracting byte k of the
// result stays one v_cvt_f32_ubyte<k>
__device__ __forceinline__ uint32_t nib_lo(uint32_t x)
{
    uint32_t r;
    asm volatile("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(x));
    return r;
}

__device__ __forceinline__ uint32_t nib_hi(uint32_t x)
{
    uint32_t r;
    asm volatile("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(x >> 4));
    return r;
}

__device__ __forceinline__ float row_max16(float v)
{
    // max over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1)
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false)));
    return v;
}

template <int D>
__device__ __forceinline__ void process_tile(
    WaveState<D> &S, const Tile<D> &T, int dt, int n_tok, const v4i *A,
    const float *wsc, const float *bq, float (*pl)[kTT], int G, int ho,
    int tl, int ts, int x)
{
    constexpr int GPD = D / 64;
    constexpr int TS = Tile<D>::TS;
    constexpr int NK = Tile<D>::NK;
    constexpr int NV = Tile<D>::NV;

    // ---- K: per sub-tile, the digit-row dots of both groups, then their
    // recombination: the exact integer dot of each digit row times its
    // weight (wsc holds 2^24, 2^16, 2^8, 1 times 2^-e/sqrt(d)), in f32.
    float sc[NK];
    float mt = -INFINITY;
#pragma unroll
    for (int k = 0; k < NK; k++) {
        v4i d[GPD];
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) {
            const uint2 raw = T.kw[k][gg];
            const v4i B = v4i{(int)nib_lo(raw.x), (int)nib_lo(raw.y), (int)nib_hi(raw.x),
                              (int)nib_hi(raw.y)};
            d[gg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[gg], B, v4i{0, 0, 0, 0}, 0, 0, 0);
        }
        float a = 0.0f;
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) {
            float u = (float)d[gg][3] * wsc[3];
            u = fmaf((float)d[gg][2], wsc[2], u);
            u = fmaf((float)d[gg][1], wsc[1], u);
            u = fmaf((float)d[gg][0], wsc[0], u);
            a = fmaf(T.ks[k][gg], u, fmaf(T.kb[k][gg], bq[gg], a));
        }
        sc[k] = dt + 16 * k + tl < n_tok ? a : -INFINITY;
        mt = fmaxf(mt, sc[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    mt = row_max16(mt);

    // ---- lazy rescale: move the running max only when a head's tile max
    // exceeds it by more than kTau, so p = exp(s - mrun) stays <= e^kTau
    const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mt), 0));
    const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mt), 16));
    const float t2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mt), 32));
    const float t3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mt), 48));
    const bool u0 = t0 > S.m0 + kTau, u1 = t1 > S.m1 + kTau;
    const bool u2 = t2 > S.m2 + kTau, u3 = t3 > S.m3 + kTau;
    if (u0 || u1 || u2 || u3) {
        const float n0 = u0 ? t0 : S.m0, n1 = u1 ? t1 : S.m1;
        const float n2 = u2 ? t2 : S.m2, n3 = u3 ? t3 : S.m3;
        const float f0 = exp2f((S.m0 - n0) * EAKV_LOG2E), f1 = exp2f((S.m1 - n1) * EAKV_LOG2E);
        const float f2 = exp2f((S.m2 - n2) * EAKV_LOG2E), f3 = exp2f((S.m3 - n3) * EAKV_LOG2E);
        S.m0 = n0; S.m1 = n1; S.m2 = n2; S.m3 = n3;
#pragma unroll
        for (int m = 0; m < 16; m++) {
            S.acc[m][0] *= f0;
            S.acc[m][1] *= f1;
            S.acc[m][2] *= f2;
            S.acc[m][3] *= f3;
        }
        S.bacc *= sel4(x, f0, f1, f2, f3);
        S.lsum *= sel4(ho, f0, f1, f2, f3);
    }
    // p in the score layout (head ho, token 16k + tl); heads >= G get 0
    const float mho = sel4(ho, S.m0, S.m1, S.m2, S.m3);
#pragma unroll
    for (int k = 0; k < NK; k++) {
        const float p = ho < G ? exp2f((sc[k] - mho) * EAKV_LOG2E) : 0.0f;
        S.lsum += p;
        pl[ho][16 * k + tl] = p;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- V: rows p*scale (4 heads) x columns 4 dims per 4x4x1 block
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const float p = pl[x][TS * j + ts];
        const float a = p * T.vs[j];
        S.bacc = fmaf(p, T.vb[j], S.bacc);
        const uint2 raw = T.vw[j];
        // low nibbles (accumulators 0-7), then high nibbles (8-15)
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const uint32_t w0 = half ? nib_hi(raw.x) : nib_lo(raw.x);
            const uint32_t w1 = half ? nib_hi(raw.y) : nib_lo(raw.y);
            float nb[8];
#pragma unroll
            for (int e = 0; e < 8; e++)
                nb[e] = (float)(((e < 4 ? w0 : w1) >> (8 * (e & 3))) & 0xffu);
#pragma unroll
            for (int e = 0; e < 8; e++)
                S.acc[8 * half + e] =
                    __builtin_amdgcn_mfma_f32_4x4x1f32(a, nb[e], S.acc[8 * half + e], 0, 0, 0);
        }
        // keep the steps apart: hoisting later steps' conversions above these
        // MFMAs only raises register pressure
        __builtin_amdgcn_sched_barrier(0);
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
    __shared__ float p_lds[kWaves][2][4][kTT];
    __shared__ float o_lds[kWaves][4][D];
    __shared__ float m_lds[kWaves][4], l_lds[kWaves][4];
    __shared__ int last_flag;

    const int ch = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
    const int L = bt.seq_len[s];
    const int t0 = ch * kChunkM;
    // the wave index is wave-uniform: say so, so that every per-wave
    // quantity (token range, tile offsets) stays in scalar registers
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = qpk;                                  // 1..4
    float *outs = out + ((int64_t)s * n_q + (int64_t)kvh * qpk) * D;
    if (t0 >= L) {
        // an empty context gives 0 * (1/0) = NaN, as the reference
        if (L == 0 && ch == 0)
            for (int i = tid; i < G * D; i += 256) outs[i] = __builtin_nanf("");
        return;
    }
    const int wb = t0 + w * kTW;
    const int n_tok = min(L, wb + kTW) - wb;            // may be <= 0
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
    float qsum[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) {
        double sum = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int dim = 64 * gg + (j < 8 ? 8 * qq + j : 32 + 8 * qq + j - 8);
            const float v = ha < G ? qs[ha * D + dim] : 0.0f;
            qv[gg][j] = v;
            amax = fmaxf(amax, fabsf(v));
            sum += (double)v;
        }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        qsum[gg] = (float)sum;
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
    }
    // constants of the head whose scores this lane receives (ho = l/16)
    const int ho = l >> 4, tl = l & 15;
    const int esh_o = __shfl(esh, 4 * ho, 64);
    float wsc[4];
#pragma unroll
    for (int p = 0; p < 4; p++) wsc[p] = ldexpf(rs, 24 - 8 * p - esh_o);
    float bq[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) bq[gg] = rs * __shfl(qsum[gg], 4 * ho, 64);

    // V lane roles: l = grp*4*TS + ts*4 + x; block (grp, ts) = token slot ts
    // of group grp, x = head (A row) and dim column (B).  Column x of
    // accumulator m is dim 64grp + 32(m>=8) + 8x + m%8.
    const int x = l & 3, ts = (l >> 2) % TS, grp = (l >> 2) / TS;

    LaneOffs P;
    {
        const int64_t wbytes = g.max_groups * 32, sbytes = g.max_groups * 4;
        P.kw = plane_rsrc(K.w, wbytes); P.ks = plane_rsrc(K.s, sbytes);
        P.kb = plane_rsrc(K.b, sbytes); P.vw = plane_rsrc(V.w, wbytes);
        P.vs = plane_rsrc(V.s, sbytes); P.vb = plane_rsrc(V.b, sbytes);
        const int64_t gk = hbase + (int64_t)(wb + tl) * GPD;
        const int64_t gv = hbase + (int64_t)(wb + ts) * GPD + grp;
        P.kwo = (uint32_t)(gk * 32 + qq * 8);
        P.kso = (uint32_t)(gk * 4);
        P.vwo = (uint32_t)(gv * 32 + x * 8);
        P.vso = (uint32_t)(gv * 4);
    }

    WaveState<D> S;
#pragma unroll
    for (int m = 0; m < 16; m++) S.acc[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    S.bacc = 0.0f;
    S.lsum = 0.0f;
    S.m0 = S.m1 = S.m2 = S.m3 = -INFINITY;

    // two tiles in flight per wave, ping-pong registers.  The barrier keeps
    // the scheduler from sinking a prefetch down to its use.
    Tile<D> ta, tb;
    auto load = [&](Tile<D> &T, int dt) {
        load_tile<D>(T, P, dt);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto proc = [&](const Tile<D> &T, int dt, float (*pl)[kTT]) {
        process_tile<D>(S, T, dt, n_tok, A, wsc, bq, pl, G, ho, tl, ts, x);
    };
    // Prefetches are unconditional so that every wait in the loop counts the
    // same number of younger loads; past the end they re-read the last tile.
    if (n_tok > 0) {
        const int last = ((n_tok - 1) / kTT) * kTT;
        load(ta, 0);
        for (int dt = 0; dt < n_tok; dt += 2 * kTT) {
            load(tb, min(dt + kTT, last));
            proc(ta, dt, p_lds[w][0]);
            if (dt + kTT >= n_tok) break;
            load(ta, min(dt + 2 * kTT, last));
            proc(tb, dt + kTT, p_lds[w][1]);
        }
    }

    // sum the token slots (lane bits 2 .. 2+log2(TS)-1)
#pragma unroll
    for (int o = 4; o < 4 * TS; o <<= 1) {
#pragma unroll
        for (int m = 0; m < 16; m++)
#pragma unroll
            for (int r = 0; r < 4; r++) S.acc[m][r] += __shfl_xor(S.acc[m][r], o, 64);
        S.bacc += __shfl_xor(S.bacc, o, 64);
    }
    // lsum lives in the score layout: head ho, summed over its 16 token lanes
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) S.lsum += __shfl_xor(S.lsum, o, 64);
    float bsum[4];
#pragma unroll
    for (int r = 0; r < 4; r++) bsum[r] = __shfl(S.bacc, grp * 4 * TS + r, 64);
    if (ts == 0) {
#pragma unroll
        for (int m = 0; m < 16; m++) {
            const int dim = 64 * grp + (m >= 8 ? 32 : 0) + 8 * x + (m & 7);
#pragma unroll
            for (int r = 0; r < 4; r++) o_lds[w][r][dim] = S.acc[m][r] + bsum[r];
        }
    }
    if ((l & 15) == 0) {
        m_lds[w][l >> 4] = sel4(l >> 4, S.m0, S.m1, S.m2, S.m3);
        l_lds[w][l >> 4] = S.lsum;
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
    // the MFMA program addresses a plane with 32-bit buffer offsets
    const bool small_planes = g->max_groups * 32 <= (int64_t)0x7fffffff;
    if (qpk <= 4 && small_planes) {
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
