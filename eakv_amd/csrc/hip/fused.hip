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
//   Each wave walks its tokens in 32-token tiles, two pipeline stages in
//   flight (ping-pong registers, buffer loads issued one stage ahead):
//   K, 16 tokens per v_mfma_i32_16x16x64_i8 and 64-dim group:
//     A = the q heads as 32-bit fixed point split into four signed bytes
//         (rows 4h+p: head h, byte p), B = the token's nibbles as int8 (the
//         packed bytes masked, no conversion).  The exact integer dot of each
//         byte row is recombined in f32 with weights 2^24, 2^16, 2^8, 1
//         (times 2^-e/sqrt(d)), and score = s*dot + b*sum(q)/sqrt(d).
//   Online softmax in the log2 domain with a lazy running max: the running
//     max of a head moves only when a tile max exceeds it by more than kTau,
//     so every p = 2^(score - max) stays <= 2^kTau and the accumulators are
//     rescaled rarely.
//   The pipeline runs V(i) beside K(i+1): the K loads of a tile are issued
//     one tile ahead of its V loads.
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
constexpr int kTT = 32;                 // tokens per tile (one pipeline stage), 2^k >= 32
#ifndef EAKV_FUSED_BLOCKS_PER_CU
#define EAKV_FUSED_BLOCKS_PER_CU 3
#endif
constexpr int kBlocksPerCU = EAKV_FUSED_BLOCKS_PER_CU;   // occupancy the register budget is set for
constexpr float kTau = 8.0f;            // lazy-rescale headroom, 2^8 (log2 units)

// Tile geometry.  K: 16-token sub-tiles (one int8 MFMA per 64-dim group).
// V: a token's packed bytes of one kv head are DW = D/8 dwords; in the V
// layout lane l holds dword u = l % DW of token slot T = l / DW, so one V
// step covers TSV = 64/DW tokens (4 at d=128, 8 at d=64).
template <int D>
struct Geo {
    static constexpr int GPD = D / 64;
    static constexpr int DW = D / 8;
    static constexpr int TSV = 64 / DW;
    static constexpr int NV = kTT / TSV;       // V steps per tile
    static constexpr int NK = kTT / 16;        // K sub-tiles per tile
};

// One lane's share of a pipeline stage in registers: the K bytes of one tile
// (MFMA B layout) and the packed V dwords of the tile before it (V layout).
// The stage's K and V scales and biases (of the K tile) go to an LDS slot of
// the wave (see load_scales).
template <int D>
struct Stage {
    static constexpr int GPD = Geo<D>::GPD, NK = Geo<D>::NK, NV = Geo<D>::NV;
    uint2 kw[NK][GPD];
    uint32_t vw[NV];
};

// The scales and biases of one tile for this lane's tokens (score layout:
// token 16k + tl), read from the LDS slot.
template <int D>
struct Scales {
    float ks[Geo<D>::NK][Geo<D>::GPD], kb[Geo<D>::NK][Geo<D>::GPD];
    float vs[Geo<D>::NK][Geo<D>::GPD], vb[Geo<D>::NK][Geo<D>::GPD];
};

// floats of one LDS scale slot: planes ks, kb, vs, vb of a tile
template <int D>
constexpr int kSlot = 4 * kTT * (D / 64);

// Buffer resources of the six planes (scalar registers) and this lane's byte
// offsets at the wave's first token.  A tile is read with buffer loads:
// resource + lane offset + uniform tile offset + immediate, so a tile costs
// no per-lane address arithmetic.  Reads past a plane's end return 0.
struct LaneOffs {
    __amdgpu_buffer_rsrc_t kw, vw, layer;
    uint32_t kwo, vwo, sco;
    uint32_t plane[4];      // byte offsets of ks, kb, vs, vb from the K block
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

__device__ __forceinline__ uint32_t ldb32(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, (int)so, 0);
}

// Loads of the tile at token offset dt of the wave.  A tile can run up to
// kTT - 1 tokens past the wave's last token; those reads stay inside the
// plane (or return 0 beyond it), their scores are masked to -inf and their
// weight is exactly 0.  dt is the same in every lane; readfirstlane makes
// that visible, so the tile offset goes to the scalar soffset operand.
template <int D>
__device__ __forceinline__ void load_k(Stage<D> &T, const LaneOffs &P, int dt)
{
    constexpr int GPD = D / 64;
    const uint32_t du = (uint32_t)__builtin_amdgcn_readfirstlane(dt);
    const uint32_t ws = du * GPD * 32;
#pragma unroll
    for (int k = 0; k < Geo<D>::NK; k++)
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
            T.kw[k][gg] = ldb64(P.kw, P.kwo + (16 * k * GPD + gg) * 32, ws);
}

// The K and V scales and biases of the tile at dt, straight into the wave's
// LDS slot (buffer loads to LDS: lane m's dword lands at slot + 4m of the
// instruction's destination).  Slot layout: plane p in {ks, kb, vs, vb} at
// p * kTT * GPD floats, then token-major, group-minor, as in the planes.
// d=128: one instruction per plane (64 dwords = 32 tokens x 2 groups);
// d=64: two planes per instruction (lanes 32-63 take the second).
template <int D>
__device__ __forceinline__ void load_scales(float *slot, const LaneOffs &P, int dt)
{
    constexpr int GPD = D / 64;
    const uint32_t du = (uint32_t)__builtin_amdgcn_readfirstlane(dt);
    const uint32_t ss = du * GPD * 4;
    typedef __attribute__((address_space(3))) void *lds_ptr;
#pragma unroll
    for (int i = 0; i < 4 / (3 - GPD); i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            P.layer, (lds_ptr)(slot + 64 * i), 4, (int)P.sco,
            (int)(P.plane[(3 - GPD) * i] + ss), 0, 0);
}

// Loads per stage: DMA scale loads, then K bytes, then V dwords (fixed by
// sched barriers).  The compiler does not order LDS reads after buffer loads
// to LDS, so the reads of a slot are preceded by an explicit wait for every
// load older than the last kYounger<D> ones: the slot's stage issued its DMA
// loads first, then kSB<D> register loads, and the next stage (kStage<D>
// loads) has been issued since.
template <int D>
constexpr int kDma = 4 / (3 - D / 64);
template <int D>
constexpr int kSB = Geo<D>::NK * (D / 64) + Geo<D>::NV;
template <int D>
constexpr int kStage = kDma<D> + kSB<D>;

// s_waitcnt vmcnt(n), no wait on the other counters (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int D>
__device__ __forceinline__ void read_scales(const float *slot, int tl, Scales<D> &C)
{
    constexpr int GPD = D / 64, PS = kTT * GPD;
#pragma unroll
    for (int k = 0; k < Geo<D>::NK; k++) {
        const int e = (16 * k + tl) * GPD;
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) {
            C.ks[k][gg] = slot[0 * PS + e + gg];
            C.kb[k][gg] = slot[1 * PS + e + gg];
            C.vs[k][gg] = slot[2 * PS + e + gg];
            C.vb[k][gg] = slot[3 * PS + e + gg];
        }
    }
}

template <int D>
__device__ __forceinline__ void load_v(Stage<D> &T, const LaneOffs &P, int dt)
{
    constexpr int GPD = D / 64;
    const uint32_t du = (uint32_t)__builtin_amdgcn_readfirstlane(dt);
    const uint32_t ws = du * GPD * 32;
#pragma unroll
    for (int j = 0; j < Geo<D>::NV; j++)
        T.vw[j] = ldb32(P.vw, P.vwo + Geo<D>::TSV * j * GPD * 32, ws);
}

// State carried across the tiles of one wave.  acc (V layout): lane (T, u)
// holds, for nibble e of its dword, the partial output of heads r = 0..3.
// Score layout (lane = head ho x token tl): the running max m of head ho,
// the softmax denominator lsum and the bias sums sum p*bias per group.
template <int D>
struct WaveState {
    v4f acc[8];
    float bacc[D / 64];
    float lsum, m;
};

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

// p * v with 0 * anything = 0 (v_mul_legacy_f32; otherwise IEEE rounding).
// A tile can cover tokens past the sequence end whose p is 0 but whose stale
// scale or bias may be non-finite; their products must stay 0.
__device__ __forceinline__ float mul_zero(float p, float v)
{
    float r;
    asm("v_mul_legacy_f32 %0, %1, %2" : "=v"(r) : "v"(p), "v"(v));
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

// Slot of a = p*scale for (group g, head h, token tau of a tile) in a wave's
// a buffer (GPD x 4*kTT floats).  Written in the score layout, read in the V
// layout; the swizzle (bits below 32 only) keeps both free of LDS bank
// conflicts.
__device__ __forceinline__ int a_slot(int g, int h, int tau)
{
    return g * 4 * kTT + ((tau * 4 + h) ^ (g * 16) ^ (((tau >> 3) & 1) * 2));
}

// K of one tile: per 16-token sub-tile, the digit-row dots of each group on
// the int8 matrix core (k_mfma), then their recombination (k_recomb).  The
// four digit rows r (weights 2^24, 2^16, 2^8, 1) are paired exactly in int32,
// H = 256*d0 + d1 and Lo = 256*d2 + d3 (|H|, |Lo| < 2^25), and
// u = H*wh + Lo*wl with wh = 2^16*wl, wl = 2^-e*log2(e)/sqrt(d).  Scores are
// in the log2 domain: sc = log2(e) * (q.k)/sqrt(d); masked tokens get -inf.
template <int D>
__device__ __forceinline__ void k_mfma(const Stage<D> &T, const v4i *A,
                                       v4i (*dk)[D / 64])
{
#pragma unroll
    for (int k = 0; k < Geo<D>::NK; k++)
#pragma unroll
        for (int gg = 0; gg < D / 64; gg++) {
            const uint2 raw = T.kw[k][gg];
            const v4i B = v4i{(int)nib_lo(raw.x), (int)nib_lo(raw.y), (int)nib_hi(raw.x),
                              (int)nib_hi(raw.y)};
            dk[k][gg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[gg], B, v4i{0, 0, 0, 0},
                                                               0, 0, 0);
        }
}

template <int D>
__device__ __forceinline__ float k_recomb(const Scales<D> &T, const v4i *d, int k,
                                          int dt, int L, float wh, float wl,
                                          const float *bq, int tl)
{
    float a = 0.0f;
#pragma unroll
    for (int gg = 0; gg < D / 64; gg++) {
        const int hi = d[gg][0] * 256 + d[gg][1];
        const int lo = d[gg][2] * 256 + d[gg][3];
        const float u = fmaf((float)hi, wh, (float)lo * wl);
        a = fmaf(T.ks[k][gg], u, fmaf(T.kb[k][gg], bq[gg], a));
    }
    return dt + 16 * k + tl < L ? a : -INFINITY;
}

// Softmax weights of sub-tile k with the running max m of this lane's head:
// p = 2^(sc - m) (0 for heads >= G), a = p*scale per group into the a
// buffer, p*bias per group into bi.  Returns p.
template <int D>
__device__ __forceinline__ float p_write(const Scales<D> &T, int k, float sc, float m,
                                         bool live, float *abuf, int ho, int tl,
                                         float *bi)
{
    const float p = live ? __builtin_amdgcn_exp2f(sc - m) : 0.0f;
#pragma unroll
    for (int gg = 0; gg < D / 64; gg++) {
        abuf[a_slot(gg, ho, 16 * k + tl)] = mul_zero(p, T.vs[k][gg]);
        bi[gg] += mul_zero(p, T.vb[k][gg]);
    }
    return p;
}

// The tile's softmax bookkeeping once the previous tile's V is accumulated.
// Lazy rescale: a head's running max moves only when the tile's max exceeds
// it by more than kTau (so p <= 2^kTau).  The common case (need false in
// every lane) only adds the tile's sums; otherwise (rare: the first tile,
// a new larger score) the moved maxima are set, the accumulators scaled by
// 2^(old - new) and the tile's weights rewritten.
template <int D>
__device__ __forceinline__ void softmax_tail(
    WaveState<D> &S, const Scales<D> &T, const float *sc, bool need, float psum,
    float *bi, bool live, float *abuf, int ho, int tl)
{
    constexpr int NK = Geo<D>::NK, GPD = D / 64;
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
        float mt = sc[0];
#pragma unroll
        for (int k = 1; k < NK; k++) mt = fmaxf(mt, sc[k]);
        mt = row_max16(mt);
        const float mn = live && mt > S.m + kTau ? mt : S.m;
        const float f = live ? __builtin_amdgcn_exp2f(S.m - mn) : 1.0f;
        S.m = mn;
        psum = 0.0f;
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) bi[gg] = 0.0f;
#pragma unroll
        for (int k = 0; k < NK; k++) psum += p_write<D>(T, k, sc[k], S.m, live, abuf, ho, tl, bi);
        S.lsum *= f;
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) S.bacc[gg] *= f;
        const float f0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), 0));
        const float f1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), 16));
        const float f2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), 32));
        const float f3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), 48));
#pragma unroll
        for (int e = 0; e < 8; e++) {
            S.acc[e][0] *= f0;
            S.acc[e][1] *= f1;
            S.acc[e][2] *= f2;
            S.acc[e][3] *= f3;
        }
    }
    S.lsum += psum;
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) S.bacc[gg] += bi[gg];
}

// This lane's a of every V step of a tile (V layout: group of its dword,
// head x = l%4, token TSV*j + T).  LDS accesses of one wave complete in
// order, so the wavefront-scope fences cost no wait; they keep the compiler
// from moving these reads above the writes of the tile.
template <int D>
__device__ __forceinline__ void read_a(const float *abuf, int gv, int x, int tv, float *ar)
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < Geo<D>::NV; j++) ar[j] = abuf[a_slot(gv, x, Geo<D>::TSV * j + tv)];
}

// One V step of a tile: the 8 nibbles of this lane's dword as f32 (v_cvt),
// then 8 outer-product MFMAs, rows a = p*scale of the 4 heads, columns the
// nibbles.  The conversion of step j+1 is issued beside the MFMAs of step j,
// so no MFMA waits for a conversion just issued.
__device__ __forceinline__ void v_cvt(uint32_t w, float *nb)
{
    const uint32_t lo = nib_lo(w), hi = nib_hi(w);
#pragma unroll
    for (int e = 0; e < 8; e++) nb[e] = (float)(((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xffu);
}

template <int D>
__device__ __forceinline__ void v_mfma(WaveState<D> &S, const float *nb, float a)
{
#pragma unroll
    for (int e = 0; e < 8; e++)
        S.acc[e] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, nb[e], S.acc[e], 0, 0, 0);
}

// Token assignment: nb = gridDim.x blocks share one (sequence, kv head).
// Its kTT-token tiles are dealt round robin, tile j to block (j / kWaves) % nb
// and wave j % kWaves, so at any time the waves of a (sequence, kv head) read
// one contiguous window of every plane (DRAM locality), and a wave's tiles
// are nb * kWaves tiles apart.  Softmax partials do not depend on which
// tokens a wave sees.  Each block writes its partial (m, l, o[D]) per q head
// of its kv head; merge_kernel combines the blocks.
template <int D>
__global__ __launch_bounds__(256, kBlocksPerCU) void mfma_kernel(
    eakvd_geom g, eakvd_batch bt, int layer, const float *__restrict__ q,
    int n_q, int qpk, float rs, float *__restrict__ part)
{
    constexpr int GPD = D / 64;
    constexpr int DW = Geo<D>::DW, NK = Geo<D>::NK, NV = Geo<D>::NV;
    __shared__ float a_lds[kWaves][2][GPD * 4 * kTT];
    __shared__ float s_lds[kWaves][2][kSlot<D>];
    __shared__ float o_lds[kWaves][4][D];
    __shared__ float m_lds[kWaves][4], l_lds[kWaves][4];

    const int ch = blockIdx.x, nb = gridDim.x, kvh = blockIdx.y, s = blockIdx.z;
    const int L = bt.seq_len[s];
    const int n_tiles = (L + kTT - 1) / kTT;
    if (ch * kWaves >= n_tiles) return;     // no tile for this block: no partial
    // the wave index is wave-uniform: say so, so that every per-wave
    // quantity (token range, tile offsets) stays in scalar registers
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = qpk;                                  // 1..4
    const int first = ch * kWaves + w;                  // this wave's first tile
    const int n_wt = first < n_tiles ? (n_tiles - first + nb * kWaves - 1) / (nb * kWaves) : 0;
    const int stride = nb * kWaves * kTT;               // tokens between its tiles
    const Planes K = planes_of(g, bt.base[s], layer, 0);
    const Planes V = planes_of(g, bt.base[s], layer, 1);
    const int64_t hbase = (int64_t)kvh * g.gph;
    const float *qs = q + ((int64_t)s * n_q + (int64_t)kvh * qpk) * D;

    // ---- q -> A operands.  Lane l: row i = l%16 (head ha = i/4, digit
    // pa = i%4), k-block qq = l/16; k-slot j of group gg holds dim
    // 64gg + 8qq + j (j < 8, low nibbles) or 64gg + 32 + 8qq + (j-8).
    // Rows of heads >= G are zero (their q is read from head 0 and dropped).
    // The q loads are issued first, then the first two pipeline stages
    // (further below), so the digit arithmetic waits only for q.
    const int ha = (l & 15) >> 2, pa = l & 3, qq = l >> 4;
    const bool qrow = ha < G;
    float qv[GPD][16];
    {
        const float4 *qh4 = (const float4 *)(qs + (qrow ? ha : 0) * D);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
                for (int v4 = 0; v4 < 2; v4++) {
                    const float4 f = qh4[(64 * gg + 32 * h2 + 8 * qq) / 4 + v4];
                    float *d = &qv[gg][8 * h2 + 4 * v4];
                    d[0] = f.x; d[1] = f.y; d[2] = f.z; d[3] = f.w;
                }
    }
    __builtin_amdgcn_sched_barrier(0);
    // score layout: this lane receives the scores of head ho for token tl
    const int ho = l >> 4, tl = l & 15;
    const bool live = ho < G;
    // V layout: lane l = (token slot tv, dword u); u is dword uw of group gv;
    // x = l%4 is the head row (A) and the column (B) of its 4x4x1 block.
    const int tv = l / DW, u = l % DW, gv = u / 8, uw = u % 8, x = l & 3;

    LaneOffs P;
    {
        const int64_t wbytes = g.max_groups * 32;
        P.kw = plane_rsrc(K.w, wbytes);
        P.vw = plane_rsrc(V.w, wbytes);
        // K and V blocks of the layer are adjacent: one resource for the
        // scale and bias planes of both
        P.layer = plane_rsrc(K.w, 2 * g.block_bytes);
        P.plane[0] = (uint32_t)g.s_off;
        P.plane[1] = (uint32_t)g.b_off;
        P.plane[2] = (uint32_t)(g.block_bytes + g.s_off);
        P.plane[3] = (uint32_t)(g.block_bytes + g.b_off);
        P.sco = GPD == 2 ? (uint32_t)((hbase + l) * 4)
                         : (uint32_t)((hbase + (l & 31)) * 4 + (l >> 5) * (g.b_off - g.s_off));
        const int64_t gk = hbase + (int64_t)tl * GPD;
        const int64_t gvv = hbase + (int64_t)tv * GPD + gv;
        P.kwo = (uint32_t)(gk * 32 + qq * 8);
        P.vwo = (uint32_t)(gvv * 32 + uw * 4);
    }

    // the first two pipeline stages (see the loop below)
    const int dt0 = first * kTT;                        // token offset of tile 0
    const int last = dt0 + (n_wt > 0 ? n_wt - 1 : 0) * stride;   // ... of its last tile
    Stage<D> sa, sb;
    float *slot_a = s_lds[w][0], *slot_b = s_lds[w][1];
    auto load_stage = [&](Stage<D> &T, float *slot, int dt) {
        load_scales<D>(slot, P, min(dt + stride, last));
        __builtin_amdgcn_sched_barrier(0);
        load_k<D>(T, P, min(dt + stride, last));
        load_v<D>(T, P, min(dt, last));
        __builtin_amdgcn_sched_barrier(0);
    };
    // unconditional (a wave without tiles reads tile dt0, in bounds or 0), so
    // the q waits below count the same younger loads on every path
    load_scales<D>(slot_a, P, dt0);
    __builtin_amdgcn_sched_barrier(0);
    load_k<D>(sa, P, dt0);
    __builtin_amdgcn_sched_barrier(0);
    load_stage(sb, slot_b, dt0);

    float amax = 0.0f;
    float qsum[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) {
        double sum = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            qv[gg][j] = qrow ? qv[gg][j] : 0.0f;
            amax = fmaxf(amax, fabsf(qv[gg][j]));
            sum += (double)qv[gg][j];
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
    // Balanced base-256 digits of z = rint(q * 2^esh): with |z| < 2^30,
    // z + 0x80808080 = sum (d_p + 128) 256^(3-p) with every d_p + 128 in
    // [0, 255], so digit p is byte 3-p of z + 0x80808080, minus 128 (as an
    // int8 bit pattern: the byte xor 0x80).
    v4i A[GPD];
    const uint32_t dsh = 8 * (3 - pa);
#pragma unroll
    for (int gg = 0; gg < GPD; gg++)
#pragma unroll
        for (int w4 = 0; w4 < 4; w4++) {
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int z = (int)rintf(ldexpf(qv[gg][4 * w4 + b], esh));
                const uint32_t u = (uint32_t)z + 0x80808080u;
                word |= ((u >> dsh) & 0xffu) << (8 * b);
            }
            A[gg][w4] = (int)(word ^ 0x80808080u);
        }

    const int esh_o = __shfl(esh, 4 * ho, 64);
    // scores are kept in the log2 domain (times log2(e))
    const float rs2 = rs * EAKV_LOG2E;
    const float wl = ldexpf(rs2, -esh_o), wh = ldexpf(rs2, 16 - esh_o);
    float bq[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) bq[gg] = rs2 * __shfl(qsum[gg], 4 * ho, 64);

    WaveState<D> S;
#pragma unroll
    for (int e = 0; e < 8; e++) S.acc[e] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) S.bacc[gg] = 0.0f;
    S.lsum = 0.0f;
    S.m = -INFINITY;

    // Software pipeline over the wave's tiles.  Stage i holds the K (and V
    // scale/bias) of tile i+1 and the V dwords of tile i; iteration i runs
    // V(i) beside K(i+1) and its softmax weights.  Two stages are in flight
    // (ping-pong registers); the next stage's loads are issued before the
    // current one is consumed.  Loads are unconditional so that every wait
    // counts the same number of younger loads; past the end they re-read
    // the last tile, and K scores past the end are masked.
    if (n_wt > 0) {
        float *ab0 = a_lds[w][0], *ab1 = a_lds[w][1];
        // One basic block holds V(i), K(i+1) and the common softmax step of
        // tile i+1.  V runs in steps of 8 MFMAs; the K and softmax work is
        // cut into pieces (recombination and weights per sub-tile, the
        // rescale test) and one piece rides along each V step, so the VALU
        // work of one fills the matrix-core time of the other.  The sched
        // barriers fix the pieces' order; inside a step the scheduler
        // interleaves freely.
        auto iter = [&](const Stage<D> &T, const float *slot, int dt, const float *av,
                        float *ak) {
            constexpr int NP = 2 * NK + 1;
            float ar[NV], sc[NK], bi[GPD], psum = 0.0f;
            bool need = false;
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) bi[gg] = 0.0f;
            v4i dk[NK][GPD];
            Scales<D> C;
            read_a<D>(av, gv, x, tv, ar);
            wait_vm<kSB<D> + kStage<D>>();
            read_scales<D>(slot, tl, C);
            k_mfma<D>(T, A, dk);
            float nb[2][8];
            v_cvt(T.vw[0], nb[0]);
#pragma unroll
            for (int h = 0; h < NV; h++) {
                if (h + 1 < NV) v_cvt(T.vw[h + 1], nb[(h + 1) & 1]);
                v_mfma<D>(S, nb[h & 1], ar[h]);
#pragma unroll
                for (int piece = 0; piece < NP; piece++) {
                    if (1 + piece * (NV - 1) / NP != h) continue;
                    if (piece < NK) {
                        sc[piece] = k_recomb<D>(C, dk[piece], piece, dt + stride, L, wh,
                                                wl, bq, tl);
                    } else if (piece < 2 * NK) {
                        const int k = piece - NK;
                        psum += p_write<D>(C, k, sc[k], S.m, live, ak, ho, tl, bi);
                    } else {
                        float mt = sc[0];
#pragma unroll
                        for (int k = 1; k < NK; k++) mt = fmaxf(mt, sc[k]);
                        need = live && mt - S.m > kTau;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            softmax_tail<D>(S, C, sc, need, psum, bi, live, ak, ho, tl);
        };
        {
            float sc[NK], bi[GPD], psum = 0.0f;
            v4i dk[NK][GPD];
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) bi[gg] = 0.0f;
            Scales<D> C;
            // slot_a's DMA, then sa's K bytes, then all of sb
            wait_vm<Geo<D>::NK * GPD + kStage<D>>();
            read_scales<D>(slot_a, tl, C);
            k_mfma<D>(sa, A, dk);
            float mt = -INFINITY;
#pragma unroll
            for (int k = 0; k < NK; k++) {
                sc[k] = k_recomb<D>(C, dk[k], k, dt0, L, wh, wl, bq, tl);
                mt = fmaxf(mt, sc[k]);
            }
#pragma unroll
            for (int k = 0; k < NK; k++) psum += p_write<D>(C, k, sc[k], S.m, live, ab0, ho, tl, bi);
            softmax_tail<D>(S, C, sc, live && mt - S.m > kTau, psum, bi, live, ab0, ho, tl);
        }
        for (int i = 0, dt = dt0;; i += 2, dt += 2 * stride) {
            load_stage(sa, slot_a, dt + stride);
            iter(sb, slot_b, dt, ab0, ab1);
            if (i + 1 >= n_wt) break;
            load_stage(sb, slot_b, dt + 2 * stride);
            iter(sa, slot_a, dt + stride, ab1, ab0);
            if (i + 2 >= n_wt) break;
        }
    }

    // ---- wave epilogue.  acc: sum the token slots (lane bits of tv).
#pragma unroll
    for (int o = DW; o < 64; o <<= 1)
#pragma unroll
        for (int e = 0; e < 8; e++)
#pragma unroll
            for (int r = 0; r < 4; r++) S.acc[e][r] += __shfl_xor(S.acc[e][r], o, 64);
    // score layout: lsum and the bias sums over the 16 token lanes of a head
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
        S.lsum += __shfl_xor(S.lsum, o, 64);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) S.bacc[gg] += __shfl_xor(S.bacc[gg], o, 64);
    }
    float bsum[4];                                  // head r, this lane's group gv
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float b = __shfl(S.bacc[0], 16 * r, 64);
        if (GPD == 2) {
            const float b1 = __shfl(S.bacc[GPD - 1], 16 * r, 64);
            b = gv ? b1 : b;
        }
        bsum[r] = b;
    }
    if (tv == 0) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int dim = 64 * gv + (e < 4 ? 0 : 32) + 4 * uw + (e & 3);
#pragma unroll
            for (int r = 0; r < 4; r++) o_lds[w][r][dim] = S.acc[e][r] + bsum[r];
        }
    }
    if (tl == 0) {
        m_lds[w][ho] = S.m;
        l_lds[w][ho] = S.lsum;
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
            const float f = __builtin_amdgcn_exp2f(m_lds[ww][h] - M);
            lt = fmaf(l_lds[ww][h], f, lt);
            ot = fmaf(o_lds[ww][h][dim], f, ot);
        }
        float *dst = part + (((int64_t)s * n_q + kvh * qpk + h) * nb + ch) * (D + 2);
        dst[2 + dim] = ot;
        if (dim == 0) {
            dst[0] = M;
            dst[1] = lt;
        }
    }
}

// Merge of the MFMA program's chunk partials (log2 domain) per (q head,
// sequence): M = max(-1e6 log2(e), m_c) (the reference's max starts at
// -1e6), l = sum l_c 2^(m_c - M), o = sum o_c 2^(m_c - M), out = o * (1/l).
// The chunks are read kMergeBatch at a time with all loads in flight and
// merged online across batches.  An empty sequence has no chunks:
// 0 * (1/0) = NaN, as the reference.
constexpr int kMergeBatch = 16;

template <int D>
__global__ __launch_bounds__(D) void merge_kernel(
    eakvd_batch bt, int n_q, int max_chunks, const float *__restrict__ part,
    float *__restrict__ out)
{
    const int qh = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    // blocks that had a tile (see mfma_kernel)
    const int n_tiles = (bt.seq_len[s] + kTT - 1) / kTT;
    const int n_chunks = min(max_chunks, (n_tiles + kWaves - 1) / kWaves);
    const float *p = part + ((int64_t)s * n_q + qh) * max_chunks * (D + 2);
    float M = -1000000.0f * EAKV_LOG2E, lt = 0.0f, ot = 0.0f;
    for (int c0 = 0; c0 < n_chunks; c0 += kMergeBatch) {
        float m[kMergeBatch], lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; j++) {
            const float *pc = p + min(c0 + j, n_chunks - 1) * (D + 2);
            m[j] = pc[0];
            lv[j] = pc[1];
            ov[j] = pc[2 + i];
        }
        float Mn = M;
#pragma unroll
        for (int j = 0; j < kMergeBatch; j++)
            if (c0 + j < n_chunks) Mn = fmaxf(Mn, m[j]);
        const float f = __builtin_amdgcn_exp2f(M - Mn);
        lt *= f;
        ot *= f;
#pragma unroll
        for (int j = 0; j < kMergeBatch; j++) {
            const float wj = c0 + j < n_chunks ? __builtin_amdgcn_exp2f(m[j] - Mn) : 0.0f;
            lt = fmaf(lv[j], wj, lt);
            ot = fmaf(ov[j], wj, ot);
        }
        M = Mn;
    }
    out[((int64_t)s * n_q + qh) * D + i] = ot * (1.0f / lt);
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

// Blocks per (sequence, kv head) of the MFMA program: enough that the grid
// fills every CU with kBlocksPerCU resident blocks once (a second, partial
// round of blocks would idle most of the chip), no more than the workspace's
// partials allow (one per kChunkV tokens) and at least one.
int mfma_blocks_per_unit(int ml, int units)
{
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) ==
                hipSuccess && v > 0)
            n_cu = v;
        else
            n_cu = 256;
    }
    const int slots = n_cu * kBlocksPerCU;
    int nb = units >= slots ? 1 : slots / units;
    const int cap = (ml + kChunkV - 1) / kChunkV;
    nb = nb < cap ? nb : cap;
    return nb < 1 ? 1 : nb;
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
                           float *out, void *work, void *stream)
{
    const hipStream_t st = (hipStream_t)stream;
    const int qpk = n_q / n_kv;
    const float rs = 1.0f / sqrtf((float)g->head_dim);
    float *part = (float *)work;
    const int ml = max_len(b);
    // the MFMA program addresses a layer's K and V blocks with 32-bit buffer
    // offsets
    const bool small_planes = 2 * g->block_bytes <= (int64_t)0x7fffffff;
    if (qpk <= 4 && small_planes) {
        const int mc = mfma_blocks_per_unit(ml, b->n_seq * n_kv);
        const dim3 grid((unsigned)mc, (unsigned)n_kv, (unsigned)b->n_seq);
        const dim3 mgrid((unsigned)n_q, (unsigned)b->n_seq);
        if (g->head_dim == 64) {
            hipLaunchKernelGGL(mfma_kernel<64>, grid, dim3(256), 0, st, *g, *b, layer,
                               q, n_q, qpk, rs, part);
            hipLaunchKernelGGL(merge_kernel<64>, mgrid, dim3(64), 0, st, *b, n_q, mc,
                               part, out);
        } else {
            hipLaunchKernelGGL(mfma_kernel<128>, grid, dim3(256), 0, st, *g, *b, layer,
                               q, n_q, qpk, rs, part);
            hipLaunchKernelGGL(merge_kernel<128>, mgrid, dim3(128), 0, st, *b, n_q, mc,
                               part, out);
        }
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
