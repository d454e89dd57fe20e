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
// wave-uniform and are read through the scalar cache.  Each block walks
// several 256-token slices with the next slice's loads in flight while it
// computes the current one.  Nibbles become floats by masking a dword to four
// byte-wide nibbles and converting its bytes (v_cvt_f32_ubyte0..3): exact,
// as the reference's int-to-float conversion of the nibble.  Grids that
// leave the chip unfilled split the work further: a group's q heads over
// blocks, or (one q head per kv head) a token's 16 accumulators over four
// lanes (k_score_mha4_kernel).
#include "common.h"

namespace {

constexpr int kKsBufs = 2;                          // slices per wave in flight, one consumed
constexpr int kKsBlocksPerCU = 2;

template <int J>
__device__ __forceinline__ void dequant4(float *klo, float *khi, uint32_t lo, uint32_t hi,
                                         float s, float b)
{
    klo[J] = fmaf(ubyte_f32<J>(lo), s, b);
    khi[J] = fmaf(ubyte_f32<J>(hi), s, b);
}

template <int D>
struct KTok {
    uint4 raw[2 * (D / 64)];
    float sc[D / 64], bi[D / 64];
};

// The packed bytes, scales and biases of the lanes' tokens in slice sl of a
// kv head whose planes start at w, sc, bi and hold L tokens.  The slice's
// buffer resources start at the slice (64-bit base arithmetic, wave-uniform)
// and end at the last token, so the lane offsets are fixed and reads past
// the last token, or of a slice past the end, return 0.
template <int D>
__device__ __forceinline__ void k_load(const uint8_t *w, const float *sc, const float *bi,
                                       int L, int sl, KTok<D> &T)
{
    constexpr int GPD = D / 64;
    const int64_t t0 = (int64_t)sl * 256;
    const int64_t left = L > t0 ? L - t0 : 0;            // tokens in this slice and after
    const int nt = (int)(left < 256 ? left : 256);
    const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w + t0 * GPD * 32),
                                                      (short)0, nt * GPD * 32, 0x00020000);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(sc + t0 * GPD),
                                                      (short)0, nt * GPD * 4, 0x00020000);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(bi + t0 * GPD),
                                                      (short)0, nt * GPD * 4, 0x00020000);
    const int vw = threadIdx.x * GPD * 32, vs = threadIdx.x * GPD * 4;
#pragma unroll
    for (int i = 0; i < 2 * GPD; i++) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rw, vw + 16 * i, 0, 0);
        T.raw[i] = uint4{v[0], v[1], v[2], v[3]};
    }
    if constexpr (GPD == 2) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b64(rs, vs, 0, 0);
        const auto b = __builtin_amdgcn_raw_buffer_load_b64(rb, vs, 0, 0);
        T.sc[0] = __uint_as_float(a[0]);
        T.sc[1] = __uint_as_float(a[1]);
        T.bi[0] = __uint_as_float(b[0]);
        T.bi[1] = __uint_as_float(b[1]);
    } else {
        T.sc[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, vs, 0, 0));
        T.bi[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, vs, 0, 0));
    }
}

// Block b takes the 256-token slices b, b + gridDim.x, ... of its kv head
// (one token per lane) and loads the next slice while it computes one.
template <int D, bool MHA>
__device__ __forceinline__ void k_score_body(
    const uint8_t *__restrict__ kw, const float *__restrict__ ks,
    const float *__restrict__ kb, int64_t gph, int L,
    const float *__restrict__ q, int qpk, float *__restrict__ scores, float rs)
{
    constexpr int GPD = D / 64;
    constexpr int NC = D / 16;
    const int kvh = blockIdx.y;
    const int n_sl = (L + 255) / 256;
    const int64_t hb = (int64_t)kvh * gph;        // the kv head's first group
    const uint8_t *hw = kw + hb * 32;
    const float *hs = ks + hb, *hbi = kb + hb;
    const float *qk = q + (int64_t)kvh * qpk * D;
    // blockIdx.z: which of gridDim.z equal parts of the group's q heads
    // this block dots (a grid too small for the chip splits the heads)
    const int qn = qpk / (int)gridDim.z, o0 = (int)blockIdx.z * qn;

    // one 256-token slice: dequantize each lane's token once, then dot it
    // with every q head of the kv head in this block's part
    auto compute = [&](const KTok<D> &T, int sl) {
        const int t = sl * 256 + threadIdx.x;
        if constexpr (MHA) {
            // one q head: each dequantized value goes straight into its fma,
            // chunks c = 4*grp + 2*nib + half in order
            float acc[16];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] = 0.0f;
            // q is read through the scalar cache per slice: the compiler
            // barrier keeps it from holding all D values in vector registers
            // across slices
            const float *qh = qk;
            asm volatile("" ::: "memory");
#pragma unroll
            for (int grp = 0; grp < GPD; grp++)
#pragma unroll
                for (int nib = 0; nib < 2; nib++)
#pragma unroll
                    for (int half = 0; half < 2; half++) {
                        const uint4 v = T.raw[grp * 2 + half];
                        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
                        const float *qc = qh + (4 * grp + 2 * nib + half) * 16;
#pragma unroll
                        for (int wd = 0; wd < 4; wd++) {
                            const uint32_t n = (nib ? w4[wd] >> 4 : w4[wd]) & 0x0f0f0f0fu;
                            float *a = &acc[4 * wd];
                            const float s = T.sc[grp], b = T.bi[grp];
                            a[0] = fmaf(fmaf(ubyte_f32<0>(n), s, b), qc[4 * wd + 0], a[0]);
                            a[1] = fmaf(fmaf(ubyte_f32<1>(n), s, b), qc[4 * wd + 1], a[1]);
                            a[2] = fmaf(fmaf(ubyte_f32<2>(n), s, b), qc[4 * wd + 2], a[2]);
                            a[3] = fmaf(fmaf(ubyte_f32<3>(n), s, b), qc[4 * wd + 3], a[3]);
                        }
                    }
            if (t < L) scores[(int64_t)kvh * L + t] = __fmul_rn(reduce16(acc), rs);
            return;
        }
        // k[c*16 + i]: chunk c = 4*grp + 2*nib + half, byte i of half `half`
        float k[D];
#pragma unroll
        for (int grp = 0; grp < GPD; grp++)
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const uint4 v = T.raw[grp * 2 + half];
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int wd = 0; wd < 4; wd++) {
                    const uint32_t lo = w4[wd] & 0x0f0f0f0fu;
                    const uint32_t hi = (w4[wd] >> 4) & 0x0f0f0f0fu;
                    float *klo = &k[(4 * grp + half) * 16 + 4 * wd];
                    float *khi = &k[(4 * grp + 2 + half) * 16 + 4 * wd];
                    dequant4<0>(klo, khi, lo, hi, T.sc[grp], T.bi[grp]);
                    dequant4<1>(klo, khi, lo, hi, T.sc[grp], T.bi[grp]);
                    dequant4<2>(klo, khi, lo, hi, T.sc[grp], T.bi[grp]);
                    dequant4<3>(klo, khi, lo, hi, T.sc[grp], T.bi[grp]);
                }
            }
        for (int o = o0; o < o0 + qn; o++) {
            const float *qv = qk + (int64_t)o * D;
            float acc[16];
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; c++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    acc[i] = fmaf(k[c * 16 + i], qv[c * 16 + i], acc[i]);
            if (t < L)
                scores[(int64_t)(kvh * qpk + o) * L + t] = __fmul_rn(reduce16(acc), rs);
        }
    };

    // kKsBufs buffers in turn: the next kKsBufs - 1 slices load while one is
    // consumed (no copies between them, so the consumer waits only for its
    // own loads).  The loads past the last slice are unconditional (past the
    // end they read 0 and cost no memory traffic), so every path waits for
    // the same loads.
    const int G = gridDim.x;
    KTok<D> buf[kKsBufs];
    int sl = blockIdx.x;
#pragma unroll
    for (int i = 0; i < kKsBufs - 1; i++) k_load<D>(hw, hs, hbi, L, sl + i * G, buf[i]);
    for (;;) {
#pragma unroll
        for (int j = 0; j < kKsBufs; j++) {
            k_load<D>(hw, hs, hbi, L, sl + (kKsBufs - 1) * G, buf[(j + kKsBufs - 1) % kKsBufs]);
            compute(buf[j], sl);
            sl += G;
            if (sl >= n_sl) return;
        }
    }
}

template <int D>
__global__ __launch_bounds__(256) void k_score_kernel(
    const uint8_t *__restrict__ kw, const float *__restrict__ ks,
    const float *__restrict__ kb, int64_t gph, int L,
    const float *__restrict__ q, int qpk, float *__restrict__ scores, float rs)
{
    k_score_body<D, false>(kw, ks, kb, gph, L, q, qpk, scores, rs);
}

// One q head per kv head, one lane per token: registers for 2 waves per
// SIMD.  Long contexts: its 16-byte loads read a token's row at once.
template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_score_mha_kernel(
    const uint8_t *__restrict__ kw, const float *__restrict__ ks,
    const float *__restrict__ kb, int64_t gph, int L,
    const float *__restrict__ q, int qpk, float *__restrict__ scores, float rs)
{
    k_score_body<D, true>(kw, ks, kb, gph, L, q, qpk, scores, rs);
}

// One q head per kv head (MHA), short contexts: four lanes per token.  Lane part j of a
// token runs the reference's accumulators 4j..4j+3 (acc_i: the fma chain,
// in chunk order, of k[c*16+i] * q[c*16+i] with k = fma(nibble, scale,
// bias)), so a lane does a quarter of a token's arithmetic and a slice's
// last tokens cost a quarter of the time after their data land.  The
// reference's pairwise halving tree (reduce16) is taken across the four
// lanes by quad permutes: v8 = a + a of the lane two over, v4 = v8 + v8 of
// the neighbour, then v2 and v1 in the lane; lane 0 of a token adds in the
// reference's operand order, so scores stay bit-exact.  A block-slice is 64
// tokens; lane j reads dword j of each 16-byte half of the token's groups.
constexpr int kMhaBufs = 4;                         // slices per wave in flight, one consumed

template <int D>
struct KQuad {
    uint32_t w[2 * (D / 64)];                       // dword j of (group, half)
    float sc[D / 64], bi[D / 64];
};

template <int D>
__device__ __forceinline__ void kq_load(const uint8_t *w, const float *sc, const float *bi,
                                        int L, int sl, int ts, int j, KQuad<D> &T)
{
    constexpr int GPD = D / 64;
    const int64_t t0 = (int64_t)sl * 64;
    const int64_t left = L > t0 ? L - t0 : 0;       // tokens in this slice and after
    const int nt = (int)(left < 64 ? left : 64);
    const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(w + t0 * GPD * 32),
                                                      (short)0, nt * GPD * 32, 0x00020000);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(sc + t0 * GPD),
                                                      (short)0, nt * GPD * 4, 0x00020000);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(bi + t0 * GPD),
                                                      (short)0, nt * GPD * 4, 0x00020000);
#pragma unroll
    for (int g = 0; g < GPD; g++)
#pragma unroll
        for (int h = 0; h < 2; h++)
            T.w[2 * g + h] = __builtin_amdgcn_raw_buffer_load_b32(
                rw, ts * GPD * 32 + g * 32 + h * 16 + 4 * j, 0, 0);
#pragma unroll
    for (int g = 0; g < GPD; g++) {
        T.sc[g] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (ts * GPD + g) * 4, 0, 0));
        T.bi[g] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, (ts * GPD + g) * 4, 0, 0));
    }
}

// the value of lane (l ^ 2) and of lane (l ^ 1) within each quad of lanes
__device__ __forceinline__ float quad_xor2(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_xor1(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
}

template <int D>
__global__ __launch_bounds__(256) void k_score_mha4_kernel(
    const uint8_t *__restrict__ kw, const float *__restrict__ ks,
    const float *__restrict__ kb, int64_t gph, int L,
    const float *__restrict__ q, float *__restrict__ scores, float rs)
{
    constexpr int GPD = D / 64;
    constexpr int NC = D / 16;
    const int kvh = blockIdx.y;
    const int j = threadIdx.x & 3, ts = threadIdx.x >> 2;
    const int n_sl = (L + 63) / 64;
    const int64_t hb = (int64_t)kvh * gph;          // the kv head's first group
    const uint8_t *hw = kw + hb * 32;
    const float *hs = ks + hb, *hbi = kb + hb;
    // this lane's q values, q[c*16 + 4j + m]
    float qv[NC][4];
    const float *qh = q + (int64_t)kvh * D;
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
        for (int m = 0; m < 4; m++) qv[c][m] = qh[c * 16 + 4 * j + m];

    auto compute = [&](const KQuad<D> &T, int sl) {
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        // chunks c = 4*grp + 2*nib + half in order
#pragma unroll
        for (int grp = 0; grp < GPD; grp++)
#pragma unroll
            for (int nib = 0; nib < 2; nib++)
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int c = 4 * grp + 2 * nib + half;
                    const uint32_t x = T.w[2 * grp + half];
                    const uint32_t n = (nib ? x >> 4 : x) & 0x0f0f0f0fu;
                    const float s = T.sc[grp], b = T.bi[grp];
                    a[0] = fmaf(fmaf(ubyte_f32<0>(n), s, b), qv[c][0], a[0]);
                    a[1] = fmaf(fmaf(ubyte_f32<1>(n), s, b), qv[c][1], a[1]);
                    a[2] = fmaf(fmaf(ubyte_f32<2>(n), s, b), qv[c][2], a[2]);
                    a[3] = fmaf(fmaf(ubyte_f32<3>(n), s, b), qv[c][3], a[3]);
                }
        float v8[4], v4[4];
#pragma unroll
        for (int m = 0; m < 4; m++) v8[m] = __fadd_rn(a[m], quad_xor2(a[m]));
#pragma unroll
        for (int m = 0; m < 4; m++) v4[m] = __fadd_rn(v8[m], quad_xor1(v8[m]));
        const float v1 = __fadd_rn(__fadd_rn(v4[0], v4[2]), __fadd_rn(v4[1], v4[3]));
        const int t = sl * 64 + ts;
        if (j == 0 && t < L) scores[(int64_t)kvh * L + t] = __fmul_rn(v1, rs);
    };

    // as k_score_body: kMhaBufs buffers in turn, the loads past the last
    // slice unconditional (0, no memory traffic)
    const int G = gridDim.x;
    KQuad<D> buf[kMhaBufs];
    int sl = blockIdx.x;
#pragma unroll
    for (int i = 0; i < kMhaBufs - 1; i++) kq_load<D>(hw, hs, hbi, L, sl + i * G, ts, j, buf[i]);
    for (;;) {
#pragma unroll
        for (int i = 0; i < kMhaBufs; i++) {
            kq_load<D>(hw, hs, hbi, L, sl + (kMhaBufs - 1) * G, ts, j,
                       buf[(i + kMhaBufs - 1) % kMhaBufs]);
            compute(buf[i], sl);
            sl += G;
            if (sl >= n_sl) return;
        }
    }
}

// Blocks per kv head: two waves per SIMD over the chip, at most one per
// 256-token slice.
int k_blocks(int n_sl, int n_kv)
{
    const int n_cu = cu_count();
    const int want = (kKsBlocksPerCU * n_cu + n_kv - 1) / n_kv;
    return want < n_sl ? want : n_sl;
}

// Parts of a group's q heads, one per block (gridDim.z): where the slices
// alone leave the chip's resident blocks unfilled (short contexts, few kv
// heads), the largest divisor of qpk that still fits, so each lane dots
// fewer heads (each part dequantizes its tokens again, from L2).  32Q/4KV
// d64 at 4096 tokens: 8 parts, 512 blocks instead of 64.
int k_head_parts(int qpk, int blocks, int n_kv)
{
    const int64_t room = (int64_t)kKsBlocksPerCU * cu_count();
    int hp = 1;
    for (int d = 2; d <= qpk; d++)
        if (qpk % d == 0 && (int64_t)n_kv * blocks * d <= room) hp = d;
    return hp;
}

}  // namespace

extern "C" int eakvd_k_score(const eakvd_geom *g, const uint8_t *base,
                             int layer, int seq_len, const float *q, int n_q,
                             int n_kv, float *scores, void *stream)
{
    if (seq_len <= 0) return 0;
    const Planes p = planes_of(*g, base, layer, 0);
    const hipStream_t st = (hipStream_t)stream;
    const int qpk = n_q / n_kv;
    const float rs = 1.0f / sqrtf((float)g->head_dim);
    const int kb = k_blocks(ceil_div_i(seq_len, 256), n_kv);
    if (qpk == 1 && (int64_t)n_kv * kb < (int64_t)kKsBlocksPerCU * cu_count()) {
        // MHA on a grid of 256-token slices that leaves the chip unfilled:
        // four lanes per token, 64-token slices
        const dim3 grid((unsigned)k_blocks(ceil_div_i(seq_len, 64), n_kv), (unsigned)n_kv);
        auto kern = g->head_dim == 64 ? k_score_mha4_kernel<64> : k_score_mha4_kernel<128>;
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, p.w, p.s, p.b, g->gph, seq_len, q,
                           scores, rs);
        return (int)hipGetLastError();
    }
    const dim3 grid((unsigned)kb, (unsigned)n_kv, (unsigned)k_head_parts(qpk, kb, n_kv));
    auto kern = g->head_dim == 64 ? (qpk == 1 ? k_score_mha_kernel<64> : k_score_kernel<64>)
                                  : (qpk == 1 ? k_score_mha_kernel<128> : k_score_kernel<128>);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, p.w, p.s, p.b, g->gph, seq_len, q, qpk,
                       scores, rs);
    return (int)hipGetLastError();
}
