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
// Two programs; each block covers a chunk of tokens of one kv head and writes
// one partial per q head, and the partials are added in a fixed order.
//
// v_sum_mha_kernel (one q head per kv head): a lane owns 16 packed bytes of a
//   token (32 dims: 16 low nibbles and the 16 high nibbles 32 dims further),
//   D/32 lanes per token, so a wave's load of one 16-byte unit per lane reads
//   1 KB of consecutive tokens.  The planes and the weight row are addressed
//   through buffer resources that end at the chunk's last token: reads past
//   it return 0 and add fma(0, 0, o) = o, so every lane runs the same
//   iterations without bounds tests.  Nibbles become floats by masking a
//   dword to four byte-wide nibbles and converting its bytes.  The last
//   block of a kv head adds the chunk partials (no second launch).
// v_sum_kernel (groups of q heads): a lane owns one packed dword of a token
//   (8 dims), D/8 lanes per token, 256/(D/8) token slots per block.  V is
//   dequantized once per token and reused by every q head of its group (HP
//   per pass: 1, 2, 4 or 8, the smallest that covers the group up to 8, so
//   registers are spent only on heads that exist).  chunk_sum_kernel adds
//   the partials.
// A lane takes a batch of tokens of its slot at a time and issues all their
// loads (V bytes, scale, bias, weights) before the arithmetic.
#include "common.h"

namespace {

constexpr int kBatch = 8;
constexpr int kChunk = 256;
// Cache policy of the MHA program's plane and weight loads: non-temporal
// (nt), each byte being read once (32 x 8192 tokens, d = 128: 8.17-8.20
// against 8.37-8.45 us per call)
constexpr int kMhaAux = 2;

// Tokens per lane per batch: 8 where the grid still fills the chip with 8,
// else 2 (short contexts: more blocks, less serial work per lane).
template <int D, int KB>
struct MhaGeo {
    static constexpr int GPD = D / 64;
    static constexpr int RB = D / 2;               // packed bytes of a token
    static constexpr int LPT = D / 32;             // lanes per token
    static constexpr int TS = 256 / LPT;           // token slots per block
    static constexpr int PAD = 4;                  // floats between rows in LDS
    static constexpr int STEP = TS * KB;           // tokens per batch of a block
};

// Block (ch, kvh): tokens [ch*chunk, min(L, ch*chunk + chunk)) of kv head kvh
// (= q head kvh), weights w[kvh][t].  With one chunk the block writes
// out[kvh][D]; otherwise it writes partial[ch][kvh][D], counts itself on the
// kv head's counter (ctr + kvh*EAKVD_CTR_STRIDE bytes), and the block that
// counts last adds the chunks' partials in chunk order into out and sets the
// counter back to zero for the next call (no other block of the launch
// touches it again).
template <int D, int KB>
__global__ __launch_bounds__(256) void v_sum_mha_kernel(
    const uint8_t *__restrict__ vw, const float *__restrict__ vs,
    const float *__restrict__ vb, int64_t gph, int L,
    const float *__restrict__ w, int chunk, int n_q, float *__restrict__ partial,
    float *__restrict__ out, uint8_t *__restrict__ ctr)
{
    using G = MhaGeo<D, KB>;
    constexpr int NR = 16;                          // row sums per block, 4 per wave
    __shared__ float red[NR * (D + G::PAD)];

    const int kvh = blockIdx.y, ch = blockIdx.x;
    const int qq = threadIdx.x % G::LPT, ts = threadIdx.x / G::LPT;
    const int t_begin = ch * chunk;
    const int n_t = min(L - t_begin, chunk);      // >= 1: the grid covers L
    const int64_t g0 = (int64_t)kvh * gph + (int64_t)t_begin * G::GPD;
    const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(vw + g0 * 32),
                                                      (short)0, n_t * G::RB, 0x00020000);
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(vs + g0), (short)0,
                                                      n_t * G::GPD * 4, 0x00020000);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(vb + g0), (short)0,
                                                      n_t * G::GPD * 4, 0x00020000);
    const auto rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(w + (int64_t)kvh * L + t_begin), (short)0, n_t * 4, 0x00020000);
    // this lane's bytes of a token: 16*qq..16*qq+15 of the row, in group qq/2
    const int vo = ts * G::RB + 16 * qq;
    const int so = (ts * G::GPD + qq / 2) * 4;
    const int wo = ts * 4;

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; i++) acc[i] = 0.0f;

    for (int base = 0; base < n_t; base += G::STEP) {
        v4i raw[KB];
        float sc[KB], bi[KB], wt[KB];
#pragma unroll
        for (int u = 0; u < KB; u++) {
            const int t = base + u * G::TS;       // the slot's token, less ts
            // whole offsets in the range-checked vector operand
            raw[u] = __builtin_amdgcn_raw_buffer_load_b128(rw, vo + t * G::RB, 0, kMhaAux);
            sc[u] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rs, so + t * G::GPD * 4, 0, kMhaAux));
            bi[u] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rb, so + t * G::GPD * 4, 0, kMhaAux));
            wt[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rq, wo + t * 4, 0, kMhaAux));
        }
#pragma unroll
        for (int u = 0; u < KB; u++) {
#pragma unroll
            for (int wd = 0; wd < 4; wd++) {
                const uint32_t x = (uint32_t)raw[u][wd];
                const uint32_t lo = x & 0x0f0f0f0fu, hi = (x >> 4) & 0x0f0f0f0fu;
                float *al = &acc[4 * wd], *ah = &acc[16 + 4 * wd];
                al[0] = fmaf(fmaf(ubyte_f32<0>(lo), sc[u], bi[u]), wt[u], al[0]);
                ah[0] = fmaf(fmaf(ubyte_f32<0>(hi), sc[u], bi[u]), wt[u], ah[0]);
                al[1] = fmaf(fmaf(ubyte_f32<1>(lo), sc[u], bi[u]), wt[u], al[1]);
                ah[1] = fmaf(fmaf(ubyte_f32<1>(hi), sc[u], bi[u]), wt[u], ah[1]);
                al[2] = fmaf(fmaf(ubyte_f32<2>(lo), sc[u], bi[u]), wt[u], al[2]);
                ah[2] = fmaf(fmaf(ubyte_f32<2>(hi), sc[u], bi[u]), wt[u], ah[2]);
                al[3] = fmaf(fmaf(ubyte_f32<3>(lo), sc[u], bi[u]), wt[u], al[3]);
                ah[3] = fmaf(fmaf(ubyte_f32<3>(hi), sc[u], bi[u]), wt[u], ah[3]);
            }
        }
    }

    // The token slots of each 16-lane row summed across the row by DPP right
    // shifts of LPT, 2 LPT (and 4 LPT where LPT = 2) lanes: its last LPT
    // lanes then hold the row's sums, one per 16-byte column.  Only these
    // 16 row sums per block go through LDS (32Q/32KV d128 at 8192 tokens:
    // 7.9-8.1 against 8.1-8.3 us per call with every slot row in LDS).
#pragma unroll
    for (int i = 0; i < 32; i++) {
        acc[i] += dpp_f<0x110 + G::LPT>(acc[i]);
        acc[i] += dpp_f<0x110 + 2 * G::LPT>(acc[i]);
        if constexpr (G::LPT == 2) acc[i] += dpp_f<0x110 + 8>(acc[i]);
    }
    if ((threadIdx.x & 15) >= 16 - G::LPT) {
        // row sums: low nibble i -> dim 64*(qq/2) + 16*(qq%2) + i, high +32
        float *r = red + (threadIdx.x >> 4) * (D + G::PAD) + 64 * (qq / 2) + 16 * (qq % 2);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            *reinterpret_cast<float4 *>(r + i) =
                make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
            *reinterpret_cast<float4 *>(r + 32 + i) =
                make_float4(acc[16 + i], acc[17 + i], acc[18 + i], acc[19 + i]);
        }
    }
    __syncthreads();
    // thread (part, dim) adds NR/P rows in order, then part 0 adds the P sums
    constexpr int P = 256 / D;
    constexpr int RPP = NR / P;
    const int dim = threadIdx.x % D, part = threadIdx.x / D;
    float sum = red[part * RPP * (D + G::PAD) + dim];
#pragma unroll 8
    for (int k = 1; k < RPP; k++) sum = __fadd_rn(sum, red[(part * RPP + k) * (D + G::PAD) + dim]);
    __syncthreads();
    red[part * D + dim] = sum;
    __syncthreads();
    const int nc = gridDim.x;
    if (part == 0) {
        float t = red[dim];
#pragma unroll
        for (int k = 1; k < P; k++) t = __fadd_rn(t, red[k * D + dim]);
        if (nc == 1)
            out[(int64_t)kvh * D + dim] = t;
        else
            st_dev(&partial[((int64_t)ch * n_q + kvh) * D + dim], t);
    }
    if (nc == 1) return;

    // every thread's partial store is complete (vmcnt 0) before the barrier,
    // and so before the count; the last block reads the partials after it
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int last;
    unsigned *uc = reinterpret_cast<unsigned *>(ctr + (int64_t)kvh * EAKVD_CTR_STRIDE);
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(uc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(nc - 1);
    __syncthreads();
    if (!last) return;
    if (threadIdx.x == 0) __hip_atomic_store(uc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x < D) {
        float sum = 0.0f;
        for (int c0 = 0; c0 < nc; c0 += 16) {
            float p[16];
#pragma unroll
            for (int j = 0; j < 16; j++)
                p[j] = ld_dev(&partial[((int64_t)min(c0 + j, nc - 1) * n_q + kvh) * D + threadIdx.x]);
#pragma unroll
            for (int j = 0; j < 16; j++)
                if (c0 + j < nc) sum = __fadd_rn(sum, p[j]);
        }
        out[(int64_t)kvh * D + threadIdx.x] = sum;
    }
}

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

// Launch shape of the MHA program: batches of 8 tokens per lane where one
// batch per block gives at least one block per CU, else of 2; tokens per
// block: whole batches, one batch per block until the grid holds about 4
// blocks per CU (4 waves per SIMD), at most 2^20 tokens (the 32-bit offsets
// of the chunk's resources).
struct MhaPlan {
    int kb, chunk, nc;
};

MhaPlan mha_plan(int D, int L, int n_kv)
{
    const int n_cu = cu_count();
    const int ts = D == 64 ? MhaGeo<64, 8>::TS : MhaGeo<128, 8>::TS;
    MhaPlan p;
    p.kb = (int64_t)n_kv * ceil_div_i(L, ts * 8) >= n_cu ? 8 : 2;
    const int step = ts * p.kb;
    const int64_t blocks = (int64_t)n_kv * ceil_div_i(L, step);
    int64_t it = blocks / (4 * (int64_t)n_cu);
    const int64_t it_max = (1 << 20) / step;
    it = it < 1 ? 1 : (it > it_max ? it_max : it);
    p.chunk = (int)(step * it);
    p.nc = ceil_div_i(L, p.chunk);
    return p;
}

}  // namespace

extern "C" size_t eakvd_v_sum_work_bytes(const eakvd_geom *g, int seq_len,
                                         int n_q)
{
    if (seq_len <= 0) return 0;
    const int n_chunks = ceil_div_i(seq_len, kChunk);
    size_t valu = (size_t)n_chunks * n_q * g->head_dim * sizeof(float);
    // the MHA program's partials (one q head per kv head: n_kv = n_q)
    const size_t mha = (size_t)mha_plan(g->head_dim, seq_len, n_q).nc * n_q * g->head_dim *
                       sizeof(float);
    valu = valu > mha ? valu : mha;
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
    const int qpk = n_q / n_kv;
    float *partial = (float *)work;
    if (qpk == 1) {
        const MhaPlan mp = mha_plan(g->head_dim, seq_len, n_kv);
        const dim3 grid((unsigned)mp.nc, (unsigned)n_kv);
        uint8_t *ctr = const_cast<uint8_t *>(base) + g->ctr_off;
        auto kern = g->head_dim == 64 ? (mp.kb == 8 ? v_sum_mha_kernel<64, 8> : v_sum_mha_kernel<64, 2>)
                                      : (mp.kb == 8 ? v_sum_mha_kernel<128, 8> : v_sum_mha_kernel<128, 2>);
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, p.w, p.s, p.b, g->gph, seq_len, w,
                           mp.chunk, n_q, partial, out, ctr);
        return (int)hipGetLastError();
    }
    const int n_chunks = ceil_div_i(seq_len, kChunk);
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
