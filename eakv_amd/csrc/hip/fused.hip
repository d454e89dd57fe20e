// fused.hip — fused decode attention on the packed cache: K-score, softmax
// and V-sum in one pass over K and V, for a batch of same-shape caches.
//
// Semantics: reference kernels/fused_attention.ea:190-373 (max with init
// -1e6, w = exp(s - max), sum, o = sum deq_v * w, out = o * (1/sum)),
// extended per q head to GQA and d=64.  Each q head h reads kv head
// h / (n_q/n_kv).
//
// Work split (flash-decoding): one block per (sequence, kv head, chunk);
// each block writes a partial (m, l, o[D]) per q head and merge_kernel
// combines the chunks.
//
// Two block programs:
//
// mfma_kernel (one or two quads of q heads per wave: up to 8 q heads per kv
//   head; larger groups as virtual kv heads of at most 8 that share the kv
//   head's tiles; also the unfused V-sum): waves walking 32-token tiles,
//   one or two groups of tile loads in flight behind the one consumed.
//   Both products run on the int8 matrix cores; on gfx950 matrix and vector
//   instructions of a SIMD do not overlap, so the design minimises their
//   sum:
//   K: per 16 tokens and 64-dim group one v_mfma_i32_16x16x64_i8, A = the q
//     heads as 32-bit fixed point split into four signed bytes (rows 4h+p),
//     B = the token's packed bytes masked to nibbles.  Exact integer dots,
//     recombined in f32: score = s*(q.n) + b*sum(q).
//   Online softmax in the log2 domain with a lazy running max (a head's max
//     moves only when a score exceeds it by more than kTau).
//   V: per 16 dims one v_mfma_i32_16x16x32_i8 over the tile's 32 tokens,
//     A = the weights a = p*scale of the 4 heads as 32-bit fixed point with
//     one exponent per (head, group, tile), split into four signed bytes
//     (rows 4h+p); B = the V nibbles, tokens along K.  The V bytes reach LDS
//     by buffer-load-to-LDS and are read back transposed (8 tokens of one
//     byte column per lane) by ds_read_b64_tr_b8; the digits of a are
//     exchanged through LDS the same way.  sum p*bias per (head, group) is
//     kept apart and added at the end.
//   Waves are merged in LDS; chunks by the last block of each unit in the
//   same launch (up to 16 chunks per unit, counters given), else by
//   merge_kernel or merge_parts_kernel in a second launch.
// valu_kernel (caches whose (layer, kv) blocks are beyond the 32-bit buffer
//   offsets of mfma_kernel, above 1 GiB; every group size has a split into
//   virtual kv heads, at worst of one q head each): one lane per token for K
//   with the reference arithmetic, then V by dims; same partial/merge scheme.
#include <string.h>

#include <mutex>
#include <type_traits>

#include "common.h"

// Static device scratch of the allocation-free entry point: the chunk
// partials of one launch.  Host code never uses this name as an address: it
// takes the device address from hipGetSymbolAddress (eakvd_scratch).
static __device__ __align__(256) uint8_t scratch[EAKVD_SCRATCH_BYTES];

namespace {

// ------------------------------------------------------------------ MFMA

constexpr int kWaves = 4;
// Tokens per tile (one pipeline stage), TT = 32 or 64 (tile_tokens).  One
// quad of q heads per wave: 32; its waves read their planes faster in
// 32-token pieces than in 64-token ones (8 x 32Q/8KV at 32767 tokens, two
// tiles dealt together: 64.5 against 61.2 us per call).  Two quads, long
// contexts: 64, so the V products of a tile are one v_mfma_i32_16x16x64_i8
// per 16 dims, and each (head, group) is recombined and given a digit
// exponent once per 64 tokens (20% fewer VALU instructions per token).
// One-quad blocks resident per CU (8 waves): fewer loads in flight per CU
// read the planes faster than 4 blocks (16 waves), and a unit has half the
// chunks to merge (8 x 32Q/8KV at 32767 tokens, merged in the launch: 63.1-64.5
// against 64.3-67.5 us per call with 4 blocks and a merge launch)
constexpr int kBlocksPerCU = 2;   // occupancy the register budget is set for
// Blocks of the kernel for HH quads of q heads per wave.  One quad: blocks
// of kWaves waves, kBlocksPerCU resident per CU.  Two quads: blocks of 8
// waves (d = 128: one per CU, 2 waves per SIMD, as the registers allow;
// d = 64: two).  Tiles are dealt statically in both, so every wave sums the
// same tiles in the same order on every call and results are reproducible
// bit for bit.
template <int HH>
constexpr int kWavesH = HH == 1 ? kWaves : 8;
template <int D, int HH>
constexpr int kBlocksPerCUH = HH == 1 ? kBlocksPerCU : (D == 64 ? 2 : 1);
constexpr float kTau = 8.0f;            // lazy-rescale headroom, 2^8 (log2 units)
// Load groups per wave: one consumed while the next is in flight.  With the
// non-temporal plane loads, two measured faster than three: 64 q / 8 kv
// heads, d = 128, 131071 tokens: 39.2 against 40.0-40.6 us per call;
// 8 x 32Q/8KV at 32767 tokens: 65.7-66.0 against 66.1-68.6 (per-step
// medians); 32Q/32KV at 8192 tokens: 14.0-14.3 against 15.0.
constexpr int kSlots = 2;

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void *lds_ptr;
typedef __attribute__((address_space(3))) v2i *lds_v2i;

// Tile geometry of TT-token tiles.  A plane stores a token's GPD groups of
// 32 packed bytes contiguously (a row of RB bytes, UPT 16-byte units).
// Loads to LDS move 16 bytes per lane, 1 KB per instruction.
template <int D, int TT>
struct Geo {
    static_assert(TT == 32 || TT == 64, "32- or 64-token tiles");
    static constexpr int GPD = D / 64;
    static constexpr int NK = TT / 16;             // K sub-tiles of 16 tokens
    static constexpr int NH = TT / 32;             // 32-token halves (V transposed reads)
    static constexpr int RB = 32 * GPD;            // bytes of a token's row
    static constexpr int UPT = RB / 16;            // 16-byte units per row
    static constexpr int TPC = 8 / GPD;            // tokens per 256 bytes
    static constexpr int NVD = TT * RB / 1024;     // V loads per tile
    static constexpr int VSLOT = TT * RB;          // LDS bytes of one V tile
    static constexpr int LP = TT * GPD / 4;        // lanes per scale plane piece (16 B each)
    static constexpr int SSLOT = 4 * TT * GPD > 256 ? 4 * TT * GPD : 256;  // floats of a scale slot
    static constexpr int NSL = SSLOT * 4 / 1024;   // scale loads per tile
    static constexpr int ZROWS = GPD * 2 * TT;     // 8-byte digit rows per tile
};

// V tile layout in LDS: token rows in order, the 16-byte units of row t
// permuted by xor with vswz(t) (bits of the token's 4-token / 8-token
// block).  With the transposed reads below, that puts the 64 lanes' 8-byte
// rows of one read on 32 distinct bank pairs (2 lanes each, the minimum),
// and keeps each 16-byte unit whole for the 16-byte loads.  vswz(t + 32) =
// vswz(t), so the second half of a 64-token tile has the same pattern.
template <int D>
__device__ __host__ constexpr int vswz(int t)
{
    return (t / Geo<D, 32>::TPC) & (Geo<D, 32>::UPT - 1);
}

// The token (within a 32-token half) of byte j (0..7) of a V operand in
// lane group kq (lanes 16kq..16kq+15).  Digits (A) and nibbles (B) use the
// same order; in a 64-token tile, bytes 8..15 of a lane's operand are the
// same tokens of the second half.
__device__ __forceinline__ int vtok(int kq, int j)
{
    return 16 * (j & 1) + 4 * kq + (j >> 1);
}

// One lane's K bytes of a pipeline stage (MFMA B layout: token 16k + tl of
// sub-tile k, bytes 8qq..8qq+7 of each group).  The V bytes and the K and V
// scales and biases of a stage go to LDS.
template <int D, int TT>
struct Stage {
    uint2 kw[Geo<D, TT>::NK][Geo<D, TT>::GPD];
};

// V-sum mode: one lane's weights of a pipeline stage (score layout: head
// 4hq + l/16 of quad hq, token 16k + l%16 of sub-tile k).
template <int D, int HH, int TT>
struct WStage {
    float wv[HH][Geo<D, TT>::NK];
};

// The scales and biases of one tile for this lane's tokens (score layout:
// token 16k + tl), read from the LDS slot.
template <int D, int TT>
struct Scales {
    float ks[Geo<D, TT>::NK][Geo<D, TT>::GPD], kb[Geo<D, TT>::NK][Geo<D, TT>::GPD];
    float vs[Geo<D, TT>::NK][Geo<D, TT>::GPD], vb[Geo<D, TT>::NK][Geo<D, TT>::GPD];
};

// Buffer resources of the planes (scalar registers) and this lane's byte
// offsets at the wave's first token.  Tile offsets are wave-uniform and go to
// the scalar soffset operand, so a tile costs no per-lane address arithmetic.
// Reads past a plane's end return 0.
struct LaneOffs {
    __amdgpu_buffer_rsrc_t kw, vw, layer;
    uint32_t kwo, vwo, sco[2];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const void *p, int64_t bytes)
{
    // dword3 0x00020000: raw (untyped) 32-bit buffer on gfx9-family parts
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)bytes, 0x00020000);
}

// Cache policy of the plane loads: non-temporal (nt), as every plane byte is
// read once per call (32 calls of 8 caches of 32768 tokens: 69.6-70.6 against
// 71.1-72.5 us per call on one box; sc0 or sc1 instead measured slower).
constexpr int kPlaneAux = 2;

__device__ __forceinline__ uint2 ldb64(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, (int)so, kPlaneAux);
    return uint2{v[0], v[1]};
}

// K bytes of the tile at token offset dt of the wave.  A tile can run up to
// TT - 1 tokens past the wave's last token; those reads stay inside the
// plane (or return 0 beyond it), their scores are masked to -inf and their
// weight is exactly 0.  dt is the same in every lane; readfirstlane makes
// that visible, so the tile offset goes to the scalar soffset operand.
template <int D, int TT>
__device__ __forceinline__ void load_k(Stage<D, TT> &T, const LaneOffs &P, int dt, uint32_t ob)
{
    constexpr int GPD = D / 64;
    const uint32_t ws = (uint32_t)__builtin_amdgcn_readfirstlane(dt) * GPD * 32;
#pragma unroll
    for (int k = 0; k < Geo<D, TT>::NK; k++)
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
            T.kw[k][gg] = ldb64(P.kw, P.kwo + ob, ws + (16 * k * GPD + gg) * 32);
}

// V-sum mode: the weights of the tile at token offset dt, w[head][dt + 16k +
// tl] from the kv head's rows (wo[hq]: byte offset of the lane's row).
// Tokens past the sequence read the row's last weight (in bounds); the
// caller masks them.
template <int D, int HH, int TT>
__device__ __forceinline__ void load_w(WStage<D, HH, TT> &T, __amdgpu_buffer_rsrc_t r,
                                       const uint32_t *wo, int dt, int tl, int L)
{
#pragma unroll
    for (int hq = 0; hq < HH; hq++)
#pragma unroll
        for (int k = 0; k < Geo<D, TT>::NK; k++) {
            const int t = min(dt + 16 * k + tl, L - 1);
            T.wv[hq][k] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(r, (int)(wo[hq] + 4u * (uint32_t)t), 0, 0));
        }
}

// The V bytes of the tile at dt into a V slot, 1 KB per instruction (buffer
// load to LDS: lane m's 16 bytes land at the instruction's LDS start + 16m;
// the lane fetches the unit that belongs there, see LaneOffs.vwo).
template <int D, int TT>
__device__ __forceinline__ void load_v(uint8_t *vslot, const LaneOffs &P, int dt, uint32_t ob)
{
    constexpr int GPD = D / 64;
    const uint32_t ws = (uint32_t)__builtin_amdgcn_readfirstlane(dt) * GPD * 32;
#pragma unroll
    for (int i = 0; i < Geo<D, TT>::NVD; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(P.vw, (lds_ptr)(vslot + 1024 * i), 16,
                                                 (int)(P.vwo + ob), (int)(ws + 1024 * i), 0,
                                                 kPlaneAux);
}

// The K and V scales and biases of the tile at dt into a scale slot, NSL
// instructions (one, or two for 64 tokens at d=128).  Slot layout: plane p
// in {ks, kb, vs, vb} at p * TT * GPD floats, then token-major,
// group-minor, as in the planes; each plane piece is LP lanes of 16 bytes
// (instruction i, lane m: plane (64i + m) / LP; at d=64 with 32-token tiles
// lanes 32-63 repeat lanes 0-31 into the unused second half of the slot).
template <int D, int TT>
__device__ __forceinline__ void load_scales(float *slot, const LaneOffs &P, int dt, uint32_t ob)
{
    constexpr int GPD = D / 64;
    const uint32_t ss = (uint32_t)__builtin_amdgcn_readfirstlane(dt) * GPD * 4;
#pragma unroll
    for (int i = 0; i < Geo<D, TT>::NSL; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(P.layer, (lds_ptr)(slot + 256 * i), 16,
                                                 (int)(P.sco[i] + ob), (int)ss, 0, kPlaneAux);
}

// Loads per group, in issue order: V chunks, scales, then the K bytes (or
// the V-sum's weights; fixed by sched barriers).  The compiler does not order LDS reads after buffer loads to
// LDS, so reads of a slot are preceded by an explicit wait for every load
// older than the ones that may still be outstanding.
template <int D, int TT>
constexpr int kDma = Geo<D, TT>::NSL;                    // scale loads
template <int D, int TT>
constexpr int kNK = Geo<D, TT>::NK * (D / 64);           // K loads

// s_waitcnt vmcnt(n), no wait on the other counters (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int D, int TT>
__device__ __forceinline__ void read_scales(const float *slot, int tl, Scales<D, TT> &C)
{
    constexpr int GPD = D / 64, PS = TT * GPD;
#pragma unroll
    for (int k = 0; k < Geo<D, TT>::NK; k++) {
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

// The low and high nibbles of four packed bytes, as bytes (int8 MFMA
// operands: values 0..15)
__device__ __forceinline__ uint32_t nib_lo(uint32_t x) { return x & 0x0f0f0f0fu; }
__device__ __forceinline__ uint32_t nib_hi(uint32_t x) { return (x >> 4) & 0x0f0f0f0fu; }

// p * v with 0 * anything = 0 (v_mul_legacy_f32; otherwise IEEE rounding).
// A tile can cover tokens past the sequence end whose p is 0 but whose stale
// scale or bias may be non-finite; their products must stay 0.
__device__ __forceinline__ float mul_zero(float p, float v)
{
    float r;
    asm("v_mul_legacy_f32 %0, %1, %2" : "=v"(r) : "v"(p), "v"(v));
    return r;
}

// max / sum over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1); every lane
// of the row ends with the result.  bound_ctrl lets the compiler fold each
// move into the DPP form of the operation.
template <int N>
__device__ __forceinline__ int dpp_ror(int v)
{
    return __builtin_amdgcn_mov_dpp(v, 0x120 + N, 0xf, 0xf, true);
}

__device__ __forceinline__ float row_max16(float v)
{
    v = fmaxf(v, __int_as_float(dpp_ror<8>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_ror<4>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_ror<2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_ror<1>(__float_as_int(v))));
    return v;
}

// the same for values >= +0 (or NaN), whose bit patterns order as integers
__device__ __forceinline__ float row_max16_pos(float v)
{
    int x = __float_as_int(v);
    x = max(x, dpp_ror<8>(x));
    x = max(x, dpp_ror<4>(x));
    x = max(x, dpp_ror<2>(x));
    x = max(x, dpp_ror<1>(x));
    return __int_as_float(x);
}

__device__ __forceinline__ float max_pos(float a, float b)
{
    return __int_as_float(max(__float_as_int(a), __float_as_int(b)));
}

__device__ __forceinline__ float row_sum16(float v)
{
    v += __int_as_float(dpp_ror<8>(__float_as_int(v)));
    v += __int_as_float(dpp_ror<4>(__float_as_int(v)));
    v += __int_as_float(dpp_ror<2>(__float_as_int(v)));
    v += __int_as_float(dpp_ror<1>(__float_as_int(v)));
    return v;
}

__device__ __forceinline__ v2i tr8(const uint8_t *p)
{
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i)p);
}

__device__ __forceinline__ long as_long(v2i v)
{
    return __builtin_bit_cast(long, v);
}

// K of one tile: per 16-token sub-tile, the digit-row dots of each group on
// the int8 matrix core (k_mfma), then their recombination (k_recomb).  The
// four digit rows r (weights 2^24, 2^16, 2^8, 1) are paired exactly in int32,
// H = 256*d0 + d1 and Lo = 256*d2 + d3 (|H|, |Lo| < 2^25), and
// u = H*wh + Lo*wl with wh = 2^16*wl, wl = 2^-e*log2(e)/sqrt(d).  Scores are
// in the log2 domain: sc = log2(e) * (q.k)/sqrt(d); masked tokens get -inf.
template <int D, int TT>
__device__ __forceinline__ void k_mfma(const Stage<D, TT> &T, const v4i *A,
                                       v4i (*dk)[D / 64])
{
#pragma unroll
    for (int k = 0; k < Geo<D, TT>::NK; k++)
#pragma unroll
        for (int gg = 0; gg < D / 64; gg++) {
            const uint2 raw = T.kw[k][gg];
            const v4i B = v4i{(int)nib_lo(raw.x), (int)nib_lo(raw.y), (int)nib_hi(raw.x),
                              (int)nib_hi(raw.y)};
            dk[k][gg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[gg], B, v4i{0, 0, 0, 0},
                                                               0, 0, 0);
        }
}

template <int D, int TT>
__device__ __forceinline__ float k_recomb(const Scales<D, TT> &T, const v4i *d, int k,
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

// The V accumulation of one (group, 16-byte column block) of a tile: one
// transposed read per 32-token half gives each lane 8 tokens' bytes at byte
// column 16*half + n of group g; the low nibbles are dims 64g + 16half + n,
// the high nibbles dims 64g + 32 + 16half + n.  Each MFMA sums the tokens of
// the tile (v_mfma_i32_16x16x32_i8 for 32, _16x16x64_i8 for 64); the four
// digit rows of a head come back in one lane (C[i], weight 256^i) and are
// recombined as (256*C3 + C2) * 2^(16-E) + (256*C1 + C0) * 2^-E.  The top
// digit of a weight below 2^30 lies in [-64, 64], so |256*C3 + C2| < 2^24
// and its conversion is exact; 256*C1 + C0 may round (64 tokens), 2^16
// times below it.
__device__ __forceinline__ float v_recomb(v4i c, float wh, float wl, float acc)
{
    const int hi = c[3] * 256 + c[2];
    const int lo = c[1] * 256 + c[0];
    return fmaf((float)hi, wh, fmaf((float)lo, wl, acc));
}

// State carried across the tiles of one wave.  acc (V output layout): lane
// (head l/16, column n = l%16) holds dims 64g + 32lh + 16half + n at
// acc[g][half][lh].  Score layout (lane = head ho x token tl): the running
// max m of head ho, the softmax denominator lsum and the bias sums
// sum p*bias per group.  wh/wl: the digit weights of the tile whose digits
// are in the digit buffer.
template <int D>
struct WaveState {
    float acc[D / 64][2][2];
    float bacc[D / 64];
    float wh[D / 64], wl[D / 64];
    float lsum, m;
};

// The chunk merge of a launch that merges its own chunks (at most kInBatch
// chunks per unit), done by the block of the unit that counts last.  Each
// thread restates, for its one or two adjacent outputs, the arithmetic of
// the merge launch the same call would make, in the same order, so both give
// the same bits: merge_kernel, and vsum_merge_kernel in V-sum mode.  Loads:
// the (m, l) pair of every (head, chunk) once per block into LDS (one 8-byte
// device-scope load each), and per thread the o values of kInBatch chunks
// (one 4- or 8-byte device-scope load each), all issued before the barrier:
// one round trip.
// (A first form had every thread load m, l and o of kInBatch clamped chunks
// for each of its outputs, 96 loads per thread; its merge cost about 3 us of
// an 8 x 32Q/8KV call at 32767 tokens.)
constexpr int kInBatch = 16;    // merge_kernel's batch
constexpr int kInParts = 8;     // vsum_merge_kernel's parts

// pu: the partials of the unit's first q head (head h, chunk c at
// (h * nb + c) * (D + 2): m, l, o[D]); stage: LDS, 2 * kInBatch floats per
// head; G q heads; outputs ou[G][D]; P adjacent outputs per thread (1 where
// G * D <= nthreads, else 2).  Every thread of the block calls it (it holds
// a barrier).
template <int D, bool VS, int P>
__device__ __forceinline__ void merge_unit_p(const float *pu, int nb, int n_chunks, int G,
                                             float *stage, float *ou, int tid)
{
    const bool has = P * tid < G * D;
    const int h = has ? P * tid / D : 0, dim = P * tid % D;
    const float *ph = pu + (int64_t)h * nb * (D + 2) + 2 + dim;
    // the (m, l) pair of (head, chunk) k = tid (G * n_chunks <= nthreads),
    // then the o values: unconditional, clamped to the last chunk, no branch
    // between the loads (entries past the last chunk hold its values); the
    // pair goes to LDS once its load is in, the o loads still in flight
    const bool stg = tid < G * n_chunks;
    const int sh = stg ? tid / n_chunks : 0, sc = stg ? tid % n_chunks : 0;
    const float2 ml = ld_dev2(pu + ((int64_t)sh * nb + sc) * (D + 2));
    float ov[kInBatch][P];
#pragma unroll
    for (int j = 0; j < kInBatch; j++) {
        const float *pj = ph + min(j, n_chunks - 1) * (D + 2);
        if constexpr (P == 2) {
            const float2 v = ld_dev2(pj);
            ov[j][0] = v.x;
            ov[j][1] = v.y;
        } else {
            ov[j][0] = ld_dev(pj);
        }
    }
    if (stg) {
        stage[sh * 2 * kInBatch + sc] = ml.x;
        stage[sh * 2 * kInBatch + kInBatch + sc] = ml.y;
    }
    __syncthreads();
    if (!has) return;
    // every staged (m, l) of the head into registers at once (16-byte LDS
    // reads; entries past the last chunk are not used or are replaced by
    // the last chunk's l), so the selects below need no LDS round trips
    const float4 *m4 = reinterpret_cast<const float4 *>(stage + h * 2 * kInBatch);
    float mv[kInBatch], lv[kInBatch];
#pragma unroll
    for (int q = 0; q < kInBatch / 4; q++) {
        const float4 a = m4[q], b = m4[kInBatch / 4 + q];
        mv[4 * q] = a.x; mv[4 * q + 1] = a.y; mv[4 * q + 2] = a.z; mv[4 * q + 3] = a.w;
        lv[4 * q] = b.x; lv[4 * q + 1] = b.y; lv[4 * q + 2] = b.z; lv[4 * q + 3] = b.w;
    }
    float r[P];
    if constexpr (!VS) {
        // softmax merge: M = max(-1e6 log2(e), m_c), l = sum l_c 2^(m_c - M),
        // o = sum o_c 2^(m_c - M), out = o * (1/l); the batch's entries past
        // the last chunk repeat the last chunk's l and o with weight 0
        const float M = -1000000.0f * EAKV_LOG2E;
        float Mn = M, lt = 0.0f, o[P];
#pragma unroll
        for (int e = 0; e < P; e++) o[e] = 0.0f;
#pragma unroll
        for (int j = 0; j < kInBatch; j++) Mn = j < n_chunks ? fmaxf(Mn, mv[j]) : Mn;
        const float f = __builtin_amdgcn_exp2f(M - Mn);
        lt *= f;
#pragma unroll
        for (int e = 0; e < P; e++) o[e] *= f;
        const float llast = stage[h * 2 * kInBatch + kInBatch + n_chunks - 1];
#pragma unroll
        for (int j = 0; j < kInBatch; j++) {
            const bool in = j < n_chunks;
            const float wj = in ? __builtin_amdgcn_exp2f(mv[j] - Mn) : 0.0f;
            lt = fmaf(in ? lv[j] : llast, wj, lt);
#pragma unroll
            for (int e = 0; e < P; e++) o[e] = fmaf(ov[j][e], wj, o[e]);
        }
#pragma unroll
        for (int e = 0; e < P; e++) r[e] = o[e] * (1.0f / lt);
    } else {
        // V-sum: the plain sum of o_c in 8 strided parts (chunks pt, pt + 8)
        // added in part order, NaN when a chunk's l is NaN (a non-finite
        // weight)
        float t[P], fl = 0.0f;
#pragma unroll
        for (int e = 0; e < P; e++) t[e] = 0.0f;
#pragma unroll
        for (int pt = 0; pt < kInParts; pt++) {
            float sm[P], bad = 0.0f;
#pragma unroll
            for (int e = 0; e < P; e++) sm[e] = 0.0f;
#pragma unroll
            for (int c = pt; c < kInBatch; c += kInParts) {
                const bool in = c < n_chunks;
#pragma unroll
                for (int e = 0; e < P; e++) sm[e] = in ? __fadd_rn(sm[e], ov[c][e]) : sm[e];
                bad = in ? bad + lv[c] : bad;     // 0, or NaN after a non-finite weight
            }
#pragma unroll
            for (int e = 0; e < P; e++) t[e] = pt == 0 ? sm[e] : __fadd_rn(t[e], sm[e]);
            fl = pt == 0 ? bad : fl + bad;
        }
#pragma unroll
        for (int e = 0; e < P; e++) r[e] = fl == fl ? t[e] : fl;
    }
#pragma unroll
    for (int e = 0; e < P; e++) ou[h * D + dim + e] = r[e];
}

template <int D, bool VS>
__device__ __forceinline__ void merge_unit(const float *pu, int nb, int n_chunks, int G,
                                           float *stage, float *ou, int tid, int nthreads)
{
    if (G * D <= nthreads) merge_unit_p<D, VS, 1>(pu, nb, n_chunks, G, stage, ou, tid);
    else merge_unit_p<D, VS, 2>(pu, nb, n_chunks, G, stage, ou, tid);
}

// Tile assignment: nb = gridDim.x blocks share one (sequence, kv head), a
// "unit" of n_tiles TT-token tiles, dealt round robin: tile j to block
// (j / kWaves) % nb and wave j % kWaves.  At any time the waves of a unit
// read one contiguous window of every plane, and a wave's tiles are
// nb * kWaves tiles apart.  Softmax partials do not depend on which tokens a
// wave sees.  Each block writes its partial (m, l, o[D]) per q head of its
// kv head; merge_kernel combines the blocks.
//
// A wave serves the G = qpk <= 4 HH q heads of its (virtual) kv head as HH
// quads of four heads: each quad has its own q digits (K MFMA rows), softmax
// state, digit rows and V MFMAs; the K bytes, the V tile in LDS and the
// nibbles taken from them are shared, so the planes are read once for all G
// heads (once per virtual kv head when a group above 8 is split).
//
// VS: the V-sum of the unfused API, o = sum_t w[h][t] v[t] with the weights
// given (q points to w[n_q][L] of one sequence).  No K, no softmax: each
// tile's weights are loaded in place of its K bytes and go straight to the
// digit rows (signed fixed point, the exponent from the largest |a|); m
// stays 0, vsum_merge_kernel adds the chunks unnormalised, and a non-finite
// weight makes its head's output NaN (lsum carries the flag).
template <int D, int HH, bool VS, int TT>
__global__ __launch_bounds__(64 * kWavesH<HH>, (kWavesH<HH> * kBlocksPerCUH<D, HH> / 4)) void mfma_kernel(
    eakvd_geom g, eakvd_batch bt, int layer, const float *__restrict__ q,
    int n_q, int qpk, float rs, float *__restrict__ part, int split,
    float *__restrict__ out, uint8_t *__restrict__ ctr, int lead)
{
    constexpr int GPD = D / 64;
    constexpr int NK = Geo<D, TT>::NK;
    constexpr int NH = Geo<D, TT>::NH;                  // 32-token halves
    // VGPR loads per group after the V and scale loads: K bytes, or weights
    constexpr int NKL = VS ? NK * HH : kNK<D, TT>;
    using StageT = std::conditional_t<VS, WStage<D, HH, TT>, Stage<D, TT>>;
    constexpr int NW = kWavesH<HH>;                     // waves per block
    // Per wave: kSlots V and scale slots and the digit rows of its HH
    // quads; after the tiles the wave's V slots 0 (and 1) hold its outputs
    // o[4][D] of quad 0 (and 1) and its digit rows its m[8], l[8] for the
    // block merge.  Every slot is its own variable: the
    // compiler then knows that a load into one slot does not write another
    // and does not make reads of a slot wait for younger loads to LDS.
    static_assert(Geo<D, TT>::VSLOT >= 4 * D * 4, "outputs fit a V slot");
    static_assert(HH == 1 || HH == 2, "one or two quads");
    static_assert(kSlots == 2, "two slot variables");
    __shared__ __attribute__((aligned(16))) uint8_t v_lds0[NW][Geo<D, TT>::VSLOT];
    __shared__ __attribute__((aligned(16))) uint8_t v_lds1[NW][Geo<D, TT>::VSLOT];
    __shared__ __attribute__((aligned(16))) float s_lds0[NW][Geo<D, TT>::SSLOT];
    __shared__ __attribute__((aligned(16))) float s_lds1[NW][Geo<D, TT>::SSLOT];
    __shared__ __attribute__((aligned(16))) uint8_t z_lds[NW][HH * Geo<D, TT>::ZROWS * 8];

    const int ch = blockIdx.x, nb = gridDim.x, kvh = blockIdx.y, s = blockIdx.z;
    const int L = bt.seq_len[s];
    const int n_tiles = (L + TT - 1) / TT;
    if (ch * NW >= n_tiles) {         // no tile for this block: no partial
        // merged here, an empty sequence's outputs are 0 * (1/0) = NaN, as
        // the reference's (and merge_kernel's)
        if constexpr (!VS)
            if (ctr && n_tiles == 0 && ch == 0) {
                const float zl = 0.0f, zo = 0.0f;
                for (int i = threadIdx.x; i < qpk * D; i += 64 * NW)
                    out[((int64_t)s * n_q + (int64_t)kvh * qpk) * D + i] = zo * (1.0f / zl);
            }
        return;
    }
    // the wave index is wave-uniform: say so, so that every per-wave
    // quantity (token range, tile offsets) stays in scalar registers
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = qpk;                                  // 1..4 HH
    const int first = ch * NW + w;                      // this wave's first tile
    const int stride = nb * NW;                         // tiles between its tiles
    const Planes K = planes_of(g, bt.base[s], layer, 0);
    const Planes V = planes_of(g, bt.base[s], layer, 1);
    // split > 1: blockIdx.y is one of `split` virtual kv heads of qpk q heads
    // each that share kv head kvh / split (more than 8 q heads per kv head)
    const int64_t hbase = (int64_t)(kvh / split) * g.gph;
    const float *qs = q + ((int64_t)s * n_q + (int64_t)kvh * qpk) * D;

    // ---- q -> A operands of K.  Lane l: row i = l%16 (head ha = i/4, digit
    // pa = i%4), k-block qq = l/16; k-slot j of group gg holds dim
    // 64gg + 8qq + j (j < 8, low nibbles) or 64gg + 32 + 8qq + (j-8).
    // Quad hq holds heads 4hq..4hq+3.  Rows of heads >= G are zero (their q
    // is read from head 0 and dropped).  Every wave of the block serves the
    // same heads, so wave hq alone computes quad hq's operands and shares
    // them through LDS.  The q loads are issued first, then the first load
    // groups (further below), so the digit arithmetic waits only for q.
    const int ha = (l & 15) >> 2, pa = l & 3, qq = l >> 4;
    bool qrow[HH];
    float qv[HH][GPD][16];
    if constexpr (!VS)
#pragma unroll
    for (int hq = 0; hq < HH; hq++) {
        qrow[hq] = 4 * hq + ha < G;
        if (w != hq) continue;
        const float4 *qh4 = (const float4 *)(qs + (qrow[hq] ? 4 * hq + ha : 0) * D);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
#pragma unroll
            for (int h2 = 0; h2 < 2; h2++)
#pragma unroll
                for (int v4 = 0; v4 < 2; v4++) {
                    const float4 f = qh4[(64 * gg + 32 * h2 + 8 * qq) / 4 + v4];
                    float *d = &qv[hq][gg][8 * h2 + 4 * v4];
                    d[0] = f.x; d[1] = f.y; d[2] = f.z; d[3] = f.w;
                }
    }
    __builtin_amdgcn_sched_barrier(0);
    // score layout: this lane receives the scores of head 4hq + ho of each
    // quad for token tl
    const int ho = l >> 4, tl = l & 15;
    bool live[HH];
#pragma unroll
    for (int hq = 0; hq < HH; hq++) live[hq] = 4 * hq + ho < G;

    LaneOffs P;
    // V-sum: the weight rows of the kv head (unused otherwise)
    const __amdgpu_buffer_rsrc_t wr = plane_rsrc(
        q + (VS ? (int64_t)kvh * qpk * L : 0), VS ? (int64_t)qpk * L * 4 : 0);
    uint32_t wo[HH];
    {
        const int64_t wbytes = g.max_groups * 32;
        P.kw = plane_rsrc(K.w, wbytes);
        P.vw = plane_rsrc(V.w, wbytes);
        // K and V blocks of the layer are adjacent: one resource for the
        // scale and bias planes of both
        P.layer = plane_rsrc(K.w, 2 * g.block_bytes);
        // scale load i: lane l fetches bytes 16e.. of plane pl's tile
        // (V-sum: only the V planes; lanes of the K planes fetch them again)
        constexpr int LP = Geo<D, TT>::LP;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int pl = (((64 * i + l) / LP) & 3) | (VS ? 2 : 0);
            const int e = l % LP;
            const int64_t poff = (pl & 2 ? g.block_bytes : 0) + (pl & 1 ? g.b_off : g.s_off);
            P.sco[i] = (uint32_t)(poff + hbase * 4 + 16 * e);
        }
        P.kwo = (uint32_t)((hbase + (int64_t)tl * GPD) * 32 + qq * 8);
        // V load: lane l's 16 bytes land at unit l of the first 1 KB of the
        // slot: token t = l / UPT, unit (l % UPT) of the permuted row
        const int vt = l / Geo<D, TT>::UPT;
        const int vu = (l % Geo<D, TT>::UPT) ^ vswz<D>(vt);
        P.vwo = (uint32_t)(hbase * 32 + vt * Geo<D, TT>::RB + 16 * vu);
        if constexpr (VS) {
            // lane (ho, tl): row kvh*qpk + 4hq + ho (head 0 past the group), token tl
#pragma unroll
            for (int hq = 0; hq < HH; hq++)
                wo[hq] = (uint32_t)((live[hq] ? 4 * hq + ho : 0) * L * 4);
        }
    }

    // LDS read/write offsets of this lane (wave-relative, bytes).
    //   vrd: the row it supplies to a transposed V read of column block
    //        (g, half): token vtok(kq, r'/2) of its lane group kq, bytes
    //        8(r'%2).. of the block's 16-byte unit (r' = l%16).
    //   zrd: the digit row it supplies: row (g, hp = r'%2, token vtok(kq, r'/2)).
    //   zwr: where its digits land: row (g, ho/2, token 16k + tl), dword ho%2.
    // Digit rows are 8 bytes, [g][hp][token]; row (g, hp, t) holds the digit
    // words of heads 2hp and 2hp+1.
    const int kq = l >> 4, rr = l & 15;
    uint32_t vrd[GPD][2], zrd, zwr;
    {
        const int t = vtok(kq, rr >> 1);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
#pragma unroll
            for (int half = 0; half < 2; half++)
                vrd[gg][half] = (uint32_t)(t * Geo<D, TT>::RB +
                                           16 * ((2 * gg + half) ^ vswz<D>(t)) + 8 * (rr & 1));
        zrd = (uint32_t)(((rr & 1) * TT + t) * 8);
        zwr = (uint32_t)(((ho >> 1) * TT + tl) * 8 + 4 * (ho & 1));
    }
    uint8_t *zb = z_lds[w];
    // slot k of this wave (k a constant)
    auto vslot = [&](auto kc) -> uint8_t * {
        constexpr int k = decltype(kc)::value;
        if constexpr (k == 0) return v_lds0[w];
        else return v_lds1[w];
    };
    auto sslot = [&](auto kc) -> float * {
        constexpr int k = decltype(kc)::value;
        if constexpr (k == 0) return s_lds0[w];
        else return s_lds1[w];
    };
    using I0 = std::integral_constant<int, 0>;

    // Tile schedule: tk[j] = T(i + j) = first + (i + j) * stride, the
    // wave's tiles from the current one on.
    int tk[kSlots + 1];
#pragma unroll
    for (int j = 0; j < kSlots; j++) tk[j] = first + j * stride;
    // token offset of a tile for loads: past-the-end tiles re-read the
    // unit's last tile (in bounds; their scores are masked)
    auto ldt = [&](int t) { return min(t, n_tiles - 1) * TT; };
    // Past-the-end tiles are also read out of range (a lane offset beyond
    // every plane: the loads return 0 at once, with no memory request), so
    // a wave's last groups, never consumed except as masked tokens, do not
    // hold up its epilogue.  The tile offset stays clamped in range.
    auto oob = [&](int t) -> uint32_t { return t >= n_tiles ? 0x80000000u : 0u; };

    StageT st[kSlots];
    // group j: V of tile T(j-1) into V slot (j-1) % kSlots, then the scales
    // and K bytes of tile T(j) into scale slot and stage j % kSlots
    auto load_group = [&](auto jc, int tv, int tkk) {
        constexpr int j = decltype(jc)::value;
        load_v<D, TT>(vslot(std::integral_constant<int, (j + kSlots - 1) % kSlots>{}), P, ldt(tv),
                      oob(tv));
        __builtin_amdgcn_sched_barrier(0);
        load_scales<D, TT>(sslot(std::integral_constant<int, j % kSlots>{}), P, ldt(tkk), oob(tkk));
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (VS) load_w<D, HH, TT>(st[j % kSlots], wr, wo, ldt(tkk), tl, L);
        else load_k<D, TT>(st[j % kSlots], P, ldt(tkk), oob(tkk));
        __builtin_amdgcn_sched_barrier(0);
    };
    // Unconditional (a wave without tiles reads the unit's last tile), so
    // the waits below count the same younger loads on every path.  One quad
    // per wave: group 1 follows at once; two quads: once group 0 has landed
    // (after the q digits, below).  Group 0 has no V tile; in its place one
    // 256-byte load of tile T(0)'s V bytes (fetched again by group 1, so no
    // extra memory traffic) goes to the V slot that iteration 0 fills.  It
    // makes the prologue load every V slot in the loop's order, which keeps
    // the compiler's wait placement at the loop head as tight as inside the
    // loop.
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        P.vw, (lds_ptr)vslot(std::integral_constant<int, kSlots - 1>{}), 4,
        (int)(P.vwo + oob(tk[0])),
        (int)((uint32_t)__builtin_amdgcn_readfirstlane(ldt(tk[0])) * GPD * 32), 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_scales<D, TT>(sslot(I0{}), P, ldt(tk[0]), oob(tk[0]));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (VS) load_w<D, HH, TT>(st[0], wr, wo, ldt(tk[0]), tl, L);
    else load_k<D, TT>(st[0], P, ldt(tk[0]), oob(tk[0]));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (HH == 1) load_group(std::integral_constant<int, 1>{}, tk[0], tk[1]);

    // scores are kept in the log2 domain (times log2(e))
    const float rs2 = rs * EAKV_LOG2E;
    v4i A[HH][GPD];
    float kwl[HH], kwh[HH], bq[HH][GPD];
    if constexpr (!VS)
#pragma unroll
    for (int hq = 0; hq < HH; hq++) {
    if (w != hq) continue;
    float amax = 0.0f;
    float qsum[GPD];
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) {
        double sum = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            qv[hq][gg][j] = qrow[hq] ? qv[hq][gg][j] : 0.0f;
            amax = fmaxf(amax, fabsf(qv[hq][gg][j]));
            sum += (double)qv[hq][gg][j];
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
    const uint32_t dsh = 8 * (3 - pa);
#pragma unroll
    for (int gg = 0; gg < GPD; gg++)
#pragma unroll
        for (int w4 = 0; w4 < 4; w4++) {
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int z = (int)rintf(ldexpf(qv[hq][gg][4 * w4 + b], esh));
                const uint32_t u = (uint32_t)z + 0x80808080u;
                word |= ((u >> dsh) & 0xffu) << (8 * b);
            }
            A[hq][gg][w4] = (int)(word ^ 0x80808080u);
        }

    const int esh_o = __shfl(esh, 4 * ho, 64);
    kwl[hq] = ldexpf(rs2, -esh_o);
    kwh[hq] = ldexpf(rs2, 16 - esh_o);
#pragma unroll
    for (int gg = 0; gg < GPD; gg++) bq[hq][gg] = rs2 * __shfl(qsum[gg], 4 * ho, 64);
    }
    if constexpr (!VS) {
        // quad hq's operands of lane l: dwords (hq*QR + f)*64 + l of the
        // digit rows, which no wave uses before its first tile's weights
        constexpr int QR = GPD * 4 + 2 + GPD;
        static_assert(HH * QR * 64 * 4 <= (int)sizeof(z_lds), "operands fit the digit rows");
        uint32_t *xq = reinterpret_cast<uint32_t *>(&z_lds[0][0]);
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            if (w != hq) continue;
            uint32_t *x = xq + hq * QR * 64 + l;
#pragma unroll
            for (int gg = 0; gg < GPD; gg++)
#pragma unroll
                for (int w4 = 0; w4 < 4; w4++) x[(gg * 4 + w4) * 64] = (uint32_t)A[hq][gg][w4];
            x[GPD * 4 * 64] = __float_as_uint(kwl[hq]);
            x[(GPD * 4 + 1) * 64] = __float_as_uint(kwh[hq]);
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) x[(GPD * 4 + 2 + gg) * 64] = __float_as_uint(bq[hq][gg]);
        }
        __syncthreads();
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            if (w == hq) continue;
            const uint32_t *x = xq + hq * QR * 64 + l;
#pragma unroll
            for (int gg = 0; gg < GPD; gg++)
#pragma unroll
                for (int w4 = 0; w4 < 4; w4++) A[hq][gg][w4] = (int)x[(gg * 4 + w4) * 64];
            kwl[hq] = __uint_as_float(x[GPD * 4 * 64]);
            kwh[hq] = __uint_as_float(x[(GPD * 4 + 1) * 64]);
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) bq[hq][gg] = __uint_as_float(x[(GPD * 4 + 2 + gg) * 64]);
        }
        // every wave has its operands before any wave writes digit rows
        __syncthreads();
    }

    // Two quads: group 1 once group 0 has landed.  Every wave of the chip
    // issues its first group at the start; holding the second back until the
    // first is in lets the first groups arrive first, so waves start on their
    // first tiles sooner and leave the start in step less (64Q/8KV d128:
    // 34.1 against 35.35 us per call at 131072 tokens, 13.25 against 13.95
    // at 20000).  One-quad waves, with half the arithmetic per tile, gained
    // nothing at 32Q/8KV 32K x 8 and lost 0.25 us at 32Q/4KV d64 4K (two
    // tiles per wave).
    // Two quads (8-wave blocks, 2 waves per SIMD): waves 4-7 share their
    // SIMDs with the older waves 0-3 and lead them for the first half of
    // their own tiles, as the second round of one-quad blocks does below
    // (64Q/8KV d128 128K: 34.16-34.18 against 34.73-34.75 us per call,
    // alternating whole bench runs).  Set before group 1, so that group's
    // block runs on into the first wait that counts it.
    int lead_left = 0;
    if constexpr (HH == 2)
        if (w >= NW / 2) {
            lead_left = ((n_tiles - first + stride - 1) / stride + 1) / 2;
            if (lead_left > 0) __builtin_amdgcn_s_setprio(1);
        }
    if constexpr (HH == 2) {
        wait_vm<0>();
        load_group(std::integral_constant<int, 1>{}, tk[0], tk[1]);
    }

    WaveState<D> S[HH];
#pragma unroll
    for (int hq = 0; hq < HH; hq++) {
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) {
            S[hq].acc[gg][0][0] = S[hq].acc[gg][0][1] = 0.0f;
            S[hq].acc[gg][1][0] = S[hq].acc[gg][1][1] = 0.0f;
            S[hq].bacc[gg] = 0.0f;
            S[hq].wh[gg] = S[hq].wl[gg] = 0.0f;
        }
        S[hq].lsum = 0.0f;
        S[hq].m = VS ? 0.0f : -INFINITY;
    }

    // The weights of one tile from its scores and the running max m:
    // p = 2^(sc - m) (0 for heads >= G), psum = sum p, bi = sum p*bias per
    // group, and a = p*scale per group as fixed point z = trunc(a * 2^E)
    // with E = 30 - (exponent of the tile's largest a of the head and
    // group), so 0 <= z < 2^30.  The balanced digits of z go to the digit
    // rows; wh/wl are 2^(16-E) and 2^-E.
    auto weights = [&](auto hqc, const Scales<D, TT> &C, const float *sc, float m, float &psum,
                       float *bi) {
        constexpr int hq = decltype(hqc)::value;
        WaveState<D> &Sq = S[hq];
        uint8_t *zq = zb + hq * Geo<D, TT>::ZROWS * 8;
        float p[NK];
        psum = 0.0f;
#pragma unroll
        for (int k = 0; k < NK; k++) {
            // V-sum: sc holds the tile's (masked) weights
            if constexpr (VS) p[k] = sc[k];
            else p[k] = live[hq] ? __builtin_amdgcn_exp2f(sc[k] - m) : 0.0f;
            psum += p[k];
        }
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) {
            float a[NK], am = 0.0f;
            bi[gg] = 0.0f;
#pragma unroll
            for (int k = 0; k < NK; k++) {
                a[k] = mul_zero(p[k], C.vs[k][gg]);
                bi[gg] += mul_zero(p[k], C.vb[k][gg]);
                am = max_pos(am, VS ? fabsf(a[k]) : a[k]);
            }
            am = row_max16_pos(am);
            const int E = 30 - __builtin_amdgcn_frexp_expf(am);
#pragma unroll
            for (int k = 0; k < NK; k++) {
                const int z = (int)__builtin_amdgcn_ldexpf(a[k], E);
                const uint32_t u = ((uint32_t)z + 0x80808080u) ^ 0x80808080u;
                *(uint32_t *)(zq + zwr + gg * 2 * TT * 8 + k * 16 * 8) = u;
            }
            Sq.wl[gg] = __builtin_amdgcn_ldexpf(1.0f, -E);
            Sq.wh[gg] = __builtin_amdgcn_ldexpf(1.0f, 16 - E);
        }
    };

    // The tile's softmax bookkeeping for every quad.  Lazy rescale: a
    // head's running max moves only when a score exceeds it by more than
    // kTau (so p <= 2^kTau).  One ballot over all quads: in the common case
    // (no lane needs a move) the code runs straight through both quads'
    // weights; otherwise (rare: the first tile, a new larger score) the
    // moved maxima are set and the accumulators scaled by 2^(old - new)
    // first.
    auto softmax = [&](const Scales<D, TT> &C, float (*sc)[NK]) {
        bool need[HH];
        float mt[HH];
        bool any = false;
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            mt[hq] = sc[hq][0];
#pragma unroll
            for (int k = 1; k < NK; k++) mt[hq] = fmaxf(mt[hq], sc[hq][k]);
            need[hq] = live[hq] && mt[hq] - S[hq].m > kTau;
            any = any || need[hq];
        }
        if (__builtin_amdgcn_ballot_w64(any) != 0) {
#pragma unroll
            for (int hq = 0; hq < HH; hq++) {
                WaveState<D> &Sq = S[hq];
                const float rm = row_max16(mt[hq]);
                const float mn = live[hq] && rm > Sq.m + kTau ? rm : Sq.m;
                const float f = live[hq] ? __builtin_amdgcn_exp2f(Sq.m - mn) : 1.0f;
                Sq.m = mn;
                Sq.lsum *= f;
#pragma unroll
                for (int gg = 0; gg < GPD; gg++) {
                    Sq.bacc[gg] *= f;
                    Sq.acc[gg][0][0] *= f;
                    Sq.acc[gg][0][1] *= f;
                    Sq.acc[gg][1][0] *= f;
                    Sq.acc[gg][1][1] *= f;
                }
            }
        }
        float psum[HH], bi[HH][GPD];
        weights(std::integral_constant<int, 0>{}, C, sc[0], S[0].m, psum[0], bi[0]);
        if constexpr (HH > 1)
            weights(std::integral_constant<int, 1>{}, C, sc[1], S[1].m, psum[1], bi[1]);
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            S[hq].lsum += psum[hq];
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) S[hq].bacc[gg] += bi[hq][gg];
        }
    };

    // K(tile at dt) from its stage and scale slot: the scores of the tile
    // for every quad, then each quad's softmax.
    auto kscores_softmax = [&](const Stage<D, TT> &T, const Scales<D, TT> &C, int dt) {
        float sc[HH][NK];
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            v4i dk[NK][GPD];
            k_mfma<D, TT>(T, A[hq], dk);
#pragma unroll
            for (int k = 0; k < NK; k++)
                sc[hq][k] = k_recomb<D, TT>(C, dk[k], k, dt, L, kwh[hq], kwl[hq], bq[hq], tl);
        }
        softmax(C, sc);
    };

    // V-sum: the weights of the tile at dt (past the sequence and for heads
    // past the group: 0) to the digit rows, sum w*bias per (head, group) to
    // bacc; a non-finite weight sets the head's lsum to NaN.
    auto vs_weights = [&](const auto &T, const Scales<D, TT> &C, int dt) {
        float pw[HH][NK];
        bool bad[HH];
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            bad[hq] = false;
#pragma unroll
            for (int k = 0; k < NK; k++) {
                const bool in = live[hq] && dt + 16 * k + tl < L;
                pw[hq][k] = in ? T.wv[hq][k] : 0.0f;
                bad[hq] = bad[hq] || !(fabsf(pw[hq][k]) <= 3.40282347e38f);
            }
        }
        float psum, bi[GPD];
        weights(std::integral_constant<int, 0>{}, C, pw[0], 0.0f, psum, bi);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) S[0].bacc[gg] += bi[gg];
        if constexpr (HH > 1) {
            weights(std::integral_constant<int, 1>{}, C, pw[1], 0.0f, psum, bi);
#pragma unroll
            for (int gg = 0; gg < GPD; gg++) S[1].bacc[gg] += bi[gg];
        }
#pragma unroll
        for (int hq = 0; hq < HH; hq++)
            if (bad[hq]) S[hq].lsum = __builtin_nanf("");
    };

    // V(tile in vslot) with the digits in the digit rows: the transposed
    // reads (vread; NH per operand, one per 32-token half, bytes 8h..8h+7 of
    // a lane's operand from half h), then the 4*GPD MFMA pairs, then their
    // recombination, so the MFMA latency is covered by the MFMAs behind it
    // (vsum).
    struct VRead {
        v2i az[HH][GPD][NH], x[GPD][2][NH];
    };
    auto vread = [&](const uint8_t *vslot, VRead &R) {
#pragma unroll
        for (int hq = 0; hq < HH; hq++)
#pragma unroll
            for (int gg = 0; gg < GPD; gg++)
#pragma unroll
                for (int h = 0; h < NH; h++)
                    R.az[hq][gg][h] = tr8(zb + hq * Geo<D, TT>::ZROWS * 8 + zrd +
                                          gg * 2 * TT * 8 + h * 32 * 8);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int h = 0; h < NH; h++)
                    R.x[gg][half][h] = tr8(vslot + vrd[gg][half] + h * 32 * Geo<D, TT>::RB);
    };
    // the MFMA of one operand pair: 32 tokens (8 bytes per lane) or 64 (16)
    auto vmfma = [](const v2i *a, const v2i *b) -> v4i {
        if constexpr (NH == 1)
            return __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a[0]), as_long(b[0]),
                                                         v4i{0, 0, 0, 0}, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i{a[0][0], a[0][1], a[1][0], a[1][1]},
                                                         v4i{b[0][0], b[0][1], b[1][0], b[1][1]},
                                                         v4i{0, 0, 0, 0}, 0, 0, 0);
    };
    auto vsum = [&](const VRead &R) {
        const auto &x = R.x;
        v2i lo[GPD][2][NH], hi[GPD][2][NH];
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int h = 0; h < NH; h++) {
                    lo[gg][half][h] = v2i{(int)nib_lo(x[gg][half][h][0]),
                                          (int)nib_lo(x[gg][half][h][1])};
                    hi[gg][half][h] = v2i{(int)nib_hi(x[gg][half][h][0]),
                                          (int)nib_hi(x[gg][half][h][1])};
                }
#pragma unroll
        for (int hq = 0; hq < HH; hq++) {
            const auto &az = R.az[hq];
            v4i c[GPD][2][2];
#pragma unroll
            for (int gg = 0; gg < GPD; gg++)
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    c[gg][half][0] = vmfma(az[gg], lo[gg][half]);
                    c[gg][half][1] = vmfma(az[gg], hi[gg][half]);
                }
            WaveState<D> &Sq = S[hq];
#pragma unroll
            for (int gg = 0; gg < GPD; gg++)
#pragma unroll
                for (int half = 0; half < 2; half++)
#pragma unroll
                    for (int lh = 0; lh < 2; lh++)
                        Sq.acc[gg][half][lh] = v_recomb(c[gg][half][lh], Sq.wh[gg], Sq.wl[gg],
                                                        Sq.acc[gg][half][lh]);
        }
    };

    // Software pipeline over the wave's tiles.  Load group j holds the V
    // bytes of tile T(j-1) and the K bytes and scales of tile T(j).
    // Iteration i waits for group i+1, reads V(T(i)) and the digits written
    // by the previous iteration from LDS, issues group i+kSlots, then runs
    // V(T(i)) and K(T(i+1)) with its softmax (digits of T(i+1)).  kSlots-1
    // groups stay in flight behind the one consumed (rotating registers and
    // LDS slots).
    constexpr int kGrp = Geo<D, TT>::NVD + kDma<D, TT> + NKL;   // loads per group
    constexpr int kLater = (kSlots - 1) * kGrp;         // loads of the groups after the oldest
    constexpr int kEarly = (kSlots - 2) * kGrp;
    // lead > 0 (one-quad waves): the grid holds two blocks per CU, dealt one
    // per CU in each of two dispatch rounds (blocks in linear order), and on
    // each SIMD the older wave wins issue, so the first round's blocks would
    // run ahead and the second's finish alone at half the CU's rate.  The
    // second round's waves issue first for their first `lead` tiles (half of
    // them), then give way.  Priority changes no arithmetic.
    if constexpr (HH == 1)
        if (lead > 0 &&
            2 * (int)((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) >=
                (int)(gridDim.x * gridDim.y * gridDim.z)) {
            lead_left = lead;
            __builtin_amdgcn_s_setprio(1);
        }
    if (tk[0] < n_tiles) {
        {
            Scales<D, TT> C;
            // group 0 (scales, K of T(0)) is complete once at most its K
            // loads and all later groups are outstanding
            wait_vm<NKL + kLater>();
            read_scales<D, TT>(sslot(I0{}), tl, C);
            if constexpr (VS) vs_weights(st[0], C, tk[0] * TT);
            else kscores_softmax(st[0], C, tk[0] * TT);
        }
        // iteration i = r (mod kSlots)
        auto iter = [&](auto rc) {
            constexpr int r = decltype(rc)::value;
            // V(T(i)): its loads were the first of group i+1
            wait_vm<kDma<D, TT> + NKL + kEarly>();
            VRead R;
            vread(vslot(rc), R);
            tk[kSlots] = tk[kSlots - 1] + stride;
            __builtin_amdgcn_sched_barrier(0);
            load_group(std::integral_constant<int, r + kSlots>{}, tk[kSlots - 1], tk[kSlots]);
            vsum(R);
            // K(T(i+1)): scales, then bytes (the compiler waits for those).
            // Past the unit's last tile there is none: its scores would all
            // be masked (weights 0, no state change), so the wave's last
            // iteration ends with V(T(i)).
            wait_vm<NKL + kLater>();
            const bool more = tk[1] < n_tiles;
            if (more) {
                Scales<D, TT> C;
                read_scales<D, TT>(sslot(std::integral_constant<int, (r + 1) % kSlots>{}), tl, C);
                if constexpr (VS) vs_weights(st[(r + 1) % kSlots], C, tk[1] * TT);
                else kscores_softmax(st[(r + 1) % kSlots], C, tk[1] * TT);
            }
#pragma unroll
            for (int j = 0; j < kSlots; j++) tk[j] = __builtin_amdgcn_readfirstlane(tk[j + 1]);
            if (lead_left > 0 && --lead_left == 0) __builtin_amdgcn_s_setprio(0);
            return more;
        };
        // The explicit waits above count the loads of every group in issue
        // order, so each group's register loads must stay in the iteration
        // that issues them.  The V-sum's weight loads, used only by the next
        // iteration, were sunk by the compiler into that iteration's block
        // (past the waits that count them, so a scale slot was read before
        // its load had landed); using every weight stage on the exit path as
        // well keeps them where they are.  (The K loads stay in place; the
        // order of every loop block is checked on the compiled code by
        // tests/test_isa_order.py.)
        auto keep = [&]() {
            if constexpr (VS)
#pragma unroll
                for (int j = 0; j < kSlots; j++)
#pragma unroll
                    for (int hq = 0; hq < HH; hq++)
#pragma unroll
                        for (int k = 0; k < NK; k++) asm volatile("" ::"v"(st[j].wv[hq][k]));
        };
        for (;;) {
            if (!iter(std::integral_constant<int, 0>{})) { keep(); break; }
            if (!iter(std::integral_constant<int, 1>{})) { keep(); break; }
        }
    }
    // loads into LDS still in flight (the clamped groups past the end) must
    // land before the block's LDS is reused or released
    wait_vm<0>();

    // ---- wave epilogue.  lsum and the bias sums over the 16 token lanes of
    // a head (score layout); lane l then holds head 4hq + l/16's bias sums,
    // as its V outputs are that head's.  Quad hq's o[4][D] goes to V slot hq
    // of the wave, m and l of head h to words h and 8 + h of its digit rows.
#pragma unroll
    for (int hq = 0; hq < HH; hq++) {
        WaveState<D> &Sq = S[hq];
        float(*o_lds)[D] = (float(*)[D])(hq == 0 ? v_lds0[w] : v_lds1[w]);
        Sq.lsum = row_sum16(Sq.lsum);
#pragma unroll
        for (int gg = 0; gg < GPD; gg++) Sq.bacc[gg] = row_sum16(Sq.bacc[gg]);
        const int n = l & 15, h = l >> 4;
#pragma unroll
        for (int gg = 0; gg < GPD; gg++)
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int lh = 0; lh < 2; lh++)
                    o_lds[h][64 * gg + 32 * lh + 16 * half + n] =
                        Sq.acc[gg][half][lh] + Sq.bacc[gg];
        if (tl == 0) {
            float *ml = (float *)z_lds[w];
            ml[4 * hq + ho] = Sq.m;
            ml[8 + 4 * hq + ho] = Sq.lsum;
        }
    }
    __syncthreads();

    // ---- merge the waves into this chunk's partial, two adjacent outputs
    // of one head per thread (their scale factors computed once)
    for (int i2 = tid; 2 * i2 < G * D; i2 += 64 * NW) {
        const int h = 2 * i2 / D, dim = 2 * i2 % D;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < NW; ww++) M = fmaxf(M, ((const float *)z_lds[ww])[h]);
        float lt = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int ww = 0; ww < NW; ww++) {
            const float *ml = (const float *)z_lds[ww];
            const float f = __builtin_amdgcn_exp2f(ml[h] - M);
            lt = fmaf(ml[8 + h], f, lt);
            const float *o = (const float *)(h < 4 ? v_lds0[ww] : v_lds1[ww]);
            const float2 ov = *reinterpret_cast<const float2 *>(o + (h & 3) * D + dim);
            o0 = fmaf(ov.x, f, o0);
            o1 = fmaf(ov.y, f, o1);
        }
        float *dst = part + (((int64_t)s * n_q + kvh * qpk + h) * nb + ch) * (D + 2);
        if (ctr) {
            st_dev2(dst + 2 + dim, o0, o1);
            if (dim == 0) st_dev2(dst, M, lt);
        } else {
            *reinterpret_cast<float2 *>(dst + 2 + dim) = make_float2(o0, o1);
            if (dim == 0) *reinterpret_cast<float2 *>(dst) = make_float2(M, lt);
        }
    }
    if (!ctr) return;

    // ---- the chunk merge in this launch: every thread's
    // partial stores are complete (vmcnt 0) before the barrier, and so
    // before the block counts itself on its unit's counter; the block that
    // counts last reads the unit's partials after it, merges them into out
    // and sets the counter back to zero (no other block of the launch
    // touches it again)
    const int n_chunks = min(nb, (n_tiles + NW - 1) / NW);   // blocks with a tile
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned *uc = reinterpret_cast<unsigned *>(
        ctr + ((int64_t)s * gridDim.y + kvh) * EAKVD_CTR_STRIDE);
    if (tid == 0)
        ((int *)z_lds[0])[0] = __hip_atomic_fetch_add(uc, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT) ==
                               (unsigned)(n_chunks - 1);
    __syncthreads();
    if (((const int *)z_lds[0])[0] == 0) return;
    if (tid == 0) __hip_atomic_store(uc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    static_assert(4 * HH * D / 2 <= 64 * NW && 4 * HH * kInBatch <= 64 * NW,
                  "one output pair and at most one (m, l) pair per thread");
    const int64_t qh0 = (int64_t)s * n_q + kvh * qpk;
    merge_unit<D, VS>(part + qh0 * nb * (D + 2), nb, n_chunks, G, &s_lds0[0][0],
                      out + qh0 * D, tid, 64 * NW);
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
    eakvd_batch bt, int n_q, int max_chunks, int wpb, int tt, const float *__restrict__ part,
    float *__restrict__ out)
{
    const int qh = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    // blocks that had a tile (see mfma_kernel; wpb waves per block, tt
    // tokens per tile)
    const int n_tiles = (bt.seq_len[s] + tt - 1) / tt;
    const int n_chunks = min(max_chunks, (n_tiles + wpb - 1) / wpb);
    const float *p = part + ((int64_t)s * n_q + qh) * max_chunks * (D + 2);
    // The (m, l) pair and o[i] of every chunk by vector buffer loads, all
    // issued before any arithmetic: one memory round trip.  (As scalar
    // loads the pairs overflow the scalar load counter, and the compiler's
    // early waits split them into several round trips.)
    const __amdgpu_buffer_rsrc_t r = plane_rsrc(p, (int64_t)max_chunks * (D + 2) * 4);
    float M = -1000000.0f * EAKV_LOG2E, lt = 0.0f, ot = 0.0f;
    for (int c0 = 0; c0 < n_chunks; c0 += kMergeBatch) {
        float m[kMergeBatch], lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
        for (int j = 0; j < kMergeBatch; j++) {
            const int so = min(c0 + j, n_chunks - 1) * (D + 2) * 4;
            const auto ml = __builtin_amdgcn_raw_buffer_load_b64(r, 0, so, 0);
            m[j] = __uint_as_float(ml[0]);
            lv[j] = __uint_as_float(ml[1]);
            ov[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4 * i, so + 8, 0));
        }
        __builtin_amdgcn_sched_barrier(0);
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

// The same merge for more than kMergeBatch chunks (long contexts): a block
// takes 32 dims of one (q head, sequence); thread (i, part) merges
// chunks part, part + 8, ... online, kPartBatch at a time with their loads
// in flight, and the 8 part results are merged in part order.  An empty
// sequence has no chunks: 0 * (1/0) = NaN, as the reference.
constexpr int kMergeParts = 8;
constexpr int kPartBatch = 8;

template <int D>
__global__ __launch_bounds__(256) void merge_parts_kernel(
    eakvd_batch bt, int n_q, int max_chunks, int wpb, int tt, const float *__restrict__ part,
    float *__restrict__ out)
{
    __shared__ float pm[kMergeParts], pl[kMergeParts], po[kMergeParts][32];
    const int qh = blockIdx.x / (D / 32), s = blockIdx.y;
    const int i = (blockIdx.x % (D / 32)) * 32 + (threadIdx.x & 31), pt = threadIdx.x >> 5;
    // blocks that had a tile (see mfma_kernel; wpb waves per block, tt
    // tokens per tile)
    const int n_tiles = (bt.seq_len[s] + tt - 1) / tt;
    const int n_chunks = min(max_chunks, (n_tiles + wpb - 1) / wpb);
    const float *p = part + ((int64_t)s * n_q + qh) * max_chunks * (D + 2);
    float M = -1000000.0f * EAKV_LOG2E, lt = 0.0f, ot = 0.0f;
    for (int c0 = pt; c0 < n_chunks; c0 += kMergeParts * kPartBatch) {
        float m[kPartBatch], lv[kPartBatch], ov[kPartBatch];
#pragma unroll
        for (int j = 0; j < kPartBatch; j++) {
            const float *pc = p + min(c0 + j * kMergeParts, n_chunks - 1) * (D + 2);
            m[j] = pc[0];
            lv[j] = pc[1];
            ov[j] = pc[2 + i];
        }
        float Mn = M;
#pragma unroll
        for (int j = 0; j < kPartBatch; j++)
            if (c0 + j * kMergeParts < n_chunks) Mn = fmaxf(Mn, m[j]);
        const float f = __builtin_amdgcn_exp2f(M - Mn);
        lt *= f;
        ot *= f;
#pragma unroll
        for (int j = 0; j < kPartBatch; j++) {
            const float wj =
                c0 + j * kMergeParts < n_chunks ? __builtin_amdgcn_exp2f(m[j] - Mn) : 0.0f;
            lt = fmaf(lv[j], wj, lt);
            ot = fmaf(ov[j], wj, ot);
        }
        M = Mn;
    }
    if ((threadIdx.x & 31) == 0) {
        pm[pt] = M;
        pl[pt] = lt;
    }
    po[pt][threadIdx.x & 31] = ot;
    __syncthreads();
    if (pt == 0) {
        float Mt = pm[0];
#pragma unroll
        for (int k = 1; k < kMergeParts; k++) Mt = fmaxf(Mt, pm[k]);
        float l = 0.0f, o = 0.0f;
#pragma unroll
        for (int k = 0; k < kMergeParts; k++) {
            const float f = __builtin_amdgcn_exp2f(pm[k] - Mt);
            l = fmaf(pl[k], f, l);
            o = fmaf(po[k][threadIdx.x], f, o);
        }
        out[((int64_t)s * n_q + qh) * D + i] = o * (1.0f / l);
    }
}

// V-sum mode's merge: out[qh][i] = the plain sum over chunks of the
// partials' o[i] (every chunk's m is 0), in a fixed order: a block takes 32
// dims of one q head; thread (i, part) adds chunks part, part + 8, ...,
// kVsBatch at a time with their loads in flight, and the 8 part sums are
// added in part order.  A chunk whose l is NaN (a non-finite weight) makes
// the head's outputs NaN.
constexpr int kVsParts = 8;
constexpr int kVsBatch = 16;

template <int D>
__global__ __launch_bounds__(256) void vsum_merge_kernel(int stride, int n_chunks,
                                                         const float *__restrict__ part,
                                                         float *__restrict__ out)
{
    __shared__ float red[kVsParts][32];
    __shared__ float flag[kVsParts];
    const int qh = blockIdx.x / (D / 32), i = (blockIdx.x % (D / 32)) * 32 + (threadIdx.x & 31);
    const int pt = threadIdx.x >> 5;
    const float *p = part + (int64_t)qh * stride * (D + 2);    // stride: chunks per head
    float sum = 0.0f, bad = 0.0f;
    for (int c0 = pt; c0 < n_chunks; c0 += kVsParts * kVsBatch) {
        float o[kVsBatch], l[kVsBatch];
#pragma unroll
        for (int j = 0; j < kVsBatch; j++) {
            const int c = min(c0 + j * kVsParts, n_chunks - 1);
            o[j] = p[(int64_t)c * (D + 2) + 2 + i];
            l[j] = p[(int64_t)c * (D + 2) + 1];
        }
#pragma unroll
        for (int j = 0; j < kVsBatch; j++)
            if (c0 + j * kVsParts < n_chunks) {
                sum = __fadd_rn(sum, o[j]);
                bad = bad + l[j];                 // 0, or NaN after a non-finite weight
            }
    }
    red[pt][threadIdx.x & 31] = sum;
    if ((threadIdx.x & 31) == 0) flag[pt] = bad;
    __syncthreads();
    if (pt == 0) {
        float t = red[0][threadIdx.x];
        float f = flag[0];
#pragma unroll
        for (int k = 1; k < kVsParts; k++) {
            t = __fadd_rn(t, red[k][threadIdx.x]);
            f = f + flag[k];
        }
        out[(int64_t)qh * D + i] = f == f ? t : f;
    }
}

// ------------------------------------------------------------------ VALU

constexpr int kChunkV = 512;      // tokens per block
// the MFMA program's chunks hold at least kChunkM tokens (the partials'
// workspace is sized by it): 4 tiles, 1 per wave of a 4-wave block
// (mfma_blocks_per_unit)
constexpr int kChunkM = 128;
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
// round of blocks would idle most of the chip), and at least one.  A chunk
// holds at least 4*kChunkM tokens (4 tiles per wave), unless that leaves
// fewer blocks than CUs (short contexts, few kv heads): then kChunkM, the
// workspace's granularity, as long as a unit keeps at most kInBatch chunks
// (merged in the launch), else 2*kChunkM.  Measured: 8Q/8KV at 2048 tokens
// 11.7 -> 10.5 us and 32Q/4KV d64 at 4096 10.3 -> 9.6 us with 256-token
// chunks, but 32Q/32KV at 8192 15.0 -> 17.5 us with them everywhere; 8Q/8KV
// at 2048 tokens 6.86 -> 6.31 us with 128-token chunks (one tile per wave).
int mfma_blocks_per_unit(int ml, int units, int per_cu)
{
    const int n_cu = cu_count();
    const int slots = n_cu * per_cu;
    int nb = units >= slots ? 1 : slots / units;
    const int coarse = (ml + 4 * kChunkM - 1) / (4 * kChunkM);
    int fine = (ml + kChunkM - 1) / kChunkM;
    if (fine > kInBatch) fine = max(kInBatch, (ml + 2 * kChunkM - 1) / (2 * kChunkM));
    const int cap = (int64_t)units * coarse < n_cu ? fine : coarse;
    nb = nb < cap ? nb : cap;
    return nb < 1 ? 1 : nb;
}

// Virtual kv heads per kv head for the MFMA program: 1 up to 8 q heads per
// kv head; above, the fewest that divide the group into parts of at most 8
// (each part reads the kv head's tiles again, through L2); 0 if none does.
int mfma_split(int qpk)
{
    if (qpk <= 8) return 1;
    for (int sp = 2; sp <= qpk; sp++)
        if (qpk % sp == 0 && qpk / sp <= 8) return sp;
    return 0;
}

int per_cu_of(int d, int hh)
{
    return d == 64 ? (hh == 1 ? kBlocksPerCUH<64, 1> : kBlocksPerCUH<64, 2>)
                   : (hh == 1 ? kBlocksPerCUH<128, 1> : kBlocksPerCUH<128, 2>);
}

// mfma_split, and for groups of 5-8 q heads whose two-quad grid leaves more
// than half of the chip's resident blocks idle (short contexts, few kv
// heads): two virtual kv heads of one quad each, whose waves carry half the
// arithmetic (each reads the kv head's tiles, the second time from L2).
// 32Q/4KV d64 at 4096 tokens: 64 two-quad blocks become 128 one-quad blocks.
int mfma_split_fill(int qpk, int d, int ml, int64_t units)
{
    const int sp = mfma_split(qpk);
    if (sp != 1 || qpk <= 4 || qpk % 2) return sp;
    const int per_cu = per_cu_of(d, 2);
    const int64_t blocks = units * mfma_blocks_per_unit(ml, (int)units, per_cu);
    return 2 * blocks < (int64_t)cu_count() * per_cu ? 2 : 1;
}

int max_len(const eakvd_batch *b)
{
    int mx = 0;
    for (int i = 0; i < b->n_seq; i++) mx = b->seq_len[i] > mx ? b->seq_len[i] : mx;
    return mx;
}

// Tokens per tile of the matrix-core program: 64 for two-quad waves that
// each get at least kMinTiles64 tiles of 64, else 32.  Short contexts keep
// the finer tiles, which give more waves work (32Q/4KV d64 at 4096 tokens:
// 8.3 us per fused call with 32-token tiles, 9.7 with 64-token ones; 64Q/8KV
// d128 at 131072 tokens: 38.9-39.0 against 39.5-39.6 us).
constexpr int kMinTiles64 = 4;

int tile_tokens(int hh, int ml, int mc, int wpb)
{
    const int64_t t64 = ((int64_t)ml + 63) / 64;
    return hh == 2 && t64 >= (int64_t)kMinTiles64 * mc * wpb ? 64 : 32;
}

// The mfma_kernel instantiation of a launch shape
template <bool VS>
auto mfma_entry(int d, int hh, int tt)
{
    if (d == 64) {
        if (hh == 1) return mfma_kernel<64, 1, VS, 32>;
        return tt == 64 ? mfma_kernel<64, 2, VS, 64> : mfma_kernel<64, 2, VS, 32>;
    }
    if (hh == 1) return mfma_kernel<128, 1, VS, 32>;
    return tt == 64 ? mfma_kernel<128, 2, VS, 64> : mfma_kernel<128, 2, VS, 32>;
}

// The launch shape of one fused call: the matrix-core program (chunks per
// unit mc, waves per block wpb, virtual kv heads per kv head split, q heads
// per virtual head qv, quads hh, tokens per tile tt) or the VALU program
// (mc chunks of kChunkV).
struct FusedPlan {
    bool mfma;
    int mc, wpb, split, qv, hh, tt;
};

FusedPlan fused_plan(const eakvd_geom *g, const eakvd_batch *b, int n_q, int n_kv)
{
    FusedPlan p{};
    const int qpk = n_q / n_kv;
    const int ml = max_len(b);
    // the MFMA program addresses a layer's K and V blocks with 32-bit buffer
    // offsets
    const bool small_planes = 2 * g->block_bytes <= (int64_t)0x7fffffff;
    p.split = mfma_split_fill(qpk, g->head_dim, ml, (int64_t)b->n_seq * n_kv);
    p.mfma = p.split > 0 && small_planes;
    if (p.mfma) {
        p.qv = qpk / p.split;
        p.hh = p.qv <= 4 ? 1 : 2;
        const int per_cu = per_cu_of(g->head_dim, p.hh);
        p.wpb = p.hh == 1 ? kWavesH<1> : kWavesH<2>;
        p.mc = mfma_blocks_per_unit(ml, b->n_seq * n_kv * p.split, per_cu);
        p.tt = tile_tokens(p.hh, ml, p.mc, p.wpb);
    } else {
        p.mc = (ml + kChunkV - 1) / kChunkV;
    }
    return p;
}

}  // namespace

extern "C" size_t eakvd_fused_work_bytes(const eakvd_geom *g,
                                         const eakvd_batch *b, int n_q)
{
    // sized for the finer (MFMA) chunking, which covers both programs
    const int mc = (max_len(b) + kChunkM - 1) / kChunkM;
    return (size_t)b->n_seq * n_q * mc * (g->head_dim + 2) * sizeof(float);
}

extern "C" size_t eakvd_fused_launch_bytes(const eakvd_geom *g, const eakvd_batch *b,
                                           int n_q, int n_kv)
{
    // partial (m, l, o[D]) of every (sequence, q head, chunk)
    const FusedPlan p = fused_plan(g, b, n_q, n_kv);
    return (size_t)b->n_seq * n_q * p.mc * (g->head_dim + 2) * sizeof(float);
}

extern "C" int eakvd_scratch(void **p)
{
    // one lookup per device: each device holds its own copy of `scratch`
    static std::mutex mu;
    static void *addr[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void *a = nullptr;
        e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        addr[dev] = a;
    }
    *p = addr[dev];
    return 0;
}

// The chunks merged in the main launch: where counters are given, every
// unit has a counter and at most kInBatch chunks (one round trip of loads).
// The merging block's tail (its partial written through, a counter round
// trip, the unit's partials read back) costs less than a dependent launch,
// measured with 8 waves per CU; with 16 waves per CU (4 one-quad blocks, 16
// chunks per unit) it cost more.
bool merge_in_launch(const eakvd_geom *g, const void *ctr, int mc, int64_t units)
{
    return ctr && mc <= kInBatch && units <= g->ctr_slots;
}

extern "C" void eakvd_fused_plan(const eakvd_geom *g, const eakvd_batch *b, int n_q, int n_kv,
                                 const void *ctr, int32_t *out)
{
    const FusedPlan p = fused_plan(g, b, n_q, n_kv);
    const int ml = max_len(b);
    out[0] = p.mfma;
    out[1] = p.mc;
    if (p.mfma) {
        const int64_t units = (int64_t)n_kv * p.split * b->n_seq;
        const int64_t n_tiles = ((int64_t)ml + p.tt - 1) / p.tt;
        const int64_t waves = (int64_t)p.mc * p.wpb;
        out[2] = merge_in_launch(g, ctr, p.mc, units);
        out[3] = p.tt;
        out[4] = p.wpb;
        out[5] = (int32_t)((n_tiles + waves - 1) / waves);
        out[6] = p.hh;
        out[7] = p.split;
    } else {
        out[2] = 0;
        out[3] = kChunkV;
        out[4] = 4;
        out[5] = 1;
        out[6] = 0;
        out[7] = 1;
    }
}

extern "C" int eakvd_fused(const eakvd_geom *g, const eakvd_batch *b,
                           int layer, const float *q, int n_q, int n_kv,
                           float *out, void *work, void *ctr, void *stream)
{
    const hipStream_t st = (hipStream_t)stream;
    const float rs = 1.0f / sqrtf((float)g->head_dim);
    float *part = (float *)work;
    const FusedPlan p = fused_plan(g, b, n_q, n_kv);
    if (p.mfma) {
        const int mc = p.mc, wpb = p.wpb, hh = p.hh;
        const dim3 grid((unsigned)mc, (unsigned)(n_kv * p.split), (unsigned)b->n_seq);
        const dim3 mgrid((unsigned)n_q, (unsigned)b->n_seq);
        // more than one batch of chunks: the merge spread over 8 parts
        const bool parts = mc > kMergeBatch;
        const dim3 pgrid((unsigned)(n_q * (g->head_dim / 32)), (unsigned)b->n_seq);
        auto kern = mfma_entry<false>(g->head_dim, hh, p.tt);
        const int64_t units = (int64_t)n_kv * p.split * b->n_seq;
        uint8_t *uc = merge_in_launch(g, ctr, mc, units) ? (uint8_t *)ctr : nullptr;
        // one-quad grids of exactly two rounds of one block per CU: the
        // second round leads for half of its tiles (32Q/8KV d128 32K x 8:
        // 54.48-54.51 against 55.07-55.13 us per layer step, alternating
        // whole bench runs on one box; 55.24-55.30 against 55.55-55.96 on
        // another)
        int lead = 0;
        if (hh == 1 && units * mc == 2 * (int64_t)cu_count()) {
            const int64_t n_tiles = ((int64_t)max_len(b) + p.tt - 1) / p.tt;
            const int64_t waves = (int64_t)mc * wpb;
            lead = (int)(((n_tiles + waves - 1) / waves + 1) / 2);
        }
        hipLaunchKernelGGL(kern, grid, dim3(64 * wpb), 0, st, *g, *b, layer, q, n_q, p.qv, rs,
                           part, p.split, out, uc, lead);
        if (uc) return (int)hipGetLastError();
        const int tt = p.tt;
        if (parts && g->head_dim == 64)
            hipLaunchKernelGGL(merge_parts_kernel<64>, pgrid, dim3(256), 0, st, *b, n_q, mc,
                               wpb, tt, part, out);
        else if (parts)
            hipLaunchKernelGGL(merge_parts_kernel<128>, pgrid, dim3(256), 0, st, *b, n_q, mc,
                               wpb, tt, part, out);
        else if (g->head_dim == 64)
            hipLaunchKernelGGL(merge_kernel<64>, mgrid, dim3(64), 0, st, *b, n_q, mc, wpb,
                               tt, part, out);
        else
            hipLaunchKernelGGL(merge_kernel<128>, mgrid, dim3(128), 0, st, *b, n_q, mc, wpb,
                               tt, part, out);
        return (int)hipGetLastError();
    }
    const int qpk = n_q / n_kv;
    const int mc = p.mc;
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

// The unfused V-sum on the matrix cores (mfma_kernel in V-sum mode) for 2 or
// more q heads per kv head (above 8 as virtual kv heads, see mfma_split):
// out[n_q][D] = sum_t w[h][t] V[t] over seq_len tokens of one cache, the
// chunk partials in `work`.  Returns -1 (nothing launched) where it does not
// apply: MHA (one q head per kv head fills a quarter of each MFMA; the VALU
// kernel measured as fast or faster there), a group size with no split into
// parts of at most 8, planes beyond 32-bit buffer offsets, or weights beyond
// 2 GiB.
extern "C" size_t eakvd_v_sum_mfma_work_bytes(const eakvd_geom *g, int seq_len, int n_q)
{
    const int mc = (seq_len + kChunkM - 1) / kChunkM;
    return (size_t)n_q * (mc > 0 ? mc : 1) * (g->head_dim + 2) * sizeof(float);
}

extern "C" int eakvd_v_sum_mfma(const eakvd_geom *g, const uint8_t *base, int layer,
                                int seq_len, const float *w, int n_q, int n_kv, float *out,
                                void *work, void *stream)
{
    const int qpk = n_q / n_kv;
    const int split = qpk < 2 ? 0 : mfma_split_fill(qpk, g->head_dim, seq_len, n_kv);
    if (split == 0 || 2 * g->block_bytes > (int64_t)0x7fffffff ||
        (int64_t)qpk * seq_len * 4 > (int64_t)0x7fffffff || seq_len <= 0)
        return -1;
    const int qv = qpk / split;                             // q heads per virtual kv head
    const hipStream_t st = (hipStream_t)stream;
    eakvd_batch b;
    memset(&b, 0, sizeof(b));
    b.n_seq = 1;
    b.base[0] = base;
    b.seq_len[0] = seq_len;
    const int hh = qv <= 4 ? 1 : 2;
    const int per_cu = per_cu_of(g->head_dim, hh);
    const int wpb = hh == 1 ? kWavesH<1> : kWavesH<2>;
    const int mc = mfma_blocks_per_unit(seq_len, n_kv * split, per_cu);
    const int tt = tile_tokens(hh, seq_len, mc, wpb);
    const dim3 grid((unsigned)mc, (unsigned)(n_kv * split), 1u);
    float *part = (float *)work;
    auto kern = mfma_entry<true>(g->head_dim, hh, tt);
    const int64_t units = (int64_t)n_kv * split;
    uint8_t *ctr = const_cast<uint8_t *>(base) + g->ctr_off;
    uint8_t *uc = merge_in_launch(g, ctr, mc, units) ? ctr : nullptr;
    hipLaunchKernelGGL(kern, grid, dim3(64 * wpb), 0, st, *g, b, layer, w, n_q, qv, 0.0f,
                       part, split, out, uc, 0);
    if (uc) return (int)hipGetLastError();
    // the chunks that hold a partial: blocks with a tile (see mfma_kernel)
    const int n_tiles = (seq_len + tt - 1) / tt;
    const int nch = min(mc, (n_tiles + wpb - 1) / wpb);
    if (g->head_dim == 64)
        hipLaunchKernelGGL(vsum_merge_kernel<64>, dim3((unsigned)(n_q * 2)), dim3(256), 0, st,
                           mc, nch, part, out);
    else
        hipLaunchKernelGGL(vsum_merge_kernel<128>, dim3((unsigned)(n_q * 4)), dim3(256), 0, st,
                           mc, nch, part, out);
    return (int)hipGetLastError();
}
