/* eakv_oracle_avx512.c — the reference's CPU kernels as they run on AVX-512
 * (compiled by the Ea compiler to 16 lanes), restated with intrinsics: the
 * fused attention (kernels/fused_attention.ea:190-373), the K-score
 * (fused_k_score*.ea) and the V-sum (fused_v_sum*.ea, fused_k_score_gqa*.ea).
 *
 * TEST INFRASTRUCTURE ONLY (see eakv_oracle.h): bench.py's CPU baseline times
 * them, and tests check them against the scalar oracle.  Per lane they do the
 * oracle's arithmetic (the dequant fma, the 16-lane fma chain over chunks,
 * the halving reduction, expf, the V fma chain over the tokens), so they
 * agree with it bit for bit.  The functions carry their own target attribute: the
 * library loads on any x86-64 CPU and orc_avx512_available() says whether
 * they may be called.
 */
#include "eakv_oracle.h"

#include <immintrin.h>
#include <math.h>

#define AVX512 __attribute__((target("avx512f,avx512bw,avx512dq,avx512vl")))

int orc_avx512_available(void)
{
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl");
}

/* Chunk cc (0..3) of a group: bytes (cc&1)*16..+15, low nibbles for cc < 2,
 * each fma(n, s, b) (fused_attention.ea dequant; orc chunk_deq). */
static inline AVX512 __m512 deq16(const uint8_t *gw, int cc, __m512 s, __m512 b)
{
    __m512i v = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i *)(gw + (cc & 1) * 16)));
    v = cc < 2 ? _mm512_and_si512(v, _mm512_set1_epi32(15)) : _mm512_srli_epi32(v, 4);
    return _mm512_fmadd_ps(_mm512_cvtepi32_ps(v), s, b);
}

/* reduce_add of 16 lanes in orc_reduce16's order: a[i] + a[i+8], then
 * v8[i] + v8[i+4], v4[i] + v4[i+2], v2[0] + v2[1]. */
static inline AVX512 float reduce16(__m512 a)
{
    __m256 v8 = _mm256_add_ps(_mm512_castps512_ps256(a), _mm512_extractf32x8_ps(a, 1));
    __m128 v4 = _mm_add_ps(_mm256_castps256_ps128(v8), _mm256_extractf128_ps(v8, 1));
    __m128 v2 = _mm_add_ps(v4, _mm_movehl_ps(v4, v4));
    __m128 v1 = _mm_add_ss(v2, _mm_shuffle_ps(v2, v2, 1));
    return _mm_cvtss_f32(v1);
}

static inline AVX512 float score(int n_chunks, const __m512 *qv, const uint8_t *kw,
                                 const float *ks, const float *kb, int64_t g0, float rs)
{
    __m512 acc = _mm512_setzero_ps();
    for (int c = 0; c < n_chunks; c++) {
        const int64_t g = g0 + c / 4;
        const __m512 k = deq16(kw + g * 32, c & 3, _mm512_set1_ps(ks[g]), _mm512_set1_ps(kb[g]));
        acc = _mm512_fmadd_ps(k, qv[c], acc);
    }
    return reduce16(acc) * rs;
}

AVX512 void orc_fused_attention_avx512(int head_dim, const float *q, const uint8_t *kw,
                                       const float *ks, const float *kb, const uint8_t *vw,
                                       const float *vs, const float *vb, float *out,
                                       int seq_len, int n_q_heads, int n_kv_heads,
                                       int64_t groups_per_head)
{
    volatile float dv = (float)head_dim;               /* as rsqrt_dim in eakv_oracle.c */
    const float rs = 1.0f / sqrtf(dv);
    const int gpd = head_dim / 64, n_chunks = head_dim / 16;
    const int qpk = n_q_heads / n_kv_heads;
    for (int qh = 0; qh < n_q_heads; qh++) {
        const int64_t goff = (int64_t)(qh / qpk) * groups_per_head;
        __m512 qv[8], o[8];
        for (int c = 0; c < n_chunks; c++) {
            qv[c] = _mm512_loadu_ps(q + (int64_t)qh * head_dim + 16 * c);
            o[c] = _mm512_setzero_ps();
        }
        /* pass 1 (:224-267): max with init 0 - 1000000 */
        float mx = 0.0f - 1000000.0f;
        for (int t = 0; t < seq_len; t++) {
            const float sc = score(n_chunks, qv, kw, ks, kb, goff + (int64_t)t * gpd, rs);
            mx = sc > mx ? sc : mx;
        }
        /* pass 2 (:280-359): recompute, exp, sum, weighted V */
        float sum = 0.0f;
        for (int t = 0; t < seq_len; t++) {
            const int64_t g0 = goff + (int64_t)t * gpd;
            const float wt = expf(score(n_chunks, qv, kw, ks, kb, g0, rs) - mx);
            sum = sum + wt;
            const __m512 w = _mm512_set1_ps(wt);
            for (int c = 0; c < n_chunks; c++) {
                const int64_t g = g0 + c / 4;
                const __m512 v = deq16(vw + g * 32, c & 3, _mm512_set1_ps(vs[g]),
                                       _mm512_set1_ps(vb[g]));
                o[c] = _mm512_fmadd_ps(v, w, o[c]);
            }
        }
        /* :361-369 */
        const __m512 inv = _mm512_set1_ps(1.0f / sum);
        for (int c = 0; c < n_chunks; c++)
            _mm512_storeu_ps(out + (int64_t)qh * head_dim + 16 * c, _mm512_mul_ps(o[c], inv));
    }
}

void orc_attention_fused_avx512(const orc_cache_t *c, const float *queries, int layer,
                                int n_q_heads, int n_kv_heads, float *output_out)
{
    const int hd = orc_cache_head_dim(c);
    const int64_t gph = (int64_t)orc_cache_max_seq_len(c) * (hd / 64);
    orc_fused_attention_avx512(hd, queries, orc_cache_weights(c, layer, 0),
                               orc_cache_scales(c, layer, 0), orc_cache_biases(c, layer, 0),
                               orc_cache_weights(c, layer, 1), orc_cache_scales(c, layer, 1),
                               orc_cache_biases(c, layer, 1), output_out, orc_cache_seq_len(c),
                               n_q_heads, n_kv_heads, gph);
}

/* The reference's unfused K-score on AVX-512 (fused_k_score.ea:161-235 and
 * fused_k_score_gqa.ea:7-99, compiled to 16 lanes): per kv head and token
 * the chunks are dequantized once (the GQA loop flip), then per q head one
 * 16-lane fma chain over the chunks, the halving reduction and x rsqrt(d),
 * which is orc_k_score_gqa's arithmetic, so the scores agree bit for bit. */
AVX512 void orc_attention_scores_avx512(const orc_cache_t *c, const float *queries, int layer,
                                        int n_q_heads, int n_kv_heads, float *scores_out)
{
    const int hd = orc_cache_head_dim(c), L = orc_cache_seq_len(c);
    const int gpd = hd / 64, n_chunks = hd / 16, qpk = n_q_heads / n_kv_heads;
    const int64_t gph = (int64_t)orc_cache_max_seq_len(c) * gpd;
    const uint8_t *kw = orc_cache_weights(c, layer, 0);
    const float *ks = orc_cache_scales(c, layer, 0), *kb = orc_cache_biases(c, layer, 0);
    volatile float dv = (float)hd;
    const float rs = 1.0f / sqrtf(dv);
    for (int kvh = 0; kvh < n_kv_heads; kvh++) {
        const int64_t goff = (int64_t)kvh * gph;
        for (int t = 0; t < L; t++) {
            const int64_t g0 = goff + (int64_t)t * gpd;
            __m512 k[8];
            for (int ch = 0; ch < n_chunks; ch++) {
                const int64_t g = g0 + ch / 4;
                k[ch] = deq16(kw + g * 32, ch & 3, _mm512_set1_ps(ks[g]), _mm512_set1_ps(kb[g]));
            }
            for (int o = 0; o < qpk; o++) {
                const int qh = kvh * qpk + o;
                const float *qv = queries + (int64_t)qh * hd;
                __m512 acc = _mm512_setzero_ps();
                for (int ch = 0; ch < n_chunks; ch++)
                    acc = _mm512_fmadd_ps(k[ch], _mm512_loadu_ps(qv + 16 * ch), acc);
                scores_out[(int64_t)qh * L + t] = reduce16(acc) * rs;
            }
        }
    }
}

/* The reference's unfused V-sum on AVX-512 (fused_v_sum.ea:83-163,
 * fused_v_sum_64.ea:55-110; GQA fused_k_score_gqa.ea:106-305, which takes
 * the q heads of a kv head in pairs and dequantizes V once per token and
 * pair): every output element is one fma chain over the tokens in order,
 * orc_v_sum_gqa's arithmetic, so the outputs agree bit for bit. */
AVX512 void orc_attention_output_avx512(const orc_cache_t *c, const float *weights, int layer,
                                        int n_q_heads, int n_kv_heads, float *output_out)
{
    const int hd = orc_cache_head_dim(c), L = orc_cache_seq_len(c);
    const int gpd = hd / 64, n_chunks = hd / 16, qpk = n_q_heads / n_kv_heads;
    const int64_t gph = (int64_t)orc_cache_max_seq_len(c) * gpd;
    const uint8_t *vw = orc_cache_weights(c, layer, 1);
    const float *vs = orc_cache_scales(c, layer, 1), *vb = orc_cache_biases(c, layer, 1);
    for (int kvh = 0; kvh < n_kv_heads; kvh++) {
        const int64_t goff = (int64_t)kvh * gph;
        for (int o0 = 0; o0 < qpk; o0 += 2) {
            const int np = qpk - o0 < 2 ? 1 : 2;
            const int qh0 = kvh * qpk + o0;
            __m512 acc[2][8];
            for (int p = 0; p < 2; p++)
                for (int ch = 0; ch < 8; ch++) acc[p][ch] = _mm512_setzero_ps();
            for (int t = 0; t < L; t++) {
                const int64_t g0 = goff + (int64_t)t * gpd;
                const __m512 w0 = _mm512_set1_ps(weights[(int64_t)qh0 * L + t]);
                const __m512 w1 = _mm512_set1_ps(np > 1 ? weights[(int64_t)(qh0 + 1) * L + t] : 0.0f);
                for (int ch = 0; ch < n_chunks; ch++) {
                    const int64_t g = g0 + ch / 4;
                    const __m512 v = deq16(vw + g * 32, ch & 3, _mm512_set1_ps(vs[g]),
                                           _mm512_set1_ps(vb[g]));
                    acc[0][ch] = _mm512_fmadd_ps(v, w0, acc[0][ch]);
                    acc[1][ch] = _mm512_fmadd_ps(v, w1, acc[1][ch]);
                }
            }
            for (int p = 0; p < np; p++)
                for (int ch = 0; ch < n_chunks; ch++)
                    _mm512_storeu_ps(output_out + (int64_t)(qh0 + p) * hd + 16 * ch, acc[p][ch]);
        }
    }
}
