/* eakv_oracle_avx512.c — the reference's CPU fused attention as it runs on
 * AVX-512 (kernels/fused_attention.ea:190-373, compiled by the Ea compiler to
 * 16-lane AVX-512), restated with intrinsics.
 *
 * TEST INFRASTRUCTURE ONLY (see eakv_oracle.h): bench.py's CPU baseline times
 * it, and a test checks it against orc_fused_attention.  Per lane it does the
 * arithmetic of orc_fused_attention (the dequant fma, the 16-lane fma chain
 * over chunks, the halving reduction, expf, the V fma chain), so the two
 * agree bit for bit.  The functions carry their own target attribute: the
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
