/* eakv_oracle.c — CPU restatement of the reference eakv hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see eakv_oracle.h).  Build with
 * -ffp-contract=off: every fused multiply-add below is an explicit fmaf, and
 * every other product and sum must round on its own, as in the reference.
 */
#include "eakv_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar helpers                                                            */

int32_t orc_to_i32(float v)
{
    /* cvttss2si: truncate toward zero, "integer indefinite" (INT32_MIN) for
     * NaN and for values outside [-2^31, 2^31). */
    if (v >= -2147483648.0f && v < 2147483648.0f)
        return (int32_t)v;
    return INT32_MIN;
}

float orc_reduce16(const float *a)
{
    float v8[8], v4[4], v2[2];
    for (int i = 0; i < 8; i++) v8[i] = a[i] + a[i + 8];
    for (int i = 0; i < 4; i++) v4[i] = v8[i] + v8[i + 4];
    for (int i = 0; i < 2; i++) v2[i] = v4[i] + v4[i + 2];
    return v2[0] + v2[1];
}

static float rsqrt_dim(int head_dim)
{
    /* reference: 1.0 / sqrt(to_f32(128)) (fused_k_score.ea:174) and
     * 1.0 / sqrt(to_f32(64)) (fused_k_score_64.ea:113), f32 */
    volatile float d = (float)head_dim;
    float r = sqrtf(d);
    return 1.0f / r;
}

/* ------------------------------------------------------------------------ */
/* quantize: kernels/quantize_simd.ea:9-59                                   */

void orc_quantize_split(const float *src, uint8_t *weights, float *scales,
                        float *biases, int64_t n_groups)
{
    const float half = 1.0f / 2.0f;                      /* :16 */
    for (int64_t g = 0; g < n_groups; g++) {
        const float *x = src + g * 64;
        float mn = x[0], mx = x[0];                       /* :21-30 */
        for (int j = 1; j < 64; j++) {
            float v = x[j];
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        float range = mx - mn;                            /* :32-38 */
        float scale = 1.0f, inv = 0.0f;
        if (range > 0.0f) {
            scale = range / 15.0f;
            inv = 15.0f / range;
        }
        scales[g] = scale;                                /* :40-41 */
        biases[g] = mn;
        uint8_t *w = weights + g * 32;                    /* :43-55 */
        for (int k = 0; k < 32; k++) {
            float vlo = (x[k] - mn) * inv;
            float vhi = (x[k + 32] - mn) * inv;
            int32_t qlo = orc_to_i32(vlo + half);
            int32_t qhi = orc_to_i32(vhi + half);
            qlo = qlo < 0 ? 0 : (qlo > 15 ? 15 : qlo);
            qhi = qhi < 0 ? 0 : (qhi > 15 ? 15 : qhi);
            w[k] = (uint8_t)(qhi * 16 + qlo);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* packed-group access                                                       */

/* Value j (0..63) of a group: byte j%32, low nibble for j<32, high otherwise
 * (quantize_simd.ea:1-7). */
static inline float nib(const uint8_t *w, int j)
{
    uint8_t b = w[j & 31];
    return (float)(j < 32 ? (b & 15) : (b >> 4));
}

void orc_dequantize(const uint8_t *weights, const float *scales,
                    const float *biases, float *out, int64_t n_groups)
{
    for (int64_t g = 0; g < n_groups; g++)
        for (int j = 0; j < 64; j++)
            out[g * 64 + j] = fmaf(nib(weights + g * 32, j), scales[g], biases[g]);
}

void orc_dequantize_range(const uint8_t *weights, const float *scales,
                          const float *biases, float *out, int64_t group_start,
                          int64_t group_count)
{
    for (int64_t i = 0; i < group_count; i++) {
        const int64_t g = group_start + i;
        for (int j = 0; j < 64; j++)
            out[i * 64 + j] = fmaf(nib(weights + g * 32, j), scales[g], biases[g]);
    }
}

void orc_ggml_quantize_row(const float *src, uint8_t *dst, int64_t k)
{
    for (int64_t i = 0; i < k / 64; i++) {
        const float *x = src + i * 64;
        uint8_t *blk = dst + i * 40;
        float mn = x[0], mx = x[0];
        for (int j = 1; j < 64; j++) {
            if (x[j] < mn) mn = x[j];
            if (x[j] > mx) mx = x[j];
        }
        const float range = mx - mn;
        const float d = range / 15.0f;
        const float id = range > 0.0f ? 15.0f / range : 0.0f;
        memcpy(blk + 32, &d, 4);
        memcpy(blk + 36, &mn, 4);
        for (int j = 0; j < 32; j++) {
            int lo = (int)(0.5f + (x[j] - mn) * id);
            int hi = (int)(0.5f + (x[j + 32] - mn) * id);
            lo = lo < 0 ? 0 : lo > 15 ? 15 : lo;
            hi = hi < 0 ? 0 : hi > 15 ? 15 : hi;
            blk[j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

void orc_ggml_dequantize_row(const uint8_t *src, float *dst, int64_t k)
{
    for (int64_t i = 0; i < k / 64; i++) {
        const uint8_t *blk = src + i * 40;
        float d, m;
        memcpy(&d, blk + 32, 4);
        memcpy(&m, blk + 36, 4);
        for (int j = 0; j < 32; j++) {
            dst[i * 64 + j] = fmaf((float)(blk[j] & 15), d, m);
            dst[i * 64 + j + 32] = fmaf((float)(blk[j] >> 4), d, m);
        }
    }
}

void orc_ggml_vec_dot(int n, float *s, size_t bs, const uint8_t *vx, size_t bx,
                      const float *vy, size_t by, int nrc)
{
    for (int r = 0; r < nrc; r++) {
        const uint8_t *x = vx + r * bx;
        const float *y = (const float *)((const char *)vy + r * by);
        float acc[16] = {0};
        for (int i = 0; i < n / 64; i++) {
            const uint8_t *blk = x + (int64_t)i * 40;
            float d, m;
            memcpy(&d, blk + 32, 4);
            memcpy(&m, blk + 36, 4);
            for (int c = 0; c < 2; c++) {
                for (int l = 0; l < 16; l++) {
                    const float v = fmaf((float)(blk[c * 16 + l] & 15), d, m);
                    acc[l] = fmaf(v, y[i * 64 + c * 16 + l], acc[l]);
                }
                for (int l = 0; l < 16; l++) {
                    const float v = fmaf((float)(blk[c * 16 + l] >> 4), d, m);
                    acc[l] = fmaf(v, y[i * 64 + c * 16 + 32 + l], acc[l]);
                }
            }
        }
        *(float *)((char *)s + r * bs) = orc_reduce16(acc);
    }
}

int32_t orc_validate(const float *scales, const float *biases, int64_t n_groups)
{
    const int32_t nan_exp = 2139095040;               /* 0x7f800000 */
    for (int64_t g = 0; g < n_groups; g++) {
        int32_t sb, bb;
        memcpy(&sb, scales + g, 4);
        memcpy(&bb, biases + g, 4);
        if (sb > nan_exp) return 1;
        if (sb < 0 && sb > -8388608) return 1;        /* 0xff800001..0xffffffff */
        if (bb > nan_exp) return 2;
        if (bb < 0 && bb > -8388608) return 2;
        if (scales[g] < 0.0f) return 3;
    }
    return 0;
}

/* The reference walks a token in 16-lane chunks c = 0..head_dim/16-1:
 * chunk c covers dims c*16..c*16+15, taken from group c/4, bytes
 * ((c%4)&1)*16..+15, low nibble for c%4 < 2 (fused_k_score.ea:195-227). */
static inline float chunk_deq(const uint8_t *gw, float s, float b, int cc,
                              int i)
{
    int byte = (cc & 1) * 16 + i;
    uint8_t v = gw[byte];
    float n = (float)(cc < 2 ? (v & 15) : (v >> 4));
    return fmaf(n, s, b);
}

/* One token's score against one q vector, reference arithmetic. */
static float token_score(int head_dim, const float *q, const uint8_t *kw,
                         const float *ks, const float *kb, int64_t g0,
                         float rsqrt_d)
{
    float acc[16];
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    int n_chunks = head_dim / 16;
    for (int c = 0; c < n_chunks; c++) {
        int64_t g = g0 + c / 4;
        const uint8_t *gw = kw + g * 32;
        float s = ks[g], b = kb[g];
        for (int i = 0; i < 16; i++)
            acc[i] = fmaf(chunk_deq(gw, s, b, c & 3, i), q[c * 16 + i],
                          acc[i]);
    }
    return orc_reduce16(acc) * rsqrt_d;
}

/* ------------------------------------------------------------------------ */
/* K-score                                                                   */

void orc_k_score_mha(int head_dim, const float *q, const uint8_t *kw,
                     const float *ks, const float *kb, float *scores,
                     int seq_len, int n_heads, int64_t groups_per_head)
{
    orc_k_score_gqa(head_dim, q, kw, ks, kb, scores, seq_len, n_heads,
                    n_heads, groups_per_head);
}

void orc_k_score_gqa(int head_dim, const float *q, const uint8_t *kw,
                     const float *ks, const float *kb, float *scores,
                     int seq_len, int n_q_heads, int n_kv_heads,
                     int64_t groups_per_head)
{
    /* fused_k_score_gqa.ea:24-98: K[kv_h, t] dequantized once, dotted with
     * each q head of the group.  Per q head the arithmetic equals the MHA
     * kernel (fused_k_score.ea:195-229), so one routine serves both. */
    const float rs = rsqrt_dim(head_dim);
    const int gpd = head_dim / 64;
    const int qpk = n_q_heads / n_kv_heads;
    for (int kvh = 0; kvh < n_kv_heads; kvh++) {
        int64_t goff = (int64_t)kvh * groups_per_head;
        for (int t = 0; t < seq_len; t++) {
            int64_t g0 = goff + (int64_t)t * gpd;
            for (int o = 0; o < qpk; o++) {
                int qh = kvh * qpk + o;
                scores[(int64_t)qh * seq_len + t] =
                    token_score(head_dim, q + (int64_t)qh * head_dim, kw, ks,
                                kb, g0, rs);
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* V-sum                                                                     */

void orc_v_sum_mha(int head_dim, const float *w, const uint8_t *vw,
                   const float *vs, const float *vb, float *out,
                   int seq_len, int n_heads, int64_t groups_per_head)
{
    orc_v_sum_gqa(head_dim, w, vw, vs, vb, out, seq_len, n_heads, n_heads,
                  groups_per_head);
}

void orc_v_sum_gqa(int head_dim, const float *w, const uint8_t *vw,
                   const float *vs, const float *vb, float *out,
                   int seq_len, int n_q_heads, int n_kv_heads,
                   int64_t groups_per_head)
{
    /* Each output element is one sequential chain over t of
     * o = fma(fma(nib, s, b), w[t], o) starting at 0 (fused_v_sum.ea:111-150;
     * the GQA kernel pairs q heads but runs the same chain per head,
     * fused_k_score_gqa.ea:152-207, :259-298). */
    const int gpd = head_dim / 64;
    const int qpk = n_q_heads / n_kv_heads;
    float o[128];
    for (int qh = 0; qh < n_q_heads; qh++) {
        int kvh = qh / qpk;
        int64_t goff = (int64_t)kvh * groups_per_head;
        const float *wr = w + (int64_t)qh * seq_len;
        for (int i = 0; i < head_dim; i++) o[i] = 0.0f;
        for (int t = 0; t < seq_len; t++) {
            float wt = wr[t];
            for (int c = 0; c < head_dim / 16; c++) {
                int64_t g = goff + (int64_t)t * gpd + c / 4;
                const uint8_t *gw = vw + g * 32;
                float s = vs[g], b = vb[g];
                for (int i = 0; i < 16; i++)
                    o[c * 16 + i] = fmaf(chunk_deq(gw, s, b, c & 3, i), wt,
                                         o[c * 16 + i]);
            }
        }
        for (int i = 0; i < head_dim; i++)
            out[(int64_t)qh * head_dim + i] = o[i];
    }
}

/* ------------------------------------------------------------------------ */
/* fused two-pass attention: kernels/fused_attention.ea:190-373              */

void orc_fused_attention(int head_dim, const float *q,
                         const uint8_t *kw, const float *ks, const float *kb,
                         const uint8_t *vw, const float *vs, const float *vb,
                         float *out, int seq_len, int n_q_heads,
                         int n_kv_heads, int64_t groups_per_head)
{
    const float rs = rsqrt_dim(head_dim);
    const int gpd = head_dim / 64;
    const int qpk = n_q_heads / n_kv_heads;
    float o[128];
    for (int qh = 0; qh < n_q_heads; qh++) {
        int kvh = qh / qpk;
        int64_t goff = (int64_t)kvh * groups_per_head;
        const float *qv = q + (int64_t)qh * head_dim;
        /* pass 1 (:224-267): max with init 0 - 1000000 */
        float mx = 0.0f - 1000000.0f;
        for (int t = 0; t < seq_len; t++) {
            float sc = token_score(head_dim, qv, kw, ks, kb,
                                   goff + (int64_t)t * gpd, rs);
            mx = sc > mx ? sc : mx;
        }
        /* pass 2 (:280-359): recompute, exp, sum, weighted V */
        float sum = 0.0f;
        for (int i = 0; i < head_dim; i++) o[i] = 0.0f;
        for (int t = 0; t < seq_len; t++) {
            int64_t g0 = goff + (int64_t)t * gpd;
            float sc = token_score(head_dim, qv, kw, ks, kb, g0, rs);
            float wt = expf(sc - mx);
            sum = sum + wt;
            for (int c = 0; c < head_dim / 16; c++) {
                int64_t g = g0 + c / 4;
                const uint8_t *gw = vw + g * 32;
                float s = vs[g], b = vb[g];
                for (int i = 0; i < 16; i++)
                    o[c * 16 + i] = fmaf(chunk_deq(gw, s, b, c & 3, i), wt,
                                         o[c * 16 + i]);
            }
        }
        /* :361-369 */
        float inv = 1.0f / sum;
        for (int i = 0; i < head_dim; i++)
            out[(int64_t)qh * head_dim + i] = o[i] * inv;
    }
}

void orc_softmax_rows(const float *scores, float *weights, int n_rows,
                      int seq_len)
{
    for (int r = 0; r < n_rows; r++) {
        const float *s = scores + (int64_t)r * seq_len;
        float *w = weights + (int64_t)r * seq_len;
        float mx = 0.0f - 1000000.0f;
        for (int t = 0; t < seq_len; t++) mx = s[t] > mx ? s[t] : mx;
        float sum = 0.0f;
        for (int t = 0; t < seq_len; t++) {
            w[t] = expf(s[t] - mx);
            sum = sum + w[t];
        }
        float inv = 1.0f / sum;
        for (int t = 0; t < seq_len; t++) w[t] = w[t] * inv;
    }
}

/* ------------------------------------------------------------------------ */
/* cache: src/cache.c and src/attention.c                                    */

struct orc_cache {
    int n_layers, n_kv_heads, head_dim, max_seq_len, seq_len;
    int64_t groups_per_token;   /* n_kv_heads*head_dim/64 (internal.h:21) */
    int64_t max_groups;         /* groups_per_token*max_seq_len (:22) */
    uint8_t *buf;               /* one zeroed allocation (cache.c:32-35) */
};

static size_t orc_block_bytes(const orc_cache_t *c)
{
    return (size_t)c->max_groups * 40;  /* weights 32 + scale 4 + bias 4 */
}

const uint8_t *orc_cache_weights(const orc_cache_t *c, int layer, int kv)
{
    return c->buf + (size_t)(layer * 2 + kv) * orc_block_bytes(c);
}

const float *orc_cache_scales(const orc_cache_t *c, int layer, int kv)
{
    return (const float *)(orc_cache_weights(c, layer, kv) +
                           (size_t)c->max_groups * 32);
}

const float *orc_cache_biases(const orc_cache_t *c, int layer, int kv)
{
    return (const float *)(orc_cache_weights(c, layer, kv) +
                           (size_t)c->max_groups * 36);
}

int64_t orc_cache_max_groups(const orc_cache_t *c) { return c->max_groups; }

orc_cache_t *orc_cache_create(int n_layers, int n_kv_heads, int head_dim,
                              int max_seq_len)
{
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 ||
        max_seq_len <= 0)
        return NULL;
    if (((int64_t)n_kv_heads * head_dim) % 64 != 0)
        return NULL;
    orc_cache_t *c = calloc(1, sizeof(*c));
    if (!c) return NULL;
    c->n_layers = n_layers;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->max_seq_len = max_seq_len;
    c->groups_per_token = (int64_t)n_kv_heads * head_dim / 64;
    c->max_groups = c->groups_per_token * max_seq_len;
    c->buf = calloc(1, orc_block_bytes(c) * 2 * (size_t)n_layers);
    if (!c->buf) { free(c); return NULL; }
    return c;
}

void orc_cache_free(orc_cache_t *c)
{
    if (!c) return;
    free(c->buf);
    free(c);
}

/* Quantize n_tokens of one head into plane (layer, kv) at token offset
 * t0 (cache.c:82-92, :137-146). */
static void orc_put_head(orc_cache_t *c, int layer, int kv, int h,
                         const float *src, int t0, int n_tokens)
{
    int64_t gpd = c->head_dim / 64;
    int64_t gph = (int64_t)c->max_seq_len * gpd;
    int64_t gbase = h * gph + (int64_t)t0 * gpd;
    uint8_t *w = (uint8_t *)orc_cache_weights(c, layer, kv);
    float *s = (float *)orc_cache_scales(c, layer, kv);
    float *b = (float *)orc_cache_biases(c, layer, kv);
    orc_quantize_split(src, w + gbase * 32, s + gbase, b + gbase,
                       (int64_t)n_tokens * gpd);
}

int orc_cache_load_raw(orc_cache_t *c, const float *data, int seq_len)
{
    if (!c || !data || seq_len <= 0) return -4;
    if (seq_len > c->max_seq_len) return -4;
    int64_t per_head = (int64_t)seq_len * c->head_dim;
    for (int l = 0; l < c->n_layers; l++)
        for (int kv = 0; kv < 2; kv++)
            for (int h = 0; h < c->n_kv_heads; h++) {
                const float *src =
                    data + (((int64_t)l * 2 + kv) * c->n_kv_heads + h) *
                               per_head;
                orc_put_head(c, l, kv, h, src, 0, seq_len);
            }
    c->seq_len = seq_len;
    return 0;
}

int orc_cache_append(orc_cache_t *c, const float *data, int layer,
                     int kv_idx, int n_tokens)
{
    if (!c || !data || n_tokens <= 0) return -4;
    if (layer < 0 || layer >= c->n_layers) return -4;
    if (kv_idx < 0 || kv_idx > 1) return -4;
    if ((int64_t)c->seq_len + n_tokens > c->max_seq_len) return -4;
    for (int h = 0; h < c->n_kv_heads; h++)
        orc_put_head(c, layer, kv_idx, h,
                     data + (int64_t)h * n_tokens * c->head_dim, c->seq_len,
                     n_tokens);
    return 0;
}

int orc_cache_advance(orc_cache_t *c, int n_tokens)
{
    if (!c || n_tokens <= 0) return -4;
    if ((int64_t)c->seq_len + n_tokens > c->max_seq_len) return -4;
    c->seq_len += n_tokens;
    return 0;
}

void orc_cache_clear(orc_cache_t *c)
{
    if (c) c->seq_len = 0;
}

int orc_checkpoint(orc_cache_t *c) { return c ? c->seq_len : 0; }

int orc_restore(orc_cache_t *c, int seq_len)
{
    if (!c) return -4;
    if (seq_len < 0 || seq_len > c->seq_len) return -4;
    c->seq_len = seq_len;
    return 0;
}

int orc_cache_seq_len(const orc_cache_t *c) { return c ? c->seq_len : 0; }
int orc_cache_n_layers(const orc_cache_t *c) { return c ? c->n_layers : 0; }
int orc_cache_n_heads(const orc_cache_t *c) { return c ? c->n_kv_heads : 0; }
int orc_cache_head_dim(const orc_cache_t *c) { return c ? c->head_dim : 0; }
int orc_cache_max_seq_len(const orc_cache_t *c)
{
    return c ? c->max_seq_len : 0;
}

float orc_cache_compression_ratio(const orc_cache_t *c)
{
    if (!c || c->seq_len == 0) return 0.0f;
    return 40.0f / 256.0f;
}

/* attention.c:3-63: head_dim 64 selects the d=64 kernels, anything else the
 * d=128 kernels; n_q == n_kv selects MHA, else GQA.  The oracle only accepts
 * head_dim 64 or 128 (the other cases read past the intended dims). */
void orc_attention_scores(const orc_cache_t *c, const float *queries,
                          int layer, int n_q_heads, int n_kv_heads,
                          float *scores_out)
{
    int64_t gph = (int64_t)c->max_seq_len * (c->head_dim / 64);
    orc_k_score_gqa(c->head_dim, queries, orc_cache_weights(c, layer, 0),
                    orc_cache_scales(c, layer, 0),
                    orc_cache_biases(c, layer, 0), scores_out, c->seq_len,
                    n_q_heads, n_kv_heads, gph);
}

void orc_attention_output(const orc_cache_t *c, const float *weights,
                          int layer, int n_q_heads, int n_kv_heads,
                          float *output_out)
{
    int64_t gph = (int64_t)c->max_seq_len * (c->head_dim / 64);
    orc_v_sum_gqa(c->head_dim, weights, orc_cache_weights(c, layer, 1),
                  orc_cache_scales(c, layer, 1),
                  orc_cache_biases(c, layer, 1), output_out, c->seq_len,
                  n_q_heads, n_kv_heads, gph);
}

void orc_attention_fused(const orc_cache_t *c, const float *queries,
                         int layer, int n_q_heads, int n_kv_heads,
                         float *output_out)
{
    int64_t gph = (int64_t)c->max_seq_len * (c->head_dim / 64);
    orc_fused_attention(c->head_dim, queries, orc_cache_weights(c, layer, 0),
                        orc_cache_scales(c, layer, 0),
                        orc_cache_biases(c, layer, 0),
                        orc_cache_weights(c, layer, 1),
                        orc_cache_scales(c, layer, 1),
                        orc_cache_biases(c, layer, 1), output_out,
                        c->seq_len, n_q_heads, n_kv_heads, gph);
}

/* ------------------------------------------------------------------------ */
/* .eakv files: src/io.c                                                     */

#define ORC_HDR 512

static size_t orc_align64(size_t x) { return (x + 63) & ~(size_t)63; }

static void put_u16(uint8_t *p, uint16_t v) { p[0] = v; p[1] = v >> 8; }
static void put_u32(uint8_t *p, uint32_t v)
{
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static uint16_t get_u16(const uint8_t *p) { return p[0] | (p[1] << 8); }
static uint32_t get_u32(const uint8_t *p)
{
    return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Header field offsets of the packed 512-byte header (io.c:11-28). */
enum { H_MAGIC = 0, H_VERSION = 4, H_QUANT = 6, H_GROUP = 8, H_DTYPE = 12,
       H_LAYERS = 14, H_HEADS = 18, H_HDIM = 22, H_SEQ = 26, H_MAXSEQ = 30,
       H_COMP = 34 };

/* io.c:39-102.  One change: the reference writes the first
 * n_kv_heads*seq_len*head_dim/64 groups of each plane, which is the intended
 * [head][pos][group] content only when seq_len == max_seq_len (the planes use
 * a per-head stride of max_seq_len); here each head's seq_len tokens are
 * written in turn, giving the same bytes in that case and the intended bytes
 * otherwise. */
int orc_cache_save(const orc_cache_t *c, const char *path)
{
    if (!c || !path) return -4;
    FILE *f = fopen(path, "wb");
    if (!f) return -1;
    int64_t gpd = c->head_dim / 64;
    int64_t gph = (int64_t)c->max_seq_len * gpd;
    int64_t g_head = (int64_t)c->seq_len * gpd;      /* groups per head */
    int64_t n_groups = (int64_t)c->n_kv_heads * c->head_dim * c->seq_len / 64;
    size_t raw = (size_t)n_groups * 40;
    size_t blk = orc_align64(raw);
    uint8_t hdr[ORC_HDR];
    memset(hdr, 0, sizeof(hdr));
    memcpy(hdr + H_MAGIC, "EAKV", 4);
    put_u16(hdr + H_VERSION, 1);
    put_u32(hdr + H_GROUP, 64);
    put_u32(hdr + H_LAYERS, (uint32_t)c->n_layers);
    put_u32(hdr + H_HEADS, (uint32_t)c->n_kv_heads);
    put_u32(hdr + H_HDIM, (uint32_t)c->head_dim);
    put_u32(hdr + H_SEQ, (uint32_t)c->seq_len);
    put_u32(hdr + H_MAXSEQ, (uint32_t)c->seq_len);   /* io.c:65 */
    fwrite(hdr, 1, ORC_HDR, f);
    size_t idx = (size_t)c->n_layers * 2 * 8;
    size_t start = orc_align64(ORC_HDR + idx);
    for (int i = 0; i < c->n_layers * 2; i++) {
        uint64_t off = start + (size_t)i * blk;
        uint8_t b[8];
        for (int k = 0; k < 8; k++) b[k] = (uint8_t)(off >> (8 * k));
        fwrite(b, 1, 8, f);
    }
    static const uint8_t zeros[64];
    fwrite(zeros, 1, start - (ORC_HDR + idx), f);
    for (int l = 0; l < c->n_layers; l++)
        for (int kv = 0; kv < 2; kv++) {
            const uint8_t *w = orc_cache_weights(c, l, kv);
            const float *s = orc_cache_scales(c, l, kv);
            const float *b = orc_cache_biases(c, l, kv);
            if (g_head > 0) {
                for (int h = 0; h < c->n_kv_heads; h++)
                    fwrite(w + h * gph * 32, 32, (size_t)g_head, f);
                for (int h = 0; h < c->n_kv_heads; h++)
                    fwrite(s + h * gph, 4, (size_t)g_head, f);
                for (int h = 0; h < c->n_kv_heads; h++)
                    fwrite(b + h * gph, 4, (size_t)g_head, f);
            }
            fwrite(zeros, 1, blk - raw, f);
        }
    int rc = ferror(f) ? -1 : 0;
    if (fclose(f) != 0) rc = -1;
    return rc;
}

/* io.c:104-160 */
int orc_cache_load(const char *path, orc_cache_t **out)
{
    if (!path || !out) return -4;
    FILE *f = fopen(path, "rb");
    if (!f) return -1;
    uint8_t hdr[ORC_HDR];
    if (fread(hdr, 1, ORC_HDR, f) != ORC_HDR) { fclose(f); return -2; }
    if (memcmp(hdr + H_MAGIC, "EAKV", 4) != 0) { fclose(f); return -2; }
    if (get_u16(hdr + H_VERSION) != 1) { fclose(f); return -2; }
    int nl = (int)get_u32(hdr + H_LAYERS), nh = (int)get_u32(hdr + H_HEADS);
    int hd = (int)get_u32(hdr + H_HDIM), sl = (int)get_u32(hdr + H_SEQ);
    orc_cache_t *c = orc_cache_create(nl, nh, hd, sl);
    if (!c) { fclose(f); return -3; }
    int64_t n_groups = (int64_t)nh * hd * sl / 64;
    size_t idx = (size_t)nl * 2 * 8;
    uint8_t *offs = malloc(idx);
    if (!offs) { orc_cache_free(c); fclose(f); return -3; }
    if (fread(offs, 1, idx, f) != idx) goto fail;
    for (int i = 0; i < nl * 2; i++) {
        uint64_t off = 0;
        for (int k = 0; k < 8; k++) off |= (uint64_t)offs[i * 8 + k] << (8 * k);
        if (fseek(f, (long)off, SEEK_SET) != 0) goto fail;
        uint8_t *w = (uint8_t *)orc_cache_weights(c, i / 2, i % 2);
        float *s = (float *)orc_cache_scales(c, i / 2, i % 2);
        float *b = (float *)orc_cache_biases(c, i / 2, i % 2);
        if (fread(w, 32, (size_t)n_groups, f) != (size_t)n_groups) goto fail;
        if (fread(s, 4, (size_t)n_groups, f) != (size_t)n_groups) goto fail;
        if (fread(b, 4, (size_t)n_groups, f) != (size_t)n_groups) goto fail;
    }
    c->seq_len = sl;
    free(offs);
    fclose(f);
    *out = c;
    return 0;
fail:
    free(offs);
    orc_cache_free(c);
    fclose(f);
    return -2;
}
