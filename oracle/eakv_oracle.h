/* eakv_oracle.h — CPU restatement of the reference eakv hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the oracle that the HIP library's
 * results are compared against; it is never linked into, loaded by or called
 * from the product library.  Only tests/, __graft_entry__.smoke() and the CPU-baseline
 * leg of bench.py may load it.
 *
 * Every function restates the arithmetic of one reference kernel (Ea source,
 * cited per function) in plain C11: explicit fmaf where the reference fuses,
 * no contraction elsewhere (built with -ffp-contract=off), f32 throughout.
 *
 * Choices the reference sources leave open (the Ea compiler is not available
 * offline, so its codegen cannot be inspected):
 *   - reduce_add over 16 lanes: pairwise halving tree
 *       v8[i]=a[i]+a[i+8]; v4[i]=v8[i]+v8[i+4]; v2[i]=v4[i]+v4[i+2]; v2[0]+v2[1]
 *   - to_i32(f32): x86 cvttss2si semantics (truncate; NaN or out of range
 *     gives INT32_MIN), which is what an LLVM fptosi lowers to on x86-64.
 *   - exp(): the C library expf.
 */
#ifndef EAKV_ORACLE_H
#define EAKV_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- kernels (one group = 64 values = 32 split-packed bytes + scale + bias) */

/* kernels/quantize_simd.ea:9-59 plus the i32->u8 narrowing of
 * src/cache.c:90-92 (lossless: every packed value is 0..255). */
void orc_quantize_split(const float *src, uint8_t *weights, float *scales,
                        float *biases, int64_t n_groups);

/* Dequantize groups to f32[n_groups][64] in dim order, value j =
 * fma(nibble_j, scale, bias) (dequantize_avx512.ea and every fused kernel,
 * e.g. fused_k_score.ea:207). */
void orc_dequantize(const uint8_t *weights, const float *scales,
                    const float *biases, float *out, int64_t n_groups);

/* kernels/dequantize_avx512.ea:55-89 (q4_dequantize_range_avx512_f32):
 * groups [group_start, group_start + group_count) to out[i*64 + j]. */
void orc_dequantize_range(const uint8_t *weights, const float *scales,
                          const float *biases, float *out, int64_t group_start,
                          int64_t group_count);

/* kernels/validate.ea:14-71 (q4_validate): the first failing group's code
 * over groups 0..n_groups-1 in order, per group 1 = NaN scale, 2 = NaN bias,
 * 3 = negative scale (NaN tested on the bits), else 0. */
int32_t orc_validate(const float *scales, const float *biases, int64_t n_groups);

/* ---- ggml block type (reference include/eakv_ggml.h:27-31): 40-byte
 * blocks {u8 qs[32] split-packed, f32 d, f32 m} of 64 values.
 * orc_ggml_quantize_row: src/ggml_type.c:21-87 (min/max scan from element 0,
 * d = range/15, id = range > 0 ? 15/range : 0, q = clamp(trunc(0.5 +
 * (x - min)*id), 0, 15); the AVX-512 and scalar paths agree on finite
 * input).  orc_ggml_dequantize_row: ggml_type.c:96-133, the AVX-512 path,
 * value = fma(nibble, d, m).  orc_ggml_vec_dot: ggml_type.c:142-242, the
 * AVX-512 path: 16 lane accumulators, per block for c = 0, 1 the low then
 * the high nibbles, acc = fma(fma(n, d, m), y, acc), then the lanes summed
 * by the tree of orc_reduce16; rows r < nrc at byte strides bs, bx, by. */
void orc_ggml_quantize_row(const float *src, uint8_t *dst, int64_t k);
void orc_ggml_dequantize_row(const uint8_t *src, float *dst, int64_t k);
void orc_ggml_vec_dot(int n, float *s, size_t bs, const uint8_t *vx, size_t bx,
                      const float *vy, size_t by, int nrc);

/* 16-lane reduce_add of the reference kernels (tree order above). */
float orc_reduce16(const float *acc);

/* x86 cvttss2si semantics. */
int32_t orc_to_i32(float v);

/* MHA K-score: kernels/fused_k_score.ea:161-235 (d=128),
 * kernels/fused_k_score_64.ea:100-153 (d=64).
 * scores[h*seq_len + t]; head h reads groups from h*groups_per_head. */
void orc_k_score_mha(int head_dim, const float *q, const uint8_t *kw,
                     const float *ks, const float *kb, float *scores,
                     int seq_len, int n_heads, int64_t groups_per_head);

/* GQA K-score: kernels/fused_k_score_gqa.ea:7-99 (d=128),
 * kernels/fused_k_score_gqa_64.ea:6-73 (d=64). */
void orc_k_score_gqa(int head_dim, const float *q, const uint8_t *kw,
                     const float *ks, const float *kb, float *scores,
                     int seq_len, int n_q_heads, int n_kv_heads,
                     int64_t groups_per_head);

/* MHA V-sum: kernels/fused_v_sum.ea:83-163 (d=128),
 * kernels/fused_v_sum_64.ea:55-110 (d=64). out[h*head_dim + i]. */
void orc_v_sum_mha(int head_dim, const float *w, const uint8_t *vw,
                   const float *vs, const float *vb, float *out,
                   int seq_len, int n_heads, int64_t groups_per_head);

/* GQA V-sum: kernels/fused_k_score_gqa.ea:106-305 (d=128),
 * kernels/fused_k_score_gqa_64.ea:79-209 (d=64). */
void orc_v_sum_gqa(int head_dim, const float *w, const uint8_t *vw,
                   const float *vs, const float *vb, float *out,
                   int seq_len, int n_q_heads, int n_kv_heads,
                   int64_t groups_per_head);

/* Two-pass fused softmax attention: kernels/fused_attention.ea:190-373
 * (MHA, d=128 in the reference).  Extended here, per q head, to GQA
 * (kv head = q/(n_q/n_kv)) and d=64 with the same two-pass arithmetic. */
void orc_fused_attention(int head_dim, const float *q,
                         const uint8_t *kw, const float *ks, const float *kb,
                         const uint8_t *vw, const float *vs, const float *vb,
                         float *out, int seq_len, int n_q_heads,
                         int n_kv_heads, int64_t groups_per_head);

/* The same on AVX-512 (eakv_oracle_avx512.c): the reference's fused kernel
 * as its compiler emits it, 16 lanes per instruction, bit-identical to
 * orc_fused_attention.  Call only where orc_avx512_available() is nonzero. */
int  orc_avx512_available(void);
void orc_fused_attention_avx512(int head_dim, const float *q,
                                const uint8_t *kw, const float *ks, const float *kb,
                                const uint8_t *vw, const float *vs, const float *vb,
                                float *out, int seq_len, int n_q_heads,
                                int n_kv_heads, int64_t groups_per_head);

/* Row softmax between K-score and V-sum (the caller's step; HOWTO.md:52),
 * defined like the fused kernel: m = max(-1e6, row), w = expf(s-m),
 * sequential sum, w *= 1/sum. */
void orc_softmax_rows(const float *scores, float *weights, int n_rows,
                      int seq_len);

/* ---- cache: restatement of src/cache.c, src/attention.c (host memory) */

typedef struct orc_cache orc_cache_t;

orc_cache_t *orc_cache_create(int n_layers, int n_kv_heads, int head_dim,
                              int max_seq_len);
void orc_cache_free(orc_cache_t *c);
int  orc_cache_load_raw(orc_cache_t *c, const float *data, int seq_len);
int  orc_cache_append(orc_cache_t *c, const float *data, int layer,
                      int kv_idx, int n_tokens);
int  orc_cache_advance(orc_cache_t *c, int n_tokens);
void orc_cache_clear(orc_cache_t *c);
int  orc_checkpoint(orc_cache_t *c);
int  orc_restore(orc_cache_t *c, int seq_len);
void orc_attention_scores(const orc_cache_t *c, const float *queries,
                          int layer, int n_q_heads, int n_kv_heads,
                          float *scores_out);
void orc_attention_output(const orc_cache_t *c, const float *weights,
                          int layer, int n_q_heads, int n_kv_heads,
                          float *output_out);
void orc_attention_fused(const orc_cache_t *c, const float *queries,
                         int layer, int n_q_heads, int n_kv_heads,
                         float *output_out);
void orc_attention_fused_avx512(const orc_cache_t *c, const float *queries,
                                int layer, int n_q_heads, int n_kv_heads,
                                float *output_out);
/* eakv_attention_scores / eakv_attention_output of the oracle cache on
 * AVX-512 (the reference's unfused kernels as the Ea compiler emits them),
 * bit-identical to orc_attention_scores / orc_attention_output.  Call only
 * where orc_avx512_available() is nonzero. */
void orc_attention_scores_avx512(const orc_cache_t *c, const float *queries,
                                 int layer, int n_q_heads, int n_kv_heads,
                                 float *scores_out);
void orc_attention_output_avx512(const orc_cache_t *c, const float *weights,
                                 int layer, int n_q_heads, int n_kv_heads,
                                 float *output_out);
int  orc_cache_seq_len(const orc_cache_t *c);
int  orc_cache_n_layers(const orc_cache_t *c);
int  orc_cache_n_heads(const orc_cache_t *c);
int  orc_cache_head_dim(const orc_cache_t *c);
int  orc_cache_max_seq_len(const orc_cache_t *c);
float orc_cache_compression_ratio(const orc_cache_t *c);

/* Plane access: pointers into the (layer, kv) block; each plane holds
 * n_kv_heads*max_seq_len*head_dim/64 groups. */
const uint8_t *orc_cache_weights(const orc_cache_t *c, int layer, int kv);
const float   *orc_cache_scales(const orc_cache_t *c, int layer, int kv);
const float   *orc_cache_biases(const orc_cache_t *c, int layer, int kv);
int64_t        orc_cache_max_groups(const orc_cache_t *c);

/* .eakv files: src/io.c:39-160 (see orc_cache_save for the one change). */
int orc_cache_save(const orc_cache_t *c, const char *path);
int orc_cache_load(const char *path, orc_cache_t **out);

#ifdef __cplusplus
}
#endif

#endif
