/* eakv.h — Q4_1 (group 64) KV-cache library, MI355X (gfx950) implementation.
 *
 * Drop-in for the reference public API (reference include/eakv.h:1-89): every
 * declaration below keeps the reference's name, signature, error codes and
 * semantics.  Cache planes live in HBM of the HIP device that was current when
 * the cache was created; every call taking host pointers copies through that
 * device and has completed when it returns.
 *
 * Distinct caches may be used from distinct threads concurrently (reference
 * include/eakv.h:3); one cache must not be used from two threads at once.
 */
#ifndef EAKV_H
#define EAKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque handle (reference include/eakv.h:15). */
typedef struct eakv_cache eakv_cache_t;

/* Error codes (reference include/eakv.h:18-22). */
#define EAKV_OK              0
#define EAKV_ERR_IO         -1
#define EAKV_ERR_FORMAT     -2
#define EAKV_ERR_ALLOC      -3
#define EAKV_ERR_INVALID    -4

/* Lifecycle (reference include/eakv.h:25-27, src/cache.c:11-58).
 * Returns NULL for non-positive dimensions, when n_kv_heads*head_dim is not a
 * multiple of 64, or when device memory cannot be allocated.  The planes are
 * zero-filled.  eakv_cache_free(NULL) is a no-op. */
eakv_cache_t *eakv_cache_create(int n_layers, int n_kv_heads,
                                int head_dim, int max_seq_len);
void          eakv_cache_free(eakv_cache_t *cache);

/* Bulk quantize (reference include/eakv.h:29-32, src/cache.c:60-100).
 * data: host f32[n_layers][2][n_kv_heads][seq_len][head_dim].  Overwrites from
 * position 0 and sets seq_len.  EAKV_ERR_INVALID for NULL arguments or
 * seq_len outside 1..max_seq_len. */
int eakv_cache_load_raw(eakv_cache_t *cache, const float *data, int seq_len);

/* Append (reference include/eakv.h:34-40, src/cache.c:102-151).
 * data: host f32[n_kv_heads][n_tokens][head_dim] for one (layer, kv_idx),
 * kv_idx 0 = K, 1 = V.  Written at the current seq_len; seq_len is NOT
 * changed (call eakv_cache_advance once all layers and K/V are appended). */
int eakv_cache_append(eakv_cache_t *cache, const float *data,
                      int layer, int kv_idx, int n_tokens);

/* seq_len += n_tokens (reference include/eakv.h:42-43, src/cache.c:153-160). */
int eakv_cache_advance(eakv_cache_t *cache, int n_tokens);

/* seq_len = 0, nothing freed (reference include/eakv.h:45-46). */
void eakv_cache_clear(eakv_cache_t *cache);

/* O(1) checkpoint / restore of seq_len (reference include/eakv.h:48-53,
 * src/cache.c:166-176).  restore accepts 0 <= seq_len <= current seq_len. */
int eakv_checkpoint(eakv_cache_t *cache);
int eakv_restore(eakv_cache_t *cache, int seq_len);

/* Attention on the packed cache (reference include/eakv.h:55-71,
 * src/attention.c:3-63).
 *   MHA: n_q_heads == n_kv_heads; GQA: q head h reads kv head h/(n_q/n_kv).
 *   queries:    host f32[n_q_heads][head_dim]
 *   scores_out: host f32[n_q_heads][seq_len]   (Q.K^T / sqrt(head_dim))
 *   weights:    host f32[n_q_heads][seq_len]   (softmax weights)
 *   output_out: host f32[n_q_heads][head_dim]
 * The reference does not validate these calls.  Here a call with head_dim not
 * 64 or 128, n_q_heads not a multiple of n_kv_heads, n_kv_heads larger than the
 * cache's, or a layer out of range writes nothing and records EAKV_ERR_INVALID
 * for eakv_last_error() (declared in eakv_hip.h). */
void eakv_attention_scores(const eakv_cache_t *cache, const float *queries,
                           int layer, int n_q_heads, int n_kv_heads,
                           float *scores_out);

void eakv_attention_output(const eakv_cache_t *cache, const float *weights,
                           int layer, int n_q_heads, int n_kv_heads,
                           float *output_out);

/* .eakv file I/O (reference include/eakv.h:73-75, src/io.c:39-160). */
int eakv_cache_save(const eakv_cache_t *cache, const char *path);
int eakv_cache_load(const char *path, eakv_cache_t **out);

/* Info (reference include/eakv.h:77-83, src/cache.c:178-201).
 * eakv_cache_n_heads returns the number of KV heads. */
int   eakv_cache_seq_len(const eakv_cache_t *cache);
int   eakv_cache_n_layers(const eakv_cache_t *cache);
int   eakv_cache_n_heads(const eakv_cache_t *cache);
int   eakv_cache_head_dim(const eakv_cache_t *cache);
int   eakv_cache_max_seq_len(const eakv_cache_t *cache);
float eakv_cache_compression_ratio(const eakv_cache_t *cache);

#ifdef __cplusplus
}
#endif

#endif /* EAKV_H */
