/* eakv_hip.h — MI355X extensions to the eakv C API (include/eakv.h).
 *
 * None of these has a counterpart in the reference, whose caches live in host
 * memory.  They exist because the reference API takes host pointers, which
 * forces a PCIe round trip per call on a GPU:
 *   - device-pointer forms of load/append/scores/output, asynchronous on a
 *     HIP stream (pass the hipStream_t as void*; NULL, or eakv_cache_stream()
 *     itself = the device's shared stream: one non-blocking stream per
 *     device, shared by every cache created on that device, so the device's
 *     caches' default-stream work runs in enqueue order);
 *   - batched append and batched fused decode attention over several caches
 *     of the same shape (one launch per layer for all sequences);
 *   - the fused single-pass softmax attention, which the reference compiles
 *     (kernels/fused_attention.ea:190-373) but never wires into its C API;
 *   - plane read-back and an error side channel for the void attention calls;
 *   - dequantization and the integrity check of GPU-resident planes, which the
 *     reference runs on its host planes from its benchmark and CLI.
 * Device-pointer calls return when the work is enqueued; results are ready
 * after eakv_cache_sync() or a wait on the stream.  The host-pointer calls
 * of include/eakv.h (and eakv_attention_fused, eakv_cache_read_planes,
 * eakv_dequantize_range, eakv_validate, eakv_cache_save/load) run on a
 * stream of the cache's own, after the device-pointer work still pending for
 * that cache on the shared stream, and wait for that stream alone: calls on
 * distinct caches from distinct threads do not wait for one another (the
 * reference's "thread-safe for distinct caches", include/eakv.h:3).  A
 * device-pointer call on a caller's stream first waits, on the device, for
 * the work pending for its caches on the shared stream; after a load or an
 * append on a caller's stream, the shared stream's later work and the
 * cache's later host-pointer calls wait for it.  Calls on one cache that use
 * its device workspace (V-sum and fused partials, host staging) are ordered
 * among themselves whatever their streams (an event recorded on a caller's
 * stream, waited for by the next use).  Any other ordering between two
 * caller streams (e.g. K/V appended on one caller's stream and read on
 * another) is the caller's, as for any work on two streams.
 */
#ifndef EAKV_HIP_H
#define EAKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "eakv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A HIP runtime or kernel launch failure. */
#define EAKV_ERR_DEVICE     -5

/* Most recent error recorded by a call on this thread (EAKV_OK if none since
 * eakv_clear_error) and its message. */
int         eakv_last_error(void);
const char *eakv_last_error_message(void);
void        eakv_clear_error(void);

/* The HIP device ordinal the cache lives on, the device's shared stream (the
 * NULL-stream default of the device-pointer calls), and a wait for all work
 * enqueued on that stream (by any cache of the device). */
int   eakv_cache_device(const eakv_cache_t *cache);
void *eakv_cache_stream(const eakv_cache_t *cache);
int   eakv_cache_sync(const eakv_cache_t *cache);

/* Copy the planes of block (layer, kv_idx) to host buffers holding
 * n_kv_heads*max_seq_len*head_dim/64 groups each (weights 32 B per group). */
int eakv_cache_read_planes(const eakv_cache_t *cache, int layer, int kv_idx,
                           uint8_t *weights, float *scales, float *biases);

/* eakv_cache_load_raw / eakv_cache_append with device input (same layout and
 * validation; seq_len is set by load_raw and untouched by append). */
int eakv_cache_load_raw_device(eakv_cache_t *cache, const float *d_data,
                               int seq_len, void *stream);
int eakv_cache_append_device(eakv_cache_t *cache, const float *d_data,
                             int layer, int kv_idx, int n_tokens,
                             void *stream);

/* Append n_tokens to every layer and both K/V of n_caches caches in one
 * launch.  d_data: f32[n_caches][n_layers][2][n_kv_heads][n_tokens][head_dim].
 * Caches must share n_layers, n_kv_heads, head_dim, max_seq_len and device;
 * seq_len is not changed (call eakv_cache_advance on each).  The launch runs
 * on `stream` (NULL: the shared stream) after the device-pointer calls
 * already enqueued there for every named cache, and later work on the shared
 * stream and every later host-pointer call on a named cache run after it. */
int eakv_append_batch_device(eakv_cache_t *const *caches, int n_caches,
                             const float *d_data, int n_tokens, void *stream);

/* eakv_attention_scores / eakv_attention_output on device buffers. */
int eakv_attention_scores_device(const eakv_cache_t *cache, const float *d_q,
                                 int layer, int n_q_heads, int n_kv_heads,
                                 float *d_scores, void *stream);
int eakv_attention_output_device(const eakv_cache_t *cache,
                                 const float *d_weights, int layer,
                                 int n_q_heads, int n_kv_heads, float *d_out,
                                 void *stream);

/* Fused decode attention softmax(q.K^T/sqrt(d)).V over the cache's seq_len
 * tokens, host pointers, synchronous: queries f32[n_q][head_dim],
 * output_out f32[n_q][head_dim]. */
int eakv_attention_fused(const eakv_cache_t *cache, const float *queries,
                         int layer, int n_q_heads, int n_kv_heads,
                         float *output_out);

/* Fused decode attention for n_caches same-shape caches (each over its own
 * seq_len) in one launch: d_q, d_out f32[n_caches][n_q][head_dim].  Uses the
 * workspace of caches[0].  The launch runs on `stream` (NULL: the shared
 * stream) after the work already enqueued there for every named cache
 * (device-pointer calls with a NULL stream, e.g. an append); with a NULL
 * stream, later host-pointer calls on any named cache run after it.  Work
 * that later overwrites their tokens from a caller's stream must wait for
 * `stream` first. */
int eakv_attention_fused_batch_device(eakv_cache_t *const *caches,
                                      int n_caches, int layer,
                                      const float *d_q, int n_q_heads,
                                      int n_kv_heads, float *d_out,
                                      void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): eakv_attention_fused_batch_device with the chunk
 * partials in the library's static device scratch of 16 MiB per device
 * instead of caches[0]'s workspace, so no call path allocates.  Same
 * arguments, results and stream ordering; EAKV_ERR_INVALID when the launch
 * would need more than 16 MiB of partials (n_caches * n_q_heads * chunks *
 * (head_dim + 2) * 4 bytes: 1.1 MB for 8 caches of 32 q heads over 32K
 * tokens, 1.1 MB for 64 q heads over 128K tokens).
 * Every call on one device shares that scratch: calls that overlap in time
 * on one device race, and ordering them is the caller's. */
int eakv_attention_fused_batch_device_noalloc(eakv_cache_t *const *caches,
                                              int n_caches, int layer,
                                              const float *d_q, int n_q_heads,
                                              int n_kv_heads, float *d_out,
                                              void *stream);

/* No counterpart in the reference (its fused kernel is one CPU loop).  The
 * launch that eakv_attention_fused_batch_device (noalloc = 0) or its
 * allocation-free form (noalloc != 0) makes for these caches at their
 * current seq_len and this head split, for diagnostics and tests; nothing is
 * launched.  plan (8 entries): [0] 1 for the matrix-core program, 0 for the
 * VALU program (layer blocks beyond 32-bit buffer offsets); [1] chunks per
 * (sequence, kv head) unit; [2] 1 when the chunks are merged inside the
 * launch (up to 16 chunks per unit), 0 when a merge launch follows; [3]
 * tokens per tile; [4] waves per
 * block; [5] the most tiles one wave walks; [6] quads of q heads per wave;
 * [7] virtual kv heads per kv head (groups above 8 q heads). */
int eakv_attention_fused_plan(eakv_cache_t *const *caches, int n_caches, int n_q_heads,
                              int n_kv_heads, int noalloc, int32_t *plan);

/* Dequantize groups [group_start, group_start + group_count) of the (layer,
 * kv_idx) planes to f32, 64 values per group in group order: value =
 * fma(nibble, scale, bias) with byte k of a group holding dim k (low nibble)
 * and dim k+32 (high nibble).  Group indices are plane indices
 * (h*max_seq_len*head_dim/64 + t*head_dim/64 + j).  Replaces the reference's
 * q4_dequantize_range_avx512_f32 (kernels/dequantize_avx512.ea:55-89; the
 * whole plane, q4_dequantize_avx512_f32, :10-53, is group_start 0 and
 * group_count n_kv_heads*max_seq_len*head_dim/64).  _device: d_out on the
 * device, asynchronous on the stream; the other form writes host memory and
 * returns when done. */
int eakv_dequantize_range_device(const eakv_cache_t *cache, int layer, int kv_idx,
                                 int64_t group_start, int64_t group_count,
                                 float *d_out, void *stream);
int eakv_dequantize_range(const eakv_cache_t *cache, int layer, int kv_idx,
                          int64_t group_start, int64_t group_count, float *out);

/* Integrity check of every (layer, kv) block, as the reference's `validate`
 * command (src/cli.c:39-98) runs q4_validate (kernels/validate.ea:14-71) on
 * the first n_kv_heads*head_dim*seq_len/64 groups of each block:
 * results[layer*2 + kv] = 0 (ok), 1 (NaN scale), 2 (NaN bias) or 3 (negative
 * scale), the code of the block's first failing group.  Synchronous. */
int eakv_validate(const eakv_cache_t *cache, int32_t *results);

/* The ggml block type of reference include/eakv_ggml.h:27-31
 * (block_q4_1_eakv: u8 qs[32] split-packed, f32 d, f32 m; 64 values in 40
 * bytes), device-pointer forms of its type-trait callbacks for a HIP ggml
 * backend, on the current HIP device and the given stream (NULL: the
 * default stream).  Pointers and byte strides are 4-byte aligned.
 *   _quantize_row:   eakv_quantize_row (src/ggml_type.c:21-90), k values
 *                    (k % 64 == 0) to k/64 blocks;
 *   _dequantize_row: eakv_dequantize_row (:96-133), value = fma(n, d, m)
 *                    (the reference's AVX-512 path; its scalar fallback
 *                    rounds n*d before adding m);
 *   _vec_dot:        eakv_vec_dot_q4_f32 (:142-242) for nrc rows of any
 *                    count: s[r] = row r of vx . row r of vy over n values,
 *                    the AVX-512 path's 16 lane accumulators and tree. */
int eakv_ggml_quantize_row_device(const float *d_src, void *d_dst, int64_t k, void *stream);
int eakv_ggml_dequantize_row_device(const void *d_src, float *d_dst, int64_t k, void *stream);
int eakv_ggml_vec_dot_device(int n, float *d_s, size_t bs, const void *d_vx, size_t bx,
                             const void *d_vy, size_t by, int nrc, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* EAKV_HIP_H */
