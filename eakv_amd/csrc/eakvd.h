/* eakvd.h — the thin C ABI between the C11 host library and the gfx950 HIP
 * kernels.  Plain C: no HIP types cross this boundary (streams are void*).
 *
 * Device layout of one cache (one hipMalloc, zero-filled):
 *   block p = layer*2 + kv  at  base + p*block_bytes, holding three planes
 *     weights  u8 [max_groups*32]   at block + 0
 *     scales   f32[max_groups]      at block + s_off
 *     biases   f32[max_groups]      at block + b_off
 *   group index inside a plane = h*gph + t*gpd + j  (gph = max_seq_len*gpd,
 *   gpd = head_dim/64), the indexing of reference src/cache.c:69,:137 and
 *   src/attention.c:7.  Block and plane starts are rounded up to 256 bytes.
 *   After the last block: EAKVD_TAIL_PAD bytes, then at ctr_off ctr_slots
 *   chunk counters, EAKVD_CTR_STRIDE bytes apart, zero between calls (the
 *   launches that merge their chunks themselves count on them).
 */
#ifndef EAKVD_H
#define EAKVD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Sequences per batched launch (kernel-argument arrays). */
#define EAKVD_MAX_BATCH 32

/* Bytes allocated after a cache's last plane: the fused kernel reads whole
 * tiles (at most 64 tokens of K and V, 64 B each, and their scales) past a
 * sequence's last token and masks them. */
#define EAKVD_TAIL_PAD (64 * 1024)

/* Bytes between two chunk counters: counters on separate 64-byte lines do
 * not serialize one another's atomics. */
#define EAKVD_CTR_STRIDE 64
/* Counters of a cache: one per kv head, and at least 256 (a fused launch
 * merges its chunks itself when every (sequence, kv head) unit of the call
 * has a counter in caches[0]; more units take a second launch). */
#define EAKVD_CTR_MIN_SLOTS 256

typedef struct {
    int     n_layers, n_kv_heads, head_dim, max_seq_len;
    int64_t gpd;          /* groups per token per head */
    int64_t gph;          /* groups per head in a plane */
    int64_t max_groups;   /* groups per plane */
    int64_t s_off, b_off; /* plane offsets inside a block, bytes */
    int64_t block_bytes;  /* bytes per (layer, kv) block */
    int64_t ctr_off;      /* chunk counters, after the blocks and the tail pad */
    int64_t ctr_slots;    /* how many */
    int64_t dev_bytes;    /* the whole device allocation */
} eakvd_geom;

void eakvd_geom_init(eakvd_geom *g, int n_layers, int n_kv_heads,
                     int head_dim, int max_seq_len);

/* ---- runtime (hip/runtime.hip); every function returns 0 or a HIP error */
int  eakvd_get_device(int *dev);
int  eakvd_set_device(int dev);
int  eakvd_malloc(void **p, size_t n);
int  eakvd_free(void *p);
int  eakvd_host_malloc(void **p, size_t n);   /* pinned */
int  eakvd_host_free(void *p);
int  eakvd_device_stream(int dev, void **s);   /* the caches' stream of device dev */
int  eakvd_stream_create(void **s);           /* non-blocking, default priority */
int  eakvd_stream_destroy(void *s);
int  eakvd_stream_sync(void *s);
int  eakvd_event_create(void **e);            /* no timing */
int  eakvd_event_destroy(void *e);
int  eakvd_event_record(void *e, void *s);
int  eakvd_event_sync(void *e);
int  eakvd_stream_wait_event(void *s, void *e);
int  eakvd_memset_async(void *p, int v, size_t n, void *s);
int  eakvd_memcpy_h2d_async(void *dst, const void *src, size_t n, void *s);
int  eakvd_memcpy_d2h_async(void *dst, const void *src, size_t n, void *s);
int  eakvd_memcpy_d2d_async(void *dst, const void *src, size_t n, void *s);
const char *eakvd_error_string(int err);

/* ---- quantize (hip/quantize.hip)
 * Source row r starts at src + r*row_stride and holds n_g groups of 64
 * contiguous f32.  Row r maps to cache c = r / (n_planes*nh),
 * plane = plane0 + (r / nh) % n_planes, head h = r % nh, and writes groups
 * h*gph + g_off[c] + g, g < n_g. */
typedef struct {
    const float *src;
    int64_t      row_stride;
    int64_t      n_rows;
    int64_t      n_g;
    int          nh;
    int          n_planes;
    int          plane0;
    int          n_caches;
    uint8_t     *base[EAKVD_MAX_BATCH];
    int64_t      g_off[EAKVD_MAX_BATCH];
} eakvd_quant_job;

int eakvd_quantize(const eakvd_geom *g, const eakvd_quant_job *job,
                   void *stream);

/* ---- attention kernels (hip/kscore.hip, hip/vsum.hip, hip/fused.hip)
 * Plane pointers come from one cache's device base and a layer. */

/* scores[qh*seq_len + t], q: [n_q][head_dim] (device pointers) */
int eakvd_k_score(const eakvd_geom *g, const uint8_t *base, int layer,
                  int seq_len, const float *q, int n_q, int n_kv,
                  float *scores, void *stream);

/* out[qh*head_dim + i] = sum_t w[qh*seq_len + t] * dequant(V[kv][t][i]).
 * work: device scratch of eakvd_v_sum_work_bytes() bytes. */
size_t eakvd_v_sum_work_bytes(const eakvd_geom *g, int seq_len, int n_q);
int eakvd_v_sum(const eakvd_geom *g, const uint8_t *base, int layer,
                int seq_len, const float *w, int n_q, int n_kv, float *out,
                void *work, void *stream);
/* The same on the matrix cores (hip/fused.hip), for 2 or more q heads per
 * kv head (above 8 as virtual kv heads of at most 8); returns -1 without
 * launching anything where it does not apply.
 * eakvd_v_sum tries it first. */
size_t eakvd_v_sum_mfma_work_bytes(const eakvd_geom *g, int seq_len, int n_q);
int eakvd_v_sum_mfma(const eakvd_geom *g, const uint8_t *base, int layer,
                     int seq_len, const float *w, int n_q, int n_kv, float *out,
                     void *work, void *stream);

/* Fused decode attention over a batch of same-geometry caches:
 * out[s][qh][i] = softmax_t(q[s][qh].K[s][kv][t] / sqrt(d)) . V[s][kv][t][i]
 * q, out: [n_seq][n_q][head_dim] device pointers. */
typedef struct {
    int            n_seq;
    const uint8_t *base[EAKVD_MAX_BATCH];
    int            seq_len[EAKVD_MAX_BATCH];
} eakvd_batch;

size_t eakvd_fused_work_bytes(const eakvd_geom *g, const eakvd_batch *b,
                              int n_q);
/* work: eakvd_fused_work_bytes() of device scratch for the per-chunk
 * partial results; launches that share it must not overlap.  ctr: the
 * counter region (g->ctr_slots counters at g->ctr_off of the cache whose
 * workspace is used, zero between calls), or NULL: the chunks are then
 * always merged by a second launch. */
int eakvd_fused(const eakvd_geom *g, const eakvd_batch *b, int layer,
                const float *q, int n_q, int n_kv, float *out, void *work,
                void *ctr, void *stream);
/* The launch eakvd_fused makes for this batch, head split and counter
 * region (ctr as eakvd_fused's): out[0] 1 for the matrix-core program (0:
 * the VALU program), [1] chunks per (sequence, virtual kv head) unit, [2] 1
 * when the chunks merge inside the launch (0: a merge launch follows), [3]
 * tokens per tile, [4] waves per block, [5] the most tiles a wave walks,
 * [6] quads of q heads per wave, [7] virtual kv heads per kv head. */
void eakvd_fused_plan(const eakvd_geom *g, const eakvd_batch *b, int n_q, int n_kv,
                      const void *ctr, int32_t *out);
/* The bytes of partials that eakvd_fused writes and reads for this batch
 * and head split (at most eakvd_fused_work_bytes()). */
size_t eakvd_fused_launch_bytes(const eakvd_geom *g, const eakvd_batch *b,
                                int n_q, int n_kv);

/* The library's static device scratch for the allocation-free entry point
 * (hip/fused.hip): EAKVD_SCRATCH_BYTES per device, held until the process
 * ends.  *p = its address on the current device (looked up once per device).
 * Returns 0 or a HIP error. */
#define EAKVD_SCRATCH_BYTES ((size_t)16 << 20)
int eakvd_scratch(void **p);

/* ---- whole-plane kernels (hip/planes.hip)
 * eakvd_dequantize: groups [g0, g0 + n) of block (layer, kv) to out
 * (f32[n][64], device).  eakvd_validate: the integrity check of the first n
 * groups of each of the n_blocks blocks; res (device, n_blocks words) gets
 * per block the minimum of g*4 + code over its failing groups, or all ones. */
int eakvd_dequantize(const eakvd_geom *g, const uint8_t *base, int layer, int kv,
                     int64_t g0, int64_t n, float *out, void *stream);
int eakvd_validate(const eakvd_geom *g, const uint8_t *base, int n_blocks,
                   int64_t n, unsigned long long *res, void *stream);

/* ---- ggml block type (hip/ggml.hip): 40-byte blocks of 64 values */
int eakvd_ggml_quantize_row(const float *src, void *dst, int64_t k, void *stream);
int eakvd_ggml_dequantize_row(const void *src, float *dst, int64_t k, void *stream);
int eakvd_ggml_vec_dot(int n, float *s, size_t bs, const void *vx, size_t bx,
                       const void *vy, size_t by, int nrc, void *stream);

#ifdef __cplusplus
}
#endif

#endif
