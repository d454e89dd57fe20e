/* attention.c — attention dispatch (host C11).
 *
 * Reference src/attention.c:3-63 picks one of four CPU kernels from
 * head_dim (64 or not) and n_q == n_kv.  Here the head_dim / GQA choice is
 * made inside the HIP launchers (eakvd.h); this file validates, stages host
 * buffers through the cache's device workspace (small ones through its
 * pinned host scratch as well) and waits for the result.
 */
#include <string.h>

#include "internal.h"

static int attn_check(const eakv_cache_t *c, int layer, int n_q, int n_kv)
{
    if (!c) return eakvi_set_error(EAKV_ERR_INVALID, "attention: NULL cache");
    if (c->head_dim != 64 && c->head_dim != 128)
        return eakvi_set_error(EAKV_ERR_INVALID,
                              "attention: head_dim %d not 64 or 128",
                              c->head_dim);
    if (layer < 0 || layer >= c->n_layers)
        return eakvi_set_error(EAKV_ERR_INVALID, "attention: layer out of range");
    if (n_kv <= 0 || n_kv > c->n_kv_heads || n_q < n_kv || n_q % n_kv != 0)
        return eakvi_set_error(EAKV_ERR_INVALID,
                              "attention: n_q %d / n_kv %d invalid for a cache "
                              "of %d kv heads", n_q, n_kv, c->n_kv_heads);
    return EAKV_OK;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }


/* ------------------------------------------------------------------------ */
/* K-score                                                                   */

int eakv_attention_scores_device(const eakv_cache_t *c, const float *d_q,
                                 int layer, int n_q, int n_kv,
                                 float *d_scores, void *stream)
{
    int rc = attn_check(c, layer, n_q, n_kv);
    if (rc) return rc;
    if (!d_q || !d_scores)
        return eakvi_set_error(EAKV_ERR_INVALID, "scores: NULL buffer");
    int prev;
    rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    void *st = eakvi_stream_or_default(c, stream);
    /* a caller's stream: after the cache's work pending on the shared stream */
    rc = eakvi_order_before((eakv_cache_t *)c, st);
    if (rc == EAKV_OK) {
        int e = eakvd_k_score(&c->geom, c->dev, layer, c->seq_len, d_q, n_q, n_kv,
                              d_scores, st);
        if (e) rc = eakvi_hip_fail(e, "k_score launch");
    }
    eakvi_leave(prev);
    return rc;
}

/* reference src/attention.c:3-32 */
void eakv_attention_scores(const eakv_cache_t *cc, const float *queries,
                           int layer, int n_q, int n_kv, float *scores_out)
{
    eakv_cache_t *c = (eakv_cache_t *)cc;
    if (attn_check(c, layer, n_q, n_kv)) return;
    if (!queries || !scores_out) {
        eakvi_set_error(EAKV_ERR_INVALID, "scores: NULL buffer");
        return;
    }
    int prev;
    if (eakvi_enter(c, &prev)) return;
    const size_t qb = (size_t)n_q * c->head_dim * 4;
    const size_t sb = (size_t)n_q * c->seq_len * 4;
    void *st = c->hstream;
    int rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, align256(qb) + sb);
    const int began = rc == EAKV_OK;
    eakvi_bounce bo = {NULL, 0};
    if (began) {
        float *dq = (float *)c->work;
        float *ds = (float *)((char *)c->work + align256(qb));
        eakvi_bounce_begin(c, qb, sb, &bo);
        int e = eakvi_bounce_in(&bo, dq, queries, qb, st);
        if (!e) e = eakvd_k_score(&c->geom, c->dev, layer, c->seq_len, dq, n_q,
                                  n_kv, ds, st);
        if (!e) e = eakvi_bounce_out(&bo, scores_out, ds, sb, st);
        if (e) rc = eakvi_hip_fail(e, "attention_scores");
    }
    rc = eakvi_host_end(c, rc, began, "attention_scores");
    eakvi_bounce_end(&bo, rc, scores_out, sb);
    eakvi_leave(prev);
}

/* ------------------------------------------------------------------------ */
/* V-sum                                                                     */

int eakv_attention_output_device(const eakv_cache_t *cc, const float *d_w,
                                 int layer, int n_q, int n_kv, float *d_out,
                                 void *stream)
{
    eakv_cache_t *c = (eakv_cache_t *)cc;
    int rc = attn_check(c, layer, n_q, n_kv);
    if (rc) return rc;
    if (!d_w || !d_out)
        return eakvi_set_error(EAKV_ERR_INVALID, "output: NULL buffer");
    int prev;
    rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    void *st = eakvi_stream_or_default(c, stream);
    /* a caller's stream: after the cache's work pending on the shared
     * stream, its workspace uses there included (a device-side wait) */
    rc = eakvi_order_before(c, st);
    if (rc == EAKV_OK)
        rc = eakvi_work_begin(c, st, eakvd_v_sum_work_bytes(&c->geom, c->seq_len, n_q));
    if (rc == EAKV_OK) {
        int e = eakvd_v_sum(&c->geom, c->dev, layer, c->seq_len, d_w, n_q, n_kv,
                            d_out, c->work, st);
        if (e) rc = eakvi_hip_fail(e, "v_sum launch");
        int e2 = eakvi_work_end(c, st);
        if (rc == EAKV_OK) rc = e2;
    }
    eakvi_leave(prev);
    return rc;
}

/* reference src/attention.c:34-63 */
void eakv_attention_output(const eakv_cache_t *cc, const float *weights,
                           int layer, int n_q, int n_kv, float *output_out)
{
    eakv_cache_t *c = (eakv_cache_t *)cc;
    if (attn_check(c, layer, n_q, n_kv)) return;
    if (!weights || !output_out) {
        eakvi_set_error(EAKV_ERR_INVALID, "output: NULL buffer");
        return;
    }
    int prev;
    if (eakvi_enter(c, &prev)) return;
    const size_t wb = (size_t)n_q * c->seq_len * 4;
    const size_t ob = (size_t)n_q * c->head_dim * 4;
    const size_t pb = eakvd_v_sum_work_bytes(&c->geom, c->seq_len, n_q);
    void *st = c->hstream;
    int rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, align256(wb) + align256(ob) + pb);
    const int began = rc == EAKV_OK;
    eakvi_bounce bo = {NULL, 0};
    if (began) {
        float *dw = (float *)c->work;
        float *dout = (float *)((char *)c->work + align256(wb));
        void *part = (char *)c->work + align256(wb) + align256(ob);
        eakvi_bounce_begin(c, wb, ob, &bo);
        int e = eakvi_bounce_in(&bo, dw, weights, wb, st);
        if (!e) e = eakvd_v_sum(&c->geom, c->dev, layer, c->seq_len, dw, n_q,
                                n_kv, dout, part, st);
        if (!e) e = eakvi_bounce_out(&bo, output_out, dout, ob, st);
        if (e) rc = eakvi_hip_fail(e, "attention_output");
    }
    rc = eakvi_host_end(c, rc, began, "attention_output");
    eakvi_bounce_end(&bo, rc, output_out, ob);
    eakvi_leave(prev);
}

/* ------------------------------------------------------------------------ */
/* fused decode attention                                                    */

/* Partials go at the end of caches[0]'s workspace (reserved by the caller). */
static int fused_launch(eakv_cache_t *const *caches, int n, int layer,
                        const float *d_q, int n_q, int n_kv, float *d_out,
                        void *stream)
{
    eakv_cache_t *c0 = caches[0];
    eakvd_batch b;
    memset(&b, 0, sizeof(b));
    b.n_seq = n;
    for (int i = 0; i < n; i++) {
        b.base[i] = caches[i]->dev;
        b.seq_len[i] = caches[i]->seq_len;
    }
    const size_t need = eakvd_fused_work_bytes(&c0->geom, &b, n_q);
    return eakvd_fused(&c0->geom, &b, layer, d_q, n_q, n_kv, d_out,
                       (char *)c0->work + (c0->work_bytes - need),
                       c0->dev + c0->geom.ctr_off, stream);
}

int eakv_attention_fused_batch_device(eakv_cache_t *const *caches,
                                      int n_caches, int layer,
                                      const float *d_q, int n_q, int n_kv,
                                      float *d_out, void *stream)
{
    if (!caches || n_caches <= 0 || n_caches > EAKVD_MAX_BATCH || !d_q || !d_out)
        return eakvi_set_error(EAKV_ERR_INVALID, "fused_batch: invalid argument");
    for (int i = 0; i < n_caches; i++) {
        if (!caches[i])
            return eakvi_set_error(EAKV_ERR_INVALID, "fused_batch: NULL cache");
        const eakv_cache_t *a = caches[0], *b = caches[i];
        if (a->n_layers != b->n_layers || a->n_kv_heads != b->n_kv_heads ||
            a->head_dim != b->head_dim || a->max_seq_len != b->max_seq_len ||
            a->device != b->device)
            return eakvi_set_error(EAKV_ERR_INVALID,
                                  "fused_batch: caches differ in shape");
    }
    eakv_cache_t *c0 = caches[0];
    int rc = attn_check(c0, layer, n_q, n_kv);
    if (rc) return rc;
    int prev;
    rc = eakvi_enter(c0, &prev);
    if (rc) return rc;
    void *st = eakvi_batch_stream(caches, n_caches, stream);
    /* a caller's stream: after the work pending for each cache on the shared
     * stream (its appends, and caches[0]'s workspace uses there), by a
     * device-side wait where there is such */
    for (int i = 0; rc == EAKV_OK && i < n_caches; i++)
        rc = eakvi_order_before(caches[i], st);
    eakvd_batch b;
    memset(&b, 0, sizeof(b));
    b.n_seq = n_caches;
    for (int i = 0; i < n_caches; i++) b.seq_len[i] = caches[i]->seq_len;
    if (rc == EAKV_OK)
        rc = eakvi_work_begin(c0, st, eakvd_fused_work_bytes(&c0->geom, &b, n_q));
    if (rc == EAKV_OK) {
        int e = fused_launch(caches, n_caches, layer, d_q, n_q, n_kv, d_out, st);
        if (e) rc = eakvi_hip_fail(e, "fused launch");
        int e2 = eakvi_work_end(c0, st);
        if (rc == EAKV_OK) rc = e2;
    }
    eakvi_leave(prev);
    return rc;
}

int eakv_attention_fused(const eakv_cache_t *cc, const float *queries,
                         int layer, int n_q, int n_kv, float *output_out)
{
    eakv_cache_t *c = (eakv_cache_t *)cc;
    int rc = attn_check(c, layer, n_q, n_kv);
    if (rc) return rc;
    if (!queries || !output_out)
        return eakvi_set_error(EAKV_ERR_INVALID, "fused: NULL buffer");
    int prev;
    rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    eakvd_batch b;
    memset(&b, 0, sizeof(b));
    b.n_seq = 1;
    b.seq_len[0] = c->seq_len;
    const size_t io = align256((size_t)n_q * c->head_dim * 4);
    const size_t pb = eakvd_fused_work_bytes(&c->geom, &b, n_q);
    void *st = c->hstream;
    rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, 2 * io + pb);
    const int began = rc == EAKV_OK;
    const size_t qb = (size_t)n_q * c->head_dim * 4;
    eakvi_bounce bo = {NULL, 0};
    if (began) {
        float *dq = (float *)c->work;
        float *dout = (float *)((char *)c->work + io);
        eakvi_bounce_begin(c, qb, qb, &bo);
        int e = eakvi_bounce_in(&bo, dq, queries, qb, st);
        if (!e) e = fused_launch(&c, 1, layer, dq, n_q, n_kv, dout, st);
        if (!e) e = eakvi_bounce_out(&bo, output_out, dout, qb, st);
        if (e) rc = eakvi_hip_fail(e, "attention_fused");
    }
    rc = eakvi_host_end(c, rc, began, "attention_fused");
    eakvi_bounce_end(&bo, rc, output_out, qb);
    eakvi_leave(prev);
    return rc;
}

/* The batched fused call with its chunk partials in the library's static
 * device scratch (eakvd_scratch) instead of caches[0]'s workspace: no
 * allocation on any path.  Calls on one device share that scratch, so calls
 * that overlap in time on one device race; their ordering is the caller's. */
int eakv_attention_fused_batch_device_noalloc(eakv_cache_t *const *caches,
                                              int n_caches, int layer,
                                              const float *d_q, int n_q, int n_kv,
                                              float *d_out, void *stream)
{
    if (!caches || n_caches <= 0 || n_caches > EAKVD_MAX_BATCH || !d_q || !d_out)
        return eakvi_set_error(EAKV_ERR_INVALID, "fused_noalloc: invalid argument");
    for (int i = 0; i < n_caches; i++) {
        if (!caches[i])
            return eakvi_set_error(EAKV_ERR_INVALID, "fused_noalloc: NULL cache");
        const eakv_cache_t *a = caches[0], *b = caches[i];
        if (a->n_layers != b->n_layers || a->n_kv_heads != b->n_kv_heads ||
            a->head_dim != b->head_dim || a->max_seq_len != b->max_seq_len ||
            a->device != b->device)
            return eakvi_set_error(EAKV_ERR_INVALID,
                                  "fused_noalloc: caches differ in shape");
    }
    eakv_cache_t *c0 = caches[0];
    int rc = attn_check(c0, layer, n_q, n_kv);
    if (rc) return rc;
    eakvd_batch b;
    memset(&b, 0, sizeof(b));
    b.n_seq = n_caches;
    for (int i = 0; i < n_caches; i++) {
        b.base[i] = caches[i]->dev;
        b.seq_len[i] = caches[i]->seq_len;
    }
    const size_t need = eakvd_fused_launch_bytes(&c0->geom, &b, n_q, n_kv);
    if (need > EAKVD_SCRATCH_BYTES)
        return eakvi_set_error(EAKV_ERR_INVALID,
                              "fused_noalloc: %zu bytes of partials needed, the static "
                              "scratch holds %zu", need, (size_t)EAKVD_SCRATCH_BYTES);
    int prev;
    rc = eakvi_enter(c0, &prev);
    if (rc) return rc;
    void *st = eakvi_batch_stream(caches, n_caches, stream);
    /* the work pending for the caches on the shared stream: device-side
     * waits with their events, which exist from creation on */
    for (int i = 0; rc == EAKV_OK && i < n_caches; i++)
        rc = eakvi_order_before(caches[i], st);
    void *scr = NULL;
    if (rc == EAKV_OK) {
        int e = eakvd_scratch(&scr);
        if (e) rc = eakvi_hip_fail(e, "fused_noalloc: scratch address");
    }
    if (rc == EAKV_OK) {
        /* no counters: the static scratch is shared by every caller */
        int e = eakvd_fused(&c0->geom, &b, layer, d_q, n_q, n_kv, d_out, scr, NULL, st);
        if (e) rc = eakvi_hip_fail(e, "fused_noalloc launch");
    }
    eakvi_leave(prev);
    return rc;
}

int eakv_attention_fused_plan(eakv_cache_t *const *caches, int n_caches, int n_q,
                              int n_kv, int noalloc, int32_t *plan)
{
    if (!caches || n_caches <= 0 || n_caches > EAKVD_MAX_BATCH || !plan)
        return eakvi_set_error(EAKV_ERR_INVALID, "fused_plan: invalid argument");
    for (int i = 0; i < n_caches; i++)
        if (!caches[i])
            return eakvi_set_error(EAKV_ERR_INVALID, "fused_plan: NULL cache");
    eakv_cache_t *c0 = caches[0];
    int rc = attn_check(c0, 0, n_q, n_kv);
    if (rc) return rc;
    eakvd_batch b;
    memset(&b, 0, sizeof(b));
    b.n_seq = n_caches;
    for (int i = 0; i < n_caches; i++) {
        b.base[i] = caches[i]->dev;
        b.seq_len[i] = caches[i]->seq_len;
    }
    int prev;
    rc = eakvi_enter(c0, &prev);
    if (rc) return rc;
    /* the workspace form merges with caches[0]'s counters; the
     * allocation-free form has none */
    eakvd_fused_plan(&c0->geom, &b, n_q, n_kv, noalloc ? NULL : c0->dev + c0->geom.ctr_off,
                     plan);
    eakvi_leave(prev);
    return EAKV_OK;
}
