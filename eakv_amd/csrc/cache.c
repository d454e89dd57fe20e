/* cache.c — cache lifecycle and quantization drivers (host C11).
 *
 * Follows reference src/cache.c:5-201: validation, error codes and seq_len
 * semantics are the reference's; the planes live in device memory and the
 * per-(layer, kv, head) quantize loop of the reference (cache.c:76-95,
 * :135-147) becomes one kernel launch over all groups.
 */
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

/* ------------------------------------------------------------------------ */
/* error side channel                                                        */

static _Thread_local int  tl_err;
static _Thread_local char tl_msg[256];

int eakvi_set_error(int code, const char *fmt, ...)
{
    va_list ap;
    tl_err = code;
    va_start(ap, fmt);
    vsnprintf(tl_msg, sizeof(tl_msg), fmt, ap);
    va_end(ap);
    return code;
}

int eakvi_hip_fail(int hip_err, const char *what)
{
    /* hipErrorOutOfMemory == 2 */
    int code = hip_err == 2 ? EAKV_ERR_ALLOC : EAKV_ERR_DEVICE;
    return eakvi_set_error(code, "%s: %s", what, eakvd_error_string(hip_err));
}

int eakv_last_error(void) { return tl_err; }
const char *eakv_last_error_message(void) { return tl_err ? tl_msg : ""; }
void eakv_clear_error(void) { tl_err = 0; tl_msg[0] = 0; }

/* ------------------------------------------------------------------------ */
/* layout and device helpers                                                 */

static int64_t round256(int64_t x) { return (x + 255) & ~(int64_t)255; }

void eakvd_geom_init(eakvd_geom *g, int n_layers, int n_kv_heads,
                     int head_dim, int max_seq_len)
{
    g->n_layers = n_layers;
    g->n_kv_heads = n_kv_heads;
    g->head_dim = head_dim;
    g->max_seq_len = max_seq_len;
    g->gpd = head_dim / 64;
    g->gph = (int64_t)max_seq_len * g->gpd;
    /* groups_per_token * max_seq_len (reference src/cache.c:26-27) */
    g->max_groups = (int64_t)n_kv_heads * head_dim / 64 * max_seq_len;
    g->s_off = round256(g->max_groups * 32);
    g->b_off = g->s_off + round256(g->max_groups * 4);
    g->block_bytes = g->b_off + round256(g->max_groups * 4);
    g->ctr_off = g->block_bytes * 2 * n_layers + EAKVD_TAIL_PAD;
    g->ctr_slots = n_kv_heads > EAKVD_CTR_MIN_SLOTS ? n_kv_heads : EAKVD_CTR_MIN_SLOTS;
    g->dev_bytes = g->ctr_off + g->ctr_slots * EAKVD_CTR_STRIDE;
}

int eakvi_enter(const eakv_cache_t *c, int *prev)
{
    int e = eakvd_get_device(prev);
    if (e) return eakvi_hip_fail(e, "hipGetDevice");
    if (*prev != c->device) {
        e = eakvd_set_device(c->device);
        if (e) return eakvi_hip_fail(e, "hipSetDevice");
    }
    return EAKV_OK;
}

void eakvi_leave(int prev)
{
    int cur = -1;
    if (eakvd_get_device(&cur) == 0 && cur != prev) eakvd_set_device(prev);
}

/* Every use of the workspace is ordered after the previous one: uses on the
 * shared stream by that stream; a use on a caller's stream records
 * work_event there, and the next use (on any stream) waits for it; the
 * host-pointer calls' uses on the cache's own stream are complete when the
 * call returns (eakvi_host_end).  A call on another stream than the shared
 * one first waits, on the device, for the cache's work pending there
 * (eakvi_order_before), which orders the other direction.  Growing the
 * workspace waits on the host for every earlier use (the shared stream
 * included) before the old buffer is freed. */
int eakvi_work_begin(eakv_cache_t *c, void *st, size_t n)
{
    if (c->work_on_caller) {
        int e = eakvd_stream_wait_event(st, c->work_event);
        if (e) return eakvi_hip_fail(e, "workspace order");
    }
    if (n <= c->work_bytes) return EAKV_OK;
    int e = eakvd_stream_sync(c->stream);
    if (!e && c->work_on_caller) e = eakvd_event_sync(c->work_event);
    if (e) return eakvi_hip_fail(e, "stream sync");
    if (c->work) eakvd_free(c->work);
    c->work = NULL;
    c->work_bytes = 0;
    size_t want = n + n / 4;
    e = eakvd_malloc(&c->work, want);
    if (e) {
        c->work = NULL;
        return eakvi_hip_fail(e, "workspace hipMalloc");
    }
    c->work_bytes = want;
    return EAKV_OK;
}

int eakvi_work_end(eakv_cache_t *c, void *st)
{
    if (st == c->stream) {
        c->work_on_caller = 0;
        return EAKV_OK;
    }
    int e = c->work_event ? 0 : eakvd_event_create(&c->work_event);
    if (!e) e = eakvd_event_record(c->work_event, st);
    if (e) {
        /* the order can no longer be tracked: wait for this use instead */
        eakvd_stream_sync(st);
        c->work_on_caller = 0;
        return eakvi_hip_fail(e, "workspace event");
    }
    c->work_on_caller = 1;
    return EAKV_OK;
}

void *eakvi_stream_or_default(const eakv_cache_t *c, void *s)
{
    /* the shared stream named explicitly (eakv_cache_stream) is the default */
    if (s && s != c->stream) return s;
    ((eakv_cache_t *)c)->own_async++;
    return c->stream;
}

void *eakvi_batch_stream(eakv_cache_t *const *caches, int n, void *s)
{
    if (s && s != caches[0]->stream) return s;
    for (int i = 0; i < n; i++) caches[i]->own_async++;
    return caches[0]->stream;
}

int eakvi_host_begin(eakv_cache_t *c)
{
    return eakvi_order_before(c, c->hstream);
}

int eakvi_pinned(eakv_cache_t *c, size_t n, void **p)
{
    if (n > c->pin_bytes) {
        /* nothing in flight uses the old buffer: every use ends in a wait */
        if (c->pin) eakvd_host_free(c->pin);
        c->pin = NULL;
        c->pin_bytes = 0;
        int e = eakvd_host_malloc(&c->pin, n);
        if (e) return e;
        c->pin_bytes = n;
    }
    *p = c->pin;
    return 0;
}

/* Inputs and results of a synchronous host-pointer call, up to kPinMax
 * bytes in all, travel through the cache's pinned host scratch: the input
 * is copied in and sent from there, the result lands there and is copied out
 * after the call's wait.  The runtime's own staging of pageable memory costs
 * more per copy (8 heads, d=128, one layer: the host-pointer V-sum
 * 27.2-27.3 against 34.8-35.0 us per call at 2048 tokens and 36.1-36.2
 * against 45.1-45.2 at 8192; the K-score 37.1-37.5 against 39.4-39.6 at
 * 8192).  Larger buffers, or no pinned memory, go from and to pageable
 * memory directly. */
#define kPinMax ((size_t)4 << 20)

void eakvi_bounce_begin(eakv_cache_t *c, size_t in_b, size_t out_b, eakvi_bounce *bo)
{
    void *p = NULL;
    bo->out_off = (in_b + 255) & ~(size_t)255;
    bo->pin = bo->out_off + out_b <= kPinMax && eakvi_pinned(c, bo->out_off + out_b, &p) == 0
                  ? (char *)p : NULL;
}

int eakvi_bounce_in(const eakvi_bounce *bo, void *d_dst, const void *src, size_t n, void *st)
{
    if (!n) return 0;
    if (!bo->pin) return eakvd_memcpy_h2d_async(d_dst, src, n, st);
    memcpy(bo->pin, src, n);
    return eakvd_memcpy_h2d_async(d_dst, bo->pin, n, st);
}

int eakvi_bounce_out(const eakvi_bounce *bo, void *dst, const void *d_src, size_t n, void *st)
{
    if (!n) return 0;
    return eakvd_memcpy_d2h_async(bo->pin ? bo->pin + bo->out_off : dst, d_src, n, st);
}

void eakvi_bounce_end(const eakvi_bounce *bo, int rc, void *dst, size_t n)
{
    if (rc == EAKV_OK && bo->pin && n) memcpy(dst, bo->pin + bo->out_off, n);
}

int eakvi_host_end(eakv_cache_t *c, int rc, int used_work, const char *what)
{
    int e = eakvd_stream_sync(c->hstream);
    if (e && rc == EAKV_OK) rc = eakvi_hip_fail(e, what);
    if (used_work) {
        if (!e) c->work_on_caller = 0;      /* the use is complete */
        else eakvi_work_end(c, c->hstream);
    }
    return rc;
}

/* Record c's order event on `from`; every stream in to[0..n) (other than
 * `from`) waits for it on the device.  If the event cannot be used, a host
 * wait for `from` orders the same work. */
static int order_wait(eakv_cache_t *c, void *from, void *const *to, int n)
{
    int e = c->order_event ? 0 : eakvd_event_create(&c->order_event);
    if (!e) e = eakvd_event_record(c->order_event, from);
    for (int i = 0; !e && i < n; i++)
        if (to[i] != from) e = eakvd_stream_wait_event(to[i], c->order_event);
    if (e) {
        int e2 = eakvd_stream_sync(from);
        if (e2) return eakvi_hip_fail(e2, "stream order");
    }
    return EAKV_OK;
}

int eakvi_order_before(eakv_cache_t *c, void *st)
{
    if (st == c->stream || c->own_async == 0 ||
        (c->own_async == c->ordered_seq && c->ordered_to == st))
        return EAKV_OK;
    int rc = order_wait(c, c->stream, &st, 1);
    if (rc == EAKV_OK) {
        c->ordered_seq = c->own_async;
        c->ordered_to = st;
    }
    return rc;
}

int eakvi_order_after(eakv_cache_t *const *caches, int n, void *st)
{
    void *to[EAKVD_MAX_BATCH];
    int k = 0;
    for (int i = 0; i < n && i < EAKVD_MAX_BATCH; i++) {
        void *s = caches[i]->stream;
        int seen = s == st;
        for (int j = 0; j < k && !seen; j++) seen = to[j] == s;
        if (!seen) to[k++] = s;
    }
    if (!k) return EAKV_OK;
    int rc = order_wait(caches[0], st, to, k);
    /* the shared stream now holds a wait for st on behalf of every named
     * cache: a later host-pointer call on one of them orders after it */
    for (int i = 0; rc == EAKV_OK && i < n; i++) caches[i]->own_async++;
    return rc;
}

/* ------------------------------------------------------------------------ */
/* lifecycle: reference src/cache.c:11-58                                    */

eakv_cache_t *eakv_cache_create(int n_layers, int n_kv_heads, int head_dim,
                                int max_seq_len)
{
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 ||
        max_seq_len <= 0) {
        eakvi_set_error(EAKV_ERR_INVALID, "cache_create: non-positive dimension");
        return NULL;
    }
    if (((int64_t)n_kv_heads * head_dim) % 64 != 0) {
        eakvi_set_error(EAKV_ERR_INVALID,
                       "cache_create: n_kv_heads*head_dim not a multiple of 64");
        return NULL;
    }
    eakv_cache_t *c = calloc(1, sizeof(*c));
    if (!c) {
        eakvi_set_error(EAKV_ERR_ALLOC, "cache_create: out of host memory");
        return NULL;
    }
    c->n_layers = n_layers;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->max_seq_len = max_seq_len;
    eakvd_geom_init(&c->geom, n_layers, n_kv_heads, head_dim, max_seq_len);
    c->dev_bytes = (size_t)c->geom.dev_bytes;

    int e = eakvd_get_device(&c->device);
    if (e) goto hip_fail;
    /* the device's caches share one stream (eakvd_device_stream) */
    e = eakvd_device_stream(c->device, &c->stream);
    if (e) goto hip_fail;
    /* the host-pointer calls' own stream */
    e = eakvd_stream_create(&c->hstream);
    if (e) goto hip_fail;
    /* created here so that ordering a batched call allocates nothing */
    e = eakvd_event_create(&c->order_event);
    if (e) goto hip_fail;
    e = eakvd_malloc((void **)&c->dev, c->dev_bytes);
    if (e) goto hip_fail;
    /* the reference calloc()s its planes (cache.c:33); the counters start
     * at zero */
    e = eakvd_memset_async(c->dev, 0, c->dev_bytes, c->hstream);
    if (!e) e = eakvd_stream_sync(c->hstream);
    if (e) goto hip_fail;
    return c;

hip_fail:
    eakvi_hip_fail(e, "cache_create");
    if (c->dev) eakvd_free(c->dev);
    if (c->order_event) eakvd_event_destroy(c->order_event);
    if (c->hstream) eakvd_stream_destroy(c->hstream);
    free(c);
    return NULL;
}

void eakv_cache_free(eakv_cache_t *c)
{
    if (!c) return;
    int prev;
    int ok = eakvi_enter(c, &prev) == EAKV_OK;
    if (c->stream) eakvd_stream_sync(c->stream);
    if (c->hstream) eakvd_stream_sync(c->hstream);
    if (c->work_on_caller) eakvd_event_sync(c->work_event);
    if (c->work_event) eakvd_event_destroy(c->work_event);
    if (c->order_event) eakvd_event_destroy(c->order_event);
    if (c->hstream) eakvd_stream_destroy(c->hstream);
    if (c->work) eakvd_free(c->work);
    if (c->pin) eakvd_host_free(c->pin);
    if (c->dev) eakvd_free(c->dev);
    if (ok) eakvi_leave(prev);
    free(c);
}

/* ------------------------------------------------------------------------ */
/* quantization drivers                                                      */

/* Quantize rows of `src` (device) into cache c: rows are (plane, head) for
 * planes plane0..plane0+n_planes-1, each n_g groups, row stride row_stride
 * floats, written at token offset t_off. */
static int quant_rows(eakv_cache_t *c, const float *src, int64_t row_stride,
                      int plane0, int n_planes, int64_t n_tok, int t_off,
                      void *stream)
{
    eakvd_quant_job job;
    memset(&job, 0, sizeof(job));
    job.src = src;
    job.row_stride = row_stride;
    job.n_rows = (int64_t)n_planes * c->n_kv_heads;
    job.n_g = n_tok * c->geom.gpd;
    job.nh = c->n_kv_heads;
    job.n_planes = n_planes;
    job.plane0 = plane0;
    job.n_caches = 1;
    job.base[0] = c->dev;
    job.g_off[0] = (int64_t)t_off * c->geom.gpd;
    int e = eakvd_quantize(&c->geom, &job, stream);
    return e ? eakvi_hip_fail(e, "quantize launch") : EAKV_OK;
}

/* reference src/cache.c:60-100 */
int eakv_cache_load_raw(eakv_cache_t *c, const float *data, int seq_len)
{
    if (!c || !data || seq_len <= 0)
        return eakvi_set_error(EAKV_ERR_INVALID, "load_raw: invalid argument");
    if (seq_len > c->max_seq_len)
        return eakvi_set_error(EAKV_ERR_INVALID, "load_raw: seq_len > max_seq_len");
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;

    /* Stage whole (layer, kv) planes through the device workspace, at most
     * ~256 MB (but at least one plane) per copy. */
    const int64_t row_elems = (int64_t)seq_len * c->head_dim;
    const int64_t plane_bytes = row_elems * c->n_kv_heads * 4;
    const int n_planes = 2 * c->n_layers;
    int per = (int)((256ll << 20) / (plane_bytes ? plane_bytes : 1));
    if (per < 1) per = 1;
    if (per > n_planes) per = n_planes;
    void *st = c->hstream;
    rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, (size_t)plane_bytes * per);
    const int began = rc == EAKV_OK;
    for (int p0 = 0; rc == EAKV_OK && p0 < n_planes; p0 += per) {
        int np = n_planes - p0 < per ? n_planes - p0 : per;
        int e = eakvd_memcpy_h2d_async(c->work, data + (int64_t)p0 * row_elems *
                                                            c->n_kv_heads,
                                       (size_t)plane_bytes * np, st);
        if (e) { rc = eakvi_hip_fail(e, "load_raw H2D"); break; }
        rc = quant_rows(c, (const float *)c->work, row_elems, p0, np, seq_len,
                        0, st);
    }
    rc = eakvi_host_end(c, rc, began, "load_raw");
    if (rc == EAKV_OK) c->seq_len = seq_len;
    eakvi_leave(prev);
    return rc;
}

int eakv_cache_load_raw_device(eakv_cache_t *c, const float *d_data,
                               int seq_len, void *stream)
{
    if (!c || !d_data || seq_len <= 0)
        return eakvi_set_error(EAKV_ERR_INVALID, "load_raw: invalid argument");
    if (seq_len > c->max_seq_len)
        return eakvi_set_error(EAKV_ERR_INVALID, "load_raw: seq_len > max_seq_len");
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    void *st = eakvi_stream_or_default(c, stream);
    /* a caller's stream: after the cache's work pending on the shared
     * stream, and that stream's (and the host calls') later work after it */
    rc = eakvi_order_before(c, st);
    if (rc == EAKV_OK)
        rc = quant_rows(c, d_data, (int64_t)seq_len * c->head_dim, 0,
                        2 * c->n_layers, seq_len, 0, st);
    if (rc == EAKV_OK) rc = eakvi_order_after(&c, 1, st);
    if (rc == EAKV_OK) c->seq_len = seq_len;
    eakvi_leave(prev);
    return rc;
}

static int append_check(const eakv_cache_t *c, const void *data, int layer,
                        int kv_idx, int n_tokens)
{
    if (!c || !data || n_tokens <= 0)
        return eakvi_set_error(EAKV_ERR_INVALID, "append: invalid argument");
    if (layer < 0 || layer >= c->n_layers)
        return eakvi_set_error(EAKV_ERR_INVALID, "append: layer out of range");
    if (kv_idx < 0 || kv_idx > 1)
        return eakvi_set_error(EAKV_ERR_INVALID, "append: kv_idx not 0 or 1");
    if ((int64_t)c->seq_len + n_tokens > c->max_seq_len)
        return eakvi_set_error(EAKV_ERR_INVALID, "append: exceeds max_seq_len");
    return EAKV_OK;
}

/* reference src/cache.c:102-151 */
int eakv_cache_append(eakv_cache_t *c, const float *data, int layer,
                      int kv_idx, int n_tokens)
{
    int rc = append_check(c, data, layer, kv_idx, n_tokens);
    if (rc) return rc;
    int prev;
    rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    const int64_t row_elems = (int64_t)n_tokens * c->head_dim;
    const size_t bytes = (size_t)row_elems * c->n_kv_heads * 4;
    void *st = c->hstream;
    rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, bytes);
    const int began = rc == EAKV_OK;
    if (rc == EAKV_OK) {
        eakvi_bounce bo;
        eakvi_bounce_begin(c, bytes, 0, &bo);
        int e = eakvi_bounce_in(&bo, c->work, data, bytes, st);
        if (e) rc = eakvi_hip_fail(e, "append H2D");
    }
    if (rc == EAKV_OK)
        rc = quant_rows(c, (const float *)c->work, row_elems,
                        layer * 2 + kv_idx, 1, n_tokens, c->seq_len, st);
    rc = eakvi_host_end(c, rc, began, "append");
    eakvi_leave(prev);
    return rc;
}

int eakv_cache_append_device(eakv_cache_t *c, const float *d_data, int layer,
                             int kv_idx, int n_tokens, void *stream)
{
    int rc = append_check(c, d_data, layer, kv_idx, n_tokens);
    if (rc) return rc;
    int prev;
    rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    void *st = eakvi_stream_or_default(c, stream);
    /* as load_raw_device */
    rc = eakvi_order_before(c, st);
    if (rc == EAKV_OK)
        rc = quant_rows(c, d_data, (int64_t)n_tokens * c->head_dim,
                        layer * 2 + kv_idx, 1, n_tokens, c->seq_len, st);
    if (rc == EAKV_OK) rc = eakvi_order_after(&c, 1, st);
    eakvi_leave(prev);
    return rc;
}

static int same_shape(const eakv_cache_t *a, const eakv_cache_t *b)
{
    return a->n_layers == b->n_layers && a->n_kv_heads == b->n_kv_heads &&
           a->head_dim == b->head_dim && a->max_seq_len == b->max_seq_len &&
           a->device == b->device;
}

int eakv_append_batch_device(eakv_cache_t *const *caches, int n_caches,
                             const float *d_data, int n_tokens, void *stream)
{
    if (!caches || n_caches <= 0 || n_caches > EAKVD_MAX_BATCH || !d_data ||
        n_tokens <= 0)
        return eakvi_set_error(EAKV_ERR_INVALID, "append_batch: invalid argument");
    for (int i = 0; i < n_caches; i++) {
        if (!caches[i] || !same_shape(caches[0], caches[i]))
            return eakvi_set_error(EAKV_ERR_INVALID,
                                  "append_batch: caches differ in shape");
        if ((int64_t)caches[i]->seq_len + n_tokens > caches[i]->max_seq_len)
            return eakvi_set_error(EAKV_ERR_INVALID,
                                  "append_batch: exceeds max_seq_len");
    }
    eakv_cache_t *c0 = caches[0];
    int prev, rc = eakvi_enter(c0, &prev);
    if (rc) return rc;
    void *st = eakvi_batch_stream(caches, n_caches, stream);
    /* the launch writes every cache: after their streams' earlier work */
    for (int i = 0; rc == EAKV_OK && i < n_caches; i++)
        rc = eakvi_order_before(caches[i], st);
    if (rc) {
        eakvi_leave(prev);
        return rc;
    }
    eakvd_quant_job job;
    memset(&job, 0, sizeof(job));
    job.src = d_data;
    job.row_stride = (int64_t)n_tokens * c0->head_dim;
    job.n_rows = (int64_t)n_caches * 2 * c0->n_layers * c0->n_kv_heads;
    job.n_g = (int64_t)n_tokens * c0->geom.gpd;
    job.nh = c0->n_kv_heads;
    job.n_planes = 2 * c0->n_layers;
    job.plane0 = 0;
    job.n_caches = n_caches;
    for (int i = 0; i < n_caches; i++) {
        job.base[i] = caches[i]->dev;
        job.g_off[i] = (int64_t)caches[i]->seq_len * c0->geom.gpd;
    }
    int e = eakvd_quantize(&c0->geom, &job, st);
    if (e) rc = eakvi_hip_fail(e, "append_batch launch");
    /* later work on each cache's own stream comes after the launch */
    if (rc == EAKV_OK) rc = eakvi_order_after(caches, n_caches, st);
    eakvi_leave(prev);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* seq_len bookkeeping: reference src/cache.c:153-201                        */

int eakv_cache_advance(eakv_cache_t *c, int n_tokens)
{
    if (!c || n_tokens <= 0)
        return eakvi_set_error(EAKV_ERR_INVALID, "advance: invalid argument");
    if ((int64_t)c->seq_len + n_tokens > c->max_seq_len)
        return eakvi_set_error(EAKV_ERR_INVALID, "advance: exceeds max_seq_len");
    c->seq_len += n_tokens;
    return EAKV_OK;
}

void eakv_cache_clear(eakv_cache_t *c)
{
    if (c) c->seq_len = 0;
}

int eakv_checkpoint(eakv_cache_t *c) { return c ? c->seq_len : 0; }

int eakv_restore(eakv_cache_t *c, int seq_len)
{
    if (!c) return eakvi_set_error(EAKV_ERR_INVALID, "restore: NULL cache");
    if (seq_len < 0 || seq_len > c->seq_len)
        return eakvi_set_error(EAKV_ERR_INVALID, "restore: seq_len out of range");
    c->seq_len = seq_len;
    return EAKV_OK;
}

int eakv_cache_seq_len(const eakv_cache_t *c) { return c ? c->seq_len : 0; }
int eakv_cache_n_layers(const eakv_cache_t *c) { return c ? c->n_layers : 0; }
int eakv_cache_n_heads(const eakv_cache_t *c) { return c ? c->n_kv_heads : 0; }
int eakv_cache_head_dim(const eakv_cache_t *c) { return c ? c->head_dim : 0; }
int eakv_cache_max_seq_len(const eakv_cache_t *c)
{
    return c ? c->max_seq_len : 0;
}

float eakv_cache_compression_ratio(const eakv_cache_t *c)
{
    if (!c || c->seq_len == 0) return 0.0f;
    return 40.0f / 256.0f;
}

int eakv_cache_device(const eakv_cache_t *c) { return c ? c->device : -1; }
void *eakv_cache_stream(const eakv_cache_t *c) { return c ? c->stream : NULL; }

int eakv_cache_sync(const eakv_cache_t *c)
{
    if (!c) return eakvi_set_error(EAKV_ERR_INVALID, "sync: NULL cache");
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    int e = eakvd_stream_sync(c->stream);
    if (e) rc = eakvi_hip_fail(e, "sync");
    eakvi_leave(prev);
    return rc;
}

int eakv_cache_read_planes(const eakv_cache_t *c, int layer, int kv_idx,
                           uint8_t *weights, float *scales, float *biases)
{
    if (!c || layer < 0 || layer >= c->n_layers || kv_idx < 0 || kv_idx > 1)
        return eakvi_set_error(EAKV_ERR_INVALID, "read_planes: invalid argument");
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    eakv_cache_t *cm = (eakv_cache_t *)c;
    const uint8_t *blk =
        c->dev + (int64_t)(layer * 2 + kv_idx) * c->geom.block_bytes;
    const size_t ng = (size_t)c->geom.max_groups;
    void *st = c->hstream;
    rc = eakvi_host_begin(cm);
    int e = 0;
    if (rc == EAKV_OK && weights) e = eakvd_memcpy_d2h_async(weights, blk, ng * 32, st);
    if (rc == EAKV_OK && !e && scales)
        e = eakvd_memcpy_d2h_async(scales, blk + c->geom.s_off, ng * 4, st);
    if (rc == EAKV_OK && !e && biases)
        e = eakvd_memcpy_d2h_async(biases, blk + c->geom.b_off, ng * 4, st);
    if (e) rc = eakvi_hip_fail(e, "read_planes");
    rc = eakvi_host_end(cm, rc, 0, "read_planes");
    eakvi_leave(prev);
    return rc;
}
