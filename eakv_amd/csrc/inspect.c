/* inspect.c — whole-plane reads of a GPU-resident cache: dequantization to
 * f32 (reference kernels/dequantize_avx512.ea, used by the reference's
 * benchmark baseline, benchmarks/bench_libeakv.c:76-98) and the integrity
 * check (reference kernels/validate.ea, run per block by the `validate`
 * command, src/cli.c:39-98). */
#include <stdlib.h>
#include <string.h>

#include "internal.h"

static int deq_args_ok(const eakv_cache_t *c, int layer, int kv_idx,
                       int64_t group_start, int64_t group_count)
{
    return c && layer >= 0 && layer < c->n_layers && kv_idx >= 0 && kv_idx <= 1 &&
           group_start >= 0 && group_count >= 0 &&
           group_start <= c->geom.max_groups - group_count;
}

int eakv_dequantize_range_device(const eakv_cache_t *c, int layer, int kv_idx,
                                 int64_t group_start, int64_t group_count,
                                 float *d_out, void *stream)
{
    if (!deq_args_ok(c, layer, kv_idx, group_start, group_count) ||
        (group_count > 0 && !d_out))
        return eakvi_set_error(EAKV_ERR_INVALID, "dequantize_range: invalid argument");
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    void *st = eakvi_stream_or_default(c, stream);
    /* a caller's stream: after the cache's work pending on the shared stream */
    rc = eakvi_order_before((eakv_cache_t *)c, st);
    if (rc == EAKV_OK) {
        int e = eakvd_dequantize(&c->geom, c->dev, layer, kv_idx, group_start, group_count,
                                 d_out, st);
        if (e) rc = eakvi_hip_fail(e, "dequantize_range");
    }
    eakvi_leave(prev);
    return rc;
}

int eakv_dequantize_range(const eakv_cache_t *cc, int layer, int kv_idx,
                          int64_t group_start, int64_t group_count, float *out)
{
    eakv_cache_t *c = (eakv_cache_t *)cc;
    if (!deq_args_ok(c, layer, kv_idx, group_start, group_count) ||
        (group_count > 0 && !out))
        return eakvi_set_error(EAKV_ERR_INVALID, "dequantize_range: invalid argument");
    if (group_count == 0) return EAKV_OK;
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    /* staged through the workspace, at most 64 MiB of f32 per pass */
    const int64_t per = (int64_t)1 << 18;              /* groups: 64 MiB */
    const int64_t chunk = group_count < per ? group_count : per;
    void *st = c->hstream;
    rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, (size_t)chunk * 256);
    const int began = rc == EAKV_OK;
    for (int64_t g = 0; began && rc == EAKV_OK && g < group_count; g += chunk) {
        const int64_t n = group_count - g < chunk ? group_count - g : chunk;
        int e = eakvd_dequantize(&c->geom, c->dev, layer, kv_idx, group_start + g, n,
                                 (float *)c->work, st);
        if (!e) e = eakvd_memcpy_d2h_async(out + g * 64, c->work, (size_t)n * 256, st);
        if (e) rc = eakvi_hip_fail(e, "dequantize_range");
        /* the next pass reuses the workspace: wait for this one */
        else if (g + chunk < group_count) rc = eakvi_host_end(c, rc, 0, "dequantize_range");
    }
    rc = eakvi_host_end(c, rc, began, "dequantize_range");
    eakvi_leave(prev);
    return rc;
}

int eakv_validate(const eakv_cache_t *cc, int32_t *results)
{
    eakv_cache_t *c = (eakv_cache_t *)cc;
    if (!c || !results)
        return eakvi_set_error(EAKV_ERR_INVALID, "validate: invalid argument");
    const int nb = 2 * c->n_layers;
    /* the groups the reference checks per block: src/cli.c:49 */
    const int64_t n = (int64_t)c->n_kv_heads * c->head_dim * c->seq_len / 64;
    int prev, rc = eakvi_enter(c, &prev);
    if (rc) return rc;
    unsigned long long *h = NULL;
    void *st = c->hstream;
    rc = eakvi_host_begin(c);
    if (rc == EAKV_OK) {
        int e = eakvi_pinned(c, (size_t)nb * sizeof(*h), (void **)&h);
        if (e) rc = eakvi_hip_fail(e, "validate: pinned host scratch");
    }
    if (rc == EAKV_OK) rc = eakvi_work_begin(c, st, (size_t)nb * sizeof(*h));
    const int began = rc == EAKV_OK;
    if (began) {
        int e = eakvd_validate(&c->geom, c->dev, nb, n, (unsigned long long *)c->work, st);
        if (!e) e = eakvd_memcpy_d2h_async(h, c->work, (size_t)nb * sizeof(*h), st);
        if (e) rc = eakvi_hip_fail(e, "validate");
    }
    rc = eakvi_host_end(c, rc, began, "validate");
    if (rc == EAKV_OK)
        for (int i = 0; i < nb; i++) results[i] = h[i] == ~0ull ? 0 : (int32_t)(h[i] & 3);
    eakvi_leave(prev);
    return rc;
}
