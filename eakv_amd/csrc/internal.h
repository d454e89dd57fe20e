/* internal.h — host-side cache object and helpers (not public). */
#ifndef EAKV_INTERNAL_H
#define EAKV_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "../../include/eakv.h"
#include "../../include/eakv_hip.h"
#include "eakvd.h"

/* Reference struct eakv_cache (src/internal.h:14-26) with the planes moved
 * to device memory: one allocation `dev` carved as described in eakvd.h. */
struct eakv_cache {
    int n_layers;
    int n_kv_heads;
    int head_dim;
    int max_seq_len;
    int seq_len;

    eakvd_geom geom;
    int        device;     /* HIP ordinal current at creation */
    uint8_t   *dev;        /* planes */
    size_t     dev_bytes;
    void      *stream;     /* default-priority, non-blocking */

    void  *work;           /* device scratch for staging and partials */
    size_t work_bytes;
};

/* error side channel (cache.c) */
int  eakvi_set_error(int code, const char *fmt, ...);
int  eakvi_hip_fail(int hip_err, const char *what);

/* Make the cache's device current; returns the previous device via *prev. */
int  eakvi_enter(const eakv_cache_t *c, int *prev);
void eakvi_leave(int prev);

/* Grow the cache's device scratch to at least n bytes (synchronizes the
 * cache's stream before freeing the old buffer). */
int  eakvi_work_reserve(eakv_cache_t *c, size_t n);

static inline void *eakvi_stream_or_default(const eakv_cache_t *c, void *s)
{
    return s ? s : c->stream;
}

#endif
