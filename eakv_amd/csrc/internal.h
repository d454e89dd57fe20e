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
    void      *stream;     /* the device's caches' stream (eakvd_device_stream):
                              default priority, non-blocking, shared */

    void  *work;           /* device scratch for staging and partials */
    size_t work_bytes;
    void  *work_event;     /* recorded after a use of `work` on a caller's stream */
    int    work_on_caller; /* the last use of `work` was on a caller's stream */
    void  *order_event;    /* orders a batched call against this cache's stream */
    unsigned own_async;    /* device-pointer calls enqueued on `stream` so far */
    unsigned ordered_seq;  /* own_async when a batched call last waited for `stream` */
    void    *ordered_to;   /* the stream that waited */
};

/* error side channel (cache.c) */
int  eakvi_set_error(int code, const char *fmt, ...);
int  eakvi_hip_fail(int hip_err, const char *what);

/* Make the cache's device current; returns the previous device via *prev. */
int  eakvi_enter(const eakv_cache_t *c, int *prev);
void eakvi_leave(int prev);

/* Begin a use of the cache's device scratch on stream st: order st after
 * the previous use when that was on a caller's stream (a stream wait, no host
 * wait), and grow the scratch to at least n bytes (waiting for every earlier
 * use before freeing the old buffer). */
int  eakvi_work_begin(eakv_cache_t *c, void *st, size_t n);
/* End a use begun on st (enqueued): on a caller's stream, record the
 * scratch's event there so that the next use waits for this one. */
int  eakvi_work_end(eakv_cache_t *c, void *st);

/* Batched calls on stream st that name several caches:
 * eakvi_order_before makes st wait, on the device, for the device-pointer
 * calls enqueued so far on c's own stream (nothing when st is that stream or
 * there are none since the last such wait by st; host-pointer calls finish
 * before they return).  eakvi_order_after makes the own streams of caches
 * [0, n) wait for the work enqueued so far on st (one event, recorded with
 * caches[0]'s order_event). */
int  eakvi_order_before(eakv_cache_t *c, void *st);
int  eakvi_order_after(eakv_cache_t *const *caches, int n, void *st);

/* The stream a device-pointer call runs on: the caller's, or (NULL) the
 * cache's own, which the call then counts as pending work on it. */
void *eakvi_stream_or_default(const eakv_cache_t *c, void *s);

#endif
