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
                              default priority, non-blocking, shared; the
                              device-pointer calls' default */
    void      *hstream;    /* this cache's own stream (default priority,
                              non-blocking): the synchronous host-pointer
                              calls of the reference API run and wait here */

    void  *work;           /* device scratch for staging and partials */
    size_t work_bytes;
    void  *work_event;     /* recorded after a use of `work` on a caller's stream */
    void  *pin;            /* pinned host scratch for small results copied back */
    size_t pin_bytes;
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

/* The stream a device-pointer call runs on: the caller's, or (NULL, or the
 * shared stream named explicitly) the device's shared stream, which the call
 * then counts as pending work of the cache on it. */
void *eakvi_stream_or_default(const eakv_cache_t *c, void *s);
/* The same for a call that names the caches [0, n): with a NULL stream the
 * launch is counted as pending work of every one of them. */
void *eakvi_batch_stream(eakv_cache_t *const *caches, int n, void *s);

/* Synchronous host-pointer calls (the reference API) run on c->hstream.
 * eakvi_host_begin orders hstream after the cache's device-pointer work still
 * pending on the shared stream (a device-side wait, only when there is
 * such); eakvi_host_end waits for hstream alone and, when that succeeds,
 * marks the workspace use st == hstream complete (otherwise it stays ordered
 * by its event).  Two threads working on distinct caches therefore wait for
 * their own work only.  Returns rc, or the wait's error if rc is EAKV_OK. */
int  eakvi_host_begin(eakv_cache_t *c);
int  eakvi_host_end(eakv_cache_t *c, int rc, int used_work, const char *what);

/* The cache's pinned host scratch, at least n bytes (grown on demand; the
 * device's copies from and into pinned memory skip the runtime's staging of
 * pageable memory).  Used between eakvi_host_begin and eakvi_host_end only.
 * Returns 0 or the HIP error of the allocation (the error text untouched). */
int  eakvi_pinned(eakv_cache_t *c, size_t n, void **p);

/* A host-pointer call's input and result through the pinned scratch when
 * they fit (pin NULL: pageable copies).  begin reserves in_b + out_b bytes;
 * in and out enqueue the copies on st; end copies the result out once the
 * call's wait has succeeded (rc). */
typedef struct {
    char  *pin;
    size_t out_off;
} eakvi_bounce;
void eakvi_bounce_begin(eakv_cache_t *c, size_t in_b, size_t out_b, eakvi_bounce *bo);
int  eakvi_bounce_in(const eakvi_bounce *bo, void *d_dst, const void *src, size_t n, void *st);
int  eakvi_bounce_out(const eakvi_bounce *bo, void *dst, const void *d_src, size_t n,
                      void *st);
void eakvi_bounce_end(const eakvi_bounce *bo, int rc, void *dst, size_t n);

#endif
