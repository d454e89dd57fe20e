// runtime.hip — device memory, streams and copies behind the C ABI of
// eakvd.h.  Every stream is created at the default priority.
#include <hip/hip_runtime.h>

#include "../eakvd.h"

extern "C" {

int eakvd_get_device(int *dev) { return (int)hipGetDevice(dev); }
int eakvd_set_device(int dev) { return (int)hipSetDevice(dev); }

int eakvd_malloc(void **p, size_t n)
{
    *p = nullptr;
    return (int)hipMalloc(p, n);
}

int eakvd_free(void *p) { return p ? (int)hipFree(p) : 0; }

int eakvd_host_malloc(void **p, size_t n)
{
    *p = nullptr;
    return (int)hipHostMalloc(p, n, hipHostMallocDefault);
}

int eakvd_host_free(void *p) { return p ? (int)hipHostFree(p) : 0; }

int eakvd_stream_create(void **s)
{
    hipStream_t st = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    *s = (void *)st;
    return (int)e;
}

int eakvd_stream_destroy(void *s)
{
    return s ? (int)hipStreamDestroy((hipStream_t)s) : 0;
}

int eakvd_stream_sync(void *s) { return (int)hipStreamSynchronize((hipStream_t)s); }

int eakvd_event_create(void **e)
{
    hipEvent_t ev = nullptr;
    hipError_t r = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    *e = (void *)ev;
    return (int)r;
}

int eakvd_event_destroy(void *e) { return e ? (int)hipEventDestroy((hipEvent_t)e) : 0; }

int eakvd_event_record(void *e, void *s)
{
    return (int)hipEventRecord((hipEvent_t)e, (hipStream_t)s);
}

int eakvd_event_sync(void *e) { return (int)hipEventSynchronize((hipEvent_t)e); }

int eakvd_stream_wait_event(void *s, void *e)
{
    return (int)hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)e, 0);
}

int eakvd_memset_async(void *p, int v, size_t n, void *s)
{
    return (int)hipMemsetAsync(p, v, n, (hipStream_t)s);
}

int eakvd_memcpy_h2d_async(void *dst, const void *src, size_t n, void *s)
{
    return (int)hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice,
                               (hipStream_t)s);
}

int eakvd_memcpy_d2h_async(void *dst, const void *src, size_t n, void *s)
{
    return (int)hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost,
                               (hipStream_t)s);
}

int eakvd_memcpy_d2d_async(void *dst, const void *src, size_t n, void *s)
{
    return (int)hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice,
                               (hipStream_t)s);
}

const char *eakvd_error_string(int err)
{
    return hipGetErrorString((hipError_t)err);
}

}  // extern "C"
