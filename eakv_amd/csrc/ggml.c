/* ggml.c — device-pointer forms of the ggml block-type callbacks of
 * reference include/eakv_ggml.h:36-52 (src/ggml_type.c:21-242), on the HIP
 * device current at the call and the given stream (NULL: the default
 * stream).  Buffers are 4-byte aligned (the blocks' f32 fields and the
 * rows are read as words); strides are in bytes, as in ggml. */
#include "internal.h"

#define ALIGNED4(p) ((((uintptr_t)(p)) & 3) == 0)

int eakv_ggml_quantize_row_device(const float *d_src, void *d_dst, int64_t k, void *stream)
{
    if (k < 0 || k % 64 != 0 || (k > 0 && (!d_src || !d_dst)) || !ALIGNED4(d_src) ||
        !ALIGNED4(d_dst))
        return eakvi_set_error(EAKV_ERR_INVALID, "ggml_quantize_row: invalid argument");
    int e = eakvd_ggml_quantize_row(d_src, d_dst, k, stream);
    return e ? eakvi_hip_fail(e, "ggml_quantize_row") : EAKV_OK;
}

int eakv_ggml_dequantize_row_device(const void *d_src, float *d_dst, int64_t k, void *stream)
{
    if (k < 0 || k % 64 != 0 || (k > 0 && (!d_src || !d_dst)) || !ALIGNED4(d_src) ||
        !ALIGNED4(d_dst))
        return eakvi_set_error(EAKV_ERR_INVALID, "ggml_dequantize_row: invalid argument");
    int e = eakvd_ggml_dequantize_row(d_src, d_dst, k, stream);
    return e ? eakvi_hip_fail(e, "ggml_dequantize_row") : EAKV_OK;
}

int eakv_ggml_vec_dot_device(int n, float *d_s, size_t bs, const void *d_vx, size_t bx,
                             const void *d_vy, size_t by, int nrc, void *stream)
{
    if (n < 0 || nrc < 0 || (nrc > 0 && (!d_s || !d_vx || !d_vy)) || !ALIGNED4(d_s) ||
        !ALIGNED4(d_vx) || !ALIGNED4(d_vy) || bs % 4 || bx % 4 || by % 4)
        return eakvi_set_error(EAKV_ERR_INVALID, "ggml_vec_dot: invalid argument");
    int e = eakvd_ggml_vec_dot(n, d_s, bs, d_vx, bx, d_vy, by, nrc, stream);
    return e ? eakvi_hip_fail(e, "ggml_vec_dot") : EAKV_OK;
}
