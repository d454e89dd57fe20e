/* io.c — .eakv files (host C11), staged through host memory.
 *
 * Byte format of reference src/io.c:6-160: a 512-byte packed little-endian
 * header (magic "EAKV", version 1, quant_scheme 0, group_size 64,
 * orig_dtype 0, n_layers, n_heads, head_dim, seq_len, max_seq_len written as
 * seq_len, compression 0, two zero 32-byte hashes, zero checksum), a table of
 * n_layers*2 u64 block offsets, then per (layer, kv) a 64-byte aligned block
 * weights | scales | biases holding n_heads*seq_len*head_dim/64 groups in
 * [head][pos][group] order.
 *
 * Writing differs from the reference in one case: the reference copies the
 * first n_groups groups of each plane, which is [head][pos][group] only when
 * seq_len == max_seq_len (planes keep a per-head stride of max_seq_len).  Each
 * head's first seq_len tokens are written here, so files are byte-identical to
 * the reference's when seq_len == max_seq_len and correct otherwise.  Reading
 * is the reference's (io.c:104-160).
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "internal.h"

#define HDR_BYTES 512

enum { H_MAGIC = 0, H_VERSION = 4, H_QUANT = 6, H_GROUP = 8, H_DTYPE = 12,
       H_LAYERS = 14, H_HEADS = 18, H_HDIM = 22, H_SEQ = 26, H_MAXSEQ = 30,
       H_COMP = 34 };

static size_t align64(size_t x) { return (x + 63) & ~(size_t)63; }

static void put_le(uint8_t *p, uint64_t v, int n)
{
    for (int i = 0; i < n; i++) p[i] = (uint8_t)(v >> (8 * i));
}

static uint64_t get_le(const uint8_t *p, int n)
{
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)p[i] << (8 * i);
    return v;
}

int eakv_cache_save(const eakv_cache_t *c, const char *path)
{
    if (!c || !path) return eakvi_set_error(EAKV_ERR_INVALID, "save: invalid argument");
    const int64_t gph = c->geom.gph;
    const int64_t g_head = (int64_t)c->seq_len * c->geom.gpd;
    const int64_t n_groups = (int64_t)c->n_kv_heads * c->head_dim * c->seq_len / 64;
    const size_t raw = (size_t)n_groups * 40, blk = align64(raw);
    const size_t ng = (size_t)c->geom.max_groups;

    uint8_t *w = malloc(ng * 32 + 1);
    float *s = malloc(ng * 4 + 4), *b = malloc(ng * 4 + 4);
    if (!w || !s || !b) {
        free(w); free(s); free(b);
        return eakvi_set_error(EAKV_ERR_ALLOC, "save: out of host memory");
    }
    FILE *f = fopen(path, "wb");
    if (!f) {
        free(w); free(s); free(b);
        return eakvi_set_error(EAKV_ERR_IO, "save: cannot open %s", path);
    }

    uint8_t hdr[HDR_BYTES];
    memset(hdr, 0, sizeof(hdr));
    memcpy(hdr + H_MAGIC, "EAKV", 4);
    put_le(hdr + H_VERSION, 1, 2);
    put_le(hdr + H_GROUP, 64, 4);
    put_le(hdr + H_LAYERS, (uint32_t)c->n_layers, 4);
    put_le(hdr + H_HEADS, (uint32_t)c->n_kv_heads, 4);
    put_le(hdr + H_HDIM, (uint32_t)c->head_dim, 4);
    put_le(hdr + H_SEQ, (uint32_t)c->seq_len, 4);
    put_le(hdr + H_MAXSEQ, (uint32_t)c->seq_len, 4);
    int ok = fwrite(hdr, 1, HDR_BYTES, f) == HDR_BYTES;

    const size_t idx = (size_t)c->n_layers * 2 * 8;
    const size_t start = align64(HDR_BYTES + idx);
    for (int i = 0; ok && i < c->n_layers * 2; i++) {
        uint8_t e8[8];
        put_le(e8, start + (size_t)i * blk, 8);
        ok = fwrite(e8, 1, 8, f) == 8;
    }
    static const uint8_t zeros[64];
    if (ok) ok = fwrite(zeros, 1, start - (HDR_BYTES + idx), f) ==
                 start - (HDR_BYTES + idx);

    int rc = EAKV_OK;
    for (int l = 0; ok && rc == EAKV_OK && l < c->n_layers; l++)
        for (int kv = 0; ok && kv < 2; kv++) {
            rc = eakv_cache_read_planes(c, l, kv, w, s, b);
            if (rc) break;
            for (int h = 0; ok && h < c->n_kv_heads && g_head > 0; h++)
                ok = fwrite(w + h * gph * 32, 32, (size_t)g_head, f) == (size_t)g_head;
            for (int h = 0; ok && h < c->n_kv_heads && g_head > 0; h++)
                ok = fwrite(s + h * gph, 4, (size_t)g_head, f) == (size_t)g_head;
            for (int h = 0; ok && h < c->n_kv_heads && g_head > 0; h++)
                ok = fwrite(b + h * gph, 4, (size_t)g_head, f) == (size_t)g_head;
            if (ok && blk > raw) ok = fwrite(zeros, 1, blk - raw, f) == blk - raw;
        }
    if (fclose(f) != 0) ok = 0;
    free(w); free(s); free(b);
    if (rc) return rc;
    return ok ? EAKV_OK : eakvi_set_error(EAKV_ERR_IO, "save: write failed");
}

int eakv_cache_load(const char *path, eakv_cache_t **out)
{
    if (!path || !out) return eakvi_set_error(EAKV_ERR_INVALID, "load: invalid argument");
    FILE *f = fopen(path, "rb");
    if (!f) return eakvi_set_error(EAKV_ERR_IO, "load: cannot open %s", path);
    uint8_t hdr[HDR_BYTES];
    if (fread(hdr, 1, HDR_BYTES, f) != HDR_BYTES ||
        memcmp(hdr + H_MAGIC, "EAKV", 4) != 0 || get_le(hdr + H_VERSION, 2) != 1) {
        fclose(f);
        return eakvi_set_error(EAKV_ERR_FORMAT, "load: not an .eakv v1 file");
    }
    const int nl = (int)get_le(hdr + H_LAYERS, 4), nh = (int)get_le(hdr + H_HEADS, 4);
    const int hd = (int)get_le(hdr + H_HDIM, 4), sl = (int)get_le(hdr + H_SEQ, 4);
    eakv_cache_t *c = eakv_cache_create(nl, nh, hd, sl);
    if (!c) {
        fclose(f);
        return eakvi_set_error(EAKV_ERR_ALLOC, "load: cannot create cache");
    }
    const int64_t n_groups = (int64_t)nh * hd * sl / 64;
    const size_t idx = (size_t)nl * 2 * 8;
    uint8_t *offs = malloc(idx);
    uint8_t *stage = malloc((size_t)n_groups * 40 + 1);
    int rc = (offs && stage) ? EAKV_OK
                             : eakvi_set_error(EAKV_ERR_ALLOC, "load: out of host memory");
    if (rc == EAKV_OK && fread(offs, 1, idx, f) != idx)
        rc = eakvi_set_error(EAKV_ERR_FORMAT, "load: truncated index");
    int prev = 0, entered = 0;
    if (rc == EAKV_OK) {
        rc = eakvi_enter(c, &prev);
        entered = rc == EAKV_OK;
    }
    /* the cache was created with max_seq_len = seq_len, so each plane's first
     * n_groups groups are exactly [head][pos][group] */
    for (int i = 0; rc == EAKV_OK && i < nl * 2; i++) {
        const uint64_t off = get_le(offs + (size_t)i * 8, 8);
        if (fseek(f, (long)off, SEEK_SET) != 0 ||
            fread(stage, 40, (size_t)n_groups, f) != (size_t)n_groups) {
            rc = eakvi_set_error(EAKV_ERR_FORMAT, "load: truncated block");
            break;
        }
        uint8_t *blk = c->dev + (int64_t)i * c->geom.block_bytes;
        int e = eakvd_memcpy_h2d_async(blk, stage, (size_t)n_groups * 32, c->hstream);
        if (!e) e = eakvd_memcpy_h2d_async(blk + c->geom.s_off, stage + n_groups * 32,
                                           (size_t)n_groups * 4, c->hstream);
        if (!e) e = eakvd_memcpy_h2d_async(blk + c->geom.b_off, stage + n_groups * 36,
                                           (size_t)n_groups * 4, c->hstream);
        if (e) rc = eakvi_hip_fail(e, "load H2D");
        rc = eakvi_host_end(c, rc, 0, "load H2D");
    }
    if (entered) eakvi_leave(prev);
    free(offs);
    free(stage);
    fclose(f);
    if (rc) {
        eakv_cache_free(c);
        return rc;
    }
    c->seq_len = sl;
    *out = c;
    return EAKV_OK;
}
