/* drop_in_caller.c — a C11 caller of libeakv.so that uses only the
 * reference's public header (include/eakv.h) and its call pattern:
 *   - bulk load vs one-token-at-a-time append of every (layer, kv) followed
 *     by eakv_cache_advance, then scores and output on both
 *     (reference tests/test_append.c:40-119);
 *   - per-layer K/V append of the newest token, advance, scores
 *     (reference examples/offload_demo.c:263-289);
 *   - row softmax of the scores in the caller, then eakv_attention_output
 *     (the caller-side step of reference README.md:101);
 *   - save / load round trip (reference include/eakv.h:73-75) and the
 *     error codes of create / load_raw / append / restore / load.
 * Usage: drop_in_caller HEAD_DIM OUT_FILE EAKV_FILE.  Prints one line per
 * check, returns 0 when all pass, and writes the inputs and results to
 * OUT_FILE for the test that compares them with the CPU oracle.  Layout of
 * OUT_FILE (host-endian i32 header, then f32 arrays):
 *   nl nh hd sl nq, data[nl][2][nh][sl][hd], q[nq][hd],
 *   scores[nq][sl] (layer nl-1), weights[nq][sl], output[nq][hd]. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "eakv.h"

static int n_checks, n_failed;

static void check(const char *what, int ok)
{
    n_checks++;
    if (!ok) n_failed++;
    printf("%s: %s\n", ok ? "ok" : "FAIL", what);
    fflush(stdout);
}

/* deterministic inputs: splitmix64 -> uniform [-4, 4) */
static uint64_t rng_state = 0xEA4BULL;
static float next_f32(void)
{
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return (float)((double)(z >> 40) / (double)(1ULL << 24) * 8.0 - 4.0);
}

/* the [nh][1][hd] slice of token t of (layer l, kv) from
 * data[nl][2][nh][sl][hd] */
static void slice(const float *data, int nh, int hd, int sl, int l, int kv, int t, float *out)
{
    for (int h = 0; h < nh; h++)
        memcpy(out + (size_t)h * hd,
               data + ((((size_t)l * 2 + kv) * nh + h) * sl + t) * hd, (size_t)hd * 4);
}

int main(int argc, char **argv)
{
    if (argc != 4) {
        fprintf(stderr, "usage: %s HEAD_DIM OUT_FILE EAKV_FILE\n", argv[0]);
        return 2;
    }
    const int hd = atoi(argv[1]);
    const int nl = 3, nh = 4, sl = 70, nq = 8;
    const size_t n_data = (size_t)nl * 2 * nh * sl * hd;
    float *data = malloc(n_data * 4);
    float *q = malloc((size_t)nq * hd * 4);
    float *tok = malloc((size_t)nh * hd * 4);
    float *sc_b = malloc((size_t)nq * sl * 4), *sc_i = malloc((size_t)nq * sl * 4);
    float *w = malloc((size_t)nq * sl * 4);
    float *o_b = malloc((size_t)nq * hd * 4), *o_i = malloc((size_t)nq * hd * 4);
    if (!data || !q || !tok || !sc_b || !sc_i || !w || !o_b || !o_i) return 3;
    for (size_t i = 0; i < n_data; i++) data[i] = next_f32();
    for (int i = 0; i < nq * hd; i++) q[i] = next_f32() * 0.25f;

    /* errors of the reference's validation */
    check("create rejects a zero dimension", eakv_cache_create(0, nh, hd, sl) == NULL);
    check("create rejects n_kv*head_dim % 64 != 0", eakv_cache_create(1, 1, 32, sl) == NULL);

    eakv_cache_t *bulk = eakv_cache_create(nl, nh, hd, sl);
    eakv_cache_t *incr = eakv_cache_create(nl, nh, hd, sl);
    check("create", bulk && incr);
    if (!bulk || !incr) return 1;
    check("load_raw rejects seq_len > max_seq_len",
          eakv_cache_load_raw(bulk, data, sl + 1) == EAKV_ERR_INVALID);
    check("load_raw", eakv_cache_load_raw(bulk, data, sl) == EAKV_OK);
    check("getters", eakv_cache_seq_len(bulk) == sl && eakv_cache_n_layers(bulk) == nl &&
                         eakv_cache_n_heads(bulk) == nh && eakv_cache_head_dim(bulk) == hd &&
                         eakv_cache_max_seq_len(bulk) == sl);
    check("compression ratio 40/256", eakv_cache_compression_ratio(bulk) == 40.0f / 256.0f);

    /* one token at a time, every layer and K/V, then advance */
    int ok = 1;
    for (int t = 0; t < sl && ok; t++) {
        for (int l = 0; l < nl && ok; l++)
            for (int kv = 0; kv < 2 && ok; kv++) {
                slice(data, nh, hd, sl, l, kv, t, tok);
                ok = eakv_cache_append(incr, tok, l, kv, 1) == EAKV_OK;
            }
        ok = ok && eakv_cache_advance(incr, 1) == EAKV_OK;
    }
    check("append + advance, token by token", ok && eakv_cache_seq_len(incr) == sl);
    check("append rejects a write past max_seq_len",
          eakv_cache_append(incr, tok, 0, 0, 1) == EAKV_ERR_INVALID);
    check("append rejects kv_idx 2", eakv_cache_append(incr, tok, 0, 2, 1) == EAKV_ERR_INVALID);
    check("advance rejects past max_seq_len", eakv_cache_advance(incr, 1) == EAKV_ERR_INVALID);

    /* scores: appended == bulk, bit for bit, on every layer (GQA 2:1) */
    for (int l = 0; l < nl; l++) {
        eakv_attention_scores(bulk, q, l, nq, nh, sc_b);
        eakv_attention_scores(incr, q, l, nq, nh, sc_i);
        char what[96];
        snprintf(what, sizeof(what), "layer %d scores: append == bulk, bit for bit", l);
        check(what, memcmp(sc_b, sc_i, (size_t)nq * sl * 4) == 0);
    }
    /* the caller's row softmax (layer nl-1 scores), then the V-sum */
    for (int h = 0; h < nq; h++) {
        const float *s = sc_b + (size_t)h * sl;
        float m = s[0], sum = 0.0f;
        for (int t = 1; t < sl; t++) m = s[t] > m ? s[t] : m;
        for (int t = 0; t < sl; t++) {
            w[(size_t)h * sl + t] = expf(s[t] - m);
            sum += w[(size_t)h * sl + t];
        }
        for (int t = 0; t < sl; t++) w[(size_t)h * sl + t] *= 1.0f / sum;
    }
    eakv_attention_output(bulk, w, nl - 1, nq, nh, o_b);
    eakv_attention_output(incr, w, nl - 1, nq, nh, o_i);
    check("output: append == bulk, bit for bit", memcmp(o_b, o_i, (size_t)nq * hd * 4) == 0);
    int finite = 1;
    for (int i = 0; i < nq * hd; i++) finite = finite && isfinite(o_b[i]);
    check("output finite", finite);

    /* checkpoint / restore (O(1) rewind) */
    const int cp = eakv_checkpoint(incr);
    check("restore rejects a longer seq_len", eakv_restore(incr, cp + 1) == EAKV_ERR_INVALID);
    check("restore", eakv_restore(incr, sl / 2) == EAKV_OK && eakv_cache_seq_len(incr) == sl / 2);
    eakv_cache_clear(incr);
    check("clear", eakv_cache_seq_len(incr) == 0);

    /* the decode pattern: per-layer append of the newest token, advance,
     * scores on layer 0 */
    eakv_cache_t *dec = eakv_cache_create(nl, nh, hd, sl);
    float *first = malloc((size_t)nl * 2 * nh * hd * 4);     /* [nl][2][nh][1][hd] */
    ok = dec && first;
    for (int l = 0; l < nl && ok; l++)
        for (int kv = 0; kv < 2; kv++)
            slice(data, nh, hd, sl, l, kv, 0, first + ((size_t)l * 2 + kv) * nh * hd);
    ok = ok && eakv_cache_load_raw(dec, first, 1) == EAKV_OK;
    free(first);
    for (int t = 1; t < sl && ok; t++) {
        for (int l = 0; l < nl && ok; l++) {
            slice(data, nh, hd, sl, l, 0, t, tok);
            ok = eakv_cache_append(dec, tok, l, 0, 1) == EAKV_OK;
            slice(data, nh, hd, sl, l, 1, t, tok);
            ok = ok && eakv_cache_append(dec, tok, l, 1, 1) == EAKV_OK;
        }
        ok = ok && eakv_cache_advance(dec, 1) == EAKV_OK;
    }
    check("decode loop", ok && eakv_cache_seq_len(dec) == sl);
    eakv_attention_scores(dec, q, 0, nq, nh, sc_i);
    eakv_attention_scores(bulk, q, 0, nq, nh, sc_b);
    check("decode cache == bulk cache (scores)", memcmp(sc_b, sc_i, (size_t)nq * sl * 4) == 0);
    eakv_cache_free(dec);

    /* save / load */
    check("save", eakv_cache_save(bulk, argv[3]) == EAKV_OK);
    eakv_cache_t *back = NULL;
    check("load", eakv_cache_load(argv[3], &back) == EAKV_OK && back);
    if (back) {
        eakv_attention_scores(back, q, nl - 1, nq, nh, sc_i);
        eakv_attention_scores(bulk, q, nl - 1, nq, nh, sc_b);
        check("loaded scores == saved scores", memcmp(sc_b, sc_i, (size_t)nq * sl * 4) == 0);
        eakv_cache_free(back);
    }
    eakv_cache_t *none = NULL;
    check("load of a missing file is EAKV_ERR_IO",
          eakv_cache_load("/nonexistent/x.eakv", &none) == EAKV_ERR_IO && none == NULL);

    FILE *f = fopen(argv[2], "wb");
    int hdr[5] = {nl, nh, hd, sl, nq};
    ok = f && fwrite(hdr, 4, 5, f) == 5 && fwrite(data, 4, n_data, f) == n_data &&
         fwrite(q, 4, (size_t)nq * hd, f) == (size_t)nq * hd &&
         fwrite(sc_b, 4, (size_t)nq * sl, f) == (size_t)nq * sl &&
         fwrite(w, 4, (size_t)nq * sl, f) == (size_t)nq * sl &&
         fwrite(o_b, 4, (size_t)nq * hd, f) == (size_t)nq * hd;
    if (f) ok = (fclose(f) == 0) && ok;
    check("results written", ok);

    eakv_cache_free(bulk);
    eakv_cache_free(incr);
    eakv_cache_free(NULL);
    free(data); free(q); free(tok); free(sc_b); free(sc_i); free(w); free(o_b); free(o_i);
    printf("%d checks, %d failed\n", n_checks, n_failed);
    return n_failed ? 1 : 0;
}
