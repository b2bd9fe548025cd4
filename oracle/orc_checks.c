/* orc_checks.c - host builds of the product's portable helpers, for tests only.
 *
 * The synthetic-input generator and the libm-compatible expf are shared headers of the
 * product (quasar_amd/csrc); compiling them here for the host lets the CPU tests pin
 * them (generator determinism, expf == host expf) and lets the oracle run on exactly the
 * bits the GPU generates. */
#define _POSIX_C_SOURCE 200809L
#include "orc_sampler.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "../quasar_amd/csrc/qs_expf.h"
#include "../quasar_amd/csrc/qs_gen.h"

void orc_gen_logits(int32_t dist, float sigma, float boost, uint64_t seed, long row0,
                    int n_rows, int n_vocab, float *out, long row_stride) {
    qs_gen_spec g;
    memset(&g, 0, sizeof g);
    g.dist = dist; g.sigma = sigma; g.boost = boost; g.seed = seed;
    for (int r = 0; r < n_rows; r++)
        for (int c = 0; c < n_vocab; c++)
            out[(long)r * row_stride + c] = qs_gen_logit(&g, (uint64_t)(row0 + r), c, n_vocab);
}

void orc_gen_hist(uint64_t seed, long row0, int n_rows, int hist_n, int n_vocab, int pool,
                  int32_t *out) {
    for (int r = 0; r < n_rows; r++)
        for (int j = 0; j < hist_n; j++)
            out[(long)r * hist_n + j] =
                qs_gen_hist_id(seed, (uint64_t)(row0 + r), j, n_vocab, pool);
}

uint64_t orc_gen_row_seed(uint64_t seed, long row) { return qs_gen_row_seed(seed, (uint64_t)row); }

float orc_product_expf(float x) { return qs_expf(x); }

/* The host C library's expf over an array (the reference's softmax numerator routine). */
void orc_libm_expf_array(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) y[i] = expf(x[i]);
}

typedef struct { uint32_t lo, hi; int neg; long bad; } orc_xjob;

/* The window variant's extended table (qs_expf_window), built before any walk starts. */
static uint64_t orc_xtab[QS_EXPF_XTAB_N];

/* Walk float bit patterns [lo, hi] of one sign: qs_expf everywhere and, inside the
 * window variant's range [-33, 0], qs_expf_window too, against the C library's expf. */
static long orc_xwalk(const orc_xjob *j) {
    long bad = 0;
    for (uint64_t b = j->lo; b <= j->hi; b++) {
        uint32_t bits = (uint32_t)b | (j->neg ? 0x80000000u : 0u);
        float x = qs_u2f(bits);
        float a = expf(x), c = qs_expf(x);
        if (qs_f2u(a) != qs_f2u(c) && !(isnan(a) && isnan(c))) bad++;
        if (x <= 0.0f && x >= -33.0f && qs_f2u(qs_expf_window(x, orc_xtab)) != qs_f2u(a)) bad++;
    }
    return bad;
}

/* Same walk with the fused multiply-adds in hardware (the result is identical; only the
 * software fallback of fma() is slow). */
__attribute__((target("fma"))) static long orc_xwalk_fma(const orc_xjob *j) {
    long bad = 0;
    for (uint64_t b = j->lo; b <= j->hi; b++) {
        uint32_t bits = (uint32_t)b | (j->neg ? 0x80000000u : 0u);
        float x = qs_u2f(bits);
        float a = expf(x), c = qs_expf(x);
        if (qs_f2u(a) != qs_f2u(c) && !(isnan(a) && isnan(c))) bad++;
        if (x <= 0.0f && x >= -33.0f && qs_f2u(qs_expf_window(x, orc_xtab)) != qs_f2u(a)) bad++;
    }
    return bad;
}

static void *orc_xrun(void *arg) {
    orc_xjob *j = (orc_xjob *)arg;
    j->bad = __builtin_cpu_supports("fma") ? orc_xwalk_fma(j) : orc_xwalk(j);
    return NULL;
}

long orc_check_expf_range(float lo, float hi, int n_threads) {
    /* Split [lo, hi] into a non-positive and a non-negative part, each a contiguous range
     * of magnitude bit patterns. */
    struct { uint32_t a, b; int neg; } parts[2];
    int np = 0;
    if (lo <= 0.0f) {
        float top = hi < 0.0f ? hi : -0.0f;
        parts[np].a = qs_f2u(top) & 0x7fffffffu;
        parts[np].b = qs_f2u(lo) & 0x7fffffffu;
        parts[np].neg = 1;
        np++;
    }
    if (hi >= 0.0f) {
        float bot = lo > 0.0f ? lo : 0.0f;
        parts[np].a = qs_f2u(bot);
        parts[np].b = qs_f2u(hi);
        parts[np].neg = 0;
        np++;
    }
    if (n_threads < 1) n_threads = 1;
    for (int i = 0; i < QS_EXPF_XTAB_N; i++) orc_xtab[i] = qs_expf_xtab_entry(qs_expf_table_host, i);
    long bad = 0;
    for (int k = 0; k < np; k++) {
        orc_xjob *jobs = (orc_xjob *)calloc((size_t)n_threads, sizeof(orc_xjob));
        pthread_t *th = (pthread_t *)calloc((size_t)n_threads, sizeof(pthread_t));
        uint64_t span = (uint64_t)parts[k].b - parts[k].a + 1;
        for (int t = 0; t < n_threads; t++) {
            jobs[t].lo = (uint32_t)(parts[k].a + span * t / n_threads);
            jobs[t].hi = (uint32_t)(parts[k].a + span * (t + 1) / n_threads - 1);
            jobs[t].neg = parts[k].neg;
            if (jobs[t].hi >= jobs[t].lo) pthread_create(&th[t], NULL, orc_xrun, &jobs[t]);
        }
        for (int t = 0; t < n_threads; t++) {
            if (jobs[t].hi >= jobs[t].lo) { pthread_join(th[t], NULL); bad += jobs[t].bad; }
        }
        free(jobs);
        free(th);
    }
    return bad;
}
