/* qs_sampler.c - the reference's sample.h API (sample.h:12-29), in C, over the device
 * batch of qs_batch.hip.
 *
 * One quasar_sampler is a one-row batch.  Its device buffers are created lazily at the
 * first pick (like sample.c's ensure_scratch, sample.c:94-104) and re-created when a
 * pick brings a wider vocabulary or a config asks for a larger history ring; the
 * generator state and the history survive a re-creation. */
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/quasar_sampler.h"
#include "qs_internal.h"

struct quasar_sampler {
    qs_batch     *batch;        /* NULL until the first pick */
    int           vocab_cap;    /* widths the device buffers hold */
    int           ring_cap;     /* history capacity of the batch */
    float        *d_logits;
    int32_t      *d_out;
    /* Host copy of the configuration, to re-apply when the batch is re-created and to
     * seed it when a config arrives before the first pick. */
    qs_row_param  prm;
    uint64_t      rng;
    int           hist_n;       /* history length while no batch exists (always 0) */
    int           warned;
};

quasar_sampler *quasar_sampler_new(void) {
    quasar_sampler *s = (quasar_sampler *)calloc(1, sizeof *s);
    if (!s) return NULL;
    qs_default_param(&s->prm, &s->rng);
    return s;
}

static void qs_release(quasar_sampler *s) {
    if (s->batch) qs_batch_free(s->batch);
    qs_device_free(s->d_logits);
    qs_device_free(s->d_out);
    s->batch = NULL;
    s->d_logits = NULL;
    s->d_out = NULL;
    s->vocab_cap = 0;
    s->ring_cap = 0;
}

void quasar_sampler_free(quasar_sampler *s) {
    if (!s) return;
    qs_release(s);
    free(s);
}

void quasar_sampler_config(quasar_sampler *s, float temperature, float top_p, int top_k,
                           float min_p, float repeat_penalty, int repeat_last_n,
                           uint64_t seed) {
    qs_clamp_config(temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n, seed,
                    s->prm.ring_cap, &s->prm, &s->rng);
    s->hist_n = 0;
    if (!s->batch) return;
    if (s->prm.ring_cap > s->ring_cap) {
        /* Larger ring: the history is emptied by config anyway, so start afresh. */
        qs_release(s);
        return;
    }
    /* The clamps are re-applied by qs_batch_config; pass the clamped values and the
     * derived state as the seed so a seed of 0 is not re-drawn from the clock. */
    if (qs_batch_config(s->batch, 0, 1, s->prm.temperature, s->prm.top_p, s->prm.top_k,
                        s->prm.min_p, s->prm.repeat_penalty, s->prm.ring_cap, &s->rng) != 0)
        qs_release(s);
}

void quasar_sampler_reset(quasar_sampler *s) {
    s->hist_n = 0;
    if (s->batch && qs_batch_reset(s->batch, 0, 1) != 0) qs_release(s);
}

/* Make the device buffers at least n_vocab wide, keeping generator state and history. */
static int qs_ensure(quasar_sampler *s, int n_vocab) {
    if (s->batch && n_vocab <= s->vocab_cap) return 0;
    uint64_t rng = s->rng;
    int32_t *hist = NULL;
    int hist_len = 0;
    if (s->batch) {
        hist = (int32_t *)malloc(sizeof(int32_t) * (size_t)(s->ring_cap > 0 ? s->ring_cap : 1));
        if (!hist) return QS_ENOMEM;
        if (qs_batch_get_state(s->batch, 0, &rng, hist, s->ring_cap, &hist_len) != 0) {
            free(hist);
            return QS_EDEVICE;
        }
    }
    qs_release(s);
    int ring = s->prm.ring_cap;
    s->batch = qs_batch_new(1, n_vocab, ring);
    s->d_logits = (float *)qs_device_alloc(sizeof(float) * (size_t)n_vocab);
    s->d_out = (int32_t *)qs_device_alloc(sizeof(int32_t));
    if (!s->batch || !s->d_logits || !s->d_out) {
        qs_release(s);
        free(hist);
        return QS_ENOMEM;
    }
    s->vocab_cap = n_vocab;
    s->ring_cap = ring;
    int rc = qs_batch_config(s->batch, 0, 1, s->prm.temperature, s->prm.top_p, s->prm.top_k,
                             s->prm.min_p, s->prm.repeat_penalty, ring, &rng);
    if (rc == 0) rc = qs_batch_set_state(s->batch, 0, rng, hist, hist_len);
    free(hist);
    if (rc != 0) qs_release(s);
    return rc;
}

int quasar_sampler_pick(quasar_sampler *s, const float *logits, int n_vocab) {
    if (n_vocab <= 0) return 0;                              /* sample.c:112 */
    int rc = qs_ensure(s, n_vocab);
    if (rc == 0) rc = qs_memcpy_h2d(s->d_logits, logits, sizeof(float) * (size_t)n_vocab);
    if (rc == 0) rc = qs_batch_pick(s->batch, s->d_logits, n_vocab, 1, n_vocab, s->d_out, NULL);
    int32_t id = -1;
    if (rc == 0) rc = qs_batch_synchronize(s->batch);
    if (rc == 0) rc = qs_memcpy_d2h(&id, s->d_out, sizeof id);
    if (rc != 0) {
        if (!s->warned) {
            fprintf(stderr, "quasar_sampler_pick: device failure: %s\n", qs_last_error());
            s->warned = 1;
        }
        return -1;
    }
    return id;
}
