/* qs_sampler.c - the reference's sample.h API (sample.h:12-29), in C, over the device
 * batch of qs_batch.hip.
 *
 * One quasar_sampler is a one-row batch.  Its device buffers are created lazily at the
 * first pick (like sample.c's ensure_scratch, sample.c:94-104) and re-created when a
 * pick brings a wider vocabulary or a config asks for a larger history ring; the
 * generator state and the history survive a re-creation.
 *
 * A pick never fails, as in the reference: where sample.c:113-115 falls back to the
 * argmax of the raw logits when its scratch cannot be allocated, this layer does the same
 * when the device cannot take the pick (no device memory, no GPU, a device error), records
 * the id and reports it once on stderr.  The history is mirrored on the host for that
 * (each returned id is appended, sample.c:83-92), so the device row can be rebuilt from
 * it at the next pick.  The generator state is mirrored the same way (one xorshift64 step
 * per sampling pick, none for a greedy one or the fallback, sample.c:130-134,170), so a
 * lost device row is rebuilt from the state the reference would hold. */
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
    uint64_t      rng;          /* generator state, mirrored on the host */
    /* Host mirror of the history ring, sample.c's hist/hist_cap/hist_len/hist_head. */
    int32_t      *hist;
    int           hist_cap, hist_len, hist_head;
    int           warned;
};

/* sample.c:83-92 on the host mirror. */
static void host_record(quasar_sampler *s, int id) {
    if (s->hist_cap <= 0) return;
    if (s->hist_len < s->hist_cap) {
        s->hist[(s->hist_head + s->hist_len) % s->hist_cap] = id;
        s->hist_len++;
    } else {
        s->hist[s->hist_head] = id;
        s->hist_head = (s->hist_head + 1) % s->hist_cap;
    }
}

/* sample.c:72-77: the generator's step; a sampling pick takes one (sample.c:170). */
static uint64_t host_xorshift(uint64_t x) {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
}

/* The mirror's ids oldest first into out[hist_len]. */
static void host_history(const quasar_sampler *s, int32_t *out) {
    for (int i = 0; i < s->hist_len; ++i) out[i] = s->hist[(s->hist_head + i) % s->hist_cap];
}

/* Size the mirror to the clamped ring capacity (sample.c:61-66: only a positive
 * repeat_last_n that differs re-sizes it) and empty it.  0, or QS_ENOMEM (no ring). */
static int host_ring(quasar_sampler *s, int cap) {
    s->hist_len = s->hist_head = 0;
    if (cap == s->hist_cap) return 0;
    free(s->hist);
    s->hist = cap > 0 ? (int32_t *)calloc((size_t)cap, sizeof(int32_t)) : NULL;
    s->hist_cap = s->hist ? cap : 0;
    return cap > 0 && !s->hist ? QS_ENOMEM : 0;
}

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
    free(s->hist);
    free(s);
}

void quasar_sampler_config(quasar_sampler *s, float temperature, float top_p, int top_k,
                           float min_p, float repeat_penalty, int repeat_last_n,
                           uint64_t seed) {
    qs_clamp_config(temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n, seed,
                    s->prm.ring_cap, &s->prm, &s->rng);
    if (host_ring(s, s->prm.ring_cap) != 0) s->prm.ring_cap = 0;   /* sample.c:64 */
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
    s->hist_len = s->hist_head = 0;
    if (s->batch && qs_batch_reset(s->batch, 0, 1) != 0) qs_release(s);
}

/* Make the device buffers at least n_vocab wide, keeping generator state and history. */
static int qs_ensure(quasar_sampler *s, int n_vocab) {
    if (s->batch && n_vocab <= s->vocab_cap) return 0;
    uint64_t rng = s->rng;
    int32_t *hist = NULL;
    int hist_len = 0;
    if (s->batch) {                /* the device's state (the generator has moved on) */
        hist = (int32_t *)malloc(sizeof(int32_t) * (size_t)(s->ring_cap > 0 ? s->ring_cap : 1));
        if (!hist) return QS_ENOMEM;
        if (qs_batch_get_state(s->batch, 0, &rng, hist, s->ring_cap, &hist_len) != 0) {
            free(hist);
            return QS_EDEVICE;
        }
        s->rng = rng;
    } else if (s->hist_len > 0) {  /* a fresh row: the host's state */
        hist = (int32_t *)malloc(sizeof(int32_t) * (size_t)s->hist_len);
        if (!hist) return QS_ENOMEM;
        host_history(s, hist);
        hist_len = s->hist_len;
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

/* sample.c:113-115: the argmax of the raw logits (first index of the largest; a NaN at
 * index 0 keeps 0). */
static int host_argmax(const float *logits, int n_vocab) {
    int bi = 0;
    for (int i = 1; i < n_vocab; ++i)
        if (logits[i] > logits[bi]) bi = i;
    return bi;
}

int quasar_sampler_pick(quasar_sampler *s, const float *logits, int n_vocab) {
    if (n_vocab <= 0) return 0;                              /* sample.c:112 */
    int rc = qs_debug_take_failure() ? QS_ENOMEM : qs_ensure(s, n_vocab);
    int32_t id = -1;
    /* the row in, the pick, the id and the error flag out, one wait */
    if (rc == 0) rc = qs_batch_pick1_host(s->batch, s->d_logits, logits, n_vocab, s->d_out, &id);
    /* A whole-window row that found no free scratch slot in time kept its state: pick it
     * again (a one-row batch has its own slot, so this is not expected). */
    for (int again = 0; rc == QS_EAGAIN && again < 3; ++again)
        rc = qs_batch_pick1_host(s->batch, s->d_logits, logits, n_vocab, s->d_out, &id);
    if (rc == 0 && (id < 0 || id >= n_vocab)) rc = QS_EDEVICE;
    if (rc == 0) {
        host_record(s, id);
        if (!(s->prm.temperature <= 0.0f)) s->rng = host_xorshift(s->rng);   /* sample.c:130 */
        return id;
    }
    /* The device could not take the pick: the reference's out-of-memory answer. */
    if (!s->warned) {
        fprintf(stderr, "quasar_sampler_pick: device unavailable (%s); returning the argmax "
                        "of the raw logits\n", qs_last_error());
        s->warned = 1;
    }
    const int bi = host_argmax(logits, n_vocab);
    host_record(s, bi);
    /* Bring the device row in line (its generator state where it still answers), or drop
     * it so the next pick rebuilds it from the host state. */
    if (s->batch) {
        int ok = 0;
        int32_t *hist = (int32_t *)malloc(sizeof(int32_t) * (size_t)(s->hist_len > 0 ? s->hist_len : 1));
        uint64_t rng = 0;
        int len = 0;
        int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * (size_t)(s->ring_cap > 0 ? s->ring_cap : 1));
        if (hist && tmp && qs_batch_get_state(s->batch, 0, &rng, tmp, s->ring_cap, &len) == 0) {
            s->rng = rng;
            host_history(s, hist);
            ok = qs_batch_set_state(s->batch, 0, rng, hist, s->hist_len) == 0;
        }
        free(hist);
        free(tmp);
        if (!ok) qs_release(s);
    }
    return bi;
}

int qs_sampler_get_state(const quasar_sampler *s, uint64_t *rng, int32_t *hist, int hist_cap,
                         int *hist_len) {
    if (!s || !rng || !hist_len || (hist_cap > 0 && !hist) || hist_cap < 0) {
        qs_set_error("qs_sampler_get_state: bad arguments");
        return QS_EINVAL;
    }
    *rng = s->rng;
    if (s->batch) {
        /* the device's state, which the host mirror must equal */
        int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * (size_t)(s->ring_cap > 0 ? s->ring_cap : 1));
        int len = 0;
        uint64_t dev = 0;
        if (!tmp) return QS_ENOMEM;
        const int rc = qs_batch_get_state(s->batch, 0, &dev, tmp, s->ring_cap, &len);
        free(tmp);
        if (rc != 0) return rc;
        if (dev != s->rng) {
            qs_set_error("qs_sampler_get_state: device generator state %llx differs from the "
                         "host mirror %llx", (unsigned long long)dev,
                         (unsigned long long)s->rng);
            return QS_EDEVICE;
        }
    }
    const int n = s->hist_len < hist_cap ? s->hist_len : hist_cap;
    int32_t *all = (int32_t *)malloc(sizeof(int32_t) * (size_t)(s->hist_len > 0 ? s->hist_len : 1));
    if (!all) return QS_ENOMEM;
    host_history(s, all);
    memcpy(hist, all + (s->hist_len - n), sizeof(int32_t) * (size_t)n);
    free(all);
    *hist_len = n;
    return 0;
}
